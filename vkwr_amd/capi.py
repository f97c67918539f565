"""ctypes binding of the C ABI (include/vkwr_amd.h) for the model executor.

The reference-compatible torch ops (vkwr._ops) cover the reference's op
surface; the decode driver additionally needs the fused entry points that
have no reference op (batched GEMMs with fused epilogues, the slot-indexed
shift-state fusion).  This module calls them directly with device pointers
taken from torch tensors, on torch's current HIP stream, so a whole decode
step can be captured into a HIP graph.  Every call checks the status code and
raises RuntimeError with the library's message.
"""
import ctypes
import os

import torch

_LIBPATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libvkwr_amd.so")
if not os.path.exists(_LIBPATH):
    raise ImportError(f"vkwr_amd: {_LIBPATH} is not built (gfx950 HIP kernels); there is no CPU fallback.")
_LIB = ctypes.CDLL(_LIBPATH)

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

GEMM_B_NK, GEMM_B_KN = 0, 1
ACT_NONE, ACT_TANH, ACT_SIGMOID, ACT_RELU_SQUARE = 0, 1, 2, 3
EPI_NONE, EPI_RELU_SQUARE, EPI_VALUE_RESIDUAL, EPI_BIAS = 0, 1, 2, 3
EPI_TANH, EPI_SIGMOID = 4, 5
MAX_GEMM_PROBLEMS = 8
FRAG_PAD = 128


def frag_pad(x):
    """Padded extent of a frag-matrix dimension (rows and K: multiples of 128)."""
    return (x + FRAG_PAD - 1) // FRAG_PAD * FRAG_PAD


def frag_empty(rows, k, device, zero=True):
    """A frag matrix [rows, k] (flat fp16 storage of frag_pad(rows) * frag_pad(k)
    halfs).  Zero-filled by default: producers never write the K pad, and the
    frag GEMM needs it finite."""
    n = frag_pad(rows) * frag_pad(k)
    return (torch.zeros if zero else torch.empty)(n, dtype=torch.float16, device=device)


class GemmProblem(ctypes.Structure):
    _fields_ = [("a", _p), ("b", _p), ("c", _p), ("m", _i64), ("n", _i64), ("k", _i64),
                ("b_layout", _i), ("a_act", _i), ("epilogue", _i), ("v", _p), ("v_first", _p), ("v0", _p)]


class FragProblem(ctypes.Structure):
    _fields_ = [("a", _p), ("b", _p), ("c", _p), ("m", _i64), ("n", _i64), ("k", _i64),
                ("epilogue", _i), ("c_frag", _i), ("v", _p), ("v_first", _p), ("v0", _p)]


class LnShiftGroup(ctypes.Structure):
    _fields_ = [("row0", _i64), ("B", ctypes.c_int32), ("T", ctypes.c_int32), ("slots", _p)]


def _sig(name, args, res=_i):
    fn = getattr(_LIB, name)
    fn.argtypes = args
    fn.restype = res
    return fn


_LIB.vkwr_last_error.restype = ctypes.c_char_p
_gemm = _sig("vkwr_gemm_f16", [_i, ctypes.POINTER(GemmProblem), _p, _i64, _p])
_gemm_ws = _sig("vkwr_gemm_f16_workspace_bytes", [_i, ctypes.POINTER(GemmProblem)], _i64)
_ln_mix = _sig("vkwr_add_layer_norm_mix_f16",
               [_i64, _i, _p, _p, _p, _p, _p, _i, ctypes.POINTER(_p), _f, _p, ctypes.POINTER(_p), _p, _p, _i64, _i64,
                _p])
_ln_last = _sig("vkwr_add_last_layer_norm_f16", [_i, _i, _i, _p, _p, _p, _p, _f, _p, _p])
_ln = _sig("vkwr_layer_norm_f16", [_i64, _i, _p, _p, _p, _p, _f, _p, _p, _p])
_gate = _sig("vkwr_tmix_kk_a_gate_f16", [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_gn = _sig("vkwr_tmix_groupnorm_bonus_gate_f16", [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_wkv_slots = _sig("vkwr_wkv7_fp32_forward_slots",
                  [_i, _i, _i, _i, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_wkv_step_rows = _sig("vkwr_wkv7_fp32_step_rows_slots", [_i, _i, _i, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_frag_gemm = _sig("vkwr_frag_gemm_f16", [_i, ctypes.POINTER(FragProblem), _p])
_act = _sig("vkwr_activation_f16", [_i, _i64, _p, _p, _p])
ACT_EW_TANH, ACT_EW_SIGMOID = 1, 2  # vkwr_activation_f16 codes
_frag_splitk = _sig("vkwr_frag_gemm_splitk_f16", [ctypes.POINTER(FragProblem), _i, _p, _i64, _p])
_frag_splitk_parts = _sig("vkwr_frag_gemm_splitk_parts_f16", [ctypes.POINTER(FragProblem), _i, _p, _i64, _p])
_ln_mix_parts = _sig("vkwr_add_layer_norm_mix_parts_frag_f16",
                     [_i64, _i, _p, _i, _i64, _p, _p, _p, _p, _i, ctypes.POINTER(_p), _f, _p, ctypes.POINTER(_p), _p,
                      _i64, _p])
_frag_splitk_ws = _sig("vkwr_frag_gemm_splitk_workspace_bytes", [_i64, _i64, _i], _i64)
_frag_pack = _sig("vkwr_frag_pack_f16", [_i64, _i64, _p, _i, _p, _p])
_frag_unpack = _sig("vkwr_frag_unpack_f16", [_i64, _i64, _p, _p, _p])
_ln_mix_frag = _sig("vkwr_add_layer_norm_mix_frag_f16",
                    [_i64, _i, _p, _p, _p, _p, _p, _i, ctypes.POINTER(_p), _f, _p, ctypes.POINTER(_p), _p, _p, _i64,
                     _i64, _p])
_ln_last_frag = _sig("vkwr_add_last_layer_norm_frag_f16", [_i, _i, _i, _p, _p, _p, _p, _f, _p, _p])
_gn_frag = _sig("vkwr_tmix_groupnorm_bonus_gate_frag_f16", [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_wkv_fused = _sig("vkwr_wkv7_decode_fused_f16", [_i, _i, _i, _p, _i, _i, _p] + [_p] * 13 + [_i, _p])
_wkv_layout = _sig("vkwr_wkv7_state_layout_f32", [_i64, _p, _p, _i, _p])
WKV_STATE_STD, WKV_STATE_ILV = 0, 1
_ln_shift_rows = _sig("vkwr_add_layer_norm_shift_rows_f16",
                      [_i64, _i, _p, _p, _p, _p, _f, _p, _i, ctypes.POINTER(_p), ctypes.POINTER(_p), _p, _i64, _i,
                       ctypes.POINTER(LnShiftGroup), _p])
_shift = _sig("vkwr_token_shift_mix_f16", [_i, _i, _i, _p, _p, _i, ctypes.POINTER(_p), ctypes.POINTER(_p), _i, _p])
_shift_slots = _sig("vkwr_token_shift_mix_slots_f16",
                    [_i, _i, _i, _p, _p, _i64, _p, _i, ctypes.POINTER(_p), ctypes.POINTER(_p), _i, _p])
_d = ctypes.c_double
_samp_setup = _sig("vkwr_sampling_setup_rand", [_i64, _i, _p, _p])
_samp_temp = _sig("vkwr_sampling_temperature_topk_topp", [_i, _i, _i, _p, _p, _p, _p, _d, _i, _d, _p])
_samp_rep = _sig("vkwr_sampling_repetition_topk_topp",
                 [_i, _i, _i, _p, _p, _p, _p, _p, _d, _d, _d, _d, _i, _d, _p])
SAMPLING_STATE_BYTES = 32
SAMPLING_REGISTER_VOCAB = 65536  # larger vocabularies need a B*V fp32 scratch buffer


def _check(st, what):
    if st != 0:
        raise RuntimeError(f"{what}: {_LIB.vkwr_last_error().decode()}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _idx(t, n, what):
    """Pointer of an index tensor the kernels read as n int32 values (slot tables, row
    gathers): int32, on the GPU, contiguous, at least n entries.  An int64 tensor would be
    read as pairs of 32-bit words -- wrong and duplicated slots that still pass the
    kernels' range checks -- so anything else is refused here."""
    if t is None:
        return None
    if t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous() or t.numel() < n:
        raise TypeError(f"{what}: expected a contiguous int32 CUDA tensor of >= {n} entries, got "
                        f"{t.dtype} {t.device} shape {tuple(t.shape)} contiguous={t.is_contiguous()}")
    return ctypes.c_void_p(t.data_ptr())


def gemm_problem(a, b, c, b_layout=GEMM_B_NK, a_act=ACT_NONE, epilogue=EPI_NONE, v=None, v_first=None, v0=None):
    """c[m,n] = epilogue(act(a)[m,k] . B): a [m,k], c [m,n]; b [n,k] (NK) or [k,n] (KN)."""
    k = a.shape[-1]
    m = a.numel() // k if k else 0
    n = b.shape[0] if b_layout == GEMM_B_NK else b.shape[1]
    assert c.numel() == m * n and b.numel() == n * k, (tuple(a.shape), tuple(b.shape), tuple(c.shape))
    for t in (a, b, c, v, v_first, v0):
        assert t is None or (t.is_contiguous() and t.dtype == torch.float16)
    return GemmProblem(a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, b_layout, a_act, epilogue,
                       _ptr(v), _ptr(v_first), _ptr(v0))


def _arr(problems):
    assert 1 <= len(problems) <= MAX_GEMM_PROBLEMS
    return (GemmProblem * len(problems))(*problems)


def gemm_workspace_bytes(problems):
    n = _gemm_ws(len(problems), _arr(problems))
    if n < 0:
        raise RuntimeError(f"vkwr_gemm_f16_workspace_bytes: {_LIB.vkwr_last_error().decode()}")
    return n


def gemm_workspace_bytes_upto(problems):
    """The largest workspace one launch of `problems` needs when every problem's row count is
    replaced by the same R, over R = 1 .. the problems' common row count.  The GEMM plan (tile
    shape, K splits, the large-M kernel's split last round) is not monotone in the row count,
    so a buffer sized for the largest batch, or for a few row counts, can fall short at others."""
    arr = _arr(problems)
    rows = {int(p.m) for p in problems}
    assert len(rows) == 1, f"problems must share the row count (got {sorted(rows)})"
    best = 0
    for m in range(1, rows.pop() + 1):
        for i in range(len(problems)):
            arr[i].m = m
        n = _gemm_ws(len(problems), arr)
        if n < 0:
            raise RuntimeError(f"vkwr_gemm_f16_workspace_bytes: {_LIB.vkwr_last_error().decode()}")
        best = max(best, n)
    return best


def gemm(problems, workspace):
    """Runs 1..8 GEMMs in one launch; workspace is a uint8 CUDA tensor (may be empty)."""
    arr = _arr(problems)
    _check(_gemm(len(problems), arr, _ptr(workspace) if workspace.numel() else None, workspace.numel(),
                 _stream()), "vkwr_gemm_f16")


def add_layer_norm_mix(x, residual, shift_state, weight, bias, mixes, x_out, outs, eps=1e-5,
                       x_rows=None, shift_slots=None, frag=False):
    """frag=True: outs are frag matrices [rows, C] (see frag_empty).  x_rows gathers rows of x
    (bounded by x's row count), shift_slots rows of shift_state (bounded by its row count); an
    index out of range gives that row NaN outputs and leaves the shift state untouched."""
    rows = x_out.shape[0]
    C = x_out.shape[-1]
    mp = (_p * len(mixes))(*[m.data_ptr() for m in mixes])
    op = (_p * len(outs))(*[o.data_ptr() for o in outs])
    fn = _ln_mix_frag if frag else _ln_mix
    _check(fn(rows, C, _ptr(x), _ptr(residual), _ptr(shift_state), _ptr(weight), _ptr(bias), len(mixes),
              mp, eps, _ptr(x_out), op, _idx(x_rows, rows, "x_rows"), _idx(shift_slots, rows, "shift_slots"),
              x.numel() // C,
              shift_state.numel() // C, _stream()),
           "vkwr_add_layer_norm_mix%s_f16" % ("_frag" if frag else ""))


def layer_norm(x, weight, bias, y, eps=1e-5, residual=None, x_out=None):
    C = x.shape[-1]
    _check(_ln(x.numel() // C, C, _ptr(x), _ptr(residual), _ptr(weight), _ptr(bias), eps, _ptr(x_out), _ptr(y),
               _stream()), "vkwr_layer_norm_f16")


def add_last_layer_norm(B, T, C, x, residual, weight, bias, y, eps=1e-5, frag=False):
    fn = _ln_last_frag if frag else _ln_last
    _check(fn(B, T, C, _ptr(x), _ptr(residual), _ptr(weight), _ptr(bias), eps, _ptr(y), _stream()),
           "vkwr_add_last_layer_norm%s_f16" % ("_frag" if frag else ""))


def kk_a_gate(B, T, C, H, k, k_k, a0, a12, k_a, new_k, neg_kk, kka, x=None, shift_state=None):
    _check(_gate(B, T, C, H, _ptr(k), _ptr(k_k), _ptr(a0), _ptr(a12), _ptr(k_a), _ptr(x), _ptr(shift_state),
                 _ptr(new_k), _ptr(neg_kk), _ptr(kka), _stream()), "vkwr_tmix_kk_a_gate_f16")


def groupnorm_bonus_gate(B, T, C, H, x, r, k, v, r_k, weight, bias, g, out, frag=False):
    fn = _gn_frag if frag else _gn
    _check(fn(B, T, C, H, _ptr(x), _ptr(r), _ptr(k), _ptr(v), _ptr(r_k), _ptr(weight), _ptr(bias), _ptr(g),
              _ptr(out), _stream()), "vkwr_tmix_groupnorm_bonus_gate%s_f16" % ("_frag" if frag else ""))


def frag_pack(src, rows, k, dst, src_layout=GEMM_B_NK):
    """Pack src ([rows,k] row-major, or [k,rows] with GEMM_B_KN) into the frag matrix dst."""
    assert src.dtype == torch.float16 and src.is_contiguous() and src.numel() == rows * k
    assert dst.numel() >= frag_pad(rows) * frag_pad(k)
    _check(_frag_pack(rows, k, _ptr(src), src_layout, _ptr(dst), _stream()), "vkwr_frag_pack_f16")


def frag_unpack(src, rows, k, dst):
    assert dst.numel() == rows * k and dst.is_contiguous()
    _check(_frag_unpack(rows, k, _ptr(src), _ptr(dst), _stream()), "vkwr_frag_unpack_f16")


def frag_problem(a, b, c, m, n, k, epilogue=EPI_NONE, c_frag=False, v=None, v_first=None, v0=None):
    """One frag GEMM: c = epilogue(a . b^T); a frag [m,k], b frag [n,k]; c row-major [m,n] or frag."""
    assert a.numel() >= frag_pad(m) * frag_pad(k), (a.numel(), m, k)
    assert b.numel() >= frag_pad(n) * frag_pad(k), (b.numel(), n, k)
    assert c.numel() >= (frag_pad(m) * frag_pad(n) if c_frag else m * n)
    return FragProblem(a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, epilogue, 1 if c_frag else 0,
                       _ptr(v), _ptr(v_first), _ptr(v0))


def frag_gemm(problems):
    """Runs 1..8 frag GEMMs in one launch."""
    arr = _arr_frag(problems)
    _check(_frag_gemm(len(problems), arr, _stream()), "vkwr_frag_gemm_f16")


def activation(act, x, out):
    """out = act(x) elementwise (ACT_EW_TANH / ACT_EW_SIGMOID); out may be x."""
    _check(_act(act, x.numel(), _ptr(x), _ptr(out), _stream()), "vkwr_activation_f16")


def frag_splitk_workspace_bytes(m, n, splits):
    """Workspace bytes vkwr_frag_gemm_splitk_f16 needs for an [m, n] output in `splits` K parts."""
    return _frag_splitk_ws(m, n, splits)


def frag_gemm_splitk(problem, splits, workspace):
    """One frag GEMM with K split over `splits` workgroups per 64x64 tile (fp32 partials in
    `workspace`, a CUDA tensor of at least frag_splitk_workspace_bytes bytes, then an ordered reduce
    that applies the epilogue)."""
    nbytes = workspace.numel() * workspace.element_size()
    _check(_frag_splitk(ctypes.byref(problem), splits, workspace.data_ptr(), nbytes, _stream()),
           "vkwr_frag_gemm_splitk_f16")


def frag_gemm_splitk_parts(problem, splits, workspace):
    """The partial planes of frag_gemm_splitk alone (epilogue NONE, row-major, c unused): plane q
    starts at float q * splitk_plane_floats(m, n), row stride frag_pad(n)."""
    nbytes = workspace.numel() * workspace.element_size()
    _check(_frag_splitk_parts(ctypes.byref(problem), splits, workspace.data_ptr(), nbytes, _stream()),
           "vkwr_frag_gemm_splitk_parts_f16")


def splitk_plane_floats(m, n):
    """Floats between consecutive partial planes of a K-split frag GEMM."""
    return (m + 63) // 64 * 64 * frag_pad(n)


def add_layer_norm_mix_parts(x_parts, n_parts, part_stride, residual, shift_state, weight, bias, mixes, x_out,
                             outs, eps=1e-5, shift_slots=None):
    """add_layer_norm_mix(frag=True) whose x is n_parts fp32 K-part planes (x_parts, a CUDA float
    tensor; plane stride part_stride floats, row stride C)."""
    rows = x_out.shape[0]
    C = x_out.shape[-1]
    mp = (_p * len(mixes))(*[m.data_ptr() for m in mixes])
    op = (_p * len(outs))(*[o.data_ptr() for o in outs])
    _check(_ln_mix_parts(rows, C, _ptr(x_parts), n_parts, part_stride, _ptr(residual), _ptr(shift_state),
                         _ptr(weight), _ptr(bias), len(mixes), mp, eps, _ptr(x_out), op,
                         _idx(shift_slots, rows, "shift_slots"),
                         shift_state.numel() // C, _stream()), "vkwr_add_layer_norm_mix_parts_frag_f16")


def _arr_frag(problems):
    assert 1 <= len(problems) <= MAX_GEMM_PROBLEMS
    return (FragProblem * len(problems))(*problems)


def wkv_slots(B, T, C, H, pool, slots, r, w, k, v, a, b, y):
    _check(_wkv_slots(B, T, C, H, _ptr(pool), pool.shape[0], _idx(slots, B, "slots"), _ptr(r), _ptr(w), _ptr(k),
                      _ptr(v),
                      _ptr(a), _ptr(b), _ptr(y), _stream()), "vkwr_wkv7_fp32_forward_slots")


def wkv_step_rows_slots(B, C, H, pool, slots, r, w, k, v, a, b, y):
    """One decode step on the slot pool in the row-split dot-product order, without LDS
    (vkwr_wkv7_fp32_step_rows_slots)."""
    _check(_wkv_step_rows(B, C, H, _ptr(pool), pool.shape[0], _idx(slots, B, "slots"), _ptr(r), _ptr(w), _ptr(k),
                          _ptr(v),
                          _ptr(a), _ptr(b), _ptr(y), _stream()), "vkwr_wkv7_fp32_step_rows_slots")


def wkv_decode_fused(B, C, H, pool, slots, r, w, k, v, a12, g, k_k, a0, k_a, r_k, ln_w, ln_b, out, frag=False,
                     state_layout=WKV_STATE_STD):
    """gate -> WKV-7 (slot pool, T = 1) -> GroupNorm + bonus + gate in one launch."""
    _check(_wkv_fused(B, C, H, _ptr(pool), pool.shape[0], state_layout, _idx(slots, B, "slots"), _ptr(r), _ptr(w),
                      _ptr(k), _ptr(v),
                      _ptr(a12), _ptr(g), _ptr(k_k), _ptr(a0), _ptr(k_a), _ptr(r_k), _ptr(ln_w), _ptr(ln_b),
                      _ptr(out), 1 if frag else 0, _stream()), "vkwr_wkv7_decode_fused_f16")


def wkv_state_layout(src, dst, to_layout):
    """Copies fp32 state blocks (src, dst: [..., 64, 64] views of the same shape) into layout to_layout."""
    assert src.shape == dst.shape and src.dtype == dst.dtype == torch.float32 and src.numel() % 4096 == 0
    _check(_wkv_layout(src.numel() // 4096, _ptr(src), _ptr(dst), to_layout, _stream()), "vkwr_wkv7_state_layout_f32")


LN_SHIFT_MAX_GROUPS = 8  # groups per vkwr_add_layer_norm_shift_rows_f16 launch


def layer_norm_shift_rows(x, weight, bias, x_out, mixes, outs, shift_state, groups, residual=None, eps=1e-5):
    """x_out = x + residual, y = LN(x_out), and per group (row0, B, T, slots [B] int32) the
    token-shift lerps of y into outs against the shift pool shift_state [P, C]: one launch
    of vkwr_add_layer_norm_shift_rows_f16 per 8 groups.  x, residual, x_out, outs [rows, C];
    the groups cover rows 0 .. rows - 1 in order."""
    C = x.shape[-1]
    rows = x.numel() // C
    if len(groups) > LN_SHIFT_MAX_GROUPS:
        # one launch per run of 8 groups, on the rows they cover (groups never share a row)
        for i in range(0, len(groups), LN_SHIFT_MAX_GROUPS):
            part = groups[i:i + LN_SHIFT_MAX_GROUPS]
            a = part[0][0]
            e = part[-1][0] + part[-1][1] * part[-1][2]
            rb = lambda t: None if t is None else t.view(rows, C)[a:e]  # noqa: E731
            layer_norm_shift_rows(rb(x), weight, bias, rb(x_out), mixes, [rb(o) for o in outs], shift_state,
                                  [(r0 - a, B, T, sl) for r0, B, T, sl in part], residual=rb(residual), eps=eps)
        return
    mp = (_p * len(mixes))(*[m.data_ptr() for m in mixes])
    op = (_p * len(outs))(*[o.data_ptr() for o in outs])
    gs = (LnShiftGroup * len(groups))(*[LnShiftGroup(r0, B, T, _idx(sl, B, "group slots"))
                                        for r0, B, T, sl in groups])
    _check(_ln_shift_rows(rows, C, _ptr(x), _ptr(residual), _ptr(weight), _ptr(bias), eps, _ptr(x_out), len(mixes),
                          mp, op, _ptr(shift_state), shift_state.numel() // C, len(groups), gs, _stream()),
           "vkwr_add_layer_norm_shift_rows_f16")


def token_shift(B, T, C, x, shift_state, mixes, outs, half_math=False, shift_slots=None):
    """Token-shift lerp of [B,T,C] x; shift_state [B,C], or a pool [P,C] indexed by shift_slots [B]."""
    mp = (_p * len(mixes))(*[m.data_ptr() for m in mixes])
    op = (_p * len(outs))(*[o.data_ptr() for o in outs])
    if shift_slots is None:
        _check(_shift(B, T, C, _ptr(x), _ptr(shift_state), len(mixes), mp, op, 1 if half_math else 0, _stream()),
               "vkwr_token_shift_mix_f16")
    else:
        _check(_shift_slots(B, T, C, _ptr(x), _ptr(shift_state), shift_state.numel() // C,
                            _idx(shift_slots, B, "shift_slots"),
                            len(mixes), mp, op, 1 if half_math else 0, _stream()), "vkwr_token_shift_mix_slots_f16")


def sampling_setup_rand(seed, states):
    """Initialises states (int8/uint8 tensor of B * SAMPLING_STATE_BYTES bytes) for B rows."""
    B = states.numel() // SAMPLING_STATE_BYTES
    _check(_samp_setup(seed, B, _ptr(states), _stream()), "vkwr_sampling_setup_rand")


def sample(logits, states, out, temperature=1.0, top_k=-1, top_p=1.0, penalties=None, presence=0.0,
           repetition=0.0, decay=1.0, scratch=None):
    """One token per row of fp32 logits [B, V] (or [B, T, V]: last token) into out [B] int32;
    with penalties [B, V] the repetition variant (penalties updated in place).  scratch
    (B*V fp32) is needed only above SAMPLING_REGISTER_VOCAB."""
    B, V = out.shape[0], logits.shape[-1]
    T = logits.shape[1] if logits.dim() == 3 else 1
    assert logits.dtype == torch.float32 and logits.is_contiguous() and logits.numel() == B * T * V
    assert out.dtype == torch.int32 and states.numel() * states.element_size() >= B * SAMPLING_STATE_BYTES
    assert penalties is None or (penalties.dtype == torch.float32 and penalties.is_contiguous()
                                 and penalties.numel() == B * V)
    assert scratch is None or (scratch.dtype == torch.float32 and scratch.numel() >= B * V)
    if penalties is None:
        st = _samp_temp(B, T, V, _ptr(logits), _ptr(states), _ptr(out), _ptr(scratch), temperature, top_k, top_p,
                        _stream())
        _check(st, "vkwr_sampling_temperature_topk_topp")
    else:
        st = _samp_rep(B, T, V, _ptr(logits), _ptr(penalties), _ptr(states), _ptr(out), _ptr(scratch), presence,
                       repetition, decay, temperature, top_k, top_p, _stream())
        _check(st, "vkwr_sampling_repetition_topk_topp")
