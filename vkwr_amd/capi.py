"""ctypes binding of the C ABI (include/vkwr_amd.h) for the model executor.

The reference-compatible torch ops (vkwr_amd._ops) cover the reference's op
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

from vkwr_amd._ops._load import load_ext

load_ext("_v1_wkv_C")  # the extension modules link (and so load) the kernel library
_LIB = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "libvkwr_amd.so"))

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

GEMM_B_NK, GEMM_B_KN = 0, 1
ACT_NONE, ACT_TANH, ACT_SIGMOID, ACT_RELU_SQUARE = 0, 1, 2, 3
EPI_NONE, EPI_RELU_SQUARE, EPI_VALUE_RESIDUAL, EPI_BIAS = 0, 1, 2, 3
MAX_GEMM_PROBLEMS = 8


class GemmProblem(ctypes.Structure):
    _fields_ = [("a", _p), ("b", _p), ("c", _p), ("m", _i64), ("n", _i64), ("k", _i64),
                ("b_layout", _i), ("a_act", _i), ("epilogue", _i), ("v", _p), ("v_first", _p), ("v0", _p)]


def _sig(name, args, res=_i):
    fn = getattr(_LIB, name)
    fn.argtypes = args
    fn.restype = res
    return fn


_LIB.vkwr_last_error.restype = ctypes.c_char_p
_gemm = _sig("vkwr_gemm_f16", [_i, ctypes.POINTER(GemmProblem), _p, _i64, _p])
_gemm_ws = _sig("vkwr_gemm_f16_workspace_bytes", [_i, ctypes.POINTER(GemmProblem)], _i64)
_ln_mix = _sig("vkwr_add_layer_norm_mix_f16",
               [_i64, _i, _p, _p, _p, _p, _p, _i, ctypes.POINTER(_p), _f, _p, ctypes.POINTER(_p), _p, _p, _p])
_ln_last = _sig("vkwr_add_last_layer_norm_f16", [_i, _i, _i, _p, _p, _p, _p, _f, _p, _p])
_ln = _sig("vkwr_layer_norm_f16", [_i64, _i, _p, _p, _p, _p, _f, _p, _p, _p])
_gate = _sig("vkwr_tmix_kk_a_gate_f16", [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_gn = _sig("vkwr_tmix_groupnorm_bonus_gate_f16", [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_wkv_slots = _sig("vkwr_wkv7_fp32_forward_slots",
                  [_i, _i, _i, _i, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p])
_shift = _sig("vkwr_token_shift_mix_f16", [_i, _i, _i, _p, _p, _i, ctypes.POINTER(_p), ctypes.POINTER(_p), _i, _p])


def _check(st, what):
    if st != 0:
        raise RuntimeError(f"{what}: {_LIB.vkwr_last_error().decode()}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


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


def gemm(problems, workspace):
    """Runs 1..8 GEMMs in one launch; workspace is a uint8 CUDA tensor (may be empty)."""
    arr = _arr(problems)
    _check(_gemm(len(problems), arr, _ptr(workspace) if workspace.numel() else None, workspace.numel(),
                 _stream()), "vkwr_gemm_f16")


def add_layer_norm_mix(x, residual, shift_state, weight, bias, mixes, x_out, outs, eps=1e-5,
                       x_rows=None, shift_slots=None):
    rows = x_out.shape[0]
    C = x_out.shape[-1]
    mp = (_p * len(mixes))(*[m.data_ptr() for m in mixes])
    op = (_p * len(outs))(*[o.data_ptr() for o in outs])
    _check(_ln_mix(rows, C, _ptr(x), _ptr(residual), _ptr(shift_state), _ptr(weight), _ptr(bias), len(mixes),
                   mp, eps, _ptr(x_out), op, _ptr(x_rows), _ptr(shift_slots), _stream()),
           "vkwr_add_layer_norm_mix_f16")


def layer_norm(x, weight, bias, y, eps=1e-5, residual=None, x_out=None):
    C = x.shape[-1]
    _check(_ln(x.numel() // C, C, _ptr(x), _ptr(residual), _ptr(weight), _ptr(bias), eps, _ptr(x_out), _ptr(y),
               _stream()), "vkwr_layer_norm_f16")


def add_last_layer_norm(B, T, C, x, residual, weight, bias, y, eps=1e-5):
    _check(_ln_last(B, T, C, _ptr(x), _ptr(residual), _ptr(weight), _ptr(bias), eps, _ptr(y), _stream()),
           "vkwr_add_last_layer_norm_f16")


def kk_a_gate(B, T, C, H, k, k_k, a0, a12, k_a, new_k, neg_kk, kka, x=None, shift_state=None):
    _check(_gate(B, T, C, H, _ptr(k), _ptr(k_k), _ptr(a0), _ptr(a12), _ptr(k_a), _ptr(x), _ptr(shift_state),
                 _ptr(new_k), _ptr(neg_kk), _ptr(kka), _stream()), "vkwr_tmix_kk_a_gate_f16")


def groupnorm_bonus_gate(B, T, C, H, x, r, k, v, r_k, weight, bias, g, out):
    _check(_gn(B, T, C, H, _ptr(x), _ptr(r), _ptr(k), _ptr(v), _ptr(r_k), _ptr(weight), _ptr(bias), _ptr(g),
               _ptr(out), _stream()), "vkwr_tmix_groupnorm_bonus_gate_f16")


def wkv_slots(B, T, C, H, pool, slots, r, w, k, v, a, b, y):
    _check(_wkv_slots(B, T, C, H, _ptr(pool), pool.shape[0], _ptr(slots), _ptr(r), _ptr(w), _ptr(k), _ptr(v),
                      _ptr(a), _ptr(b), _ptr(y), _stream()), "vkwr_wkv7_fp32_forward_slots")


def token_shift(B, T, C, x, shift_state, mixes, outs, half_math=False):
    mp = (_p * len(mixes))(*[m.data_ptr() for m in mixes])
    op = (_p * len(outs))(*[o.data_ptr() for o in outs])
    _check(_shift(B, T, C, _ptr(x), _ptr(shift_state), len(mixes), mp, op, 1 if half_math else 0, _stream()),
           "vkwr_token_shift_mix_f16")
