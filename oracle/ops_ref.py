"""CPU oracle (numpy, float64) for the LayerNorm / GroupNorm / token-shift /
gate / activation ops of the RWKV-7 hot path -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may use this module; the product (``vkwr``, ``vkwr_amd``) never does.

Each function restates the arithmetic of the reference kernel it names (paths
relative to the reference root) in float64 and rounds to fp16 at the points
where the reference rounds; intermediate fp32 rounding of the reference is not
emulated (the GPU comparisons are tolerance-based, see tests/).  Inputs and
outputs are numpy arrays; fp16 tensors are ``np.float16``.
"""
import numpy as np

F64 = np.float64
F16 = np.float16

KK_EPS = 1.0e-12          # csrc/v1/mix/mix_ops.cu:17
GROUPNORM_EPS = 64.0e-5   # csrc/v1/mix/mix_ops.cu:18


def _f(x):
    return np.asarray(x).astype(F64)


def sigmoid(x):
    x = _f(x)
    return 1.0 / (1.0 + np.exp(-x))


def layer_norm(x, weight, bias, eps=1e-5, residual=None):
    """Two-pass LayerNorm over the last axis (norm_ops.cu:74-110); with a
    residual, v = x + residual and the statistics use the unrounded v
    (norm_ops.cu:112-153).  Returns (x_out = fp16(v) or None, y fp16)."""
    v = _f(x) if residual is None else _f(x) + _f(residual)
    mean = v.mean(axis=-1, keepdims=True)
    var = ((v - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (v - mean) / np.sqrt(var + eps) * _f(weight) + _f(bias)
    return (None if residual is None else v.astype(F16)), y.astype(F16)


def add_last_layer_norm(x, residual, weight, bias, eps=1e-5):
    """LN of the last token only (norm_ops.cu:602-733): [B,T,C] -> [B,C]."""
    return layer_norm(x[:, -1], weight, bias, eps, residual=residual[:, -1])[1]


def emb_ln0(emb_bf16_bits, weight_bits, bias_bits, eps=1e-5):
    """bf16 table -> LN -> fp16 (norm_ops.cu:26-59).  Arguments are uint16 bf16 bit patterns."""
    def bf(b):
        return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32).astype(F64)
    return layer_norm(bf(emb_bf16_bits), bf(weight_bits), bf(bias_bits), eps)[1]


def lerp16(cur16, prev16, mix16):
    """fp16(cur + (prev - cur) * mix) from fp16 operands (mix_ops.cu:84-96)."""
    c = _f(cur16)
    return (c + (_f(prev16) - c) * _f(mix16)).astype(F16)


def lerp16_half_math(cur16, prev16, mix16):
    """half_math path (mix_ops.cu:124-131): dx = fp16(prev - cur) then one fp16 FMA."""
    dx = (_f(prev16) - _f(cur16)).astype(F16)
    return (_f(dx) * _f(mix16) + _f(cur16)).astype(F16)  # exact product + sum, one rounding


def add_layer_norm_mix(x, residual, shift_state, weight, bias, mixes, eps=1e-5):
    """Decode fusion (norm_ops.cu:317-600): x_out = fp16(x+res); y = fp16(LN(x+res));
    outputs lerp(y, prev=shift_state); shift_state := y (in place).
    x, residual [B,1,C]; shift_state [B,C].  Returns [x_out, *outs]."""
    x_out, y = layer_norm(x, weight, bias, eps, residual=residual)
    prev = shift_state.reshape(y.shape).copy()
    outs = [lerp16(y, prev, m) for m in mixes]
    shift_state[...] = y.reshape(shift_state.shape)
    return [x_out] + outs


def token_shift(x, shift_state, mixes, half_math=False):
    """Token-shift lerp over T tokens (mix_ops.cu:42-102, 104-160, 432-462) with
    prev at t = 0 the entry value of shift_state; shift_state := x[:, T-1] (in place).
    x [B,T,C]; shift_state [B,C]."""
    prev = np.concatenate([shift_state[:, None, :], x[:, :-1, :]], axis=1)
    f = lerp16_half_math if half_math else lerp16
    outs = [f(x, prev, m) for m in mixes]
    shift_state[...] = x[:, -1, :]
    return outs


def kk_a_gate(k, k_k, a0, a12, k_a, H):
    """tmix_kk_a_gate (mix_ops.cu:162-211).  k, a12 [B,T,C]; vectors [C].
    Returns (new_k, neg_kk, kka) fp16."""
    B, T, C = k.shape
    u = (_f(k) * _f(k_k)).reshape(B, T, H, 64)
    norm = np.sqrt((u * u).sum(-1, keepdims=True))
    kk = (u / np.maximum(norm, KK_EPS)).reshape(B, T, C)
    a = sigmoid(_f(a0) + _f(a12))
    ka = _f(k_a)
    new_k = _f(k) * (a * ka + (1.0 - ka))
    return new_k.astype(F16), (-kk).astype(F16), (kk * a).astype(F16)


def groupnorm_bonus_gate(x, r, k, v, r_k, weight, bias, g, H):
    """tmix_lnx_rkvres_xg (mix_ops.cu:213-276): per-head GroupNorm (eps 64e-5),
    plus (sum_head r*k*r_k) * v, times g."""
    B, T, C = x.shape
    xh = _f(x).reshape(B, T, H, 64)
    mean = xh.mean(-1, keepdims=True)
    var = ((xh - mean) ** 2).mean(-1, keepdims=True)
    xn = ((xh - mean) / np.sqrt(var + GROUPNORM_EPS)).reshape(B, T, C)
    rkv = (_f(r) * _f(k) * _f(r_k)).reshape(B, T, H, 64).sum(-1, keepdims=True)
    bonus = (rkv * _f(v).reshape(B, T, H, 64)).reshape(B, T, C)
    return ((xn * _f(weight) + _f(bias) + bonus) * _f(g)).astype(F16)


def vres_gate(v, v_first, v0, v12):
    """tmix_vres_gate (mix_ops.cu:278-294): v + (v_first - v) * sigmoid(v0 + v12)."""
    vv = _f(v)
    return (vv + (_f(v_first) - vv) * sigmoid(_f(v0) + _f(v12))).astype(F16)


def relu_square(x):
    r = np.maximum(_f(x), 0.0)
    return (r * r).astype(F16)


def act_tanh(x):
    return np.tanh(_f(x)).astype(F16)


def act_sigmoid(x):
    return sigmoid(x).astype(F16)


def add_vec(x, vec):
    return (_f(x) + _f(vec)).astype(F16)


def add16(x, y):
    return (_f(x) + _f(y)).astype(F16)


def ulp16(x):
    """Spacing of fp16 at |x| (at least the subnormal quantum 2^-24)."""
    a = np.abs(np.asarray(x, dtype=F64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.maximum(2.0 ** (e - 10), 2.0 ** -24)


# ---------------------------------------------------------------- GEMMs

def _act(x, act):
    if act == "tanh":
        return np.tanh(x)
    if act == "sigmoid":
        return sigmoid(x)
    if act == "relu2":
        r = np.maximum(x, 0.0)
        return r * r
    return x


def gemm(a, b, b_layout="nk", a_act=None, epi=None, v=None, v_first=None, v0=None, round_act=True):
    """fp16 GEMM with fp32-or-better accumulation, restated in float64
    (reference csrc/v1/linear/linear_ops.cu:1001-1011 cuBLAS fp16 in / fp32
    compute / fp16 out; rank adapters csrc/v1/rank/rank_ops.cu:16-333).
    b is [N,K] ("nk", y = a.b^T) or [K,N] ("kn", y = a.b).  a_act in
    {None, "tanh", "sigmoid", "relu2"} is applied to a elementwise and, with
    round_act, rounded to fp16 (the reference keeps it in fp32 for the rank
    adapters and rounds it for the sparse FFN).  epi in {None, "relu2",
    "vres"}.  Returns (y fp16, abs_sum) where abs_sum = sum_k |a_k b_k| bounds
    the accumulation error."""
    a64 = _act(_f(a), a_act)
    if a_act is not None and round_act:
        a64 = a64.astype(F16).astype(F64)
    w = _f(b)
    wt = w.T if b_layout == "nk" else w
    y = a64 @ wt
    abs_sum = np.abs(a64) @ np.abs(wt)
    if epi == "relu2":
        r = np.maximum(y, 0.0)
        y = r * r
    elif epi == "vres":
        vv = _f(v)
        y = vv + (_f(v_first) - vv) * sigmoid(_f(v0) + y)
    return y.astype(F16), abs_sum


def cmix_sparse(x, shift_state, x_k, key_fc, value_fc):
    """Channel mix (reference csrc/v1/mix/mix_ops.cu:296-863): mixed = lerp(x, prev);
    act = fp16(relu(mixed . key_fc^T)^2); out = act . value_fc; shift_state := x[:, T-1].
    The mixed input is rounded to fp16 first (as this build's token-shift op does).
    x [B,T,C]; shift_state [B,C] (in place); key_fc, value_fc [F,C]."""
    B, T, C = x.shape
    mixed = token_shift(x, shift_state, [x_k])[0].reshape(B * T, C)
    act, _ = gemm(mixed, key_fc, "nk", epi="relu2")
    out, abs_sum = gemm(act, value_fc, "kn")
    return out.reshape(B, T, C), act, abs_sum.reshape(B, T, C)
