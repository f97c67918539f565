"""End-to-end oracle of the RWKV-7 decode step -- test infrastructure only.

A plain torch float32 restatement of the layer composition that
vkwr.model_executor.rwkv7 runs on the HIP kernels.  The reference ships no
model code (its vkwr/model_executor is empty); the composition follows its op
contracts and test docstrings (reference tests/ops/test_v1_wkv_ops.py:74-96:
r: LN -> mix -> linear; w: -> linear -> tanh -> linear; a = -kk;
b = kk * sigmoid(a0 + a12)) and the op semantics of csrc/v1/norm/norm_ops.cu,
csrc/v1/mix/mix_ops.cu, csrc/v1/rank/rank_ops.cu and csrc/v1/wkv/wkv_fp32_v2.cu
cited per function below.

Each stage is a function of its own so the tests can pin it against the
numpy / C oracle functions that restate the same reference kernel
(oracle/ops_ref.py, oracle/wkv_oracle.c); decode_step only wires them.
Runs on any torch device.  With round_fp16=True every stage output is rounded
to fp16 where the GPU path stores fp16, so the comparison isolates the kernels'
arithmetic; with round_fp16=False it is the float32 model the fp16 pipeline
approximates.  The recurrent state (wkv fp32 [L,P,H,64,64], att_shift /
ffn_shift [L,P,C]) is updated in place like the engine's.
"""
import math

import torch
import torch.nn.functional as F

E_HALF = math.exp(-0.5)
TMIX = ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g")


def _r(x, on):
    return x.half().float() if on else x


def add_layer_norm(x, res, w, b, rd, eps=1e-5):
    """x_out = fp16(x + res); y = fp16(LN(x + res)) with the statistics of the unrounded sum
    (reference norm_ops.cu:112-153, 317-378).  Returns (x_out, y)."""
    s = x + res
    return _r(s, rd), _r(F.layer_norm(s, (s.shape[-1],), w, b, eps), rd)


def lerp(cur, prev, mix, rd):
    """Token-shift lerp cur + (prev - cur) * mix (reference mix_ops.cu:84-96)."""
    return _r(cur + (prev - cur) * mix, rd)


def kk_a_gate(k, k_k, a0, a12, k_a, H, rd):
    """kk = normalize(k * k_k) per head (eps 1e-12), a = sigmoid(a0 + a12),
    new_k = k * (a * k_a + 1 - k_a); returns (new_k, -kk, kk * a) (reference
    mix_ops.cu:162-211)."""
    B, C = k.shape
    kk = F.normalize((k * k_k).view(B, H, 64), dim=-1, eps=1e-12).reshape(B, C)
    a = torch.sigmoid(a0 + a12)
    return _r(k * (a * k_a + (1 - k_a)), rd), _r(-kk, rd), _r(kk * a, rd)


def decay(w):
    """exp(-e^{-1/2} sigmoid(w)) (reference wkv_fp32_v2.cu:27-29)."""
    return torch.exp(-E_HALF * torch.sigmoid(w))


def wkv7(S, r, w, k, v, a, b, rd):
    """One WKV-7 token per (sequence, head) on gathered states S [B,H,64,64] (S[i][j], i the
    value index): S' = S diag(d) + (S a) b^T + v k^T, y = S' r (reference wkv_fp32_v2.cu:93-118).
    Returns (y [B,C], S')."""
    B, H = S.shape[:2]
    d = decay(w).view(B, H, 1, 64)
    sa = torch.matmul(S, a.view(B, H, 64, 1))
    S = S * d + sa * b.view(B, H, 1, 64) + v.view(B, H, 64, 1) * k.view(B, H, 1, 64)
    y = _r(torch.matmul(S, r.view(B, H, 64, 1)).reshape(B, H * 64), rd)
    return y, S


def groupnorm_bonus_gate(y, r, k, v, r_k, w, b, g, H, rd):
    """((GroupNorm_head(y) * w + b) + (sum_head r k r_k) v) * g, GroupNorm eps 64e-5
    (reference mix_ops.cu:213-276)."""
    B, C = y.shape
    yh = y.view(B, H, 64)
    mean = yh.mean(-1, keepdim=True)
    var = ((yh - mean) ** 2).mean(-1, keepdim=True)
    yn = ((yh - mean) / torch.sqrt(var + 64e-5)).reshape(B, C)
    bonus = (r * k * r_k).view(B, H, 64).sum(-1, keepdim=True) * v.view(B, H, 64)
    return _r((yn * w + b + bonus.reshape(B, C)) * g, rd)


def linear(x, W, rd):
    """x W^T with W in nn.Linear layout [out, in] (fp16 GEMM semantics, reference
    linear_ops.cu:1001-1011)."""
    return _r(x @ W.t(), rd)


def time_mix(W, x, res, att_prev, S, v_first, first, H, rd):
    """One layer's time mix.  x: previous block output; res: residual stream; att_prev: the
    layer's shift rows of these sequences; S: their WKV states.  Returns
    (res', o, new shift rows, S', v_first)."""
    res, xx = add_layer_norm(x, res, W["ln1_w"], W["ln1_b"], rd)
    xr, xw, xk, xv, xa, xg = (lerp(xx, att_prev, W[m], rd) for m in TMIX)
    r, k, v = linear(xr, W["Wr"], rd), linear(xk, W["Wk"], rd), linear(xv, W["Wv"], rd)
    w = _r(W["w0"] + linear(_r(torch.tanh(linear(xw, W["w1"], rd)), rd), W["w2"], False), rd)
    a12 = linear(linear(xa, W["a1"], rd), W["a2"], rd)
    g = linear(_r(torch.sigmoid(linear(xg, W["g1"], rd)), rd), W["g2"], rd)
    if first:
        v_first = v
    else:  # value residual (reference rank_ops.cu:145-333, linear_t_vres_f16)
        v12 = linear(xv, W["v1"], rd) @ W["v2"].t()
        v = _r(v + (v_first - v) * torch.sigmoid(W["v0"] + v12), rd)
    new_k, neg_kk, kka = kk_a_gate(k, W["k_k"], W["a0"], a12, W["k_a"], H, rd)
    y, S = wkv7(S, r, w, new_k, v, neg_kk, kka, rd)
    o_in = groupnorm_bonus_gate(y, r, new_k, v, W["r_k"], W["lnx_w"], W["lnx_b"], g, H, rd)
    return res, linear(o_in, W["Wo"], rd), xx, S, v_first


def channel_mix(W, o, res, ffn_prev, rd):
    """One layer's channel mix: res' = o + res; x = relu(lerp(LN2(res'), prev) K^T)^2 V^T.
    Returns (res', x, new shift rows)."""
    res, xx = add_layer_norm(o, res, W["ln2_w"], W["ln2_b"], rd)
    xk = lerp(xx, ffn_prev, W["x_k_ffn"], rd)
    act = _r(torch.relu(xk @ W["key"].t()) ** 2, rd)
    return res, linear(act, W["value"], rd), xx


def decode_step(model, wkv, att_shift, ffn_shift, tokens, slots, round_fp16=True):
    """model: an RWKV7Model-like object (cfg, layers, emb, ln_out_w/b, head; fp16 weights,
    converted here); tokens, slots: int tensors [B].  Returns float32 logits [B, V]."""
    cfg = model.cfg
    dev = wkv.device
    H = cfg.n_head
    f = lambda t: t.to(dev).float()  # noqa: E731
    tok = tokens.to(dev).long()
    sl = slots.to(dev).long()
    rd = round_fp16
    x = f(model.emb)[tok]                      # LN0'd embedding rows
    res = torch.zeros_like(x)
    v_first = None
    for l, L in enumerate(model.layers):
        W = {k: f(v) for k, v in L.items()}
        res, o, xx, S, v_first = time_mix(W, x, res, att_shift[l, sl].float(), wkv[l, sl].clone(), v_first,
                                          l == 0, H, rd)
        att_shift[l, sl] = xx.to(att_shift.dtype)
        wkv[l, sl] = S
        res, x, xx2 = channel_mix(W, o, res, ffn_shift[l, sl].float(), rd)
        ffn_shift[l, sl] = xx2.to(ffn_shift.dtype)
    h = _r(F.layer_norm(x + res, (x.shape[-1],), f(model.ln_out_w), f(model.ln_out_b), 1e-5), rd)
    return h @ f(model.head).t()
