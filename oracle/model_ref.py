"""End-to-end oracle of the RWKV-7 decode step -- test infrastructure only.

A plain torch float32 restatement of the layer composition that
vkwr.model_executor.rwkv7 runs on the HIP kernels (the reference ships no
model code; the composition follows its op contracts, see that module's
docstring).  Runs on any torch device.  With round_fp16=True every op output
is rounded to fp16 where the GPU path stores fp16, so the comparison isolates
the kernels' arithmetic; with round_fp16=False it is the float32 model the
fp16 pipeline approximates.  The recurrent state (wkv fp32 [L,P,H,64,64],
att_shift / ffn_shift [L,P,C]) is updated in place like the engine's.
"""
import math

import torch
import torch.nn.functional as F

E_HALF = math.exp(-0.5)


def _r(x, on):
    return x.half().float() if on else x


def _ln(x, w, b, eps=1e-5):
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def decode_step(model, wkv, att_shift, ffn_shift, tokens, slots, round_fp16=True):
    """model: vkwr.model_executor.rwkv7.RWKV7Model (fp16 weights, converted here);
    tokens, slots: int tensors [B].  Returns float32 logits [B, V]."""
    cfg = model.cfg
    dev = wkv.device
    H, C = cfg.n_head, cfg.n_embd
    f = lambda t: t.to(dev).float()  # noqa: E731
    tok = tokens.to(dev).long()
    sl = slots.to(dev).long()
    B = tok.shape[0]
    rd = round_fp16
    x = f(model.emb)[tok]                      # LN0'd embedding rows
    res = torch.zeros_like(x)
    v_first = None
    for l, L in enumerate(model.layers):
        W = {k: f(v) for k, v in L.items()}
        res = _r(x + res, rd)
        xx = _r(_ln(res, W["ln1_w"], W["ln1_b"]), rd)
        prev = att_shift[l, sl].float()
        mixes = [_r(xx + (prev - xx) * W[k], rd) for k in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g")]
        att_shift[l, sl] = xx.to(att_shift.dtype)
        xr, xw, xk, xv, xa, xg = mixes
        r = _r(xr @ W["Wr"].t(), rd)
        k = _r(xk @ W["Wk"].t(), rd)
        v = _r(xv @ W["Wv"].t(), rd)
        w1 = _r(xw @ W["w1"].t(), rd)
        a1 = _r(xa @ W["a1"].t(), rd)
        g1 = _r(xg @ W["g1"].t(), rd)
        w = _r(W["w0"] + _r(torch.tanh(w1), rd) @ W["w2"].t(), rd)
        a12 = _r(a1 @ W["a2"].t(), rd)
        g = _r(_r(torch.sigmoid(g1), rd) @ W["g2"].t(), rd)
        if l == 0:
            v_first = v
        else:
            v1 = _r(xv @ W["v1"].t(), rd)
            v = _r(v + (v_first - v) * torch.sigmoid(W["v0"] + v1 @ W["v2"].t()), rd)
        u = (k * W["k_k"]).view(B, H, 64)
        kk = F.normalize(u, dim=-1, eps=1e-12).reshape(B, C)
        a = torch.sigmoid(W["a0"] + a12)
        new_k = _r(k * (a * W["k_a"] + (1 - W["k_a"])), rd)
        neg_kk, kka = _r(-kk, rd), _r(kk * a, rd)
        # WKV-7 on the gathered states
        S = wkv[l, sl].clone()                                  # [B,H,64,64] fp32, S[i][j]
        d = torch.exp(-E_HALF * torch.sigmoid(w)).view(B, H, 1, 64)
        sa = torch.matmul(S, neg_kk.view(B, H, 64, 1))           # [B,H,64,1]
        S = S * d + sa * kka.view(B, H, 1, 64) + v.view(B, H, 64, 1) * new_k.view(B, H, 1, 64)
        y = _r(torch.matmul(S, r.view(B, H, 64, 1)).view(B, C), rd)
        wkv[l, sl] = S
        # GroupNorm + bonus + gate, output projection
        yh = y.view(B, H, 64)
        mean = yh.mean(-1, keepdim=True)
        var = ((yh - mean) ** 2).mean(-1, keepdim=True)
        yn = ((yh - mean) / torch.sqrt(var + 64e-5)).reshape(B, C)
        bonus = (r * new_k * W["r_k"]).view(B, H, 64).sum(-1, keepdim=True) * v.view(B, H, 64)
        o_in = _r((yn * W["lnx_w"] + W["lnx_b"] + bonus.reshape(B, C)) * g, rd)
        o = _r(o_in @ W["Wo"].t(), rd)
        # channel mix
        res = _r(o + res, rd)
        xx2 = _r(_ln(res, W["ln2_w"], W["ln2_b"]), rd)
        prev2 = ffn_shift[l, sl].float()
        xk2 = _r(xx2 + (prev2 - xx2) * W["x_k_ffn"], rd)
        ffn_shift[l, sl] = xx2.to(ffn_shift.dtype)
        act = _r(torch.relu(xk2 @ W["key"].t()) ** 2, rd)
        x = _r(act @ W["value"].t(), rd)
    h = _r(_ln(x + res, f(model.ln_out_w), f(model.ln_out_b)), rd)
    return h @ f(model.head).t()
