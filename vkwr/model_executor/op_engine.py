"""RWKV-7 batched decode composed only of the reference's op surface.

`OpDecodeEngine.step` runs the same decode step as `DecodeEngine` (same model,
same state pools, same layer order), but every kernel it launches is one of the
reference's torch ops, called through the reference's own wrapper modules --
what an executor written against the reference's `vkwr._ops` (its
vkwr/model_executor is empty) calls.  Per layer:

  time mix
    x_out, xr, xw, xk, xv, xa, xg = add_layer_norm_tmix_mix6_f16(x, res, shift, ...)
                                            (reference vkwr/_ops/v1/v1_norm_ops.py:110)
    r, k, v = linear_f16_orig(x*, W*)       (reference vkwr/_ops/v1/v1_linear_ops.py:24)
    w1, a1, g1(, v1) = linear_wag(v)_rank_in_f16(...)
    w, a12, g(, v) = linear_wag(v)_rank_out_f16(...)      (tanh / sigmoid / value residual;
                                            reference vkwr/_ops/v1/v1_rank_ops.py:1-57)
    w = add_vec(C, w, w0)                   (reference vkwr/_ops/v1/v1_mix_ops.py)
    new_k, -kk, kk*a = tmix_kk_a_gate(...)
    y = wkv_forward_slots_fp32(pool, slots, ...)   (gather + step + scatter in one call), or
        index_select -> wkv_forward_fp32 -> index_copy_ (reference v1_wkv_ops.py:81-84)
    o = linear_f16_orig(tmix_lnx_rkvres_xg(y, r, new_k, v, ...), Wo)
  channel mix
    x_out2, xk = add_layer_norm_cmix_mix_f16(o, x_out, shift, ...)
    x = linear_f16_orig(relu_square(linear_f16_orig(xk, key)), value)          (ffn="dense"), or
    x = cmix_sparse_down_relu_rows(linear_f16_orig(xk, key), value_fc)         (ffn="sparse")
  head
    logits = linear_f16_orig(add_last_layer_norm_f16(x, res, ...), head)

The reference ops take a dense token-shift state [B, C] (updated in place), so
the batch's shift rows of every layer are gathered from the slot pools with one
index_select per pool at the start of the step, each layer's ops update its dense
[B, C] rows in place, and one index_copy_ per pool writes them back at the end
(per layer, the four gathers and scatters cost ~18 us of a ~160 us layer).  The ops allocate
their outputs, as the reference's do (the caching allocator serves them; under
a HIP graph capture they come from the graph's pool).  The only weight the ops
want in another layout is the FFN value, which cmix_sparse_* takes as [F, C]:
with ffn="sparse" it is transposed once when the engine is built.  At 128 rows
the dense form is the faster one: its down projection streams the [N, K] weight,
where cmix_sparse_down_relu_rows gathers [K, N] fragments column by column.
"""
import torch

from vkwr._ops.v1 import v1_linear_ops as LIN
from vkwr._ops.v1 import v1_mix_ops as MIX
from vkwr._ops.v1 import v1_norm_ops as NORM
from vkwr._ops.v1 import v1_rank_ops as RANK
from vkwr._ops.v1 import v1_wkv_ops as WKV
from vkwr_amd import capi


class OpDecodeEngine:
    """Batched T=1 decode on the reference op surface (see the module docstring).

    wkv="slots" steps the WKV state through the slot-pool op (one launch per layer);
    wkv="gather" gathers the batch's states with index_select, calls the reference's
    dense wkv_forward_fp32 and scatters them back with index_copy_.  ffn selects the
    channel mix's down projection: "dense" (relu_square, then linear_f16_orig) or
    "sparse" (cmix_sparse_down_relu_rows)."""

    def __init__(self, model, wkv="slots", ffn="dense"):
        assert wkv in ("slots", "gather") and ffn in ("dense", "sparse")
        self.model, self.cfg, self.wkv, self.ffn = model, model.cfg, wkv, ffn
        # cmix_sparse_* take the FFN value weight as [F, C] (value_fc); the model keeps [C, F]
        self.value_fc = [L["value"].t().contiguous() for L in model.layers] if ffn == "sparse" else None

    def step(self, state, tokens, slots):
        """One decode step for B = len(tokens) sequences: tokens, slots int32 [B] on the
        device (slots distinct, < state.n_slots; the WKV pool in the row-major layout).
        Updates `state` in place and returns the fp16 logits [B, vocab]."""
        assert state.layout == capi.WKV_STATE_STD, "the reference ops read the row-major WKV layout"
        assert tokens.dtype == torch.int32 and slots.dtype == torch.int32 and slots.shape == tokens.shape
        cfg, m = self.cfg, self.model
        B = tokens.shape[0]
        C, H, F = cfg.n_embd, cfg.n_head, cfg.dim_ffn
        Rw, Ra, Rg, Rv = cfg.rank_w, cfg.rank_a, cfg.rank_g, cfg.rank_v
        sl = slots.long()
        x = m.emb.index_select(0, tokens.long()).view(B, 1, C)
        res = torch.zeros_like(x)
        v_first = None
        att_all = state.att_shift.index_select(1, sl)  # [L, B, C]: this batch's rows of every layer
        ffn_all = state.ffn_shift.index_select(1, sl)
        d2 = lambda t: t.view(B, C)  # noqa: E731  (the rank ops take [M, K] matrices)
        d3 = lambda t: t.view(B, 1, C)  # noqa: E731  (the mix and WKV ops take [B, T, C])
        for l, L in enumerate(m.layers):
            first = l == 0
            # ---- time mix
            res, xr, xw, xk, xv, xa, xg = NORM.add_layer_norm_tmix_mix6_f16(
                x, res, att_all[l], L["ln1_w"], L["ln1_b"], L["x_r"], L["x_w"], L["x_k"], L["x_v"], L["x_a"],
                L["x_g"])
            r = LIN.linear_f16_orig(xr, L["Wr"])
            k = LIN.linear_f16_orig(xk, L["Wk"])
            v = LIN.linear_f16_orig(xv, L["Wv"])
            if first:
                w1, a1, g1 = RANK.linear_wag_rank_in_f16(B, C, Rw, Ra, Rg, d2(xw), d2(xa), d2(xg), L["w1"], L["a1"],
                                                         L["g1"])
                w, a12, g = RANK.linear_wag_rank_out_f16(B, C, Rw, Ra, Rg, w1, a1, g1, L["w2"], L["a2"], L["g2"])
                v_first = v
            else:
                w1, a1, g1, v1 = RANK.linear_wagv_rank_in_f16(B, C, Rw, Ra, Rg, Rv, d2(xw), d2(xa), d2(xg),
                                                              d2(xv), L["w1"], L["a1"], L["g1"], L["v1"])
                w, a12, g, v = RANK.linear_wagv_rank_out_f16(B, C, Rw, Ra, Rg, Rv, w1, a1, g1, v1, L["w2"],
                                                             L["a2"], L["g2"], L["v2"], d2(v), d2(v_first),
                                                             L["v0"])
                v = d3(v)
            w = d3(MIX.add_vec(C, w, L["w0"]))
            new_k, neg_kk, kka = MIX.tmix_kk_a_gate(B, 1, C, H, k, L["k_k"], L["a0"], d3(a12), L["k_a"])
            if self.wkv == "slots":
                y = torch.empty(B, 1, C, dtype=torch.float16, device=x.device)
                torch.ops.vkwr_v1_wkv.wkv_forward_slots_fp32(B, 1, C, H, state.wkv[l], slots, r, w, new_k, v,
                                                             neg_kk, kka, y)
            else:
                S = state.wkv[l].index_select(0, sl)
                y = WKV.wkv_forward_fp32(B, 1, C, H, S, r, w, new_k, v, neg_kk, kka)
                state.wkv[l].index_copy_(0, sl, S)
            o_in = MIX.tmix_lnx_rkvres_xg(B, 1, C, H, y, r, new_k, v, L["r_k"], L["lnx_w"], L["lnx_b"], d3(g))
            o = LIN.linear_f16_orig(o_in, L["Wo"])
            # ---- channel mix
            res, xk2 = NORM.add_layer_norm_cmix_mix_f16(o, res, ffn_all[l], L["ln2_w"], L["ln2_b"], L["x_k_ffn"])
            pre = LIN.linear_f16_orig(xk2, L["key"])
            if self.ffn == "dense":
                x = LIN.linear_f16_orig(MIX.relu_square(pre), L["value"])
            else:
                x = MIX.cmix_sparse_down_relu_rows(B, 1, C, F, pre, self.value_fc[l])
        state.att_shift.index_copy_(1, sl, att_all)
        state.ffn_shift.index_copy_(1, sl, ffn_all)
        h = NORM.add_last_layer_norm_f16(x, res, m.ln_out_w, m.ln_out_b)
        return LIN.linear_f16_orig(h, m.head)
