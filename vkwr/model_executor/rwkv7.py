"""RWKV-7 batched decode on the vkwr_amd kernels.

The reference ships no model code (its vkwr/model_executor is empty); the
layer order below is the RWKV-7 time-mix / channel-mix composition implied by
the reference's op contracts (its tests document r: LN -> mix -> linear;
w: -> linear -> tanh -> linear; a = -kk; b = kk * sigmoid(a0 + a12) --
tests/ops/test_v1_wkv_ops.py:74-96), one decode step per call:

  per layer l (x: previous block output, res: residual stream)
    res, xr,xw,xk,xv,xa,xg = add + LN1 + 6 token-shift lerps   (att shift pool, slot-indexed)
    r, k, v, w1, a1, g1, v1 = projections + rank-in             (one GEMM launch)
    w   = w0 + tanh(w1) W2^T ; a12 = a1 A2^T ; g = sigmoid(g1) G2^T
    v   = v + (v_first - v) sigmoid(v0 + v1 V2^T)   (layers > 0; layer 0 sets v_first = v)
                                                                (one GEMM launch)
    k', -kk, kk*a = kk/a gate(k, k_k, a0, a12, k_a)
    y   = WKV-7(state pool[slot], r, w, k', v, -kk, kk*a)
    o   = (GroupNorm(y) + (r.k'.r_k) v) * g  W_o^T
    res, xk = add + LN2 + 1 token-shift lerp                    (ffn shift pool, slot-indexed)
    x   = relu(xk K^T)^2 V^T
  logits = LN_out(x + res) Head^T

Weights are random-initialised (std 0.02, embedding std 1e-4) in nn.Linear
layout [out, in]; the embedding table is stored after its LN0.  All
activations are fp16, the WKV state fp32.  `DecodeEngine` preallocates every
buffer (activations, GEMM workspace), so a decode step allocates nothing and
can be captured into a HIP graph.

GEMM path: by default the engine packs every projection weight once into the
fragment layout of include/vkwr_amd.h (vkwr_frag_pack_f16) and the producers
of each projection input (the LN + token-shift fusions, the GroupNorm gate, the
final LN, and the GEMMs whose output only feeds another GEMM: the low-rank
inputs and the FFN hidden) write it directly in that layout, so every GEMM is a
vkwr_frag_gemm_f16 launch streaming the weights with fully coalesced loads.
The low-rank activations (tanh, sigmoid) are applied to the fp32 accumulator
of the producing GEMM and rounded to fp16 once.  The kk/a gate, the WKV
update and the GroupNorm/bonus/gate run as one kernel
(vkwr_wkv7_decode_fused_f16, bit-identical to the three separate launches),
which streams the WKV pool in the interleaved block layout
(capi.WKV_STATE_ILV: lane i loads row i with fully coalesced 16-byte loads, no
LDS staging).  `frag=False` runs the same
step on row-major weights through vkwr_gemm_f16 (the reference-op GEMM).
"""
import math
from dataclasses import dataclass

import torch

from vkwr_amd import capi

HEAD = 64


@dataclass(frozen=True)
class RWKV7Config:
    n_layer: int
    n_embd: int
    dim_ffn: int
    rank_w: int
    rank_a: int
    rank_v: int
    rank_g: int
    vocab: int

    @property
    def n_head(self):
        return self.n_embd // HEAD

    @staticmethod
    def preset(name):
        return {
            "1.5b": RWKV7Config(24, 2048, 8192, 96, 96, 64, 256, 65536),
            "7b": RWKV7Config(32, 4096, 16384, 128, 128, 96, 480, 65536),
            "tiny": RWKV7Config(2, 256, 1024, 32, 32, 16, 64, 1024),
        }[name]

    def weight_bytes(self):
        C, F = self.n_embd, self.dim_ffn
        r = self.rank_w + self.rank_a + self.rank_g + self.rank_v
        per_layer = 4 * C * C + 2 * C * r + 2 * C * F
        return 2 * (self.n_layer * per_layer + self.vocab * C)  # fp16; head only (emb rows are gathered)


LAYER_VECS = ("ln1_w", "ln1_b", "ln2_w", "ln2_b", "x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "a0", "v0",
              "k_k", "k_a", "r_k", "lnx_w", "lnx_b", "x_k_ffn")


class RWKV7Model:
    """Random-initialised fp16 weights of the given shape on `device`."""

    def __init__(self, cfg, device, seed=0, std=0.02, emb_std=1e-4):
        self.cfg = cfg
        g = torch.Generator(device=device).manual_seed(seed)
        C, F = cfg.n_embd, cfg.dim_ffn

        def mat(*shape, s=std):
            return (torch.randn(*shape, generator=g, device=device) * s).half()

        def vec(kind):
            if kind in ("ln1_w", "ln2_w", "lnx_w"):
                return (1.0 + 0.1 * torch.randn(C, generator=g, device=device)).half()
            if kind.startswith("x_"):
                return torch.rand(C, generator=g, device=device).half()
            if kind == "k_k":
                return (0.85 + 0.1 * torch.rand(C, generator=g, device=device)).half()
            if kind == "k_a":
                return (1.0 + 0.1 * torch.randn(C, generator=g, device=device)).half()
            if kind == "w0":
                return (-6.0 + 5.0 * torch.rand(C, generator=g, device=device)).half()
            return (0.1 * torch.randn(C, generator=g, device=device)).half()

        emb = (torch.randn(cfg.vocab, C, generator=g, device=device) * emb_std).half()
        ln0_w, ln0_b = vec("ln1_w"), vec("ln1_b")
        self.emb = torch.empty_like(emb)
        capi.layer_norm(emb, ln0_w, ln0_b, self.emb)  # LN0 folded into the table once
        del emb
        self.layers = []
        for l in range(cfg.n_layer):
            L = {k: vec(k) for k in LAYER_VECS}
            L.update(Wr=mat(C, C), Wk=mat(C, C), Wv=mat(C, C), Wo=mat(C, C),
                     w1=mat(cfg.rank_w, C), w2=mat(C, cfg.rank_w, s=0.1),
                     a1=mat(cfg.rank_a, C), a2=mat(C, cfg.rank_a, s=0.1),
                     g1=mat(cfg.rank_g, C), g2=mat(C, cfg.rank_g, s=0.1),
                     key=mat(F, C), value=mat(C, F))
            if l > 0:
                L.update(v1=mat(cfg.rank_v, C), v2=mat(C, cfg.rank_v, s=0.1))
            self.layers.append(L)
        self.ln_out_w, self.ln_out_b = vec("ln1_w"), vec("ln1_b")
        self.head = mat(cfg.vocab, C)


class RWKV7State:
    """Per-sequence recurrent state in slot pools: WKV [L, P, H, 64, 64] fp32 and
    the two token-shift rows [L, P, C] fp16 (time mix, channel mix).

    `layout` is the layout of each 64x64 WKV block: capi.WKV_STATE_STD (row-major,
    the reference ops' layout) or capi.WKV_STATE_ILV (interleaved; what the fused
    decode kernel streams, the default).  wkv_standard() returns a row-major copy."""

    def __init__(self, cfg, n_slots, device, std=0.1, seed=1, layout=capi.WKV_STATE_ILV):
        g = torch.Generator(device=device).manual_seed(seed)
        H, C = cfg.n_head, cfg.n_embd
        self.n_slots, self.layout = n_slots, layout
        self.wkv = torch.empty(cfg.n_layer, n_slots, H, HEAD, HEAD, dtype=torch.float32, device=device)
        self.wkv.normal_(0.0, std, generator=g) if std else self.wkv.zero_()
        self.att_shift = torch.zeros(cfg.n_layer, n_slots, C, dtype=torch.float16, device=device)
        self.ffn_shift = torch.zeros(cfg.n_layer, n_slots, C, dtype=torch.float16, device=device)

    def wkv_standard(self):
        """The WKV pool as row-major [L, P, H, 64, 64] blocks (a copy)."""
        if self.layout == capi.WKV_STATE_STD:
            return self.wkv.clone()
        out = torch.empty_like(self.wkv)
        capi.wkv_state_layout(self.wkv, out, capi.WKV_STATE_STD)
        return out

    def set_wkv_standard(self, wkv_std):
        """Overwrites the pool from row-major blocks."""
        if self.layout == capi.WKV_STATE_STD:
            self.wkv.copy_(wkv_std)
        else:
            capi.wkv_state_layout(wkv_std.contiguous(), self.wkv, capi.WKV_STATE_ILV)

    def bytes_per_token_step(self, cfg):
        """State bytes one decode step moves per sequence (read + write)."""
        return cfg.n_layer * (2 * cfg.n_head * HEAD * HEAD * 4 + 2 * 2 * cfg.n_embd * 2)


FRAG_WEIGHTS = ("Wr", "Wk", "Wv", "Wo", "w1", "w2", "a1", "a2", "g1", "g2", "v1", "v2", "key", "value")


class DecodeEngine:
    """Batched T=1 decode of up to `max_batch` sequences with preallocated buffers."""

    def __init__(self, model, max_batch, frag=True, fused_wkv=True):
        cfg = model.cfg
        self.model, self.cfg, self.max_batch, self.frag = model, cfg, max_batch, frag
        self.fused_wkv = fused_wkv  # frag path: gate + WKV + GroupNorm in one kernel
        dev = model.head.device
        B, C, F = max_batch, cfg.n_embd, cfg.dim_ffn
        if frag:
            self._init_frag(dev)
            return

        def buf(*shape):
            return torch.empty(*shape, dtype=torch.float16, device=dev)

        self.res = [buf(B, C), buf(B, C)]       # residual stream (ping-pong between blocks)
        self.mix = [buf(B, C) for _ in range(6)]
        self.r, self.k, self.v, self.v_first, self.v_new = buf(B, C), buf(B, C), buf(B, C), buf(B, C), buf(B, C)
        self.w1, self.a1 = buf(B, cfg.rank_w), buf(B, cfg.rank_a)
        self.g1, self.v1 = buf(B, cfg.rank_g), buf(B, cfg.rank_v)
        self.w, self.a12, self.g = buf(B, C), buf(B, C), buf(B, C)
        self.new_k, self.neg_kk, self.kka = buf(B, C), buf(B, C), buf(B, C)
        self.y, self.o_in, self.o = buf(B, C), buf(B, C), buf(B, C)
        self.xk_ffn, self.act, self.ffn = buf(B, C), buf(B, F), buf(B, C)
        self.h = buf(B, C)
        self.logits = buf(B, cfg.vocab)
        # GEMM workspace: the largest K-split need of any launch at any batch size (every
        # size is evaluated: the plan is not monotone in the row count)
        need = max(capi.gemm_workspace_bytes_upto(ps) for ps in self._all_gemms(B))
        self.ws = torch.empty(max(need, 0), dtype=torch.uint8, device=dev)

    def _init_frag(self, dev):
        cfg, m = self.cfg, self.model
        B, C, F = self.max_batch, cfg.n_embd, cfg.dim_ffn

        def packed(w):
            n, k = w.shape
            out = capi.frag_empty(n, k, dev, zero=False)
            capi.frag_pack(w.contiguous(), n, k, out)
            return out

        self.pw = [{name: packed(L[name]) for name in FRAG_WEIGHTS if name in L} for L in m.layers]
        self.p_head = packed(m.head)

        def buf(*shape):
            return torch.empty(*shape, dtype=torch.float16, device=dev)

        fr = lambda k: capi.frag_empty(B, k, dev)  # noqa: E731
        self.res = [buf(B, C), buf(B, C)]
        self.mixf = [fr(C) for _ in range(6)]
        self.r, self.k, self.v, self.v_first, self.v_new = buf(B, C), buf(B, C), buf(B, C), buf(B, C), buf(B, C)
        self.w1f, self.a1f, self.g1f, self.v1f = fr(cfg.rank_w), fr(cfg.rank_a), fr(cfg.rank_g), fr(cfg.rank_v)
        self.w, self.a12, self.g = buf(B, C), buf(B, C), buf(B, C)
        self.new_k, self.neg_kk, self.kka = buf(B, C), buf(B, C), buf(B, C)
        self.y, self.o = buf(B, C), buf(B, C)
        self.o_in_f, self.xk_f, self.act_f, self.h_f = fr(C), fr(C), fr(F), fr(C)
        self.ffn = buf(B, C)
        self.logits = buf(B, cfg.vocab)
        # FFN value (K = F): K split over workgroups, fp32 partials in a workspace
        # sized for the largest batch.
        nbytes = max(capi.frag_splitk_workspace_bytes(b, C, self._value_splits(b)) for b in range(1, B + 1))
        self.value_ws = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=dev)

    def _value_splits(self, B):
        """K parts of the FFN value GEMM at batch B: enough 64x64-tile parts to give
        the 256 CUs one workgroup each, each part at least 256 deep in K."""
        C, F = self.cfg.n_embd, self.cfg.dim_ffn
        tiles = -(-B // 64) * (capi.frag_pad(C) // 64)
        splits = max(1, min(16, 256 // max(tiles, 1)))
        while splits > 1 and capi.frag_pad(F) % (256 * splits):
            splits //= 2
        return splits

    def _step_frag(self, state, tokens, slots):
        cfg, m, s = self.cfg, self.model, self
        B = tokens.shape[0]
        C, H, F = cfg.n_embd, cfg.n_head, cfg.dim_ffn
        fp = capi.frag_problem
        x, res_in, parts = None, None, 0
        splits = self._value_splits(B)
        # FFN value K parts reduced inside the next layer's LayerNorm (2, 4 or 8 parts)
        parts_ok = splits in (2, 4, 8) and C % 128 == 0 and C <= 4096
        for l, L in enumerate(m.layers):
            first = l == 0
            P = s.pw[l]
            res = s.res[l % 2][:B]
            # ---- time mix
            mixes = [L["x_r"], L["x_w"], L["x_k"], L["x_v"], L["x_a"], L["x_g"]]
            if parts:  # the previous layer's FFN value, still as K parts: reduced here
                capi.add_layer_norm_mix_parts(s.value_ws, parts, capi.splitk_plane_floats(B, C), res_in,
                                              state.att_shift[l], L["ln1_w"], L["ln1_b"], mixes, res, s.mixf,
                                              shift_slots=slots)
            else:
                capi.add_layer_norm_mix(
                    m.emb if first else x, None if first else res_in, state.att_shift[l], L["ln1_w"], L["ln1_b"],
                    mixes, res, s.mixf, x_rows=tokens if first else None, shift_slots=slots, frag=True)
            xr, xw, xk, xv, xa, xg = s.mixf
            v_out = (s.v_first if first else s.v)[:B]
            probs = [fp(xr, P["Wr"], s.r, B, C, C), fp(xk, P["Wk"], s.k, B, C, C), fp(xv, P["Wv"], v_out, B, C, C),
                     fp(xw, P["w1"], s.w1f, B, cfg.rank_w, C, epilogue=capi.EPI_TANH, c_frag=True),
                     fp(xa, P["a1"], s.a1f, B, cfg.rank_a, C, c_frag=True),
                     fp(xg, P["g1"], s.g1f, B, cfg.rank_g, C, epilogue=capi.EPI_SIGMOID, c_frag=True)]
            if not first:
                probs.append(fp(xv, P["v1"], s.v1f, B, cfg.rank_v, C, c_frag=True))
            capi.frag_gemm(probs)
            probs = [fp(s.w1f, P["w2"], s.w, B, C, cfg.rank_w, epilogue=capi.EPI_BIAS, v0=L["w0"]),
                     fp(s.a1f, P["a2"], s.a12, B, C, cfg.rank_a),
                     fp(s.g1f, P["g2"], s.g, B, C, cfg.rank_g)]
            if not first:
                probs.append(fp(s.v1f, P["v2"], s.v_new, B, C, cfg.rank_v, epilogue=capi.EPI_VALUE_RESIDUAL,
                                v=s.v, v_first=s.v_first, v0=L["v0"]))
            capi.frag_gemm(probs)
            v = (s.v_first if first else s.v_new)[:B]
            if s.fused_wkv:
                capi.wkv_decode_fused(B, C, H, state.wkv[l], slots, s.r, s.w, s.k, v, s.a12, s.g, L["k_k"],
                                      L["a0"], L["k_a"], L["r_k"], L["lnx_w"], L["lnx_b"], s.o_in_f, frag=True,
                                      state_layout=state.layout)
            else:
                capi.kk_a_gate(B, 1, C, H, s.k[:B], L["k_k"], L["a0"], s.a12[:B], L["k_a"], s.new_k[:B],
                               s.neg_kk[:B], s.kka[:B])
                capi.wkv_slots(B, 1, C, H, state.wkv[l], slots, s.r[:B], s.w[:B], s.new_k[:B], v,
                               s.neg_kk[:B], s.kka[:B], s.y[:B])
                capi.groupnorm_bonus_gate(B, 1, C, H, s.y[:B], s.r[:B], s.new_k[:B], v, L["r_k"], L["lnx_w"],
                                          L["lnx_b"], s.g[:B], s.o_in_f, frag=True)
            capi.frag_gemm([fp(s.o_in_f, P["Wo"], s.o, B, C, C)])
            # ---- channel mix
            res2 = s.res[(l + 1) % 2][:B]
            capi.add_layer_norm_mix(s.o[:B], res, state.ffn_shift[l], L["ln2_w"], L["ln2_b"], [L["x_k_ffn"]],
                                    res2, [s.xk_f], shift_slots=slots, frag=True)
            capi.frag_gemm([fp(s.xk_f, P["key"], s.act_f, B, F, C, epilogue=capi.EPI_RELU_SQUARE, c_frag=True)])
            parts = 0
            if parts_ok and l + 1 < len(m.layers):
                capi.frag_gemm_splitk_parts(fp(s.act_f, P["value"], s.ffn, B, C, F), splits, s.value_ws)
                parts = splits
            elif splits > 1:
                capi.frag_gemm_splitk(fp(s.act_f, P["value"], s.ffn, B, C, F), splits, s.value_ws)
            else:
                capi.frag_gemm([fp(s.act_f, P["value"], s.ffn, B, C, F)])
            x, res_in = s.ffn[:B], res2
        capi.add_last_layer_norm(B, 1, C, x, res_in, m.ln_out_w, m.ln_out_b, s.h_f, frag=True)
        capi.frag_gemm([fp(s.h_f, s.p_head, s.logits, B, cfg.vocab, C)])
        return s.logits[:B]

    # -- GEMM batches of one layer (shared by planning and execution)
    def _proj_problems(self, L, B, first):
        s = self
        # layer 0's value projection is v_first itself
        ps = [capi.gemm_problem(s.mix[0][:B], L["Wr"], s.r[:B]),
              capi.gemm_problem(s.mix[2][:B], L["Wk"], s.k[:B]),
              capi.gemm_problem(s.mix[3][:B], L["Wv"], (s.v_first if first else s.v)[:B]),
              capi.gemm_problem(s.mix[1][:B], L["w1"], s.w1[:B]),
              capi.gemm_problem(s.mix[4][:B], L["a1"], s.a1[:B]),
              capi.gemm_problem(s.mix[5][:B], L["g1"], s.g1[:B])]
        if not first:
            ps.append(capi.gemm_problem(s.mix[3][:B], L["v1"], s.v1[:B]))
        return ps

    def _rank_out_problems(self, L, B, first):
        s = self
        ps = [capi.gemm_problem(s.w1[:B], L["w2"], s.w[:B], a_act=capi.ACT_TANH, epilogue=capi.EPI_BIAS,
                                v0=L["w0"]),
              capi.gemm_problem(s.a1[:B], L["a2"], s.a12[:B]),
              capi.gemm_problem(s.g1[:B], L["g2"], s.g[:B], a_act=capi.ACT_SIGMOID)]
        if not first:
            ps.append(capi.gemm_problem(s.v1[:B], L["v2"], s.v_new[:B], epilogue=capi.EPI_VALUE_RESIDUAL,
                                        v=s.v[:B], v_first=s.v_first[:B], v0=L["v0"]))
        return ps

    def _all_gemms(self, B):
        m, s = self.model, self
        out = []
        for l, L in enumerate(m.layers[:2]):
            out.append(self._proj_problems(L, B, l == 0))
            out.append(self._rank_out_problems(L, B, l == 0))
        L = m.layers[-1]
        out.append([capi.gemm_problem(s.o_in[:B], L["Wo"], s.o[:B])])
        out.append([capi.gemm_problem(s.xk_ffn[:B], L["key"], s.act[:B], epilogue=capi.EPI_RELU_SQUARE)])
        out.append([capi.gemm_problem(s.act[:B], L["value"], s.ffn[:B])])
        out.append([capi.gemm_problem(s.h[:B], m.head, s.logits[:B])])
        return out

    def step(self, state, tokens, slots):
        """One decode step for B = len(tokens) sequences: tokens, slots int32 [B] on the
        device (slots distinct, < state.n_slots).  Updates `state` in place and returns
        the logits view [B, vocab] (valid until the next step)."""
        B = tokens.shape[0]
        assert 0 < B <= self.max_batch and slots.shape[0] == B
        if self.frag:
            assert self.fused_wkv or state.layout == capi.WKV_STATE_STD, "unfused WKV needs the row-major pool"
            return self._step_frag(state, tokens, slots)
        assert state.layout == capi.WKV_STATE_STD, "the row-major engine needs the row-major WKV pool"
        cfg, m, s = self.cfg, self.model, self
        C, H = cfg.n_embd, cfg.n_head
        ws = self.ws
        x, res_in = None, None
        for l, L in enumerate(m.layers):
            first = l == 0
            res = s.res[l % 2][:B]
            # ---- time mix
            capi.add_layer_norm_mix(
                m.emb if first else x, None if first else res_in, state.att_shift[l], L["ln1_w"], L["ln1_b"],
                [L["x_r"], L["x_w"], L["x_k"], L["x_v"], L["x_a"], L["x_g"]], res, [t[:B] for t in s.mix],
                x_rows=tokens if first else None, shift_slots=slots)
            capi.gemm(self._proj_problems(L, B, first), ws)
            capi.gemm(self._rank_out_problems(L, B, first), ws)
            v = (s.v_first if first else s.v_new)[:B]
            capi.kk_a_gate(B, 1, C, H, s.k[:B], L["k_k"], L["a0"], s.a12[:B], L["k_a"], s.new_k[:B],
                           s.neg_kk[:B], s.kka[:B])
            capi.wkv_slots(B, 1, C, H, state.wkv[l], slots, s.r[:B], s.w[:B], s.new_k[:B], v, s.neg_kk[:B],
                           s.kka[:B], s.y[:B])
            capi.groupnorm_bonus_gate(B, 1, C, H, s.y[:B], s.r[:B], s.new_k[:B], v, L["r_k"], L["lnx_w"],
                                      L["lnx_b"], s.g[:B], s.o_in[:B])
            capi.gemm([capi.gemm_problem(s.o_in[:B], L["Wo"], s.o[:B])], ws)
            # ---- channel mix
            res2 = s.res[(l + 1) % 2][:B]
            capi.add_layer_norm_mix(s.o[:B], res, state.ffn_shift[l], L["ln2_w"], L["ln2_b"], [L["x_k_ffn"]],
                                    res2, [s.xk_ffn[:B]], shift_slots=slots)
            capi.gemm([capi.gemm_problem(s.xk_ffn[:B], L["key"], s.act[:B], epilogue=capi.EPI_RELU_SQUARE)], ws)
            capi.gemm([capi.gemm_problem(s.act[:B], L["value"], s.ffn[:B])], ws)
            x, res_in = s.ffn[:B], res2
        capi.add_last_layer_norm(B, 1, C, x, res_in, m.ln_out_w, m.ln_out_b, s.h[:B])
        capi.gemm([capi.gemm_problem(s.h[:B], m.head, s.logits[:B])], ws)
        return s.logits[:B]


def gbytes_per_step(cfg, batch):
    """Algorithmic HBM bytes of one decode step at batch `batch`: every weight
    once (the embedding only for the gathered rows), the WKV state and both
    shift rows read and written per sequence and layer, the logits written."""
    w = cfg.weight_bytes() + batch * cfg.n_embd * 2
    state = cfg.n_layer * batch * (2 * cfg.n_head * HEAD * HEAD * 4 + 2 * 2 * 2 * cfg.n_embd)
    return w + state + batch * cfg.vocab * 2


def flops_per_step(cfg, batch):
    C, F = cfg.n_embd, cfg.dim_ffn
    r = cfg.rank_w + cfg.rank_a + cfg.rank_g + cfg.rank_v
    per_layer = 2 * batch * (4 * C * C + 2 * C * r + 2 * C * F)
    return cfg.n_layer * per_layer + 2 * batch * C * cfg.vocab


__all__ = ["RWKV7Config", "RWKV7Model", "RWKV7State", "DecodeEngine", "gbytes_per_step", "flops_per_step",
           "math"]
