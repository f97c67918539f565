"""RWKV-7 forward step over a mixed batch: decode rows plus prefill chunks.

A continuous-batching server (256 decode rows plus 4 prefill
chunks of 512 tokens per step on the 7B shape) runs every row of a step through
the same projection / FFN GEMM launches -- M = all rows, so the GEMMs are large
and matrix-core bound -- while the per-sequence recurrent parts run per group:

  group = (B sequences, T tokens each, first row, slots); decode rows form one
          group with T = 1, each prefill chunk length another.

Per layer (x: previous block output, res: residual stream, rows = all rows):
  res, xr..xg = add + LN1 + token-shift lerps per group (slot-indexed att shift
          pool; one launch over all groups, the LN output never leaves the CUs)
  r, k, v, tanh(w1), a1, sigmoid(g1), v1 = projections over rows (one GEMM launch,
          the activations in its epilogue)
  w, a12, g, v = low-rank outputs (tanh / - / sigmoid / value residual) (one launch;
          the adapter ranks padded to multiples of 64 with zeros, so the launch runs on
          the large-M kernel)
  k', -kk, kk*a = kk/a gate over rows
  y   = WKV-7 per group on the slot pool (T > 1: the chunked prefill kernel; the T = 1
        decode group in the row-split order, on a second stream beside the prefill)
  o   = (GroupNorm(y) + bonus) * g  W_o^T over rows
  res, xk = add + LN2 + token shift per group (ffn shift pool; one launch)
  x   = relu(xk K^T)^2 V^T over rows
logits of the last row of every group's sequences = LN_out(x + res) Head^T.

The same layer composition as DecodeEngine (rwkv7.py), on the reference-op GEMM
(vkwr_gemm_f16, row-major weights) and the row-major WKV pool.  A prefill chunk
of T tokens gives the same recurrent state and last-token logits as T decode
steps (same arithmetic per token, GEMM rows independent); tests/test_serving_gpu.py
checks that, and the decode rows against DecodeEngine.

Every buffer is preallocated for `max_rows` rows, so a step allocates nothing.
"""
import torch

from vkwr_amd import capi
from vkwr.model_executor.rwkv7 import HEAD

TMIX_MIX = ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g")
RANK_ALIGN = 64  # the large-M GEMM kernel takes K in multiples of 64


def _pad_rank(w1, w2, r):
    """Low-rank adapter pair (w1 [rank, C], w2 [C, rank]) with the rank padded to r: zero
    rows of w1 give zero inputs to w2's zero columns, which add exact zeros (also through
    the tanh / sigmoid applied in between: their values meet zero weights)."""
    rank, C = w1.shape
    if rank == r:
        return w1, w2
    p1 = torch.zeros(r, C, dtype=w1.dtype, device=w1.device)
    p1[:rank] = w1
    p2 = torch.zeros(w2.shape[0], r, dtype=w2.dtype, device=w2.device)
    p2[:, :rank] = w2
    return p1, p2


class MixedEngine:
    """Forward step over up to `max_rows` rows in decode and prefill groups."""

    def __init__(self, model, max_rows, max_seqs=None):
        cfg = model.cfg
        self.model, self.cfg, self.max_rows = model, cfg, max_rows
        self.max_seqs = max_seqs or max_rows
        dev = model.head.device
        R, C, F = max_rows, cfg.n_embd, cfg.dim_ffn

        def buf(*shape):
            return torch.empty(*shape, dtype=torch.float16, device=dev)

        self.tok = torch.empty(R, dtype=torch.int32, device=dev)
        self.x0 = buf(R, C)
        self.res = [buf(R, C), buf(R, C)]
        self.mix = [buf(R, C) for _ in range(6)]
        self.r, self.k, self.v, self.v_first, self.v_new = (buf(R, C) for _ in range(5))
        # Low-rank adapters with the rank padded to a multiple of 64 (96 -> 128, 480 -> 512 at
        # the 7B shape), so that the rank-out batch runs on the large-M kernel.
        up = lambda r: -(-r // RANK_ALIGN) * RANK_ALIGN  # noqa: E731
        self.ranks = {k: up(getattr(cfg, "rank_" + k)) for k in ("w", "a", "g", "v")}
        self.lw = []
        for l, L in enumerate(model.layers):
            d = {}
            for k in ("w", "a", "g", "v"):
                if k + "1" in L:
                    d[k + "1"], d[k + "2"] = _pad_rank(L[k + "1"], L[k + "2"], self.ranks[k])
            self.lw.append(d)
        rk = self.ranks
        self.w1, self.a1, self.g1, self.v1 = buf(R, rk["w"]), buf(R, rk["a"]), buf(R, rk["g"]), buf(R, rk["v"])
        self.w, self.a12, self.g = buf(R, C), buf(R, C), buf(R, C)
        self.new_k, self.neg_kk, self.kka, self.y, self.o_in, self.o = (buf(R, C) for _ in range(6))
        self.xk = buf(R, C)
        self.act = buf(R, F)
        self.ffn = buf(R, C)
        self.h = buf(self.max_seqs, C)
        self.logits = buf(self.max_seqs, cfg.vocab)
        # GEMM workspace: the largest need of any launch at any row count a step can have
        # (the plan is not monotone in the row count, so every count is evaluated).
        need = max(capi.gemm_workspace_bytes_upto(ps) for ps in self._gemm_batches(max_rows, 1))
        need = max(need, capi.gemm_workspace_bytes_upto(self._head_problem(self.max_seqs)))
        self.ws = torch.empty(max(need, 0), dtype=torch.uint8, device=dev)
        # The decode rows' WKV step runs on a second stream beside the prefill chunks' (its
        # kernel uses no LDS, so it fits on the CUs the chunk kernel holds); default priority.
        self.side = torch.cuda.Stream(device=dev) if dev.type == "cuda" else None
        self.fork = torch.cuda.Event() if dev.type == "cuda" else None
        self.join = torch.cuda.Event() if dev.type == "cuda" else None

    # -- GEMM batches (shared by planning and execution)
    def _proj(self, L, W, R, first):
        s, gp = self, capi.gemm_problem
        ps = [gp(s.mix[0][:R], L["Wr"], s.r[:R]), gp(s.mix[2][:R], L["Wk"], s.k[:R]),
              gp(s.mix[3][:R], L["Wv"], (s.v_first if first else s.v)[:R]),
              gp(s.mix[1][:R], W["w1"], s.w1[:R], epilogue=capi.EPI_TANH), gp(s.mix[4][:R], W["a1"], s.a1[:R]),
              gp(s.mix[5][:R], W["g1"], s.g1[:R], epilogue=capi.EPI_SIGMOID)]
        if not first:
            ps.append(gp(s.mix[3][:R], W["v1"], s.v1[:R]))
        return ps

    def _rank_out(self, L, W, R, first):
        """The low-rank output GEMMs.  Their inputs tanh(w1) and sigmoid(g1) come activated
        from the projection batch's epilogue (once per element, on the fp32 sum, as in the
        decode engine's frag GEMM; as an A-operand activation every column tile of this GEMM
        recomputed them, 56 of the 103 us of g2 at the 7B shape)."""
        s, gp = self, capi.gemm_problem
        # (the large-M GEMM gives every XCD an equal share of each problem's tiles, longest K
        # first, whatever the order of the batch)
        ps = [gp(s.g1[:R], W["g2"], s.g[:R]),
              gp(s.w1[:R], W["w2"], s.w[:R], epilogue=capi.EPI_BIAS, v0=L["w0"]),
              gp(s.a1[:R], W["a2"], s.a12[:R])]
        if not first:
            ps.append(gp(s.v1[:R], W["v2"], s.v_new[:R], epilogue=capi.EPI_VALUE_RESIDUAL, v=s.v[:R],
                         v_first=s.v_first[:R], v0=L["v0"]))
        return ps

    def _gemm_batches(self, R, nl):
        m, s, gp = self.model, self, capi.gemm_problem
        out = []
        for l, L in enumerate(m.layers[:max(nl, 2)]):
            out += [self._proj(L, self.lw[l], R, l == 0), self._rank_out(L, self.lw[l], R, l == 0)]
        L = m.layers[-1]
        out += [[gp(s.o_in[:R], L["Wo"], s.o[:R])],
                [gp(s.xk[:R], L["key"], s.act[:R], epilogue=capi.EPI_RELU_SQUARE)],
                [gp(s.act[:R], L["value"], s.ffn[:R])]]
        return out

    def _wkv_gn(self, groups, pool, v, L):
        """WKV-7 of every group on the slot pool, then the GroupNorm + bonus + gate of its rows:
        prefill groups (T > 1) on the current stream, the decode group (T = 1, row-split order,
        no LDS) on the side stream, forked after the gate and joined before the o projection.
        The decode rows' HBM-bound state traffic runs while the prefill chunks occupy the
        matrix cores, and each side's GroupNorm runs as soon as its own WKV is done."""
        C, H = self.cfg.n_embd, self.cfg.n_head
        s = self
        args = lambda r0, n: (s.r[r0:r0 + n], s.w[r0:r0 + n], s.new_k[r0:r0 + n], v[r0:r0 + n],  # noqa: E731
                              s.neg_kk[r0:r0 + n], s.kka[r0:r0 + n], s.y[r0:r0 + n])

        def gn(r0, n):
            sl = slice(r0, r0 + n)
            capi.groupnorm_bonus_gate(n, 1, C, H, s.y[sl], s.r[sl], s.new_k[sl], v[sl], L["r_k"], L["lnx_w"],
                                      L["lnx_b"], s.g[sl], s.o_in[sl])

        dec = [g for g in groups if g[1] == 1]
        main = torch.cuda.current_stream()
        if dec:
            s.fork.record(main)
        for B, T, r0, slots, _ in groups:
            if T > 1:
                capi.wkv_slots(B, T, C, H, pool, slots, *args(r0, B * T))
                gn(r0, B * T)
        for B, _, r0, slots, _ in dec:
            s.side.wait_event(s.fork)
            with torch.cuda.stream(s.side):
                capi.wkv_step_rows_slots(B, C, H, pool, slots, *args(r0, B))
                gn(r0, B)
            s.join.record(s.side)
            main.wait_event(s.join)

    def _head_problem(self, S):
        return [capi.gemm_problem(self.h[:S], self.model.head, self.logits[:S])]

    # -- the step
    def step(self, state, decode=None, prefill=()):
        """decode: (tokens [Bd] int32, slots [Bd] int32) or None; prefill: sequence of
        (tokens [Bg, Tg] int32, slots [Bg] int32).  All on the device, slots distinct over the
        whole step and < state.n_slots.  Updates `state` in place and returns logits
        [Bd + sum Bg, V]: the decode rows, then each prefill sequence's last chunk token
        (a view valid until the next step)."""
        cfg, m, s = self.cfg, self.model, self
        assert state.layout == capi.WKV_STATE_STD, "the mixed step uses the row-major WKV pool"
        C, H = cfg.n_embd, cfg.n_head
        groups = []  # (B, T, row0, slots, seq0)
        row, seq = 0, 0
        if decode is not None:
            tokens, slots = decode
            B = tokens.shape[0]
            s.tok[row:row + B].copy_(tokens)
            groups.append((B, 1, row, slots, seq))
            row, seq = row + B, seq + B
        for tokens, slots in prefill:
            B, T = tokens.shape
            s.tok[row:row + B * T].copy_(tokens.reshape(-1))
            groups.append((B, T, row, slots, seq))
            row, seq = row + B * T, seq + B
        R, S = row, seq
        assert 0 < R <= self.max_rows and S <= self.max_seqs
        ws = self.ws
        torch.index_select(m.emb, 0, s.tok[:R], out=s.x0[:R])
        shift_groups = [(r0, B, T, slots) for B, T, r0, slots, _ in groups]
        x, res_in = s.x0[:R], None
        for l, L in enumerate(m.layers):
            first = l == 0
            # the LN launches read neighbouring rows of their inputs, so each writes the residual
            # stream into the buffer it does not read: LN1 into res[1], LN2 into res[0]
            res = s.res[1][:R]
            # ---- time mix: res = x + res_in, LN1 and the six lerps against the shift pool
            capi.layer_norm_shift_rows(x, L["ln1_w"], L["ln1_b"], res, [L[k] for k in TMIX_MIX],
                                       [t[:R] for t in s.mix], state.att_shift[l], shift_groups, residual=res_in)
            capi.gemm(self._proj(L, s.lw[l], R, first), ws)
            capi.gemm(self._rank_out(L, s.lw[l], R, first), ws)
            v = (s.v_first if first else s.v_new)[:R]
            capi.kk_a_gate(R, 1, C, H, s.k[:R], L["k_k"], L["a0"], s.a12[:R], L["k_a"], s.new_k[:R],
                           s.neg_kk[:R], s.kka[:R])
            self._wkv_gn(groups, state.wkv[l], v, L)
            capi.gemm([capi.gemm_problem(s.o_in[:R], L["Wo"], s.o[:R])], ws)
            # ---- channel mix
            res2 = s.res[0][:R]
            capi.layer_norm_shift_rows(s.o[:R], L["ln2_w"], L["ln2_b"], res2, [L["x_k_ffn"]], [s.xk[:R]],
                                       state.ffn_shift[l], shift_groups, residual=res)
            capi.gemm([capi.gemm_problem(s.xk[:R], L["key"], s.act[:R], epilogue=capi.EPI_RELU_SQUARE)], ws)
            capi.gemm([capi.gemm_problem(s.act[:R], L["value"], s.ffn[:R])], ws)
            x, res_in = s.ffn[:R], res2
        for B, T, r0, _, q0 in groups:
            n = B * T
            capi.add_last_layer_norm(B, T, C, x[r0:r0 + n], res_in[r0:r0 + n], m.ln_out_w, m.ln_out_b,
                                     s.h[q0:q0 + B])
        capi.gemm(self._head_problem(S), ws)
        return s.logits[:S]


def gemm_flops(cfg, rows, seqs):
    """Matrix-core flops of one mixed step: every projection and FFN GEMM over `rows`
    rows, the head over `seqs` rows."""
    C, F = cfg.n_embd, cfg.dim_ffn
    r = cfg.rank_w + cfg.rank_a + cfg.rank_g + cfg.rank_v
    per_layer = 2 * rows * (4 * C * C + 2 * C * r + 2 * C * F)
    return cfg.n_layer * per_layer + 2 * seqs * C * cfg.vocab


__all__ = ["MixedEngine", "gemm_flops", "HEAD"]
