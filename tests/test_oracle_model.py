"""Pins oracle/model_ref.py, the float32 restatement of the RWKV-7 decode step that
the GPU decode driver is compared with (the reference ships no model code).

Three kinds of check, none of which retypes model_ref's own formulas:
  * each stage function of model_ref agrees with the already-pinned oracle
    function restating the same reference kernel (ops_ref.py, wkv_oracle.c);
  * decode_step agrees with an independent step-by-step composition of those
    pinned functions (numpy float64 stages, the C WKV oracle), and three wiring
    mistakes planted in that composition -- k instead of new_k in the bonus, the
    channel mix fed from the block input instead of the residual stream, the r
    and k lerps swapped -- each disagree with it far beyond the tolerance;
  * closed forms the mathematics fixes: with W_o = value = 0 every layer is the
    identity on the residual stream; with every lerp weight 1 the WKV update
    cannot depend on the current token, with every lerp weight 0 not on the
    shift rows; a zero state and r orthogonal to k' give y = 0.
"""
import math
import types

import numpy as np
import pytest
import torch

from oracle import model_ref as M
from oracle import ops_ref as R
from oracle import oracle as orc
from vkwr.model_executor.rwkv7 import LAYER_VECS, RWKV7Config

F16, F64 = np.float16, np.float64
TMIX = M.TMIX
CFG = RWKV7Config(n_layer=2, n_embd=128, dim_ffn=256, rank_w=16, rank_a=16, rank_v=8, rank_g=32, vocab=64)


def tiny_model(cfg=CFG, seed=0):
    """Host fp16 weights scaled so every path carries O(1) signal: projections std
    1/sqrt(in), embedding rows N(0,1), decays spread over (0.55, 1)."""
    g = torch.Generator().manual_seed(seed)
    C, F = cfg.n_embd, cfg.dim_ffn

    def mat(o, i, s=1.0):
        return (torch.randn(o, i, generator=g) * s / math.sqrt(i)).half()

    def vec(kind):
        if kind in ("ln1_w", "ln2_w", "lnx_w", "k_a"):
            return (1.0 + 0.2 * torch.randn(C, generator=g)).half()
        if kind.startswith("x_"):
            return torch.rand(C, generator=g).half()
        if kind == "k_k":
            return (0.7 + 0.3 * torch.rand(C, generator=g)).half()
        if kind == "w0":
            return (-3.0 + 4.0 * torch.rand(C, generator=g)).half()
        return (0.3 * torch.randn(C, generator=g)).half()

    layers = []
    for l in range(cfg.n_layer):
        L = {k: vec(k) for k in LAYER_VECS}
        L.update(Wr=mat(C, C), Wk=mat(C, C), Wv=mat(C, C), Wo=mat(C, C, 0.5), w1=mat(cfg.rank_w, C),
                 w2=mat(C, cfg.rank_w), a1=mat(cfg.rank_a, C), a2=mat(C, cfg.rank_a), g1=mat(cfg.rank_g, C),
                 g2=mat(C, cfg.rank_g), key=mat(F, C), value=mat(C, F, 0.5))
        if l > 0:
            L.update(v1=mat(cfg.rank_v, C), v2=mat(C, cfg.rank_v))
        layers.append(L)
    return types.SimpleNamespace(cfg=cfg, layers=layers, emb=torch.randn(cfg.vocab, C, generator=g).half(),
                                 ln_out_w=vec("ln1_w"), ln_out_b=vec("ln1_b"), head=mat(cfg.vocab, C))


def tiny_state(cfg=CFG, P=6, seed=1):
    g = torch.Generator().manual_seed(seed)
    wkv = torch.randn(cfg.n_layer, P, cfg.n_head, 64, 64, generator=g) * 0.3
    att = torch.randn(cfg.n_layer, P, cfg.n_embd, generator=g).half()
    ffn = torch.randn(cfg.n_layer, P, cfg.n_embd, generator=g).half()
    return wkv, att, ffn


def ref_step(model, state, tokens, slots, rd=True):
    wkv, att, ffn = (t.clone() for t in state)
    logits = M.decode_step(model, wkv, att, ffn, torch.tensor(tokens), torch.tensor(slots), round_fp16=rd)
    return logits.numpy().astype(F64), (wkv, att, ffn)


def n(t):
    return t.numpy()


# ------------------------------------------------------------------ composition of pinned functions


def compose(model, state, tokens, slots, plant=None):
    """The decode step wired from the pinned oracle functions: ops_ref (float64 stages, fp16
    outputs) and the C WKV oracle (fp32, the reference's one-chain order).  `plant` names a
    wiring mistake to insert.  Returns (logits float64, (wkv, att, ffn) numpy)."""
    cfg = model.cfg
    H, C = cfg.n_head, cfg.n_embd
    wkv, att, ffn = (n(t).copy() for t in state)
    tok, sl = np.asarray(tokens), np.asarray(slots)
    B = len(tok)
    x = n(model.emb)[tok]
    res = np.zeros_like(x)
    v_first = None
    for l, Lt in enumerate(model.layers):
        L = {k: n(v) for k, v in Lt.items()}
        x_in = x
        # ---- time mix
        res, xx = R.layer_norm(x, L["ln1_w"], L["ln1_b"], residual=res)
        prev = att[l, sl].copy()
        mix = {m: R.lerp16(xx, prev, L[m]) for m in TMIX}
        att[l, sl] = xx
        xr, xk = (mix["x_k"], mix["x_r"]) if plant == "swap_rk_lerp" else (mix["x_r"], mix["x_k"])
        r = R.gemm(xr, L["Wr"])[0]
        k = R.gemm(xk, L["Wk"])[0]
        v = R.gemm(mix["x_v"], L["Wv"])[0]
        w1 = R.gemm(mix["x_w"], L["w1"])[0]
        w = (R._f(L["w0"]) + R._f(R.act_tanh(w1)) @ R._f(L["w2"]).T).astype(F16)
        a12 = R.gemm(R.gemm(mix["x_a"], L["a1"])[0], L["a2"])[0]
        g = R.gemm(R.act_sigmoid(R.gemm(mix["x_g"], L["g1"])[0]), L["g2"])[0]
        if l == 0:
            v_first = v
        else:
            v12 = R._f(R.gemm(mix["x_v"], L["v1"])[0]) @ R._f(L["v2"]).T
            v = R.vres_gate(v, v_first, L["v0"], v12)
        new_k, neg_kk, kka = (t[:, 0] for t in R.kk_a_gate(k[:, None], L["k_k"], L["a0"], a12[:, None], L["k_a"], H))
        y = orc.wkv_fp32_slots(B, 1, C, H, wkv[l], sl.astype(np.int64),
                               *(t.reshape(B, 1, C) for t in (r, w, new_k, v, neg_kk, kka)))[:, 0]
        bonus_k = k if plant == "bonus_k" else new_k
        o_in = R.groupnorm_bonus_gate(y[:, None], r[:, None], bonus_k[:, None], v[:, None], L["r_k"], L["lnx_w"],
                                      L["lnx_b"], g[:, None], H)[:, 0]
        o = R.gemm(o_in, L["Wo"])[0]
        # ---- channel mix
        res, xx2 = R.layer_norm(o, L["ln2_w"], L["ln2_b"], residual=x_in if plant == "ffn_residual" else res)
        xk2 = R.lerp16(xx2, ffn[l, sl].copy(), L["x_k_ffn"])
        ffn[l, sl] = xx2
        act = R.gemm(xk2, L["key"], epi="relu2")[0]
        x = R.gemm(act, L["value"])[0]
    h = R.layer_norm(x, n(model.ln_out_w), n(model.ln_out_b), residual=res)[1]
    return R._f(h) @ R._f(n(model.head)).T, (wkv, att, ffn)


TOKENS, SLOTS = [5, 17, 63, 0], [3, 0, 5, 2]


def _rel_err(a, b):
    return np.abs(a - b).max() / np.abs(b).max()


COMPOSE_TOL = 1e-2  # measured ~1e-3: fp16 rounding flips of float32-vs-float64 intermediates


def test_decode_step_equals_composition_of_pinned_functions():
    model, state = tiny_model(), tiny_state()
    got, (wkv, att, ffn) = ref_step(model, state, TOKENS, SLOTS)
    want, (wkv_c, att_c, ffn_c) = compose(model, state, TOKENS, SLOTS)
    err = _rel_err(got, want)
    print(f"model_ref vs composition: logits rel err {err:.3g}")
    assert err <= COMPOSE_TOL
    np.testing.assert_allclose(n(wkv), wkv_c, atol=2e-2 * np.abs(wkv_c).max())
    # the shift rows are fp16 LN outputs: equal up to rare one-ulp flips
    for a, b in ((att, att_c), (ffn, ffn_c)):
        d = np.abs(R._f(n(a)) - R._f(b))
        assert (d <= 2 * R.ulp16(b) + 1e-3).mean() >= 0.99
    untouched = [s for s in range(wkv.shape[1]) if s not in SLOTS]
    assert torch.equal(wkv[:, untouched], state[0][:, untouched])
    assert torch.equal(att[:, untouched], state[1][:, untouched])


@pytest.mark.parametrize("plant", ["bonus_k", "ffn_residual", "swap_rk_lerp"])
def test_planted_wiring_mistakes_are_caught(plant):
    """Each mistake moves the logits far outside the tolerance the correct wiring meets."""
    model, state = tiny_model(), tiny_state()
    got, _ = ref_step(model, state, TOKENS, SLOTS)
    bad, _ = compose(model, state, TOKENS, SLOTS, plant=plant)
    assert _rel_err(got, bad) > 10 * COMPOSE_TOL, plant


# ------------------------------------------------------------------ stage functions


def _t(x):
    return torch.from_numpy(R._f(x)).float()


def _within_ulp(got, want, ulps=1, atol=2e-5):
    g = R._f(got.numpy() if torch.is_tensor(got) else got)
    w = R._f(want)
    assert (np.abs(g - w) <= ulps * R.ulp16(w) + atol).all(), np.abs(g - w).max()


rng = np.random.default_rng(3)


def h16(*s, sc=1.0):
    return (rng.standard_normal(s) * sc).astype(F16)


def test_stage_add_layer_norm_and_lerp():
    x, res, w, b = h16(5, 256), h16(5, 256, sc=3), 1 + h16(256, sc=0.1), h16(256, sc=0.1)
    x_out, y = M.add_layer_norm(_t(x), _t(res), _t(w), _t(b), True)
    xo_r, y_r = R.layer_norm(x, w, b, residual=res)
    _within_ulp(x_out, xo_r)
    _within_ulp(y, y_r)
    prev, mu = h16(5, 256), rng.random(256).astype(F16)
    _within_ulp(M.lerp(_t(y_r), _t(prev), _t(mu), True), R.lerp16(y_r, prev, mu))


def test_stage_kk_a_gate_and_groupnorm():
    H = 4
    k, a12 = h16(3, 256), h16(3, 256)
    k_k, a0, k_a = (0.8 + 0.2 * rng.random(256)).astype(F16), h16(256, sc=0.5), 1 + h16(256, sc=0.1)
    got = M.kk_a_gate(_t(k), _t(k_k), _t(a0), _t(a12), _t(k_a), H, True)
    want = R.kk_a_gate(k[:, None], k_k, a0, a12[:, None], k_a, H)
    for g_, w_ in zip(got, want):
        _within_ulp(g_, w_[:, 0])
    y, r, kk, v, g = (h16(3, 256) for _ in range(5))
    r_k, lw, lb = h16(256, sc=0.5), 1 + h16(256, sc=0.1), h16(256, sc=0.1)
    got = M.groupnorm_bonus_gate(_t(y), _t(r), _t(kk), _t(v), _t(r_k), _t(lw), _t(lb), _t(g), H, True)
    want = R.groupnorm_bonus_gate(y[:, None], r[:, None], kk[:, None], v[:, None], r_k, lw, lb, g[:, None], H)[:, 0]
    _within_ulp(got, want, ulps=2, atol=1e-4)


def test_stage_decay_equals_pinned_decay():
    ws = np.arange(65536, dtype=np.uint16).view(F16)
    ws = ws[np.isfinite(ws)][::7]
    got = M.decay(torch.from_numpy(ws.astype(np.float32))).numpy().astype(F64)
    want = np.array([orc.decay(float(w)) for w in ws])
    assert np.abs(got / want - 1).max() < 1e-6


def test_stage_wkv7_equals_c_oracle():
    """model_ref's WKV (torch float32, matmul order) against the C oracle's fp32 recurrence on
    config-0 distributions: equal within fp32 re-association."""
    from tests.wkv_inputs import make_state, make_wkv_inputs
    B, H = 3, 2
    C = H * 64
    ins = make_wkv_inputs(B, 1, H, seed=9)
    S0 = make_state(B, H, seed=9, std=0.5)
    S_c = S0.copy()
    y_c = orc.wkv_fp32(B, 1, C, H, S_c, *ins)
    y, S = M.wkv7(torch.from_numpy(S0), *(_t(t[:, 0]) for t in ins), True)
    np.testing.assert_allclose(S.numpy(), S_c, rtol=0, atol=2e-6)
    _within_ulp(y, y_c[:, 0], ulps=1, atol=1e-5)


def test_stage_wkv7_zero_state_orthogonal_r_gives_zero():
    """S = 0: S' = v k'^T (the sa term vanishes), so y = v (k' . r) = 0 for r orthogonal to k'."""
    B, H = 2, 2
    C = H * 64
    g = np.random.default_rng(4)
    k = g.standard_normal((B, C))
    r = g.standard_normal((B, C))
    kh, rh = k.reshape(B, H, 64), r.reshape(B, H, 64)
    rh -= (rh * kh).sum(-1, keepdims=True) / (kh * kh).sum(-1, keepdims=True) * kh
    w, v, a, b = (torch.from_numpy(g.standard_normal((B, C))).float() for _ in range(4))
    y, S = M.wkv7(torch.zeros(B, H, 64, 64), torch.from_numpy(rh.reshape(B, C)).float(), w,
                  torch.from_numpy(k).float(), v, a, b, False)
    assert y.abs().max().item() < 1e-5
    assert torch.allclose(S, v.view(B, H, 64, 1) * torch.from_numpy(k).float().view(B, H, 1, 64))


# ------------------------------------------------------------------ closed forms


def test_closed_form_zero_output_projections_make_layers_identity():
    """W_o = value = 0: every block adds 0 to the residual stream, so
    logits = LN_out(emb[tok]) . head^T, and each layer's shift rows are LN1 / LN2 of emb[tok]."""
    model = tiny_model()
    for L in model.layers:
        L["Wo"] = torch.zeros_like(L["Wo"])
        L["value"] = torch.zeros_like(L["value"])
    state = tiny_state()
    got, (_, att, ffn) = ref_step(model, state, TOKENS, SLOTS)
    e = n(model.emb)[TOKENS]
    h = R.layer_norm(e, n(model.ln_out_w), n(model.ln_out_b))[1]
    want = R._f(h) @ R._f(n(model.head)).T
    assert _rel_err(got, want) < 1e-5
    for l, L in enumerate(model.layers):
        _within_ulp(att[l, SLOTS], R.layer_norm(e, n(L["ln1_w"]), n(L["ln1_b"]))[1])
        _within_ulp(ffn[l, SLOTS], R.layer_norm(e, n(L["ln2_w"]), n(L["ln2_b"]))[1])


def _set_mix(model, value):
    for L in model.layers:
        for m in TMIX + ("x_k_ffn",):
            L[m] = torch.full_like(L[m], value)


def test_closed_form_unit_lerps_make_the_wkv_update_token_independent():
    """Every lerp weight 1: each mix is the previous token's LN output exactly, so every WKV
    input of every layer comes from the shift rows and the state update cannot see the token.
    Two slots with equal states, fed different tokens, stay bitwise equal; their new shift
    rows (the LN of the current token's residual) differ."""
    model = tiny_model()
    _set_mix(model, 1.0)
    wkv, att, ffn = tiny_state()
    for t in (wkv, att, ffn):
        t[:, 4] = t[:, 1]
    _, (wkv2, att2, ffn2) = ref_step(model, (wkv, att, ffn), [7, 40], [1, 4])
    assert torch.equal(wkv2[:, 1], wkv2[:, 4])
    assert not torch.equal(att2[:, 1], att2[:, 4])
    assert not torch.equal(wkv2[:, 1], wkv[:, 1])


def test_closed_form_zero_lerps_make_the_wkv_update_shift_independent():
    """Every lerp weight 0: each mix is the current token's LN output, so with the same token
    and the same WKV state, different shift rows give the same WKV state and logits."""
    model = tiny_model()
    _set_mix(model, 0.0)
    wkv, att, ffn = tiny_state()
    wkv[:, 4] = wkv[:, 1]
    assert not torch.equal(att[:, 1], att[:, 4])
    logits, (wkv2, _, _) = ref_step(model, (wkv, att, ffn), [7, 7], [1, 4])
    assert torch.equal(wkv2[:, 1], wkv2[:, 4])
    assert np.array_equal(logits[0], logits[1])
