"""Pins the LayerNorm / GroupNorm / token-shift / gate / GEMM oracle
(oracle/ops_ref.py) against independent routines: torch's float64 layer_norm,
group_norm, normalize, lerp, sigmoid and matmul, and brute-force loops for the
token shift, the GEMM and the channel mix.  Planted mistakes (unbiased
variance, a transposed weight) are shown to be caught."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops_ref as R

rng = np.random.default_rng(0)


def h(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def t64(x):
    return torch.from_numpy(np.asarray(x).astype(np.float64))


@pytest.mark.parametrize("C", [64, 2048, 4096, 8192, 77])
def test_layer_norm_matches_torch(C):
    x, w, b = h(3, 5, C, scale=2.0), h(C), h(C)
    _, y = R.layer_norm(x, w, b, 1e-5)
    ref = F.layer_norm(t64(x), (C,), t64(w), t64(b), 1e-5).numpy().astype(np.float16)
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16))


def test_layer_norm_with_residual_uses_unrounded_sum():
    C = 512
    x, r, w, b = h(4, C, scale=3.0), h(4, C, scale=3.0), h(C), h(C)
    x_out, y = R.layer_norm(x, w, b, 1e-5, residual=r)
    v = t64(x) + t64(r)
    assert np.array_equal(x_out, v.numpy().astype(np.float16))
    ref = F.layer_norm(v, (C,), t64(w), t64(b), 1e-5).numpy().astype(np.float16)
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16))


def test_planted_unbiased_variance_is_caught():
    C = 64
    x, w, b = h(8, C, scale=2.0), np.ones(C, np.float16), np.zeros(C, np.float16)
    v = x.astype(np.float64)
    bad = ((v - v.mean(-1, keepdims=True)) / np.sqrt(v.var(-1, ddof=1, keepdims=True) + 1e-5)).astype(np.float16)
    ref = F.layer_norm(t64(x), (C,), eps=1e-5).numpy().astype(np.float16)
    assert not np.array_equal(bad, ref)
    assert np.array_equal(R.layer_norm(x, w, b)[1], ref)


def test_add_last_layer_norm_takes_last_token():
    B, T, C = 3, 4, 128
    x, r, w, b = h(B, T, C), h(B, T, C), h(C), h(C)
    y = R.add_last_layer_norm(x, r, w, b)
    ref = F.layer_norm(t64(x[:, -1]) + t64(r[:, -1]), (C,), t64(w), t64(b), 1e-5).numpy().astype(np.float16)
    assert y.shape == (B, C) and np.array_equal(y, ref)


def test_emb_ln0_bf16_decoding():
    V, C = 5, 256
    e = torch.randn(V, C).to(torch.bfloat16)
    w = torch.randn(C).to(torch.bfloat16)
    b = torch.randn(C).to(torch.bfloat16)
    y = R.emb_ln0(e.view(torch.int16).numpy().view(np.uint16), w.view(torch.int16).numpy().view(np.uint16),
                  b.view(torch.int16).numpy().view(np.uint16))
    ref = F.layer_norm(e.double(), (C,), w.double(), b.double(), 1e-5).numpy().astype(np.float16)
    assert np.array_equal(y, ref)


def test_groupnorm_bonus_gate_matches_torch():
    B, T, H = 2, 3, 4
    C = 64 * H
    x, r, k, v, g = (h(B, T, C) for _ in range(5))
    r_k, w, b = h(C), h(C), h(C)
    got = R.groupnorm_bonus_gate(x, r, k, v, r_k, w, b, g, H)
    gn = F.group_norm(t64(x).reshape(B * T, C), H, t64(w), t64(b), eps=64e-5).reshape(B, T, C)
    bonus = (t64(r) * t64(k) * t64(r_k)).reshape(B, T, H, 64).sum(-1, keepdim=True) * t64(v).reshape(B, T, H, 64)
    ref = ((gn + bonus.reshape(B, T, C)) * t64(g)).numpy().astype(np.float16)
    assert np.array_equal(got, ref)


def test_kk_a_gate_matches_torch():
    B, T, H = 2, 2, 3
    C = 64 * H
    k, a12 = h(B, T, C), h(B, T, C)
    k_k, a0, k_a = h(C), h(C), h(C)
    new_k, neg_kk, kka = R.kk_a_gate(k, k_k, a0, a12, k_a, H)
    u = (t64(k) * t64(k_k)).reshape(B, T, H, 64)
    kk = F.normalize(u, dim=-1, eps=1e-12).reshape(B, T, C)
    a = torch.sigmoid(t64(a0) + t64(a12))
    assert np.array_equal(neg_kk, (-kk).numpy().astype(np.float16))
    assert np.array_equal(kka, (kk * a).numpy().astype(np.float16))
    ref_k = (t64(k) * (1 + (a - 1) * t64(k_a))).numpy()
    assert np.abs(new_k.astype(np.float64) - ref_k).max() <= R.ulp16(ref_k).max()
    # BASELINE's a = -kk, b = kk * a_vec construction is this op with k_k = 1.
    ones = np.ones(C, np.float16)
    _, neg_kk1, _ = R.kk_a_gate(k, ones, a0, a12, k_a, H)
    kk1 = F.normalize(t64(k).reshape(B, T, H, 64), dim=-1).reshape(B, T, C)
    assert np.array_equal(neg_kk1, (-kk1).numpy().astype(np.float16))


@pytest.mark.parametrize("T", [1, 2, 5, 33])
def test_token_shift_brute_force(T):
    B, C = 3, 16
    x = h(B, T, C)
    shift0 = h(B, C)
    mixes = [h(C) for _ in range(6)]
    shift = shift0.copy()
    outs = R.token_shift(x, shift, mixes)
    for i, m in enumerate(mixes):
        for b in range(B):
            for t in range(T):
                prev = shift0[b] if t == 0 else x[b, t - 1]
                ref = torch.lerp(t64(x[b, t]), t64(prev), t64(m)).numpy().astype(np.float16)
                assert np.array_equal(outs[i][b, t], ref)
    assert np.array_equal(shift, x[:, -1])


def test_token_shift_half_math_rounds_difference_first():
    cur = np.array([1.0], np.float16)
    prev = np.array([1.0 + 2 ** -10], np.float16)   # prev - cur = 2^-10, exact in fp16
    mix = np.array([0.5], np.float16)
    assert R.lerp16_half_math(cur, prev, mix)[0] == np.float16(1.0 + 2 ** -11)
    prev = np.array([2 ** -25 + 0.0], np.float16)    # underflows to 0 in fp16
    assert R.lerp16(np.array([0.0], np.float16), prev, mix)[0] == 0


def test_add_layer_norm_mix_updates_shift():
    B, C = 4, 256
    x, r, w, b = h(B, 1, C), h(B, 1, C), h(C), h(C)
    shift = h(B, C)
    prev = shift.copy()
    mixes = [h(C) for _ in range(6)]
    res = R.add_layer_norm_mix(x, r, shift, w, b, mixes)
    x_out, y = R.layer_norm(x, w, b, residual=r)
    assert np.array_equal(res[0], x_out)
    assert np.array_equal(shift, y.reshape(B, C))
    for m, o in zip(mixes, res[1:]):
        assert np.array_equal(o, torch.lerp(t64(y), t64(prev).reshape(B, 1, C), t64(m)).numpy().astype(np.float16))


def test_vres_gate_and_activations_match_torch():
    v, vf, v12 = h(2, 3, 64), h(2, 3, 64), h(2, 3, 64)
    v0 = h(64)
    ref = torch.lerp(t64(v), t64(vf), torch.sigmoid(t64(v0) + t64(v12))).numpy().astype(np.float16)
    assert np.array_equal(R.vres_gate(v, vf, v0, v12), ref)
    x = h(1000, scale=3.0)
    assert np.array_equal(R.relu_square(x), (torch.relu(t64(x)) ** 2).numpy().astype(np.float16))
    assert np.array_equal(R.act_tanh(x), torch.tanh(t64(x)).numpy().astype(np.float16))
    assert np.array_equal(R.act_sigmoid(x), torch.sigmoid(t64(x)).numpy().astype(np.float16))


def test_ulp16():
    assert R.ulp16(1.0) == 2 ** -10
    assert R.ulp16(1.5) == 2 ** -10
    assert R.ulp16(2.0) == 2 ** -9
    assert R.ulp16(0.0) == 2 ** -24
    assert R.ulp16(65504.0) == 32.0


# ---------------------------------------------------------------- GEMM oracle

@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_gemm_matches_torch_and_brute_force(layout):
    a = h(5, 37)
    w = h(23, 37, scale=0.1) if layout == "nk" else h(37, 23, scale=0.1)
    y, abs_sum = R.gemm(a, w, layout)
    wt = t64(w).t() if layout == "nk" else t64(w)
    assert np.array_equal(y, (t64(a) @ wt).numpy().astype(np.float16))
    assert np.allclose(abs_sum, (t64(a).abs() @ wt.abs()).numpy())
    # brute-force loop on a few entries
    for i, j in [(0, 0), (4, 22), (2, 11)]:
        s = sum(float(a[i, k]) * float(w[j, k] if layout == "nk" else w[k, j]) for k in range(37))
        assert abs(float(y[i, j]) - s) <= float(R.ulp16(s))


def test_gemm_planted_transposition_is_caught():
    a, w = h(8, 16), h(16, 16, scale=0.1)  # square: both layouts are shape-valid
    y_nk, _ = R.gemm(a, w, "nk")
    y_kn, _ = R.gemm(a, w, "kn")
    assert not np.array_equal(y_nk, y_kn)
    assert np.array_equal(y_nk, R.gemm(a, np.ascontiguousarray(w.T), "kn")[0])


def test_gemm_activation_and_epilogues():
    a, w = h(6, 40), h(30, 40, scale=0.2)
    for act, f in (("tanh", torch.tanh), ("sigmoid", torch.sigmoid), ("relu2", lambda x: torch.relu(x) ** 2)):
        a_act = f(t64(a)).numpy()
        y, _ = R.gemm(a, w, "nk", a_act=act)  # round_act: the activation is rounded to fp16 first
        assert np.array_equal(y, (torch.from_numpy(a_act.astype(np.float16).astype(np.float64)) @ t64(w).t())
                              .numpy().astype(np.float16))
        y32, _ = R.gemm(a, w, "nk", a_act=act, round_act=False)
        assert np.array_equal(y32, (torch.from_numpy(a_act) @ t64(w).t()).numpy().astype(np.float16))
    acc = (t64(a) @ t64(w).t()).numpy()
    y, _ = R.gemm(a, w, "nk", epi="relu2")
    assert np.array_equal(y, R.relu_square(acc))
    v, vf, v0 = h(6, 30), h(6, 30), h(30)
    y, _ = R.gemm(a, w, "nk", epi="vres", v=v, v_first=vf, v0=v0)
    assert np.array_equal(y, R.vres_gate(v, vf, v0, acc))  # the independently pinned gate on the fp64 accumulator
    eye = np.eye(40, dtype=np.float16)
    assert np.array_equal(R.gemm(a, eye, "nk")[0], a)  # identity weight


def test_cmix_sparse_brute_force():
    B, T, C, F = 2, 3, 8, 5
    x, shift = h(B, T, C), h(B, C)
    x_k = rng.random(C).astype(np.float16)
    key, value = h(F, C, scale=0.3), h(F, C, scale=0.3)
    shift_ref = shift.copy()
    out, act, _ = R.cmix_sparse(x, shift, x_k, key, value)
    assert np.array_equal(shift, x[:, -1])
    for b in range(B):
        for t in range(T):
            prev = shift_ref[b] if t == 0 else x[b, t - 1]
            mixed = [np.float16(float(x[b, t, c]) + (float(prev[c]) - float(x[b, t, c])) * float(x_k[c]))
                     for c in range(C)]
            hid = [np.float16(max(sum(float(mixed[c]) * float(key[f, c]) for c in range(C)), 0.0) ** 2)
                   for f in range(F)]
            assert np.array_equal(np.array(hid, dtype=np.float16), act[b * T + t])
            for c in range(C):
                s = sum(float(hid[f]) * float(value[f, c]) for f in range(F))
                assert abs(float(out[b, t, c]) - s) <= float(R.ulp16(s))
