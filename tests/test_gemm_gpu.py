"""GPU parity of the fp16 GEMM family (vkwr_v1_linear, vkwr_v1_rank, the
vkwr_v1_mix channel-mix ops) against the float64 oracle (oracle/ops_ref.py).

Bar (floating point): |gpu - oracle| <= 1 fp16 ulp of the oracle value
+ 1e-5 * sum_k |a_k b_k| (fp32 accumulation over K, with the split-K partial
sums), + 2^-11 * sum_k |act(a_k) b_k| where the A-operand activation is rounded
to fp16 on the GPU but not in the reference's rank adapters.  Epilogues are
checked through their derivatives.  Also restated: the reference's own linear
tests (tests/ops/test_v1_linear_ops.py) -- shapes, NaN, zero input, torch.matmul
at atol/rtol 5e-3 -- and its validation errors for the tuning arguments.
"""
import numpy as np
import pytest
import torch

from oracle import ops_ref as R

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(7)
ACC = 1e-5          # fp32 accumulation slack, relative to sum |a b|
ACT = 2.0 ** -11    # fp16 rounding of an activated A operand (half an ulp, relative)


def h(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


def check(got, ref, slack, what=""):
    g = got.detach().cpu().numpy().astype(np.float64) if torch.is_tensor(got) else got.astype(np.float64)
    r = ref.astype(np.float64)
    bound = R.ulp16(r) + slack
    bad = np.abs(g - r) > bound
    assert not bad.any(), (what, int(bad.sum()), float(np.abs(g - r).max()), float(bound.min()))


GEMM_SHAPES = [  # (M, K, N)
    (1, 64, 64), (1, 4096, 512), (3, 72, 100), (5, 70, 40), (128, 2048, 2048), (128, 2048, 96),
    (128, 96, 2048), (64, 256, 320), (17, 512, 1024), (300, 1024, 768), (1024, 512, 512),
]


@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_gemm_vs_oracle(gpu, M, K, N, layout):
    from vkwr._ops.v1 import v1_linear_ops as L
    a = h(M, K)
    w = h(N, K, scale=0.05) if layout == "nk" else h(K, N, scale=0.05)
    y = (L.linear_f16_orig if layout == "nk" else L.linear_f16)(dev(a, gpu), dev(w, gpu))
    assert y.shape == (M, N) and y.dtype == torch.float16
    ref, abs_sum = R.gemm(a, w, layout)
    check(y, ref, ACC * abs_sum, f"{layout} {M}x{K}x{N}")


def test_gemm_deterministic_and_split_k(gpu):
    """Small-M shapes take the K-split path; results are run-to-run identical."""
    from vkwr._ops.v1 import v1_linear_ops as L
    a, w = dev(h(128, 8192), gpu), dev(h(2048, 8192, scale=0.02), gpu)
    y1 = L.linear_f16_orig(a, w)
    y2 = L.linear_f16_orig(a, w)
    assert torch.equal(y1, y2)
    ref, abs_sum = R.gemm(a.cpu().numpy(), w.cpu().numpy(), "nk")
    check(y1, ref, ACC * abs_sum, "128x8192x2048")


def test_all_linear_ops_compute_the_same_function(gpu):
    from vkwr._ops.v1 import v1_linear_ops as L
    B, T, K, N = 2, 3, 256, 512
    x = dev(h(B, T, K), gpu)
    w_kn = dev(h(K, N, scale=0.05), gpu)
    w_nk = w_kn.t().contiguous()
    base = L.linear_f16(x, w_kn)
    assert base.shape == (B, T, N)
    same = [
        L.linear_f16_lt(x, w_kn), L.linear_f16_rows_splitk(x, w_kn, 256),
        L.linear_f16_orig(x, w_nk), L.linear_orig_rows_f16(x, w_nk, 4, 8),
        L.linear_orig_rows_cfg_f16(x, w_nk, 64, 4, 4), L.linear_orig_wmma16_f16(x, w_nk),
        L.linear_f16_orig_lt(x, w_nk), L.linear_f16_orig_lt_cfg(x, w_nk, 4, 0), L.linear_t_f16(x, w_nk),
    ]
    for y in same:
        assert torch.equal(y, base)
    x1 = dev(h(1, K), gpu)
    b1 = L.linear_f16(x1, w_kn)
    for y in (L.linear_f16_m1_splitk(x1, w_kn), L.linear_f16_m1_splitk_cfg(x1, w_kn, 160),
              L.linear_f16_m1_splitk_tile(x1, w_kn, 128, 128), L.linear_f16_m1_splitk_warpred_tile(x1, w_kn, 64, 64)):
        assert y.shape == (1, N) and torch.equal(y, b1)
    x2 = dev(h(2, K), gpu)
    assert torch.equal(L.linear_orig_rows_exact_f16(x2, w_nk, 128, 2, False), L.linear_f16_orig(x2, w_nk))
    assert torch.equal(L.linear_orig_rows_exact_f16(x1, w_nk, 128, 2, True), L.linear_f16_orig(x1, w_nk))


def test_linear_validation_errors(gpu):
    from vkwr._ops.v1 import v1_linear_ops as L
    K, N = 128, 256
    x = dev(h(2, 4, K), gpu)
    w = dev(h(K, N), gpu)
    wo = w.t().contiguous()
    bad_calls = [
        lambda: L.linear_f16(dev(h(2, 4, K + 1), gpu), w),          # shape mismatch
        lambda: L.linear_f16(x.float(), w),                          # dtype
        lambda: L.linear_f16(dev(h(2, 4, 2 * K), gpu)[..., ::2], w),  # non-contiguous
        lambda: L.linear_orig_rows_f16(x, wo, 5, 2),
        lambda: L.linear_orig_rows_cfg_f16(x, wo, 128, 4, 4),
        lambda: L.linear_orig_rows_exact_f16(x, wo, 128, 2, False),  # 8 rows
        lambda: L.linear_f16_orig_lt_cfg(x, wo, 2048, 0),
        lambda: L.linear_f16_orig_lt_cfg(x, wo, 4, 64),
        lambda: L.linear_f16_m1_splitk(x, w),                         # M != 1
        lambda: L.linear_f16_m1_splitk_cfg(dev(h(1, K), gpu), w, 100),
        lambda: L.linear_f16_m1_splitk_tile(dev(h(1, K), gpu), w, 128, 32),
        lambda: L.linear_f16_m1_splitk_warpred_tile(dev(h(1, K), gpu), w, 384, 64),
        lambda: L.linear_f16_rows_splitk(x, w, 64),
        lambda: L.linear_t_act_f16(dev(h(1, 64), gpu), dev(h(1024, 64), gpu), 3),
        lambda: L.linear_t_act_f16(dev(h(8, 64), gpu), dev(h(1024, 64), gpu), 1),  # M > 4
        lambda: L.linear_orig_wmma16_f16(dev(h(2, 72), gpu), dev(h(64, 72), gpu)),
    ]
    for i, call in enumerate(bad_calls):
        with pytest.raises(RuntimeError):
            call()
            pytest.fail(f"call {i} did not raise")
    v = dev(h(1, 1024), gpu)
    with pytest.raises(RuntimeError):  # v0 shape (reference test_linear_t_vres_f16_v0_shape_mismatch)
        L.linear_t_vres_f16(dev(h(1, 64), gpu), dev(h(1024, 64), gpu), v, v, dev(h(512), gpu))


@pytest.mark.parametrize("act", [1, 2])
def test_linear_t_act_and_vres(gpu, act):
    from vkwr._ops.v1 import v1_linear_ops as L
    M, K, N = 4, 96, 2048
    x, w = h(M, K), h(N, K, scale=0.1)
    y = L.linear_t_act_f16(dev(x, gpu), dev(w, gpu), act)
    ref, abs_sum = R.gemm(x, w, "nk", a_act="tanh" if act == 1 else "sigmoid", round_act=False)
    check(y, ref, (ACC + ACT) * abs_sum, "t_act")
    v, vf, v0 = h(M, N), h(M, N), h(N)
    y = L.linear_t_vres_f16(dev(x, gpu), dev(w, gpu), dev(v, gpu), dev(vf, gpu), dev(v0, gpu))
    ref, abs_sum = R.gemm(x, w, "nk", epi="vres", v=v, v_first=vf, v0=v0)
    check(y, ref, 0.25 * np.abs(vf.astype(np.float64) - v) * ACC * abs_sum, "t_vres")


def test_linear_reference_unit_tests(gpu):
    """reference tests/ops/test_v1_linear_ops.py: shapes, NaN, zero input, vs torch.matmul."""
    from vkwr._ops.v1 import v1_linear_ops as L
    for B, T, K, N in [(1, 1, 64, 128), (2, 4, 128, 256), (1, 16, 256, 512), (4, 8, 512, 1024)]:
        x = torch.randn(B, T, K, dtype=torch.float16, device=gpu)
        w = torch.randn(K, N, dtype=torch.float16, device=gpu)
        y = L.linear_f16(x, w)
        assert y.shape == (B, T, N) and not torch.isnan(y).any()
    x = torch.randn(2, 4, 128, dtype=torch.float16, device=gpu)
    w = torch.randn(128, 256, dtype=torch.float16, device=gpu)
    torch.testing.assert_close(L.linear_f16(x, w), torch.matmul(x.float(), w.float()).half(), atol=5e-3, rtol=5e-3)
    wo = torch.randn(256, 128, dtype=torch.float16, device=gpu)
    torch.testing.assert_close(L.linear_f16_orig(x, wo), torch.matmul(x.float(), wo.float().t()).half(),
                               atol=5e-3, rtol=5e-3)
    torch.testing.assert_close(L.linear_t_f16(x, wo), torch.matmul(x.float(), wo.float().t()).half(),
                               atol=5e-3, rtol=5e-3)
    assert (L.linear_f16(torch.zeros_like(x), w) == 0).all()
    y = L.linear_f16(torch.randn(1, 1, 4096, dtype=torch.float16, device=gpu),
                     torch.randn(4096, 8192, dtype=torch.float16, device=gpu) * 0.02)
    assert y.shape == (1, 1, 8192) and not torch.isnan(y).any()


# ------------------------------------------------------------------ rank adapters

@pytest.mark.parametrize("M,C,ranks", [(128, 2048, (96, 96, 256, 64)), (3, 256, (32, 16, 64, 8)),
                                       (1, 4096, (128, 128, 480, 96))])
def test_rank_in_out(gpu, M, C, ranks):
    from vkwr._ops.v1 import v1_rank_ops as K
    Rw, Ra, Rg, Rv = ranks
    xs = [h(M, C) for _ in range(4)]
    w1s = [h(r, C, scale=0.02) for r in ranks]
    outs = K.linear_wagv_rank_in_f16(M, C, Rw, Ra, Rg, Rv, *(dev(a, gpu) for a in xs + w1s))
    assert [tuple(o.shape) for o in outs] == [(M, r) for r in ranks]
    for o, x, w in zip(outs, xs, w1s):
        ref, abs_sum = R.gemm(x, w, "nk")
        check(o, ref, ACC * abs_sum, "rank_in")
    outs3 = K.linear_wag_rank_in_f16(M, C, Rw, Ra, Rg, *(dev(a, gpu) for a in xs[:3] + w1s[:3]))
    assert all(torch.equal(a, b) for a, b in zip(outs3, outs[:3]))

    ins = [o.cpu().numpy() for o in outs]
    w2s = [h(C, r, scale=0.1) for r in ranks]
    v, vf, v0 = h(M, C), h(M, C), h(C)
    res = K.linear_wagv_rank_out_f16(M, C, Rw, Ra, Rg, Rv, *(dev(a, gpu) for a in ins + w2s + [v, vf, v0]))
    acts = ["tanh", None, "sigmoid", None]
    for i, (o, x, w, act) in enumerate(zip(res, ins, w2s, acts)):
        if i < 3:
            ref, abs_sum = R.gemm(x, w, "nk", a_act=act, round_act=False)
            check(o, ref, (ACC + (ACT if act else 0)) * abs_sum, f"rank_out {i}")
        else:
            ref, abs_sum = R.gemm(x, w, "nk", epi="vres", v=v, v_first=vf, v0=v0)
            check(o, ref, 0.25 * np.abs(vf.astype(np.float64) - v) * ACC * abs_sum, "rank_out v")
    res3 = K.linear_wag_rank_out_f16(M, C, Rw, Ra, Rg, *(dev(a, gpu) for a in ins[:3] + w2s[:3]))
    assert all(torch.equal(a, b) for a, b in zip(res3, res[:3]))


def test_rank_validation_errors(gpu):
    from vkwr._ops.v1 import v1_rank_ops as K
    M, C = 2, 128
    x = dev(h(M, C), gpu)
    w = dev(h(16, C), gpu)
    with pytest.raises(RuntimeError):
        K.linear_wag_rank_in_f16(M, C, 16, 16, 8, x, x, x, w, w, w)  # g1_t shape
    with pytest.raises(RuntimeError):
        K.linear_wag_rank_out_f16(M, C, 16, 16, 16, x, x, x, w, w, w)  # w1 shape


# ------------------------------------------------------------------ channel mix (FFN)

@pytest.mark.parametrize("B,T,C,F", [(1, 1, 256, 256), (2, 8, 256, 512), (128, 1, 2048, 8192), (1, 4, 512, 1024)])
def test_cmix_sparse(gpu, B, T, C, F):
    from vkwr._ops.v1 import v1_mix_ops as M
    x, shift0 = h(B, T, C), h(B, C)
    x_k = rng.random(C).astype(np.float16)
    key, value = h(F, C, scale=0.05), h(F, C, scale=0.05)
    shift = dev(shift0, gpu)
    if B == 1 and T == 1:
        y = M.cmix_sparse_one(C, F, dev(x, gpu), shift, dev(x_k, gpu), dev(key, gpu), dev(value, gpu))
    else:
        y = M.cmix_sparse_rows(B, T, C, F, dev(x, gpu), shift, dev(x_k, gpu), dev(key, gpu), dev(value, gpu))
    assert y.shape == (B, T, C)
    s_ref = shift0.copy()
    ref, act, abs_sum = R.cmix_sparse(x, s_ref, x_k, key, value)
    assert np.array_equal(shift.cpu().numpy(), s_ref)
    # act may differ by 1 fp16 ulp where the up projection straddles a rounding boundary
    act_slack = ((np.abs(act.astype(np.float64)) * 2.0 ** -9) @ np.abs(value.astype(np.float64))).reshape(B, T, C)
    check(y, ref, ACC * abs_sum + act_slack, "cmix")


def test_cmix_down_ops(gpu):
    from vkwr._ops.v1 import v1_mix_ops as M
    B, T, C, F = 2, 3, 512, 1024
    pre = h(B, T, F)
    value = h(F, C, scale=0.05)
    act = R.relu_square(pre)
    y = M.cmix_sparse_down_rows(B, T, C, F, dev(act, gpu), dev(value, gpu))
    ref, abs_sum = R.gemm(act.reshape(B * T, F), value, "kn")
    check(y.reshape(B * T, C), ref, ACC * abs_sum, "down_rows")
    for fn in (M.cmix_sparse_down_relu_rows, M.cmix_sparse_down_relu_rows_t512):
        y2 = fn(B, T, C, F, dev(pre, gpu), dev(value, gpu))
        assert torch.equal(y2, y)
    y1 = M.cmix_sparse_down_one(C, F, dev(act[0, 0], gpu), dev(value, gpu))
    assert y1.shape == (1, 1, C)
    check(y1.view(1, C), ref[:1], ACC * abs_sum[:1], "down_one")
    y1r = M.cmix_sparse_down_relu_one(C, F, dev(pre[0, 0], gpu), dev(value, gpu))
    assert torch.equal(y1r, y1)
    with pytest.raises(RuntimeError):
        M.cmix_sparse_down_relu_rows_t512(B, T, 256, F, dev(h(B, T, F), gpu), dev(h(F, 256), gpu))
    with pytest.raises(RuntimeError):
        x100 = dev(h(1, 1, 100), gpu)
        M.cmix_sparse_one(100, 128, x100, dev(h(1, 100), gpu), dev(h(100), gpu), dev(h(128, 100), gpu),
                          dev(h(128, 100), gpu))


@pytest.mark.parametrize("M,K,N", [(1, 8192, 2048), (2, 16384, 4096), (4, 1032, 1000), (1, 2048, 65536)])
def test_gemv_kn_skips_zero_activation_rows(gpu, M, K, N):
    """The [K,N] GEMV reads only the weight rows where some activation row is nonzero (the
    reference's activation-sparse down projection, mix_ops.cu:522-583): weight rows under an
    all-zero activation column are filled with NaN here, and the result must still be the
    dense product of the remaining rows.  Zeros are +0 and -0 alike; the pattern has
    runs of zeros longer and shorter than a wave's 64-row ballot, and one K part with no
    nonzero row at all."""
    from vkwr._ops.v1 import v1_linear_ops as L
    a = h(M, K)
    live = rng.random(K) < 0.3
    live[: min(K, 700)] = False        # a run of zero rows across ballots and K parts
    live[K // 2: K // 2 + 5] = True
    a[:, ~live] = 0.0
    a[0, ~live & (np.arange(K) % 3 == 0)] = np.float16(-0.0)
    if M > 1:
        # a row live in only one of the activation rows is still read
        a[1:, K // 2] = 0.0
    w = h(K, N, scale=0.05)
    ref, abs_sum = R.gemm(a, w, "kn")
    w[~live, :] = np.nan
    y = L.linear_f16(dev(a, gpu), dev(w, gpu))
    assert torch.isfinite(y).all()
    check(y, ref, ACC * abs_sum, f"sparse kn {M}x{K}x{N}")
    z = L.linear_f16(dev(np.zeros((M, K), np.float16), gpu), dev(w, gpu))
    assert torch.equal(z, torch.zeros_like(z))


def test_cmix_down_relu_one_sparse_shapes(gpu):
    """cmix_sparse_down_relu_one at the 1.5B and 7B FFN shapes (relu^2 leaves about half
    of the rows zero) against the oracle."""
    from vkwr._ops.v1 import v1_mix_ops as M
    for C, F in ((2048, 8192), (4096, 16384)):
        pre = h(F)
        value = h(F, C, scale=0.05)
        act = R.relu_square(pre)
        ref, abs_sum = R.gemm(act.reshape(1, F), value, "kn")
        y = M.cmix_sparse_down_relu_one(C, F, dev(pre, gpu), dev(value, gpu))
        check(y.view(1, C), ref, ACC * abs_sum, f"down_relu_one {C}x{F}")


# ---------------------------------------------------------------- large-M path

def _big_vs_rowmajor(gpu, shapes, epis, seed):
    """One launch over `shapes` ([N,K] weights: the 256x256 large-M kernel when eligible) and
    the same launch over the transposed [K,N] copies (never eligible: the row-major kernel,
    unsplit for M > 256).  Both feed the same MFMA operands in the same k order from zero
    and apply the same epilogue arithmetic, so the results are the same bits."""
    from vkwr_amd import capi
    outs = []
    for layout in (capi.GEMM_B_NK, capi.GEMM_B_KN):
        probs, keep = [], []
        for i, ((M, K, N), epi) in enumerate(zip(shapes, epis)):
            g = torch.Generator(device=gpu).manual_seed(seed + 1000 * i)  # same tensors for both layouts
            a = torch.randn(M, K, device=gpu, generator=g).half()
            w = (torch.randn(N, K, device=gpu, generator=g) * 0.05).half()
            c = torch.empty(M, N, dtype=torch.float16, device=gpu)
            v = torch.randn(M, N, device=gpu, generator=g).half()
            vf = torch.randn(M, N, device=gpu, generator=g).half()
            v0 = torch.randn(N, device=gpu, generator=g).half()
            b = w if layout == capi.GEMM_B_NK else w.t().contiguous()
            probs.append(capi.gemm_problem(a, b, c, b_layout=layout, epilogue=epi, v=v, v_first=vf, v0=v0))
            keep += [a, b, c, v, vf, v0]
        ws = torch.empty(max(capi.gemm_workspace_bytes(probs), 0), dtype=torch.uint8, device=gpu)
        capi.gemm(probs, ws)
        torch.cuda.synchronize()
        outs.append([keep[i * 6 + 2].clone() for i in range(len(shapes))])
    return outs


@pytest.mark.parametrize("shapes,epis", [
    ([(300, 1024, 768)], [0]),
    ([(257, 64, 1000)], [1]),                        # one row past a tile, K of one stage, relu^2
    ([(768, 448, 1280)], [3]),                       # 15 tiles (not a multiple of the 8 XCDs), bias
    ([(600, 512, 700), (600, 512, 96), (600, 512, 256), (600, 512, 512)], [1, 0, 3, 2]),  # mixed epilogues
    ([(2304, 4096, 4096)], [0]),                     # the 7B o-projection shape: 192-row tiles (192 of them)
    ([(2304, 128, 4096), (2304, 512, 4096)], [3, 2]),  # 7B low-rank outputs: bias, value residual
])
def test_big_gemm_bitwise_equals_rowmajor_kernel(gpu, shapes, epis):
    """Launches whose tiles all run whole (no k-parts), in 256- or 192-row tiles: the same bits as
    the row-major kernel."""
    big, ref = _big_vs_rowmajor(gpu, shapes, epis, seed=11)
    for i, (x, y) in enumerate(zip(big, ref)):
        assert torch.equal(x, y), (shapes[i], epis[i], float((x.float() - y.float()).abs().max()))


def test_big_gemm_split_small_batch_tanh_sigmoid(gpu):
    """The 7B low-rank inputs alone (w1 padded to 128 columns with tanh, g1 to 512 with sigmoid):
    36 tiles of 192 rows, each split into k-parts (fp32 partials, ordered fixup): within one fp16
    ulp plus the fp32 re-association bound of the row-major kernel's result (the activations'
    slopes are at most 1), and run-to-run identical."""
    shapes, epis = [(2304, 4096, 128), (2304, 4096, 512)], [4, 5]
    big, ref = _big_vs_rowmajor(gpu, shapes, epis, seed=11)
    big2, _ = _big_vs_rowmajor(gpu, shapes, epis, seed=11)
    for i, (M, K, N) in enumerate(shapes):
        g = torch.Generator(device=gpu).manual_seed(11 + 1000 * i)
        a = torch.randn(M, K, device=gpu, generator=g).half()
        w = (torch.randn(N, K, device=gpu, generator=g) * 0.05).half()
        abs_sum = (a.abs().float() @ w.abs().float().t()).double()
        r = ref[i].double()
        ulp = torch.exp2(torch.floor(torch.log2(r.abs().clamp_min(2.0 ** -14))) - 10)
        err = (big[i].double() - r).abs()
        bound = ulp + ACC * abs_sum
        assert bool((err <= bound).all()), (shapes[i], float(err.max()), int((err > bound).sum()))
        assert torch.equal(big[i], big2[i])


@pytest.mark.parametrize("M,K,N", [(300, 256, 200), (2304, 512, 256)])
def test_tanh_sigmoid_epilogues(gpu, M, K, N):
    """c = tanh(a b^T) and sigmoid(a b^T), fp32 accumulation, against torch in float64."""
    from vkwr_amd import capi
    g = torch.Generator(device=gpu).manual_seed(M + N)
    a = torch.randn(M, K, device=gpu, generator=g).half()
    w = (torch.randn(N, K, device=gpu, generator=g) * 0.05).half()
    ref = a.double() @ w.double().t()
    for epi, fn in ((capi.EPI_TANH, torch.tanh), (capi.EPI_SIGMOID, torch.sigmoid)):
        c = torch.empty(M, N, dtype=torch.float16, device=gpu)
        p = [capi.gemm_problem(a, w, c, epilogue=epi)]
        ws = torch.empty(max(capi.gemm_workspace_bytes(p), 0), dtype=torch.uint8, device=gpu)
        capi.gemm(p, ws)
        torch.cuda.synchronize()
        # fp16 output rounding (2^-11 relative, |y| <= 1) plus the fp32 sum's rounding
        assert (c.double() - fn(ref)).abs().max().item() <= 2e-3


def test_big_gemm_batch_with_empty_problem_and_oracle(gpu):
    """A launch whose batch holds an empty problem between eligible ones; every output against
    the float64 oracle."""
    from vkwr_amd import capi
    shapes = [(384, 256, 520), (0, 256, 64), (384, 256, 200)]
    a = [h(M, K) for M, K, N in shapes]
    w = [h(N, K, scale=0.05) for M, K, N in shapes]
    da = [dev(x, gpu) for x in a]
    dw = [dev(x, gpu) for x in w]
    c = [torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu) for M, K, N in shapes]
    probs = [capi.gemm_problem(x, y, z) for x, y, z in zip(da, dw, c)]
    capi.gemm(probs, torch.empty(0, dtype=torch.uint8, device=gpu))
    torch.cuda.synchronize()
    for i, (M, K, N) in enumerate(shapes):
        if M == 0:
            continue
        ref, abs_sum = R.gemm(a[i], w[i], "nk")
        check(c[i], ref, ACC * abs_sum, f"batch problem {i}")


@pytest.mark.parametrize("M,K,N", [
    (128, 1024, 8192),   # 64x64 tiles for both layouts (256 tiles)
    (64, 512, 16384),    # the same with one row tile
    (100, 2048, 8200),   # ragged M and N
])
def test_small_m_kn_fragments_equal_nk_bitwise(gpu, M, K, N):
    """Where both weight layouts get the same 64x64 tiles of the small-M kernel, its [K,N]
    fragments (transposing LDS reads) and [N,K] fragments (plain 16-byte reads) feed the
    matrix cores the same operand values in the same lanes and order, so the two layouts of
    one weight give the same bits (a wrong lane layout of the transposing read would not).
    The other [K,N] shapes are checked against the oracle in test_gemm_vs_oracle."""
    from vkwr_amd import capi
    g = torch.Generator(device=gpu).manual_seed(M + K + N)
    a = torch.randn(M, K, device=gpu, generator=g).half()
    w = (torch.randn(N, K, device=gpu, generator=g) * 0.02).half()
    out = []
    for b, layout in ((w, capi.GEMM_B_NK), (w.t().contiguous(), capi.GEMM_B_KN)):
        c = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
        p = [capi.gemm_problem(a, b, c, b_layout=layout, a_act=capi.ACT_RELU_SQUARE)]
        ws = torch.empty(max(capi.gemm_workspace_bytes(p), 1), dtype=torch.uint8, device=gpu)
        capi.gemm(p, ws)
        out.append(c)
    torch.cuda.synchronize()
    assert not torch.isnan(out[0]).any()
    assert torch.equal(out[0], out[1])


@pytest.mark.parametrize("M,K,N", [
    (1024, 16384, 2048),   # 32 tiles, long K: every tile split into 8 k-parts
    (2304, 16384, 4096),   # the 7B FFN value shape: 144 tiles of 256 stages, layered split
                           # (144 stages per CU: [0, 144) of every tile, [144, 256) of 112 tiles
                           # whole, the other 32 in 16-stage pieces)
    (2304, 8192, 4096),    # 144 tiles of 128 stages: per 72, layered with 8-stage pieces
    (4096, 16384, 6400),   # 400 tiles: 256 whole, the other 144 layered (tile indices offset by 256)
    (2304, 4096, 8192),    # 288 tiles: one whole round + a 32-tile tail split in 6
    (2304, 4096, 16384),   # the 7B FFN key shape: 768 whole 192-row tiles (three rounds, no split)
])
def test_big_gemm_split_tail(gpu, M, K, N):
    """Tail tiles split into k-parts or balanced pieces (fp32 partials, ordered fixup): against the row-major
    kernel on the transposed weight within the fp32 re-association bound, and run-to-run
    bitwise identical (also through the relu^2 epilogue)."""
    from vkwr_amd import capi
    g = torch.Generator(device=gpu).manual_seed(M + K + N)
    a = torch.randn(M, K, device=gpu, generator=g).half()
    w = (torch.randn(N, K, device=gpu, generator=g) * 0.02).half()
    wt = w.t().contiguous()

    def run(b, layout, epi=capi.EPI_NONE):
        c = torch.empty(M, N, dtype=torch.float16, device=gpu)
        p = [capi.gemm_problem(a, b, c, b_layout=layout, epilogue=epi)]
        ws = torch.empty(max(capi.gemm_workspace_bytes(p), 0), dtype=torch.uint8, device=gpu)
        capi.gemm(p, ws)
        return c

    nk = run(w, capi.GEMM_B_NK)
    kn = run(wt, capi.GEMM_B_KN)
    abs_sum = (a.abs().float() @ w.abs().float().t())
    torch.cuda.synchronize()
    ref = kn.double()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - 10)
    bound = ulp + ACC * abs_sum.double()
    err = (nk.double() - ref).abs()
    assert bool((err <= bound).all()), (float(err.max()), int((err > bound).sum()))
    r1 = run(w, capi.GEMM_B_NK, capi.EPI_RELU_SQUARE)
    r2 = run(w, capi.GEMM_B_NK, capi.EPI_RELU_SQUARE)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2)


# (M, K, N, layout): decode-sized shapes that take the small-M LDS-staged kernel, one per tile
# shape -- 64 x 64 (M > 32, enough tiles), 32 x 64, 32 x 32, [K,N] weights at 64 and 32 rows --
# with ragged M, K (a multiple of 8, not of 64) and N.
RM_SHAPES = [
    (128, 2048, 8192, "nk"), (100, 1000, 8200, "nk"), (128, 2048, 2048, "nk"), (8, 2048, 16384, "nk"),
    (24, 264, 16392, "nk"), (128, 2048, 8192, "kn"), (77, 1032, 10248, "kn"), (5, 4096, 16384, "kn"),
]
# GEMV-shaped (M <= 4): [N,K] rows streamed per wave; [K,N] columns per workgroup, K split
# over workgroups (fp32 partials + ordered reduce) when the columns alone leave CUs idle.
GV_SHAPES = [
    (1, 4096, 4096, "nk"), (3, 1000, 1032, "nk"), (4, 8192, 2056, "nk"), (2, 2048, 96, "nk"),
    (1, 4096, 4096, "kn"), (1, 2048, 65536, "kn"), (2, 16384, 4096, "kn"), (3, 1032, 1000, "kn"),
    (4, 4096, 16384, "kn"),
]


@pytest.mark.parametrize("M,K,N,layout", RM_SHAPES + GV_SHAPES)
def test_small_m_lds_kernel_vs_oracle(gpu, M, K, N, layout):
    from vkwr._ops.v1 import v1_linear_ops as L
    a = h(M, K)
    w = h(N, K, scale=0.05) if layout == "nk" else h(K, N, scale=0.05)
    y = (L.linear_f16_orig if layout == "nk" else L.linear_f16)(dev(a, gpu), dev(w, gpu))
    y2 = (L.linear_f16_orig if layout == "nk" else L.linear_f16)(dev(a, gpu), dev(w, gpu))
    assert torch.equal(y, y2)  # deterministic
    ref, abs_sum = R.gemm(a, w, layout)
    check(y, ref, ACC * abs_sum, f"{layout} {M}x{K}x{N}")


@pytest.mark.parametrize("act,epi", [("tanh", "none"), ("sigmoid", "bias"), ("relu2", "vres"), (None, "relu2")])
def test_small_m_lds_kernel_activations_and_epilogues(gpu, act, epi):
    """A-operand activations (rounded to fp16, as the staging kernels do) and the fused
    epilogues on the small-M kernel, in a batch of three problems (M = 96, N = 2048..4104)."""
    from vkwr_amd import capi
    acts = {None: capi.ACT_NONE, "tanh": capi.ACT_TANH, "sigmoid": capi.ACT_SIGMOID, "relu2": capi.ACT_RELU_SQUARE}
    epis = {"none": capi.EPI_NONE, "bias": capi.EPI_BIAS, "vres": capi.EPI_VALUE_RESIDUAL, "relu2": capi.EPI_RELU_SQUARE}
    M, K = 96, 512
    probs, keep, refs = [], [], []
    for N in (2048, 4104, 3072):
        a, w = h(M, K), h(N, K, scale=0.05)
        v, vf, v0 = h(M, N), h(M, N), h(N)
        c = torch.empty(M, N, dtype=torch.float16, device=gpu)
        ta, tw, tv, tvf, tv0 = (dev(x, gpu) for x in (a, w, v, vf, v0))
        probs.append(capi.gemm_problem(ta, tw, c, a_act=acts[act], epilogue=epis[epi],
                                       v=tv if epi == "vres" else None, v_first=tvf if epi == "vres" else None,
                                       v0=tv0 if epi in ("bias", "vres") else None))
        keep += [ta, tw, tv, tvf, tv0, c]
        y64, abs_sum = R.gemm(a, w, "nk", a_act=act, epi="relu2" if epi == "relu2" else None)
        if epi in ("bias", "vres"):
            pre, abs_sum = R.gemm(a, w, "nk", a_act=act)
            a64 = R._act(R._f(a), act)
            if act is not None:
                a64 = a64.astype(np.float16).astype(np.float64)
            z = a64 @ R._f(w).T
            if epi == "bias":
                y64 = (z + R._f(v0)).astype(np.float16)
            else:
                y64 = R.vres_gate(v, vf, v0, z)
        refs.append((c, y64, abs_sum))
    assert capi.gemm_workspace_bytes(probs) == 0  # the small-M kernel needs no workspace
    capi.gemm(probs, torch.empty(0, dtype=torch.uint8, device=gpu))
    torch.cuda.synchronize()
    for c, y64, abs_sum in refs:
        # epilogue derivatives are bounded by 1 (sigmoid gate: 1/4 of |v_first - v| <= a few)
        slack = ACC * abs_sum * (8.0 if epi == "vres" else 1.0)
        if epi == "relu2":
            slack = 2 * np.abs(np.sqrt(y64.astype(np.float64))) * ACC * abs_sum + ACC * abs_sum
        check(c, y64, slack, f"{act} {epi}")


@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("act,epi", [("tanh", "none"), ("sigmoid", "bias"), (None, "vres"), ("relu2", "relu2")])
def test_gemv_activations_and_epilogues(gpu, layout, act, epi):
    """The GEMV kernels (M = 3) with A-operand activations and fused epilogues."""
    from vkwr_amd import capi
    acts = {None: capi.ACT_NONE, "tanh": capi.ACT_TANH, "sigmoid": capi.ACT_SIGMOID, "relu2": capi.ACT_RELU_SQUARE}
    epis = {"none": capi.EPI_NONE, "bias": capi.EPI_BIAS, "vres": capi.EPI_VALUE_RESIDUAL, "relu2": capi.EPI_RELU_SQUARE}
    M, K, N = 3, 2048, 1032
    a = h(M, K)
    w = h(N, K, scale=0.05) if layout == "nk" else h(K, N, scale=0.05)
    v, vf, v0 = h(M, N), h(M, N), h(N)
    c = torch.empty(M, N, dtype=torch.float16, device=gpu)
    ta, tw, tv, tvf, tv0 = (dev(x, gpu) for x in (a, w, v, vf, v0))
    prob = capi.gemm_problem(ta, tw, c, b_layout=capi.GEMM_B_NK if layout == "nk" else capi.GEMM_B_KN,
                             a_act=acts[act], epilogue=epis[epi], v=tv if epi == "vres" else None,
                             v_first=tvf if epi == "vres" else None, v0=tv0 if epi in ("bias", "vres") else None)
    ws = torch.empty(max(capi.gemm_workspace_bytes([prob]), 1), dtype=torch.uint8, device=gpu)
    capi.gemm([prob], ws)
    torch.cuda.synchronize()
    a64 = R._act(R._f(a), act)
    if act is not None:
        a64 = a64.astype(np.float16).astype(np.float64)
    wt = R._f(w).T if layout == "nk" else R._f(w)
    z = a64 @ wt
    abs_sum = np.abs(a64) @ np.abs(wt)
    if epi == "none":
        y64 = z.astype(np.float16)
    elif epi == "bias":
        y64 = (z + R._f(v0)).astype(np.float16)
    elif epi == "vres":
        y64 = R.vres_gate(v, vf, v0, z)
    else:
        y64 = (np.maximum(z, 0) ** 2).astype(np.float16)
    slack = ACC * abs_sum * (8.0 if epi == "vres" else 1.0)
    if epi == "relu2":
        slack = 2 * np.sqrt(np.abs(y64.astype(np.float64))) * ACC * abs_sum + ACC * abs_sum
    check(c, y64, slack, f"{layout} {act} {epi}")
