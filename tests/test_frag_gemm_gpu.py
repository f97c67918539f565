"""GPU parity of the fragment-layout path (vkwr_frag_* of include/vkwr_amd.h):
the weight / activation packing, the decode GEMM with every epilogue and
output layout, and the frag-output producers, against the float64 oracle
(oracle/ops_ref.py) and against the row-major entry points.

Bar (floating point): |gpu - oracle| <= 1 fp16 ulp of the oracle value
+ 1e-5 * sum_k |a_k b_k| (fp32 accumulation; the K split over waves adds the
partials in a fixed order).  Packing is exact (bit-identical round trip, zero
pads).  The frag-output producers are bit-identical to their row-major
siblings packed afterwards (same arithmetic, different store address).
"""
import numpy as np
import pytest
import torch

from oracle import ops_ref as R

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(11)
ACC = 1e-5


def h(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


def check(got, ref, slack, what=""):
    g = got.detach().cpu().numpy().astype(np.float64)
    r = ref.astype(np.float64)
    bound = R.ulp16(r) + slack
    bad = np.abs(g - r) > bound
    assert not bad.any(), (what, int(bad.sum()), float(np.abs(g - r).max()), float(bound.min()))


def pack(x, gpu, rows, k, layout=0):
    from vkwr_amd import capi
    src = dev(x, gpu)
    dst = capi.frag_empty(rows, k, gpu, zero=False).fill_(float("nan"))  # pads must be written as zero
    capi.frag_pack(src, rows, k, dst, layout)
    return dst


def unpack(p, rows, k, gpu):
    from vkwr_amd import capi
    out = torch.empty(rows, k, dtype=torch.float16, device=gpu)
    capi.frag_unpack(p, rows, k, out)
    return out


def frag_to_dense(p, rows, k):
    """Host-side decode of the frag layout, written from its definition:
    fragment (row block, 16-k step) = 64 lanes x 8 halfs, lane = half-of-k * 32 + row % 32."""
    from vkwr_amd import capi
    rp, kp = capi.frag_pad(rows), capi.frag_pad(k)
    t = p.cpu().numpy()[: rp * kp].reshape(rp // 32, kp // 16, 2, 32, 8)  # [rb, ks, k-half, r%32, k%8]
    dense = t.transpose(0, 3, 1, 2, 4).reshape(rp, kp)
    return dense


@pytest.mark.parametrize("rows,k", [(1, 1), (5, 70), (32, 16), (128, 2048), (130, 96), (2048, 128), (96, 8200)])
def test_pack_round_trip_and_layout(gpu, rows, k):
    x = h(rows, k)
    p = pack(x, gpu, rows, k)
    dense = frag_to_dense(p, rows, k)
    assert np.array_equal(dense[:rows, :k].view(np.uint16), x.view(np.uint16))
    assert not dense[rows:].any() and not dense[:, k:].any()  # zero pads (no NaN left)
    back = unpack(p, rows, k, gpu).cpu().numpy()
    assert np.array_equal(back.view(np.uint16), x.view(np.uint16))


def test_pack_kn_equals_pack_of_transpose(gpu):
    w_kn = h(200, 96)  # [K, N]
    a = pack(w_kn, gpu, 96, 200, layout=1)
    b = pack(np.ascontiguousarray(w_kn.T), gpu, 96, 200, layout=0)
    assert torch.equal(a, b)


# (M, N, K): each line exercises one tile configuration of the launcher
CONFIG_SHAPES = [
    (128, 65536, 128),   # >= 1024 tiles of 64x64: 128x64 tiles, 4 waves
    (64, 65536, 256),    # the same with one row block half empty
    (128, 8192, 256),    # 64x64 tiles, KS 2
    (128, 4096, 128),    # 64x64 tiles, KS 1
    (128, 2048, 512),    # 32x32 tiles, KS 4
    (128, 2048, 256),    # 32x32 tiles, KS 2
    (100, 1024, 128),    # 32x32 tiles, KS 1, ragged M
    (17, 8192, 256),     # M <= 32: 32x64 tiles
    (1, 512, 2048),      # M <= 32: 32x32 tiles
    (5, 96, 96),         # padded N and K
    (200, 2048, 2048),   # M > 128
]


@pytest.mark.parametrize("M,N,K", CONFIG_SHAPES)
def test_frag_gemm_vs_oracle(gpu, M, N, K):
    from vkwr_amd import capi
    a, w = h(M, K), h(N, K, scale=0.05)
    pa, pw = pack(a, gpu, M, K), pack(w, gpu, N, K)
    n8 = (N + 7) // 8 * 8
    c = torch.full((M, n8), float("nan"), dtype=torch.float16, device=gpu)
    if n8 == N:
        capi.frag_gemm([capi.frag_problem(pa, pw, c, M, N, K)])
        ref, abs_sum = R.gemm(a, w, "nk")
        check(c, ref, ACC * abs_sum, f"{M}x{N}x{K}")
    cf = capi.frag_empty(M, N, gpu)
    capi.frag_gemm([capi.frag_problem(pa, pw, cf, M, N, K, c_frag=True)])
    dense = frag_to_dense(cf, M, N)
    ref, abs_sum = R.gemm(a, w, "nk")
    check(torch.from_numpy(dense[:M, :N].copy()), ref, ACC * abs_sum, f"frag {M}x{N}x{K}")
    assert not dense[:M, N:].any()  # pad columns = epilogue(0) = 0


def test_frag_gemm_head_rows_do_not_depend_on_batch(gpu):
    """Each wave takes the same k blocks and the wave partials are added in the same order
    whatever the batch, so the first 64 rows of the M = 128 head product equal the M = 64
    product bit for bit."""
    from vkwr_amd import capi
    N, K = 65536, 2048
    a, w = h(128, K), h(N, K, scale=0.05)
    pw = pack(w, gpu, N, K)
    c128 = torch.empty(128, N, dtype=torch.float16, device=gpu)
    c64 = torch.empty(64, N, dtype=torch.float16, device=gpu)
    capi.frag_gemm([capi.frag_problem(pack(a, gpu, 128, K), pw, c128, 128, N, K)])
    capi.frag_gemm([capi.frag_problem(pack(a[:64], gpu, 64, K), pw, c64, 64, N, K)])
    torch.cuda.synchronize()
    assert torch.equal(c128[:64], c64)


@pytest.mark.parametrize("epi", ["relu2", "tanh", "sigmoid"])
@pytest.mark.parametrize("c_frag", [False, True])
def test_frag_gemm_activation_epilogues(gpu, epi, c_frag):
    from vkwr_amd import capi
    M, N, K = 128, 2048, 2048
    code = {"relu2": capi.EPI_RELU_SQUARE, "tanh": capi.EPI_TANH, "sigmoid": capi.EPI_SIGMOID}[epi]
    a, w = h(M, K), h(N, K, scale=0.05)
    pa, pw = pack(a, gpu, M, K), pack(w, gpu, N, K)
    y, abs_sum = R.gemm(a, w, "nk")
    y64 = (a.astype(np.float64) @ w.astype(np.float64).T)
    ref = R._act(y64, epi)
    # derivative bound of the activation times the accumulation slack
    deriv = {"relu2": 2 * np.abs(y64) + 1e-3, "tanh": np.ones_like(y64), "sigmoid": 0.25 * np.ones_like(y64)}[epi]
    if c_frag:
        cf = capi.frag_empty(M, N, gpu)
        capi.frag_gemm([capi.frag_problem(pa, pw, cf, M, N, K, epilogue=code, c_frag=True)])
        got = torch.from_numpy(frag_to_dense(cf, M, N)[:M, :N].copy())
    else:
        got = torch.empty(M, N, dtype=torch.float16, device=gpu)
        capi.frag_gemm([capi.frag_problem(pa, pw, got, M, N, K, epilogue=code)])
    check(got, ref.astype(np.float16), deriv * ACC * abs_sum + 2e-6, epi)


def test_frag_gemm_value_residual_and_bias(gpu):
    from vkwr_amd import capi
    M, N, K = 128, 2048, 128
    a, w = h(M, K), h(N, K, scale=0.1)
    v, vf, v0 = h(M, N), h(M, N), h(N)
    pa, pw = pack(a, gpu, M, K), pack(w, gpu, N, K)
    out_v = torch.empty(M, N, dtype=torch.float16, device=gpu)
    out_b = torch.empty(M, N, dtype=torch.float16, device=gpu)
    capi.frag_gemm([
        capi.frag_problem(pa, pw, out_v, M, N, K, epilogue=capi.EPI_VALUE_RESIDUAL,
                          v=dev(v, gpu), v_first=dev(vf, gpu), v0=dev(v0, gpu)),
        capi.frag_problem(pa, pw, out_b, M, N, K, epilogue=capi.EPI_BIAS, v0=dev(v0, gpu)),
    ])
    ref_v, abs_sum = R.gemm(a, w, "nk", epi="vres", v=v, v_first=vf, v0=v0)
    d = np.abs(vf.astype(np.float64) - v.astype(np.float64)) * 0.25  # |d out / d acc| <= |vf - v| / 4
    check(out_v, ref_v, d * ACC * abs_sum + 2e-6, "vres")
    y = a.astype(np.float64) @ w.astype(np.float64).T + v0.astype(np.float64)
    check(out_b, y.astype(np.float16), ACC * abs_sum, "bias")


def test_frag_gemm_batch_mixed_problems_and_determinism(gpu):
    """The decode projection batch: r/k/v-like plus the low-rank inputs (N = 96,
    96, 256, 64, written as frag matrices with tanh / none / sigmoid)."""
    from vkwr_amd import capi
    M, K = 128, 2048
    specs = [(2048, capi.EPI_NONE, False), (2048, capi.EPI_NONE, False), (96, capi.EPI_TANH, True),
             (96, capi.EPI_NONE, True), (256, capi.EPI_SIGMOID, True), (64, capi.EPI_NONE, True)]
    acts = [h(M, K) for _ in specs]
    ws = [h(n, K, scale=0.05) for n, _, _ in specs]
    pas = [pack(x, gpu, M, K) for x in acts]
    pws = [pack(w, gpu, n, K) for w, (n, _, _) in zip(ws, specs)]
    outs = [capi.frag_empty(M, n, gpu) if f else torch.empty(M, n, dtype=torch.float16, device=gpu)
            for n, _, f in specs]
    probs = [capi.frag_problem(pa, pw, o, M, n, K, epilogue=e, c_frag=f)
             for pa, pw, o, (n, e, f) in zip(pas, pws, outs, specs)]
    capi.frag_gemm(probs)
    first = [o.clone() for o in outs]
    capi.frag_gemm(probs)
    for o, f0 in zip(outs, first):
        assert torch.equal(o, f0)
    for x, w, o, (n, e, f) in zip(acts, ws, outs, specs):
        y64 = x.astype(np.float64) @ w.astype(np.float64).T
        _, abs_sum = R.gemm(x, w, "nk")
        name = {capi.EPI_NONE: None, capi.EPI_TANH: "tanh", capi.EPI_SIGMOID: "sigmoid"}[e]
        ref = R._act(y64, name)
        got = torch.from_numpy(frag_to_dense(o, M, n)[:M, :n].copy()) if f else o
        check(got, ref.astype(np.float16), ACC * abs_sum + 2e-6, f"n={n}")


def test_frag_gemm_rank_out_chain(gpu):
    """tanh(x . w1^T) written as a frag matrix with its zero-weight pad columns
    feeds the next GEMM (K = 96 padded to 128) unchanged."""
    from vkwr_amd import capi
    M, C, R_ = 128, 2048, 96
    x, w1, w2 = h(M, C), h(R_, C, scale=0.05), h(C, R_, scale=0.1)
    px, pw1, pw2 = pack(x, gpu, M, C), pack(w1, gpu, R_, C), pack(w2, gpu, C, R_)
    hid = capi.frag_empty(M, R_, gpu)
    out = torch.empty(M, C, dtype=torch.float16, device=gpu)
    capi.frag_gemm([capi.frag_problem(px, pw1, hid, M, R_, C, epilogue=capi.EPI_TANH, c_frag=True)])
    capi.frag_gemm([capi.frag_problem(hid, pw2, out, M, C, R_)])
    h16 = np.tanh(x.astype(np.float64) @ w1.astype(np.float64).T).astype(np.float16)
    ref, abs_sum = R.gemm(h16, w2, "nk")
    # the hidden values differ from the oracle's by <= 1 ulp + accumulation slack
    _, s1 = R.gemm(x, w1, "nk")
    hid_err = (R.ulp16(h16.astype(np.float64)) + ACC * s1) @ np.abs(w2.astype(np.float64)).T
    check(out, ref, ACC * abs_sum + hid_err, "rank chain")


@pytest.mark.parametrize("M,N,K,splits", [(128, 2048, 8192, 4), (100, 2048, 8192, 8), (128, 512, 2048, 2),
                                          (1, 128, 1024, 4), (64, 256, 256, 1)])
def test_frag_gemm_splitk_vs_oracle(gpu, M, N, K, splits):
    """vkwr_frag_gemm_splitk_f16: K parts added in order by the reduce kernel;
    same bar as the unsplit kernel, run-to-run identical, and the workspace
    size formula."""
    from vkwr_amd import capi
    a, w = h(M, K), h(N, K, scale=0.05)
    pa, pw = pack(a, gpu, M, K), pack(w, gpu, N, K)
    need = capi.frag_splitk_workspace_bytes(M, N, splits)
    assert need == splits * ((M + 63) // 64 * 64) * capi.frag_pad(N) * 4
    ws = torch.full((need // 4,), float("nan"), dtype=torch.float32, device=gpu)
    c = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    capi.frag_gemm_splitk(capi.frag_problem(pa, pw, c, M, N, K), splits, ws)
    ref, abs_sum = R.gemm(a, w, "nk")
    check(c, ref, ACC * abs_sum, f"split {M}x{N}x{K}/{splits}")
    first = c.clone()
    capi.frag_gemm_splitk(capi.frag_problem(pa, pw, c, M, N, K), splits, ws)
    assert torch.equal(c, first)


@pytest.mark.parametrize("epi", ["relu2_frag", "tanh_frag", "vres", "bias"])
def test_frag_gemm_splitk_epilogues(gpu, epi):
    from vkwr_amd import capi
    M, N, K, splits = 128, 512, 4096, 4
    a, w = h(M, K), h(N, K, scale=0.02)
    v, vf, v0 = h(M, N), h(M, N), h(N)
    pa, pw = pack(a, gpu, M, K), pack(w, gpu, N, K)
    ws = torch.empty(capi.frag_splitk_workspace_bytes(M, N, splits) // 4, dtype=torch.float32, device=gpu)
    y64 = a.astype(np.float64) @ w.astype(np.float64).T
    _, abs_sum = R.gemm(a, w, "nk")
    if epi.endswith("_frag"):
        name = epi[:-5]
        code = {"relu2": capi.EPI_RELU_SQUARE, "tanh": capi.EPI_TANH}[name]
        cf = capi.frag_empty(M, N, gpu)
        capi.frag_gemm_splitk(capi.frag_problem(pa, pw, cf, M, N, K, epilogue=code, c_frag=True), splits, ws)
        got = torch.from_numpy(frag_to_dense(cf, M, N)[:M, :N].copy())
        deriv = 2 * np.abs(y64) + 1e-3 if name == "relu2" else np.ones_like(y64)
        check(got, R._act(y64, name).astype(np.float16), deriv * ACC * abs_sum + 2e-6, epi)
        return
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    if epi == "vres":
        capi.frag_gemm_splitk(capi.frag_problem(pa, pw, out, M, N, K, epilogue=capi.EPI_VALUE_RESIDUAL,
                                                v=dev(v, gpu), v_first=dev(vf, gpu), v0=dev(v0, gpu)), splits, ws)
        ref, _ = R.gemm(a, w, "nk", epi="vres", v=v, v_first=vf, v0=v0)
        d = np.abs(vf.astype(np.float64) - v.astype(np.float64)) * 0.25
        check(out, ref, d * ACC * abs_sum + 2e-6, epi)
    else:
        capi.frag_gemm_splitk(capi.frag_problem(pa, pw, out, M, N, K, epilogue=capi.EPI_BIAS, v0=dev(v0, gpu)),
                              splits, ws)
        check(out, (y64 + v0.astype(np.float64)).astype(np.float16), ACC * abs_sum, epi)


def test_frag_gemm_splitk_rejects_bad_arguments(gpu):
    from vkwr_amd import capi
    a = capi.frag_empty(128, 1024, gpu)
    b = capi.frag_empty(128, 1024, gpu)
    c = torch.empty(128 * 128, dtype=torch.float16, device=gpu)
    ws = torch.empty(capi.frag_splitk_workspace_bytes(128, 128, 4) // 4, dtype=torch.float32, device=gpu)
    p = capi.frag_problem(a, b, c, 128, 128, 1024)
    with pytest.raises(RuntimeError, match="multiple of 256"):
        capi.frag_gemm_splitk(p, 8, ws)  # 1024 / 8 < 256
    with pytest.raises(RuntimeError, match="workspace of"):
        capi.frag_gemm_splitk(p, 4, ws[:-4])
    with pytest.raises(RuntimeError, match="splits"):
        capi.frag_gemm_splitk(p, 0, ws)


def test_frag_gemm_rejects_bad_arguments(gpu):
    from vkwr_amd import capi
    a = capi.frag_empty(128, 128, gpu)
    b = capi.frag_empty(128, 128, gpu)
    c = torch.empty(128 * 128, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError, match="row-major output"):
        capi.frag_gemm([capi.frag_problem(a, b, c, 128, 128, 128, epilogue=capi.EPI_BIAS, c_frag=True, v0=c)])
    with pytest.raises(RuntimeError, match="n % 8"):
        capi.frag_gemm([capi.frag_problem(a, b, c, 128, 100, 128)])
    big = capi.frag_empty(256, 128, gpu)
    with pytest.raises(RuntimeError, match="aligned"):
        capi.frag_gemm([capi.frag_problem(big[1:], b, c, 128, 128, 128)])


# ------------------------------------------------------------ frag producers

def test_ln_mix_frag_equals_packed_row_major(gpu):
    from vkwr_amd import capi
    rows, C = 100, 2048
    x, res = dev(h(rows, C), gpu), dev(h(rows, C), gpu)
    wt, bs = dev(h(C), gpu), dev(h(C), gpu)
    mixes = [dev(rng.random(C).astype(np.float16), gpu) for _ in range(6)]
    shift0 = dev(h(rows, C), gpu)
    s1, s2 = shift0.clone(), shift0.clone()
    xo1, xo2 = torch.empty_like(x), torch.empty_like(x)
    outs = [torch.empty_like(x) for _ in range(6)]
    fouts = [capi.frag_empty(rows, C, gpu) for _ in range(6)]
    capi.add_layer_norm_mix(x, res, s1, wt, bs, mixes, xo1, outs)
    capi.add_layer_norm_mix(x, res, s2, wt, bs, mixes, xo2, fouts, frag=True)
    assert torch.equal(xo1, xo2) and torch.equal(s1, s2)
    for o, f in zip(outs, fouts):
        assert np.array_equal(frag_to_dense(f, rows, C)[:rows].view(np.uint16), o.cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("rows,C,K,splits,n_mix", [(128, 2048, 8192, 4, 6), (100, 2048, 4096, 8, 6),
                                                   (64, 4096, 2048, 2, 1)])
def test_ln_mix_parts_equals_reduce_then_ln(gpu, rows, C, K, splits, n_mix):
    """vkwr_add_layer_norm_mix_parts_frag_f16 on the unreduced planes of
    vkwr_frag_gemm_splitk_parts_f16 is bit-identical to
    vkwr_frag_gemm_splitk_f16 followed by vkwr_add_layer_norm_mix_frag_f16."""
    from vkwr_amd import capi
    a, w = h(rows, K), h(C, K, scale=0.05)
    pa, pw = pack(a, gpu, rows, K), pack(w, gpu, C, K)
    res = dev(h(rows, C), gpu)
    wt, bs = dev(h(C), gpu), dev(h(C), gpu)
    mixes = [dev(rng.random(C).astype(np.float16), gpu) for _ in range(n_mix)]
    shift0 = dev(h(rows, C), gpu)
    s1, s2 = shift0.clone(), shift0.clone()
    xo1, xo2 = torch.empty(rows, C, dtype=torch.float16, device=gpu), torch.empty(rows, C, dtype=torch.float16,
                                                                                 device=gpu)
    o1 = [capi.frag_empty(rows, C, gpu) for _ in range(n_mix)]
    o2 = [capi.frag_empty(rows, C, gpu) for _ in range(n_mix)]
    ws = torch.empty(capi.frag_splitk_workspace_bytes(rows, C, splits) // 4, dtype=torch.float32, device=gpu)
    y = torch.empty(rows, C, dtype=torch.float16, device=gpu)
    capi.frag_gemm_splitk(capi.frag_problem(pa, pw, y, rows, C, K), splits, ws)
    capi.add_layer_norm_mix(y, res, s1, wt, bs, mixes, xo1, o1, frag=True)
    ws.fill_(float("nan"))
    capi.frag_gemm_splitk_parts(capi.frag_problem(pa, pw, y, rows, C, K), splits, ws)
    capi.add_layer_norm_mix_parts(ws, splits, capi.splitk_plane_floats(rows, C), res, s2, wt, bs, mixes, xo2, o2)
    assert torch.equal(xo1, xo2) and torch.equal(s1, s2)
    for f1, f2 in zip(o1, o2):
        assert torch.equal(f1, f2)


def test_last_ln_and_groupnorm_frag_equal_packed_row_major(gpu):
    from vkwr_amd import capi
    B, T, C, H = 7, 3, 256, 4
    x, res = dev(h(B, T, C), gpu), dev(h(B, T, C), gpu)
    wt, bs = dev(h(C), gpu), dev(h(C), gpu)
    y = torch.empty(B, C, dtype=torch.float16, device=gpu)
    yf = capi.frag_empty(B, C, gpu)
    capi.add_last_layer_norm(B, T, C, x, res, wt, bs, y)
    capi.add_last_layer_norm(B, T, C, x, res, wt, bs, yf, frag=True)
    assert np.array_equal(frag_to_dense(yf, B, C)[:B].view(np.uint16), y.cpu().numpy().view(np.uint16))
    r, k, v, g, xx = (dev(h(B, T, C), gpu) for _ in range(5))
    rk = dev(h(C), gpu)
    o = torch.empty(B, T, C, dtype=torch.float16, device=gpu)
    of = capi.frag_empty(B * T, C, gpu)
    capi.groupnorm_bonus_gate(B, T, C, H, xx, r, k, v, rk, wt, bs, g, o)
    capi.groupnorm_bonus_gate(B, T, C, H, xx, r, k, v, rk, wt, bs, g, of, frag=True)
    assert np.array_equal(frag_to_dense(of, B * T, C)[:B * T].view(np.uint16),
                          o.reshape(B * T, C).cpu().numpy().view(np.uint16))
