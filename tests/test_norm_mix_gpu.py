"""GPU parity of the LayerNorm / GroupNorm / token-shift / gate / activation ops
against the CPU oracle (oracle/ops_ref.py), through the torch ops.

Bar: these ops are floating point with fp32 statistics on the GPU and float64
in the oracle, so outputs are compared in fp16 ulps of the oracle value:
within 1 ulp (2 for ops with sqrt/exp/division) plus an absolute floor, and at
least 99 % bit-equal.  The floor covers cancellation: an output such as
t*w + b ~ 1e-4 built from O(1) terms carries the fp32 evaluation error of
those terms (~1e-7 absolute), which is several fp16 ulps at that magnitude;
2e-5 is 1/50 of the reference's own 1e-3 tolerance for these ops.
Ops computed from an fp16-rounded intermediate (the decode fusion's lerps) are
checked against the oracle applied to the GPU's own intermediate.  Also
restated: the reference's unit tests (tests/ops/test_v1_norm_ops.py,
tests/ops/test_v1_mix_ops.py): shapes, return counts, NaN, mutation, errors.
"""
import numpy as np
import pytest
import torch

from oracle import ops_ref as R

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(1)


def h(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


ATOL = 2e-5


def close_ulp(got, ref, ulps=1, min_equal=0.99, what="", atol=ATOL):
    g = got.detach().cpu().numpy() if torch.is_tensor(got) else got
    g64, r64 = g.astype(np.float64), ref.astype(np.float64)
    err = np.abs(g64 - r64)
    bound = ulps * R.ulp16(r64) + atol
    assert np.isfinite(g64).all() == np.isfinite(r64).all(), what
    bad = err > bound
    assert not bad.any(), (what, int(bad.sum()), float(err.max()))
    eq = np.mean(g.view(np.uint16) == ref.view(np.uint16)) if g.size else 1.0
    assert eq >= min_equal, (what, eq)


# ------------------------------------------------------------------ LayerNorm

@pytest.mark.parametrize("rows,C", [(1, 64), (16, 2048), (128, 2048), (7, 4096), (3, 8192), (5, 77), (4, 1000)])
def test_layer_norm(gpu, rows, C):
    from vkwr._ops.v1 import v1_norm_ops as N
    x, w, b = h(rows, C, scale=2.0), h(C), h(C)
    y = N.layer_norm_f16(dev(x, gpu), dev(w, gpu), dev(b, gpu))
    close_ulp(y, R.layer_norm(x, w, b)[1], what=f"ln {rows}x{C}")


def test_layer_norm_misaligned_view_uses_scalar_path(gpu):
    from vkwr._ops.v1 import v1_norm_ops as N
    C = 256
    big = h(4 * C + 1)
    x = dev(big, gpu)[1:].view(4, C)  # 2-byte offset: not 16-byte aligned
    w, b = h(C), h(C)
    y = N.layer_norm_f16(x, dev(w, gpu), dev(b, gpu))
    close_ulp(y, R.layer_norm(big[1:].reshape(4, C), w, b)[1])


@pytest.mark.parametrize("shape", [(2, 8, 512), (128, 1, 2048), (3, 5, 130)])
def test_add_layer_norm(gpu, shape):
    from vkwr._ops.v1 import v1_norm_ops as N
    C = shape[-1]
    x, r, w, b = h(*shape, scale=3.0), h(*shape, scale=3.0), h(C), h(C)
    x_out, y = N.add_layer_norm_f16(dev(x, gpu), dev(r, gpu), dev(w, gpu), dev(b, gpu))
    xo_ref, y_ref = R.layer_norm(x, w, b, residual=r)
    close_ulp(x_out, xo_ref, ulps=0.5, min_equal=1.0, what="x_out", atol=0)
    close_ulp(y, y_ref, what="y")


@pytest.mark.parametrize("B,T,C", [(1, 1, 2048), (4, 3, 4096), (2, 5, 66)])
def test_add_last_layer_norm(gpu, B, T, C):
    from vkwr._ops.v1 import v1_norm_ops as N
    x, r, w, b = h(B, T, C), h(B, T, C), h(C), h(C)
    y = N.add_last_layer_norm_f16(dev(x, gpu), dev(r, gpu), dev(w, gpu), dev(b, gpu))
    assert y.shape == (B, C)
    close_ulp(y, R.add_last_layer_norm(x, r, w, b))


def test_emb_ln0(gpu):
    from vkwr._ops.v1 import v1_norm_ops as N
    V, C = 64, 2048
    e = torch.randn(V, C).to(torch.bfloat16)
    w = torch.randn(C).to(torch.bfloat16)
    b = torch.randn(C).to(torch.bfloat16)
    y = N.emb_ln0_bf16_to_f16(e.to(gpu), w.to(gpu), b.to(gpu))
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    close_ulp(y, R.emb_ln0(bits(e), bits(w), bits(b)))


def test_add_f16(gpu):
    from vkwr._ops.v1 import v1_norm_ops as N
    for shape in [(4, 1024), (3, 7, 2)]:
        x, y = h(*shape), h(*shape)
        close_ulp(N.add_f16(dev(x, gpu), dev(y, gpu)), R.add16(x, y), ulps=0.5, min_equal=1.0, atol=0)
    x = dev(h(2, 64), gpu)
    torch.testing.assert_close(N.add_f16(x, torch.zeros_like(x)), x, atol=0, rtol=0)


@pytest.mark.parametrize("n_mix,B,C", [(6, 128, 2048), (1, 128, 2048), (6, 4, 4096), (1, 3, 4096), (6, 2, 130)])
def test_add_layer_norm_mix(gpu, n_mix, B, C):
    from vkwr._ops.v1 import v1_norm_ops as N
    x, r, w, b = h(B, 1, C, scale=2.0), h(B, 1, C, scale=2.0), h(C), h(C)
    shift0 = h(B, C)
    mixes = [(rng.random(C)).astype(np.float16) for _ in range(n_mix)]
    shift = dev(shift0, gpu)
    args = [dev(x, gpu), dev(r, gpu), shift, dev(w, gpu), dev(b, gpu)] + [dev(m, gpu) for m in mixes]
    if n_mix == 6:
        outs = N.add_layer_norm_tmix_mix6_f16(*args)
        assert len(outs) == 7
    else:
        outs = N.add_layer_norm_cmix_mix_f16(*args)
        assert len(outs) == 2
    xo_ref, y_ref = R.layer_norm(x, w, b, residual=r)
    close_ulp(outs[0], xo_ref, ulps=0.5, min_equal=1.0, what="x_out", atol=0)
    y_gpu = shift.cpu().numpy()
    close_ulp(y_gpu, y_ref.reshape(B, C), what="shift := y")
    for m, o in zip(mixes, outs[1:]):
        close_ulp(o, R.lerp16(y_gpu.reshape(B, 1, C), shift0.reshape(B, 1, C), m), what="lerp")


def test_add_layer_norm_mix_variants_agree(gpu):
    """_cfg and _scalar_stats (C=4096 only) compute the same function."""
    from vkwr._ops.v1 import v1_norm_ops as N
    B, C = 3, 4096
    x, r, w, b = (dev(a, gpu) for a in (h(B, 1, C), h(B, 1, C), h(C), h(C)))
    mixes = [dev(rng.random(C).astype(np.float16), gpu) for _ in range(6)]
    s0 = dev(h(B, C), gpu)
    base = [t.clone() for t in (s0,)]
    o1 = N.add_layer_norm_tmix_mix6_f16(x, r, base[0], w, b, *mixes)
    for fn, extra in ((N.add_layer_norm_tmix_mix6_f16_cfg, (1e-5, 512)),
                      (N.add_layer_norm_tmix_mix6_f16_scalar_stats, ())):
        s = s0.clone()
        o2 = fn(x, r, s, w, b, *mixes, *extra)
        assert all(torch.equal(a, c) for a, c in zip(o1, o2)) and torch.equal(s, base[0])
    s = s0.clone()
    c1 = N.add_layer_norm_cmix_mix_f16(x, r, s, w, b, mixes[2])
    for fn, extra in ((N.add_layer_norm_cmix_mix_f16_cfg, (1e-5, 1024)),
                      (N.add_layer_norm_cmix_mix_f16_scalar_stats, ())):
        s2 = s0.clone()
        c2 = fn(x, r, s2, w, b, mixes[2], *extra)
        assert all(torch.equal(a, c) for a, c in zip(c1, c2)) and torch.equal(s2, s)


def test_norm_validation_errors(gpu):
    from vkwr._ops.v1 import v1_norm_ops as N
    C = 10000
    x = torch.randn(1, 1, C, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):
        N.layer_norm_f16(x, torch.ones(C, dtype=torch.float16, device=gpu), torch.zeros(C, dtype=torch.float16, device=gpu))
    C = 2048
    x = torch.randn(1, 1, C, dtype=torch.float16, device=gpu)
    w, b = torch.ones(C, dtype=torch.float16, device=gpu), torch.zeros(C, dtype=torch.float16, device=gpu)
    for fn in (N.layer_norm_f16_small, N.layer_norm_f16_small512):
        with pytest.raises(RuntimeError):
            fn(x, w, b)
    with pytest.raises(RuntimeError):  # bf16 required
        N.emb_ln0_bf16_to_f16(x[0], w, b)
    s = torch.zeros(1, C, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):
        N.add_layer_norm_cmix_mix_f16_cfg(x, x, s, w, b, w, 1e-5, 384)
    with pytest.raises(RuntimeError):  # T must be 1
        x2 = torch.randn(1, 2, C, dtype=torch.float16, device=gpu)
        N.add_layer_norm_cmix_mix_f16(x2, x2, s, w, b, w)
    with pytest.raises(RuntimeError):  # cfg requires C = 4096
        N.add_layer_norm_tmix_mix6_f16_cfg(x, x, s, w, b, w, w, w, w, w, w, 1e-5, 256)


def test_norm_reference_unit_tests(gpu):
    """reference tests/ops/test_v1_norm_ops.py: shapes, dtype, 1-D input, NaN."""
    from vkwr._ops.v1 import v1_norm_ops as N
    for B, T, C in [(1, 1, 64), (2, 8, 256), (1, 16, 1024), (4, 4, 4096)]:
        x = torch.randn(B, T, C, dtype=torch.float16, device=gpu)
        w, b = torch.randn(C, dtype=torch.float16, device=gpu), torch.randn(C, dtype=torch.float16, device=gpu)
        y = N.layer_norm_f16(x, w, b)
        assert y.shape == x.shape and y.dtype == torch.float16 and not torch.isnan(y).any()
    x = torch.randn(256, dtype=torch.float16, device=gpu)
    assert N.layer_norm_f16(x, torch.ones_like(x), torch.zeros_like(x)).shape == (256,)
    x = torch.randn(2, 4096, dtype=torch.float16, device=gpu)
    for fn in (N.layer_norm_f16_small, N.layer_norm_f16_small512):
        assert fn(x, torch.ones(4096, dtype=torch.float16, device=gpu), torch.zeros(4096, dtype=torch.float16, device=gpu)).shape == x.shape
    e = torch.randn(16, 128, dtype=torch.bfloat16, device=gpu)
    y = N.emb_ln0_bf16_to_f16(e, torch.ones(128, dtype=torch.bfloat16, device=gpu), torch.zeros(128, dtype=torch.bfloat16, device=gpu))
    assert y.dtype == torch.float16 and y.shape == e.shape


# ------------------------------------------------------------------ token shift

@pytest.mark.parametrize("n_mix,B,T,C", [(6, 128, 1, 2048), (6, 2, 40, 256), (1, 3, 17, 4096), (1, 2, 3, 70), (6, 1, 1, 4096)])
def test_token_shift(gpu, n_mix, B, T, C):
    from vkwr._ops.v1 import v1_mix_ops as M
    x, shift0 = h(B, T, C), h(B, C)
    mixes = [rng.random(C).astype(np.float16) for _ in range(n_mix)]
    shift = dev(shift0, gpu)
    if n_mix == 6:
        outs = M.tmix_mix6(B, T, C, dev(x, gpu), shift, *[dev(m, gpu) for m in mixes])
    else:
        outs = [M.cmix_mix(B, T, C, dev(x, gpu), shift, dev(mixes[0], gpu))]
    s_ref = shift0.copy()
    refs = R.token_shift(x, s_ref, mixes)
    for o, ref in zip(outs, refs):
        close_ulp(o, ref, min_equal=0.999, what="token shift")
    assert np.array_equal(shift.cpu().numpy(), s_ref), "shift_state := x[:, T-1]"


def test_token_shift_prev_is_entry_value_for_long_prefill(gpu):
    """T > 1: every sequence's t = 0 output uses shift_state as it was at entry."""
    from vkwr._ops.v1 import v1_mix_ops as M
    B, T, C = 64, 300, 512

    def unit_range(*shape):  # |values| in [0.5, 2): prev - cur is exact in fp32
        mag = rng.uniform(0.5, 2.0, shape)
        return (np.where(rng.random(shape) < 0.5, -mag, mag)).astype(np.float16)

    x, shift0 = unit_range(B, T, C), unit_range(B, C)
    mix = np.ones(C, np.float16)  # out = cur + (prev - cur) = prev exactly
    shift = dev(shift0, gpu)
    out = M.cmix_mix(B, T, C, dev(x, gpu), shift, dev(mix, gpu)).cpu().numpy()
    assert np.array_equal(out[:, 0], shift0)
    assert np.array_equal(out[:, 1:], x[:, :-1])
    assert np.array_equal(shift.cpu().numpy(), x[:, -1])


@pytest.mark.parametrize("half_math", [False, True])
def test_tmix_mix6_t1_c4096(gpu, half_math):
    from vkwr._ops.v1 import v1_mix_ops as M
    B, C = 5, 4096
    x, shift0 = h(B, 1, C), h(B, C)
    mixes = [rng.random(C).astype(np.float16) for _ in range(6)]
    shift = dev(shift0, gpu)
    outs = M.tmix_mix6_t1_c4096(B, dev(x, gpu), shift, *[dev(m, gpu) for m in mixes], 256, 4, half_math)
    s_ref = shift0.copy()
    refs = R.token_shift(x, s_ref, mixes, half_math=half_math)
    for o, ref in zip(outs, refs):
        close_ulp(o, ref, min_equal=0.999)
    assert np.array_equal(shift.cpu().numpy(), s_ref)


def test_mix_validation_errors(gpu):
    from vkwr._ops.v1 import v1_mix_ops as M
    B, T, C = 1, 2, 63
    x = torch.randn(B, T, C, dtype=torch.float16, device=gpu)
    s = torch.zeros(B, C, dtype=torch.float16, device=gpu)
    v = torch.ones(C, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):  # odd C
        M.tmix_mix6(B, T, C, x, s, v, v, v, v, v, v)
    C = 64
    x = torch.randn(B, T, C, dtype=torch.float16, device=gpu)
    s = torch.zeros(B, C, dtype=torch.float16, device=gpu)
    v = torch.ones(C, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):
        M.tmix_mix6_cfg(B, T, C, x, s, v, v, v, v, v, v, 100)
    with pytest.raises(RuntimeError):
        M.cmix_mix_cfg(B, T, C, x, s, v, 64)
    with pytest.raises(ValueError):
        M.tmix_mix6_t1_c4096(B, x, s, v, v, v, v, v, v)
    x1 = torch.randn(1, 1, 4096, dtype=torch.float16, device=gpu)
    s1 = torch.zeros(1, 4096, dtype=torch.float16, device=gpu)
    v1 = torch.ones(4096, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):
        M.tmix_mix6_t1_c4096(1, x1, s1, v1, v1, v1, v1, v1, v1, 256, 3)
    with pytest.raises(RuntimeError):  # update_shift needs T = 1
        k = torch.randn(1, 2, 64, dtype=torch.float16, device=gpu)
        M.tmix_kk_a_gate_update_shift(1, 2, 64, 1, k, v, v, k, v, k, s)
    with pytest.raises(RuntimeError):  # head size 64 only
        k = torch.randn(1, 1, 96, dtype=torch.float16, device=gpu)
        v96 = torch.ones(96, dtype=torch.float16, device=gpu)
        M.tmix_kk_a_gate(1, 1, 96, 1, k, v96, v96, k, v96)
    with pytest.raises(RuntimeError):  # add_vec: last dim must equal C
        M.add_vec(32, x, torch.ones(32, dtype=torch.float16, device=gpu))


# ------------------------------------------------------------------ per-head ops

@pytest.mark.parametrize("B,T,H", [(128, 1, 32), (2, 4, 4), (1, 1, 1)])
def test_kk_a_gate(gpu, B, T, H):
    from vkwr._ops.v1 import v1_mix_ops as M
    C = 64 * H
    k, a12 = h(B, T, C), h(B, T, C)
    k_k, a0, k_a = h(C), h(C), h(C)
    outs = M.tmix_kk_a_gate(B, T, C, H, *(dev(a, gpu) for a in (k, k_k, a0, a12, k_a)))
    for o, ref, name in zip(outs, R.kk_a_gate(k, k_k, a0, a12, k_a, H), ("new_k", "neg_kk", "kka")):
        close_ulp(o, ref, ulps=2, min_equal=0.95, what=name)


def test_kk_a_gate_update_shift(gpu):
    from vkwr._ops.v1 import v1_mix_ops as M
    B, H = 4, 2
    C = 64 * H
    k, a12, x = h(B, 1, C), h(B, 1, C), h(B, 1, C)
    vecs = [h(C) for _ in range(3)]
    shift = torch.zeros(B, C, dtype=torch.float16, device=gpu)
    outs = M.tmix_kk_a_gate_update_shift(B, 1, C, H, dev(k, gpu), dev(vecs[0], gpu), dev(vecs[1], gpu),
                                         dev(a12, gpu), dev(vecs[2], gpu), dev(x, gpu), shift)
    assert len(outs) == 3
    assert np.array_equal(shift.cpu().numpy(), x.reshape(B, C))


@pytest.mark.parametrize("B,T,H", [(128, 1, 32), (2, 4, 4), (1, 1, 1)])
def test_groupnorm_bonus_gate(gpu, B, T, H):
    from vkwr._ops.v1 import v1_mix_ops as M
    C = 64 * H
    x, r, k, v, g = (h(B, T, C) for _ in range(5))
    r_k, w, b = h(C), h(C), h(C)
    out = M.tmix_lnx_rkvres_xg(B, T, C, H, *(dev(a, gpu) for a in (x, r, k, v, r_k, w, b, g)))
    ref = R.groupnorm_bonus_gate(x, r, k, v, r_k, w, b, g, H)
    got = out.cpu().numpy().astype(np.float64)
    # absolute slack for cancellation in the bonus sum: 64 products of O(1) terms in fp32
    assert (np.abs(got - ref.astype(np.float64)) <= 2 * R.ulp16(ref) + 1e-4 * np.abs(g).astype(np.float64) * 64).all()


def test_vres_gate_and_elementwise(gpu):
    from vkwr._ops.v1 import v1_mix_ops as M
    B, T, C = 3, 5, 256
    v, vf, v12, v0 = h(B, T, C), h(B, T, C), h(B, T, C), h(C)
    close_ulp(M.tmix_vres_gate(B, T, C, *(dev(a, gpu) for a in (v, vf, v0, v12))), R.vres_gate(v, vf, v0, v12),
              ulps=2, min_equal=0.95)
    for shape in [(1024,), (3, 7, 6), (2, 4096)]:
        x = h(*shape, scale=3.0)
        close_ulp(M.relu_square(dev(x, gpu)), R.relu_square(x), min_equal=0.999)
        close_ulp(M.act_tanh(dev(x, gpu)), R.act_tanh(x), ulps=2, min_equal=0.95)
        close_ulp(M.act_sigmoid(dev(x, gpu)), R.act_sigmoid(x), ulps=2, min_equal=0.95)
    x, vec = h(4, 3, 512), h(512)
    close_ulp(M.add_vec(512, dev(x, gpu), dev(vec, gpu)), R.add_vec(x, vec), ulps=0.5, min_equal=1.0, atol=0)
    xd = dev(x, gpu)
    assert torch.equal(M.add_vec(512, xd, torch.zeros(512, dtype=torch.float16, device=gpu)), xd)
    neg = -torch.rand(64, dtype=torch.float16, device=gpu)
    assert torch.equal(M.relu_square(neg), torch.zeros_like(neg))


def test_mix_reference_unit_tests(gpu):
    """reference tests/ops/test_v1_mix_ops.py: shapes, return counts, NaN, mutation."""
    from vkwr._ops.v1 import v1_mix_ops as M
    for B, T, C in [(1, 1, 64), (2, 8, 256), (1, 16, 4096)]:
        x = torch.randn(B, T, C, dtype=torch.float16, device=gpu)
        s = torch.randn(B, C, dtype=torch.float16, device=gpu)
        vs = [torch.rand(C, dtype=torch.float16, device=gpu) for _ in range(6)]
        before = s.clone()
        outs = M.tmix_mix6(B, T, C, x, s, *vs)
        assert len(outs) == 6 and all(o.shape == x.shape and not torch.isnan(o).any() for o in outs)
        assert not torch.equal(s, before)
        for threads in (128, 256, 512, 1024):
            assert len(M.tmix_mix6_cfg(B, T, C, x, s.clone(), *vs, threads)) == 6
    x = torch.randn(2, 1, 4096, dtype=torch.float16, device=gpu)
    s = torch.randn(2, 4096, dtype=torch.float16, device=gpu)
    vs = [torch.rand(4096, dtype=torch.float16, device=gpu) for _ in range(6)]
    for threads in (128, 256):
        for vec in (1, 2, 4, 8):
            for hm in (False, True):
                assert len(M.tmix_mix6_t1_c4096(2, x, s.clone(), *vs, threads, vec, hm)) == 6
    for B, T, C, H in [(1, 1, 64, 1), (2, 4, 256, 4), (1, 16, 512, 8)]:
        k = torch.randn(B, T, C, dtype=torch.float16, device=gpu)
        vv = [torch.randn(C, dtype=torch.float16, device=gpu) for _ in range(3)]
        outs = M.tmix_kk_a_gate(B, T, C, H, k, vv[0], vv[1], torch.randn_like(k), vv[2])
        assert len(outs) == 3 and all(o.shape == k.shape and not torch.isnan(o).any() for o in outs)
        y = M.tmix_lnx_rkvres_xg(B, T, C, H, k, k, k, k, vv[0], torch.ones_like(vv[0]), torch.zeros_like(vv[0]), k)
        assert y.shape == k.shape and not torch.isnan(y).any()


# ------------------------------------------------------------------ slot-indexed shift rows


@pytest.mark.parametrize("n_mix", [1, 6])
def test_token_shift_slots_bounds(gpu, n_mix):
    """vkwr_token_shift_mix_slots_f16: in-range sequences equal the dense form on gathered
    shift rows (bitwise, pool rows written back); a slot outside [0, n_slots) -- here n_slots
    and -1, rejected by the kernel's own check before any pool access -- gives NaN outputs and
    leaves the pool bitwise unchanged."""
    from vkwr_amd import capi
    B, T, C, P = 5, 3, 256, 9
    x = dev(h(B, T, C), gpu)
    pool = dev(h(P, C), gpu)
    mixes = [dev(rng.random(C).astype(np.float16), gpu) for _ in range(n_mix)]
    slots_l = [4, P, 0, -1, 7]
    slots = torch.tensor(slots_l, dtype=torch.int32, device=gpu)
    outs = [torch.empty(B, T, C, dtype=torch.float16, device=gpu) for _ in range(n_mix)]
    before = pool.clone()
    capi.token_shift(B, T, C, x, pool, mixes, outs, shift_slots=slots)
    ok = [0, 2, 4]
    sel = torch.tensor([slots_l[b] for b in ok], device=gpu).long()
    shift = before.index_select(0, sel).contiguous()
    xs = x[ok].contiguous()
    refs = [torch.empty(len(ok), T, C, dtype=torch.float16, device=gpu) for _ in range(n_mix)]
    capi.token_shift(len(ok), T, C, xs, shift, mixes, refs)
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        assert torch.equal(o[ok], r)
        assert torch.isnan(o[1]).all() and torch.isnan(o[3]).all()
    want = before.clone()
    want.index_copy_(0, sel, shift)
    assert torch.equal(pool, want)


@pytest.mark.parametrize("frag", [False, True])
def test_ln_mix_slots_and_rows_bounds(gpu, frag):
    """vkwr_add_layer_norm_mix{,_frag}_f16 with x_rows (embedding gather) and shift_slots:
    in-range rows equal the dense form on gathered rows; a row whose x_rows entry is past the
    table or whose slot is past the pool gets NaN outputs and no shift row is touched."""
    from vkwr_amd import capi
    rows, C, V, P = 6, 256, 40, 10
    emb = dev(h(V, C), gpu)
    res = dev(h(rows, C), gpu)
    pool = dev(h(P, C), gpu)
    wt, bs = dev(1 + h(C, scale=0.1), gpu), dev(h(C, scale=0.1), gpu)
    mixes = [dev(rng.random(C).astype(np.float16), gpu) for _ in range(6)]
    toks_l, slots_l = [3, 39, V, 0, 12, 7], [1, 9, 2, P, -1, 5]
    toks = torch.tensor(toks_l, dtype=torch.int32, device=gpu)
    slots = torch.tensor(slots_l, dtype=torch.int32, device=gpu)
    x_out = torch.empty(rows, C, dtype=torch.float16, device=gpu)
    mk = (lambda: capi.frag_empty(rows, C, gpu)) if frag else (lambda: torch.empty(rows, C, dtype=torch.float16,
                                                                                 device=gpu))
    outs = [mk() for _ in range(6)]
    before = pool.clone()
    capi.add_layer_norm_mix(emb, res, pool, wt, bs, mixes, x_out, outs, x_rows=toks, shift_slots=slots, frag=frag)
    ok, bad = [0, 1, 5], [2, 3, 4]
    xs = emb.index_select(0, torch.tensor([toks_l[r] for r in ok], device=gpu).long()).contiguous()
    sel = torch.tensor([slots_l[r] for r in ok], device=gpu).long()
    shift = before.index_select(0, sel).contiguous()
    xo_ref = torch.empty(len(ok), C, dtype=torch.float16, device=gpu)
    refs = [torch.empty(len(ok), C, dtype=torch.float16, device=gpu) for _ in range(6)]
    capi.add_layer_norm_mix(xs, res[ok].contiguous(), shift, wt, bs, mixes, xo_ref, refs)
    got = outs
    if frag:
        got = []
        for o in outs:
            u = torch.empty(rows, C, dtype=torch.float16, device=gpu)
            capi.frag_unpack(o, rows, C, u)
            got.append(u)
    torch.cuda.synchronize()
    assert torch.equal(x_out[ok], xo_ref)
    assert torch.isnan(x_out[bad]).all()
    for o, r in zip(got, refs):
        assert torch.equal(o[ok], r)
        assert torch.isnan(o[bad]).all()
    want = before.clone()
    want.index_copy_(0, sel, shift)
    assert torch.equal(pool, want)


def _ln_shift_rows_case(gpu, C, n_mix, with_res, shapes, P=16, bad_group=None):
    """Fused LayerNorm + token shift over row groups against vkwr_layer_norm_f16 followed by
    vkwr_token_shift_mix_slots_f16 per group: bit-equal outputs, x_out and shift pool."""
    from vkwr_amd import capi
    f16 = dict(dtype=torch.float16, device=gpu)
    rows = sum(B * T for B, T in shapes)
    x, res = dev(h(rows, C), gpu), dev(h(rows, C), gpu) if with_res else None
    wt, bs = dev(h(C, scale=0.5) + 1, gpu), dev(h(C, scale=0.1), gpu)
    mixes = [dev(rng.random(C).astype(np.float16), gpu) for _ in range(n_mix)]
    pool0 = dev(h(P, C), gpu)
    perm = rng.permutation(P)
    groups, r0, k = [], 0, 0
    for gi, (B, T) in enumerate(shapes):
        sl = [int(s) for s in perm[k:k + B]]
        if gi == bad_group:
            sl[0] = P  # one slot past the pool: that sequence's rows are NaN
        groups.append((r0, B, T, torch.tensor(sl, dtype=torch.int32, device=gpu)))
        r0, k = r0 + B * T, k + B
    pool = pool0.clone()
    x_out, outs = torch.empty(rows, C, **f16), [torch.empty(rows, C, **f16) for _ in range(n_mix)]
    capi.layer_norm_shift_rows(x, wt, bs, x_out, mixes, outs, pool, groups, residual=res)

    y, xo_ref = torch.empty(rows, C, **f16), torch.empty(rows, C, **f16)
    capi.layer_norm(x, wt, bs, y, residual=res, x_out=xo_ref)
    pool_ref = pool0.clone()
    refs = [torch.full((rows, C), float("nan"), **f16) for _ in range(n_mix)]
    for gi, (g0, B, T, sl) in enumerate(groups):
        if gi == bad_group:
            sl = sl[1:]
            g0, B = g0 + T, B - 1
            if B == 0:
                continue
        n = B * T
        capi.token_shift(B, T, C, y[g0:g0 + n], pool_ref, mixes, [o[g0:g0 + n] for o in refs], shift_slots=sl)
    torch.cuda.synchronize()
    bad_rows = torch.zeros(rows, dtype=torch.bool, device=gpu)
    if bad_group is not None:
        g0, _, T, _ = groups[bad_group]
        bad_rows[g0:g0 + T] = True
    ok = ~bad_rows
    assert torch.equal(x_out[ok], xo_ref[ok])
    assert torch.isnan(x_out[bad_rows]).all()
    for o, r in zip(outs, refs):
        assert torch.equal(o[ok], r[ok])
        assert torch.isnan(o[bad_rows]).all()
    assert torch.equal(pool, pool_ref), "shift pool := LN of each sequence's last row"


@pytest.mark.parametrize("C", [2048, 4096, 64])
@pytest.mark.parametrize("n_mix", [6, 1])
@pytest.mark.parametrize("with_res", [True, False])
def test_layer_norm_shift_rows_matches_ln_then_shift(gpu, C, n_mix, with_res):
    """Decode rows (T = 1) and prefill sequences (T > 1, including T = 2) in one launch."""
    _ln_shift_rows_case(gpu, C, n_mix, with_res, [(5, 1), (2, 7), (1, 2), (1, 1), (3, 4)])


def test_layer_norm_shift_rows_more_groups_than_one_launch_takes(gpu):
    """11 groups: the wrapper splits them over two launches (8 + 3 groups), same bits."""
    _ln_shift_rows_case(gpu, 256, 6, True, [(2, 1), (1, 3), (1, 2), (2, 2), (1, 5), (3, 1), (1, 4), (1, 6),
                                            (2, 3), (1, 1), (1, 7)], P=32)


def test_layer_norm_shift_rows_bad_slot(gpu):
    """A slot outside the pool: that sequence's rows are NaN, its shift row untouched, the rest exact."""
    _ln_shift_rows_case(gpu, 2048, 6, True, [(4, 1), (2, 5), (1, 3)], bad_group=1)
    _ln_shift_rows_case(gpu, 2048, 1, True, [(4, 1), (1, 3)], bad_group=0)


def test_layer_norm_shift_rows_errors(gpu):
    from vkwr_amd import capi
    C = 256
    x = torch.zeros(6, C, dtype=torch.float16, device=gpu)
    wt, bs = torch.ones(C, dtype=torch.float16, device=gpu), torch.zeros(C, dtype=torch.float16, device=gpu)
    pool = torch.zeros(8, C, dtype=torch.float16, device=gpu)
    sl = torch.arange(3, dtype=torch.int32, device=gpu)
    xo, out = torch.empty_like(x), [torch.empty_like(x)]
    with pytest.raises(RuntimeError, match="cover"):  # groups cover 3 of 6 rows
        capi.layer_norm_shift_rows(x, wt, bs, xo, [wt], out, pool, [(0, 3, 1, sl)])
    with pytest.raises(RuntimeError, match="starts at row"):
        capi.layer_norm_shift_rows(x, wt, bs, xo, [wt], out, pool, [(0, 3, 1, sl), (4, 3, 1, sl)])
    with pytest.raises(RuntimeError, match="starts at row"):  # split over two launches, still checked
        capi.layer_norm_shift_rows(x, wt, bs, xo, [wt], out, pool, [(r, 1, 1, sl) for r in range(6)] * 2)
    with pytest.raises(RuntimeError, match="must not overlap"):  # in place on the residual
        capi.layer_norm_shift_rows(x, wt, bs, xo, [wt], out, pool, [(0, 3, 2, sl)], residual=xo)
    with pytest.raises(RuntimeError, match="must not overlap"):  # an output over x
        capi.layer_norm_shift_rows(x, wt, bs, xo, [wt], [x], pool, [(0, 3, 2, sl)])
    with pytest.raises(RuntimeError, match="n_mix"):
        capi.layer_norm_shift_rows(x, wt, bs, xo, [wt, wt], out * 2, pool, [(0, 3, 2, sl)])
