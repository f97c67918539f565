"""GPU parity of the WKV-7 kernels against the CPU oracle, through the torch ops.

Bar (north_star): state gather/scatter and slot indexing bit-exact; y within
max-abs 2e-2 / mean-rel 5e-3 (fp16); final fp32 state within max-abs 1e-3.
The token-by-token kernels perform the oracle's IEEE operations in the oracle's
order, so their tests demand (and report) bit equality, which implies those
tolerances.  The chunked prefill kernel (T >= 16 through mode 0 and the slot op)
computes the same recurrence as products of 16-token blocks on the matrix cores:
its results are checked against the reference-order oracle: y within max-abs
2e-2 wherever |y| < 32 and within one fp16 ulp where |y| >= 32 (there one ulp,
2^-5 or more, exceeds 2e-2 -- a stated departure from the literal bound for
those values), mean-rel <= 2e-6, at most 0.3 % of values off at all, and the
state within 1e-3 and 2e-5 of its largest value (the two agree to fp32
rounding).  wkv_forward_seq_fp32 is the bit-exact path in the reference order.
Also restated: the reference's own WKV unit tests
(reference tests/ops/test_v1_wkv_ops.py:161-466).
"""
import os
import time

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.wkv_inputs import make_state, make_wkv_inputs

pytestmark = pytest.mark.gpu

Y_MAX_ABS, Y_MEAN_REL, STATE_MAX_ABS = 2e-2, 5e-3, 1e-3


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    orc.set_threads(min(16, len(os.sched_getaffinity(0))))


def _dev(xs, device):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(device) for x in xs]


def _check_y(y_gpu, y_ref, what):
    yg = y_gpu.detach().cpu().numpy().astype(np.float64)
    yr = y_ref.astype(np.float64)
    err = np.abs(yg - yr)
    mean_rel = err.sum() / max(np.abs(yr).sum(), 1e-30)
    assert err.max() <= Y_MAX_ABS and mean_rel <= Y_MEAN_REL, (what, err.max(), mean_rel)
    assert np.array_equal(y_gpu.detach().cpu().numpy().view(np.uint16), y_ref.view(np.uint16)), (
        what, "y not bit-identical", int((yg != yr).sum()))


def _check_state(s_gpu, s_ref, what):
    sg = s_gpu.detach().cpu().numpy()
    assert np.abs(sg.astype(np.float64) - s_ref.astype(np.float64)).max() <= STATE_MAX_ABS, what
    assert np.array_equal(sg.view(np.uint8), s_ref.view(np.uint8)), (what, "state not bit-identical")


CHUNK_MIN_T = 16           # mode 0 / slot op prefills of at least this many tokens run chunked
CHUNK_Y_MEAN_REL = 2e-6    # chunked vs reference order: fp32 rounding only (measured ~2e-7)
CHUNK_STATE_REL = 2e-5     # ... max |dS| / max |S|
CHUNK_ULP_FRAC = 3e-3      # ... at most this fraction of y values one fp16 ulp or more off
BIG_Y = 32.0               # |y| from which one fp16 ulp (2^-5) exceeds the 2e-2 max-abs bound


def _check_y_chunked(y_gpu, y_ref, what):
    """The chunked kernel's y contract against the reference-order oracle.

    Every y with |y_ref| < 32 is within north_star's literal max-abs 2e-2.  Where |y_ref| >= 32
    one fp16 ulp (2^-5 or more) is itself larger than 2e-2, and any kernel whose fp32 sums are
    not in the reference's order may round such a y to the neighbouring fp16 value: there the
    bound is one ulp.  This is a deliberate departure from the literal north_star bound for
    those values only; wkv_forward_seq_fp32 (and modes 2-3) keep the reference order and are
    bit-exact.  Mean-relative error <= 2e-6 (north_star: 5e-3), and at most 0.3 % of the
    values may differ from the oracle at all (measured: 0.14 % at config 0, 0.16 % at config 2).
    Returns (max-abs, mean-rel, number of y values that differ by >= 1 fp16 ulp)."""
    yg = y_gpu.detach().cpu().numpy().astype(np.float64)
    yr = y_ref.astype(np.float64)
    err = np.abs(yg - yr)
    big = np.abs(yr) >= BIG_Y
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(yr), 2.0 ** -14))) - 10)
    mean_rel = err.sum() / max(np.abs(yr).sum(), 1e-30)
    small_err = float(err[~big].max()) if (~big).any() else 0.0
    assert small_err <= Y_MAX_ABS, (what, "|y| < 32 beyond 2e-2", small_err)
    assert (err[big] <= ulp[big]).all(), (what, "|y| >= 32 beyond one fp16 ulp", float(err[big].max()))
    assert mean_rel <= CHUNK_Y_MEAN_REL, (what, "chunked y off the recurrence", mean_rel)
    n_off = int((yg != yr).sum())
    assert n_off <= CHUNK_ULP_FRAC * yr.size, (what, "too many y values off the oracle", n_off, yr.size)
    return float(err.max()), float(mean_rel), n_off


def _check_state_chunked(s_gpu, s_ref, what):
    sg = s_gpu.detach().cpu().numpy().astype(np.float64)
    sr = s_ref.astype(np.float64)
    d = np.abs(sg - sr).max()
    assert d <= STATE_MAX_ABS, (what, d)
    assert d <= CHUNK_STATE_REL * max(np.abs(sr).max(), 1e-30), (what, "chunked state off the recurrence", d)


# ---------------------------------------------------------------- fp32 dense

FP32_CASES = [
    # (B, T, H, dist, state_std)
    (1, 1, 1, "realistic", 0.0),
    (1, 4, 2, "realistic", 0.0),
    (2, 8, 4, "realistic", 0.1),
    (1, 16, 2, "realistic", 0.1),
    (3, 5, 3, "baseline", 0.1),
    (2, 128, 12, "baseline", 0.0),
    (1, 33, 2, "realistic", 0.1),    # row-split kernel: two full 16-token chunks + a 1-token tail
    (2, 47, 3, "baseline", 0.1),     # ... odd tail inside the last chunk
    (16, 20, 32, "realistic", 0.1),  # B*H = 512: one workgroup per (sequence, head), 2 rows per lane
    (1, 2, 1, "realistic", 0.1),     # modes 1-3: the latency-scheduled kernel's shortest sequence
    (33, 3, 32, "realistic", 0.1),   # ... B*H = 1056 > 4 x CUs: the many-waves kernel
]


def _order(mode, T):
    """Mode 0 (wkv_forward_fp32) runs the chunked kernel at T >= 16 ("chunk": checked at
    tolerance against the reference order) and the row-split kernel at 1 < T < 16; every
    other call reduces each dot product in one chain (the reference's row-per-thread order)."""
    if mode == "wkv_forward_fp32" and T >= CHUNK_MIN_T:
        return "chunk"
    return "rows" if mode == "wkv_forward_fp32" and T > 1 else "seq"


@pytest.mark.parametrize("mode", ["wkv_forward_fp32", "wkv_forward_seq_fp32", "wkv_forward_small_fp32", "wkv_forward_block_fp32"])
@pytest.mark.parametrize("B,T,H,dist,std", FP32_CASES)
def test_fp32_dense_matches_oracle(gpu, mode, B, T, H, dist, std):
    """Every mode at every case, config 0 included: mode 0 at T >= 16 runs the chunked
    kernel (tolerance against the reference order; the figures are printed), at 1 < T < 16
    the row-split kernel (bit-exact against the oracle's row-split order); modes 1-3, and
    every mode at T = 1, run the row-per-lane kernel (bit-exact against the reference's
    one-chain order)."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=B * 100 + T, dist=dist)
    S0 = make_state(B, H, seed=T, std=std)
    S_ref = S0.copy()
    order = _order(mode, T)
    y_ref = orc.wkv_fp32(B, T, C, H, S_ref, *ins, order="seq" if order == "chunk" else order)
    state = torch.from_numpy(S0).to(gpu)
    y = getattr(ops, mode)(B, T, C, H, state, *_dev(ins, gpu))
    torch.cuda.synchronize()
    if order == "chunk":
        mx, mr, nulp = _check_y_chunked(y, y_ref, mode)
        _check_state_chunked(state, S_ref, mode)
        print(f"chunked {B}x{T}x{H} {dist}: y max-abs {mx:.3g} mean-rel {mr:.3g} "
              f">=1-ulp mismatches {nulp}/{y_ref.size}", flush=True)
    else:
        _check_y(y, y_ref, mode)
        _check_state(state, S_ref, mode)


# ---------------------------------------------------------------- slot pool


def test_slots_config1_steps_match_oracle(gpu):
    """BASELINE config 1 at full size: pool 512 x H=32, 128 distinct slots, 3 decode steps."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    P, B, H = 512, 128, 32
    C = H * 64
    pool_np = make_state(P, H, seed=1)
    slots_np = np.random.default_rng(1).permutation(P)[:B].astype(np.int32)
    pool = torch.from_numpy(pool_np).to(gpu)
    slots = torch.from_numpy(slots_np).to(gpu)
    ops.validate_slots(slots, P)
    for step in range(3):
        ins = make_wkv_inputs(B, 1, H, seed=1000 + step)
        y_ref = orc.wkv_fp32_slots(B, 1, C, H, pool_np, slots_np.astype(np.int64), *ins)
        y = ops.wkv_one_slots_fp32(B, C, H, pool, slots, *_dev([x.reshape(B, C) for x in ins], gpu))
        torch.cuda.synchronize()
        _check_y(y.view(B, 1, C), y_ref, f"slots step {step}")
    _check_state(pool, pool_np, "pool after 3 steps")  # includes the 384 untouched slots


def test_slots_equal_gather_dense_scatter(gpu):
    """Fused slot op == index_select -> wkv_forward_fp32 -> index_copy_, bitwise, T=3."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    P, B, T, H = 40, 9, 3, 4
    C = H * 64
    pool = torch.from_numpy(make_state(P, H, seed=2)).to(gpu)
    pool2 = pool.clone()
    slots = torch.randperm(P, generator=torch.Generator().manual_seed(2))[:B].to(torch.int32).to(gpu)
    ins = _dev(make_wkv_inputs(B, T, H, seed=2), gpu)
    y1 = ops.wkv_forward_slots_fp32(B, T, C, H, pool, slots, *ins, validate=True)
    st = pool2.index_select(0, slots.long())
    y2 = ops.wkv_forward_fp32(B, T, C, H, st, *ins)
    pool2.index_copy_(0, slots.long(), st)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(pool, pool2)


def test_slots_out_of_range_is_skipped(gpu):
    """A slot outside [0,P) (device-side bounds check): NaN y rows, pool bitwise unchanged."""
    P, B, H = 8, 3, 2
    C = H * 64
    pool = torch.from_numpy(make_state(P, H, seed=3)).to(gpu)
    before = pool.clone()
    slots = torch.tensor([1, P + 5, 4], dtype=torch.int32, device=gpu)
    ins = _dev(make_wkv_inputs(B, 1, H, seed=3), gpu)
    y = torch.empty(B, 1, C, dtype=torch.float16, device=gpu)
    torch.ops.vkwr_v1_wkv.wkv_forward_slots_fp32(B, 1, C, H, pool, slots, *ins, y)
    torch.cuda.synchronize()
    assert torch.isnan(y[1]).all() and not torch.isnan(y[0]).any() and not torch.isnan(y[2]).any()
    untouched = [0, 2, 3, 5, 6, 7]
    assert torch.equal(pool[untouched], before[untouched])
    with pytest.raises(RuntimeError):
        from vkwr._ops.v1 import v1_wkv_ops as ops
        ops.wkv_forward_slots_fp32(B, 1, C, H, pool, slots, *ins, validate=True)


@pytest.mark.parametrize("layout", ["std", "ilv"])
@pytest.mark.parametrize("frag", [False, True], ids=["rowmajor_out", "frag_out"])
def test_decode_fused_equals_gate_wkv_groupnorm_sequence(gpu, frag, layout):
    """vkwr_wkv7_decode_fused_f16 == kk_a_gate -> wkv7_fp32_forward_slots ->
    groupnorm_bonus_gate, bit for bit (pool and output), including an
    out-of-range slot (pool untouched, NaN output row) and a ragged batch; with
    the pool in either block layout (the interleaved pool converted back)."""
    from vkwr_amd import capi
    rng = np.random.default_rng(5)
    B, H, P = 37, 4, 50
    C = 64 * H
    h16 = lambda *s, sc=1.0: torch.from_numpy((rng.standard_normal(s) * sc).astype(np.float16)).to(gpu)  # noqa
    r, w, k, v, a12, g = h16(B, C), h16(B, C, sc=2.0), h16(B, C), h16(B, C), h16(B, C), h16(B, C)
    k_k = torch.from_numpy((0.85 + 0.1 * rng.random(C)).astype(np.float16)).to(gpu)
    a0, k_a, r_k, ln_w, ln_b = h16(C, sc=0.5), h16(C, sc=0.1) + 1, h16(C, sc=0.5), h16(C, sc=0.1) + 1, h16(C, sc=0.1)
    slots_np = rng.permutation(P)[:B].astype(np.int32)
    slots_np[7] = P  # out of range
    slots = torch.from_numpy(slots_np).to(gpu)
    pool0 = torch.from_numpy((rng.standard_normal((P, H, 64, 64)) * 0.1).astype(np.float32)).to(gpu)
    # unfused
    pool_u = pool0.clone()
    new_k, neg_kk, kka, y = (torch.empty(B, C, dtype=torch.float16, device=gpu) for _ in range(4))
    capi.kk_a_gate(B, 1, C, H, k, k_k, a0, a12, k_a, new_k, neg_kk, kka)
    capi.wkv_slots(B, 1, C, H, pool_u, slots, r, w, new_k, v, neg_kk, kka, y)
    out_u = torch.empty(B, C, dtype=torch.float16, device=gpu)
    capi.groupnorm_bonus_gate(B, 1, C, H, y, r, new_k, v, r_k, ln_w, ln_b, g, out_u)
    # fused
    ilv = layout == "ilv"
    pool_f = pool0.clone()
    if ilv:
        capi.wkv_state_layout(pool0, pool_f, capi.WKV_STATE_ILV)
    out_f = capi.frag_empty(B, C, gpu) if frag else torch.empty(B, C, dtype=torch.float16, device=gpu)
    capi.wkv_decode_fused(B, C, H, pool_f, slots, r, w, k, v, a12, g, k_k, a0, k_a, r_k, ln_w, ln_b, out_f,
                          frag=frag, state_layout=capi.WKV_STATE_ILV if ilv else capi.WKV_STATE_STD)
    if ilv:
        back = torch.empty_like(pool_f)
        capi.wkv_state_layout(pool_f, back, capi.WKV_STATE_STD)
        pool_f = back
    assert torch.equal(pool_f, pool_u)
    if frag:
        out_f_rm = torch.empty(B, C, dtype=torch.float16, device=gpu)
        capi.frag_unpack(out_f, B, C, out_f_rm)
        out_f = out_f_rm
    ok = torch.ones(B, dtype=torch.bool, device=gpu)
    ok[7] = False
    assert torch.equal(out_f[ok], out_u[ok])
    assert torch.isnan(out_f[7]).all() and torch.isnan(out_u[7]).all()


def test_state_layout_round_trip_and_definition(gpu):
    """Interleaved block layout: S[i][4q+e] at float (64q + i)*4 + e; std -> ilv -> std is the identity."""
    from vkwr_amd import capi
    x = torch.randn(3, 2, 64, 64, device=gpu)
    ilv = torch.empty_like(x)
    capi.wkv_state_layout(x, ilv, capi.WKV_STATE_ILV)
    want = x.reshape(6, 64, 16, 4).permute(0, 2, 1, 3).reshape(3, 2, 64, 64)
    assert torch.equal(ilv, want)
    back = torch.empty_like(x)
    capi.wkv_state_layout(ilv, back, capi.WKV_STATE_STD)
    assert torch.equal(back, x)


def test_prefill_config2_reduced_matches_oracle(gpu):
    """BASELINE config 2 shape (T=1024, H=32) at B=2, slots gathered from a pool: the chunked
    kernel against the reference order; the 14 pool entries no slot names stay bitwise."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    P, B, T, H = 16, 2, 1024, 32
    C = H * 64
    pool_np = make_state(P, H, seed=4)
    slots_np = np.array([11, 3], dtype=np.int32)
    ins = make_wkv_inputs(B, T, H, seed=4)
    pool = torch.from_numpy(pool_np).to(gpu)
    y = ops.wkv_forward_slots_fp32(B, T, C, H, pool, torch.from_numpy(slots_np).to(gpu), *_dev(ins, gpu))
    y_ref = orc.wkv_fp32_slots(B, T, C, H, pool_np, slots_np.astype(np.int64), *ins, order="seq")
    torch.cuda.synchronize()
    mx, mr, nulp = _check_y_chunked(y, y_ref, "prefill B=2 T=1024")
    print(f"chunked slots 2x1024x32: y max-abs {mx:.3g} mean-rel {mr:.3g} >=1-ulp {nulp}/{y_ref.size}", flush=True)
    _check_state_chunked(pool[slots_np.tolist()], pool_np[slots_np], "prefill pool")
    others = [i for i in range(P) if i not in slots_np.tolist()]
    assert np.array_equal(pool[others].cpu().numpy(), pool_np[others])


def test_prefill_config2_full_matches_oracle(gpu):
    """BASELINE config 2 at full size (B=8, T=1024, H=32, inputs drawn as in config 0, state
    ~ N(0, 0.1) gathered from 8 random slots of a 512-slot pool and scattered back) through
    the slot op (the chunked kernel) against the C oracle in the reference order, at the
    chunked kernel's contract; the 504 slots no sequence names stay bitwise."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    P, B, T, H = 512, 8, 1024, 32
    C = H * 64
    pool_np = make_state(P, H, seed=7)
    slots_np = np.random.default_rng(7).permutation(P)[:B].astype(np.int32)
    ins = make_wkv_inputs(B, T, H, seed=7)
    pool = torch.from_numpy(pool_np).to(gpu)
    y = ops.wkv_forward_slots_fp32(B, T, C, H, pool, torch.from_numpy(slots_np).to(gpu), *_dev(ins, gpu))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    y_ref = orc.wkv_fp32_slots(B, T, C, H, pool_np, slots_np.astype(np.int64), *ins, order="seq")
    t_or = time.perf_counter() - t0
    mx, mr, nulp = _check_y_chunked(y, y_ref, "config 2 full")
    print(f"config 2 full (oracle {t_or:.1f} s): y max-abs {mx:.3g} mean-rel {mr:.3g} "
          f">=1-ulp {nulp}/{y_ref.size}", flush=True)
    got = pool.cpu().numpy()
    _check_state_chunked(torch.from_numpy(got[slots_np]), pool_np[slots_np], "config 2 pool")
    others = np.setdiff1d(np.arange(P), slots_np)
    assert np.array_equal(got[others], pool_np[others])


def _config2_inputs(gpu, B, T, H, seed=5):
    C = H * 64
    g = torch.Generator(device=gpu).manual_seed(seed)
    # config 0's distributions (the raw w input is exp(-0.6065 sigmoid(N(0,1))))
    ins = [torch.randn(B, T, C, device=gpu, generator=g).half() for _ in range(6)]
    ins[1] = torch.exp(-0.6065 * torch.sigmoid(ins[1].float())).half()
    ins[4] = -torch.nn.functional.normalize(ins[2].float().view(B, T, H, 64), dim=-1).reshape(B, T, C).half()
    ins[5] = (-ins[4].float() * torch.sigmoid(torch.randn(B, T, C, device=gpu, generator=g))).half()
    s0 = (torch.randn(B, H, 64, 64, device=gpu, generator=g) * 0.1).contiguous()
    return ins, s0


def test_prefill_config2_full_equals_decode_steps(gpu):
    """BASELINE config 2 at full size (B=8,T=1024,H=32): one row-per-lane prefill call (mode 1)
    == 1024 decode calls, bitwise (size-independent property; the oracle covers B=2 above)."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, H = 8, 1024, 32
    C = H * 64
    ins, s1 = _config2_inputs(gpu, B, T, H)
    s2 = s1.clone()
    y1 = ops.wkv_forward_seq_fp32(B, T, C, H, s1, *ins)
    y2 = torch.empty_like(y1)
    for t in range(T):
        y2[:, t:t + 1] = ops.wkv_forward_fp32(B, 1, C, H, s2, *(x[:, t:t + 1].contiguous() for x in ins))
    torch.cuda.synchronize()
    assert torch.equal(s1, s2)
    assert torch.equal(y1, y2)


def test_prefill_config2_full_rows_chunking_and_tolerance(gpu):
    """Config 2 at full size through mode 0 (the chunked kernel): one T=1024 call == four
    T=256 calls == 64 calls of T=16, bitwise -- chunk boundaries fall at the same tokens, and
    a chunk's arithmetic does not depend on where the call starts -- and, with 512 calls of
    T=2 (the row-split kernel) and the row-per-lane kernel (mode 1), within the stated
    tolerances (y max-abs 2e-2 / mean-rel 5e-3, state 1e-3)."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, H = 8, 1024, 32
    C = H * 64
    ins, s1 = _config2_inputs(gpu, B, T, H, seed=6)
    s2, s3, s4, s5 = s1.clone(), s1.clone(), s1.clone(), s1.clone()
    y1 = ops.wkv_forward_fp32(B, T, C, H, s1, *ins)
    y2 = torch.cat([ops.wkv_forward_fp32(B, 256, C, H, s2, *(x[:, t:t + 256].contiguous() for x in ins))
                    for t in range(0, T, 256)], dim=1)
    y5 = torch.cat([ops.wkv_forward_fp32(B, 16, C, H, s5, *(x[:, t:t + 16].contiguous() for x in ins))
                    for t in range(0, T, 16)], dim=1)
    y3 = torch.cat([ops.wkv_forward_fp32(B, 2, C, H, s3, *(x[:, t:t + 2].contiguous() for x in ins))
                    for t in range(0, T, 2)], dim=1)
    y4 = ops.wkv_forward_seq_fp32(B, T, C, H, s4, *ins)
    torch.cuda.synchronize()
    assert torch.equal(s1, s2) and torch.equal(y1, y2)
    assert torch.equal(s1, s5) and torch.equal(y1, y5)
    for yy, ss in ((y3, s3), (y4, s4)):
        err = (y1.double() - yy.double()).abs()
        ulp = torch.exp2(torch.floor(torch.log2(yy.double().abs().clamp_min(2.0 ** -14))) - 10)
        assert bool((err <= torch.maximum(ulp, torch.full_like(ulp, Y_MAX_ABS))).all()), err.max().item()
        assert err.sum().item() / yy.double().abs().sum().item() <= CHUNK_Y_MEAN_REL
        assert (s1 - ss).abs().max().item() <= CHUNK_STATE_REL * ss.abs().max().item()
    # |y| here reaches ~100, where one fp16 ulp (2^-5 above 32) exceeds the 2e-2 max-abs
    # bound: two fp32 summation orders may round y to neighbouring fp16 values, so the
    # elementwise bound is max(2e-2, one fp16 ulp of |y|); the mean-relative bound is as stated.
    err = (y1.double() - y4.double()).abs()
    ulp = torch.exp2(torch.floor(torch.log2(y4.double().abs().clamp_min(2.0 ** -14))) - 10)
    assert bool((err <= torch.maximum(ulp, torch.full_like(ulp, Y_MAX_ABS))).all()), err.max().item()
    assert err.sum().item() / y4.double().abs().sum().item() <= Y_MEAN_REL
    assert (s1 - s4).abs().max().item() <= STATE_MAX_ABS
    assert not torch.equal(s1, s4)  # the two kernels really reduce in different orders


def test_rows_kernel_split_forms_are_identical(gpu):
    """Below 2 x CUs (sequence, head) pairs the row-split kernel gives each pair two
    workgroups of 32 rows; above, one workgroup of 64.  Both keep every row's lane
    mapping and reduction order: a B=16, H=32 call (512 pairs, one workgroup each) equals
    the same work as two B=8 calls (256 pairs, two workgroups each), bitwise."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, H = 16, 13, 32  # T < 16: the row-split kernel
    C = H * 64
    ins = _dev(make_wkv_inputs(B, T, H, seed=44, dist="realistic"), gpu)
    s_all = torch.from_numpy(make_state(B, H, seed=44, std=0.1)).to(gpu)
    s_half = s_all.clone()
    y_all = ops.wkv_forward_fp32(B, T, C, H, s_all, *ins)
    ys = []
    for b0 in (0, 8):
        st = s_half[b0:b0 + 8].contiguous()
        ys.append(ops.wkv_forward_fp32(8, T, C, H, st, *(x[b0:b0 + 8].contiguous() for x in ins)))
        s_half[b0:b0 + 8] = st
    torch.cuda.synchronize()
    assert torch.equal(y_all, torch.cat(ys, dim=0))
    assert torch.equal(s_all, s_half)


@pytest.mark.parametrize("T", [11, 21])
def test_rows_kernel_unaligned_inputs_match_oracle(gpu, T):
    """r..b and y starting 2 bytes past a 16-byte boundary take the kernels' scalar load/store
    paths: the row-split kernel (T = 11, the same bits as the oracle's row-split order) and the
    chunked kernel (T = 21, at tolerance against the reference order)."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, H = 2, 2
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=31, dist="realistic")
    S0 = make_state(B, H, seed=31, std=0.1)
    S_ref = S0.copy()
    chunked = T >= CHUNK_MIN_T
    y_ref = orc.wkv_fp32(B, T, C, H, S_ref, *ins, order="seq" if chunked else "rows")

    def shifted(x):
        buf = torch.empty(x.size + 1, dtype=torch.float16, device=gpu)
        v = buf[1:].view(B, T, C)
        v.copy_(torch.from_numpy(np.ascontiguousarray(x)).to(gpu))
        return v

    d = [shifted(x) for x in ins]
    y = shifted(np.zeros((B, T, C), dtype=np.float16))
    assert all(t.data_ptr() % 16 == 2 for t in d + [y])
    state = torch.from_numpy(S0).to(gpu)
    torch.ops.vkwr_v1_wkv.wkv_forward_fp32(B, T, C, H, state, *d, y)
    torch.cuda.synchronize()
    if chunked:
        _check_y_chunked(y, y_ref, "unaligned")
        _check_state_chunked(state, S_ref, "unaligned")
    else:
        _check_y(y, y_ref, "unaligned")
        _check_state(state, S_ref, "unaligned")


# ---------------------------------------------------------------- fp16 family

# T > 1 with at most 4 x CUs (sequence, head) chains runs the latency-scheduled sequence
# kernel (two tokens per loop trip, a trailing odd token); 33 x 32 chains run the
# one-wave-per-chain kernel that T = 1 uses.  Both must give the oracle's bits.
FP16_CASES = [(1, 1, 1), (1, 4, 1), (2, 8, 2), (4, 4, 4), (1, 16, 2), (3, 7, 3),
              (1, 2, 1), (2, 3, 2), (2, 64, 4), (33, 3, 32)]


@pytest.mark.parametrize("variant", ["seq", "seq_w0", "one", "one_w0", "legacy_seq", "legacy_one"])
@pytest.mark.parametrize("B,T,H", FP16_CASES)
def test_fp16_family_matches_oracle(gpu, variant, B, T, H):
    if variant.endswith("one"):
        T = 1
    if variant in ("one", "one_w0") and T != 1:
        T = 1
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=7 * B + T, dist="realistic")
    S0 = make_state(B, H, seed=B + T, std=0.1, dtype=np.float16)
    el = np.random.default_rng(B * T).integers(0, 1 << 30, size=B).astype(np.int32)
    w0 = (np.random.default_rng(T).standard_normal(C) * 0.1).astype(np.float16) if "w0" in variant else None
    legacy = variant.startswith("legacy")
    S_ref = S0.copy()
    y_ref = orc.wkv_fp16(B, T, C, H, S_ref, *ins, el, w0=w0, legacy=legacy)

    state = torch.from_numpy(S0).to(gpu)
    d = _dev(ins, gpu)
    elt = torch.from_numpy(el).to(gpu)
    y = torch.empty(B, T, C, dtype=torch.float16, device=gpu)
    ns = torch.ops.vkwr_v1_wkv
    if variant == "seq":
        ns.wkv_seq_fp16(B, T, C, H, state, *d, y, elt)
    elif variant == "seq_w0":
        ns.wkv_seq_w0_fp16(B, T, C, H, state, d[0], d[1], torch.from_numpy(w0).to(gpu), *d[2:], y, elt)
    elif variant == "one":
        y = y.view(B, C)
        ns.wkv_one_fp16(B, C, H, state, *(x.view(B, C) for x in d), y, elt)
    elif variant == "one_w0":
        y = y.view(B, C)
        dd = [x.view(B, C) for x in d]
        ns.wkv_one_w0_fp16(B, C, H, state, dd[0], dd[1], torch.from_numpy(w0).to(gpu), *dd[2:], y, elt)
    elif variant == "legacy_seq":
        torch.ops.vkwr_rwkv7.forward_seq(B, T, C, H, state, *d, y, elt)
    else:
        y = y.view(B, C)
        torch.ops.vkwr_rwkv7.forward_one(B, C, H, state, *(x.view(B, C) for x in d), y, elt)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().reshape(B, T, C).view(np.uint16), y_ref.view(np.uint16)), variant
    assert np.array_equal(state.cpu().numpy().view(np.uint16), S_ref.view(np.uint16)), variant


def test_fp16_w0_one_token_state_shape_from_reference_tests(gpu):
    """The reference tests pass w0 as [B,T,C]; only the first C values are used."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, C = 2, 8, 128
    H = C // 64
    state = torch.zeros(B, H, 64, 64, dtype=torch.float16, device=gpu)
    r, w, k, v, a, b = _dev(make_wkv_inputs(B, T, H, seed=9, dist="realistic"), gpu)
    w0 = (torch.randn(B, T, C, device=gpu) * 0.1).half()
    y, el = ops.wkv_seq_w0_fp16(B, T, C, H, state, r, w, w0, k, v, a, b)
    state2 = torch.zeros_like(state)
    y2, _ = ops.wkv_seq_w0_fp16(B, T, C, H, state2, r, w, w0.reshape(-1)[:C].contiguous(), k, v, a, b)
    assert torch.equal(y, y2) and torch.equal(state, state2)


def test_legacy_state_as_1_c_64(gpu):
    """The legacy golden test reshapes the state to [1,C,64] (reference test_monkey_patch.py:39-43)."""
    from vkwr._ops import rwkv7_ops

    C = 128
    ins = _dev(make_wkv_inputs(1, 3, 2, seed=10, dist="realistic"), gpu)
    st_a = torch.zeros(1, C, 64, dtype=torch.float16, device=gpu)
    st_b = torch.zeros(1, 2, 64, 64, dtype=torch.float16, device=gpu)
    el = torch.zeros(1, dtype=torch.int32, device=gpu)
    ya = rwkv7_ops.rwkv7_fwd_seq(1, 3, C, st_a, *ins, el)
    yb = rwkv7_ops.rwkv7_fwd_seq(1, 3, C, st_b, *ins, el)
    assert torch.equal(ya, yb) and torch.equal(st_a.view(-1), st_b.view(-1))


# ---------------------------------------------------------------- reference unit tests, restated


def _fp16_inputs(B, T, C, device):
    return [torch.randn(B, T, C, dtype=torch.float16, device=device) for _ in range(6)]


@pytest.mark.parametrize("B,T,C", [(1, 1, 64), (1, 4, 64), (2, 8, 128), (4, 4, 256), (1, 16, 128)])
def test_ref_wkv_seq_fp16_basic(gpu, B, T, C):
    from vkwr._ops.v1 import v1_wkv_ops as ops

    H = C // 64
    state = torch.zeros(B, H, 64, 64, dtype=torch.float16, device=gpu)
    y, el = ops.wkv_seq_fp16(B, T, C, H, state, *_fp16_inputs(B, T, C, gpu))
    assert y.shape == (B, T, C) and y.dtype == torch.float16 and y.device.type == "cuda"
    assert el.shape == (B,) and el.dtype == torch.int32


def test_ref_fp16_not_nan_mutation_zero_determinism(gpu):
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, C = 2, 8, 256
    H = C // 64
    state = torch.zeros(B, H, 64, 64, dtype=torch.float16, device=gpu)
    ins = _dev(make_wkv_inputs(B, T, H, seed=1, dist="realistic"), gpu)
    y, _ = ops.wkv_seq_fp16(B, T, C, H, state, *ins)
    assert not torch.isnan(y).any() and not torch.isinf(y).any()
    assert not torch.equal(state, torch.zeros_like(state))
    z = torch.zeros(1, 4, 128, dtype=torch.float16, device=gpu)
    y0, _ = ops.wkv_seq_fp16(1, 4, 128, 2, torch.zeros(1, 2, 64, 64, dtype=torch.float16, device=gpu), z, z, z, z, z, z)
    assert not torch.isnan(y0).any()
    s1 = torch.zeros(B, H, 64, 64, dtype=torch.float16, device=gpu)
    s2 = torch.zeros_like(s1)
    y1, _ = ops.wkv_seq_fp16(B, T, C, H, s1, *[x.clone() for x in ins])
    y2, _ = ops.wkv_seq_fp16(B, T, C, H, s2, *[x.clone() for x in ins])
    torch.testing.assert_close(y1, y2, atol=0, rtol=0)
    yo1, _ = ops.wkv_one_fp16(B, C, H, s1.clone(), *[x[:, 0].contiguous() for x in ins])
    yo2, _ = ops.wkv_one_fp16(B, C, H, s1.clone(), *[x[:, 0].contiguous() for x in ins])
    torch.testing.assert_close(yo1, yo2, atol=0, rtol=0)


@pytest.mark.parametrize("fn", ["wkv_forward_fp32", "wkv_forward_seq_fp32", "wkv_forward_small_fp32", "wkv_forward_block_fp32"])
def test_ref_fp32_basic_mutation_zero(gpu, fn):
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, C = 2, 8, 256
    H = C // 64
    state = torch.zeros(B, H, 64, 64, dtype=torch.float32, device=gpu)
    y = getattr(ops, fn)(B, T, C, H, state, *_dev(make_wkv_inputs(B, T, H, seed=2, dist="realistic"), gpu))
    assert y.shape == (B, T, C) and y.dtype == torch.float16 and not torch.isnan(y).any()
    assert not torch.equal(state, torch.zeros_like(state))
    z = torch.zeros(1, 4, 128, dtype=torch.float16, device=gpu)
    y0 = getattr(ops, fn)(1, 4, 128, 2, torch.zeros(1, 2, 64, 64, device=gpu), z, z, z, z, z, z)
    assert not torch.isnan(y0).any()


def test_ref_validation_errors(gpu):
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, C, H = 1, 4, 100, 2
    state = torch.zeros(B, H, 64, 64, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):
        ops.wkv_seq_fp16(B, T, C, H, state, *_fp16_inputs(B, T, C, gpu))
    B, T, C, H = 1, 4, 128, 2
    bad_state = torch.zeros(B, C, 64, dtype=torch.float16, device=gpu)
    y = torch.empty(B, T, C, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):
        torch.ops.vkwr_v1_wkv.wkv_forward_fp32(B, T, C, H, bad_state, *_fp16_inputs(B, T, C, gpu), y)
    with pytest.raises(RuntimeError):  # fp32 inputs where fp16 is required
        ins = [x.float() for x in _fp16_inputs(B, T, C, gpu)]
        torch.ops.vkwr_v1_wkv.wkv_forward_fp32(B, T, C, H, torch.zeros(B, H, 64, 64, device=gpu), *ins, y)
    with pytest.raises(RuntimeError):  # non-contiguous input
        ins = _fp16_inputs(B, T, 2 * C, gpu)
        ins = [x[:, :, ::2] for x in ins]
        torch.ops.vkwr_v1_wkv.wkv_forward_fp32(B, T, C, H, torch.zeros(B, H, 64, 64, device=gpu), *ins, y)
    with pytest.raises(RuntimeError):
        ops.advance_i32(torch.zeros(4, dtype=torch.int64, device=gpu), 1)
    with pytest.raises(RuntimeError):
        ops.advance_i32(torch.zeros(2, 4, dtype=torch.int32, device=gpu), 1)


def test_ref_advance_i32(gpu):
    from vkwr._ops.v1 import v1_wkv_ops as ops

    x = torch.zeros(4, dtype=torch.int32, device=gpu)
    assert ops.advance_i32(x, 5) is None
    assert (x == 5).all()
    x = torch.zeros(2, dtype=torch.int32, device=gpu)
    ops.advance_i32(x, 3)
    ops.advance_i32(x, 7)
    assert (x == 10).all()
    x = torch.full((3,), 100, dtype=torch.int32, device=gpu)
    ops.advance_i32(x, -10)
    assert (x == 90).all()
    x = torch.zeros(4, dtype=torch.int32, device=gpu)
    ops.advance_i32(x, 2 ** 30)
    assert (x == 2 ** 30).all()
    x = torch.tensor([2 ** 31 - 1, -5], dtype=torch.int32, device=gpu)
    ops.advance_i32(x, 1)
    assert x.tolist() == [-(2 ** 31), -4]
    big = torch.arange(100003, dtype=torch.int32, device=gpu)
    ops.advance_i32(big, -7)
    assert torch.equal(big, torch.arange(100003, dtype=torch.int32, device=gpu) - 7)


def test_ref_wkv_seq_fp16_performance(gpu):
    """Liveness bound of the reference (tests/ops/test_v1_wkv_ops.py:454-466): < 200 ms/call."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, T, C = 2, 64, 1024
    H = C // 64
    state = torch.zeros(B, H, 64, 64, dtype=torch.float16, device=gpu)
    ins = _dev(make_wkv_inputs(B, T, H, seed=3, dist="realistic"), gpu)
    ops.wkv_seq_fp16(B, T, C, H, state.clone(), *ins)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(30):
        ops.wkv_seq_fp16(B, T, C, H, state.clone(), *[x.clone() for x in ins])
    torch.cuda.synchronize()
    assert (time.perf_counter() - t0) / 30 * 1000 < 200.0


def test_slots_large_pool_nontemporal_path_same_bits(gpu):
    """A pool larger than the 256 MiB memory-side cache takes the decode step's
    non-temporal state path: same bits as the cached path on a small pool (y and the
    updated slot states), other slots untouched."""
    from vkwr._ops.v1 import v1_wkv_ops as ops

    B, H = 5, 32
    C = H * 64
    P_big = 520  # 520 x 32 x 16 KiB = 260 MiB > 256 MiB
    big = torch.zeros(P_big, H, 64, 64, device=gpu)
    small = torch.from_numpy(make_state(B, H, seed=40)).to(gpu)
    slots_big = torch.tensor([513, 7, 260, 0, 519], dtype=torch.int32, device=gpu)
    big[slots_big.long()] = small
    before = big.clone()
    ins = _dev([x.reshape(B, C) for x in make_wkv_inputs(B, 1, H, seed=40)], gpu)
    y_big = ops.wkv_one_slots_fp32(B, C, H, big, slots_big, *ins)
    y_small = ops.wkv_one_slots_fp32(B, C, H, small, torch.arange(B, dtype=torch.int32, device=gpu), *ins)
    torch.cuda.synchronize()
    assert torch.equal(y_big, y_small)
    assert torch.equal(big[slots_big.long()], small)
    others = torch.ones(P_big, dtype=torch.bool, device=gpu)
    others[slots_big.long()] = False
    assert torch.equal(big[others], before[others])


@pytest.mark.parametrize("P,B,H", [(512, 128, 32), (520, 5, 32), (40, 9, 4)])
def test_step_rows_slots_match_rows_oracle(gpu, P, B, H):
    """vkwr_wkv7_fp32_step_rows_slots: y and the pool bit-exact against the oracle's row-split
    order (order="rows") at T = 1, two steps, untouched slots unchanged.  P = 520 at H = 32 is
    a 260 MiB pool: the non-temporal state path."""
    from vkwr_amd import capi
    C = H * 64
    pool_np = make_state(P, H, seed=P + B)
    slots_np = np.random.default_rng(P + B).permutation(P)[:B].astype(np.int32)
    pool = torch.from_numpy(pool_np).to(gpu)
    slots = torch.from_numpy(slots_np).to(gpu)
    for step in range(2):
        ins = make_wkv_inputs(B, 1, H, seed=2000 + step)
        y_ref = orc.wkv_fp32_slots(B, 1, C, H, pool_np, slots_np.astype(np.int64), *ins, order="rows")
        y = torch.empty(B, C, dtype=torch.float16, device=gpu)
        capi.wkv_step_rows_slots(B, C, H, pool, slots, *_dev([x.reshape(B, C) for x in ins], gpu), y)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint16), y_ref.reshape(B, C).view(np.uint16)), step
    assert np.array_equal(pool.cpu().numpy(), pool_np)


def test_step_rows_slots_out_of_range_is_skipped(gpu):
    """A slot outside [0, P): NaN y rows for that sequence, pool bitwise unchanged there."""
    from vkwr_amd import capi
    P, B, H = 8, 3, 2
    C = H * 64
    pool = torch.from_numpy(make_state(P, H, seed=5)).to(gpu)
    before = pool.clone()
    slots = torch.tensor([1, P + 5, 4], dtype=torch.int32, device=gpu)
    ins = _dev([x.reshape(B, C) for x in make_wkv_inputs(B, 1, H, seed=5)], gpu)
    y = torch.empty(B, C, dtype=torch.float16, device=gpu)
    capi.wkv_step_rows_slots(B, C, H, pool, slots, *ins, y)
    torch.cuda.synchronize()
    assert torch.isnan(y[1]).all() and not torch.isnan(y[0]).any() and not torch.isnan(y[2]).any()
    untouched = [0, 2, 3, 5, 6, 7]
    assert torch.equal(pool[untouched], before[untouched])
