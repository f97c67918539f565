"""GPU tests of the sampling kernels through the reference op surface
(torch.ops.vkwr_sampling, csrc/sampling/torch_bindings.cpp:36-48) and the C ABI.

The draw is pinned value by value: the kernel's token for row b on its c-th
call must be the oracle's inverse CDF of the kept weights at the Philox uniform
of (seed, row b, call c) (oracle/sampling_ref.py).  Probabilities differ from
the oracle's by float32 rounding, so where the two tokens differ, the kernel's
token must still own the part of the oracle's CDF (in the kernel's draw order)
that holds the draw target, to within 1e-5 of the total; on random logits such
near-boundary draws must also be rare.  The random stream is the product's
Philox4x32-10, not the reference's curand stream: parity of the stream itself is
not claimed.
"""
import numpy as np
import pytest
import torch

from oracle import sampling_ref as sr

pytestmark = pytest.mark.gpu

MARGIN = 1e-5


def _ops():
    from vkwr._ops import sampling_ops
    return sampling_ops


def _logits(B, V, seed, scale=3.0, T=None):
    g = torch.Generator().manual_seed(seed)
    shape = (B, V) if T is None else (B, T, V)
    return torch.randn(shape, generator=g) * scale


def _check_draws(toks, logits, seed, call, temperature, top_k, top_p, pens=None):
    """toks [B] from the kernel vs the oracle; returns the number of near-boundary rows."""
    near = 0
    last = logits[:, -1] if logits.dim() == 3 else logits
    for b in range(last.shape[0]):
        u = sr.uniforms(seed, b, call + 1)[call]
        pen = None if pens is None else pens[b]
        want, margin, w = sr.sample_row(last[b].numpy(), u, temperature, top_k, top_p, pen)
        got = int(toks[b])
        assert w[got] > 0, (b, got)          # never a truncated token
        if got != want:
            lo, hi, total = sr.cdf_interval(w, sr.draw_order(w.shape[0]), got)
            target = u * total
            assert lo - MARGIN * total <= target <= hi + MARGIN * total, (b, got, want, lo, hi, target)
            near += 1
    return near


CASES = [
    # B, V, temperature, top_k, top_p
    (4, 4, 1.0, -1, 1.0),
    (8, 1000, 0.8, 50, 0.9),
    (16, 4096, 1.0, -1, 0.6),
    (8, 50000, 1.3, 20, 1.0),
    (32, 65536, 1.0, -1, 0.95),       # the model vocabulary: one row in VGPRs
    (8, 65536, 0.7, 40, 0.8),
    (4, 65532, 1.0, 7, 1.0),          # padding lanes at the end of the row
    (4, 100000, 1.0, 100, 0.9),       # above 65536: scratch-buffer mode
    (2, 1048576, 1.5, -1, 0.5),       # the largest vocabulary allowed
    # the first window from the lane maxima: q = ceil(top_k / 16) lanes per wave
    (4, 65536, 1.0, 1024, 1.0),       # q = 64: every lane of every wave
    (4, 65536, 0.9, 1, 0.5),          # q = 1, with a mass limit
    (4, 65536, 0.8, 17, 0.99),        # q = 2
]


@pytest.mark.parametrize("B,V,temp,top_k,top_p", CASES)
def test_draws_follow_oracle(gpu, B, V, temp, top_k, top_p):
    ops = _ops()
    seed = 1000 + V
    logits = _logits(B, V, V)
    states = ops.setup_rand(seed, B)
    near = 0
    for call in range(3):
        toks = ops.temperature_topk_topp(logits.to(gpu), states, temp, top_k, top_p).cpu()
        assert toks.dtype == torch.int32 and toks.shape == (B,)
        near += _check_draws(toks, logits, seed, call, temp, top_k, top_p)
    assert near <= max(1, 3 * B // 50)


def test_untruncated_flat_row(gpu):
    # many near-equal probabilities: the draw goes deep into the row
    ops = _ops()
    B, V = 8, 65536
    logits = _logits(B, V, 5, scale=0.01)
    states = ops.setup_rand(77, B)
    toks = ops.temperature_topk_topp(logits.to(gpu), states, 1.0, 0, 1.0).cpu()
    assert _check_draws(toks, logits, 77, 0, 1.0, 0, 1.0) <= 1


@pytest.mark.parametrize("V,top_k,top_p", [(65536, 2000, 1.0), (65536, -1, 0.5), (100000, 3000, 0.9),
                                         (65536, 40, 1.0), (65536, 5, 0.9)])
def test_large_ties(gpu, V, top_k, top_p):
    # a few large logits over a flat floor: the threshold lands on a value shared by
    # tens of thousands of entries, so the kept weight of every tied entry is the
    # compensation share and the search ends over more entries than it compacts
    # (top_k 40: the lane maxima's window is the whole floor; top_k 5: the 10 peaks tie)
    ops = _ops()
    B = 4
    logits = torch.zeros(B, V)
    for b in range(B):
        logits[b, torch.arange(10) * 997 + b] = 5.0
    states = ops.setup_rand(11, B)
    for call in range(3):
        toks = ops.temperature_topk_topp(logits.to(gpu), states, 1.0, top_k, top_p).cpu()
        # steps of the tied entries are below the margin: near-boundary draws are
        # common here, each one still checked against its CDF interval
        _check_draws(toks, logits, 11, call, 1.0, top_k, top_p)


@pytest.mark.parametrize("top_k,top_p", [(40, 1.0), (40, 0.9), (500, 1.0)])
def test_tied_top_values(gpu, top_k, top_p):
    # 300 equal largest logits spread over the row, above a random floor: the lane maxima
    # of every wave include the tied value, so the first window is that single value,
    # shared by more entries than top_k (kept weights: the compensation share)
    ops = _ops()
    B, V = 4, 65536
    logits = _logits(B, V, 21, scale=1.0)
    for b in range(B):
        logits[b, (torch.arange(300) * 211 + 7 * b) % V] = 8.0
    states = ops.setup_rand(13, B)
    for call in range(2):
        toks = ops.temperature_topk_topp(logits.to(gpu), states, 1.0, top_k, top_p).cpu()
        _check_draws(toks, logits, 13, call, 1.0, top_k, top_p)


def test_scratch_mode_uses_last_token(gpu):
    ops = _ops()
    B, T, V = 3, 2, 100000
    logits = _logits(B, V, 14, T=T)
    a = ops.temperature_topk_topp(logits.to(gpu), ops.setup_rand(6, B), 0.8, 64, 0.9).cpu()
    _check_draws(a, logits, 6, 0, 0.8, 64, 0.9)
    b = ops.temperature_topk_topp(logits[:, -1].contiguous().to(gpu), ops.setup_rand(6, B), 0.8, 64, 0.9).cpu()
    assert torch.equal(a, b)


@pytest.mark.parametrize("V", [1000, 65536, 100000])
def test_greedy(gpu, V):
    ops = _ops()
    B = 64
    logits = _logits(B, V, 3)
    want = logits.argmax(-1).to(torch.int32)
    states = ops.setup_rand(1, B)
    assert torch.equal(ops.temperature_topk_topp(logits.to(gpu), states, 0.7, 1, 1.0).cpu(), want)
    assert torch.equal(ops.temperature_topk_topp(logits.to(gpu), states, 1.0, 0, 0.0).cpu(), want)
    pens = torch.zeros(B, V, device=gpu)
    assert torch.equal(ops.repetition_topk_topp(logits.to(gpu), pens, states, 0.0, 0.0, 1.0, 1.0, 1, 1.0).cpu(),
                       want)


@pytest.mark.parametrize("V", [4096, 65536, 100000])
def test_repetition_penalties(gpu, V):
    ops = _ops()
    B, seed = 8, 31
    logits = _logits(B, V, 9, scale=1.0)
    g = torch.Generator().manual_seed(10)
    pens = torch.rand(B, V, generator=g) * 2.0
    pens[torch.rand(B, V, generator=g) < 0.5] = 0.0
    presence, repetition, decay, temp, top_k, top_p = 1.5, 0.4, 0.996, 0.9, 64, 0.85
    states = ops.setup_rand(seed, B)
    pens_gpu = pens.to(gpu)
    for call in range(3):
        before = pens_gpu.cpu()
        toks = ops.repetition_topk_topp(logits.to(gpu), pens_gpu, states, presence, repetition, decay, temp, top_k,
                                        top_p).cpu()
        _check_draws(toks, logits, seed, call, temp, top_k, top_p, before.numpy())
        after = pens_gpu.cpu().numpy()
        for b in range(B):
            want = sr.update_penalties(before[b].numpy(), int(toks[b]), presence, repetition, decay)
            # fma in float32 vs float64 product + add rounded once: at most 1 ulp apart
            np.testing.assert_array_max_ulp(after[b], want, maxulp=1)


def test_uses_last_token_of_each_row(gpu):
    ops = _ops()
    B, T, V = 6, 3, 2048
    logits = _logits(B, V, 4, T=T)
    a = ops.temperature_topk_topp(logits.to(gpu), ops.setup_rand(5, B), 1.0, 30, 0.9).cpu()
    b = ops.temperature_topk_topp(logits[:, -1].contiguous().to(gpu), ops.setup_rand(5, B), 1.0, 30, 0.9).cpu()
    assert torch.equal(a, b)
    _check_draws(a, logits, 5, 0, 1.0, 30, 0.9)
    pens = torch.zeros(B, V, device=gpu)
    c = ops.repetition_topk_topp(logits.to(gpu), pens, ops.setup_rand(5, B), 0.0, 0.0, 1.0, 1.0, 30, 0.9).cpu()
    assert torch.equal(a, c)


def test_state_layout_and_determinism(gpu):
    ops = _ops()
    B, V, seed = 5, 4096, (7 << 32) | 123
    st = ops.setup_rand(seed, B)
    assert st.dtype == torch.int8 and st.numel() == B * ops.STATE_BYTES and st.is_cuda
    words = st.cpu().view(torch.int32).view(B, 8).numpy().astype(np.uint32)
    for b in range(B):
        assert words[b].tolist() == [123, 7, 0, 0, b, 0, 0, 0]   # key, counter (0, 0, b, 0), reserved
    logits = _logits(B, V, 8).to(gpu)
    st2 = ops.setup_rand(seed, B)
    runs = [ops.temperature_topk_topp(logits, st, 1.0, -1, 1.0).cpu() for _ in range(4)]
    runs2 = [ops.temperature_topk_topp(logits, st2, 1.0, -1, 1.0).cpu() for _ in range(4)]
    assert all(torch.equal(x, y) for x, y in zip(runs, runs2))            # same seed, same tokens
    assert st.cpu().view(torch.int32).view(B, 8)[:, 2].tolist() == [4] * B  # one counter block per call


def test_nan_and_inf_logits(gpu):
    ops = _ops()
    B, V = 4, 65536
    logits = _logits(B, V, 12)
    hot = [3, 40000, 65535, 12345]
    for b, j in enumerate(hot):
        logits[b, j] = float("inf")
    logits[:, 17] = float("nan")
    states = ops.setup_rand(2, B)
    for _ in range(3):
        assert ops.temperature_topk_topp(logits.to(gpu), states, 1.0, -1, 1.0).cpu().tolist() == hot
    # NaN acts as logit 0: with every other logit very negative, the NaN entry wins
    logits = torch.full((B, V), -1e4)
    logits[:, 17] = float("nan")
    assert ops.temperature_topk_topp(logits.to(gpu), states, 1.0, -1, 1.0).cpu().tolist() == [17] * B


def test_law_of_the_draw(gpu):
    # 4096 rows of the same logits, 5 calls: frequencies follow the kept weights
    ops = _ops()
    B, V = 4096, 64
    row = _logits(1, V, 21, scale=1.5)
    logits = row.expand(B, V).contiguous()
    states = ops.setup_rand(2024, B)
    toks = torch.cat([ops.temperature_topk_topp(logits.to(gpu), states, 1.0, 10, 0.9).cpu() for _ in range(5)])
    top_k, top_p = sr.normalize_params(V, 10, 0.9)
    w = sr.kept_weights(sr.probabilities(row[0].numpy(), 1.0), top_k, top_p)
    q = w / w.sum()
    freq = np.bincount(toks.numpy(), minlength=V) / len(toks)
    keep = q > 0
    assert freq[~keep].sum() == 0
    chi2 = np.sum((freq[keep] - q[keep]) ** 2 / q[keep]) * len(toks)
    assert chi2 < 40.0


def test_validation_matches_reference_messages(gpu):
    ops = _ops()
    st = ops.setup_rand(0, 2)
    with pytest.raises(Exception, match="Vocabulary size must be multiple of 4"):
        ops.temperature_topk_topp(torch.zeros(2, 6, device=gpu), st, 1.0, -1, 1.0)
    with pytest.raises(Exception, match="Temperature outside range"):
        ops.temperature_topk_topp(torch.zeros(2, 8, device=gpu), st, 0.0, -1, 1.0)
    with pytest.raises(Exception, match="Logits tensor must be of type float32"):
        ops.temperature_topk_topp(torch.zeros(2, 8, device=gpu, dtype=torch.float16), st, 1.0, -1, 1.0)
    with pytest.raises(RuntimeError, match="states holds"):
        ops.temperature_topk_topp(torch.zeros(3, 8, device=gpu), st, 1.0, -1, 1.0)
    with pytest.raises(Exception, match="B and T must be positive"):
        ops.temperature_topk_topp(torch.zeros(0, 8, device=gpu), st, 1.0, -1, 1.0)


def test_capi_matches_op(gpu):
    from vkwr_amd import capi
    ops = _ops()
    B, V = 16, 65536
    logits = _logits(B, V, 30).to(gpu)
    a = ops.temperature_topk_topp(logits, ops.setup_rand(9, B), 0.9, 25, 0.85)
    st = torch.empty(B * capi.SAMPLING_STATE_BYTES, dtype=torch.uint8, device=gpu)
    capi.sampling_setup_rand(9, st)
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    capi.sample(logits, st, out, 0.9, 25, 0.85)
    assert torch.equal(a, out)
