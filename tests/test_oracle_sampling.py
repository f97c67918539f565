"""Pins the sampling oracle (oracle/sampling_ref.py) and the product's host-side
Philox block without a GPU.

  * Philox4x32-10 against the Random123 known-answer vectors (kat_vectors,
    philox4x32 10 rounds), both the oracle's numpy version and the product's
    vkwr_sampling_philox4x32_10 (the function the kernels compile).
  * The truncation rule against closed forms: top_k = 1 is argmax, top-k alone
    keeps the k largest entries, top-p alone keeps the shortest descending
    prefix reaching top_p and scales its last entry so the kept mass is exactly
    top_p, ties share the remaining budget equally.
  * Probabilities against softmax(l / T) (the base-2 form is the same function),
    the NaN / inf rules, the inverse CDF and the penalty update on hand examples.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import sampling_ref as sr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBPATH = os.path.join(ROOT, "vkwr_amd", "libvkwr_amd.so")

# Random123 kat_vectors, "philox4x32 10": counter (4 words), key (2 words), output (4 words)
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,out", PHILOX_KAT)
def test_oracle_philox_known_answers(ctr, key, out):
    assert tuple(int(x) for x in sr.philox4x32_10(np.array(ctr), np.array(key))) == out


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (bind to torch's HIP runtime first)

    assert os.path.exists(LIBPATH), "libvkwr_amd.so not built (run __graft_entry__.build())"
    return ctypes.CDLL(LIBPATH)


def _product_philox(L, ctr, key):
    U = ctypes.c_uint32
    o = (U * 4)()
    L.vkwr_sampling_philox4x32_10((U * 4)(*ctr), (U * 2)(*key), o)
    return tuple(o)


@pytest.mark.parametrize("ctr,key,out", PHILOX_KAT)
def test_product_philox_known_answers(lib, ctr, key, out):
    assert _product_philox(lib, ctr, key) == out


def test_product_philox_matches_oracle_on_random_blocks(lib):
    rng = np.random.default_rng(7)
    ctr = rng.integers(0, 1 << 32, size=(200, 4), dtype=np.uint64)
    key = rng.integers(0, 1 << 32, size=(200, 2), dtype=np.uint64)
    want = sr.philox4x32_10(ctr, key)
    for i in range(200):
        assert _product_philox(lib, [int(x) for x in ctr[i]], [int(x) for x in key[i]]) == tuple(
            int(x) for x in want[i])


def test_uniforms_range_and_streams():
    u = sr.uniforms(1234, 0, 100000)
    assert u.min() > 0.0 and u.max() <= 1.0
    assert abs(u.mean() - 0.5) < 0.005
    assert abs(u.var() - 1.0 / 12) < 0.002
    assert not np.array_equal(u[:64], sr.uniforms(1234, 1, 64))      # rows: own subsequence
    assert not np.array_equal(u[:64], sr.uniforms(1235, 0, 64))      # seeds: own key
    # the counter runs over both low words: call 2^32 uses counter (0, 1, row, 0)
    blk = sr.philox4x32_10(np.array([0, 1, 0, 0]), np.array([1234, 0]))
    assert blk[0] != sr.philox4x32_10(np.array([0, 0, 0, 0]), np.array([1234, 0]))[0]


def test_normalize_params():
    assert sr.normalize_params(100, 0, 0.5) == (100, 0.5)
    assert sr.normalize_params(100, 101, 0.5) == (100, 0.5)
    assert sr.normalize_params(100, -3, 1.5) == (100, 1.0)
    assert sr.normalize_params(100, 7, -0.1) == (7, 1.0)
    assert sr.normalize_params(100, 7, 0.0) == (1, 1.0)


def _probs(V, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    return sr.probabilities(rng.standard_normal(V).astype(np.float32) * scale, 1.0)


def test_probabilities_are_softmax():
    rng = np.random.default_rng(1)
    l = (rng.standard_normal(1000) * 4).astype(np.float32)
    pen = (rng.random(1000) * 2).astype(np.float32)
    for T in (0.5, 1.0, 2.7):
        for pn in (None, pen):
            z = (l.astype(np.float64) - (0 if pn is None else pn.astype(np.float64))) / T
            want = np.exp(z - z.max())
            want /= want.sum()
            np.testing.assert_allclose(sr.probabilities(l, T, pn), want, rtol=2e-6, atol=1e-12)


def test_probabilities_nan_and_inf():
    l = np.array([1.0, np.nan, 0.0, -np.inf], dtype=np.float32)
    p = sr.probabilities(l, 1.0)
    assert p[1] == p[2] > 0 and p[3] == 0.0       # NaN acts as 0, -inf as -FLT_MAX
    l = np.array([1.0, np.inf, 5.0, 0.0], dtype=np.float32)
    np.testing.assert_array_equal(sr.probabilities(l, 1.0), [0.0, 1.0, 0.0, 0.0])


def test_top_k_one_is_argmax():
    for seed in range(5):
        p = _probs(5000, seed)
        w = sr.kept_weights(p, 1, 1.0)
        assert np.flatnonzero(w).tolist() == [int(np.argmax(p))]


@pytest.mark.parametrize("k", [2, 5, 50, 999])
def test_top_k_keeps_k_largest(k):
    p = _probs(1000, k)
    w = sr.kept_weights(p, k, 1.0)
    assert set(np.flatnonzero(w)) == set(np.argsort(-p)[:k].tolist())
    np.testing.assert_array_equal(w[w > 0], p[w > 0])  # distinct values: no compensation


@pytest.mark.parametrize("top_p", [0.05, 0.3, 0.77, 0.999])
def test_top_p_keeps_shortest_prefix_with_exact_mass(top_p):
    p = _probs(2000, 11, scale=2.0)
    w = sr.kept_weights(p, 2000, top_p)
    order = np.argsort(-p)
    n = int(np.searchsorted(np.cumsum(p[order]), top_p)) + 1  # shortest prefix reaching top_p
    assert set(np.flatnonzero(w)) == set(order[:n].tolist())
    assert abs(w.sum() - top_p) < 1e-12
    np.testing.assert_array_equal(w[order[:n - 1]], p[order[:n - 1]])


def test_top_k_and_top_p_together_take_the_smaller_set():
    p = _probs(3000, 5, scale=1.0)  # flat: top-p 0.5 needs many entries
    w = sr.kept_weights(p, 20, 0.5)
    assert np.count_nonzero(w) == 20
    p = _probs(3000, 5, scale=6.0)  # peaked: top-p 0.5 needs few
    w = sr.kept_weights(p, 200, 0.5)
    assert np.count_nonzero(w) < 200 and abs(w.sum() - 0.5) < 1e-12


def test_ties_share_the_budget():
    p = np.full(8, 1.0 / 8)
    w = sr.kept_weights(p, 3, 1.0)
    np.testing.assert_allclose(w, np.full(8, 3.0 / 64))     # 3 entries' worth, spread evenly
    p = np.array([0.4, 0.2, 0.2, 0.2])
    w = sr.kept_weights(p, 2, 1.0)                        # 0.4 kept, one of three 0.2s
    np.testing.assert_allclose(w, [0.4, 0.2 / 3, 0.2 / 3, 0.2 / 3])
    w = sr.kept_weights(p, 4, 0.5)                        # 0.4 + 0.1 spread over the ties
    np.testing.assert_allclose(w, [0.4, 0.1 / 3, 0.1 / 3, 0.1 / 3])


def test_inverse_cdf():
    w = np.array([0.0, 1.0, 0.0, 3.0])
    assert sr.inverse_cdf(w, 0.25)[0] == 1
    assert sr.inverse_cdf(w, 0.2500001)[0] == 3
    assert sr.inverse_cdf(w, 1.0)[0] == 3
    assert sr.inverse_cdf(w, 1e-7)[0] == 1
    tok, margin = sr.inverse_cdf(w, 0.5)
    assert tok == 3 and abs(margin - 0.25) < 1e-12


def test_draw_order_is_a_permutation():
    for V in (4, 4096, 4100, 65532, 65536, 100000):
        o = sr.draw_order(V)
        assert np.array_equal(np.sort(o), np.arange(V))
    o = sr.draw_order(8192)
    assert o[:8].tolist() == [0, 1, 2, 3, 4096, 4097, 4098, 4099]   # lane 0: slots 0 and 1024
    assert o[8:12].tolist() == [4, 5, 6, 7]                          # then lane 1
    w = np.zeros(8192)
    w[[4096, 5]] = 1.0   # vocabulary order meets 5 first, the draw order 4096
    assert sr.inverse_cdf(w, 0.5)[0] == 5
    assert sr.inverse_cdf(w, 0.5, o)[0] == 4096


def test_top_p_one_sets_no_mass_limit():
    p = _probs(1000, 2)
    w = sr.kept_weights(p, 10, 1.0)
    assert set(np.flatnonzero(w)) == set(np.argsort(-p)[:10].tolist())


def test_sampling_law_matches_kept_weights():
    # inverse CDF at Philox uniforms: frequencies follow the kept weights
    p = _probs(64, 3, scale=1.5)
    w = sr.kept_weights(p, 10, 0.9)
    u = sr.uniforms(99, 0, 40000)
    toks = np.searchsorted(np.cumsum(w), u * w.sum(), side="left")
    freq = np.bincount(toks, minlength=64) / len(u)
    q = w / w.sum()
    keep = q > 0
    chi2 = np.sum((freq[keep] - q[keep]) ** 2 / q[keep]) * len(u)
    assert chi2 < 40.0  # <= 10 categories: p ~ 1e-5 at 40
    assert freq[~keep].sum() == 0


def test_update_penalties():
    pen = np.array([0.0, 0.5, 0.0], dtype=np.float32)
    np.testing.assert_array_equal(sr.update_penalties(pen, 0, 1.5, 0.25, 0.5), [1.5, 0.25, 0.0])
    np.testing.assert_array_equal(sr.update_penalties(pen, 1, 1.5, 0.25, 0.5), [0.0, 0.5, 0.0])
    np.testing.assert_array_equal(sr.update_penalties(pen, 2, 1.5, 0.25, 1.0), [0.0, 0.5, 1.5])
