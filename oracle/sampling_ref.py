"""CPU oracle (numpy) for token sampling -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may use this module; the product (``vkwr``, ``vkwr_amd``) never does.

Restates the reference's sampling kernels (csrc/sampling/sampling.cu; paths
relative to the reference root) one batch row at a time:

  probabilities   sampling.cu:183-226 (repetition), 470-505 (temperature):
                  u = sf((sf(l) - pen) * log2(e)/temperature), p = 2^(u - max u) / sum
  threshold       sampling.cu:228-282: the largest p value v whose set {p >= v}
                  holds >= top_k entries or >= top_p mass (the reference bisects
                  over float bit patterns; the answer is always one of the p values,
                  so this oracle scans the distinct values instead)
  compensation    sampling.cu:284-306: entries equal to tau keep the share of the
                  top_k / top_p budget left after the entries above tau
  draw            sampling.cu:307-343: a uniform in (0, 1] times the kept total,
                  first entry whose running kept sum reaches it.  The reference
                  visits the row in its own two-level order over its threads; the
                  product visits it in lane order (``draw_order``), which this
                  oracle follows.  The law of the draw is the same for any order.
  penalties       sampling.cu:345-358: pen <- fma(pen, decay, tok ? (pen == 0 ?
                  presence : repetition) : 0)
  parameters      sampling.cu:896-901: top_k <= 0 or > V -> V; top_p outside
                  [0, 1] -> 1; top_p == 0 -> top_k = 1, top_p = 1.  top_p = 1
                  sets no mass limit (the reference's mass test can then only
                  fire through float rounding of a sum that should stay below 1).

The draw's uniform comes from Philox4x32-10 (Salmon et al., SC'11), the
generator the product runs: key = seed (low word, high word), counter =
(call index low, call index high, row, 0), u = ((x0 >> 8) + 1) / 2^24.  The
reference draws from curand's Philox stream instead, which is not reproduced:
the oracle pins the product's law of the draw and its generator (against the
Random123 known-answer vectors), not the reference's random stream.

Probabilities are formed from float32 u as the kernels do and then carried in
float64, so they differ from a GPU's float32 values by a few ulp; tests choose
inputs whose kept set does not hinge on that and allow a token mismatch only
where the draw target lies within a relative 1e-5 of a CDF step.
"""
import numpy as np

LOG2E = 1.4426950408889634
FLT_MAX = np.float32(np.finfo(np.float32).max)

PHILOX_M = (0xD2511F53, 0xCD9E8D57)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)
MASK32 = 0xFFFFFFFF
THREADS = 1024  # lanes of the product's sampling workgroup


def philox4x32_10(ctr, key):
    """Philox4x32-10 blocks.  ctr: uint32 [..., 4], key: uint32 [..., 2] (broadcast)."""
    ctr = np.asarray(ctr, dtype=np.uint64)
    key = np.asarray(key, dtype=np.uint64)
    shape = np.broadcast_shapes(ctr.shape[:-1], key.shape[:-1])
    c = [np.broadcast_to(ctr[..., i], shape).copy() for i in range(4)]
    k0 = np.broadcast_to(key[..., 0], shape).copy()
    k1 = np.broadcast_to(key[..., 1], shape).copy()
    m0, m1 = np.uint64(PHILOX_M[0]), np.uint64(PHILOX_M[1])
    mask = np.uint64(MASK32)
    for r in range(10):
        if r:
            k0 = (k0 + np.uint64(PHILOX_W[0])) & mask
            k1 = (k1 + np.uint64(PHILOX_W[1])) & mask
        p0 = m0 * c[0]  # < 2^64: exact in uint64
        p1 = m1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & mask
        hi1, lo1 = p1 >> np.uint64(32), p1 & mask
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return np.stack(c, axis=-1).astype(np.uint32)


def uniforms(seed, row, calls):
    """The uniforms rows `row` draws on its calls 0..calls-1 after setup_rand(seed)."""
    n = np.arange(calls, dtype=np.uint64)
    ctr = np.stack([n & np.uint64(MASK32), n >> np.uint64(32),
                    np.full_like(n, row), np.zeros_like(n)], axis=-1)
    key = np.array([seed & MASK32, (seed >> 32) & MASK32], dtype=np.uint64)
    x0 = philox4x32_10(ctr, key)[..., 0].astype(np.uint64)
    return ((x0 >> np.uint64(8)) + np.uint64(1)).astype(np.float64) / float(1 << 24)


def normalize_params(V, top_k, top_p):
    """sampling.cu:896-901."""
    if top_k <= 0 or top_k > V:
        top_k = V
    if top_p < 0 or top_p > 1:
        top_p = 1.0
    if top_p == 0:
        top_k, top_p = 1, 1.0
    return top_k, float(np.float32(top_p))


def draw_order(V):
    """Vocabulary indices in the order the product's draw visits them: lane t of
    1024 owns the float4 slots t, t + 1024, t + 2048, ...; lanes in order, a lane's
    slots in order, the 4 entries of a slot in order."""
    V4 = V // 4
    J = -(-V4 // THREADS)
    slots = (np.arange(THREADS)[:, None] + THREADS * np.arange(J)[None, :]).reshape(-1)
    slots = slots[slots < V4]
    return (4 * slots[:, None] + np.arange(4)[None, :]).reshape(-1)


def _sf(x):
    x = np.where(np.isnan(x), np.float32(0), x).astype(np.float32)
    return np.where(np.isinf(x), np.copysign(FLT_MAX, x), x).astype(np.float32)


def probabilities(logits, temperature, penalties=None):
    """p (float64) of one row of fp32 logits [V]."""
    l = _sf(np.asarray(logits, dtype=np.float32))
    pen = np.zeros_like(l) if penalties is None else np.asarray(penalties, dtype=np.float32)
    scale = np.float32(LOG2E / temperature)
    with np.errstate(over="ignore", invalid="ignore"):
        u = _sf((l - pen).astype(np.float32) * scale)
    e = np.exp2(u.astype(np.float64) - float(u.max()))
    return e / e.sum()


def threshold(p, top_k, top_p):
    """(tau, comp) for probabilities p and normalised top_k / top_p."""
    order = np.sort(p)[::-1]                        # descending
    csum = np.cumsum(order)
    vals = np.unique(p)[::-1]                       # distinct values, descending
    cnt = np.searchsorted(-order, -vals, side="right")  # #(p >= v) for each distinct v
    use_mass = top_p < 1.0
    ok = (cnt >= top_k) | (use_mass & (csum[cnt - 1] >= top_p))   # the set {p >= v} is not small
    tau = vals[int(np.argmax(ok))] if ok.any() else vals[-1]
    neq = int(np.count_nonzero(p == tau))
    gt = p > tau
    ngt, mgt = int(np.count_nonzero(gt)), float(p[gt].sum())
    comp = 1.0
    if neq > 0:
        comp = min((top_k - ngt) / neq, 1.0)
        if use_mass:
            comp = min((top_p - mgt) / (tau * neq), comp)
        comp = max(comp, 0.0)
    return float(tau), comp


def kept_weights(p, top_k, top_p):
    """Weights of the truncated distribution (unnormalised), vocabulary order."""
    V = p.shape[0]
    if top_k >= V and top_p >= 1.0:
        return p.copy()
    tau, comp = threshold(p, top_k, top_p)
    return np.where(p > tau, p, np.where(p == tau, p * comp, 0.0))


def inverse_cdf(w, u, order=None):
    """(token, margin): first index (visiting w in `order`, default vocabulary order)
    whose running sum of w reaches u * sum(w), and the distance of that target from
    the nearest CDF step, relative to the total."""
    if order is not None:
        tok, margin = inverse_cdf(w[order], u)
        return int(order[tok]), margin
    c = np.cumsum(w)
    total = c[-1]
    target = total * u
    tok = int(np.searchsorted(c, target, side="left"))
    tok = min(tok, int(np.flatnonzero(w > 0)[-1]))
    steps = np.concatenate([[0.0], c[w > 0]])
    margin = float(np.min(np.abs(steps - target)) / total)
    return tok, margin


def cdf_interval(w, order, tok):
    """(start, end, total): the part of [0, total] that token `tok` covers when w is
    visited in `order`."""
    c = np.cumsum(w[order])
    k = int(np.flatnonzero(order == tok)[0])
    return (float(c[k - 1]) if k else 0.0), float(c[k]), float(c[-1])


def sample_row(logits, u, temperature=1.0, top_k=-1, top_p=1.0, penalties=None):
    """(token, margin, kept weights) of one row drawn at uniform u."""
    logits = np.asarray(logits, dtype=np.float32)
    top_k, top_p = normalize_params(logits.shape[-1], top_k, top_p)
    p = probabilities(logits, temperature, penalties)
    w = kept_weights(p, top_k, top_p)
    tok, margin = inverse_cdf(w, u, draw_order(logits.shape[-1]))
    return tok, margin, w


def update_penalties(pen, tok, presence, repetition, decay):
    """pen [V] fp32 after drawing tok (fma evaluated exactly, then rounded once)."""
    pen = np.asarray(pen, dtype=np.float32)
    add = np.zeros(pen.shape, dtype=np.float64)
    add[tok] = np.float32(presence) if pen[tok] == 0 else np.float32(repetition)
    exact = pen.astype(np.float64) * float(np.float32(decay)) + add  # pen*decay is exact in float64
    return exact.astype(np.float32)
