"""Router rows with engineered near-ties for the routing-identity tests.

The reference ranks experts by p = softmax of router logits it computes as sequential fp32
sums (c/qwen.c:178-189, 332-336, 807-817).  Two experts whose exact dots x . w differ by
less than the rounding of those sums can come out in the opposite order in the reference:
a device that ranks by exact (or any other) arithmetic picks differently.  near_tie_router
builds such pairs on purpose for a given input row x: it takes the experts at two adjacent
ranks and rewrites the lower one as a copy of the upper one with two coordinates moved so
that the exact dot moves by < 1e-7 while the sequential fp32 sum lands on the other side,
with p values that still differ (so the pair is not the documented exact-tie class).  The
pairs sit at ranks (1, 2) (order inside the top K) and (K, K + 1) (which expert is picked).
"""
import numpy as np

from _util import P


def seq_logits(orc, x, W, E, D):
    """The reference's logits (orc_matmul_f32 is bit-identical to c/qwen.c:178-189)."""
    y = np.empty(E, np.float32)
    orc.orc_matmul_f32(P(y), P(np.ascontiguousarray(x, np.float32)), P(np.ascontiguousarray(W, np.float32)), 1, D, E)
    return y


def exact_logits(x, W, D):
    return W.reshape(-1, D).astype(np.float64) @ x.astype(np.float64)


def route_ref(orc, logits, K):
    """The reference's picks (orc_route_topk restates c/qwen.c:332-336, 807-817)."""
    pr = np.array(logits, np.float32)
    idx = np.empty(K, np.int32)
    val = np.empty(K, np.float32)
    orc.orc_route_topk(P(pr), pr.size, K, P(idx), P(val))
    return idx, val


def exact_rank(x, W, D, K):
    """The K best by exact dot (ties to the lower index): what exact arithmetic picks."""
    ex = exact_logits(x, W, D)
    return np.lexsort((np.arange(ex.size), -ex))[:K].astype(np.int32)


def _tie_pair(orc, x, W, D, hi, lo, rng, tries=400):
    """Make row lo a near-tie of row hi whose sequential-sum order is the opposite of its
    exact order.  Returns True on success (W modified in place)."""
    base = W[hi].copy()
    for _ in range(tries):
        j, k = sorted(rng.choice(D, 2, replace=False))
        if abs(x[j]) < 0.3 or abs(x[k]) < 0.3 or k - j < D // 4:
            continue
        d1 = np.float32(rng.choice([-1, 1]) * rng.uniform(0.005, 0.02))
        w = base.copy()
        w[j] = np.float32(w[j] + d1)
        dj = np.float64(w[j]) - np.float64(base[j])
        w[k] = np.float32(np.float64(base[k]) - dj * np.float64(x[j]) / np.float64(x[k]))
        ex_d = float(exact_logits(x, np.stack([base, w]), D) @ np.array([-1.0, 1.0]))   # exact(lo) - exact(hi)
        sq = seq_logits(orc, x, np.stack([base, w]), 2, D)
        sq_d = float(sq[1]) - float(sq[0])
        if ex_d != 0.0 and abs(ex_d) < 1e-7 and sq_d != 0.0 and np.sign(ex_d) != np.sign(sq_d):
            old = W[lo].copy()
            W[lo] = w
            p = seq_logits(orc, x, W, W.shape[0], D)
            orc.orc_softmax_row(P(p), p.size)
            if p[hi] != p[lo]:   # distinct p: the reference's order is by value, not the tie rule
                return True
            W[lo] = old
    return False


def near_tie_router(orc, gen, x, E, D, K, seed, sigma=0.02):
    """f32 router [E, D] (flat) with near-ties at ranks (1, 2) and (K, K + 1) for input x,
    each resolved one way by the reference's sequential sums and the other way by exact
    arithmetic.  Raises if no such construction was found."""
    x = np.ascontiguousarray(x, np.float32)
    rng = np.random.default_rng(seed)
    for attempt in range(20):
        W = gen.f32rows(E, D, gen.stream(seed, attempt), sigma).reshape(E, D).copy()
        order = np.argsort(-exact_logits(x, W, D), kind="stable")
        ex = exact_logits(x, W, D)
        # keep the pairs away from their neighbours (>= 5e-3) so only the pair is close
        gaps = -np.diff(ex[order])
        if gaps[1] < 5e-3 or gaps[K] < 5e-3 or gaps[K - 2] < 5e-3:
            continue
        if not _tie_pair(orc, x, W, D, order[0], order[1], rng):
            continue
        if not _tie_pair(orc, x, W, D, order[K - 1], order[K], rng):
            continue
        return np.ascontiguousarray(W.reshape(-1), np.float32)
    raise RuntimeError("no near-tie construction found")
