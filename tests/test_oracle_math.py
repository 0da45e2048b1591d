"""Pins of the CPU oracle that do not depend on the reference build: closed forms of the
fmt=6 GEMV, f64 brute force, invariants of the routing selection (c/qwen.c:806-817),
exact-tie behaviour, and known-answer values of the synthetic-data generator.

Each check is chosen so a plausible slip in the restatement (a dropped zero-point term,
a swapped nibble order, a wrong group index, ties resolved to the higher index) fails.
"""
import numpy as np
import pytest

from _util import P, brute_fmt6, eptr, int8_rows, maxrel, normrel


def gemv(orc, q, sz, x, I, O, gs):
    y = np.empty(O, np.float32)
    orc.orc_matmul_q4g_asym(P(y), P(x), P(q), P(sz), I, O, gs)
    return y


def test_splitmix64_known_answers(orc):
    # splitmix64 (Steele, Lea, Flood 2014) seeded with 0 and with 1234567: published outputs
    assert [orc.orc_hash(0, i) for i in range(4)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert orc.orc_hash(1234567, 0) == 0x599ED017FB08FC85


def test_generator_distributions(gen):
    b = gen.bytes(1 << 20, 3)
    lo, hi = b & 15, b >> 4
    for n in (lo, hi):
        c = np.bincount(n, minlength=16) / n.size
        assert np.all(np.abs(c - 1 / 16) < 0.003)
    x = gen.normal(1 << 18, 4).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    sz = gen.sz(1 << 16, 5, 0.02)
    s, z = sz[0::2].astype(np.float64), sz[1::2]
    assert np.all(s >= 0) and abs(s.mean() - 0.02 * np.sqrt(2 / np.pi)) < 3e-4
    assert np.array_equal(np.unique(z), np.arange(16, dtype=np.float32))
    # scales are binary16 values
    assert np.array_equal(s.astype(np.float16).astype(np.float64), s)


def test_f16_round_matches_numpy(orc):
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.normal(0, 0.02, 5000), rng.normal(0, 1e-6, 500), [0.0, 65504.0, 6.1e-5, 3e-8]])
    got = np.array([orc.orc_f16_round(float(a)) for a in v], np.float32)
    want = v.astype(np.float16).astype(np.float32)   # IEEE round-to-nearest-even
    assert np.array_equal(got, want)


@pytest.mark.parametrize("O,I,gs", [(64, 2048, 128), (31, 250, 32), (16, 129, 8), (8, 512, 512)])
def test_fmt6_brute_force(orc, gen, O, I, gs):
    q, sz = gen.fmt6(O, I, gs, O * 131 + I)
    x = gen.normal(I, 9)
    y = gemv(orc, q, sz, x, I, O, gs)
    yb = brute_fmt6(q, sz, x, I, O, gs)
    assert maxrel(y, yb) < 1e-4 and normrel(y, yb) < 1e-6


def test_fmt6_integer_dot(orc, gen):
    """s=1, z=0: y is the exact integer-weighted dot with integer x."""
    O, I, gs = 16, 256, 64
    q = gen.bytes(O * I // 2, 11)
    sz = np.zeros(O * (I // gs) * 2, np.float32)
    sz[0::2] = 1.0
    x = (np.arange(I) % 7 - 3).astype(np.float32)
    y = gemv(orc, q, sz, x, I, O, gs)
    nib = np.stack([q.reshape(O, -1) & 15, q.reshape(O, -1) >> 4], -1).reshape(O, I).astype(np.int64)
    assert np.array_equal(y.astype(np.int64), nib @ x.astype(np.int64))


def test_fmt6_constant_nibbles(orc, gen):
    """every nibble n, one group: y = s (n - z) sum(x)."""
    O, I = 4, 128
    for n in (0, 7, 15):
        q = np.full(O * I // 2, n | (n << 4), np.uint8)
        sz = np.array([0.5, 3.0] * O, np.float32)
        x = gen.normal(I, 12)
        y = gemv(orc, q, sz, x, I, O, I)
        want = 0.5 * (n - 3.0) * x.astype(np.float64).sum()
        assert np.allclose(y, want, rtol=1e-5, atol=1e-5)


def test_fmt6_nibble_order(orc):
    """element i in byte i>>1, low nibble for even i (c/qwen.c:222)."""
    I, O = 8, 1
    q = np.array([0x21, 0x43, 0x65, 0x87], np.uint8)   # elements 1,2,3,...,8
    sz = np.array([1.0, 0.0], np.float32)
    x = np.zeros(I, np.float32)
    for i in range(I):
        x[:] = 0
        x[i] = 1
        assert gemv(orc, q, sz, x, I, O, 8)[0] == i + 1


def test_fmt6_group_index(orc):
    """group g covers elements [g*gs, (g+1)*gs): a per-group scale hits only its group."""
    I, O, gs = 64, 1, 16
    q = np.full(I // 2, 0x11, np.uint8)
    sz = np.zeros(2 * (I // gs), np.float32)
    x = np.ones(I, np.float32)
    for g in range(I // gs):
        sz[:] = 0
        sz[2 * g] = 2.0
        assert gemv(orc, q, sz, x, I, O, gs)[0] == 2.0 * gs


def test_quant_rows_roundtrip(orc, gen):
    """RTN fmt 6: |w - (q - z) s| <= s/2 and zero points are real-valued (c/qwen.c:246-265)."""
    O, I, gs = 32, 512, 128
    W = gen.normal(O * I, 13, 0.05)
    q = np.empty(O * I // 2, np.uint8)
    sz = np.empty(O * (I // gs) * 2, np.float32)
    orc.orc_quant_rows(P(W), I, O, 6, gs, P(q), P(sz))
    nib = np.stack([q.reshape(O, -1) & 15, q.reshape(O, -1) >> 4], -1).reshape(O, I).astype(np.float64)
    s = sz.reshape(O, -1, 2)[:, np.arange(I) // gs, 0].astype(np.float64)
    z = sz.reshape(O, -1, 2)[:, np.arange(I) // gs, 1].astype(np.float64)
    err = np.abs(W.reshape(O, I) - (nib - z) * s)
    assert np.all(err <= s * 0.5 + 1e-6)
    assert np.any(z != np.round(z))


def route(orc, logits, K):
    pr = np.array(logits, np.float32)
    idx = np.empty(K, np.int32)
    val = np.empty(K, np.float32)
    orc.orc_route_topk(P(pr), pr.size, K, P(idx), P(val))
    return idx, val, pr


def test_int8_pow2_scale_equals_f32(orc, gen):
    """The GPU tests check an int8 (fmt 1) router against the f32 oracle on rows q * s
    with s = 2^-k: the two products must agree bit for bit, and a scale applied to the
    wrong row or dropped must not."""
    E, D, S = 32, 256, 4
    q, s, f = int8_rows(gen, 0x1A8, E, D)
    assert len(set(s.tolist())) == 3
    for t in range(S):
        x = gen.normal(D, 0x1B0 + t)
        y8, yf = np.empty(E, np.float32), np.empty(E, np.float32)
        orc.orc_matmul_q8(P(y8), P(x), P(q.view(np.uint8)), P(s), D, E)
        orc.orc_matmul_f32(P(yf), P(x), P(f), 1, D, E)
        assert np.array_equal(y8, yf)
        y64 = (q.astype(np.float64) @ x.astype(np.float64)) * s
        assert maxrel(y8, y64) < 1e-4
        ys = np.empty(E, np.float32)
        orc.orc_matmul_q8(P(ys), P(x), P(q.view(np.uint8)), P(np.roll(s, 1)), D, E)
        assert not np.allclose(ys, yf, rtol=1e-3)


def test_route_invariants(orc, gen):
    for seed in range(20):
        lg = gen.normal(256, 100 + seed, 0.9)
        idx, val, prob = route(orc, lg, 8)
        assert len(set(idx.tolist())) == 8
        assert np.all(np.diff(prob[idx]) <= 0)                       # rank order
        assert set(idx.tolist()) == set(np.argsort(-lg, kind="stable")[:8].tolist())
        sm = np.exp(lg[idx].astype(np.float64) - lg.max())
        assert np.allclose(val, sm / sm.sum(), rtol=1e-5)            # softmax over chosen
        assert abs(float(val.astype(np.float64).sum()) - 1) < 1e-6


def test_route_ties_lower_index(orc):
    lg = np.zeros(16, np.float32)
    lg[[3, 9, 12]] = 2.0
    lg[[5, 1]] = 1.5
    idx, val, _ = route(orc, lg, 4)
    assert idx.tolist() == [3, 9, 12, 1]
    assert val[0] == val[1] == val[2]


def test_argmax_topk(orc, gen):
    v = gen.normal(10000, 7)
    v[[10, 5000, 9999]] = 9.0
    assert orc.orc_argmax(P(v), v.size) == 10
    idx = np.empty(8, np.int32)
    val = np.empty(8, np.float32)
    orc.orc_topk_logits(P(v), v.size, 8, P(idx), P(val))
    want = np.lexsort((np.arange(v.size), -v))[:8]
    assert np.array_equal(idx, want) and np.array_equal(val, v[want])


def test_rmsnorm_zc_closed_form(orc, gen):
    D = 2048
    x = gen.normal(D, 21)
    w = gen.normal(D, 22, 0.1)
    y = np.empty(D, np.float32)
    orc.orc_rmsnorm_zc(P(y), P(x), P(w), D, np.float32(1e-6))
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean() + 1e-6) * (1 + w.astype(np.float64))
    assert np.allclose(y, want, rtol=2e-6, atol=1e-6)


def test_moe_prefill_equals_per_token(orc, gen):
    """Grouping by expert changes only the summation order (c/qwen.c:1050-1183 vs :804-920)."""
    from _util import MoeWeights
    D, I, E, K, gs, S = 128, 64, 16, 4, 32, 12
    mw = MoeWeights(gen, 77, D, I, E, gs)
    ex = mw.orc_experts()
    xs = gen.normal(S * D, 78)
    out = np.empty(S * D, np.float32)
    tidx = np.empty(S * K, np.int32)
    tval = np.empty(S * K, np.float32)
    orc.orc_moe_prefill(P(xs), S, P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(out), P(tidx), P(tval))
    for s in range(S):
        o1 = np.empty(D, np.float32)
        i1 = np.empty(K, np.int32)
        v1 = np.empty(K, np.float32)
        x = xs[s * D:(s + 1) * D].copy()
        orc.orc_moe_decode(P(x), P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(o1), P(i1), P(v1),
                           None, None)
        assert np.array_equal(i1, tidx[s * K:(s + 1) * K]) and np.array_equal(v1, tval[s * K:(s + 1) * K])
        assert np.allclose(out[s * D:(s + 1) * D], o1, rtol=1e-5, atol=1e-6)


def test_moe_decode_composition(orc, gen):
    """moe_decode == sum_k val_k * expert_k(x) + sigmoid(sh_gate.x) * shared(x), from parts."""
    from _util import MoeWeights
    D, I, E, K, gs = 256, 64, 32, 8, 64
    mw = MoeWeights(gen, 91, D, I, E, gs)
    ex = mw.orc_experts()
    x = gen.normal(D, 92)
    out = np.empty(D, np.float32)
    idx = np.empty(K, np.int32)
    val = np.empty(K, np.float32)
    orc.orc_moe_decode(P(x), P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(out), P(idx), P(val),
                       None, None)
    acc = np.zeros(D, np.float64)
    for k in range(K):
        y = np.empty(D, np.float32)
        orc.orc_expert_mlp_fmt6(eptr(ex, int(idx[k])), P(x), D, I, gs, P(y))
        acc += float(val[k]) * y
    y = np.empty(D, np.float32)
    orc.orc_expert_mlp_fmt6(eptr(ex, E), P(x), D, I, gs, P(y))
    g = 1 / (1 + np.exp(-np.dot(mw.sh_gate.astype(np.float64), x)))
    acc += g * y
    assert np.allclose(out, acc, rtol=1e-5, atol=1e-6)
    # expert MLP from its definition: down(silu(gate x) * (up x)), f64
    g_, u_, d_ = mw.exp[int(idx[0])]
    hg = brute_fmt6(g_[0], g_[1], x, D, I, gs)
    hu = brute_fmt6(u_[0], u_[1], x, D, I, gs)
    h = hg / (1 + np.exp(-hg)) * hu
    y0 = brute_fmt6(d_[0], d_[1], h.astype(np.float32), I, D, gs)
    yk = np.empty(D, np.float32)
    orc.orc_expert_mlp_fmt6(eptr(ex, int(idx[0])), P(x), D, I, gs, P(yk))
    assert normrel(yk, y0) < 1e-5


def test_neartie_construction_flips_exact_ranking(orc, gen):
    """The near-tie routers of the GPU routing tests really separate the two orders: the
    reference's picks (sequential fp32 logits, c/qwen.c:178-189, 807-817) differ from the
    picks of exact arithmetic both in order (ranks 1-2) and in the set (rank K), so a device
    that ranked by exact logits would fail those tests."""
    import _neartie
    D, E, K = 2048, 256, 8
    for seed in (0x7E1, 0x7E2, 0x7E3):
        x = gen.normal(D, seed)
        W = _neartie.near_tie_router(orc, gen, x, E, D, K, seed)
        ref, _ = _neartie.route_ref(orc, _neartie.seq_logits(orc, x, W, E, D), K)
        ex = _neartie.exact_rank(x, W, D, K)
        assert ref[0] == ex[1] and ref[1] == ex[0], (ref, ex)          # order flipped
        assert ref[K - 1] != ex[K - 1] and set(ref[:K - 1]) == set(ex[:K - 1])   # the K-th pick differs
