"""The CPU oracle is bit-identical to the reference's own CPU kernels.

tests/golden/*.npz hold outputs written by the reference's c/qwen.c compiled unmodified
(oracle/_ref, tests/golden/make_golden.py) on seeded inputs; the inputs are regenerated
here and checked against their SHA-256 before the comparison.  Where the reference build
is present, random shapes are also compared live.
"""
import glob
import hashlib
import os

import numpy as np
import pytest

import _util
from _util import P, eptr

FIX = sorted(glob.glob(os.path.join(_util.GOLDEN, "*.npz")))


def load(name):
    return np.load(os.path.join(_util.GOLDEN, name + ".npz"), allow_pickle=False)


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_fixtures_present():
    assert len(FIX) >= 12


@pytest.mark.parametrize("name", ["cfg0", "odd_I", "ragged_group", "gs8", "expert_down"])
def test_gemv_golden(orc, gen, name):
    f = load(f"gemv_{name}")
    O, I, gs, seed = (int(f[k]) for k in ("O", "I", "gs", "seed"))
    q, sz = gen.fmt6(O, I, gs, seed)
    x = gen.normal(I, gen.stream(seed, 7))
    assert digest(q, sz, x) == str(f["digest"])
    y = np.empty(O, np.float32)
    orc.orc_matmul_q4g_asym(P(y), P(x), P(q), P(sz), I, O, gs)
    assert np.array_equal(bits(y), bits(f["y"]))


def test_dense_golden(orc, gen):
    f = load("matmul_f32")
    O, I, S, seed = (int(f[k]) for k in ("O", "I", "S", "seed"))
    W = gen.f32rows(O, I, seed, 0.02)
    x = gen.normal(S * I, gen.stream(seed, 7))
    assert digest(W, x) == str(f["digest"])
    y = np.empty(S * O, np.float32)
    orc.orc_matmul_f32(P(y), P(x), P(W), S, I, O)
    assert np.array_equal(bits(y), bits(f["y"]))

    g = load("quant_rows")
    q6 = np.empty(O * I // 2, np.uint8)
    s6 = np.empty(O * (I // 128) * 2, np.float32)
    orc.orc_quant_rows(P(W), I, O, 6, 128, P(q6), P(s6))
    assert np.array_equal(q6, g["q6"]) and np.array_equal(bits(s6), bits(g["s6"]))
    q1 = np.empty(O * I, np.uint8)
    s1 = np.empty(O, np.float32)
    orc.orc_quant_rows(P(W), I, O, 1, 0, P(q1), P(s1))
    assert np.array_equal(q1, g["q1"]) and np.array_equal(bits(s1), bits(g["s1"]))
    y1 = np.empty(O, np.float32)
    orc.orc_matmul_q8(P(y1), P(x), P(q1), P(s1), I, O)
    assert np.array_equal(bits(y1), bits(g["y1"]))


def test_norm_softmax_golden(orc, gen):
    f = load("rmsnorm_zc")
    D = int(f["D"])
    x = gen.normal(D, 0xD1)
    w = gen.normal(D, 0xD2, 0.1)
    assert digest(x, w) == str(f["digest"])
    y = np.empty(D, np.float32)
    orc.orc_rmsnorm_zc(P(y), P(x), P(w), D, np.float32(1e-6))
    assert np.array_equal(bits(y), bits(f["y"]))
    f = load("softmax_row")
    lg = gen.normal(256, 0xD3, 0.9)
    assert digest(lg) == str(f["digest"])
    orc.orc_softmax_row(P(lg), 256)
    assert np.array_equal(bits(lg), bits(f["p"]))


@pytest.mark.parametrize("name", ["small", "cfg2"])
def test_moe_token_golden(orc, gen, name):
    """moe_token (c/qwen.c:922-928 -> :804-920): outputs bit-identical, and the chosen
    experts (the reference's usage counters) identical."""
    f = load(f"moe_token_{name}")
    D, I, E, K, gs, base, T = (int(f[k]) for k in ("D", "I", "E", "K", "gs", "base", "T"))
    mw = _util.MoeWeights(gen, base, D, I, E, gs)
    ex = mw.orc_experts()
    xs = gen.normal(T * D, gen.stream(base, 5))
    assert digest(mw.router, mw.sh_gate, xs) == str(f["digest"])
    for t in range(T):
        out = np.empty(D, np.float32)
        idx = np.empty(K, np.int32)
        x = xs[t * D:(t + 1) * D].copy()
        orc.orc_moe_decode(P(x), P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(out),
                           P(idx), None, None, None)
        assert np.array_equal(bits(out), bits(f["out"][t]))
        usage = np.zeros(E, np.uint32)
        usage[idx] = 1
        assert np.array_equal(usage, f["usage"][t])
    ye = np.empty(D, np.float32)
    orc.orc_expert_mlp_fmt6(eptr(ex, 3), P(xs[:D].copy()), D, I, gs, P(ye))
    assert np.array_equal(bits(ye), bits(f["expert3_y"]))


def test_moe_batch_golden(orc, gen):
    """moe_batch (c/qwen.c:1185-1190 -> :1050-1183): expert-grouped order, bit-identical."""
    f = load("moe_batch_small")
    D, I, E, K, gs, base, S = (int(f[k]) for k in ("D", "I", "E", "K", "gs", "base", "S"))
    mw = _util.MoeWeights(gen, base, D, I, E, gs)
    ex = mw.orc_experts()
    xs = gen.normal(S * D, gen.stream(base, 5))
    assert digest(mw.router, mw.sh_gate, xs) == str(f["digest"])
    out = np.empty(S * D, np.float32)
    tidx = np.empty(S * K, np.int32)
    orc.orc_moe_prefill(P(xs), S, P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(out),
                        P(tidx), None)
    assert np.array_equal(bits(out), bits(f["out"]))
    assert np.array_equal(np.bincount(tidx, minlength=E).astype(np.uint32), f["usage"])


@pytest.mark.parametrize("O,I,gs", [(97, 384, 64), (5, 2048, 128), (40, 200, 40)])
def test_gemv_live_vs_reference(orc, ref, gen, O, I, gs):
    q, sz = gen.fmt6(O, I, gs, O + I)
    x = gen.normal(I, 3)
    y1 = np.empty(O, np.float32)
    y2 = np.empty(O, np.float32)
    orc.orc_matmul_q4g_asym(P(y1), P(x), P(q), P(sz), I, O, gs)
    ref.ref_matmul_q4g_asym(P(y2), P(x), P(q), P(sz), I, O, gs)
    assert np.array_equal(bits(y1), bits(y2))


def test_moe_live_vs_reference(orc, ref, gen):
    D, I, E, K, gs = 128, 64, 24, 6, 32
    mw = _util.MoeWeights(gen, 0xF00, D, I, E, gs)
    ex = mw.orc_experts()
    for t in range(4):
        x = gen.normal(D, 500 + t)
        o1 = np.empty(D, np.float32)
        o2 = np.empty(D, np.float32)
        orc.orc_moe_decode(P(x), P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(o1),
                           None, None, None, None)
        ref.ref_moe_token(P(x), P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(o2), None)
        assert np.array_equal(bits(o1), bits(o2))
