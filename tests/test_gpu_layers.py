"""Attention (GQA) and GatedDeltaNet blocks, the residual stream and the route tail on the
GPU vs the CPU oracle (c/qwen.c:581-776 and :1228-1352 restated in oracle/oracle.c).

Tolerance: block outputs and residuals within maxrel_scaled 1e-3 (fp32 accumulation);
KV rows and recurrent state within 1e-4 relative to their magnitude; routed expert ids
identical to the oracle's on the same normed input (the stream's nrm read back).
"""
import numpy as np
import pytest

import _layers
import _stack
import _util
from _moe import Layer, Table
from _util import P

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def lorc(orc):
    _layers.bind(orc)
    return orc


def rel_to_max(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(1e-30, float(np.max(np.abs(ref)))))


# ---------------------------------------------------------------- GQA block
GQA_SHAPES = {   # D, H, KH, hd, rot, gs, max_t, layer
    "small": (256, 4, 2, 64, 16, 64, 16, 3),
    "cfg3": (2048, 16, 2, 256, 64, 128, 64, 4),
    # query heads per kv head 1, 3 and 16: the partial kernel's P.V splits a group's heads
    # over two thread halves (odd groups, an empty half, the largest group)
    "mha": (256, 4, 4, 64, 16, 64, 40, 140),
    "g3": (256, 6, 2, 64, 32, 64, 40, 141),
    "g16": (512, 32, 2, 128, 32, 128, 40, 142),
}


@pytest.mark.parametrize("shape", sorted(GQA_SHAPES))
def test_gqa_full(lib, lorc, gen, shape):
    """coli_vk_gqa_full over consecutive positions (one call per token and one call of
    several tokens), KV mirror rows checked against the oracle's cache."""
    D, H, KH, hd, rot, gs, max_t, layer = GQA_SHAPES[shape]
    W = _layers.GqaWeights(gen, gen.stream(0x9A00, layer), D, H, KH, hd, rot, gs)
    tq, tk, tv, to = (m.upload(lib) for m in (W.q, W.k, W.v, W.o))
    lib.kv_ensure(layer, KH * max_t, hd, hd)
    lib.gqa_norm_weight(layer, W.qn, W.kn)
    cache = W.new_cache(max_t)
    T = 7
    xs = [gen.normal(D, 0x9A10 + t) for t in range(T)]
    for t in range(4):
        y = lib.gqa_full(layer, xs[t], tq, tk, tv, to, 1, H, KH, hd, rot, t, max_t, W.eps, W.theta)
        ref = W.oracle(lorc, cache, max_t, t, xs[t])
        err = _util.maxrel_scaled(y, ref)
        print(f"gqa {shape} pos {t}: maxrel_scaled {err:.2e}", flush=True)
        assert err <= TOL, (t, err)
    y = lib.gqa_full(layer, np.concatenate(xs[4:]), tq, tk, tv, to, 3, H, KH, hd, rot, 4, max_t, W.eps, W.theta)
    for t in range(4, T):
        ref = W.oracle(lorc, cache, max_t, t, xs[t])
        assert _util.maxrel_scaled(y[(t - 4) * D:(t - 3) * D], ref) <= TOL, t
    for h in range(KH):
        Kd, Vd = lib.kv_read(layer, h * max_t, T, hd, hd)
        Kr = cache[0].reshape(KH, max_t, hd)[h, :T]
        Vr = cache[1].reshape(KH, max_t, hd)[h, :T]
        assert rel_to_max(Kd, Kr) < 1e-4 and rel_to_max(Vd, Vr) < 1e-5


def test_gqa_long_cache(lib, lorc, gen):
    """The config-3 block at the end of a 4096-position cache (decode at pos 4095 and
    earlier positions that split the window unevenly): rows seeded on both sides."""
    D, H, KH, hd, rot, gs, max_t, layer = 2048, 16, 2, 256, 64, 128, 4096, 5
    W = _layers.GqaWeights(gen, gen.stream(0x9B00, 1), D, H, KH, hd, rot, gs)
    tq, tk, tv, to = (m.upload(lib) for m in (W.q, W.k, W.v, W.o))
    lib.kv_ensure(layer, KH * max_t, hd, hd)
    lib.gqa_norm_weight(layer, W.qn, W.kn)
    Kc = gen.normal(KH * max_t * hd, 0x9B10, 1.0)
    Vc = gen.normal(KH * max_t * hd, 0x9B11, 1.0)
    lib.kv_load(layer, 0, Kc.reshape(-1, hd), Vc.reshape(-1, hd))
    cache = (Kc.copy(), Vc.copy())
    for pos in (4095, 1000, 31, 32):
        x = gen.normal(D, 0x9B20 + pos)
        y = lib.gqa_full(layer, x, tq, tk, tv, to, 1, H, KH, hd, rot, pos, max_t, W.eps, W.theta)
        ref = W.oracle(lorc, cache, max_t, pos, x)
        err = _util.maxrel_scaled(y, ref)
        print(f"gqa pos {pos}: maxrel_scaled {err:.2e}", flush=True)
        assert err <= TOL, (pos, err)


@pytest.fixture(scope="module")
def lorc_omp(orc_omp):
    _layers.bind(orc_omp)
    return orc_omp


GQA_ROWS = {   # D, H, KH, hd, rot, gs, max_t, layer, S, pos_base, S2 (a continuation call)
    "cfg3": (2048, 16, 2, 256, 64, 128, 4096, 20, 512, 0, 64),
    "hd128": (512, 32, 2, 128, 32, 128, 200, 21, 37, 3, 9),
    "hd64": (256, 4, 2, 64, 16, 128, 100, 22, 20, 30, 5),
}


@pytest.mark.parametrize("shape", sorted(GQA_ROWS))
def test_gqa_full_rows(lib, lorc_omp, gen, shape):
    """coli_vk_gqa_full with S >= 4 rows: one batched pass (q/k/v and o-projection GEMMs on
    MFMA, the norms, RoPE and KV writes of all rows, causal attention on fp32 MFMA) against
    the oracle's token loop (c/qwen.c:581-667), then a continuation call of S2 rows; cache
    rows before pos_base are seeded, partial 16-row query tiles occur; the KV rows the passes
    write against the oracle's cache."""
    D, H, KH, hd, rot, gs, max_t, layer, S, pos_base, S2 = GQA_ROWS[shape]
    W = _layers.GqaWeights(gen, gen.stream(0x9E00, layer), D, H, KH, hd, rot, gs)
    tq, tk, tv, to = (m.upload(lib) for m in (W.q, W.k, W.v, W.o))
    lib.kv_ensure(layer, KH * max_t, hd, hd)
    lib.gqa_norm_weight(layer, W.qn, W.kn)
    Kc = gen.normal(KH * max_t * hd, 0x9E10 + layer, 1.0)
    Vc = gen.normal(KH * max_t * hd, 0x9E11 + layer, 1.0)
    lib.kv_load(layer, 0, Kc.reshape(-1, hd), Vc.reshape(-1, hd))
    cache = (Kc.copy(), Vc.copy())
    pos = pos_base
    for n, seed in ((S, 0x9E20), (S2, 0x9E21)):
        xs = gen.normal(n * D, seed + layer)
        y = lib.gqa_full(layer, xs, tq, tk, tv, to, n, H, KH, hd, rot, pos, max_t, W.eps, W.theta)
        worst = 0.0
        for t in range(n):
            ref = W.oracle(lorc_omp, cache, max_t, pos + t, xs[t * D:(t + 1) * D])
            worst = max(worst, _util.maxrel_scaled(y[t * D:(t + 1) * D], ref))
        print(f"gqa rows {shape}: S={n} at pos {pos}: worst maxrel_scaled {worst:.2e}", flush=True)
        assert worst <= TOL, (n, pos, worst)
        pos += n
    for h in range(KH):
        Kd, Vd = lib.kv_read(layer, h * max_t + pos_base, pos - pos_base, hd, hd)
        Kr = cache[0].reshape(KH, max_t, hd)[h, pos_base:pos]
        Vr = cache[1].reshape(KH, max_t, hd)[h, pos_base:pos]
        assert rel_to_max(Kd, Kr) < 1e-4 and rel_to_max(Vd, Vr) < 1e-5


# ---------------------------------------------------------------- GDN block
host_params = _layers.gdn_host_params


@pytest.mark.parametrize("shape", ["small", "cfg3"])
def test_gdn_full_seq(lib, lorc, gen, shape):
    """coli_vk_gdn_full_seq (host params) over a few tokens from a fresh state; the
    device conv ring and recurrent state against the oracle's."""
    if shape == "small":
        D, KH, KD, VH, VD, K, gs, layer = 256, 2, 64, 4, 32, 4, 64, 7
    else:
        D, KH, KD, VH, VD, K, gs, layer = 2048, 16, 128, 32, 128, 4, 128, 8
    W = _layers.GdnWeights(gen, gen.stream(0x9C00, layer), D, KH, KD, VH, VD, K, gs)
    tqkv, tz, tout = (m.upload(lib) for m in (W.qkv, W.z, W.out))
    lib.gdn_setup(layer, VH, KD, VD, K, W.CD, W.conv)
    lib.gdn_reset()
    st = W.new_state()
    T = 5
    xs = [gen.normal(D, 0x9C10 + t) for t in range(T)]
    ps = [host_params(lorc, W, x) for x in xs]
    for t in range(2):
        y = lib.gdn_full_seq(layer, xs[t], ps[t], tqkv, tz, tout, 1, KH, KD, VH, VD, W.CD, K, W.eps)
        ref = W.oracle(lorc, st, xs[t])
        err = _util.maxrel_scaled(y, ref)
        print(f"gdn {shape} token {t}: maxrel_scaled {err:.2e}", flush=True)
        assert err <= TOL, (t, err)
    y = lib.gdn_full_seq(layer, np.concatenate(xs[2:]), np.concatenate(ps[2:]), tqkv, tz, tout, T - 2, KH, KD, VH,
                         VD, W.CD, K, W.eps)
    for t in range(2, T):
        ref = W.oracle(lorc, st, xs[t])
        assert _util.maxrel_scaled(y[(t - 2) * D:(t - 1) * D], ref) <= TOL, t
    ring, S = lib.gdn_state_read(layer, K, W.CD, VH, KD, VD)
    assert rel_to_max(ring, st[0]) < 1e-5
    assert rel_to_max(S, st[1]) < 1e-4


# ---------------------------------------------------------------- the decode stream
SMALL = dict(D=256, gqa=dict(H=4, KH=2, hd=64, rot=16, gs=64), gdn=dict(KH=2, KD=64, VH=4, VD=32, K=4, gs=64))


@pytest.fixture(scope="module")
def moe_small(lib, gen):
    return Table(lib, [Layer(lib, gen, 0x9D00, 256, 128, 32, 64)])


def run_stream(lib, lorc, gen, stack, router, K, T, fused, base):
    """T tokens through the stream: per token stream_begin, every layer's route_pipe
    (fused MoE, or top-k read back + expert_group_issue_pipe), stream_end."""
    D = stack.D
    L = stack.moe
    resid_h = None
    for t in range(T):
        x = gen.normal(D, base + t)
        lib.stream_begin(x)
        ref = x.copy()
        ids = []
        for i in range(len(stack.layers)):
            idx, val = stack.pipe_layer(lib, i, t, K, router)
            assert lib.stream_moe_fused() == fused
            ref, nrm_o, idx_o, val_o = stack.oracle_layer(lorc, i, ref, t, K)
            if not fused:
                nrm = lib.stream_nrm(D)
                # identical routing on the same normed row: the oracle's router + top-k
                _, i2, v2, _ = L.oracle(lorc, nrm, K)
                assert np.array_equal(idx, i2), (t, i, idx, i2)
                np.testing.assert_allclose(val, v2, rtol=1e-5, atol=1e-7)
                assert _util.maxrel_scaled(nrm, nrm_o) <= TOL
                ex = [L.t[e] for e in idx] + [L.t[L.E]]
                shgt = 1.0 / (1.0 + np.exp(-np.float64(np.dot(L.mw.sh_gate.astype(np.float64), nrm))))
                lib.expert_group_issue_pipe([e[0] for e in ex], [e[1] for e in ex], [e[2] for e in ex],
                                            list(val) + [np.float32(shgt)])
            ids.append(idx_o)
        resid_h = lib.stream_end(D)
        err = _util.maxrel_scaled(resid_h, ref)
        print(f"stream token {t} ({'fused' if fused else 'pipe'}): resid maxrel_scaled {err:.2e}", flush=True)
        assert err <= TOL, (t, err)
        if fused:
            for i in range(len(stack.layers)):
                assert np.array_equal(lib.stream_ix_hist(stack.first + i, K), ids[i]), (t, i)
    return resid_h


def test_stream_fused_small(lib, lorc, gen, moe_small):
    """4 layers (3 GDN with device a/b + 1 GQA), the MoE of every layer fused on the device."""
    L = moe_small.activate()[0]
    lib.eg_table_init(4, L.E, L.D, L.I, L.gs)
    for l in range(4):
        L.register(lib, l)
    stack = _stack.Stack(lib, gen, 0x9E00, 4, 256, SMALL["gqa"], SMALL["gdn"], L, max_t=16)
    run_stream(lib, lorc, gen, stack, L.router, 4, 4, True, 0x9E80)
    assert lib.moe_error() == 0
    import _moe
    _moe._active[0] = None   # the table was re-dimensioned here


def test_stream_pipe_small(lib, lorc, gen, moe_small):
    """The same stack with no expert table for its layers: device top-k read back, experts
    through coli_vk_expert_group_issue_pipe into the device residual (c/qwen.c:934-998)."""
    L = moe_small[0]
    lib.eg_table_init(1, L.E, L.D, L.I, L.gs)   # layers 10.. have no table slots
    import _moe
    _moe._active[0] = None
    stack = _stack.Stack(lib, gen, 0x9F00, 4, 256, SMALL["gqa"], SMALL["gdn"], L, max_t=16, ab_fmt=0,
                         first_layer=10)
    run_stream(lib, lorc, gen, stack, L.router, 8, 3, False, 0x9F80)


def test_gqa_full_route(lib, lorc, gen):
    """coli_vk_gqa_full_route (prefill form, S tokens): residual, nrm and router logits."""
    D, H, KH, hd, rot, gs, max_t, layer, ln = 256, 4, 2, 64, 16, 64, 16, 9, 30
    W = _layers.GqaWeights(gen, gen.stream(0xA000, 1), D, H, KH, hd, rot, gs)
    tq, tk, tv, to = (m.upload(lib) for m in (W.q, W.k, W.v, W.o))
    lib.kv_ensure(layer, KH * max_t, hd, hd)
    lib.gqa_norm_weight(layer, W.qn, W.kn)
    lib.layer_norm_weight(ln, W.in_ln, W.post_ln)
    E = 32
    rw = gen.f32rows(E, D, 0xA001, 0.02)
    router = lib.tensor(rw, None, 0, D, E)
    S = 3
    resid = gen.normal(S * D, 0xA002)
    ro, no, pr = lib.gqa_full_route(layer, resid, tq, tk, tv, to, router, ln, S, H, KH, hd, rot, 0, max_t, W.eps,
                                    W.theta)
    cache = W.new_cache(max_t)
    for s in range(S):
        r = resid[s * D:(s + 1) * D]
        x = _stack.rms(lorc, r, W.in_ln, W.eps)
        r2 = (r + W.oracle(lorc, cache, max_t, s, x)).astype(np.float32)
        n2 = _stack.rms(lorc, r2, W.post_ln, W.eps)
        p2 = np.empty(E, np.float32)
        lorc.orc_matmul_f32(P(p2), P(n2), P(rw), 1, D, E)
        assert _util.maxrel_scaled(ro[s * D:(s + 1) * D], r2) <= TOL
        assert _util.maxrel_scaled(no[s * D:(s + 1) * D], n2) <= TOL
        assert _util.maxrel_scaled(pr[s * E:(s + 1) * E], p2) <= TOL
