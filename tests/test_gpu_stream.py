"""The engine's own stream path on the GPU, at the argument formats and shapes the unchanged
c/qwen.c passes (c/qwen.c:1228-1290, 1392, 1436-1440, 1876-1878), against the CPU oracle.

- coli_vk_stream_norm_argmax (final zero-centred RMSNorm + lm_head + argmax, the call that
  emits every token of the stream path) at the configs[1] shape, including forced exact ties;
- *_route_pipe with an int8 (fmt 1) router and int8 GDN a/b, as vk_dense_init uploads them,
  fused (device expert table) and through the host-routed pipe;
- a configs[3]-geometry stream: 3 GatedDeltaNet layers (device fmt-6 a/b: the 4-segment
  in-projection) + 1 gated GQA layer decoding at positions 4094 and 4095 of a 4096-row
  cache, each with the configs[2] MoE (256 + 1 experts) fused.

Tolerance: residuals within maxrel_scaled 1e-3 (fp32 accumulation); routed ids identical to
the oracle's; the argmax equal to the oracle's unless the two logits lie within the GEMV
tolerance of each other (then the device's pick must be exact on the oracle's logits up to
that tolerance).
"""
import ctypes

import numpy as np
import pytest

import _layers
import _stack
import _util
from _moe import Layer
from _util import P

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def lorc(orc):
    _layers.bind(orc)
    return orc


# ---------------------------------------------------------------- final norm + lm_head argmax
def _final(lib, gen, orc, resid, fnw, q, sz, O, I, gs, eps):
    """The oracle's final step of step_top1 (c/qwen.c:1392, 1463-1474): logits of
    rmsnorm_zc(resid, final_norm) and the host argmax (ties -> lowest index)."""
    xn = np.empty(I, np.float32)
    orc.orc_rmsnorm_zc(P(xn), P(resid), P(fnw), I, np.float32(eps))
    y = np.empty(O, np.float32)
    orc.orc_matmul_q4g_asym(P(y), P(xn), P(q), P(sz), I, O, gs)
    return y, int(orc.orc_argmax(P(y), O))


def test_stream_norm_argmax_cfg1(lib, orc_omp, gen):
    """stream_begin(x) -> final_norm_weight -> stream_norm_argmax over the configs[1]
    lm_head (248320 x 2048, gs 128), then the same with the winning row copied to a lower
    index (forced exact tie: the lower index must win, c/shaders/argmax.comp:7-9)."""
    O, I, gs, eps = 248320, 2048, 128, 1e-6
    q, sz = gen.fmt6(O, I, gs, 0xE1)
    fnw = gen.normal(I, 0xE2, 0.1)
    resid = gen.normal(I, 0xE3, 3.0)
    lib.final_norm_weight(fnw)
    t = lib.tensor(q, sz, 6, I, O, gs)
    lib.stream_begin(resid)
    idx, val = lib.stream_norm_argmax(t, eps)
    lib.stream_end(I, read=False)
    y, io = _final(lib, gen, orc_omp, resid, fnw, q, sz, O, I, gs, eps)
    tol = 2e-4 * float(np.abs(y).max())
    print(f"stream_norm_argmax: device {idx} ({val:.6f}), oracle {io} ({y[io]:.6f})", flush=True)
    assert 0 <= idx < O
    assert abs(val - float(y[idx])) <= tol
    if idx != io:
        assert abs(float(y[idx]) - float(y[io])) <= tol, (idx, io)
    # forced tie: the winning row copied to a lower index
    lo = idx // 2
    rb = I // 2
    q2, sz2 = q.copy(), sz.copy()
    q2[lo * rb:(lo + 1) * rb] = q[idx * rb:(idx + 1) * rb]
    sz2[lo * 32:(lo + 1) * 32] = sz[idx * 32:(idx + 1) * 32]
    t2 = lib.tensor(q2, sz2, 6, I, O, gs)
    lib.stream_begin(resid)
    idx2, val2 = lib.stream_norm_argmax(t2, eps)
    lib.stream_end(I, read=False)
    assert idx2 == lo and val2 == val, (idx2, lo, val2, val)
    if idx == io:   # the oracle's host scan resolves the same tie to the same row
        y2, io2 = _final(lib, gen, orc_omp, resid, fnw, q2, sz2, O, I, gs, eps)
        assert io2 == lo


def test_stream_norm_argmax_ahead(lib, orc_omp, gen):
    """stream_end(NULL) launches the next stream_norm_argmax's work ahead, with the last
    call's arguments (the engine's order, c/qwen.c:1282, 1437-1441).  Tokens in that order
    get the oracle's winners; so do calls with other arguments right after such a launch
    (another tensor, another eps), a token begun again without its argmax, and a call after
    the final norm weight changed."""
    O, I, gs, eps = 65536, 2048, 128, 1e-6
    q, sz = gen.fmt6(O, I, gs, 0xA1)
    q2, sz2 = gen.fmt6(O, I, gs, 0xA2)
    fnw = gen.normal(I, 0xA3, 0.1)
    lib.final_norm_weight(fnw)
    t, t2 = lib.tensor(q, sz, 6, I, O, gs), lib.tensor(q2, sz2, 6, I, O, gs)

    def check(tag, resid, w, tq, tsz, e, idx, val):
        y, io = _final(lib, gen, orc_omp, resid, w, tq, tsz, O, I, gs, e)
        tol = 2e-4 * float(np.abs(y).max())
        print(f"ahead {tag}: device {idx} ({val:.6f}), oracle {io} ({y[io]:.6f})", flush=True)
        assert 0 <= idx < O and abs(val - float(y[idx])) <= tol, tag
        if idx != io:
            assert abs(float(y[idx]) - float(y[io])) <= tol, (tag, idx, io)

    plan = [("first", t, q, sz, eps), ("same", t, q, sz, eps), ("same", t, q, sz, eps),
            ("other tensor", t2, q2, sz2, eps), ("same", t2, q2, sz2, eps), ("other eps", t2, q2, sz2, 1e-5),
            ("back", t, q, sz, eps), ("same", t, q, sz, eps)]
    for k, (tag, tt, tq, tsz, e) in enumerate(plan):
        resid = gen.normal(I, 0xA10 + k, 3.0)
        lib.stream_begin(resid)
        lib.stream_end(I, read=False)
        idx, val = lib.stream_norm_argmax(tt, e)
        check(tag, resid, fnw, tq, tsz, e, idx, val)
    # a token begun again before its argmax: the launch ahead is dropped
    lib.stream_begin(gen.normal(I, 0xA20, 3.0))
    lib.stream_end(I, read=False)
    resid = gen.normal(I, 0xA21, 3.0)
    lib.stream_begin(resid)
    lib.stream_end(I, read=False)
    idx, val = lib.stream_norm_argmax(t, eps)
    check("begun again", resid, fnw, q, sz, eps, idx, val)
    # the final norm weight replaced between stream_end and the argmax
    resid = gen.normal(I, 0xA22, 3.0)
    lib.stream_begin(resid)
    lib.stream_end(I, read=False)
    fnw2 = gen.normal(I, 0xA23, 0.1)
    lib.final_norm_weight(fnw2)
    idx, val = lib.stream_norm_argmax(t, eps)
    check("new norm weight", resid, fnw2, q, sz, eps, idx, val)
    # the residual read back at stream_end: no launch ahead, the call runs as usual
    resid = gen.normal(I, 0xA24, 3.0)
    lib.stream_begin(resid)
    got = lib.stream_end(I, read=True)
    assert np.array_equal(got, resid)
    idx, val = lib.stream_norm_argmax(t, eps)
    check("resid read", resid, fnw2, q, sz, eps, idx, val)
    # the lm_head handle freed after a launch ahead (the library forgets it; the launch read
    # arena memory, which is never reused), then a new handle of other weights
    resid = gen.normal(I, 0xA25, 3.0)
    lib.stream_begin(resid)
    lib.stream_end(I, read=False)
    lib.L.coli_vk_tensor_free(t.handle)
    t.handle = ctypes.c_void_p(None)
    t3 = lib.tensor(q2, sz2, 6, I, O, gs)
    idx, val = lib.stream_norm_argmax(t3, eps)
    check("freed handle", resid, fnw2, q2, sz2, eps, idx, val)


# ---------------------------------------------------------------- int8 router and GDN a/b
SMALL = dict(gqa=dict(H=4, KH=2, hd=64, rot=16, gs=64), gdn=dict(KH=2, KD=64, VH=4, VD=32, K=4, gs=64))


@pytest.fixture(scope="module")
def moe_small(lib, gen):
    return Layer(lib, gen, 0xE400, 256, 128, 32, 64)


def _run_stream(lib, lorc, stack, router, K, T, fused, base, gen, pos0=0, router_f=None):
    """T tokens through the stream (pos0 + t), every layer's route_pipe; the fused path's ids
    come back through stream_ix_hist, the pipe path's through route_pipe (checked on the
    device's own nrm, then the experts go through expert_group_issue_pipe)."""
    D, L = stack.D, stack.moe
    for t in range(T):
        pos = pos0 + t
        x = gen.normal(D, base + t)
        lib.stream_begin(x)
        ref = x.copy()
        ids = []
        for i in range(len(stack.layers)):
            idx, val = stack.pipe_layer(lib, i, pos, K, router)
            assert lib.stream_moe_fused() == fused
            ref, nrm_o, idx_o, val_o = stack.oracle_layer(lorc, i, ref, pos, K)
            if not fused:
                nrm = lib.stream_nrm(D)
                _, i2, v2, _ = L.oracle(lorc, nrm, K, router=router_f)
                assert np.array_equal(idx, i2), (t, i, idx, i2)
                np.testing.assert_allclose(val, v2, rtol=1e-5, atol=1e-7)
                assert _util.maxrel_scaled(nrm, nrm_o) <= TOL
                ex = [L.t[e] for e in idx] + [L.t[L.E]]
                shgt = 1.0 / (1.0 + np.exp(-np.float64(np.dot(L.mw.sh_gate.astype(np.float64), nrm))))
                lib.expert_group_issue_pipe([e[0] for e in ex], [e[1] for e in ex], [e[2] for e in ex],
                                            list(val) + [np.float32(shgt)])
            ids.append(idx_o)
        resid = lib.stream_end(D)
        err = _util.maxrel_scaled(resid, ref)
        print(f"stream pos {pos} ({'fused' if fused else 'pipe'}): resid maxrel_scaled {err:.2e}", flush=True)
        assert err <= TOL, (t, err)
        if fused:
            for i in range(len(stack.layers)):
                assert np.array_equal(lib.stream_ix_hist(stack.first + i, K), ids[i]), (t, i)


@pytest.mark.parametrize("fused", [True, False])
def test_stream_int8_router_and_ab(lib, lorc, gen, moe_small, fused):
    """The formats vk_dense_init uploads (c/qwen.c:1876-1878): router and GDN a/b as fmt 1
    (int8 rows, per-row scale), 3 GDN + 1 GQA layers."""
    L = moe_small
    rt, rf = L.int8_router(lib, gen, 0xE410)
    import _moe
    _moe._active[0] = None
    first = 20 if fused else 40
    if fused:
        lib.eg_table_init(first + 4, L.E, L.D, L.I, L.gs)
        for l in range(first, first + 4):
            L.register(lib, l)
    else:
        lib.eg_table_init(1, L.E, L.D, L.I, L.gs)   # no table slots for layers 40..43
    stack = _stack.Stack(lib, gen, 0xE420 + first, 4, 256, SMALL["gqa"], SMALL["gdn"], L, max_t=16, ab_fmt=1,
                         first_layer=first, router_f=rf, state_base=100)
    assert stack.layers[0]["t"][2].fmt == 1 and stack.layers[0]["t"][3].fmt == 1
    _run_stream(lib, lorc, stack, rt, 8, 3, fused, 0xE480 + first, gen, router_f=rf)
    assert lib.moe_error() == 0


# ---------------------------------------------------------------- configs[3] geometry
@pytest.fixture(scope="module")
def moe_cfg(lib, gen):
    """configs[2]'s layer: router f32 256 x 2048, 256 + 1 experts (gate/up 512 x 2048, down
    2048 x 512, fmt 6 gs 128)."""
    return Layer(lib, gen, 0xE500, 2048, 512, 256, 128)


def test_stream_cfg3_geometry(lib, lorc, gen, moe_cfg):
    """4 layers at configs[3] shapes (GDN KH 16, KD 128, VH 32, VD 128, conv 4, a/b fmt 6:
    the 4-segment in-projection; GQA H 16, KH 2, hd 256, rot 64), the configs[2] MoE fused
    on every layer, decoding at positions 4094 and 4095 of a 4096-row cache seeded with
    4094 random rows."""
    L = moe_cfg
    import _moe
    _moe._active[0] = None
    first = 60
    lib.eg_table_init(first + 4, L.E, L.D, L.I, L.gs)
    for l in range(first, first + 4):
        L.register(lib, l)
    gqa = dict(H=16, KH=2, hd=256, rot=64, gs=128)
    gdn = dict(KH=16, KD=128, VH=32, VD=128, K=4, gs=128)
    stack = _stack.Stack(lib, gen, 0xE510, 4, 2048, gqa, gdn, L, max_t=4096, ab_fmt=6, first_layer=first,
                         kv_rows=4094, state_base=110)
    assert [l["kind"] for l in stack.layers] == ["gdn", "gdn", "gdn", "gqa"]
    _run_stream(lib, lorc, stack, L.router, 8, 2, True, 0xE580, gen, pos0=4094)
    assert lib.moe_error() == 0
    # the attention layer wrote the two new cache rows
    W = stack.layers[3]["W"]
    for h in range(W.KH):
        Kd, Vd = lib.kv_read(stack.layers[3]["idx"], h * 4096 + 4094, 2, W.hd, W.hd)
        cache = stack.layers[3]["cache"]
        Kr = cache[0].reshape(W.KH, 4096, W.hd)[h, 4094:4096]
        Vr = cache[1].reshape(W.KH, 4096, W.hd)[h, 4094:4096]
        assert np.max(np.abs(Kd - Kr)) <= 1e-4 * max(1.0, float(np.abs(Kr).max()))
        assert np.max(np.abs(Vd - Vr)) <= 1e-4 * max(1.0, float(np.abs(Vr).max()))
