"""The configs[3] decode step as bench.py's decode_cfg3 runs it, against the CPU oracle: 40
layers (30 GatedDeltaNet + 10 gated GQA, c/qwen.c:398) at configs[3] shapes, every layer in
its own expert-table slot with the configs[2] MoE fused, each GQA cache seeded with 4094
rows, two tokens at positions 4094 and 4095 through stream_begin -> 40 x *_route_pipe ->
stream_end -> stream_norm_argmax (c/qwen.c:1228-1290, 1392, 1436-1441).  The layers share
one set of 256 + 1 experts and one router (host memory); their attention / GatedDeltaNet
weights, norms, caches and states are all distinct.

Checked per layer, on the device's own residual (copied after every layer with
coli_vk_stream_copy_resid): the routed ids of the fused MoE (stream_ix_hist) equal the
oracle's route of that layer on the same input, and the layer's output residual is within
maxrel_scaled 1e-3 of the oracle's layer applied to the device's input.  The final id of
stream_norm_argmax is the oracle's argmax of the device's final residual, or a row whose
logit is within the lm_head tolerance of it.  The oracle's own 40-layer composition (no
re-synchronisation) is run beside it: its drift from the device is reported and, while its
routes agree with the device's, bounded.
"""
import copy

import numpy as np
import pytest

import _layers
import _moe
import _stack
import _util
from _moe import Layer
from _util import P

pytestmark = pytest.mark.gpu
TOL = 1e-3
NL, D, K, MAX_T, POS0 = 40, 2048, 8, 4096, 4094
GQA = dict(H=16, KH=2, hd=256, rot=64, gs=128)
GDN = dict(KH=16, KD=128, VH=32, VD=128, K=4, gs=128)


@pytest.fixture(scope="module")
def lorc(orc_omp):
    _layers.bind(orc_omp)
    return orc_omp


def _oracle_states(stack):
    return [copy.deepcopy(l.get("cache", l.get("state"))) for l in stack.layers]


def _swap_states(stack, states):
    old = []
    for l, s in zip(stack.layers, states):
        key = "cache" if l["kind"] == "gqa" else "state"
        old.append(l[key])
        l[key] = s
    return old


def test_decode_40_layers(lib, lorc, gen):
    L = Layer(lib, gen, 0xD400, D, 512, 256, 128)
    _moe._active[0] = None
    lib.eg_table_init(NL, L.E, L.D, L.I, L.gs)
    for l in range(NL):
        L.register(lib, l)
    stack = _stack.Stack(lib, gen, 0xD410, NL, D, GQA, GDN, L, max_t=MAX_T, ab_fmt=6, first_layer=0,
                         kv_rows=POS0, state_base=60)
    kinds = [l["kind"] for l in stack.layers]
    assert kinds.count("gdn") == 30 and kinds.count("gqa") == 10
    O, gs, eps = 248320, 128, float(stack.eps)
    q, sz = gen.fmt6(O, D, gs, 0xD4F0)
    lm = lib.tensor(q, sz, 6, D, O, gs)
    fnw = gen.normal(D, 0xD4F1, 0.1)
    lib.final_norm_weight(fnw)
    free = _oracle_states(stack)   # the oracle's own chain, never re-synchronised
    for t in range(2):
        pos = POS0 + t
        x = gen.normal(D, 0xD4E0 + t)
        lib.stream_begin(x)
        r_dev, r_free, worst, flips = x.copy(), x.copy(), 0.0, 0
        ids_o, ids_free = [], []
        for i in range(NL):
            stack.pipe_layer(lib, i, pos, K, L.router)
            assert lib.stream_moe_fused()
            r_o, _, idx_o, _ = stack.oracle_layer(lorc, i, r_dev, pos, K)
            ids_o.append(idx_o)
            r_next = lib.stream_copy_resid(D)
            err = _util.maxrel_scaled(r_next, r_o)
            worst = max(worst, err)
            assert err <= TOL, (t, i, err)
            old = _swap_states(stack, free)
            try:
                r_free, _, idx_f, _ = stack.oracle_layer(lorc, i, r_free, pos, K)
            finally:
                free = _swap_states(stack, old)
            ids_free.append(idx_f)
            r_dev = r_next
        final = lib.stream_end(D)
        assert np.array_equal(final, r_dev)
        idx, val = lib.stream_norm_argmax(lm, eps)
        for i in range(NL):
            got = lib.stream_ix_hist(i, K)
            assert np.array_equal(got, ids_o[i]), (t, i, got, ids_o[i])
            flips += int(not np.array_equal(got, ids_free[i]))
        xn = np.empty(D, np.float32)
        lorc.orc_rmsnorm_zc(P(xn), P(final), P(fnw), D, np.float32(eps))
        y = np.empty(O, np.float32)
        lorc.orc_matmul_q4g_asym(P(y), P(xn), P(q), P(sz), D, O, gs)
        io = int(lorc.orc_argmax(P(y), O))
        tol = 2e-4 * float(np.abs(y).max())
        drift = _util.maxrel_scaled(final, r_free)
        print(f"decode40 pos {pos}: worst layer maxrel_scaled {worst:.2e}; argmax device {idx} oracle {io}; "
              f"oracle-chain drift {drift:.2e} ({flips} layers routed differently)", flush=True)
        assert abs(val - float(y[idx])) <= tol
        assert idx == io or abs(float(y[idx]) - float(y[io])) <= tol, (idx, io)
        if flips == 0:
            assert drift <= 1e-2, drift
    assert lib.moe_error() == 0
