"""The fused GatedDeltaNet layer kernel (in-projection -> recurrence -> out-projection in one
launch, tiles handing over tagged words) against the three separate launches, on the
engine's stream path at configs[3] geometry (c/qwen.c:1228-1290, the layer as
c/backend_vulkan.c:1905-2017 records it).

The fused kernel runs the same device code in the same order per output, so the residual
after every token, the conv rings and recurrent states must be identical bit for bit; the
oracle comparison of the same stream is tests/test_gpu_stream.py::test_stream_cfg3_geometry
(the separate launches, the default)."""
import numpy as np
import pytest

import _layers
import _moe
import _stack
from _moe import Layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lorc(orc):
    _layers.bind(orc)
    return orc


def _run(lib, stack, router, K, xs, pos0):
    """Tokens through the stream; the residual after each and every GDN layer's state."""
    lib.gdn_reset()
    res = []
    for t, x in enumerate(xs):
        lib.stream_begin(x)
        for i in range(len(stack.layers)):
            stack.pipe_layer(lib, i, pos0 + t, K, router)
        res.append(lib.stream_end(stack.D))
    states = []
    for L in stack.layers:
        if L["kind"] == "gdn":
            W = L["W"]
            states.append(lib.gdn_state_read(L["idx"], W.K, W.CD, W.VH, W.KD, W.VD))
    return res, states


def test_fused_gdn_layer_matches_separate_launches(lib, lorc, gen):
    D, I, E, gs, K = 2048, 512, 256, 128, 8
    L = Layer(lib, gen, 0xF100, D, I, E, gs)
    _moe._active[0] = None
    first = 70
    lib.eg_table_init(first + 4, E, D, I, gs)
    for l in range(first, first + 4):
        L.register(lib, l)
    gqa = dict(H=16, KH=2, hd=256, rot=64, gs=128)
    gdn = dict(KH=16, KD=128, VH=32, VD=128, K=4, gs=128)
    stack = _stack.Stack(lib, gen, 0xF110, 4, D, gqa, gdn, L, max_t=64, ab_fmt=6, first_layer=first, state_base=130)
    xs = [gen.normal(D, 0xF120 + t) for t in range(5)]   # more tokens than conv taps: the ring wraps
    prev = lib.layer_fuse(False)
    try:
        sep, sep_st = _run(lib, stack, L.router, K, xs, 0)
        lib.layer_fuse(True)
        fus, fus_st = _run(lib, stack, L.router, K, xs, 0)
    finally:
        lib.layer_fuse(prev)
    for t in range(len(xs)):
        assert np.array_equal(sep[t], fus[t]), (t, float(np.max(np.abs(sep[t] - fus[t]))))
    for (r0, s0), (r1, s1) in zip(sep_st, fus_st):
        assert np.array_equal(r0, r1) and np.array_equal(s0, s1)
    assert lib.moe_error() == 0
    _moe._active[0] = None
