"""coli_hip_moe_decode_noalloc (the MoE block with its cross-block words in a static device
array, no allocation) against coli_hip_moe_decode on the same inputs, and against the CPU
oracle (c/qwen.c:804-928): two calls in a row, the second with a smaller input (fewer
routed experts, so fewer tag words), then a geometry whose tag words exceed the static
array, which the no-alloc entry point must refuse while the allocating one runs it.

Bar: routed ids and weights identical to the allocating entry point's (same kernel), outputs
bit-identical; ids identical to the oracle's and outputs within maxrel_scaled 1e-3.
"""
import numpy as np
import pytest

import _moe
import _util
from _moe import Layer

pytestmark = pytest.mark.gpu


def _both(lib, torch, dev, L, layer, K, x):
    dx = torch.from_numpy(x).to(dev)
    outs = []
    for fn in ("alloc", "noalloc"):
        out = torch.full((L.D,), float("nan"), device=dev)
        idx = torch.full((K,), -1, dtype=torch.int32, device=dev)
        val = torch.zeros(K + 1, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        if fn == "alloc":
            lib.moe_decode_dev(layer, L.router, K, dx.data_ptr(), out.data_ptr(), False, idx.data_ptr(),
                               val.data_ptr())
        else:
            assert lib.moe_decode_noalloc_dev(layer, L.router, K, dx.data_ptr(), out.data_ptr(), False,
                                              idx.data_ptr(), val.data_ptr()) == 1
        lib.sync()
        outs.append((out.cpu().numpy(), idx.cpu().numpy(), val.cpu().numpy()))
    return outs


def test_noalloc_matches_alloc(lib, orc, gen, torch_dev):
    import torch
    L = Layer(lib, gen, 0xAA00, 2048, 512, 256, 128)
    _moe._active[0] = None
    lib.eg_table_init(1, L.E, L.D, L.I, L.gs)
    L.register(lib, 0)
    for n, K in enumerate((8, 4)):   # the second call uses fewer tag words
        x = gen.normal(L.D, 0xAA10 + n)
        (oa, ia, va), (on, i_n, vn) = _both(lib, torch, torch_dev, L, 0, K, x)
        ro, ri, rv, rsh = L.oracle(orc, x, K)
        print(f"call {n} (K={K}): ids {i_n.tolist()}, maxrel_scaled vs oracle {_util.maxrel_scaled(on, ro):.2e}",
              flush=True)
        assert np.array_equal(i_n, ia) and np.array_equal(vn, va)
        assert np.array_equal(on, oa)
        assert np.array_equal(i_n, ri)
        np.testing.assert_allclose(vn[:K], rv, rtol=1e-5, atol=1e-7)
        assert _util.maxrel_scaled(on, ro) <= 1e-3
    assert lib.moe_error() == 0


def test_noalloc_refuses_beyond_static_scratch(lib, orc, gen, torch_dev):
    """D = 4096, K = 8: 27 + 128 + 9 * (512 + 4096) = 41627 tag words > the 32736 the static
    array holds: refused (0); the allocating entry point still runs the block."""
    import torch
    L = Layer(lib, gen, 0xAB00, 4096, 512, 8, 128)
    _moe._active[0] = None
    lib.eg_table_init(1, L.E, L.D, L.I, L.gs)
    L.register(lib, 0)
    x = gen.normal(L.D, 0xAB10)
    dx = torch.from_numpy(x).to(torch_dev)
    out = torch.zeros(L.D, device=torch_dev)
    torch.cuda.synchronize()
    assert lib.moe_decode_noalloc_dev(0, L.router, 8, dx.data_ptr(), out.data_ptr()) == 0
    lib.moe_decode_dev(0, L.router, 8, dx.data_ptr(), out.data_ptr())
    lib.sync()
    ro, _, _, _ = L.oracle(orc, x, 8)
    assert _util.maxrel_scaled(out.cpu().numpy(), ro) <= 1e-3
    # a smaller K fits again: 27 + 128 + 3 * 4608 = 13979 words
    on = torch.zeros(L.D, device=torch_dev)
    assert lib.moe_decode_noalloc_dev(0, L.router, 2, dx.data_ptr(), on.data_ptr()) == 1
    lib.moe_decode_dev(0, L.router, 2, dx.data_ptr(), out.data_ptr())
    lib.sync()
    assert np.array_equal(on.cpu().numpy(), out.cpu().numpy())
    assert lib.moe_error() == 0
    _moe._active[0] = None
