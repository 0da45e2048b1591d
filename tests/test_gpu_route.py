"""Routing identity with the CPU reference on engineered near-ties (tests/_neartie.py): router
rows whose exact dots order the experts one way while the reference's sequential fp32 sums
(c/qwen.c:178-189) order them the other way, at ranks 1-2 (order of the picks) and K, K + 1
(which expert is picked).  tests/test_oracle_math.py pins that exact arithmetic picks
differently on these rows, so equal ids here mean the device resolved the near-ties as the
reference does.

- decode: the one-launch MoE block (coli_hip_moe_decode, configs[2]'s router shape);
- stream: a GatedDeltaNet layer's route tail, host-routed (route_pipe returns the ids) and
  fused (the MoE block normalizes the residual itself; ids via stream_ix_hist);
- prefill: coli_hip_moe_prefill over 64 tokens, a quarter of them on the near-tie row.

Bar: ids identical to the oracle's (rank order), weights within 1e-5, block outputs within
maxrel_scaled 1e-3.
"""
import numpy as np
import pytest

import _layers
import _moe
import _neartie
import _stack
import _util
from _moe import Layer

pytestmark = pytest.mark.gpu
D, E, I, GS, K = 2048, 256, 128, 128, 8


@pytest.fixture(scope="module")
def lay(lib, gen):
    """A 256-expert layer at D = 2048 (small I: routing is what is tested)."""
    return Layer(lib, gen, 0xB700, D, I, E, GS)


def _oracle_route(orc, x, W):
    return _neartie.route_ref(orc, _neartie.seq_logits(orc, x, W, E, D), K)


@pytest.mark.parametrize("seed", [0xB711, 0xB712, 0xB713])
def test_neartie_decode_block(lib, orc, gen, torch_dev, lay, seed):
    import torch
    _moe._active[0] = None
    lib.eg_table_init(1, E, D, I, GS)
    lay.register(lib, 0)
    x = gen.normal(D, seed)
    W = _neartie.near_tie_router(orc, gen, x, E, D, K, seed)
    rt = lib.tensor(W, None, 0, D, E)
    dx = torch.from_numpy(x).to(torch_dev)
    out = torch.zeros(D, device=torch_dev)
    di = torch.full((K,), -1, dtype=torch.int32, device=torch_dev)
    dv = torch.zeros(K + 1, device=torch_dev)
    torch.cuda.synchronize()
    lib.moe_decode_dev(0, rt, K, dx.data_ptr(), out.data_ptr(), False, di.data_ptr(), dv.data_ptr())
    lib.sync()
    ri, rv = _oracle_route(orc, x, W)
    idx = di.cpu().numpy()
    print(f"decode near-tie: device {idx.tolist()} reference {ri.tolist()} "
          f"exact {_neartie.exact_rank(x, W, D, K).tolist()}", flush=True)
    assert np.array_equal(idx, ri)
    np.testing.assert_allclose(dv.cpu().numpy()[:K], rv, rtol=1e-5, atol=1e-7)
    ro, oi, _, _ = lay.oracle(orc, x, K, router=W)
    assert np.array_equal(oi, ri)
    assert _util.maxrel_scaled(out.cpu().numpy(), ro) <= 1e-3
    assert lib.moe_error() == 0


def _decode(lib, torch, dev, rt, x):
    dx = torch.from_numpy(x).to(dev)
    out = torch.zeros(D, device=dev)
    di = torch.full((K,), -1, dtype=torch.int32, device=dev)
    dv = torch.zeros(K + 1, device=dev)
    torch.cuda.synchronize()
    lib.moe_decode_dev(0, rt, K, dx.data_ptr(), out.data_ptr(), False, di.data_ptr(), dv.data_ptr())
    lib.sync()
    return out.cpu().numpy(), di.cpu().numpy(), dv.cpu().numpy()


@pytest.mark.parametrize("rfmt", [0, 1])
def test_certify_all_decode_block(lib, orc, gen, torch_dev, lay, rfmt):
    """Every route certified (coli_hip_moe_cert_all): each top-K candidate's logit recomputed
    as the reference's sequential sum (two groups of 16 rows at E = 256) and ranked by it.
    Ids must be the reference's, and the block output, ids and weights bit-identical to the
    default launch (which certifies only ambiguous routes).  f32 router, and an int8 router
    with power-of-two scales, whose reference logits equal the f32 sums of q * s exactly."""
    import torch
    _moe._active[0] = None
    lib.eg_table_init(1, E, D, I, GS)
    lay.register(lib, 0)
    if rfmt == 0:
        W = lay.mw.router
        rt = lay.router
    else:
        rt, W = lay.int8_router(lib, gen, 0xB7A0)
    cases = [gen.normal(D, 0xB7B0 + t) for t in range(4)]
    xt = gen.normal(D, 0xB7C0)   # plus one near-tie row pair
    Wt = _neartie.near_tie_router(orc, gen, xt, E, D, K, 0xB7C1) if rfmt == 0 else None
    prev = lib.moe_cert_all(False)
    try:
        for t, x in enumerate(cases + ([xt] if Wt is not None else [])):
            w, r = (Wt, lib.tensor(Wt, None, 0, D, E)) if t == len(cases) else (W, rt)
            lib.moe_cert_all(False)
            o0, i0, v0 = _decode(lib, torch, torch_dev, r, x)
            lib.moe_cert_all(True)
            o1, i1, v1 = _decode(lib, torch, torch_dev, r, x)
            ri, rv = _oracle_route(orc, x, w)
            assert np.array_equal(i1, ri), (t, i1, ri)
            assert np.array_equal(i0, i1) and np.array_equal(v0, v1) and np.array_equal(o0, o1), t
            np.testing.assert_allclose(v1[:K], rv, rtol=1e-5, atol=1e-7)
    finally:
        lib.moe_cert_all(prev)
    assert lib.moe_error() == 0


@pytest.mark.parametrize("cert_all", [False, True])
def test_neartie_stream(lib, orc, gen, lay, cert_all):
    """One GatedDeltaNet layer (position 0) whose post-attention norm feeds the router.  A
    first host-routed pass reads the device's normed row back; the near-tie router is built
    for that row; the same token then runs host-routed and fused (after gdn_reset).  With
    cert_all every route (host-routed route_row and the fused block) is certified."""
    prev = lib.moe_cert_all(cert_all)
    try:
        _neartie_stream(lib, orc, gen, lay)
    finally:
        lib.moe_cert_all(prev)


def _neartie_stream(lib, orc, gen, lay):
    _layers.bind(orc)
    gdn = dict(KH=2, KD=64, VH=4, VD=32, K=4, gs=128)
    first = 80
    _moe._active[0] = None
    lib.eg_table_init(1, E, D, I, GS)   # no table slots for layer 80 yet: host-routed
    st = _stack.Stack(lib, gen, 0xB720, 1, D, dict(H=4, KH=2, hd=64, rot=16, gs=128), gdn, lay, max_t=16,
                      first_layer=first, state_base=120)
    x = gen.normal(D, 0xB721)
    lib.stream_begin(x)
    st.pipe_layer(lib, 0, 0, K, lay.router)
    nrm = lib.stream_nrm(D)
    lib.stream_end(D, read=False)
    W = _neartie.near_tie_router(orc, gen, nrm, E, D, K, 0xB722)
    rt = lib.tensor(W, None, 0, D, E)
    ri, rv = _oracle_route(orc, nrm, W)
    print(f"stream near-tie: reference {ri.tolist()} exact {_neartie.exact_rank(nrm, W, D, K).tolist()}", flush=True)
    # host-routed: route_pipe returns the device top-k (route_row)
    lib.gdn_reset()
    lib.stream_begin(x)
    idx, val = st.pipe_layer(lib, 0, 0, K, rt)
    assert np.array_equal(lib.stream_nrm(D), nrm)
    lib.stream_end(D, read=False)
    assert np.array_equal(idx, ri), (idx, ri)
    np.testing.assert_allclose(val, rv, rtol=1e-5, atol=1e-7)
    # fused: the MoE block of the expert table normalizes and routes on the device
    lib.eg_table_init(first + 1, E, D, I, GS)
    lay.register(lib, first)
    lib.gdn_reset()
    lib.stream_begin(x)
    st.pipe_layer(lib, 0, 0, K, rt)
    assert lib.stream_moe_fused()
    lib.stream_end(D, read=False)
    assert np.array_equal(lib.stream_ix_hist(first, K), ri)
    assert lib.moe_error() == 0
    _moe._active[0] = None


def test_neartie_prefill(lib, orc, gen, torch_dev, lay):
    """Prefill logits are the reference's bits (sequential fp32 per output), so the picks of
    every token match, near-ties included."""
    import torch
    _moe._active[0] = None
    lib.eg_table_init(1, E, D, I, GS)
    lay.register(lib, 0)
    S = 64
    xstar = gen.normal(D, 0xB731)
    W = _neartie.near_tie_router(orc, gen, xstar, E, D, K, 0xB732)
    xs = gen.normal(S * D, 0xB733).reshape(S, D)
    xs[::4] = xstar
    xs = np.ascontiguousarray(xs.reshape(-1))
    rt = lib.tensor(W, None, 0, D, E)
    dxs = torch.from_numpy(xs).to(torch_dev)
    dout = torch.zeros(S * D, device=torch_dev)
    didx = torch.full((S * K,), -1, dtype=torch.int32, device=torch_dev)
    dval = torch.zeros(S * K, device=torch_dev)
    torch.cuda.synchronize()
    lib.moe_prefill_dev(0, rt, K, dxs.data_ptr(), S, dout.data_ptr(), didx.data_ptr(), dval.data_ptr())
    lib.sync()
    out, tidx, tval = lay.oracle_prefill(orc, xs, S, K, router=W)
    ri, _ = _oracle_route(orc, xstar, W)
    assert np.array_equal(tidx[:K], ri)
    assert np.array_equal(didx.cpu().numpy(), tidx)
    np.testing.assert_allclose(dval.cpu().numpy(), tval, rtol=1e-5, atol=1e-7)
    got = dout.cpu().numpy()
    worst = max(_util.maxrel_scaled(got[t * D:(t + 1) * D], out[t * D:(t + 1) * D]) for t in range(S))
    assert worst <= 1e-3, worst
