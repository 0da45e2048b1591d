"""MoE block on the GPU vs the CPU oracle (c/qwen.c:804-928 restated in oracle/oracle.c).

* coli_hip_moe_decode (one launch: router -> softmax/top-K -> K routed + shared expert ->
  weighted combine over the coli_vk_eg_table_* expert table): routed expert ids
  identical to the oracle's, in the same rank order; renormed weights and the shared
  gate within 1e-5; the block output within maxrel 1e-3 (fp32-accumulation tolerance).
* coli_vk_expert_group / _issue / _take / _issue_id and coli_vk_gate_up (host-routed
  drop-in path) vs the oracle's expert MLP.
Shapes: a small layer and the config-2 layer (D=2048, I=512, E=256, K=8, gs=128).
"""
import numpy as np
import pytest

import _util
from _moe import Layer, Table
from _util import P, eptr

pytestmark = pytest.mark.gpu

TOL = 1e-3


def run_moe(lib, torch, dev, layer, L, K, x, accumulate=False, resid=None, router=None):
    dx = torch.from_numpy(x).to(dev)
    dout = torch.from_numpy(resid.copy()).to(dev) if resid is not None else torch.full((L.D,), np.nan, device=dev)
    didx = torch.full((K,), -1, dtype=torch.int32, device=dev)
    dval = torch.zeros(K + 1, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    lib.moe_decode_dev(layer, L.router if router is None else router, K, dx.data_ptr(), dout.data_ptr(), accumulate, didx.data_ptr(),
                       dval.data_ptr())
    lib.sync()
    return dout.cpu().numpy(), didx.cpu().numpy(), dval.cpu().numpy()


@pytest.fixture(scope="module")
def small(lib, gen):
    """Two layers of a small MoE in one table (layer 1 has different weights)."""
    D, I, E, gs = 256, 128, 32, 64
    return Table(lib, [Layer(lib, gen, 0x5EED, D, I, E, gs, layer=l) for l in range(2)])


def moe_f64(L, x, idx, val, shgt):
    """The block in float64 from the format definition (brute-force dequant), on the
    oracle's routing: an accuracy yardstick for both the oracle and the GPU."""
    x = x.astype(np.float64)
    out = np.zeros(L.D)
    for e, w in list(zip(idx, val)) + [(L.E, shgt)]:
        (gq, gsz), (uq, usz), (dq, dsz) = L.mw.exp[e]
        g = _util.brute_fmt6(gq, gsz, x, L.D, L.I, L.gs)
        u = _util.brute_fmt6(uq, usz, x, L.D, L.I, L.gs)
        h = g / (1 + np.exp(-g)) * u
        out += float(w) * _util.brute_fmt6(dq, dsz, h, L.I, L.D, L.gs)
    return out


def check(orc, L, K, x, got, tol=TOL, f64=False, router=None):
    out, idx, val, shgt = L.oracle(orc, x, K, router)
    gout, gidx, gval = got
    assert np.array_equal(gidx, idx), (gidx, idx)
    np.testing.assert_allclose(gval[:K], val, rtol=1e-5, atol=1e-7)
    assert abs(gval[K] - shgt) <= 1e-6 * max(1.0, abs(shgt))
    err = _util.maxrel_scaled(gout, out)
    assert err <= tol, err
    if f64:
        ex = moe_f64(L, x, idx, val, shgt)
        e_gpu, e_orc = _util.normrel(gout, ex), _util.normrel(out, ex)
        print(f"  maxrel_scaled vs oracle {err:.2e}; normrel vs f64: gpu {e_gpu:.2e} oracle {e_orc:.2e}", flush=True)
        assert e_gpu <= 1e-5
    return out


@pytest.mark.parametrize("K", [1, 4, 8])
def test_moe_small(lib, orc, gen, torch_dev, small, K):
    import torch

    small.activate()
    for t in range(6):
        layer = t % 2
        x = gen.normal(small[0].D, 0x100 + t)
        got = run_moe(lib, torch, torch_dev, layer, small[layer], K, x)
        print(f"small K={K} token {t} layer {layer}: ids {got[1].tolist()}", flush=True)
        check(orc, small[layer], K, x, got)
    assert lib.moe_error() == 0


@pytest.mark.parametrize("D,I,E,gs", [(320, 192, 40, 64), (448, 384, 24, 64)])
def test_moe_odd_geometry(lib, orc, gen, torch_dev, D, I, E, gs):
    """Row widths that are not a power of two of lanes (D = 320 or 448: 5 or 7 lanes of a
    gate/up row; I = 192 or 384: 3 or 6 lanes of a down row), so the tiles carry padding
    lanes, against the oracle."""
    import torch

    L = Layer(lib, gen, 0x0DD0 + D, D, I, E, gs)
    Table(lib, [L]).activate()
    for K in (3, 8):
        for t in range(3):
            x = gen.normal(D, 0x0DE0 + 16 * K + t)
            check(orc, L, K, x, run_moe(lib, torch, torch_dev, 0, L, K, x))
    assert lib.moe_error() == 0


def test_moe_accumulate(lib, orc, gen, torch_dev, small):
    """accumulate=1: out = resid + moe (the residual-stream form)."""
    import torch

    L, K = small.activate()[1], 8
    x = gen.normal(L.D, 0x200)
    resid = gen.normal(L.D, 0x201)
    got = run_moe(lib, torch, torch_dev, 1, L, K, x, accumulate=True, resid=resid)
    out, idx, _, _ = L.oracle(orc, x, K)
    assert np.array_equal(got[1], idx)
    ref = resid + out
    assert _util.maxrel_scaled(got[0], ref) <= TOL
    assert lib.moe_error() == 0


def test_moe_back_to_back(lib, orc, gen, torch_dev, small):
    """Consecutive launches without a host sync between them (launch epochs)."""
    import torch

    L, K, n = small.activate()[0], 4, 5
    xs = [gen.normal(L.D, 0x300 + t) for t in range(n)]
    dx = [torch.from_numpy(x).to(torch_dev) for x in xs]
    dout = [torch.zeros(L.D, device=torch_dev) for _ in range(n)]
    didx = [torch.zeros(K, dtype=torch.int32, device=torch_dev) for _ in range(n)]
    torch.cuda.synchronize()
    for t in range(n):
        lib.moe_decode_dev(0, L.router, K, dx[t].data_ptr(), dout[t].data_ptr(), False, didx[t].data_ptr(), None)
    lib.sync()
    for t in range(n):
        out, idx, _, _ = L.oracle(orc, xs[t], K)
        assert np.array_equal(didx[t].cpu().numpy(), idx)
        assert _util.maxrel_scaled(dout[t].cpu().numpy(), out) <= TOL
    assert lib.moe_error() == 0


def test_moe_router_ties(lib, orc, gen, torch_dev):
    """Duplicate router rows give equal probabilities: the lower expert id ranks first
    (c/qwen.c:812 strict '>' from the lowest index)."""
    import torch

    D, I, E, gs, K = 256, 128, 32, 64, 8
    L = Layer(lib, gen, 0x7E5, D, I, E, gs)
    r = L.mw.router.reshape(E, D)
    for a, b in [(3, 17), (5, 6), (30, 2)]:
        r[b] = r[a]
    L.router = lib.tensor(L.mw.router, None, 0, D, E)
    Table(lib, [L]).activate()
    for t in range(8):
        x = gen.normal(D, 0x400 + t)
        got = run_moe(lib, torch, torch_dev, 0, L, K, x)
        check(orc, L, K, x, got)
    assert lib.moe_error() == 0


@pytest.mark.parametrize("K", [4, 8])
def test_moe_router_int8(lib, orc, gen, torch_dev, small, K):
    """fmt 1 router (int8 rows, per-row scale applied after the dot, c/qwen.c:230-238), the
    format the reference uploads for the router when it quantises to int8."""
    import torch
    L = small.activate()[0]
    rt, rf = L.int8_router(lib, gen, 0x1A8)
    for t in range(6):
        x = gen.normal(L.D, 0x1A9 + t)
        check(orc, L, K, x, run_moe(lib, torch, torch_dev, 0, L, K, x, router=rt), router=rf)
    assert lib.moe_error() == 0


@pytest.fixture(scope="module")
def cfg2(lib, gen):
    """The config-2 layer: router f32 256x2048, 256 + 1 experts of gate/up 512x2048 and
    down 2048x512, fmt 6 gs 128, all resident."""
    D, I, E, gs = 2048, 512, 256, 128
    return Table(lib, [Layer(lib, gen, 0xC0F2, D, I, E, gs)])


def test_moe_cfg2(lib, orc, gen, torch_dev, cfg2):
    import torch

    K = 8
    L = cfg2.activate()[0]
    seen = set()
    for t in range(12):
        x = gen.normal(L.D, 0x500 + t)
        got = run_moe(lib, torch, torch_dev, 0, L, K, x)
        print(f"cfg2 token {t}: ids {got[1].tolist()}", flush=True)
        check(orc, L, K, x, got, f64=t < 3)
        seen.update(got[1].tolist())
    assert len(seen) > 24   # the routed experts change from token to token
    assert lib.moe_error() == 0


def test_expert_group_cfg2(lib, orc, gen, cfg2):
    """coli_vk_expert_group: packed rows of several experts (c/backend_vulkan.c:1418-1697)."""
    L = cfg2[0]
    eids = [7, 255, 256, 0]
    rows = [1, 2, 1, 3]
    n = sum(rows)
    x = gen.normal(n * L.D, 0x600)
    y = lib.expert_group([L.t[e][0] for e in eids], [L.t[e][1] for e in eids], [L.t[e][2] for e in eids], rows, x)
    p = 0
    for e, r in zip(eids, rows):
        for _ in range(r):
            ref = np.empty(L.D, np.float32)
            orc.orc_expert_mlp_fmt6(eptr(L.ex, e), P(x[p * L.D:(p + 1) * L.D].copy()), L.D, L.I, L.gs, P(ref))
            assert _util.maxrel_scaled(y[p * L.D:(p + 1) * L.D], ref) <= TOL
            p += 1
    # issue/take: one group in flight; a second issue is refused until take
    assert lib.expert_group_issue([L.t[3][0]], [L.t[3][1]], [L.t[3][2]], [1], x[:L.D])
    assert not lib.expert_group_issue([L.t[3][0]], [L.t[3][1]], [L.t[3][2]], [1], x[:L.D])
    y1 = lib.expert_group_take(1, L.D)
    ref = np.empty(L.D, np.float32)
    orc.orc_expert_mlp_fmt6(eptr(L.ex, 3), P(x[:L.D].copy()), L.D, L.I, L.gs, P(ref))
    assert _util.maxrel_scaled(y1, ref) <= TOL


def test_expert_group_issue_id(lib, orc, gen, cfg2):
    """Prefill form: rows named by token id from bound xs (c/backend_vulkan.c:1656-1670)."""
    L, S = cfg2[0], 6
    xs = gen.normal(S * L.D, 0x700)
    lib.eg_xs_bind(xs, S, L.D)
    eids, rows, tok = [12, 40], [3, 2], [5, 0, 2, 2, 4]
    assert lib.expert_group_issue_id([L.t[e][0] for e in eids], [L.t[e][1] for e in eids],
                                     [L.t[e][2] for e in eids], rows, tok)
    y = lib.expert_group_take(len(tok), L.D)
    p = 0
    for e, r in zip(eids, rows):
        for _ in range(r):
            ref = np.empty(L.D, np.float32)
            xr = xs[tok[p] * L.D:(tok[p] + 1) * L.D].copy()
            orc.orc_expert_mlp_fmt6(eptr(L.ex, e), P(xr), L.D, L.I, L.gs, P(ref))
            assert _util.maxrel_scaled(y[p * L.D:(p + 1) * L.D], ref) <= TOL
            p += 1


def test_gate_up(lib, orc, gen, cfg2):
    """coli_vk_gate_up: hidden = silu(gate x) * up x for S rows."""
    L, S = cfg2[0], 3
    g, u, _ = L.t[9]
    x = gen.normal(S * L.D, 0x800)
    h = lib.gate_up(g, u, x, S)
    (gq, gsz), (uq, usz), _ = L.mw.exp[9]
    for s in range(S):
        xr = x[s * L.D:(s + 1) * L.D].copy()
        gv = np.empty(L.I, np.float32)
        uv = np.empty(L.I, np.float32)
        orc.orc_matmul_q4g_asym(P(gv), P(xr), P(gq), P(gsz), L.D, L.I, L.gs)
        orc.orc_matmul_q4g_asym(P(uv), P(xr), P(uq), P(usz), L.D, L.I, L.gs)
        ref = gv / (1 + np.exp(-gv.astype(np.float64))) * uv
        assert _util.maxrel_scaled(h[s * L.I:(s + 1) * L.I], ref) <= TOL
