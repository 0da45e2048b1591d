"""Prefill MoE block on the GPU (coli_hip_moe_prefill) vs the CPU oracle's restatement of
moe_batch_from_logits (c/qwen.c:1050-1183), which is bit-identical to the compiled
reference on the committed fixture tests/golden/moe_batch_small.npz.

Per token: routed expert ids identical to the oracle's (rank order), renormed weights
within 1e-5, output within maxrel 1e-3 (floor scaled to the output magnitude, see
_util.maxrel_scaled).  The expert projections run as grouped GEMMs on MFMA with exact
integer group sums, so fp32-accumulation tolerance applies.
"""
import numpy as np
import pytest

import _util
from _moe import Layer, Table

pytestmark = pytest.mark.gpu

TOL = 1e-3


def run_prefill(lib, torch, dev, L, K, xs, S, router=None):
    dxs = torch.from_numpy(xs).to(dev)
    dout = torch.full((S * L.D,), np.nan, device=dev)
    didx = torch.full((S * K,), -1, dtype=torch.int32, device=dev)
    dval = torch.zeros(S * K, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    lib.moe_prefill_dev(0, L.router if router is None else router, K, dxs.data_ptr(), S, dout.data_ptr(), didx.data_ptr(), dval.data_ptr())
    lib.sync()
    return dout.cpu().numpy(), didx.cpu().numpy(), dval.cpu().numpy()


def check(orc, L, K, xs, S, got, router=None):
    out, tidx, tval = L.oracle_prefill(orc, xs, S, K, router)
    gout, gidx, gval = got
    assert np.array_equal(gidx, tidx), np.nonzero(gidx != tidx)[0][:10]
    np.testing.assert_allclose(gval, tval, rtol=1e-5, atol=1e-7)
    worst = max(_util.maxrel_scaled(gout[t * L.D:(t + 1) * L.D], out[t * L.D:(t + 1) * L.D]) for t in range(S))
    print(f"  S={S}: worst per-token maxrel_scaled {worst:.2e}", flush=True)
    assert worst <= TOL, worst


@pytest.mark.parametrize("S,K", [(1, 4), (37, 4), (64, 8), (200, 8)])
def test_prefill_small(lib, orc, gen, torch_dev, S, K):
    import torch
    L = Layer(lib, gen, 0x9F1, 256, 128, 32, 128)
    Table(lib, [L]).activate()
    xs = gen.normal(S * L.D, 0x9F2 + S)
    check(orc, L, K, xs, S, run_prefill(lib, torch, torch_dev, L, K, xs, S))


@pytest.mark.parametrize("S,K", [(37, 6), (130, 8)])
def test_prefill_odd_geometry(lib, orc, gen, torch_dev, S, K):
    """Hidden and intermediate sizes of 3 groups (D = I = 384): supersteps of 4 groups with
    one missing, and a token count that leaves partial 16- and 32-row tiles."""
    import torch
    L = Layer(lib, gen, 0x9F8, 384, 384, 24, 128)
    Table(lib, [L]).activate()
    xs = gen.normal(S * L.D, 0x9F9 + S)
    check(orc, L, K, xs, S, run_prefill(lib, torch, torch_dev, L, K, xs, S))


@pytest.mark.parametrize("S", [1, 64, 200])
def test_prefill_router_int8(lib, orc, gen, torch_dev, S):
    """fmt 1 router: int8 rows, the per-row scale applied after the dot (c/qwen.c:230-238)."""
    import torch
    L = Layer(lib, gen, 0x9F1, 256, 128, 32, 128)
    Table(lib, [L]).activate()
    rt, rf = L.int8_router(lib, gen, 0x9F3)
    xs = gen.normal(S * L.D, 0x9F4 + S)
    check(orc, L, 8, xs, S, run_prefill(lib, torch, torch_dev, L, 8, xs, S, router=rt), router=rf)


@pytest.fixture(scope="module")
def cfg4(lib, gen):
    """configs[4]'s layer: router f32 256x2048, 256 + 1 experts (gate/up 512x2048, down
    2048x512, fmt 6 gs 128)."""
    return Table(lib, [Layer(lib, gen, 0xC0F4, 2048, 512, 256, 128)])


@pytest.mark.parametrize("S", [128, 512])
def test_prefill_cfg4(lib, orc_omp, gen, torch_dev, cfg4, S):
    """configs[4] at its full M = 512 tokens (and at 128): experts get up to ~30 rows, so the
    two-x-tile gate/up body runs at D = 2048."""
    import torch
    L, K = cfg4.activate()[0], 8
    xs = gen.normal(S * L.D, 0xC0F5)
    got = run_prefill(lib, torch, torch_dev, L, K, xs, S)
    check(orc_omp, L, K, xs, S, got)
    counts = np.bincount(got[1], minlength=L.E)
    print(f"  rows per expert: max {counts.max()}, empty experts {(counts == 0).sum()}", flush=True)
    assert counts.max() > 8 and (counts == 0).sum() < L.E   # ragged groups
    if S == 512:
        assert counts.max() > 16   # an expert with more than one 16-row x tile


def test_prefill_cfg4_router_int8(lib, orc_omp, gen, torch_dev, cfg4):
    """configs[4] shape with an int8 (fmt 1) router: the split-K router pass over int8 rows."""
    import torch
    L, K, S = cfg4.activate()[0], 8, 64
    rt, rf = L.int8_router(lib, gen, 0xC0F6)
    xs = gen.normal(S * L.D, 0xC0F7)
    check(orc_omp, L, K, xs, S, run_prefill(lib, torch, torch_dev, L, K, xs, S, router=rt), router=rf)


# ---------------------------------------------------------------- the engine's prefill calls
# The unchanged engine runs prefill MoE through the host-routed expert group
# (c/qwen.c:1094-1161): chunks of <= 64 experts and <= 1024 rows over the bound rows, then
# the shared expert over all S rows.  Groups with more than one row per expert run as the
# grouped MFMA GEMMs (the reference's multi-row kernels, c/backend_vulkan.c:1462-1466).

def _rows_check(orc, L, eids, rows, xrows, y):
    p, worst = 0, 0.0
    for e, r in zip(eids, rows):
        for _ in range(r):
            ref = np.empty(L.D, np.float32)
            orc.orc_expert_mlp_fmt6(_util.eptr(L.ex, e), _util.P(xrows[p].copy()), L.D, L.I, L.gs, _util.P(ref))
            worst = max(worst, _util.maxrel_scaled(y[p * L.D:(p + 1) * L.D], ref))
            p += 1
    return worst


def test_expert_group_rows_mfma(lib, orc_omp, gen, cfg4):
    """Packed rows, 1 to 40 per expert (units of 32 and 16 rows, a single-row expert in the
    group): MFMA path against the oracle per row, and the GEMV items (forced) likewise."""
    L = cfg4[0]
    eids, rows = [3, 256, 100, 7, 200, 255], [2, 40, 17, 1, 33, 16]
    n = sum(rows)
    x = gen.normal(n * L.D, 0xE900)
    xr = x.reshape(n, L.D)
    g, u, d = ([L.t[e][i] for e in eids] for i in range(3))
    y = lib.expert_group(g, u, d, rows, x)
    w_mfma = _rows_check(orc_omp, L, eids, rows, xr, y)
    prev = lib.eg_force_gemv(True)
    try:
        y2 = lib.expert_group(g, u, d, rows, x)
    finally:
        lib.eg_force_gemv(prev)
    w_gemv = _rows_check(orc_omp, L, eids, rows, xr, y2)
    print(f"  rows {rows}: worst maxrel_scaled mfma {w_mfma:.2e}, gemv {w_gemv:.2e}", flush=True)
    assert w_mfma <= TOL and w_gemv <= TOL


@pytest.mark.parametrize("S", [64, 512])
def test_engine_moe_batch_cfg4(lib, orc_omp, gen, cfg4, S):
    """configs[4]'s layer through the engine's own call sequence (_engine.engine_moe_batch):
    per token within 1e-3 of the oracle's moe_batch_from_logits.  At S = 512 the 4096 pairs
    need several chunks and at least one expert is split across two chunks (c/qwen.c:1104)."""
    import _engine
    L, K = cfg4[0], 8
    xs = gen.normal(S * L.D, 0xE910 + S)
    out, tidx, tval = L.oracle_prefill(orc_omp, xs, S, K)
    ecnt, _ = _engine.group_by_expert(tidx, L.E)
    chs = _engine.chunks(ecnt, L.E)
    got = _engine.engine_moe_batch(lib, L.t, xs, S, L.D, K, tidx, tval, L.mw.sh_gate)
    ref = out.reshape(S, L.D)
    worst = max(_util.maxrel_scaled(got[t], ref[t]) for t in range(S))
    split = sum(1 for a, b in zip(chs, chs[1:]) if a[-1][0] == b[0][0])
    print(f"  S={S}: {len(chs)} chunks, {split} split experts, worst per-token maxrel_scaled {worst:.2e}", flush=True)
    assert worst <= TOL
    if S == 512:
        assert len(chs) >= 4 and split >= 1


def test_engine_moe_batch_rebind(lib, orc_omp, gen, cfg4):
    """Two prefill layers' worth of calls in a row on rows of the same shape: the second
    bind's rows are the ones used (the digit planes of the bound rows are not stale)."""
    import _engine
    L, K, S = cfg4[0], 8, 96
    for seed in (0xE920, 0xE921):
        xs = gen.normal(S * L.D, seed)
        out, tidx, tval = L.oracle_prefill(orc_omp, xs, S, K)
        got = _engine.engine_moe_batch(lib, L.t, xs, S, L.D, K, tidx, tval, L.mw.sh_gate)
        ref = out.reshape(S, L.D)
        worst = max(_util.maxrel_scaled(got[t], ref[t]) for t in range(S))
        assert worst <= TOL, (seed, worst)
