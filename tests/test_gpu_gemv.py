"""GPU parity of the fmt=6 GEMV (c/qwen.c:211-229), fmt 1/0 GEMVs and the fused device
argmax / top-k (c/shaders/argmax.comp, c/qwen.c:1471-1472) against the CPU oracle.

Tolerance: fp32 accumulation, max relative error <= 1e-3 with the
reference's own metric (|ref| floored at 1e-2, c/backend_vulkan.c:4462), and a normwise
relative error <= 1e-5.  Selections (argmax / top-k) are exact on the GPU's own outputs
and agree with the oracle's except where two candidates lie within the GEMV tolerance.
"""
import numpy as np
import pytest

from _util import P, brute_fmt6, maxrel, normrel

pytestmark = pytest.mark.gpu

TOL_MAXREL = 1e-3
TOL_NORM = 1e-5


def _oracle_gemv(orc, q, sz, x, I, O, gs):
    y = np.empty(O, np.float32)
    orc.orc_matmul_q4g_asym(P(y), P(x), P(q), P(sz), I, O, gs)
    return y


def test_cfg0_matmul(lib, orc, gen):
    """Config 0: W 4096 x 2048, gs 128, x ~ N(0,1)."""
    O, I, gs = 4096, 2048, 128
    q, sz = gen.fmt6(O, I, gs, 0xC0)
    x = gen.normal(I, gen.stream(0xC0, 7))
    t = lib.tensor(q, sz, 6, I, O, gs)
    y = lib.matmul(t, x)
    yo = _oracle_gemv(orc, q, sz, x, I, O, gs)
    yb = brute_fmt6(q, sz, x, I, O, gs)
    print(f"cfg0 maxrel vs oracle {maxrel(y, yo):.2e}, vs f64 {maxrel(y, yb):.2e} "
          f"(oracle vs f64 {maxrel(yo, yb):.2e})")
    assert maxrel(y, yo) <= TOL_MAXREL
    assert normrel(y, yo) <= TOL_NORM
    # the HIP path is at least as close to the exact value as the fp32 CPU oracle, up to 2x
    assert normrel(y, yb) <= 2 * normrel(yo, yb) + 1e-7


@pytest.mark.parametrize("O,I,gs", [
    (1, 32, 32), (7, 256, 128), (64, 512, 128), (33, 2048, 64), (5, 4096, 128),
    (3, 6144, 128), (2, 8192, 256), (16, 250, 32), (9, 129, 32),          # fast path
    (7, 1024, 256), (5, 960, 96), (3, 2048, 512), (4, 4096, 4096),        # fast path, group max by LDS atomics
    (9, 8200, 128), (17, 100, 8), (8, 264, 24), (4, 2048, 16), (6, 520, 40),  # generic path
])
def test_fmt6_shapes(lib, orc, gen, O, I, gs):
    q, sz = gen.fmt6(O, I, gs, 1000 + O * 7 + I)
    x = gen.normal(I, gen.stream(I, O))
    t = lib.tensor(q, sz, 6, I, O, gs)
    y = lib.matmul(t, x)
    yo = _oracle_gemv(orc, q, sz, x, I, O, gs)
    assert maxrel(y, yo) <= TOL_MAXREL, (O, I, gs)
    assert normrel(y, yo) <= TOL_NORM


def test_fmt6_real_valued_zero(lib, orc, gen):
    """Startup RTN quantization gives non-integer zero points (c/qwen.c:246-265)."""
    O, I, gs = 256, 2048, 128
    W = gen.normal(O * I, 77, 0.05)
    q = np.empty(O * I // 2, np.uint8)
    sz = np.empty(O * (I // gs) * 2, np.float32)
    orc.orc_quant_rows(P(W), I, O, 6, gs, P(q), P(sz))
    assert np.any(sz[1::2] != np.round(sz[1::2]))
    x = gen.normal(I, 78)
    y = lib.matmul(lib.tensor(q, sz, 6, I, O, gs), x)
    yo = _oracle_gemv(orc, q, sz, x, I, O, gs)
    assert maxrel(y, yo) <= TOL_MAXREL


def test_fmt6_wide_dynamic_range(lib, orc, gen):
    """x groups spanning very different magnitudes (block exponents per group)."""
    O, I, gs = 128, 2048, 128
    q, sz = gen.fmt6(O, I, gs, 91)
    x = gen.normal(I, 92)
    x *= np.repeat(np.float32(10.0) ** np.arange(-8, 8, dtype=np.float32), gs)[:I]
    x[5] = 0.0
    x[gs:2 * gs] = 0.0           # an all-zero group
    y = lib.matmul(lib.tensor(q, sz, 6, I, O, gs), x)
    yo = _oracle_gemv(orc, q, sz, x, I, O, gs)
    yb = brute_fmt6(q, sz, x, I, O, gs)
    assert normrel(y, yb) <= 1e-5
    assert normrel(y, yo) <= 1e-5


def test_multirow_S(lib, orc, gen):
    O, I, gs, S = 300, 1024, 128, 3
    q, sz = gen.fmt6(O, I, gs, 5)
    x = gen.normal(S * I, 6)
    y = lib.matmul(lib.tensor(q, sz, 6, I, O, gs), x, S=S).reshape(S, O)
    for s in range(S):
        yo = _oracle_gemv(orc, q, sz, x[s * I:(s + 1) * I].copy(), I, O, gs)
        assert maxrel(y[s], yo) <= TOL_MAXREL


def test_fmt1_router(lib, orc, gen):
    """int8 per-row router / GDN a,b as the engine uploads them (c/qwen.c:1876-1878)."""
    O, I = 256, 2048
    W = gen.normal(O * I, 11, 0.02)
    q = np.empty(O * I, np.uint8)
    s = np.empty(O, np.float32)
    orc.orc_quant_rows(P(W), I, O, 1, 0, P(q), P(s))
    x = gen.normal(I, 12)
    y = lib.matmul(lib.tensor(q, s, 1, I, O, 0), x)
    yo = np.empty(O, np.float32)
    orc.orc_matmul_q8(P(yo), P(x), P(q), P(s), I, O)
    assert maxrel(y, yo) <= TOL_MAXREL


def test_fmt0_router(lib, orc, gen):
    O, I = 256, 2048
    W = gen.normal(O * I, 13, 0.02)
    x = gen.normal(I, 14)
    y = lib.matmul(lib.tensor(W, None, 0, I, O, 0), x)
    yo = np.empty(O, np.float32)
    orc.orc_matmul_f32(P(yo), P(x), P(W), 1, I, O)
    assert maxrel(y, yo) <= TOL_MAXREL
    assert normrel(y, yo) <= TOL_NORM


def _int8_rows(orc, gen, O, I, seed):
    W = gen.normal(O * I, seed, 0.02)
    q = np.empty(O * I, np.uint8)
    s = np.empty(O, np.float32)
    orc.orc_quant_rows(P(W), I, O, 1, 0, P(q), P(s))
    return q, s


@pytest.mark.parametrize("fmt,O,I,S", [(1, 256, 2048, 512), (1, 32, 2048, 37), (0, 256, 2048, 5), (0, 100, 132, 2),
                                       (1, 17, 260, 3)])
def test_rows_f01(lib, orc, gen, fmt, O, I, S):
    """fmt 1 / fmt 0 rows over S >= 2 rows of x (the engine's router and GDN a/b over the
    prefill rows, c/qwen.c:1189,1359): one launch, the reference's sequential fp32 sums
    (c/qwen.c:178-189, 230-238) bit for bit."""
    x = gen.normal(S * I, 0x3100 + S)
    if fmt == 1:
        q, s = _int8_rows(orc, gen, O, I, 0x3101)
        t = lib.tensor(q, s, 1, I, O, 0)
    else:
        W = gen.normal(O * I, 0x3102, 0.02)
        t = lib.tensor(W, None, 0, I, O, 0)
    y = lib.matmul(t, x, S).reshape(S, O)
    for r in range(S):
        yo = np.empty(O, np.float32)
        xr = np.ascontiguousarray(x[r * I:(r + 1) * I])
        if fmt == 1:
            orc.orc_matmul_q8(P(yo), P(xr), P(q), P(s), I, O)
        else:
            orc.orc_matmul_f32(P(yo), P(xr), P(W), 1, I, O)
        assert np.array_equal(y[r], yo), (r, maxrel(y[r], yo))


def test_rows_f01_pair(lib, orc, gen):
    """GatedDeltaNet b and a over S rows as one coli_vk_matmul_pair (c/qwen.c:1359), fmt 1."""
    S, I, VH = 37, 2048, 32
    qb, sb = _int8_rows(orc, gen, VH, I, 0x3201)
    qa, sa = _int8_rows(orc, gen, VH, I, 0x3202)
    tb, ta = lib.tensor(qb, sb, 1, I, VH, 0), lib.tensor(qa, sa, 1, I, VH, 0)
    x = gen.normal(S * I, 0x3203)
    yb, ya = lib.matmul_pair(tb, ta, x, S)
    for r in range(S):
        xr = np.ascontiguousarray(x[r * I:(r + 1) * I])
        for y, q, s in ((yb, qb, sb), (ya, qa, sa)):
            yo = np.empty(VH, np.float32)
            orc.orc_matmul_q8(P(yo), P(xr), P(q), P(s), I, VH)
            assert np.array_equal(y.reshape(S, VH)[r], yo), r


def test_matmul_pair(lib, orc, gen):
    I, gs = 2048, 128
    q1, s1 = gen.fmt6(512, I, gs, 21)
    q2, s2 = gen.fmt6(1000, I, gs, 22)
    x = gen.normal(I, 23)
    t1, t2 = lib.tensor(q1, s1, 6, I, 512, gs), lib.tensor(q2, s2, 6, I, 1000, gs)
    y1, y2 = lib.matmul_pair(t1, t2, x)
    assert maxrel(y1, _oracle_gemv(orc, q1, s1, x, I, 512, gs)) <= TOL_MAXREL
    assert maxrel(y2, _oracle_gemv(orc, q2, s2, x, I, 1000, gs)) <= TOL_MAXREL


def test_tensor_ensure_semantics(lib, gen):
    """An existing handle only re-checks (fmt, I, O) (c/backend_vulkan.c:1057); gs not a
    multiple of 8 is refused (:1058-1059)."""
    q, sz = gen.fmt6(8, 256, 32, 31)
    t = lib.tensor(q, sz, 6, 256, 8, 32)
    L = lib.L
    assert L.coli_vk_tensor_ensure(t.ref, None, None, 6, 256, 8, 32) == 1
    assert L.coli_vk_tensor_ensure(t.ref, None, None, 6, 256, 9, 32) == 0
    from ctypes import byref, c_void_p
    h = c_void_p(None)
    assert L.coli_vk_tensor_ensure(byref(h), P(q), P(sz), 6, 256, 8, 12) == 0
    # the weight bytes only, as the reference (c/backend_vulkan.c:4137 returns wbytes)
    assert t.nbytes() == 8 * t.info()["row_bytes"] and t.info()["row_bytes"] >= 128


def _lmhead(lib, gen, O, seed, dup_rows=()):
    I, gs = 2048, 128
    q, sz = gen.fmt6(O, I, gs, seed)
    rb = I // 2
    for a, b in dup_rows:          # forced exact ties: row b := row a
        q[b * rb:(b + 1) * rb] = q[a * rb:(a + 1) * rb]
        sz[b * 32:(b + 1) * 32] = sz[a * 32:(a + 1) * 32]
    x = gen.normal(I, gen.stream(seed, 9))
    return q, sz, x, lib.tensor(q, sz, 6, I, O, gs)


@pytest.mark.parametrize("k", [1, 8])
def test_lmhead_topk(lib, orc_omp, gen, torch_dev, k):
    """Config 1: lm_head 248320 x 2048 GEMV + device top-k over the logits."""
    import torch
    O, I = 248320, 2048
    q, sz, x, t = _lmhead(lib, gen, O, 0xC1)
    dx = torch.from_numpy(x).to(torch_dev)
    dy = torch.empty(O, dtype=torch.float32, device=torch_dev)
    di = torch.empty(8, dtype=torch.int32, device=torch_dev)
    dv = torch.empty(8, dtype=torch.float32, device=torch_dev)
    torch.cuda.synchronize()
    lib.gemv_topk_dev(t, dx.data_ptr(), dy.data_ptr(), k, di.data_ptr(), dv.data_ptr())
    lib.sync()
    y = dy.cpu().numpy()
    idx, val = di.cpu().numpy()[:k], dv.cpu().numpy()[:k]
    # exact selection on the GPU's own outputs
    oi = np.empty(8, np.int32)
    ov = np.empty(8, np.float32)
    orc_omp.orc_topk_logits(P(y), O, k, P(oi), P(ov))
    assert np.array_equal(idx, oi[:k]) and np.array_equal(val, ov[:k])
    # against the oracle's logits
    yo = _oracle_gemv(orc_omp, q, sz, x, I, O, 128)
    assert maxrel(y, yo) <= TOL_MAXREL
    orc_omp.orc_topk_logits(P(yo), O, k, P(oi), P(ov))
    tol = 2e-4 * float(np.abs(yo).max())
    for r in range(k):
        if idx[r] != oi[r]:
            assert abs(float(yo[idx[r]]) - float(ov[r])) <= tol, (r, idx, oi[:k])


def test_argmax_ties(lib, orc, gen):
    """Duplicate maxima resolve to the lowest index (c/shaders/argmax.comp:7-9), the
    reference's run_argmax_case methodology (c/backend_vulkan.c:4480-4517)."""
    O = 20000
    q, sz, x, t = _lmhead(lib, gen, O, 0xA1)
    y = lib.matmul(t, x)
    best = int(np.argmax(y))
    # copy the winning row to a lower and a higher index: the lower must win
    lo, hi = max(best // 2, 0), min(best + 977, O - 1)
    if lo == best:
        lo = best + 1 if best + 1 < O else best - 1
    q2, sz2, x2, t2 = _lmhead(lib, gen, O, 0xA1, dup_rows=[(best, lo), (best, hi)])
    y2 = lib.matmul(t2, x2)
    assert y2[lo] == y2[best] == y2[hi]
    idx, val = lib.matmul_argmax(t2, x2)
    assert idx == min(lo, best) and val == y2[best]
    assert idx == orc.orc_argmax(P(y2), O)


def test_topk_ties(lib, orc, gen, torch_dev):
    import torch
    O = 5000
    q, sz, x, t = _lmhead(lib, gen, O, 0xA2)
    y = lib.matmul(t, x)
    top = np.argsort(-y, kind="stable")[:3]
    dups = [(int(top[0]), 4999), (int(top[0]), 0), (int(top[1]), 17)]
    q2, sz2, x2, t2 = _lmhead(lib, gen, O, 0xA2, dup_rows=dups)
    dx = torch.from_numpy(x2).to(torch_dev)
    di = torch.empty(8, dtype=torch.int32, device=torch_dev)
    dv = torch.empty(8, dtype=torch.float32, device=torch_dev)
    dy = torch.empty(O, dtype=torch.float32, device=torch_dev)
    torch.cuda.synchronize()
    lib.gemv_topk_dev(t2, dx.data_ptr(), dy.data_ptr(), 8, di.data_ptr(), dv.data_ptr())
    lib.sync()
    y2 = dy.cpu().numpy()
    oi = np.empty(8, np.int32)
    ov = np.empty(8, np.float32)
    orc.orc_topk_logits(P(y2), O, 8, P(oi), P(ov))
    assert np.array_equal(di.cpu().numpy(), oi)
    assert np.array_equal(dv.cpu().numpy(), ov)
    assert oi[0] == 0  # the duplicated maximum sits at row 0 now


def device_layout(q, O, I, gs):
    """Host rows -> the library's fmt-6 device bytes (kLayoutLanes in csrc/internal.h:
    lane j holds host chunks 2j, 2j+1 at chunk slots c*nl + j; bytes XOR 0x88)."""
    rb = (I + 1) // 2
    nch = (rb + 15) // 16
    nl = (nch + 1) // 2
    pad = np.zeros((O, nl * 2 * 16), np.uint8)
    pad[:, :rb] = q.reshape(O, rb)
    ch = pad.reshape(O, nl, 2, 16).transpose(0, 2, 1, 3)
    return (ch.reshape(O, -1) ^ 0x88).reshape(-1)


def test_device_synth_matches_host(lib, gen):
    """coli_hip_tensor_synth == host generator + upload (bytes exact, scales exact)."""
    O, I, gs, seed = 777, 2048, 128, 0x5EED
    t = lib.tensor_synth(6, I, O, gs, seed, 0.02)
    info = t.info()
    w = np.empty(O * info["row_bytes"], np.uint8)
    s = np.empty(O * (I // gs) * 2, np.float32)
    lib.memcpy(w.ctypes.data, info["d_w"], w.nbytes)
    lib.memcpy(s.ctypes.data, info["d_sz"], s.nbytes)
    q, sz = gen.fmt6(O, I, gs, seed)
    assert np.array_equal(w, device_layout(q, O, I, gs))
    assert np.array_equal(s, sz)
    # the upload path lays out the same bytes
    tu = lib.tensor(q, sz, 6, I, O, gs)
    wu = np.empty_like(w)
    lib.memcpy(wu.ctypes.data, tu.info()["d_w"], wu.nbytes)
    assert np.array_equal(wu, w)
    # odd I: partial last chunk / lane
    O2, I2 = 5, 129
    q2, s2 = gen.fmt6(O2, I2, 32, 3)
    t2 = lib.tensor(q2, s2, 6, I2, O2, 32)
    w2 = np.empty(O2 * t2.info()["row_bytes"], np.uint8)
    lib.memcpy(w2.ctypes.data, t2.info()["d_w"], w2.nbytes)
    assert np.array_equal(w2, device_layout(q2, O2, I2, 32))
    # f32 rows (router)
    tr = lib.tensor_synth(0, I, 64, 0, seed, 0.02)
    inf = tr.info()
    r = np.empty(64 * inf["row_bytes"] // 4, np.float32)
    lib.memcpy(r.ctypes.data, inf["d_w"], r.nbytes)
    assert np.array_equal(r.reshape(64, -1)[:, :I].reshape(-1), gen.f32rows(64, I, seed, 0.02))


def test_topk_fused_many_launches(lib, orc, torch_dev):
    """300 fused top-8 launches in a row (the 8-bit launch tag wraps), new x each time:
    every result equals the exact selection over that launch's logits."""
    import torch
    O, I = 3000, 2048
    t = lib.tensor_synth(6, I, O, 128, 0x70F, 0.02)
    dx = torch.empty(I, dtype=torch.float32, device=torch_dev)
    dy = torch.empty(O, dtype=torch.float32, device=torch_dev)
    di = torch.empty(8, dtype=torch.int32, device=torch_dev)
    dv = torch.empty(8, dtype=torch.float32, device=torch_dev)
    oi = np.empty(8, np.int32)
    ov = np.empty(8, np.float32)
    for n in range(300):
        lib.synth_normal_dev(dx.data_ptr(), I, 1000 + n, 1.0)
        k = 1 + n % 8
        lib.gemv_topk_dev(t, dx.data_ptr(), dy.data_ptr(), k, di.data_ptr(), dv.data_ptr())
        lib.sync()
        y = dy.cpu().numpy()
        orc.orc_topk_logits(P(y), O, k, P(oi), P(ov))
        assert np.array_equal(di.cpu().numpy()[:k], oi[:k]), n
        assert np.array_equal(dv.cpu().numpy()[:k], ov[:k]), n


def test_topk_unfused_shape(lib, orc, torch_dev):
    """A shape whose rows per wave exceed the fused merge (O=300000, I=256): GEMV then a
    separate top-k pass; same exact selection."""
    import torch
    O, I = 300000, 256
    t = lib.tensor_synth(6, I, O, 64, 0x7A1, 0.02)
    dx = torch.empty(I, dtype=torch.float32, device=torch_dev)
    dy = torch.empty(O, dtype=torch.float32, device=torch_dev)
    di = torch.empty(8, dtype=torch.int32, device=torch_dev)
    dv = torch.empty(8, dtype=torch.float32, device=torch_dev)
    lib.synth_normal_dev(dx.data_ptr(), I, 5, 1.0)
    lib.gemv_topk_dev(t, dx.data_ptr(), dy.data_ptr(), 8, di.data_ptr(), dv.data_ptr())
    lib.sync()
    y = dy.cpu().numpy()
    oi = np.empty(8, np.int32)
    ov = np.empty(8, np.float32)
    orc.orc_topk_logits(P(y), O, 8, P(oi), P(ov))
    assert np.array_equal(di.cpu().numpy(), oi) and np.array_equal(dv.cpu().numpy(), ov)
