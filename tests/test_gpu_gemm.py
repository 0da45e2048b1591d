"""Prefill on MFMA outside the MoE block, against the CPU oracle:

- the dense fmt6 GEMM that coli_vk_matmul / coli_vk_matmul_pair run for S >= 4 rows of x
  (the reference switches to qmatmul_mm at S >= 4, c/backend_vulkan.c:282-299,
  c/shaders/qmatmul_mm.comp), at shapes that exercise partial row blocks, one-row passes,
  a row count that is not a multiple of 4, a single group (I = 128) and I = 4096;
- coli_vk_gdn_full_seq with S >= 4 (c/backend_vulkan.c:2018-2157): qkv and z of a chunk
  in one GEMM, the recurrence of the chunk in one launch, the gated norm and out-projection
  in one more GEMM; outputs per token, conv ring and recurrent state against the oracle's
  token-by-token run, across two calls, a chunk boundary, and a decode token afterwards.

Bar: the reference's own VK_TEST bar against the f64 dequantised product (relative error
<= 1e-3 wherever |ref| > 1e-2, c/backend_vulkan.c:4462-4474), and every row within
maxrel_scaled 1e-3 of the oracle's matmul_q4g_asym (an fp32 computation whose own rounding,
~1e-5 absolute at I = 2048, is what a fixed 1e-2 floor would grade); GDN outputs within
maxrel_scaled 1e-3, ring within 1e-5 and state within 1e-4 relative to their magnitude.
"""
import numpy as np
import pytest

import _layers
import _util
from _util import P, maxrel_scaled

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _oracle_rows(orc, q, sz, x, S, I, O, gs):
    y = np.empty((S, O), np.float32)
    for s in range(S):
        xs = np.ascontiguousarray(x[s * I:(s + 1) * I])
        orc.orc_matmul_q4g_asym(P(y[s]), P(xs), P(q), P(sz), I, O, gs)
    return y


def vk_test_maxrel(got, ref):
    """c/backend_vulkan.c:4462-4474: max |got - ref| / |ref| over the elements |ref| > 1e-2."""
    got, ref = np.asarray(got, np.float64).ravel(), np.asarray(ref, np.float64).ravel()
    m = np.abs(ref) > 1e-2
    return float(np.max(np.abs(got[m] - ref[m]) / np.abs(ref[m]))) if m.any() else 0.0


def _check(y, q, sz, x, S, I, O, gs, yo, tag):
    y64 = _f64_rows(q, sz, x, S, I, O, gs)
    vk = vk_test_maxrel(y, y64)
    sc = max(maxrel_scaled(y[s], yo[s]) for s in range(S))
    print(f"{tag}: VK_TEST maxrel vs f64 {vk:.2e}, worst row maxrel_scaled vs oracle {sc:.2e}", flush=True)
    assert vk <= TOL and sc <= TOL


def _f64_rows(q, sz, x, S, I, O, gs):
    """Dequantised product in float64: w = (nibble - zero) * scale, element j in the low
    (j even) or high nibble of byte j / 2 (c/tools/convert_qwen35_moe.py:124-144)."""
    b = q.reshape(O, I // 2)
    nib = np.empty((O, I), np.float64)
    nib[:, 0::2] = b & 15
    nib[:, 1::2] = b >> 4
    s = sz.reshape(O, I // gs, 2).astype(np.float64)
    w = (nib.reshape(O, I // gs, gs) - s[:, :, 1:2]) * s[:, :, 0:1]
    return x.reshape(S, I).astype(np.float64) @ w.reshape(O, I).T


@pytest.mark.parametrize("O,I,S", [(4096, 2048, 4), (1000, 2048, 33), (8192, 2048, 64), (2048, 4096, 48),
                                   (130, 128, 17), (12, 256, 5), (512, 2048, 600), (20000, 2048, 8)])
def test_gemm_rows(lib, orc_omp, gen, O, I, S):
    gs = 128
    q, sz = gen.fmt6(O, I, gs, 0x6E00 + O + S)
    x = gen.normal(S * I, 0x6E01 + I)
    y = lib.matmul(lib.tensor(q, sz, 6, I, O, gs), x, S=S).reshape(S, O)
    yo = _oracle_rows(orc_omp, q, sz, x, S, I, O, gs)
    _check(y, q, sz, x, S, I, O, gs, yo, f"gemm O={O} I={I} S={S}")


def test_gemm_wide_range_rows(lib, orc_omp, gen):
    """Rows of x whose groups span many binades (each group scaled by 2^k, k in -20..20):
    the per-(row, group) exponent of the digit decomposition follows each group."""
    O, I, S, gs = 512, 2048, 12, 128
    q, sz = gen.fmt6(O, I, gs, 0x6E10)
    x = gen.normal(S * I, 0x6E11).reshape(S, I // gs, gs)
    k = np.random.default_rng(0x6E12).integers(-20, 21, size=(S, I // gs, 1))
    x = np.ascontiguousarray((x * np.exp2(k)).astype(np.float32).reshape(-1))
    y = lib.matmul(lib.tensor(q, sz, 6, I, O, gs), x, S=S).reshape(S, O)
    y64 = _f64_rows(q, sz, x, S, I, O, gs)
    for s in range(S):
        err = np.max(np.abs(y[s] - y64[s])) / max(1e-30, np.max(np.abs(y64[s])))
        assert err <= 1e-4, (s, err)


def test_gemm_pair_rows(lib, orc_omp, gen):
    """matmul_pair at S = 40: one digit decomposition of x serves both tensors."""
    I, gs, S = 2048, 128, 40
    q1, s1 = gen.fmt6(512, I, gs, 0x6E20)
    q2, s2 = gen.fmt6(1000, I, gs, 0x6E21)
    x = gen.normal(S * I, 0x6E22)
    t1, t2 = lib.tensor(q1, s1, 6, I, 512, gs), lib.tensor(q2, s2, 6, I, 1000, gs)
    y1, y2 = lib.matmul_pair(t1, t2, x, S=S)
    r1 = _oracle_rows(orc_omp, q1, s1, x, S, I, 512, gs)
    r2 = _oracle_rows(orc_omp, q2, s2, x, S, I, 1000, gs)
    _check(y1.reshape(S, 512), q1, s1, x, S, I, 512, gs, r1, "pair 1")
    _check(y2.reshape(S, 1000), q2, s2, x, S, I, 1000, gs, r2, "pair 2")


def test_gemm_other_group_size_rows(lib, orc_omp, gen):
    """gs 64 is not the GEMM's: S rows still run, one GEMV launch per row."""
    O, I, gs, S = 300, 1024, 64, 9
    q, sz = gen.fmt6(O, I, gs, 0x6E30)
    x = gen.normal(S * I, 0x6E31)
    y = lib.matmul(lib.tensor(q, sz, 6, I, O, gs), x, S=S).reshape(S, O)
    yo = _oracle_rows(orc_omp, q, sz, x, S, I, O, gs)
    _check(y, q, sz, x, S, I, O, gs, yo, "gs 64")


# ---------------------------------------------------------------- GDN prefill
@pytest.fixture(scope="module")
def lorc(orc_omp):
    _layers.bind(orc_omp)
    return orc_omp


def _gdn_run(lib, lorc, gen, W, ts, layer, st, calls, K):
    """calls: token counts of consecutive coli_vk_gdn_full_seq calls; every token's output
    against the oracle's token-by-token run on the same state."""
    D = W.D
    t = 0
    for n in calls:
        xs = [gen.normal(D, 0x6F10 + t + i) for i in range(n)]
        ps = [_layers.gdn_host_params(lorc, W, x) for x in xs]
        y = lib.gdn_full_seq(layer, np.concatenate(xs), np.concatenate(ps), *ts, n, W.KH, W.KD, W.VH, W.VD, W.CD, K,
                             W.eps)
        worst = 0.0
        for i in range(n):
            ref = W.oracle(lorc, st, xs[i])
            worst = max(worst, _util.maxrel_scaled(y[i * W.out.O:(i + 1) * W.out.O], ref))
        print(f"gdn seq call of {n} tokens (from token {t}): worst maxrel_scaled {worst:.2e}", flush=True)
        assert worst <= TOL, (t, n, worst)
        t += n


def _rel_to_max(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(1e-30, float(np.max(np.abs(ref)))))


@pytest.fixture(params=["chunked", "token loop"])
def gdn_path(request, lib):
    """The prefill recurrence: closed form per 64-token chunk (the default) or the
    token-by-token loop (the fallback for shapes the chunked kernels do not take)."""
    prev = lib.gdn_chunked(request.param == "chunked")
    yield request.param
    lib.gdn_chunked(prev)


def test_gdn_seq_cfg3(lib, lorc, gen, gdn_path):
    """configs[3] GatedDeltaNet geometry (KH 16, KD 128, VH 32, VD 128, conv 4, gs 128):
    40 tokens in one call, 6 in a second, then one decode token (S = 1, the per-token
    kernels) on the ring and state the chunks left."""
    D, KH, KD, VH, VD, K, gs, layer = 2048, 16, 128, 32, 128, 4, 128, 9
    W = _layers.GdnWeights(gen, gen.stream(0x6F00, layer), D, KH, KD, VH, VD, K, gs)
    ts = tuple(m.upload(lib) for m in (W.qkv, W.z, W.out))
    lib.gdn_setup(layer, VH, KD, VD, K, W.CD, W.conv)
    lib.gdn_reset()
    st = W.new_state()
    _gdn_run(lib, lorc, gen, W, ts, layer, st, [40, 6, 1], K)
    ring, S = lib.gdn_state_read(layer, K, W.CD, VH, KD, VD)
    assert _rel_to_max(ring, st[0]) < 1e-5
    assert _rel_to_max(S, st[1]) < 1e-4


def test_gdn_seq_chunks(lib, lorc, gen, gdn_path):
    """A small layer (D 256, KH 2, KD 64, VH 4, VD 32, gs 128) over 1030 tokens: two input
    pieces (1024 + 6) in one call, the ring carried across the piece boundary; the chunked
    recurrence takes 16 full 64-token chunks and a 6-token one."""
    D, KH, KD, VH, VD, K, gs, layer = 256, 2, 64, 4, 32, 4, 128, 10
    W = _layers.GdnWeights(gen, gen.stream(0x6F80, layer), D, KH, KD, VH, VD, K, gs)
    ts = tuple(m.upload(lib) for m in (W.qkv, W.z, W.out))
    lib.gdn_setup(layer, VH, KD, VD, K, W.CD, W.conv)
    lib.gdn_reset()
    st = W.new_state()
    _gdn_run(lib, lorc, gen, W, ts, layer, st, [1030, 5], K)
    ring, S = lib.gdn_state_read(layer, K, W.CD, VH, KD, VD)
    assert _rel_to_max(ring, st[0]) < 1e-5
    assert _rel_to_max(S, st[1]) < 1e-4
