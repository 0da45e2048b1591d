"""The oracle's attention (GQA) and GatedDeltaNet blocks against the compiled reference
and against the mathematics.

* Golden: tests/golden/layer_{gqa,gdn}_{small,cfg3}.npz hold outputs of the reference's own
  attention() / gdn_step() (c/qwen.c:581-667, :669-776, compiled unmodified) over a
  sequence of tokens from a zeroed cache / state; the oracle must reproduce them bit for
  bit, together with the final caches and states.
* Brute force: a float64 restatement in matrix form (numpy, independent of the C loops:
  projections dequantized from the format definition, RoPE as a 2x2 rotation of the
  (j, j + rot/2) pairs, attention as softmax(K q / sqrt(hd)) V, the delta rule as
  S' = d S + beta k (v - d S^T k)^T) agrees within fp32 accumulation error.
* Closed forms: RoPE at position 0 is the identity and preserves pair norms; at position 0
  attention is exactly the value row (softmax over one key).
"""
import hashlib
import os

import numpy as np
import pytest

import _layers
import _util


@pytest.fixture(scope="module")
def lorc(orc):
    _layers.bind(orc)
    return orc


def load(name):
    return np.load(os.path.join(_util.GOLDEN, name + ".npz"), allow_pickle=False)


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def gqa_from(f, gen):
    g = lambda k: int(f[k])  # noqa: E731
    return _layers.GqaWeights(gen, g("base"), g("D"), g("H"), g("KH"), g("hd"), g("rot"), g("gs"))


def gdn_from(f, gen):
    g = lambda k: int(f[k])  # noqa: E731
    return _layers.GdnWeights(gen, g("base"), g("D"), g("KH"), g("KD"), g("VH"), g("VD"), g("K"), g("gs"))


@pytest.mark.parametrize("name", ["small", "cfg3"])
def test_gqa_golden(lorc, gen, name):
    f = load(f"layer_gqa_{name}")
    W = gqa_from(f, gen)
    D, T, max_t = int(f["D"]), int(f["T"]), int(f["max_t"])
    xs = gen.normal(T * D, gen.stream(int(f["base"]), 50))
    assert digest(W.q.q, W.o.sz, W.qn, W.kn, xs) == str(f["digest"])
    cache = W.new_cache(max_t)
    for t in range(T):
        y = W.oracle(lorc, cache, max_t, t, xs[t * D:(t + 1) * D].copy())
        assert np.array_equal(bits(y), bits(f["out"][t])), t
    if "K" in f:
        assert np.array_equal(bits(cache[0]), bits(f["K"])) and np.array_equal(bits(cache[1]), bits(f["V"]))


@pytest.mark.parametrize("name", ["small", "cfg3"])
def test_gdn_golden(lorc, gen, name):
    f = load(f"layer_gdn_{name}")
    W = gdn_from(f, gen)
    D, T = int(f["D"]), int(f["T"])
    xs = gen.normal(T * D, gen.stream(int(f["base"]), 50))
    assert digest(W.qkv.q, W.out.sz, W.a.w, W.conv, xs) == str(f["digest"])
    st = W.new_state()
    for t in range(T):
        y = W.oracle(lorc, st, xs[t * D:(t + 1) * D].copy())
        assert np.array_equal(bits(y), bits(f["out"][t])), t
    if "S" in f:
        assert np.array_equal(bits(st[0]), bits(f["conv"])) and np.array_equal(bits(st[1]), bits(f["S"]))
    else:
        assert digest(st[0], st[1]) == str(f["state_digest"])


# ---------------------------------------------------------------- float64 restatements
def proj64(m, x):
    if m.fmt == 6:
        return _util.brute_fmt6(m.q, m.sz, x, m.I, m.O, m.gs)
    return m.w.reshape(m.O, m.I).astype(np.float64) @ np.asarray(x, np.float64)


def rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * (1.0 + w.astype(np.float64))


def rope64(x, pos, rot, theta):
    x = np.array(x, np.float64)
    hr = rot // 2
    ang = pos * float(theta) ** (-2.0 * np.arange(hr) / rot)
    lo, hi = x[..., :hr].copy(), x[..., hr:rot].copy()
    x[..., :hr] = lo * np.cos(ang) - hi * np.sin(ang)
    x[..., hr:rot] = hi * np.cos(ang) + lo * np.sin(ang)
    return x


def gqa64(W, Ks, Vs, pos, x):
    """One token; Ks/Vs lists [KH] of f64 key/value rows so far (appended in place)."""
    H, KH, hd = W.H, W.KH, W.hd
    qg = proj64(W.q, x).reshape(H, 2, hd)
    q, gate = qg[:, 0], qg[:, 1]
    k = proj64(W.k, x).reshape(KH, hd)
    v = proj64(W.v, x).reshape(KH, hd)
    q = rope64(rms64(q, W.qn, W.eps), pos, W.rot, W.theta)
    k = rope64(rms64(k, W.kn, W.eps), pos, W.rot, W.theta)
    for h in range(KH):
        Ks[h].append(k[h])
        Vs[h].append(v[h])
    ctx = np.empty((H, hd))
    for h in range(H):
        kv = h // (H // KH)
        Kh, Vh = np.array(Ks[kv]), np.array(Vs[kv])
        s = Kh @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        ctx[h] = (p / p.sum()) @ Vh / (1.0 + np.exp(-gate[h]))
    return proj64(W.o, ctx.reshape(-1))


def gdn64(W, conv, S, x):
    """One token; conv: list of the last K-1 inputs (f64), S: [VH, KD, VD] f64 (updated)."""
    KH, KD, VH, VD, K = W.KH, W.KD, W.VH, W.VD, W.K
    qkv = proj64(W.qkv, x)
    z = proj64(W.z, x).reshape(VH, VD)
    win = np.array(conv[-(K - 1):] + [qkv]) if K > 1 else qkv[None]
    cw = W.conv.reshape(-1, K).astype(np.float64)
    c = np.sum(cw.T * win, axis=0)
    cv = c / (1.0 + np.exp(-c))
    conv.append(qkv)
    q = cv[:KH * KD].reshape(KH, KD)
    k = cv[KH * KD:2 * KH * KD].reshape(KH, KD)
    v = cv[2 * KH * KD:].reshape(VH, VD)
    q = q / np.sqrt(np.sum(q * q, axis=1, keepdims=True) + W.eps) / np.sqrt(KD)
    k = k / np.sqrt(np.sum(k * k, axis=1, keepdims=True) + W.eps)
    a, b = proj64(W.a, x), proj64(W.b, x)
    sp = np.where(a + W.dtb > 20, a + W.dtb, np.log1p(np.exp(a + W.dtb)))
    decay = np.exp(-np.exp(W.alog.astype(np.float64)) * sp)
    beta = 1.0 / (1.0 + np.exp(-b))
    y = np.empty((VH, VD))
    for h in range(VH):
        src = h // (VH // KH)
        Sd = decay[h] * S[h]
        S[h] = Sd + beta[h] * np.outer(k[src], v[h] - Sd.T @ k[src])
        yh = S[h].T @ q[src]
        y[h] = yh / np.sqrt(np.mean(yh * yh) + W.eps) * W.gnorm * (z[h] / (1.0 + np.exp(-z[h])))
    return proj64(W.out, y.reshape(-1))


def test_gqa_brute_f64(lorc, gen):
    W = _layers.GqaWeights(gen, 0x71, 256, 4, 2, 64, 16, 32, theta=1e4)
    max_t, T = 8, 5
    cache = W.new_cache(max_t)
    Ks, Vs = [[] for _ in range(W.KH)], [[] for _ in range(W.KH)]
    for t in range(T):
        x = gen.normal(W.D, 0x710 + t)
        y = W.oracle(lorc, cache, max_t, t, x)
        e = gqa64(W, Ks, Vs, t, x)
        assert _util.normrel(y, e) < 2e-6, t
    # the cache rows are the normed + rotated keys and the raw values
    kc = cache[0].reshape(W.KH, max_t, W.hd)[:, :T]
    assert np.allclose(kc, np.array(Ks), rtol=1e-5, atol=1e-5)


def test_gqa_pos0_is_value_row(lorc, gen):
    """One key: softmax is exactly 1, so ctx_h = v_{h / (H/KH)} * sigmoid(gate_h)."""
    W = _layers.GqaWeights(gen, 0x72, 256, 4, 2, 64, 16, 32)
    x = gen.normal(W.D, 0x720)
    y = W.oracle(lorc, W.new_cache(4), 4, 0, x)
    qg = proj64(W.q, x).reshape(W.H, 2, W.hd)
    v = proj64(W.v, x).reshape(W.KH, W.hd)
    ctx = np.stack([v[h // (W.H // W.KH)] / (1.0 + np.exp(-qg[h, 1])) for h in range(W.H)])
    assert _util.normrel(y, proj64(W.o, ctx.reshape(-1))) < 2e-6


def test_rope_identities(lorc, gen):
    rot, hd, theta = 16, 64, np.float32(1e7)
    x = gen.normal(hd, 0x730)
    y = x.copy()
    lorc.orc_rope_partial(_util.P(y), 0, rot, theta)
    assert np.array_equal(y, x)   # position 0: cos 1, sin 0
    for pos in (1, 7, 4095):
        y = x.copy()
        lorc.orc_rope_partial(_util.P(y), pos, rot, theta)
        hr = rot // 2
        n0 = np.hypot(x[:hr].astype(np.float64), x[hr:rot])
        n1 = np.hypot(y[:hr].astype(np.float64), y[hr:rot])
        assert np.allclose(n0, n1, rtol=1e-6)          # rotations keep pair norms
        assert np.array_equal(y[rot:], x[rot:])          # dims past rot untouched
        assert np.allclose(y[:rot], rope64(x, pos, rot, theta)[:rot], rtol=0, atol=2e-5 * np.abs(x).max())


def test_gdn_brute_f64(lorc, gen):
    W = _layers.GdnWeights(gen, 0x74, 256, 2, 32, 4, 32, 4, 32)
    st = W.new_state()
    conv = [np.zeros(W.CD) for _ in range(W.K - 1)]
    S = np.zeros((W.VH, W.KD, W.VD))
    for t in range(5):
        x = gen.normal(W.D, 0x740 + t)
        y = W.oracle(lorc, st, x)
        e = gdn64(W, conv, S, x)
        assert _util.normrel(y, e) < 1e-5, t
    assert _util.normrel(st[1], S.reshape(-1)) < 1e-5
    ring = np.array(conv[-W.K:])
    assert np.allclose(st[0].reshape(W.K, W.CD), ring, rtol=0, atol=1e-5 * np.abs(ring).max())


def test_gdn_fmt6_ab(lorc, gen):
    """a/b as fmt 6 projections (the config-3 synthetic model) follow the same math."""
    W = _layers.GdnWeights(gen, 0x75, 256, 2, 32, 4, 32, 4, 32, ab_fmt=6)
    st = W.new_state()
    conv = [np.zeros(W.CD) for _ in range(W.K - 1)]
    S = np.zeros((W.VH, W.KD, W.VD))
    for t in range(3):
        x = gen.normal(W.D, 0x750 + t)
        assert _util.normrel(W.oracle(lorc, st, x), gdn64(W, conv, S, x)) < 1e-5, t
