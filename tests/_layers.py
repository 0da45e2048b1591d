"""Attention (GQA) and GatedDeltaNet layer weights for the tests: seeded synthetic host
weights, their ctypes views for the oracle (orc_gqa_decode / orc_gdn_step) and the
compiled reference (ref_attention / ref_gdn_step), and one-token oracle steps.

Weight statistics: projections fmt 6 as config 0 (codes U{0..15}, scale |N(0,0.02)| at
fp16 precision, zero U{0..15}); norm weights N(0, 0.1) (zero-centred norms) or
1 + N(0, 0.1) (the GDN gated norm); conv N(0, 0.3); A_log N(0, 0.5); dt_bias N(0, 1);
GDN a/b f32 rows N(0, 0.02) (as the reference CPU branch keeps them) or fmt 6.
"""
import ctypes as C

import numpy as np

import _util
from _util import P

_P = C.c_void_p
_I = C.c_int
_F = C.c_float


class OrcMat(C.Structure):
    _fields_ = [("fmt", _I), ("w", _P), ("sz", _P), ("I", _I), ("O", _I), ("gs", _I)]


class OrcGqa(C.Structure):
    _fields_ = [("q", OrcMat), ("k", OrcMat), ("v", OrcMat), ("o", OrcMat), ("qn", _P), ("kn", _P),
                ("H", _I), ("KH", _I), ("hd", _I), ("rot", _I), ("theta", _F), ("eps", _F)]


class OrcGdn(C.Structure):
    _fields_ = [("qkv", OrcMat), ("z", OrcMat), ("a", OrcMat), ("b", OrcMat), ("out", OrcMat), ("conv", _P),
                ("alog", _P), ("dtb", _P), ("gnorm", _P), ("KH", _I), ("KD", _I), ("VH", _I), ("VD", _I),
                ("K", _I), ("eps", _F)]


class RefQ6(C.Structure):
    _fields_ = [("q", _P), ("s", _P)]


def bind(orc, ref=None):
    sig = {
        "orc_proj": (None, [_P, _P, _P]),
        "orc_rope_partial": (None, [_P, _I, _I, _F]),
        "orc_gqa_decode": (None, [_P, _P, _P, _I, _I, _P, _P]),
        "orc_gdn_step": (None, [_P, _P, _P, _P, _P]),
    }
    for n, (r, a) in sig.items():
        f = getattr(orc, n)
        f.restype, f.argtypes = r, a
    if ref is not None:
        ref.ref_attention.restype = None
        ref.ref_attention.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _I, _P, _P, _I, _I, _P, _P]
        ref.ref_gdn_step.restype = None
        ref.ref_gdn_step.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P,
                                     _P]


class Mat:
    """A projection y = W x, W [O, I]: fmt 6 (q, sz), fmt 0 (f32 rows) or fmt 1 (int8 rows
    with per-row power-of-two scales, as vk_dense_init uploads the router and GDN a/b,
    c/qwen.c:1876-1878).  The oracle sees a fmt-1 matrix as its exact f32 equivalent
    q * s (_util.int8_rows: bit-identical products for power-of-two scales)."""

    def __init__(self, gen, seed, O, I, gs, fmt=6, sigma=0.02):
        self.O, self.I, self.gs, self.fmt = O, I, gs, fmt
        if fmt == 6:
            self.q, self.sz = gen.fmt6(O, I, gs, seed)
            self.w = self.q
        elif fmt == 1:
            q8, self.s8, self.w = _util.int8_rows(gen, seed, O, I, sigma)
            self.q8 = q8.view(np.uint8).reshape(-1)
            self.q, self.sz = None, None
        else:
            self.w = gen.f32rows(O, I, seed, sigma)
            self.q, self.sz = None, None

    def orc(self):
        return OrcMat(0 if self.fmt == 1 else self.fmt, P(self.w), P(self.sz), self.I, self.O, self.gs)

    def ref6(self):
        return RefQ6(P(self.q), P(self.sz))

    def upload(self, lib):
        if self.fmt == 1:
            return lib.tensor(self.q8, self.s8, 1, self.I, self.O)
        return lib.tensor(self.w, self.sz, self.fmt, self.I, self.O, self.gs)


class GqaWeights:
    def __init__(self, gen, base, D, H, KH, hd, rot, gs, theta=1e7, eps=1e-6):
        self.D, self.H, self.KH, self.hd, self.rot, self.gs = D, H, KH, hd, rot, gs
        self.theta, self.eps = np.float32(theta), np.float32(eps)
        s = lambda t: gen.stream(base, t)  # noqa: E731
        self.q = Mat(gen, s(1), 2 * H * hd, D, gs)
        self.k = Mat(gen, s(2), KH * hd, D, gs)
        self.v = Mat(gen, s(3), KH * hd, D, gs)
        self.o = Mat(gen, s(4), D, H * hd, gs)
        self.qn = gen.normal(hd, s(5), 0.1)
        self.kn = gen.normal(hd, s(6), 0.1)
        self.in_ln = gen.normal(D, s(7), 0.1)
        self.post_ln = gen.normal(D, s(8), 0.1)
        self.st = OrcGqa(self.q.orc(), self.k.orc(), self.v.orc(), self.o.orc(), P(self.qn), P(self.kn), H, KH, hd,
                         rot, self.theta, self.eps)

    def new_cache(self, max_t):
        return (np.zeros(self.KH * max_t * self.hd, np.float32), np.zeros(self.KH * max_t * self.hd, np.float32))

    def oracle(self, orc, cache, max_t, pos, x):
        out = np.empty(self.D, np.float32)
        orc.orc_gqa_decode(C.addressof(self.st), P(cache[0]), P(cache[1]), max_t, pos, P(x), P(out))
        return out

    def reference(self, ref, cache, max_t, pos, x):
        out = np.empty(self.D, np.float32)
        q, k, v, o = (m.ref6() for m in (self.q, self.k, self.v, self.o))
        ref.ref_attention(C.byref(q), C.byref(k), C.byref(v), C.byref(o), P(self.qn), P(self.kn), self.D, self.H,
                          self.KH, self.hd, self.rot, self.theta, self.eps, self.gs, P(cache[0]), P(cache[1]), max_t,
                          pos, P(x), P(out))
        return out


class GdnWeights:
    def __init__(self, gen, base, D, KH, KD, VH, VD, K, gs, ab_fmt=0, eps=1e-6):
        self.D, self.KH, self.KD, self.VH, self.VD, self.K, self.gs = D, KH, KD, VH, VD, K, gs
        self.eps = np.float32(eps)
        self.CD = 2 * KH * KD + VH * VD
        s = lambda t: gen.stream(base, t)  # noqa: E731
        self.qkv = Mat(gen, s(1), self.CD, D, gs)
        self.z = Mat(gen, s(2), VH * VD, D, gs)
        self.out = Mat(gen, s(3), D, VH * VD, gs)
        self.a = Mat(gen, s(4), VH, D, gs, fmt=ab_fmt)
        self.b = Mat(gen, s(5), VH, D, gs, fmt=ab_fmt)
        self.conv = gen.normal(self.CD * K, s(6), 0.3)
        self.alog = gen.normal(VH, s(7), 0.5)
        self.dtb = gen.normal(VH, s(8), 1.0)
        self.gnorm = (1.0 + gen.normal(VD, s(9), 0.1)).astype(np.float32)
        self.in_ln = gen.normal(D, s(10), 0.1)
        self.post_ln = gen.normal(D, s(11), 0.1)
        self.st = OrcGdn(self.qkv.orc(), self.z.orc(), self.a.orc(), self.b.orc(), self.out.orc(), P(self.conv),
                         P(self.alog), P(self.dtb), P(self.gnorm), KH, KD, VH, VD, K, self.eps)

    def new_state(self):
        """(conv ring [K][CD], recurrent state [VH][KD][VD]) of a fresh sequence."""
        return (np.zeros(self.K * self.CD, np.float32), np.zeros(self.VH * self.KD * self.VD, np.float32))

    def oracle(self, orc, state, x):
        out = np.empty(self.D, np.float32)
        orc.orc_gdn_step(C.addressof(self.st), P(state[0]), P(state[1]), P(x), P(out))
        return out

    def reference(self, ref, state, x):
        assert self.a.fmt == 0 and self.b.fmt == 0, "the reference CPU branch reads f32 a/b"
        out = np.empty(self.D, np.float32)
        qkv, z, o = (m.ref6() for m in (self.qkv, self.z, self.out))
        ref.ref_gdn_step(C.byref(qkv), C.byref(z), C.byref(o), P(self.a.w), P(self.b.w), P(self.conv), P(self.alog),
                         P(self.dtb), P(self.gnorm), self.D, self.KH, self.KD, self.VH, self.VD, self.K, self.eps,
                         self.gs, P(state[0]), P(state[1]), P(x), P(out))
        return out


def gdn_host_params(orc, W, x):
    """[decay(VH) | beta(VH) | gnorm(VD)] as the engine packs them (c/qwen.c:679-688)."""
    a = np.empty(W.VH, np.float32)
    b = np.empty(W.VH, np.float32)
    orc.orc_proj(C.byref(W.a.orc()), P(x), P(a))
    orc.orc_proj(C.byref(W.b.orc()), P(x), P(b))
    sp_in = (a + W.dtb).astype(np.float32)
    sp = np.where(sp_in > 20, sp_in, np.log1p(np.exp(sp_in.astype(np.float64)))).astype(np.float32)
    decay = np.exp(-np.exp(W.alog.astype(np.float64)) * sp).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-b.astype(np.float64)))).astype(np.float32)
    return np.concatenate([decay, beta, W.gnorm]).astype(np.float32)
