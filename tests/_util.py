"""Test helpers: ctypes bindings of the CPU oracle (oracle/liboracle.so) and of the
compiled reference kernels (oracle/_ref/libqwenref.so, present only where the reference
checkout was available at build time), synthetic inputs, and error metrics.

Only tests use this module; the oracle is the checker, never the thing measured.
"""
import ctypes as C
import importlib.util
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
ORACLE_OMP_SO = os.path.join(ROOT, "oracle", "liboracle_omp.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libqwenref.so")
GOLDEN = os.path.join(ROOT, "tests", "golden")

_P = C.c_void_p
_I = C.c_int
_F = C.c_float


def P(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class OrcExpert(C.Structure):
    _fields_ = [("g", _P), ("u", _P), ("d", _P), ("gs", _P), ("us", _P), ("ds", _P)]


def eptr(arr, i=0):
    """Address of element i of a ctypes OrcExpert array (for `const OrcExpert *` args)."""
    return C.addressof(arr) + i * C.sizeof(OrcExpert)


def load_oracle(omp=False):
    L = C.CDLL(ORACLE_OMP_SO if omp else ORACLE_SO)
    sig = {
        "orc_matmul_q4g_asym": (None, [_P, _P, _P, _P, _I, _I, _I]),
        "orc_matmul_f32": (None, [_P, _P, _P, _I, _I, _I]),
        "orc_matmul_q8": (None, [_P, _P, _P, _P, _I, _I]),
        "orc_quant_rows": (None, [_P, _I, _I, _I, _I, _P, _P]),
        "orc_rmsnorm_zc": (None, [_P, _P, _P, _I, _F]),
        "orc_softmax_row": (None, [_P, _I]),
        "orc_route_topk": (None, [_P, _I, _I, _P, _P]),
        "orc_expert_mlp_fmt6": (None, [_P, _P, _I, _I, _I, _P]),
        "orc_moe_decode": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
        "orc_moe_prefill": (None, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P]),
        "orc_argmax": (_I, [_P, _I]),
        "orc_topk_logits": (None, [_P, _I, _I, _P, _P]),
        "orc_mix64": (C.c_uint64, [C.c_uint64]),
        "orc_hash": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "orc_stream": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "orc_normal": (C.c_double, [C.c_uint64, C.c_uint64]),
        "orc_f16_round": (_F, [C.c_double]),
        "orc_gen_bytes": (None, [_P, C.c_size_t, C.c_uint64]),
        "orc_gen_sz": (None, [_P, C.c_size_t, C.c_uint64, C.c_double]),
        "orc_gen_normal": (None, [_P, C.c_size_t, C.c_uint64, C.c_double]),
    }
    for n, (r, a) in sig.items():
        f = getattr(L, n)
        f.restype, f.argtypes = r, a
    return L


def load_ref():
    if not os.path.exists(REF_SO):
        return None
    L = C.CDLL(REF_SO)
    sig = {
        "ref_matmul_q4g_asym": (None, [_P, _P, _P, _P, _I, _I, _I]),
        "ref_matmul": (None, [_P, _P, _P, _I, _I, _I]),
        "ref_matmul_q8": (None, [_P, _P, _P, _P, _I, _I]),
        "ref_quant_rows": (None, [_P, _I, _I, _I, _I, _P, _P]),
        "ref_rmsnorm_zc": (None, [_P, _P, _P, _I, _F]),
        "ref_softmax_row": (None, [_P, _I]),
        "ref_expert_mlp_fmt6": (None, [_P, _P, _I, _I, _I, _P]),
        "ref_moe_token": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
        "ref_moe_batch": (None, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    }
    for n, (r, a) in sig.items():
        f = getattr(L, n)
        f.restype, f.argtypes = r, a
    return L


def load_product():
    """The product binding (qwen3.c_amd/__init__.py), imported by path."""
    path = os.path.join(ROOT, "qwen3.c_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location("qwen3_c_amd", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


# ---------------------------------------------------------------- synthetic inputs
class Gen:
    """Host side of the synthetic-data spec shared with the device generator."""

    def __init__(self, orc):
        self.o = orc

    def stream(self, base, tag):
        return int(self.o.orc_stream(base, tag))

    def bytes(self, n, seed):
        a = np.empty(n, np.uint8)
        self.o.orc_gen_bytes(P(a), n, seed)
        return a

    def sz(self, ngroups, seed, sigma=0.02):
        a = np.empty(2 * ngroups, np.float32)
        self.o.orc_gen_sz(P(a), ngroups, seed, sigma)
        return a

    def normal(self, n, seed, sigma=1.0):
        a = np.empty(n, np.float32)
        self.o.orc_gen_normal(P(a), n, seed, sigma)
        return a

    def fmt6(self, O, I, gs, seed, sigma=0.02):
        """(q [O*(I+1)//2] u8, sz [O*ng*2] f32): the host copy of coli_hip_tensor_synth."""
        ng = (I + gs - 1) // gs
        q = self.bytes(O * ((I + 1) // 2), self.stream(seed, 1))
        s = self.sz(O * ng, self.stream(seed, 2), sigma)
        return q, s

    def f32rows(self, O, I, seed, sigma):
        return self.normal(O * I, self.stream(seed, 3), sigma)


def expert_seed(gen, base, layer, eid):
    """Seed of expert eid (eid == E: the shared expert) of a layer."""
    return gen.stream(base, 1000 + layer * 4096 + eid)


def int8_rows(gen, base, O, I, sigma=0.02):
    """int8 rows q [O, I] with per-row power-of-two scales s, and f = q * s as f32 [O*I].
    With s = 2^-k the fmt-1 product (sum x*q, then * s, c/qwen.c:230-238) equals the f32
    dot with rows q * s bit for bit: scaling by a power of two commutes with every rounding
    of the sum (nothing overflows or underflows at these magnitudes), so an f32 oracle pins
    an int8 path."""
    s = np.ldexp(np.ones(O, np.float32), -(11 + np.arange(O) % 3)).astype(np.float32)
    w = gen.normal(O * I, gen.stream(base, 30), sigma).reshape(O, I)
    q = np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8)
    f = (q.astype(np.float32) * s[:, None]).astype(np.float32).reshape(-1)
    return q, s, f


class MoeWeights:
    """One MoE layer: f32 router [E, D], E fmt-6 experts + shared, f32 sh_gate [D]."""

    def __init__(self, gen, base, D, I, E, gs, layer=0, experts=True):
        self.D, self.I, self.E, self.gs = D, I, E, gs
        self.router = gen.f32rows(E, D, gen.stream(base, 10 + layer), 0.02)
        self.sh_gate = gen.normal(D, gen.stream(base, 20 + layer), 0.02)
        self.exp = []
        if experts:
            for e in range(E + 1):
                s = expert_seed(gen, base, layer, e)
                g = gen.fmt6(I, D, gs, gen.stream(s, 1))
                u = gen.fmt6(I, D, gs, gen.stream(s, 2))
                d = gen.fmt6(D, I, gs, gen.stream(s, 3))
                self.exp.append((g, u, d))

    def orc_experts(self):
        arr = (OrcExpert * (self.E + 1))()
        for e, (g, u, d) in enumerate(self.exp):
            arr[e] = OrcExpert(P(g[0]), P(u[0]), P(d[0]), P(g[1]), P(u[1]), P(d[1]))
        return arr


# ---------------------------------------------------------------- metrics
def maxrel(got, ref, floor=1e-2):
    """max |got-ref| / max(|ref|, floor): the VK_TEST metric of the reference
    (c/backend_vulkan.c:4462,4474 compares only where |ref| > 1e-2)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor)))


def maxrel_scaled(got, ref):
    """maxrel with the floor scaled to the output's magnitude: 1e-2 * max(1, max|ref|).
    For O(1) outputs this is the VK_TEST metric; for outputs of magnitude M (a MoE block
    sums K+1 expert outputs) fp32 accumulation leaves absolute errors ~M * 2^-24 * sqrt(n)
    on every element, so a fixed 1e-2 floor would grade cancellation, not accuracy."""
    ref = np.asarray(ref, np.float64)
    return maxrel(got, ref, floor=1e-2 * max(1.0, float(np.max(np.abs(ref)))))


def normrel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def brute_fmt6(q, sz, x, I, O, gs):
    """f64 dequant-dot straight from the format definition (independent of the oracle)."""
    rb = (I + 1) // 2
    ng = (I + gs - 1) // gs
    b = q.reshape(O, rb)
    nib = np.empty((O, 2 * rb), np.float64)
    nib[:, 0::2] = b & 15
    nib[:, 1::2] = b >> 4
    nib = nib[:, :I]
    s = sz.reshape(O, ng, 2).astype(np.float64)
    gidx = np.arange(I) // gs
    w = (nib - s[:, gidx, 1]) * s[:, gidx, 0]
    return w @ x.astype(np.float64)
