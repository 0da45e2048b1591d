"""Host-side binding of libcoli_hip.so (the MI355X drop-in for qwen3.c's Vulkan backend).

The product is the C ABI in include/coli_hip.h; this module is the thin ctypes mirror
that the parity tests and bench.py drive it through.  It loads the in-tree library and
raises if it is missing: there is no fallback implementation behind it.

Functions take numpy arrays for host buffers (the c/backend_vulkan.h entry points) and
integer device addresses for the coli_hip_* device-pointer forms (the caller owns the
device memory, e.g. torch tensors' data_ptr()).
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcoli_hip.so")

_P = C.c_void_p
_I = C.c_int
_F = C.c_float

# name -> (restype, argtypes) for the entry points this binding drives
_SIGS = {
    "coli_vk_init": (_I, [C.c_char_p]),
    "coli_vk_shutdown": (None, []),
    "coli_vk_available": (_I, []),
    "coli_vk_mem_info": (None, [_P, _P]),
    "coli_vk_mem_budget": (_I, [_P, _P]),
    "coli_vk_tensor_ensure": (_I, [_P, _P, _P, _I, _I, _I, _I]),
    "coli_vk_tensor_free": (None, [_P]),
    "coli_vk_tensor_bytes": (C.c_size_t, [_P]),
    "coli_vk_matmul": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "coli_vk_matmul_pair": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _P, _I, _I, _I]),
    "coli_vk_matmul_argmax": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P]),
    "coli_hip_tensor_info": (_I, [_P, _P, _P, _P, _P, _P, _P, _P]),
    "coli_hip_stream": (_P, []),
    "coli_hip_sync": (_I, [_P]),
    "coli_hip_memcpy": (_I, [_P, _P, C.c_size_t]),
    "coli_hip_gemv": (_I, [_P, _P, _P, _I, _P]),
    "coli_hip_gemv_topk": (_I, [_P, _P, _P, _I, _P, _P, _P]),
    "coli_hip_tensor_synth": (_I, [_P, _I, _I, _I, _I, C.c_uint64, C.c_double]),
    "coli_hip_synth_normal": (_I, [_P, C.c_size_t, C.c_uint64, C.c_double, _P]),
    "coli_vk_gate_up": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "coli_vk_expert_group": (_I, [_P, _P, _P, _P, _I, _P, _P]),
    "coli_vk_expert_group_issue": (_I, [_P, _P, _P, _P, _I, _P]),
    "coli_vk_expert_group_take": (_I, [_P]),
    "coli_vk_eg_xs_bind": (_I, [_P, _I, _I]),
    "coli_vk_expert_group_issue_id": (_I, [_P, _P, _P, _P, _I, _P]),
    "coli_vk_moe_ix_available": (_I, []),
    "coli_vk_eg_table_init": (_I, [_I, _I, _I, _I, _I]),
    "coli_vk_eg_table_set": (_I, [_I, _I, _P, _P, _P]),
    "coli_vk_eg_table_set_shared": (_I, [_I, _P, _P, _P, _P, _I]),
    "coli_hip_moe_decode": (_I, [_I, _P, _I, _P, _P, _I, _P, _P, _P]),
    "coli_hip_moe_error": (_I, []),
    "coli_hip_moe_prefill": (_I, [_I, _P, _I, _P, _I, _P, _P, _P, _P]),
}


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Tensor:
    """A ColiVkTensor* handle (device copy of one quantized weight)."""

    def __init__(self, lib, fmt, I, O, gs):
        self.lib, self.fmt, self.I, self.O, self.gs = lib, fmt, I, O, gs
        self.handle = C.c_void_p(None)

    @property
    def ref(self):
        return C.byref(self.handle)

    def info(self):
        f, i, o, g, rb = (C.c_int() for _ in range(5))
        w, s = C.c_void_p(), C.c_void_p()
        if not self.lib.L.coli_hip_tensor_info(self.handle, C.byref(f), C.byref(i), C.byref(o),
                                                C.byref(g), C.byref(rb), C.byref(w), C.byref(s)):
            raise RuntimeError("coli_hip_tensor_info failed")
        return dict(fmt=f.value, I=i.value, O=o.value, gs=g.value, row_bytes=rb.value,
                    d_w=w.value, d_sz=s.value)

    def nbytes(self):
        return int(self.lib.L.coli_vk_tensor_bytes(self.handle))


class Lib:
    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
        self.path = path
        # torch ships its own HIP runtime (libamdhip64.so.7).  Importing it first makes
        # this library bind to that already-loaded runtime, so the process has exactly
        # one HIP runtime and torch device pointers are valid here.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        self.L = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(self.L, name)
            fn.restype = res
            fn.argtypes = args

    # ---- device bring-up -------------------------------------------------------
    def init(self):
        if not self.L.coli_vk_init(b""):
            raise RuntimeError("coli_vk_init failed (no gfx950 device?)")
        return self

    def available(self):
        return bool(self.L.coli_vk_available())

    def stream(self):
        return self.L.coli_hip_stream()

    # ---- tensors ----------------------------------------------------------------
    def tensor(self, w, s, fmt, I, O, gs=0):
        """Upload host weights (c/backend_vulkan.h:105 semantics)."""
        t = Tensor(self, fmt, I, O, gs)
        w = np.ascontiguousarray(w)
        s = None if s is None else np.ascontiguousarray(s, dtype=np.float32)
        if not self.L.coli_vk_tensor_ensure(t.ref, _ptr(w), _ptr(s), fmt, I, O, gs):
            raise RuntimeError(f"coli_vk_tensor_ensure(fmt={fmt}, I={I}, O={O}, gs={gs}) failed")
        return t

    def tensor_synth(self, fmt, I, O, gs, seed, sigma):
        """Tensor generated on the device with the synthetic-data spec."""
        t = Tensor(self, fmt, I, O, gs)
        if not self.L.coli_hip_tensor_synth(t.ref, fmt, I, O, gs, C.c_uint64(seed), sigma):
            raise RuntimeError("coli_hip_tensor_synth failed")
        return t

    # ---- host-buffer entry points (drop-in ABI) ------------------------------------
    def matmul(self, t, x, S=1, w=None, s=None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(S * t.O, np.float32)
        if not self.L.coli_vk_matmul(t.ref, _ptr(y), _ptr(x), _ptr(w), _ptr(s), t.fmt, S, t.I, t.O, t.gs):
            raise RuntimeError("coli_vk_matmul failed")
        return y

    def matmul_pair(self, t1, t2, x, S=1):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y1 = np.empty(S * t1.O, np.float32)
        y2 = np.empty(S * t2.O, np.float32)
        if not self.L.coli_vk_matmul_pair(t1.ref, _ptr(y1), None, None, t1.O, t2.ref, _ptr(y2), None, None,
                                          t2.O, t1.fmt, _ptr(x), S, t1.I, t1.gs):
            raise RuntimeError("coli_vk_matmul_pair failed")
        return y1, y2

    def matmul_argmax(self, t, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        idx, val = C.c_int(), C.c_float()
        if not self.L.coli_vk_matmul_argmax(t.ref, None, None, t.fmt, t.I, t.O, t.gs, _ptr(x),
                                            C.byref(idx), C.byref(val)):
            raise RuntimeError("coli_vk_matmul_argmax failed")
        return idx.value, val.value

    # ---- device-pointer entry points ---------------------------------------------
    def gemv_dev(self, t, d_x, d_y, S=1, stream=None):
        if not self.L.coli_hip_gemv(t.handle, d_x, d_y, S, stream):
            raise RuntimeError("coli_hip_gemv failed")

    def gemv_topk_dev(self, t, d_x, d_y, k, d_idx, d_val, stream=None):
        if not self.L.coli_hip_gemv_topk(t.handle, d_x, d_y, k, d_idx, d_val, stream):
            raise RuntimeError("coli_hip_gemv_topk failed")

    def sync(self, stream=None):
        if not self.L.coli_hip_sync(stream):
            raise RuntimeError("coli_hip_sync failed")

    def memcpy(self, dst, src, nbytes):
        """Blocking copy; dst/src are integer addresses (host or device)."""
        if not self.L.coli_hip_memcpy(dst, src, nbytes):
            raise RuntimeError("coli_hip_memcpy failed")

    def synth_normal_dev(self, d_dst, n, seed, sigma, stream=None):
        if not self.L.coli_hip_synth_normal(d_dst, n, C.c_uint64(seed), sigma, stream):
            raise RuntimeError("coli_hip_synth_normal failed")

    # ---- MoE: expert MLPs on host buffers (c/backend_vulkan.h:75-101) ---------------
    def gate_up(self, g, u, x, S=1):
        x = np.ascontiguousarray(x, dtype=np.float32)
        h = np.empty(S * g.O, np.float32)
        if not self.L.coli_vk_gate_up(g.ref, u.ref, _ptr(h), _ptr(x), None, None, None, None, g.fmt, S, g.I,
                                      g.O, g.gs):
            raise RuntimeError("coli_vk_gate_up failed")
        return h

    @staticmethod
    def _group(gates, ups, downs, rows):
        n = len(gates)
        arr = lambda ts: (C.c_void_p * n)(*[t.handle.value for t in ts])
        return arr(gates), arr(ups), arr(downs), (C.c_int * n)(*rows)

    def expert_group(self, gates, ups, downs, rows, x):
        """y[sum(rows), D]: row block c = down_c(silu(gate_c x) * up_c x)."""
        g, u, d, r = self._group(gates, ups, downs, rows)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(sum(rows) * gates[0].I, np.float32)
        if not self.L.coli_vk_expert_group(g, u, d, r, len(gates), _ptr(y), _ptr(x)):
            raise RuntimeError("coli_vk_expert_group failed")
        return y

    def expert_group_issue(self, gates, ups, downs, rows, x):
        g, u, d, r = self._group(gates, ups, downs, rows)
        x = np.ascontiguousarray(x, dtype=np.float32)
        return bool(self.L.coli_vk_expert_group_issue(g, u, d, r, len(gates), _ptr(x)))

    def expert_group_take(self, n_rows, D):
        y = np.empty(n_rows * D, np.float32)
        if not self.L.coli_vk_expert_group_take(_ptr(y)):
            raise RuntimeError("coli_vk_expert_group_take failed")
        return y

    def eg_xs_bind(self, xs, S, D):
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        if not self.L.coli_vk_eg_xs_bind(_ptr(xs), S, D):
            raise RuntimeError("coli_vk_eg_xs_bind failed")

    def expert_group_issue_id(self, gates, ups, downs, rows, tok_ids):
        g, u, d, r = self._group(gates, ups, downs, rows)
        ids = np.ascontiguousarray(tok_ids, dtype=np.int32)
        return bool(self.L.coli_vk_expert_group_issue_id(g, u, d, r, len(gates), _ptr(ids)))

    # ---- MoE: device expert table + one-launch block (c/backend_vulkan.h:243-252) ----
    def eg_table_init(self, n_layers, E, D, I, gs):
        if not self.L.coli_vk_eg_table_init(n_layers, E, D, I, gs):
            raise RuntimeError("coli_vk_eg_table_init failed")

    def eg_table_set(self, layer, eid, g, u, d):
        if not self.L.coli_vk_eg_table_set(layer, eid, g.handle, u.handle, d.handle):
            raise RuntimeError(f"coli_vk_eg_table_set({layer}, {eid}) failed")

    def eg_table_set_shared(self, layer, g, u, d, sh_gate):
        sg = np.ascontiguousarray(sh_gate, dtype=np.float32)
        if not self.L.coli_vk_eg_table_set_shared(layer, g.handle, u.handle, d.handle, _ptr(sg), sg.size):
            raise RuntimeError("coli_vk_eg_table_set_shared failed")

    def moe_decode_dev(self, layer, router, K, d_x, d_out, accumulate=False, d_idx=None, d_val=None,
                       stream=None):
        if not self.L.coli_hip_moe_decode(layer, router.handle, K, d_x, d_out, int(accumulate), d_idx, d_val,
                                          stream):
            raise RuntimeError("coli_hip_moe_decode failed")

    def moe_prefill_dev(self, layer, router, K, d_xs, S, d_out, d_idx=None, d_val=None, stream=None):
        if not self.L.coli_hip_moe_prefill(layer, router.handle, K, d_xs, S, d_out, d_idx, d_val, stream):
            raise RuntimeError("coli_hip_moe_prefill failed")

    def moe_error(self):
        return int(self.L.coli_hip_moe_error())
