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
# COLI_HIP_LIB names another build of the library (a variant with other launch constants,
# for side-by-side timing); the default is the in-tree build.
LIB_PATH = os.environ.get("COLI_HIP_LIB") or os.path.join(HERE, "libcoli_hip.so")

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
    "coli_hip_moe_force_error": (_I, [_I]),
    "coli_hip_moe_decode_noalloc": (_I, [_I, _P, _I, _P, _P, _I, _P, _P, _P]),
    "coli_hip_gemv_error": (_I, []),
    "coli_hip_moe_prefill": (_I, [_I, _P, _I, _P, _I, _P, _P, _P, _P]),
    # attention / GatedDeltaNet layer blocks and the residual stream (c/backend_vulkan.h:110-279)
    "coli_vk_kv_ensure": (_I, [_I, _I, _I, _I]),
    "coli_vk_kv_row": (_I, [_I, _I, _P, _P]),
    "coli_vk_kv_reset": (None, []),
    "coli_hip_kv_load": (_I, [_I, _I, _I, _P, _P]),
    "coli_hip_kv_read": (_I, [_I, _I, _I, _P, _P]),
    "coli_vk_gqa_norm_weight": (_I, [_I, _P, _P, _I]),
    "coli_vk_gqa_full": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _F, _I]),
    "coli_vk_gdn_state_ensure": (_I, [_I, _I, _I, _I]),
    "coli_vk_gdn_reset": (None, []),
    "coli_vk_gdn_conv_ensure": (_I, [_I, _I, _I]),
    "coli_vk_gdn_conv_weight": (_I, [_I, _P, _I, _I]),
    "coli_vk_gdn_ba_weight": (_I, [_I, _P, _P, _P, _I, _I]),
    "coli_hip_gdn_state_read": (_I, [_I, _P, _P]),
    "coli_hip_layer_fuse": (_I, [_I]),
    "coli_hip_moe_cert_all": (_I, [_I]),
    "coli_hip_eg_force_gemv": (_I, [_I]),
    "coli_hip_gqa_seq": (_I, [_I]),
    "coli_hip_gdn_chunked": (_I, [_I]),
    "coli_hip_st_open": (_P, [C.c_char_p]),
    "coli_hip_st_close": (None, [_P]),
    "coli_hip_st_count": (_I, [_P]),
    "coli_hip_st_find": (_I, [_P, C.c_char_p, _P, _P, _P, _P, _P]),
    "coli_hip_st_read_f32": (C.c_int64, [_P, C.c_char_p, _P, C.c_int64]),
    "coli_hip_st_read_raw": (C.c_int64, [_P, C.c_char_p, _P, C.c_int64]),
    "coli_hip_st_tensor": (_I, [_P, C.c_char_p, _P, _I, _I, _I, _I]),
    "coli_hip_st_experts": (_I, [_P, _I, _I, _I, _I, _I]),
    "coli_vk_gdn_full": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I]),
    "coli_vk_gdn_full_seq": (_I, [_I, _P, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I]),
    "coli_vk_layer_norm_weight": (_I, [_I, _P, _P, _I]),
    "coli_vk_gqa_full_route": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                    _F, _F, _I, _I]),
    "coli_vk_gdn_full_route": (_I, [_I, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                    _F, _I, _I]),
    "coli_vk_stream_available": (_I, []),
    "coli_vk_stream_begin": (_I, [_P, _I]),
    "coli_vk_stream_end": (_I, [_P, _I]),
    "coli_vk_stream_add": (_I, [_P, _I]),
    "coli_vk_stream_nrm": (_P, []),
    "coli_vk_stream_copy_resid": (_I, [_P, _I]),
    "coli_vk_final_norm_weight": (_I, [_P, _I]),
    "coli_vk_stream_norm_argmax": (_I, [_P, _P, _P, _I, _I, _I, _I, _F, _P, _P]),
    "coli_vk_gqa_full_route_pipe": (_I, [_I, _I, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                         _F, _F, _I, _I]),
    "coli_vk_gdn_full_route_pipe": (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                         _F, _I, _I]),
    "coli_vk_expert_group_issue_pipe": (_I, [_P, _P, _P, _P, _P, _I, _I]),
    "coli_vk_expert_group_take_pipe": (_I, []),
    "coli_vk_stream_moe_fused": (_I, []),
    "coli_vk_stream_ix_pending": (_I, []),
    "coli_vk_stream_ix_hist": (_I, [_I, _P, _I]),
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


class Container:
    """A ColiHipSt* (fmt=6 safetensors container index).  Opening needs no device."""

    DTYPES = {0: "BF16", 1: "F16", 2: "F32", 3: "U8"}

    def __init__(self, lib, path):
        self.lib = lib
        self.h = lib.L.coli_hip_st_open(os.fsencode(path))
        if not self.h:
            raise ValueError(f"coli_hip_st_open({path}) refused the container")

    def close(self):
        if self.h:
            self.lib.L.coli_hip_st_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self):
        return int(self.lib.L.coli_hip_st_count(self.h))

    def find(self, name):
        """(dtype name, numel, nbytes, shape) or None."""
        dt, ne, nb, nd = C.c_int(), C.c_int64(), C.c_int64(), C.c_int()
        shape = (C.c_int64 * 8)()
        if not self.lib.L.coli_hip_st_find(self.h, name.encode(), C.byref(dt), C.byref(ne), C.byref(nb),
                                           C.byref(nd), shape):
            return None
        return self.DTYPES[dt.value], ne.value, nb.value, tuple(shape[i] for i in range(nd.value))

    def read_f32(self, name, cap):
        out = np.empty(max(cap, 1), np.float32)
        n = self.lib.L.coli_hip_st_read_f32(self.h, name.encode(), _ptr(out), cap)
        return None if n < 0 else out[:n]

    def read_raw(self, name, cap):
        out = np.empty(max(cap, 1), np.uint8)
        n = self.lib.L.coli_hip_st_read_raw(self.h, name.encode(), _ptr(out), cap)
        return None if n < 0 else out[:n]

    def tensor(self, name, fmt, I, O, gs=0):
        t = Tensor(self.lib, fmt, I, O, gs)
        if not self.lib.L.coli_hip_st_tensor(self.h, name.encode(), t.ref, fmt, I, O, gs):
            raise RuntimeError(f"coli_hip_st_tensor({name}) failed")
        return t

    def experts(self, layer, E, D, I, gs):
        if not self.lib.L.coli_hip_st_experts(self.h, layer, E, D, I, gs):
            raise RuntimeError(f"coli_hip_st_experts(layer {layer}) failed")


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

    def mem_info(self):
        """(device bytes held by live tensors, live tensor count), coli_vk_mem_info."""
        b, n = C.c_size_t(), C.c_size_t()
        self.L.coli_vk_mem_info(C.byref(b), C.byref(n))
        return b.value, n.value

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

    def expert_group_take_into(self, y):
        """take into a caller's float32 buffer (reused across calls, as the engine's heap
        block is); y must hold the issued rows."""
        assert y.dtype == np.float32 and y.flags.c_contiguous
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

    def moe_decode_noalloc_dev(self, layer, router, K, d_x, d_out, accumulate=False, d_idx=None, d_val=None,
                               stream=None):
        """coli_hip_moe_decode_noalloc; returns its 0/1 result (0: refused)."""
        return int(self.L.coli_hip_moe_decode_noalloc(layer, router.handle, K, d_x, d_out, int(accumulate), d_idx,
                                                      d_val, stream))

    def moe_error(self):
        return int(self.L.coli_hip_moe_error())

    def moe_force_error(self, code=1):
        self._ok(self.L.coli_hip_moe_force_error(code), "coli_hip_moe_force_error")

    def gemv_error(self):
        return int(self.L.coli_hip_gemv_error())

    # ---- attention / GatedDeltaNet state (c/backend_vulkan.h:110-116, 146-156, 258-279) ----
    def _ok(self, r, what):
        if not r:
            raise RuntimeError(f"{what} failed")

    def kv_ensure(self, layer, max_rows, K, Rd):
        self._ok(self.L.coli_vk_kv_ensure(layer, max_rows, K, Rd), "coli_vk_kv_ensure")

    def kv_load(self, layer, row0, Krows, Vrows):
        Krows = np.ascontiguousarray(Krows, dtype=np.float32)
        Vrows = np.ascontiguousarray(Vrows, dtype=np.float32)
        n = Krows.shape[0]
        self._ok(self.L.coli_hip_kv_load(layer, row0, n, _ptr(Krows), _ptr(Vrows)), "coli_hip_kv_load")

    def kv_read(self, layer, row0, n, kd, vd):
        K = np.empty((n, kd), np.float32)
        V = np.empty((n, vd), np.float32)
        self._ok(self.L.coli_hip_kv_read(layer, row0, n, _ptr(K), _ptr(V)), "coli_hip_kv_read")
        return K, V

    def gqa_norm_weight(self, layer, qn, kn):
        qn = np.ascontiguousarray(qn, dtype=np.float32)
        kn = np.ascontiguousarray(kn, dtype=np.float32)
        self._ok(self.L.coli_vk_gqa_norm_weight(layer, _ptr(qn), _ptr(kn), qn.size), "coli_vk_gqa_norm_weight")

    def gdn_setup(self, layer, VH, KD, VD, K, CD, conv, alog=None, dtb=None, gnorm=None):
        self._ok(self.L.coli_vk_gdn_state_ensure(layer, VH, KD, VD), "coli_vk_gdn_state_ensure")
        self._ok(self.L.coli_vk_gdn_conv_ensure(layer, K, CD), "coli_vk_gdn_conv_ensure")
        conv = np.ascontiguousarray(conv, dtype=np.float32)
        self._ok(self.L.coli_vk_gdn_conv_weight(layer, _ptr(conv), K, CD), "coli_vk_gdn_conv_weight")
        if alog is not None:
            a, d, g = (np.ascontiguousarray(v, dtype=np.float32) for v in (alog, dtb, gnorm))
            self._ok(self.L.coli_vk_gdn_ba_weight(layer, _ptr(a), _ptr(d), _ptr(g), VH, VD), "coli_vk_gdn_ba_weight")

    def layer_fuse(self, on):
        """Fused layer launches on/off (test hook); returns the previous setting."""
        return bool(self.L.coli_hip_layer_fuse(1 if on else 0))

    def eg_force_gemv(self, on):
        """Host-routed expert groups with rows > 1 on GEMV items (True) or MFMA (False);
        returns the previous setting."""
        return bool(self.L.coli_hip_eg_force_gemv(1 if on else 0))

    def gqa_seq(self, on):
        """coli_vk_gqa_full over S >= 4 rows batched (True) or token by token (False);
        returns the previous setting."""
        return bool(self.L.coli_hip_gqa_seq(1 if on else 0))

    def gdn_chunked(self, on):
        """coli_vk_gdn_full_seq's recurrence per 64-token chunk (True) or token by token;
        returns the previous setting."""
        return bool(self.L.coli_hip_gdn_chunked(1 if on else 0))

    def moe_cert_all(self, on):
        """Certify every decode route on/off (test hook); returns the previous setting."""
        return bool(self.L.coli_hip_moe_cert_all(1 if on else 0))

    def gdn_reset(self):
        self.L.coli_vk_gdn_reset()

    def gdn_state_read(self, layer, K, CD, VH, KD, VD):
        ring = np.empty(K * CD, np.float32)
        S = np.empty(VH * KD * VD, np.float32)
        self._ok(self.L.coli_hip_gdn_state_read(layer, _ptr(ring), _ptr(S)), "coli_hip_gdn_state_read")
        return ring, S

    def layer_norm_weight(self, layer, in_ln, post_ln):
        a = np.ascontiguousarray(in_ln, dtype=np.float32)
        b = np.ascontiguousarray(post_ln, dtype=np.float32)
        self._ok(self.L.coli_vk_layer_norm_weight(layer, _ptr(a), _ptr(b), a.size), "coli_vk_layer_norm_weight")

    # ---- layer blocks on host rows ---------------------------------------------------
    def gqa_full(self, layer, x, tq, tk, tv, to, S, H, KH, hd, rot, pos_base, max_t, eps, theta):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(S * to.O, np.float32)
        self._ok(self.L.coli_vk_gqa_full(layer, _ptr(x), tq.I, tq.handle, tk.handle, tv.handle, to.handle, _ptr(out),
                                         S, H, KH, hd, rot, pos_base, max_t, eps, theta, to.O), "coli_vk_gqa_full")
        return out

    def gdn_full_seq(self, layer, x, params, tqkv, tz, tout, S, KH, KD, VH, VD, CD, K, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        p = np.ascontiguousarray(params, dtype=np.float32)
        out = np.empty(S * tout.O, np.float32)
        self._ok(self.L.coli_vk_gdn_full_seq(layer, _ptr(x), S, tqkv.I, tqkv.handle, tz.handle, _ptr(p), tout.handle,
                                             _ptr(out), KH, KD, VH, VD, CD, K, eps, tout.O), "coli_vk_gdn_full_seq")
        return out

    def gqa_full_route(self, layer, resid, tq, tk, tv, to, router, ln_layer, S, H, KH, hd, rot, pos_base, max_t,
                       eps, theta):
        resid = np.ascontiguousarray(resid, dtype=np.float32)
        D, E = tq.I, router.O
        ro, no, pr = np.empty(S * D, np.float32), np.empty(S * D, np.float32), np.empty(S * E, np.float32)
        self._ok(self.L.coli_vk_gqa_full_route(layer, _ptr(resid), D, tq.handle, tk.handle, tv.handle, to.handle,
                                               router.handle, ln_layer, _ptr(ro), _ptr(no), _ptr(pr), S, H, KH, hd,
                                               rot, pos_base, max_t, eps, theta, D, E), "coli_vk_gqa_full_route")
        return ro, no, pr

    def gdn_full_route(self, layer, x_in, resid, params, tqkv, tz, tout, router, ln_layer, KH, KD, VH, VD, CD, K,
                       eps):
        x_in = np.ascontiguousarray(x_in, dtype=np.float32)
        resid = np.ascontiguousarray(resid, dtype=np.float32)
        p = np.ascontiguousarray(params, dtype=np.float32)
        D, E = tqkv.I, router.O
        ro, no, pr = np.empty(D, np.float32), np.empty(D, np.float32), np.empty(E, np.float32)
        self._ok(self.L.coli_vk_gdn_full_route(layer, _ptr(x_in), _ptr(resid), D, tqkv.handle, tz.handle, _ptr(p),
                                               tout.handle, router.handle, ln_layer, _ptr(ro), _ptr(no), _ptr(pr),
                                               KH, KD, VH, VD, CD, K, eps, D, E), "coli_vk_gdn_full_route")
        return ro, no, pr

    # ---- residual stream (c/backend_vulkan.h:199-252) ----------------------------------
    def stream_begin(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        self._ok(self.L.coli_vk_stream_begin(_ptr(x), x.size), "coli_vk_stream_begin")

    def stream_end(self, D, read=True):
        x = np.empty(D, np.float32) if read else None
        self._ok(self.L.coli_vk_stream_end(_ptr(x), D), "coli_vk_stream_end")
        return x

    def gqa_route_pipe(self, layer, tq, tk, tv, to, router, ln_layer, topk, H, KH, hd, rot, pos, max_t, eps, theta):
        idx = np.full(topk, -1, np.int32)
        val = np.zeros(topk, np.float32)
        self._ok(self.L.coli_vk_gqa_full_route_pipe(layer, tq.I, tq.handle, tk.handle, tv.handle, to.handle,
                                                    router.handle, ln_layer, _ptr(idx), _ptr(val), topk, H, KH, hd,
                                                    rot, pos, max_t, eps, theta, to.O, router.O),
                 "coli_vk_gqa_full_route_pipe")
        return idx, val

    def gdn_route_pipe(self, layer, tqkv, tz, ta, tb, tout, router, ln_layer, topk, KH, KD, VH, VD, CD, K, eps):
        idx = np.full(topk, -1, np.int32)
        val = np.zeros(topk, np.float32)
        self._ok(self.L.coli_vk_gdn_full_route_pipe(layer, tqkv.I, tqkv.handle, tz.handle, ta.handle, tb.handle,
                                                    tout.handle, router.handle, ln_layer, _ptr(idx), _ptr(val), topk,
                                                    KH, KD, VH, VD, CD, K, eps, tout.O, router.O),
                 "coli_vk_gdn_full_route_pipe")
        return idx, val

    def stream_moe_fused(self):
        return bool(self.L.coli_vk_stream_moe_fused())

    def stream_ix_hist(self, layer, K):
        idx = np.full(K, -1, np.int32)
        n = self.L.coli_vk_stream_ix_hist(layer, _ptr(idx), K)
        return idx[:n]

    def stream_nrm(self, D):
        p = self.L.coli_vk_stream_nrm()
        return None if not p else np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (D,)).copy()

    def expert_group_issue_pipe(self, gates, ups, downs, weights):
        g, u, d, r = self._group(gates, ups, downs, [1] * len(gates))
        w = np.ascontiguousarray(weights, dtype=np.float32)
        self._ok(self.L.coli_vk_expert_group_issue_pipe(g, u, d, r, _ptr(w), len(gates), gates[0].I),
                 "coli_vk_expert_group_issue_pipe")
        self._ok(self.L.coli_vk_expert_group_take_pipe(), "coli_vk_expert_group_take_pipe")

    def final_norm_weight(self, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        self._ok(self.L.coli_vk_final_norm_weight(_ptr(w), w.size), "coli_vk_final_norm_weight")

    def stream_norm_argmax(self, t, eps):
        idx, val = C.c_int(), C.c_float()
        self._ok(self.L.coli_vk_stream_norm_argmax(t.ref, None, None, t.fmt, t.I, t.O, t.gs, eps, C.byref(idx),
                                                   C.byref(val)), "coli_vk_stream_norm_argmax")
        return idx.value, val.value

    def stream_copy_resid(self, D):
        x = np.empty(D, np.float32)
        self._ok(self.L.coli_vk_stream_copy_resid(_ptr(x), D), "coli_vk_stream_copy_resid")
        return x
