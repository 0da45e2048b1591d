"""Failure handling of the drop-in ABI on the GPU, forced from the host so that every kernel
still exits normally (c/backend_vulkan.c:1094-1124,1280: a failed wait disables the device,
every later call returns 0 and the engine computes on the CPU).

Each case runs in a child process: a sticky failure disables the library for the rest of
its process, which must not be the test session's.
  - a MoE error word set before a fused layer: the stream entry points that read the
    residual back (stream_end, stream_norm_argmax, stream_copy_resid) return 0 and the
    device stays disabled;
  - COLI_HIP_FAIL_AFTER=n: the (n+1)-th checked call reports a device loss, and every
    later call returns 0.
"""
import os
import subprocess
import sys
import textwrap

import pytest

pytestmark = pytest.mark.gpu
TESTS = os.path.dirname(os.path.abspath(__file__))


def _child(body, env=None, timeout=240):
    code = textwrap.dedent("""
        import sys
        sys.path.insert(0, %r)
        import numpy as np
        import _util
        mod = _util.load_product()
        lib = mod.Lib().init()
        orc = _util.load_oracle()
        gen = _util.Gen(orc)
    """ % TESTS) + textwrap.dedent(body)
    e = dict(os.environ)
    e.update(env or {})
    r = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0, r.returncode
    return r.stdout


@pytest.mark.parametrize("argmax_first", [False, True])
def test_moe_give_up_disables_stream(argmax_first):
    """The engine's order (stream_end, then stream_norm_argmax) and the reverse: whichever
    call reads back first after the failing launches reports it (the error words ride on its
    read-back), and every later call returns 0."""
    out = _child("""
        argmax_first = %r
        import _stack, _layers
        from _moe import Layer
        L = Layer(lib, gen, 0xF100, 256, 128, 32, 64)
        lib.eg_table_init(4, L.E, L.D, L.I, L.gs)
        for l in range(4):
            L.register(lib, l)
        st = _stack.Stack(lib, gen, 0xF110, 4, 256, dict(H=4, KH=2, hd=64, rot=16, gs=64),
                          dict(KH=2, KD=64, VH=4, VD=32, K=4, gs=64), L, max_t=16)
        lm = lib.tensor(*gen.fmt6(512, 256, 64, 0xF120), 6, 256, 512, 64)
        lib.final_norm_weight(gen.normal(256, 0xF121, 0.1))
        # a clean token first: every call succeeds
        lib.stream_begin(gen.normal(256, 0xF122))
        for i in range(4):
            st.pipe_layer(lib, i, 0, 8, L.router)
        assert lib.L.coli_vk_stream_end(None, 256) == 1
        idx, val = lib.stream_norm_argmax(lm, 1e-6)
        assert 0 <= idx < 512
        assert lib.moe_error() == 0
        # the error word set from the host: the fused layers' waits give up
        lib.stream_begin(gen.normal(256, 0xF123))
        lib.moe_force_error(1)
        for i in range(4):
            st.pipe_layer(lib, i, 1, 8, L.router)
        import ctypes as C
        i2, v2 = C.c_int(-7), C.c_float()
        if argmax_first:
            r_arg = lib.L.coli_vk_stream_norm_argmax(lm.ref, None, None, 6, 256, 512, 64, 1e-6, C.byref(i2), C.byref(v2))
            r_end = lib.L.coli_vk_stream_end(None, 256)
        else:
            r_end = lib.L.coli_vk_stream_end(None, 256)
            r_arg = lib.L.coli_vk_stream_norm_argmax(lm.ref, None, None, 6, 256, 512, 64, 1e-6, C.byref(i2), C.byref(v2))
        x = np.empty(256, np.float32)
        r_cp = lib.L.coli_vk_stream_copy_resid(_util.P(x), 256)
        print("results", r_end, r_arg, r_cp, i2.value, lib.available(), flush=True)
        assert r_end == 0 and r_arg == 0 and r_cp == 0 and i2.value == -7
        assert not lib.available()
        print("ok", flush=True)
    """ % argmax_first)
    assert "ok" in out


def test_fail_after_is_sticky():
    out = _child("""
        q, sz = gen.fmt6(64, 256, 64, 0xF200)
        x = gen.normal(256, 0xF201)
        t = lib.tensor(q, sz, 6, 256, 64, 64)   # checked calls 1-2 (ensure + upload)
        import ctypes as C
        y = np.empty(64, np.float32)
        rs = []
        for n in range(6):
            rs.append(lib.L.coli_vk_matmul(t.ref, _util.P(y), _util.P(x), None, None, 6, 1, 256, 64, 64))
        print("results", rs, lib.available(), flush=True)
        assert rs[0] == 1 and rs[-1] == 0 and not lib.available()
        k = rs.index(0)
        assert all(r == 0 for r in rs[k:])
        print("ok", flush=True)
    """, env={"COLI_HIP_FAIL_AFTER": "3"})
    assert "ok" in out
