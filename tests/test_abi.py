"""The drop-in boundary: libcoli_hip.so exports every entry point include/coli_hip.h
declares, the declarations match the reference's c/backend_vulkan.h signature for
signature, and the reference engine c/qwen.c links against the library unchanged.
(No device calls: these run on CPU-only hosts.)
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

import _util

ROOT = _util.ROOT
HDR = os.path.join(ROOT, "include", "coli_hip.h")
LIB = os.path.join(ROOT, "qwen3.c_amd", "libcoli_hip.so")
REF_C = "/root/reference/c"


def declared():
    txt = open(HDR).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(coli_(?:vk|hip)_[a-z0-9_]+)\s*\(", txt)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_library_built():
    assert os.path.exists(LIB), "run __graft_entry__.build()"


def test_every_declared_symbol_exported():
    names = declared()
    assert len(names) >= 70
    missing = [n for n in names if n not in exported()]
    assert not missing, missing


def test_no_undeclared_exports():
    extra = sorted(n for n in exported() if n.startswith("coli_") and n not in declared())
    assert not extra, extra


@pytest.mark.skipif(not os.path.isdir(REF_C), reason="reference checkout absent")
def test_signatures_match_reference_header():
    """Both headers in one translation unit: any differing prototype is a compile error."""
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "sig.c")
        with open(src, "w") as f:
            f.write(f'#include "{REF_C}/backend_vulkan.h"\n#include "{HDR}"\nint main(void) {{ return 0; }}\n')
        r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-c", src, "-o", os.path.join(d, "sig.o")],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.isdir(REF_C) or shutil.which("gcc") is None, reason="reference checkout absent")
def test_reference_engine_links():
    """c/qwen.c built with -DCOLI_VULKAN (c/Makefile:48-53) resolves every coli_vk_* call
    against libcoli_hip.so."""
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "qwen")
        cmd = ["gcc", "-O1", "-std=c11", "-D_GNU_SOURCE", "-include", "sys/resource.h", "-DCOLI_VULKAN",
               f"-I{REF_C}", "-w", "-o", exe, f"{REF_C}/qwen.c", f"{REF_C}/qwen_opts.c",
               f"-L{os.path.dirname(LIB)}", "-lcoli_hip", "-lm"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 (or a WORLD_SIZE above 1) exits with status 2
    and a message, before it touches a device."""
    env = dict(os.environ, WORLD_SIZE="1")
    r = subprocess.run(["python3", os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       env=env, timeout=120)
    assert r.returncode == 2 and "one GPU only" in r.stderr
    env["WORLD_SIZE"] = "2"
    r = subprocess.run(["python3", os.path.join(ROOT, "bench.py")], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 2 and "one GPU only" in r.stderr
