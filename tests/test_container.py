"""The fmt=6 container reader's host side (no device): shard index, header checks and the
float / raw reads of coli_hip_st_* (c/st.h:120-456), against files written by the
safetensors package and by hand.

- Files from safetensors.numpy.save_file (the writer c/tools/convert_qwen35_moe.py uses):
  every tensor found with the dtype, shape and byte count the package reports, and read
  back bit for bit; BF16 (which numpy cannot hold) from a hand-written file.
- F16 -> F32 conversion on all 65536 bit patterns against numpy's.
- Shards: names from every *.safetensors file of the directory; a duplicate name resolves
  to the first file in name order; other files are ignored.
- Each header rule of c/st.h:241-331 broken once (and a few the JSON grammar adds): the
  open is refused, the process survives.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest
from safetensors import safe_open
from safetensors.numpy import save_file

import _util

ql = _util.load_product()


@pytest.fixture(scope="module")
def lib():
    """The product library without a device: the index and the reads are host code."""
    return ql.Lib()


def _raw_file(path, header, data=b"", hlen=None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if hlen is None else hlen))
        f.write(h)
        f.write(data)


def _st(path, tensors):
    """Hand-written safetensors file: tensors = {name: (dtype, shape, bytes)}."""
    hdr, blob = {}, b""
    for name, (dt, shape, b) in tensors.items():
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [len(blob), len(blob) + len(b)]}
        blob += b
    _raw_file(path, hdr, blob)


def test_safetensors_package_file(lib, tmp_path):
    rng = np.random.default_rng(1)
    arrs = {
        "model.layers.0.mlp.experts.0.gate_proj.weight": rng.integers(0, 256, (64, 128), dtype=np.uint8),
        "model.layers.0.mlp.experts.0.gate_proj.weight.qs": rng.normal(size=(64, 4)).astype(np.float32),
        "model.norm.weight": rng.normal(size=(256,)).astype(np.float32),
        "half": rng.normal(size=(3, 5, 7)).astype(np.float16),
        "empty": np.zeros((0, 4), np.float32),
    }
    save_file(arrs, str(tmp_path / "out-layer-00.safetensors"), metadata={"format": "np"})
    st = ql.Container(lib, str(tmp_path))
    assert len(st) == len(arrs)
    with safe_open(str(tmp_path / "out-layer-00.safetensors"), framework="np") as f:
        for name in f.keys():
            a = f.get_tensor(name)
            dt, ne, nb, shape = st.find(name)
            assert shape == a.shape and ne == a.size and nb == a.nbytes, name
            assert dt == {np.dtype(np.uint8): "U8", np.dtype(np.float32): "F32", np.dtype(np.float16): "F16"}[a.dtype]
            raw = st.read_raw(name, nb)
            assert raw is not None and raw.tobytes() == a.tobytes()
            if a.dtype != np.uint8:
                v = st.read_f32(name, max(ne, 1))
                assert v is not None and np.array_equal(v, a.astype(np.float32).ravel())
    assert st.find("absent") is None
    # caps: a read larger than the caller's buffer is refused; U8 is not a float tensor
    assert st.read_f32("model.norm.weight", 255) is None
    assert st.read_raw("model.norm.weight", 1023) is None
    assert st.read_f32("model.layers.0.mlp.experts.0.gate_proj.weight", 1 << 20) is None


def test_bf16_and_f16_conversion(lib, tmp_path):
    bits = np.arange(65536, dtype=np.uint16)
    _st(tmp_path / "a.safetensors", {"b": ("BF16", [65536], bits.tobytes()), "h": ("F16", [256, 256], bits.tobytes())})
    st = ql.Container(lib, str(tmp_path))
    b = st.read_f32("b", 65536)
    ref_b = (bits.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(b.view(np.uint32), ref_b.view(np.uint32))
    h = st.read_f32("h", 65536)
    ref_h = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref_h)
    assert np.array_equal(np.isnan(h), nan)
    assert np.array_equal(h[~nan].view(np.uint32), ref_h[~nan].view(np.uint32))


def test_shards_and_duplicates(lib, tmp_path):
    one = np.arange(4, dtype=np.float32)
    _st(tmp_path / "model-00001-of-00002.safetensors", {"a": ("F32", [4], one.tobytes()),
                                                         "dup": ("F32", [4], one.tobytes())})
    _st(tmp_path / "model-00002-of-00002.safetensors", {"b": ("F32", [2], one[:2].tobytes()),
                                                         "dup": ("F32", [2], one[:2].tobytes())})
    (tmp_path / "config.json").write_text("{}")   # not a shard
    st = ql.Container(lib, str(tmp_path))
    assert len(st) == 3
    assert st.find("a")[3] == (4,) and st.find("b")[3] == (2,)
    assert st.find("dup")[3] == (4,)   # the first shard in name order
    assert np.array_equal(st.read_f32("b", 2), one[:2])


def _ok_hdr():
    return {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}


HOSTILE = {
    "hlen_past_end": dict(hlen=10 ** 6),
    "hlen_huge": dict(hlen=1 << 62),
    "not_json": dict(header=b"{nope"),
    "array_root": dict(header=[1, 2]),
    "trailing": dict(header=json.dumps(_ok_hdr()).encode() + b" x"),
    "missing_dtype": dict(header={"t": {"shape": [2], "data_offsets": [0, 8]}}),
    "dtype_not_string": dict(header={"t": {"dtype": 2, "shape": [2], "data_offsets": [0, 8]}}),
    "offsets_one": dict(header={"t": {"dtype": "F32", "shape": [2], "data_offsets": [0]}}),
    "offsets_reversed": dict(header={"t": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}}),
    "offsets_negative": dict(header={"t": {"dtype": "F32", "shape": [2], "data_offsets": [-8, 0]}}),
    "offsets_past_end": dict(header={"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 9]}}),
    "offsets_float": dict(header={"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8.0]}}),
    "shape_negative": dict(header={"t": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 8]}}),
    "shape_overflow": dict(header={"t": {"dtype": "U8", "shape": [1 << 32, 1 << 32, 4], "data_offsets": [0, 8]}}),
    "shape_not_int": dict(header={"t": {"dtype": "U8", "shape": ["8"], "data_offsets": [0, 8]}}),
    "numel_bytes_mismatch": dict(header={"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}),
    "unknown_dtype": dict(header={"t": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}),
    "deep_nesting": dict(header=b'{"__metadata__":' + b"[" * 40 + b"]" * 40 + b"}"),
    "bad_escape": dict(header=b'{"t\\q": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}'),
    "lone_surrogate": dict(header=b'{"t\\udc00": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}'),
}


@pytest.mark.parametrize("case", sorted(HOSTILE))
def test_hostile_header_refused(lib, tmp_path, case):
    spec = HOSTILE[case]
    _raw_file(tmp_path / "x.safetensors", spec.get("header", _ok_hdr()), b"\0" * 8, spec.get("hlen"))
    with pytest.raises(ValueError):
        ql.Container(lib, str(tmp_path))


def test_truncated_and_empty(lib, tmp_path):
    (tmp_path / "a.safetensors").write_bytes(b"\x10\0\0")   # shorter than the length word
    with pytest.raises(ValueError):
        ql.Container(lib, str(tmp_path))
    os.remove(tmp_path / "a.safetensors")
    with pytest.raises(ValueError):   # no shard at all
        ql.Container(lib, str(tmp_path))
    # a well-formed file with escapes and metadata is accepted
    hdr = {"__metadata__": {"k": "vé😀"}, "té": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    _raw_file(tmp_path / "b.safetensors", json.dumps(hdr, ensure_ascii=True).encode(), np.ones(2, np.float32).tobytes())
    st = ql.Container(lib, str(tmp_path))
    assert st.find("té") is not None


_MUT_DATA = bytes(range(40))


def _mutations(n=600):
    """n seeded mutations (byte flips, insertions, truncations) of a valid two-tensor header."""
    hdr = json.dumps({"__metadata__": {"a": "b"}, "w": {"dtype": "U8", "shape": [4, 2], "data_offsets": [0, 8]},
                      "w.qs": {"dtype": "F32", "shape": [4, 2], "data_offsets": [8, 40]}}).encode()
    rng = np.random.default_rng(0xC0FFEE)
    alphabet = b'{}[]":,0123456789-.eE\\u tnrfalsedtype' + bytes([0, 0x7F, 0xC3, 0xFF])
    for _ in range(n):
        h = bytearray(hdr)
        for _ in range(int(rng.integers(1, 4))):
            op, at = int(rng.integers(0, 3)), int(rng.integers(0, len(h)))
            if op == 0:
                h[at] = alphabet[int(rng.integers(0, len(alphabet)))]
            elif op == 1:
                h.insert(at, alphabet[int(rng.integers(0, len(alphabet)))])
            else:
                del h[at:at + int(rng.integers(1, 8))]
        yield bytes(h)


def test_mutated_headers_never_crash(lib, tmp_path):
    """600 seeded mutations of a valid two-tensor header: every open either succeeds or is
    refused; an accepted index still answers find and bounded reads."""
    for h in _mutations():
        _raw_file(tmp_path / "m.safetensors", h, _MUT_DATA)
        try:
            st = ql.Container(lib, str(tmp_path))
        except ValueError:
            continue
        for name in ("w", "w.qs"):
            r = st.find(name)
            if r is not None and r[2] <= 64:
                st.read_raw(name, 64)
        st.close()


def test_reader_under_address_sanitizer(lib, tmp_path):
    """The reader's host side (csrc/st_host.cpp) built alone with -fsanitize=address,undefined
    (tests/st_asan.cpp drives it): the hostile headers, the 600 mutations, truncated shards,
    the BF16 / F16 file and the safetensors package's file are opened and every indexed tensor
    read.  No sanitizer report, and each directory gets the same verdict (open or refused) as
    from the product library."""
    exe = tmp_path / "st_asan"
    src = os.path.join(_util.ROOT, "qwen3.c_amd", "csrc", "st_host.cpp")
    drv = os.path.join(_util.ROOT, "tests", "st_asan.cpp")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                        "-fno-sanitize-recover=undefined", drv, src, "-o", str(exe)], capture_output=True, text=True)
    if r.returncode != 0 and "asan" in (r.stderr or "").lower():
        pytest.skip("no AddressSanitizer runtime for the host compiler")
    assert r.returncode == 0, r.stderr
    dirs = []

    def new_dir():
        d = tmp_path / f"d{len(dirs)}"
        d.mkdir()
        dirs.append(d)
        return d

    for case in sorted(HOSTILE):
        spec = HOSTILE[case]
        _raw_file(new_dir() / "x.safetensors", spec.get("header", _ok_hdr()), b"\0" * 8, spec.get("hlen"))
    for h in _mutations():
        _raw_file(new_dir() / "m.safetensors", h, _MUT_DATA)
    for cut in (1, 3, 8, 20):   # a valid file cut short, inside the length word, header and data
        d = new_dir()
        _raw_file(d / "t.safetensors", _ok_hdr(), np.ones(2, np.float32).tobytes())
        b = (d / "t.safetensors").read_bytes()
        (d / "t.safetensors").write_bytes(b[:min(cut, len(b) - 1)] if cut < 8 else b[:-cut // 4])
    bits = np.arange(65536, dtype=np.uint16)
    _st(new_dir() / "a.safetensors", {"b": ("BF16", [65536], bits.tobytes()), "h": ("F16", [256, 256], bits.tobytes())})
    rng = np.random.default_rng(2)
    save_file({"u": rng.integers(0, 256, (64, 128), dtype=np.uint8), "f": rng.normal(size=(3, 5)).astype(np.float32),
               "e": np.zeros((0, 4), np.float32)}, str(new_dir() / "p.safetensors"))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)] + [str(d) for d in dirs], capture_output=True, text=True, errors="replace", env=env,
                       timeout=300)
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, r.stderr[-4000:]
    verdict = {}
    for line in r.stdout.splitlines():
        word, path = line.split()[:2]
        verdict[path] = word
    assert len(verdict) == len(dirs)
    for d in dirs:
        try:
            ql.Container(lib, str(d)).close()
            want = "open"
        except ValueError:
            want = "refused"
        assert verdict[str(d)] == want, d
    assert sum(v == "open" for v in verdict.values()) >= 3
