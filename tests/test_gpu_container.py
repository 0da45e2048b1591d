"""The fmt=6 container reader on the GPU (coli_hip_st_tensor / coli_hip_st_experts, the
path c/qwen.c:509-536 + 1743-1805 takes from c/st.h into coli_vk_tensor_ensure), against
the host-array upload and the oracle.

Containers are written with safetensors.numpy.save_file in the converter's layout
(c/tools/convert_qwen35_moe.py:124-144, 322-330): per projection a U8 [O, ceil(I/2)] tensor
of nibbles and an F32 [O, 2 ceil(I/gs)] ".qs" tensor of [scale, zero] pairs.

Bar: device weights and scales byte-identical to coli_vk_tensor_ensure's from the same
arrays (so every kernel result is too); GEMV within maxrel_scaled 1e-3 of the oracle; the
MoE block from container experts bit-identical to the block from uploaded experts, routing
ids identical to the oracle's and outputs within maxrel_scaled 1e-3.
"""
import json
import struct

import numpy as np
import pytest
from safetensors.numpy import save_file

import _moe
import _util
from _util import P

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _arrays(q, sz, I, O, gs):
    ng = (I + gs - 1) // gs
    return q.reshape(O, (I + 1) // 2), sz.reshape(O, 2 * ng)


def _device_bytes(lib, t):
    """(weights, scales) of a tensor copied back from HBM."""
    info = t.info()
    w = np.empty(info["row_bytes"] * t.O, np.uint8)
    lib.memcpy(w.ctypes.data, info["d_w"], w.nbytes)
    ng = (t.I + t.gs - 1) // t.gs
    s = np.empty(t.O * ng * 2, np.float32)
    lib.memcpy(s.ctypes.data, info["d_sz"], s.nbytes)
    return w, s


@pytest.mark.parametrize("O,I,gs", [(1000, 2048, 128), (300, 301, 32), (257, 200, 8)])
def test_st_tensor_fmt6(lib, orc, gen, tmp_path, O, I, gs):
    """Lanes layout (gs % 32 == 0), an odd I, and the rows layout (gs 8)."""
    mod = _util.load_product()
    q, sz = gen.fmt6(O, I, gs, 0x5C00 + I)
    wq, ws = _arrays(q, sz, I, O, gs)
    save_file({"blk.weight": wq, "blk.weight.qs": ws}, str(tmp_path / "out-dense.safetensors"))
    st = mod.Container(lib, str(tmp_path))
    t_st = st.tensor("blk.weight", 6, I, O, gs)
    t_up = lib.tensor(q, sz, 6, I, O, gs)
    a, b = _device_bytes(lib, t_st), _device_bytes(lib, t_up)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    x = gen.normal(I, 0x5C01)
    y = lib.matmul(t_st, x)
    yo = np.empty(O, np.float32)
    orc.orc_matmul_q4g_asym(P(yo), P(x), P(q), P(sz), I, O, gs)
    assert _util.maxrel_scaled(y, yo) <= TOL
    with pytest.raises(RuntimeError):   # the shape the caller asks for must match the file
        st.tensor("blk.weight", 6, I, O + 1, gs)


def test_st_tensor_fmt0_bf16(lib, orc, gen, tmp_path):
    """A BF16 router [E, D] read as f32 rows: the same device tensor as uploading the
    converted array."""
    mod = _util.load_product()
    E, D = 256, 2048
    f = gen.normal(E * D, 0x5C10, 0.02)
    bf = (f.view(np.uint32) >> 16).astype(np.uint16)
    hdr_path = tmp_path / "r.safetensors"
    h = json.dumps({"mlp.gate.weight": {"dtype": "BF16", "shape": [E, D], "data_offsets": [0, bf.nbytes]}}).encode()
    hdr_path.write_bytes(struct.pack("<Q", len(h)) + h + bf.tobytes())
    st = mod.Container(lib, str(tmp_path))
    t = st.tensor("mlp.gate.weight", 0, D, E)
    fr = (bf.astype(np.uint32) << 16).view(np.float32)
    x = gen.normal(D, 0x5C11)
    y = lib.matmul(t, x)
    assert np.array_equal(y, lib.matmul(lib.tensor(fr, None, 0, D, E), x))
    yo = np.empty(E, np.float32)
    orc.orc_matmul_f32(P(yo), P(x), P(fr), 1, D, E)
    assert _util.maxrel_scaled(y, yo) <= TOL


def _write_experts(path, mw, layer, shards=2):
    """The layer's routed experts in the converter's names, split over `shards` files."""
    names = ("gate_proj", "up_proj", "down_proj")
    per = (mw.E + shards - 1) // shards
    for s in range(shards):
        t = {}
        for e in range(s * per, min(mw.E, (s + 1) * per)):
            for j, (q, sz) in enumerate(mw.exp[e]):
                I, O = (mw.D, mw.I) if j < 2 else (mw.I, mw.D)
                wq, ws = _arrays(q, sz, I, O, mw.gs)
                t[f"model.layers.{layer}.mlp.experts.{e}.{names[j]}.weight"] = wq
                t[f"model.layers.{layer}.mlp.experts.{e}.{names[j]}.weight.qs"] = ws
        save_file(t, str(path / f"out-layer-{layer:02d}-{s}.safetensors"))


def test_st_experts_moe_block(lib, orc, gen, torch_dev, tmp_path):
    """64 experts (D 2048, I 512, gs 128: configs[2]'s expert shapes) of model layer 3 from
    a two-shard container into the table; the MoE block over them bit-identical to the
    block over the same experts uploaded from host arrays, and against the oracle."""
    import torch
    mod = _util.load_product()
    D, I, E, gs, K, layer = 2048, 512, 64, 128, 8, 3
    L = _moe.Layer(lib, gen, 0x5D00, D, I, E, gs)
    _write_experts(tmp_path, L.mw, layer)
    st = mod.Container(lib, str(tmp_path))
    _moe._active[0] = None
    lib.eg_table_init(layer + 2, E, D, I, gs)
    st.experts(layer, E, D, I, gs)
    lib.eg_table_set_shared(layer, *L.t[E], L.mw.sh_gate)
    L.register(lib, layer + 1)   # the same experts uploaded from host arrays
    for i in range(3):
        x = gen.normal(D, 0x5D10 + i)
        dx = torch.from_numpy(x).to(torch_dev)
        outs, ids = [], []
        for ly in (layer, layer + 1):
            out = torch.zeros(D, device=torch_dev)
            di = torch.full((K,), -1, dtype=torch.int32, device=torch_dev)
            torch.cuda.synchronize()
            lib.moe_decode_dev(ly, L.router, K, dx.data_ptr(), out.data_ptr(), False, di.data_ptr(), None)
            lib.sync()
            outs.append(out.cpu().numpy())
            ids.append(di.cpu().numpy())
        assert np.array_equal(outs[0], outs[1]) and np.array_equal(ids[0], ids[1])
        ro, oi, _, _ = L.oracle(orc, x, K)
        assert np.array_equal(ids[0], oi)
        assert _util.maxrel_scaled(outs[0], ro) <= TOL
    assert lib.moe_error() == 0
    _moe._active[0] = None


def test_st_experts_refuses_wrong_container(lib, gen, tmp_path):
    """A down projection one byte short (c/qwen.c:522-525's check): nothing is uploaded
    for the layer and the call reports failure; the device stays usable."""
    mod = _util.load_product()
    D, I, E, gs, layer = 256, 128, 4, 64, 0
    mw = _util.MoeWeights(gen, 0x5E00, D, I, E, gs)
    _write_experts(tmp_path, mw, layer, shards=1)
    name = f"model.layers.{layer}.mlp.experts.2.down_proj.weight"
    from safetensors.numpy import load_file
    f = tmp_path / f"out-layer-{layer:02d}-0.safetensors"
    t = load_file(str(f))
    t[name] = t[name][:, :-1].copy()
    save_file(t, str(f))
    st = mod.Container(lib, str(tmp_path))
    _moe._active[0] = None
    lib.eg_table_init(1, E, D, I, gs)
    with pytest.raises(RuntimeError):
        st.experts(layer, E, D, I, gs)
    assert lib.available()


def test_st_experts_failure_releases_uploads(lib, gen, tmp_path):
    """A shard cut short after it was indexed, under the last expert of a layer whose reads
    need two batches (64 configs[2] experts, ~113 MB): the first batch is already on the
    device when the read fails.  The call returns 0 and the library's tensor count and bytes
    are back where they were; a table of the wrong shape is refused before any upload; the
    device stays usable and the intact layer then loads."""
    mod = _util.load_product()
    D, I, E, gs, layer = 2048, 512, 64, 128, 5
    mw = _util.MoeWeights(gen, 0x5F00, D, I, E, gs)
    _write_experts(tmp_path, mw, layer, shards=2)
    st = mod.Container(lib, str(tmp_path))
    _moe._active[0] = None
    lib.eg_table_init(layer + 1, E, D, 2 * I, gs)   # wrong I: refused up front
    before = lib.mem_info()
    with pytest.raises(RuntimeError):
        st.experts(layer, E, D, I, gs)
    assert lib.mem_info() == before
    lib.eg_table_init(layer + 1, E, D, I, gs)
    shard = tmp_path / f"out-layer-{layer:02d}-1.safetensors"
    full = shard.read_bytes()
    shard.write_bytes(full[:len(full) - 4096])   # the index was built from the whole file
    with pytest.raises(RuntimeError):
        st.experts(layer, E, D, I, gs)
    assert lib.mem_info() == before
    assert lib.available()
    shard.write_bytes(full)
    st.experts(layer, E, D, I, gs)
    assert lib.mem_info()[1] == before[1] + 3 * E
    _moe._active[0] = None


def test_st_tensor_half_scales(lib, orc, gen, tmp_path):
    """A .qs tensor stored as F16 (c/qwen.c:528-534 reads it through st_read_f32, which
    converts): the same device tensor as the upload of the converted f32 scales."""
    mod = _util.load_product()
    O, I, gs = 512, 2048, 128
    q, sz = gen.fmt6(O, I, gs, 0x5F10)
    sz16 = sz.astype(np.float16)
    wq, ws = _arrays(q, sz16.astype(np.float32), I, O, gs)
    save_file({"h.weight": wq, "h.weight.qs": ws.astype(np.float16)}, str(tmp_path / "h.safetensors"))
    st = mod.Container(lib, str(tmp_path))
    t_st = st.tensor("h.weight", 6, I, O, gs)
    t_up = lib.tensor(q, sz16.astype(np.float32), 6, I, O, gs)
    a, b = _device_bytes(lib, t_st), _device_bytes(lib, t_up)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
