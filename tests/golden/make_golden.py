#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ by running the reference's OWN CPU
kernels - c/qwen.c compiled unmodified from the reference checkout into
oracle/_ref/libqwenref.so (oracle/Makefile target `ref`) - on seeded synthetic inputs.

Inputs are regenerated from their seeds by the shared synthetic-data spec (the tests
check a SHA-256 of every regenerated input before comparing); each fixture stores the
seeds, shapes, input digests and the reference's outputs, so the fixtures are data only.

Run (in a container with the reference checkout):  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import _layers  # noqa: E402
import _util  # noqa: E402
from _util import P, eptr  # noqa: E402


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def gemv_cases(ref, gen):
    out = {}
    for name, (O, I, gs, seed) in {
        "cfg0": (4096, 2048, 128, 0xC0),
        "odd_I": (37, 129, 32, 0xC3),
        "ragged_group": (21, 250, 64, 0xC4),
        "gs8": (16, 100, 8, 0xC5),
        "expert_down": (2048, 512, 128, 0xC6),
    }.items():
        q, sz = gen.fmt6(O, I, gs, seed)
        x = gen.normal(I, gen.stream(seed, 7))
        y = np.empty(O, np.float32)
        ref.ref_matmul_q4g_asym(P(y), P(x), P(q), P(sz), I, O, gs)
        out[f"gemv_{name}"] = dict(O=O, I=I, gs=gs, seed=seed, digest=digest(q, sz, x), y=y)
    return out


def dense_cases(ref, gen):
    out = {}
    # f32 router: W [256, 2048] ~ N(0, 0.02), 3 rows of x
    O, I, S, seed = 256, 2048, 3, 0xD0
    W = gen.f32rows(O, I, seed, 0.02)
    x = gen.normal(S * I, gen.stream(seed, 7))
    y = np.empty(S * O, np.float32)
    ref.ref_matmul(P(y), P(x), P(W), S, I, O)
    out["matmul_f32"] = dict(O=O, I=I, S=S, seed=seed, digest=digest(W, x), y=y)
    # startup quantizers: fmt 6 (gs 128) and fmt 1 of W, then the fmt 1 GEMV
    q6 = np.empty(O * I // 2, np.uint8)
    s6 = np.empty(O * (I // 128) * 2, np.float32)
    ref.ref_quant_rows(P(W), I, O, 6, 128, P(q6), P(s6))
    q1 = np.empty(O * I, np.uint8)
    s1 = np.empty(O, np.float32)
    ref.ref_quant_rows(P(W), I, O, 1, 0, P(q1), P(s1))
    y1 = np.empty(O, np.float32)
    ref.ref_matmul_q8(P(y1), P(x), P(q1), P(s1), I, O)
    out["quant_rows"] = dict(O=O, I=I, seed=seed, digest=digest(W, x), q6=q6, s6=s6, q1=q1, s1=s1, y1=y1)
    # rmsnorm_zc
    D = 2048
    xr = gen.normal(D, 0xD1)
    w = gen.normal(D, 0xD2, 0.1)
    yr = np.empty(D, np.float32)
    ref.ref_rmsnorm_zc(P(yr), P(xr), P(w), D, np.float32(1e-6))
    out["rmsnorm_zc"] = dict(D=D, digest=digest(xr, w), y=yr)
    # softmax_row
    lg = gen.normal(256, 0xD3, 0.9)
    pr = lg.copy()
    ref.ref_softmax_row(P(pr), 256)
    out["softmax_row"] = dict(n=256, digest=digest(lg), p=pr)
    return out


def moe_cases(ref, gen):
    out = {}
    specs = {
        # name: (D, I, E, K, gs, base, tokens)
        "small": (256, 64, 32, 8, 32, 0xE0, 8),
        "cfg2": (2048, 512, 256, 8, 128, 0xE2, 2),
    }
    for name, (D, I, E, K, gs, base, T) in specs.items():
        mw = _util.MoeWeights(gen, base, D, I, E, gs)
        ex = mw.orc_experts()
        xs = gen.normal(T * D, gen.stream(base, 5))
        outs, usage = [], []
        for t in range(T):
            o = np.empty(D, np.float32)
            u = np.zeros(E, np.uint32)
            x = xs[t * D:(t + 1) * D].copy()
            ref.ref_moe_token(P(x), P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(o), P(u))
            outs.append(o)
            usage.append(u)
        xe = xs[:D].copy()
        ye = np.empty(D, np.float32)
        ref.ref_expert_mlp_fmt6(eptr(ex, 3), P(xe), D, I, gs, P(ye))
        out[f"moe_token_{name}"] = dict(D=D, I=I, E=E, K=K, gs=gs, base=base, T=T,
                                         digest=digest(mw.router, mw.sh_gate, xs), out=np.stack(outs),
                                         usage=np.stack(usage), expert3_y=ye)
    # prefill grouping (moe_batch), small shape, S tokens
    D, I, E, K, gs, base, S = 256, 64, 32, 8, 32, 0xE4, 24
    mw = _util.MoeWeights(gen, base, D, I, E, gs)
    ex = mw.orc_experts()
    xs = gen.normal(S * D, gen.stream(base, 5))
    o = np.empty(S * D, np.float32)
    u = np.zeros(E, np.uint32)
    ref.ref_moe_batch(P(xs), S, P(mw.router), eptr(ex), eptr(ex, E), P(mw.sh_gate), D, I, E, K, gs, P(o), P(u))
    out["moe_batch_small"] = dict(D=D, I=I, E=E, K=K, gs=gs, base=base, S=S,
                                  digest=digest(mw.router, mw.sh_gate, xs), out=o, usage=u)
    return out


# GQA / GDN layer blocks: (shape..., base, tokens); the reference runs the tokens in order
# from a zeroed KV cache / recurrent state, so the later outputs depend on the earlier.
GQA_SPECS = {
    "small": dict(D=256, H=4, KH=2, hd=64, rot=16, gs=32, max_t=8, base=0x6A, T=6),
    "cfg3": dict(D=2048, H=16, KH=2, hd=256, rot=64, gs=128, max_t=4096, base=0x6C, T=3),
}
GDN_SPECS = {
    "small": dict(D=256, KH=2, KD=32, VH=4, VD=32, K=4, gs=32, base=0x6B, T=4),
    "cfg3": dict(D=2048, KH=16, KD=128, VH=32, VD=128, K=4, gs=128, base=0x6D, T=2),
}


def layer_cases(ref, gen):
    out = {}
    for name, sp in GQA_SPECS.items():
        W = _layers.GqaWeights(gen, sp["base"], sp["D"], sp["H"], sp["KH"], sp["hd"], sp["rot"], sp["gs"])
        cache = W.new_cache(sp["max_t"])
        xs = gen.normal(sp["T"] * sp["D"], gen.stream(sp["base"], 50))
        ys = [W.reference(ref, cache, sp["max_t"], t, xs[t * sp["D"]:(t + 1) * sp["D"]].copy()) for t in range(sp["T"])]
        extra = dict(K=cache[0], V=cache[1]) if name == "small" else {}
        out[f"layer_gqa_{name}"] = dict(**sp, digest=digest(W.q.q, W.o.sz, W.qn, W.kn, xs), out=np.stack(ys),
                                        **extra)
    for name, sp in GDN_SPECS.items():
        W = _layers.GdnWeights(gen, sp["base"], sp["D"], sp["KH"], sp["KD"], sp["VH"], sp["VD"], sp["K"], sp["gs"])
        st = W.new_state()
        xs = gen.normal(sp["T"] * sp["D"], gen.stream(sp["base"], 50))
        ys = [W.reference(ref, st, xs[t * sp["D"]:(t + 1) * sp["D"]].copy()) for t in range(sp["T"])]
        extra = dict(conv=st[0], S=st[1]) if name == "small" else dict(state_digest=digest(st[0], st[1]))
        out[f"layer_gdn_{name}"] = dict(**sp, digest=digest(W.qkv.q, W.out.sz, W.a.w, W.conv, xs), out=np.stack(ys),
                                        **extra)
    return out


def main():
    ref = _util.load_ref()
    if ref is None:
        sys.exit("oracle/_ref/libqwenref.so missing: build it with `make -C oracle ref`")
    orc = _util.load_oracle()
    _layers.bind(orc, ref)
    gen = _util.Gen(orc)
    cases = {}
    cases.update(gemv_cases(ref, gen))
    cases.update(dense_cases(ref, gen))
    cases.update(moe_cases(ref, gen))
    cases.update(layer_cases(ref, gen))
    for name, d in cases.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **{k: np.asarray(v) for k, v in d.items()})
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
