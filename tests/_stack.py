"""A hybrid decode stack for the GPU tests: n layers, GatedDeltaNet except every 4th
(c/qwen.c:398: is_full = (i + 1) % 4 == 0), each followed by the MoE block; host weights for
the oracle, the same weights uploaded to the library.

The oracle composition of a layer is c/qwen.c:1340-1352:
  x = rmsnorm_zc(resid, in_ln); resid += block(x); nrm = rmsnorm_zc(resid, post_ln);
  resid += moe(nrm)
"""
import numpy as np

import _layers
from _util import P


def rms(orc, x, w, eps):
    y = np.empty_like(x)
    orc.orc_rmsnorm_zc(P(y), P(x), P(w), x.size, np.float32(eps))
    return y


class Stack:
    def __init__(self, lib, gen, base, n_layers, D, gqa, gdn, moe_layer, max_t, ab_fmt=6, first_layer=0,
                 router_f=None, kv_rows=0, state_base=0):
        """gqa: dict(H, KH, hd, rot, gs); gdn: dict(KH, KD, VH, VD, K, gs); moe_layer: a tests/_moe.py
        Layer whose experts every layer shares (each layer keeps its own norms).  router_f:
        the f32 rows the oracle routes with (the exact equivalent of an int8 router; default
        the layer's f32 router).  kv_rows > 0: every attention cache is seeded with that many
        random rows (device and oracle alike), so decoding starts deep in the window.
        state_base: first KV-mirror / GDN-state index of the stack (the library keys that
        state by index and refuses other dimensions for an index already in use)."""
        self.D, self.max_t, self.moe, self.router_f = D, max_t, moe_layer, router_f
        self.eps = np.float32(1e-6)
        self.layers = []
        kvi = gi = state_base
        for i in range(n_layers):
            seed = gen.stream(base, 100 + i)
            if (i + 1) % 4 == 0:
                W = _layers.GqaWeights(gen, seed, D, gqa["H"], gqa["KH"], gqa["hd"], gqa["rot"], gqa["gs"])
                t = [m.upload(lib) for m in (W.q, W.k, W.v, W.o)]
                lib.kv_ensure(kvi, W.KH * max_t, W.hd, W.hd)
                lib.gqa_norm_weight(kvi, W.qn, W.kn)
                cache = W.new_cache(max_t)
                if kv_rows:
                    for h in range(W.KH):   # rows [h * max_t, h * max_t + kv_rows)
                        kr = gen.normal(kv_rows * W.hd, gen.stream(seed, 50 + h), 1.0)
                        vr = gen.normal(kv_rows * W.hd, gen.stream(seed, 60 + h), 1.0)
                        r0 = h * max_t * W.hd
                        cache[0][r0:r0 + kv_rows * W.hd] = kr
                        cache[1][r0:r0 + kv_rows * W.hd] = vr
                        lib.kv_load(kvi, h * max_t, kr.reshape(kv_rows, W.hd), vr.reshape(kv_rows, W.hd))
                self.layers.append(dict(kind="gqa", W=W, t=t, idx=kvi, cache=cache))
                kvi += 1
            else:
                W = _layers.GdnWeights(gen, seed, D, gdn["KH"], gdn["KD"], gdn["VH"], gdn["VD"], gdn["K"], gdn["gs"],
                                       ab_fmt=ab_fmt)
                t = [m.upload(lib) for m in (W.qkv, W.z, W.a, W.b, W.out)]
                lib.gdn_setup(gi, W.VH, W.KD, W.VD, W.K, W.CD, W.conv, W.alog, W.dtb, W.gnorm)
                self.layers.append(dict(kind="gdn", W=W, t=t, idx=gi, state=W.new_state()))
                gi += 1
            lib.layer_norm_weight(first_layer + i, W.in_ln, W.post_ln)
        self.first = first_layer
        lib.gdn_reset()

    # ---- oracle ---------------------------------------------------------------------
    def oracle_layer(self, orc, i, resid, pos, K):
        L = self.layers[i]
        W = L["W"]
        x = rms(orc, resid, W.in_ln, self.eps)
        out = W.oracle(orc, L["cache"], self.max_t, pos, x) if L["kind"] == "gqa" else W.oracle(orc, L["state"], x)
        resid = (resid + out).astype(np.float32)
        nrm = rms(orc, resid, W.post_ln, self.eps)
        moe, idx, val, _ = self.moe.oracle(orc, nrm, K, router=self.router_f)
        return (resid + moe).astype(np.float32), nrm, idx, val

    # ---- device (stream route_pipe) ---------------------------------------------------
    def pipe_layer(self, lib, i, pos, K, router):
        L = self.layers[i]
        W = L["W"]
        if L["kind"] == "gqa":
            tq, tk, tv, to = L["t"]
            return lib.gqa_route_pipe(L["idx"], tq, tk, tv, to, router, self.first + i, K, W.H, W.KH, W.hd, W.rot,
                                      pos, self.max_t, W.eps, W.theta)
        tqkv, tz, ta, tb, tout = L["t"]
        return lib.gdn_route_pipe(L["idx"], tqkv, tz, ta, tb, tout, router, self.first + i, K, W.KH, W.KD, W.VH, W.VD,
                                  W.CD, W.K, W.eps)
