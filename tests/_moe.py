"""MoE layers for the GPU tests: host weights for the oracle plus the uploaded tensors and
the library's expert table (coli_vk_eg_table_*)."""
import numpy as np

import _util
from _util import P, eptr


class Layer:
    """Host weights (oracle side) + uploaded tensors (device side) of one MoE layer."""

    def __init__(self, lib, gen, base, D, I, E, gs, layer=0, router_fmt=0):
        self.mw = _util.MoeWeights(gen, base, D, I, E, gs, layer)
        self.ex = self.mw.orc_experts()
        self.D, self.I, self.E, self.gs = D, I, E, gs
        self.t = []
        for g, u, d in self.mw.exp:
            self.t.append((lib.tensor(g[0], g[1], 6, D, I, gs), lib.tensor(u[0], u[1], 6, D, I, gs),
                           lib.tensor(d[0], d[1], 6, I, D, gs)))
        self.router = lib.tensor(self.mw.router, None, 0, D, E)

    def int8_router(self, lib, gen, base):
        """An int8 (fmt 1) router [E, D] uploaded, and its exact f32 equivalent q * s
        (_util.int8_rows)."""
        q, s, f = _util.int8_rows(gen, base, self.E, self.D)
        return lib.tensor(q.view(np.uint8).reshape(-1), s, 1, self.D, self.E), f

    def register(self, lib, layer):
        for e in range(self.E):
            lib.eg_table_set(layer, e, *self.t[e])
        lib.eg_table_set_shared(layer, *self.t[self.E], self.mw.sh_gate)

    def oracle(self, orc, x, K, router=None):
        out = np.empty(self.D, np.float32)
        idx = np.empty(K, np.int32)
        val = np.empty(K, np.float32)
        shgt = np.empty(1, np.float32)
        orc.orc_moe_decode(P(x), P(self.mw.router if router is None else router), eptr(self.ex), eptr(self.ex, self.E), P(self.mw.sh_gate),
                           self.D, self.I, self.E, K, self.gs, P(out), P(idx), P(val), P(shgt), None)
        return out, idx, val, float(shgt[0])

    def oracle_prefill(self, orc, xs, S, K, router=None):
        """moe_batch_from_logits (c/qwen.c:1050-1183) restated: out [S, D], ids/weights [S, K]."""
        out = np.empty(S * self.D, np.float32)
        tidx = np.empty(S * K, np.int32)
        tval = np.empty(S * K, np.float32)
        orc.orc_moe_prefill(P(xs), S, P(self.mw.router if router is None else router), eptr(self.ex), eptr(self.ex, self.E), P(self.mw.sh_gate),
                            self.D, self.I, self.E, K, self.gs, P(out), P(tidx), P(tval))
        return out, tidx, tval


_active = [None]


class Table(list):
    """Layers of one expert table.  The library holds one table: activate() re-creates it
    (coli_vk_eg_table_init) when another test's table is current."""

    def __init__(self, lib, layers):
        super().__init__(layers)
        self.lib = lib

    def activate(self):
        if _active[0] is not self:
            L0 = self[0]
            self.lib.eg_table_init(len(self), L0.E, L0.D, L0.I, L0.gs)
            for l, L in enumerate(self):
                L.register(self.lib, l)
            _active[0] = self
        return self
