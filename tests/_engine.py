"""The reference engine's prefill MoE call sequence over the ABI, restated in Python for the
GPU tests and the bench (the engine itself, c/qwen.c, is C and calls the same entry points).

engine_moe_batch follows moe_batch_from_logits (c/qwen.c:1050-1183) from the routing on:
the (token, slot) pairs are bucketed by expert (:1076-1083), the routed experts go out in
ascending id in chunks of at most MOEB_MAXE experts and MOEB_MAXROWS rows, an expert with
more rows than fit being split and resumed in the next chunk (:1099-1112); each chunk is
one coli_vk_expert_group_issue_id over the bound rows (:1094,1120) and one take, whose rows
are added as out[tok] += w * y (:1024-1027,1133); the shared expert then runs over all S
rows as one coli_vk_expert_group_issue of packed rows and is added with its sigmoid gate
(:1149-1161).  The float32 adds happen in the engine's order, so the result can be compared
with the oracle's restatement of the whole block.
"""
import numpy as np

MOEB_MAXE = 64       # c/qwen.c:1044
MOEB_MAXROWS = 1024  # c/qwen.c:1045


def group_by_expert(tidx, E):
    """(ecnt [E + 1] offsets, epair [S K] pair indices by expert) as c/qwen.c:1076-1083."""
    flat = np.asarray(tidx, np.int64).reshape(-1)
    cnt = np.bincount(flat, minlength=E)
    ecnt = np.zeros(E + 1, np.int64)
    ecnt[1:] = np.cumsum(cnt)
    epair = np.argsort(flat, kind="stable")   # pairs of one expert in pair order
    return ecnt, epair


def chunks(ecnt, E):
    """The engine's chunks: lists of (expert, first row, rows), c/qwen.c:1099-1112."""
    gpu = [e for e in range(E) if ecnt[e + 1] > ecnt[e]]
    out, gi, roff = [], 0, 0
    while gi < len(gpu):
        ch, total = [], 0
        while gi < len(gpu) and len(ch) < MOEB_MAXE and total < MOEB_MAXROWS:
            e = gpu[gi]
            have = int(ecnt[e + 1] - ecnt[e]) - roff
            nr = min(have, MOEB_MAXROWS - total)
            ch.append((e, roff, nr))
            total += nr
            roff += nr
            if roff == ecnt[e + 1] - ecnt[e]:
                gi += 1
                roff = 0
        out.append(ch)
    return out


def plan(tidx, tval, K, E):
    """The engine's chunks as ABI arguments: per chunk (experts, rows, token ids, weights)."""
    tval = np.asarray(tval, np.float32).reshape(-1)
    ecnt, epair = group_by_expert(tidx, E)
    out = []
    for ch in chunks(ecnt, E):
        rtok, rw = [], []
        for e, r0, nr in ch:
            pairs = epair[ecnt[e] + r0:ecnt[e] + r0 + nr]
            rtok.extend((pairs // K).tolist())
            rw.extend(tval[pairs].tolist())
        out.append(([c[0] for c in ch], [c[2] for c in ch], np.asarray(rtok, np.int32), np.asarray(rw, np.float32)))
    return out


def issue_chunks(lib, tensors, xs, S, D, chs, shared=True):
    """The ABI calls alone (c/qwen.c:1094,1120-1121,1149-1152): bind, one issue_id + take per
    chunk, then the shared expert over all S rows.  Returns the y blocks (the last one the
    shared expert's)."""
    E = len(tensors) - 1
    lib.eg_xs_bind(xs, S, D)
    ys = []
    for es, rows, rtok, _ in chs:
        if not lib.expert_group_issue_id([tensors[e][0] for e in es], [tensors[e][1] for e in es],
                                         [tensors[e][2] for e in es], rows, rtok):
            raise RuntimeError("coli_vk_expert_group_issue_id refused a chunk")
        ys.append(lib.expert_group_take(len(rtok), D).reshape(-1, D))
    if shared:
        g, u, d = tensors[E]
        if not lib.expert_group_issue([g], [u], [d], [S], xs):
            raise RuntimeError("coli_vk_expert_group_issue refused the shared expert")
        ys.append(lib.expert_group_take(S, D).reshape(S, D))
    return ys


def issue_chunks_into(lib, tensors, xs, S, D, chs, ybuf):
    """issue_chunks with every take into one host buffer ybuf (at least max rows x D floats):
    the engine allocates and frees its y block per chunk (c/qwen.c:1115,1141,1155), which
    the C heap hands back warm after the first chunk."""
    E = len(tensors) - 1
    lib.eg_xs_bind(xs, S, D)
    for es, rows, rtok, _ in chs:
        if not lib.expert_group_issue_id([tensors[e][0] for e in es], [tensors[e][1] for e in es],
                                         [tensors[e][2] for e in es], rows, rtok):
            raise RuntimeError("coli_vk_expert_group_issue_id refused a chunk")
        lib.expert_group_take_into(ybuf[:len(rtok) * D])
    g, u, d = tensors[E]
    if not lib.expert_group_issue([g], [u], [d], [S], xs):
        raise RuntimeError("coli_vk_expert_group_issue refused the shared expert")
    lib.expert_group_take_into(ybuf[:S * D])


def prepare_chunks(lib, tensors, S, chs):
    """The ctypes arguments of every call issue_chunks_into makes, built once: the engine
    builds its handle arrays in C, so a timing of the library calls leaves this out."""
    E = len(tensors) - 1
    prep = []
    for es, rows, rtok, _ in chs:
        g, u, d, r = lib._group([tensors[e][0] for e in es], [tensors[e][1] for e in es],
                                [tensors[e][2] for e in es], rows)
        prep.append((g, u, d, r, len(es), np.ascontiguousarray(rtok, np.int32)))
    shared = lib._group([tensors[E][0]], [tensors[E][1]], [tensors[E][2]], [S])
    return prep, shared


def issue_prepared(lib, prepared, xs, S, D, ybuf):
    """issue_chunks_into over arguments from prepare_chunks: the same ABI calls in the same
    order (bind, issue_id / take per chunk, the shared expert's issue / take)."""
    import ctypes as C
    L = lib.L
    prep, (sg, su, sd, sr) = prepared
    px, py = xs.ctypes.data_as(C.c_void_p), ybuf.ctypes.data_as(C.c_void_p)
    if not L.coli_vk_eg_xs_bind(px, S, D):
        raise RuntimeError("coli_vk_eg_xs_bind failed")
    for g, u, d, r, n, ids in prep:
        if not L.coli_vk_expert_group_issue_id(g, u, d, r, n, ids.ctypes.data_as(C.c_void_p)):
            raise RuntimeError("coli_vk_expert_group_issue_id refused a chunk")
        if not L.coli_vk_expert_group_take(py):
            raise RuntimeError("coli_vk_expert_group_take failed")
    if not L.coli_vk_expert_group_issue(sg, su, sd, sr, 1, px):
        raise RuntimeError("coli_vk_expert_group_issue refused the shared expert")
    if not L.coli_vk_expert_group_take(py):
        raise RuntimeError("coli_vk_expert_group_take failed")


def engine_moe_batch(lib, tensors, xs, S, D, K, tidx, tval, sh_gate):
    """out [S, D] of the routed experts and the shared expert (tensors[e] = (g, u, d) for
    e < E, tensors[E] the shared expert), through the ABI as the engine calls it."""
    E = len(tensors) - 1
    xs = np.ascontiguousarray(xs, np.float32).reshape(S, D)
    chs = plan(tidx, tval, K, E)
    ys = issue_chunks(lib, tensors, xs, S, D, chs)
    out = np.zeros((S, D), np.float32)
    for (_, _, rtok, rw), y in zip(chs, ys):
        for r, t in enumerate(rtok):   # c/qwen.c:1024-1027,1133: rows in chunk order
            out[t] += rw[r] * y[r]
    y = ys[-1]
    sg = np.asarray(sh_gate, np.float32)
    for s in range(S):
        # c/qwen.c:1158: gt += sh_gate[d] * x[d] in index order (accumulate is sequential)
        gt = np.add.accumulate((sg * xs[s]).astype(np.float32), dtype=np.float32)[-1]
        sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-gt, dtype=np.float32))   # sigmoidf_, c/qwen.c:172
        out[s] += sig * y[s]
    return out
