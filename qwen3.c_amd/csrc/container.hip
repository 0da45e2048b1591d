// container.hip - the device side of the fmt=6 container reader: safetensors shards written
// by c/tools/convert_qwen35_moe.py (U8 int4 nibbles + ".qs" [scale, zero] pairs per group,
// :124-144 and :254-334) read straight into device tensors and the resident expert table.
// The shard index, its header rules (c/st.h:120-456) and the host reads are in st_host.cpp.
//
// An expert's projection is "model.layers.L.mlp.experts.E.{gate,up,down}_proj.weight" with
// exactly O ceil(I / 2) bytes, plus ".qs" with exactly O ceil(I / gs) 2 elements of a float
// dtype (F32 as the converter writes it; F16 / BF16 converted, as st_read_f32 does;
// c/qwen.c:520-534).  Differences from the reference: a bad file makes the call return 0
// with a message instead of exiting the process, and whatever the call had uploaded is
// released again; reads go to pinned buffers that several threads fill while the device
// converts the previous batch (the reference reads one expert at a time into a host slot
// and copies it again at upload).
#include "internal.h"
#include "st_host.h"

#include "moe_common.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <thread>
#include <vector>

extern "C" int coli_vk_eg_table_set(int layer, int eid, ColiVkTensor *g, ColiVkTensor *u, ColiVkTensor *d);
extern "C" int coli_vk_tensor_ensure(ColiVkTensor **, const void *, const float *, int, int, int, int);
extern "C" void coli_vk_tensor_free(ColiVkTensor *t);

namespace coli {

// ---------------------------------------------------------------- device loads
struct Pinned {
    void *p = nullptr;
    size_t cap = 0;
};
static Pinned g_pin[2];
static void *g_dstage[2] = {nullptr, nullptr};
static size_t g_dstage_cap[2] = {0, 0};
static hipEvent_t g_ev[2] = {nullptr, nullptr};

void container_shutdown() {
    for (int i = 0; i < 2; i++) {
        host_scratch_free(&g_pin[i].p, &g_pin[i].cap);
        scratch_free(&g_dstage[i], &g_dstage_cap[i]);
        if (g_ev[i]) (void)hipEventDestroy(g_ev[i]);
        g_ev[i] = nullptr;
    }
}

// One fmt6 projection: host bytes of weights and scales and where they go.
struct Piece {
    const StTensor *w, *s;
    int I, O, gs;
    size_t wb, sb, at;   // weight and f32 scale bytes, offset of the weights in the batch
    size_t so;           // offset of the scales after the weights (16-byte aligned)
    ColiVkTensor *t;
};

static bool piece_check(const Shards &S, const std::string &name, int I, int O, int gs, Piece &pc) {
    const int ng = (I + gs - 1) / gs;
    pc.w = find(S, name);
    pc.s = find(S, name + ".qs");
    pc.I = I;
    pc.O = O;
    pc.gs = gs;
    pc.wb = (size_t)O * ((I + 1) / 2);
    pc.sb = (size_t)O * ng * 2 * 4;
    pc.so = (pc.wb + 15) & ~(size_t)15;
    pc.t = nullptr;
    if (!pc.w || pc.w->dtype != kU8 || (size_t)pc.w->nbytes != pc.wb) {   // c/qwen.c:522-525
        fprintf(stderr, "[HIP] container: %s: %lld bytes, expected %zu U8 - wrong container?\n", name.c_str(),
                (long long)(pc.w ? pc.w->nbytes : -1), pc.wb);
        return false;
    }
    if (!pc.s || pc.s->dtype == kU8 || pc.s->numel != (int64_t)O * ng * 2) {   // c/qwen.c:528-534
        fprintf(stderr, "[HIP] container: %s.qs: %lld elements, expected %lld float\n", name.c_str(),
                (long long)(pc.s ? pc.s->numel : -1), (long long)O * ng * 2);
        return false;
    }
    return true;
}

// Reads pieces[0, n) into the pinned slot (threads split the pieces) and converts them to
// device tensors on the stream: one copy of the batch to device staging, then per piece
// the relayout into its arena slice and the scales' copy.  The slot may be refilled once
// g_ev[slot] has completed.
static size_t piece_bytes(const Piece &pc) { return (pc.so + pc.sb + 255) & ~(size_t)255; }

static bool load_batch(std::vector<Piece> &pcs, size_t i0, size_t i1, int slot, int nthreads) {
    size_t bytes = 0;
    for (size_t i = i0; i < i1; i++) {
        pcs[i].at = bytes;
        bytes += piece_bytes(pcs[i]);
    }
    if (g_ev[slot]) {   // the slot's previous batch has left for the device
        const hipError_t e = hipEventSynchronize(g_ev[slot]);
        if (e != hipSuccess) return fail("container slot wait", e);
    }
    if (!host_scratch(&g_pin[slot].p, &g_pin[slot].cap, bytes) ||
        !scratch(&g_dstage[slot], &g_dstage_cap[slot], bytes))
        return false;
    uint8_t *hp = (uint8_t *)g_pin[slot].p;
    bool good = true;
    {
        std::vector<std::thread> th;
        std::vector<char> ok_t((size_t)nthreads, 1);
        for (int k = 0; k < nthreads; k++)
            th.emplace_back([&, k]() {
                for (size_t i = i0 + (size_t)k; i < i1; i += (size_t)nthreads) {
                    const Piece &pc = pcs[i];
                    if (!pread_full(pc.w->fd, hp + pc.at, (int64_t)pc.wb, pc.w->off) ||
                        !read_f32(*pc.s, (float *)(hp + pc.at + pc.so))) {
                        ok_t[(size_t)k] = 0;
                        return;
                    }
                }
            });
        for (auto &t : th) t.join();
        for (char c : ok_t) good = good && c;
    }
    if (!good) return false;
    hipStream_t st = stream();
    uint8_t *dp = (uint8_t *)g_dstage[slot];
    hipError_t e = hipMemcpyAsync(dp, hp, bytes, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return fail("container upload", e);
    if (!g_ev[slot] && (e = hipEventCreateWithFlags(&g_ev[slot], hipEventDisableTiming)) != hipSuccess)
        return fail("container event", e);
    if ((e = hipEventRecord(g_ev[slot], st)) != hipSuccess) return fail("container event", e);
    for (size_t i = i0; i < i1; i++) {
        Piece &pc = pcs[i];
        ColiVkTensor *t = tensor_alloc(6, pc.I, pc.O, pc.gs);
        if (!t) return false;
        if (tensor_host_row_bytes(t) != (size_t)((pc.I + 1) / 2) || !tensor_fill_rows(t, dp + pc.at, 0, pc.O, st)) {
            free(t);
            return false;
        }
        e = hipMemcpyAsync(t->sz, dp + pc.at + pc.so, pc.sb, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) {
            free(t);
            return fail("container scales", e);
        }
        tensor_register(t);
        pc.t = t;
    }
    return true;
}

static int reader_threads() {
    const char *v = getenv("COLI_HIP_READ_THREADS");
    int n = v ? atoi(v) : (int)std::thread::hardware_concurrency();
    return std::max(1, std::min(n, 16));
}

// Releases the tensors of pieces (made by an unfinished call): their handles and the
// library's counts.  The arena slices stay reserved, as for every freed tensor.
static void release(std::vector<Piece> &pcs) {
    for (Piece &pc : pcs) {
        coli_vk_tensor_free(pc.t);
        pc.t = nullptr;
    }
}

// pieces in order, batches of at most kBatchBytes, two slots alternating; on a failure
// every tensor made so far is released
static bool load_pieces(std::vector<Piece> &pcs) {
    constexpr size_t kBatchBytes = (size_t)64 << 20;
    const int nt = reader_threads();
    size_t i0 = 0;
    int slot = 0;
    while (i0 < pcs.size()) {
        size_t i1 = i0, bytes = 0;
        while (i1 < pcs.size() && (i1 == i0 || bytes + piece_bytes(pcs[i1]) <= kBatchBytes)) {
            bytes += piece_bytes(pcs[i1]);
            i1++;
        }
        if (!load_batch(pcs, i0, i1, slot, nt)) {
            release(pcs);
            return false;
        }
        i0 = i1;
        slot ^= 1;
    }
    if (!sync_stream("container load")) {
        release(pcs);
        return false;
    }
    return true;
}

}  // namespace coli

using namespace coli;

// A device tensor straight from the container, in place of reading it into host memory
// and calling coli_vk_tensor_ensure (c/qwen.c:509-536 then c/backend_vulkan.c:1055-1085):
// fmt 6 reads `name` (U8 [O, ceil(I/2)]) and `name`.qs (float [O, 2 ceil(I/gs)]); fmt 0 reads
// an F32 / BF16 / F16 [O, I] tensor as f32 rows.  *tensor must be NULL (a new handle).
COLI_API int coli_hip_st_tensor(const ColiHipSt *st, const char *name, ColiVkTensor **tensor, int fmt, int I, int O,
                                int gs) {
    if (!st || !name || !tensor || *tensor || I < 1 || O < 1 || !ok()) return 0;
    if (fmt == 6) {
        if (gs < 8 || gs % 8) return 0;
        std::vector<Piece> pcs(1);
        if (!piece_check(st->s, name, I, O, gs, pcs[0]) || !load_pieces(pcs)) return 0;
        *tensor = pcs[0].t;
        return 1;
    }
    if (fmt == 0) {
        const StTensor *t = find(st->s, name);
        if (!t || t->dtype == kU8 || t->numel != (int64_t)O * I) {
            fprintf(stderr, "[HIP] container: %s: %lld elements, expected %lld float\n", name,
                    (long long)(t ? t->numel : -1), (long long)O * I);
            return 0;
        }
        std::vector<float> h((size_t)t->numel);
        if (!read_f32(*t, h.data())) return 0;
        return coli_vk_tensor_ensure(tensor, h.data(), nullptr, 0, I, O, 0);
    }
    return 0;
}

// The E routed experts of model layer `layer` (gate/up [I, D], down [D, I], fmt 6, group
// size gs; c/tools/convert_qwen35_moe.py:322-330 names) into slots (layer, 0..E-1) of the
// resident expert table (coli_vk_eg_table_init first).  All reads and the table's shape are
// checked before any upload, and every slot is checked before any is set; reads of one
// batch run on several threads while the device converts the previous one.  Returns 1 when
// every expert is resident; 0 leaves the table and the library's tensor count as they were.
COLI_API int coli_hip_st_experts(const ColiHipSt *st, int layer, int E, int D, int I, int gs) {
    if (!st || layer < 0 || E < 1 || D < 1 || I < 1 || gs < 8 || gs % 8 || !ok()) return 0;
    if (!eg_table_dims(layer, E, D, I, gs)) {
        fprintf(stderr, "[HIP] container: layer %d, %d experts of %d x %d (gs %d) do not fit the expert table "
                        "(coli_vk_eg_table_init shape?)\n", layer, E, D, I, gs);
        return 0;
    }
    static const char *kProj[3] = {"gate_proj", "up_proj", "down_proj"};
    std::vector<Piece> pcs((size_t)E * 3);
    char nm[256];
    for (int e = 0; e < E; e++)
        for (int j = 0; j < 3; j++) {
            snprintf(nm, sizeof(nm), "model.layers.%d.mlp.experts.%d.%s.weight", layer, e, kProj[j]);
            if (!piece_check(st->s, nm, j < 2 ? D : I, j < 2 ? I : D, gs, pcs[(size_t)e * 3 + j])) return 0;
        }
    if (!load_pieces(pcs)) return 0;
    for (int e = 0; e < E; e++)
        if (!eg_table_check(layer, e, pcs[(size_t)e * 3].t, pcs[(size_t)e * 3 + 1].t, pcs[(size_t)e * 3 + 2].t,
                            nullptr)) {
            fprintf(stderr, "[HIP] container: expert table slot (%d, %d) refused (geometry)\n", layer, e);
            release(pcs);
            return 0;
        }
    for (int e = 0; e < E; e++)   // can fail only on a device error (sticky, the device is off)
        if (!coli_vk_eg_table_set(layer, e, pcs[(size_t)e * 3].t, pcs[(size_t)e * 3 + 1].t, pcs[(size_t)e * 3 + 2].t))
            return 0;
    return 1;
}
