// runtime.hip - device bring-up, weight arena, tensor upload and the lifetime part of
// the drop-in C ABI (c/backend_vulkan.h).  MI355X (gfx950) only: init refuses any
// other device so that a caller falls back to its CPU path instead of running kernels
// that were never built for it.
#include "internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <condition_variable>
#include <mutex>
#include <thread>

namespace coli {

struct ArenaBlock {
    uint8_t *base;
    size_t cap, off;
};

struct Runtime {
    int ready = 0;
    int dev = 0;
    int ncu = 0;
    hipStream_t st = nullptr;
    ArenaBlock blocks[4096];
    int nblocks = 0;
    size_t used_bytes = 0, tensor_count = 0;
    long fail_after = -1;   // COLI_HIP_FAIL_AFTER=n: the (n+1)-th checked call reports a device loss
    unsigned gen = 1;       // bumped by every shutdown: handles of an earlier generation are dead
};
Runtime G;

// Weight slices come from 1 GiB blocks: a few large allocations instead of one per
// tensor (the reference packs uploads into 256 MiB arenas for the same reason,
// c/backend_vulkan.c:1003-1012).  Slices are never reclaimed individually.
static const size_t kArenaBlock = (size_t)1 << 30;

bool fail(const char *what, hipError_t e) {
    if (G.ready) fprintf(stderr, "[HIP] %s failed: %s - disabling GPU offload\n", what, hipGetErrorString(e));
    G.ready = 0;
    return false;
}

bool ok() {
    if (!G.ready) return false;
    if (G.fail_after >= 0) {
        if (G.fail_after == 0) {
            fprintf(stderr, "[HIP] injected device failure (COLI_HIP_FAIL_AFTER)\n");
            G.ready = 0;
            return false;
        }
        G.fail_after--;
    }
    return true;
}

hipStream_t stream() { return G.st; }
int n_cu() { return G.ncu; }

void *arena_alloc(size_t bytes) {
    bytes = (bytes + 255) & ~(size_t)255;
    for (int i = 0; i < G.nblocks; i++) {
        ArenaBlock &b = G.blocks[i];
        if (b.off + bytes <= b.cap) {
            void *p = b.base + b.off;
            b.off += bytes;
            return p;
        }
    }
    if (G.nblocks == (int)(sizeof(G.blocks) / sizeof(G.blocks[0]))) return nullptr;
    size_t cap = bytes > kArenaBlock ? bytes : kArenaBlock;
    void *base = nullptr;
    hipError_t e = hipMalloc(&base, cap);
    if (e != hipSuccess) {
        fprintf(stderr, "[HIP] arena: hipMalloc(%zu) failed: %s\n", cap, hipGetErrorString(e));
        return nullptr;
    }
    ArenaBlock &b = G.blocks[G.nblocks++];
    b.base = (uint8_t *)base;
    b.cap = cap;
    b.off = bytes;
    return base;
}

bool scratch(void **p, size_t *cap, size_t need) {
    if (need <= *cap && *p) return true;
    size_t want = need < 4096 ? 4096 : need;
    if (*p) {
        hipError_t e = hipStreamSynchronize(G.st);   // old buffer may still be in use
        if (e != hipSuccess) return fail("scratch sync", e);
        (void)hipFree(*p);
        *p = nullptr;
        *cap = 0;
    }
    hipError_t e = hipMalloc(p, want);
    if (e != hipSuccess) return fail("scratch hipMalloc", e);
    e = hipMemsetAsync(*p, 0, want, G.st);
    if (e != hipSuccess) return fail("scratch memset", e);
    *cap = want;
    return true;
}

void scratch_free(void **p, size_t *cap) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
}

void host_scratch_free(void **p, size_t *cap) {
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
}

bool host_scratch(void **p, size_t *cap, size_t need) {
    if (need <= *cap && *p) return true;
    size_t want = need < 4096 ? 4096 : need;
    if (*p) {
        hipError_t e = hipStreamSynchronize(G.st);
        if (e != hipSuccess) return fail("host scratch sync", e);
        (void)hipHostFree(*p);
        *p = nullptr;
        *cap = 0;
    }
    hipError_t e = hipHostMalloc(p, want, hipHostMallocDefault);
    if (e != hipSuccess) return fail("hipHostMalloc", e);
    *cap = want;
    return true;
}

bool sync_stream(const char *who) {
    hipError_t e = hipStreamSynchronize(G.st);
    if (e != hipSuccess) return fail(who, e);
    return true;
}

// ---------------------------------------------------------------- pinned <-> device copies
// Transfers between device memory and pinned host memory (hipHostMalloc: mapped into the
// device's address space) run as these kernels, one launch per piece: the launch returns at
// once, where a hipMemcpyAsync between them held the host thread for about as long as the
// transfer (the runtime's own blit kernel), so the pieces went out one at a time.  16-byte
// words when both ends and the size are 16-byte aligned, else 4-byte words when they are
// 4-byte aligned (every transfer here is of floats or ints), else bytes.
__global__ void pin_copy16(uint4 *__restrict__ d, const uint4 *__restrict__ s, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        d[i] = s[i];
}
__global__ void pin_copy4(uint32_t *__restrict__ d, const uint32_t *__restrict__ s, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        d[i] = s[i];
}
__global__ void pin_copy1(uint8_t *__restrict__ d, const uint8_t *__restrict__ s, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        d[i] = s[i];
}

bool pin_copy(void *dst, const void *src, size_t n, hipStream_t st, const char *who) {
    if (!n) return true;
    const uintptr_t al = (uintptr_t)dst | (uintptr_t)src | n;
    const size_t w = (al & 15) == 0 ? 16 : (al & 3) == 0 ? 4 : 1, words = n / w;
    const unsigned blocks = (unsigned)((words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024);
    if (w == 16)
        hipLaunchKernelGGL(pin_copy16, dim3(blocks), dim3(256), 0, st, (uint4 *)dst, (const uint4 *)src, words);
    else if (w == 4)
        hipLaunchKernelGGL(pin_copy4, dim3(blocks), dim3(256), 0, st, (uint32_t *)dst, (const uint32_t *)src, words);
    else
        hipLaunchKernelGGL(pin_copy1, dim3(blocks), dim3(256), 0, st, (uint8_t *)dst, (const uint8_t *)src, words);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(who, e);
    return true;
}

// ---------------------------------------------------------------- host copy helper
// One helper thread shares the host side of read-backs and uploads: a cold copy by one
// thread runs at ~20-26 GB/s on these hosts, by two at ~35-45 GB/s, which keeps up with
// the ~45 GB/s transfers.  The calling thread hands it the odd pieces of a job and does
// the even ones, then waits for it.  The helper starts on the first job and is joined at
// shutdown.
namespace {
struct CopyHelper {
    std::thread th;
    std::mutex m;
    std::condition_variable go, done;
    void (*fn)(void *, int) = nullptr;   // the job: fn(ctx, piece) for the helper's pieces
    void *ctx = nullptr;
    int count = 0;
    uint64_t posted = 0, finished = 0;
    bool ok = true, stop = false;
};
CopyHelper *g_ch = nullptr;

void helper_loop(CopyHelper *h) {
    (void)hipSetDevice(G.dev);   // the current device is per thread; its launches go to the library's device
    uint64_t seen = 0;
    for (;;) {
        void (*fn)(void *, int);
        void *ctx;
        int count;
        {
            std::unique_lock<std::mutex> lk(h->m);
            h->go.wait(lk, [&] { return h->stop || h->posted != seen; });
            if (h->stop) return;
            seen = h->posted;
            fn = h->fn, ctx = h->ctx, count = h->count;
        }
        for (int i = 1; i < count; i += 2) fn(ctx, i);
        {
            std::lock_guard<std::mutex> lk(h->m);
            h->finished = seen;
        }
        h->done.notify_one();
    }
}

// Runs fn(ctx, i) for i in [0, count): the helper the odd i, this thread the even ones.
// Without a helper (thread start failed) this thread runs all of them.
void split_pieces(void (*fn)(void *, int), void *ctx, int count) {
    if (count > 1 && !g_ch) {
        CopyHelper *h = new (std::nothrow) CopyHelper;
        if (h) {
            try {
                h->th = std::thread(helper_loop, h);
                g_ch = h;
            } catch (...) {
                delete h;
            }
        }
    }
    if (count < 2 || !g_ch) {
        for (int i = 0; i < count; i++) fn(ctx, i);
        return;
    }
    CopyHelper *h = g_ch;
    uint64_t job;
    {
        std::lock_guard<std::mutex> lk(h->m);
        h->fn = fn, h->ctx = ctx, h->count = count;
        job = ++h->posted;
    }
    h->go.notify_one();
    for (int i = 0; i < count; i += 2) fn(ctx, i);
    std::unique_lock<std::mutex> lk(h->m);
    h->done.wait(lk, [&] { return h->finished == job; });
}

void copy_helper_stop() {
    if (!g_ch) return;
    {
        std::lock_guard<std::mutex> lk(g_ch->m);
        g_ch->stop = true;
    }
    g_ch->go.notify_one();
    g_ch->th.join();
    delete g_ch;
    g_ch = nullptr;
}
}  // namespace

// ---------------------------------------------------------------- read-backs
// A read-back into a caller's (pageable) buffer goes through pinned staging: the device
// copies in up to 8 pieces (pin_copy), each with its event, and each piece is copied out on
// the host as soon as it has arrived (this thread and the copy helper take turns), so the
// host copies overlap the transfers of the later pieces.
namespace {
void *g_rb = nullptr;   // pinned staging of read_back
size_t g_rb_cap = 0;
PieceEvents g_rb_pe;
}  // namespace

namespace {
void *g_up = nullptr;   // write-combined pinned staging of upload
size_t g_up_cap = 0;
hipEvent_t g_up_done = nullptr;   // after the last transfer out of g_up
bool g_up_busy = false;
}  // namespace

void read_back_shutdown() {
    copy_helper_stop();
    host_scratch_free(&g_rb, &g_rb_cap);
    piece_events_free(g_rb_pe);
    if (g_up_busy) (void)hipEventSynchronize(g_up_done);
    g_up_busy = false;
    host_scratch_free(&g_up, &g_up_cap);
    if (g_up_done) (void)hipEventDestroy(g_up_done);
    g_up_done = nullptr;
}

// ---------------------------------------------------------------- uploads
// Caller (pageable) buffers to the device through pinned staging, laid out one after the
// other: each 1 MiB piece is copied into the staging on the host (this thread and the copy
// helper take turns) and its transfer (pin_copy) issued at once, so transfers overlap the
// host copies (a pageable hipMemcpyAsync does them in turn).  The staging is write-combined:
// the host only writes it and the device only reads it.  The next upload reuses it once the
// last transfer out of it is done (an event); the caller's buffers are free again on return.
bool upload(const Upload *u, int nu, hipStream_t st, const char *who) {
    constexpr size_t kPiece = (size_t)1 << 20;
    size_t total = 0;
    for (int i = 0; i < nu; i++) total += (u[i].n + 4095) & ~(size_t)4095;
    if (!total) return true;
    if (g_up_busy) {
        const hipError_t e = hipEventSynchronize(g_up_done);
        if (e != hipSuccess) return fail(who, e);
        g_up_busy = false;
    }
    if (total > g_up_cap || !g_up) {
        host_scratch_free(&g_up, &g_up_cap);
        const hipError_t e = hipHostMalloc(&g_up, total, hipHostMallocWriteCombined);
        if (e != hipSuccess) {
            g_up = nullptr;
            return fail("hipHostMalloc (upload staging)", e);
        }
        g_up_cap = total;
    }
    // the pieces of all transfers in one list, copied and issued by this thread and the helper
    constexpr int kMaxPieces = 256;
    struct Piece {
        void *d;
        const void *h;
        uint8_t *s;
        size_t len;
    };
    Piece pcs[kMaxPieces];
    int np = 0;
    size_t off = 0, piece = kPiece;
    for (int i = 0; i < nu; i++) {
        const size_t np_i = (u[i].n + kPiece - 1) / kPiece;
        if ((size_t)np + np_i > (size_t)kMaxPieces) piece = 0;   // too many: one plain pass below
        for (size_t o = 0; piece && o < u[i].n; o += kPiece)
            pcs[np++] = {(uint8_t *)u[i].d + o, (const uint8_t *)u[i].h + o, (uint8_t *)g_up + off + o,
                         u[i].n - o < kPiece ? u[i].n - o : kPiece};
        off += (u[i].n + 4095) & ~(size_t)4095;
    }
    if (!piece) {   // more than kMaxPieces MiB in one upload: this thread alone
        off = 0;
        for (int i = 0; i < nu; i++) {
            memcpy((uint8_t *)g_up + off, u[i].h, u[i].n);
            __atomic_thread_fence(__ATOMIC_SEQ_CST);
            if (!pin_copy(u[i].d, (uint8_t *)g_up + off, u[i].n, st, who)) return false;
            off += (u[i].n + 4095) & ~(size_t)4095;
        }
    } else {
        struct Ctx {
            const Piece *p;
            hipStream_t st;
            std::atomic<int> bad;
        } c{pcs, st, {0}};
        split_pieces(
            [](void *v, int i) {
                Ctx &c = *(Ctx *)v;
                const Piece &p = c.p[i];
                memcpy(p.s, p.h, p.len);
                __atomic_thread_fence(__ATOMIC_SEQ_CST);   // the write-combined stores out before the launch
                if (!pin_copy(p.d, p.s, p.len, c.st, "upload")) c.bad = 1;
            },
            &c, np);
        if (c.bad) return fail(who, hipErrorUnknown);
    }
    hipError_t e = g_up_done ? hipSuccess : hipEventCreateWithFlags(&g_up_done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(g_up_done, st);
    if (e != hipSuccess) return fail(who, e);
    g_up_busy = true;
    return true;
}

// Up to PieceEvents::kMax pieces of at least 1 MiB each.
bool issue_pieces(PieceEvents &pe, void *hdst, const void *dsrc, size_t n, hipStream_t st) {
    size_t piece = (size_t)1 << 20;
    if (n > piece * PieceEvents::kMax) piece = (n + PieceEvents::kMax - 1) / PieceEvents::kMax;
    piece = (piece + 4095) & ~(size_t)4095;
    pe.piece = piece;
    pe.n = n;
    pe.count = n ? (int)((n + piece - 1) / piece) : 0;
    for (int i = 0; i < pe.count; i++) {
        const size_t o = (size_t)i * piece, len = n - o < piece ? n - o : piece;
        if (!pin_copy((uint8_t *)hdst + o, (const uint8_t *)dsrc + o, len, st, "read-back issue")) return false;
        hipError_t e = pe.ev[i] ? hipSuccess : hipEventCreateWithFlags(&pe.ev[i], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventRecord(pe.ev[i], st);
        if (e != hipSuccess) return fail("read-back issue", e);
    }
    return true;
}

bool copy_out(PieceEvents &pe, void *dst, const void *hsrc, const char *who) {
    struct Ctx {
        PieceEvents *pe;
        uint8_t *dst;
        const uint8_t *src;
        std::atomic<int> bad;
    } c{&pe, (uint8_t *)dst, (const uint8_t *)hsrc, {0}};
    split_pieces(
        [](void *p, int i) {
            Ctx &c = *(Ctx *)p;
            if (hipEventSynchronize(c.pe->ev[i]) != hipSuccess) {
                c.bad = 1;
                return;
            }
            const size_t o = (size_t)i * c.pe->piece, len = c.pe->n - o < c.pe->piece ? c.pe->n - o : c.pe->piece;
            memcpy(c.dst + o, c.src + o, len);
        },
        &c, pe.count);
    if (c.bad) return fail(who, hipErrorUnknown);
    return true;
}

void piece_events_free(PieceEvents &pe) {
    for (int i = 0; i < PieceEvents::kMax; i++)
        if (pe.ev[i]) (void)hipEventDestroy(pe.ev[i]);
    pe = PieceEvents();
}

bool read_back(void *dst, const void *dsrc, size_t n, hipStream_t st, const char *who) {
    if (!n) return true;
    if (!host_scratch(&g_rb, &g_rb_cap, n)) return false;
    return issue_pieces(g_rb_pe, g_rb, dsrc, n, st) && copy_out(g_rb_pe, dst, g_rb, who);
}

// Device layout of a tensor (see ColiVkTensor) and its arena slice.
ColiVkTensor *tensor_alloc(int fmt, int I, int O, int gs) {
    if (I < 1 || O < 1) return nullptr;
    if (fmt == 6 && !(gs >= 8 && gs % 8 == 0)) return nullptr;
    if (fmt != 6 && fmt != 1 && fmt != 0) return nullptr;
    ColiVkTensor *t = (ColiVkTensor *)calloc(1, sizeof(ColiVkTensor));
    if (!t) return nullptr;
    t->fmt = fmt;
    t->I = I;
    t->O = O;
    t->gs = fmt == 6 ? gs : 0;
    t->ng = fmt == 6 ? (I + gs - 1) / gs : 0;
    t->nchunks = (int)((tensor_host_row_bytes(t) + 15) / 16);
    t->nl = (t->nchunks + kLaneChunks - 1) / kLaneChunks;
    // the lanes kernels address a tensor with 32-bit offsets (plus one grid step of slack)
    const bool fits = (size_t)O * t->nl * kLaneChunks * 16 < ((size_t)1 << 31) - ((size_t)1 << 28);
    t->layout = (fmt == 6 && gs % 32 == 0 && I <= kLaneMaxI && fits) ? kLayoutLanes : kLayoutRows;
    t->row_bytes = t->layout == kLayoutLanes ? t->nl * kLaneChunks * 16 : t->nchunks * 16;
    const size_t wbytes = (size_t)t->row_bytes * O;
    const size_t sfl = fmt == 6 ? (size_t)O * t->ng * 2 : fmt == 1 ? (size_t)O : 0;
    const size_t sbytes = sfl * sizeof(float);
    uint8_t *base = (uint8_t *)arena_alloc(wbytes + ((sbytes + 255) & ~(size_t)255));
    if (!base) {
        free(t);
        return nullptr;
    }
    t->w = base;
    t->sz = sfl ? (float *)(base + wbytes) : nullptr;
    t->bytes = wbytes + sbytes;
    t->wbytes = wbytes;
    t->gen = G.gen;
    return t;
}

bool tensor_live(const ColiVkTensor *t) { return t && t->gen == G.gen && t->w; }

size_t tensor_host_row_bytes(const ColiVkTensor *t) {
    return t->fmt == 6 ? (size_t)(t->I + 1) / 2 : t->fmt == 1 ? (size_t)t->I : (size_t)t->I * 4;
}

// One thread per 16-byte device chunk: copy (rows layout) or permute + XOR (lanes layout).
__global__ void fill_rows_kernel(uint8_t *__restrict__ dst, const uint8_t *__restrict__ src, int rows,
                                 int host_rb, int nchunks, int nl, int row_bytes, int lanes) {
    const int per_row = row_bytes / 16;
    const size_t n = (size_t)rows * per_row;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(k / per_row), p = (int)(k - (size_t)r * per_row);
        const int h = lanes ? (p % nl) * kLaneChunks + p / nl : p;   // host chunk held by device slot p
        const uint8_t *s = src + (size_t)r * host_rb + (size_t)h * 16;
        uint8_t b[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int off = h * 16 + i;
            const uint8_t v = (h < nchunks && off < host_rb) ? s[i] : 0;
            b[i] = lanes ? (uint8_t)(v ^ 0x88) : v;
        }
        uint4 o;
        memcpy(&o, b, 16);
        *(uint4 *)(dst + (size_t)r * row_bytes + (size_t)p * 16) = o;
    }
}

bool tensor_fill_rows(ColiVkTensor *t, const uint8_t *d_src, int r0, int rows, hipStream_t st) {
    const int per_row = t->row_bytes / 16;
    size_t nb = ((size_t)rows * per_row + 255) / 256;
    const size_t cap = (size_t)G.ncu * 16;
    if (nb > cap) nb = cap;
    if (nb < 1) nb = 1;
    hipLaunchKernelGGL(fill_rows_kernel, dim3((unsigned)nb), dim3(256), 0, st, t->w + (size_t)r0 * t->row_bytes,
                       d_src, rows, (int)tensor_host_row_bytes(t), t->nchunks, t->nl, t->row_bytes,
                       t->layout == kLayoutLanes ? 1 : 0);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("tensor relayout", e);
    return true;
}

// staging buffer for uploads (host rows -> device, then relayout)
static void *g_stage = nullptr;
static size_t g_stage_cap = 0;
static const size_t kStageBytes = (size_t)64 << 20;

bool stage_buffer(void **p, size_t *cap_rows, size_t host_rb) {
    if (!scratch(&g_stage, &g_stage_cap, kStageBytes)) return false;
    *p = g_stage;
    *cap_rows = kStageBytes / (host_rb ? host_rb : 1);
    return *cap_rows > 0;
}

void tensor_register(ColiVkTensor *t) {
    G.used_bytes += t->bytes;
    G.tensor_count++;
}

// Upload semantics follow c/backend_vulkan.c:1055-1085: an existing handle is only
// checked for (fmt, I, O); fmt 6 needs gs >= 8 and gs % 8 == 0; host buffers are copied
// (the caller keeps its quantized copy as CPU fallback).  Added here: fmt 0 (f32 rows),
// which the f32 MoE router of the benchmark configurations uses.
static bool upload(ColiVkTensor **out, const void *w, const float *s, int fmt, int I, int O, int gs) {
    if (*out) return tensor_live(*out) && (*out)->fmt == fmt && (*out)->I == I && (*out)->O == O;
    if (!w || ((fmt == 6 || fmt == 1) && !s)) return false;
    ColiVkTensor *t = tensor_alloc(fmt, I, O, gs);
    if (!t) return false;
    const size_t host_rb = tensor_host_row_bytes(t);
    const size_t sbytes = fmt == 6 ? (size_t)O * t->ng * 2 * 4 : fmt == 1 ? (size_t)O * 4 : 0;
    void *stg = nullptr;
    size_t cap_rows = 0;
    if (!stage_buffer(&stg, &cap_rows, host_rb)) {
        free(t);
        return false;
    }
    hipError_t e = hipSuccess;
    for (int r0 = 0; r0 < O && e == hipSuccess; r0 += (int)cap_rows) {
        const int rows = (int)((size_t)(O - r0) < cap_rows ? (size_t)(O - r0) : cap_rows);
        e = hipMemcpyAsync(stg, (const uint8_t *)w + (size_t)r0 * host_rb, (size_t)rows * host_rb,
                           hipMemcpyHostToDevice, G.st);
        if (e == hipSuccess && !tensor_fill_rows(t, (const uint8_t *)stg, r0, rows, G.st)) {
            free(t);
            return false;
        }
        if (e == hipSuccess) e = hipStreamSynchronize(G.st);   // staging is reused
    }
    if (e == hipSuccess && sbytes) e = hipMemcpyAsync(t->sz, s, sbytes, hipMemcpyHostToDevice, G.st);
    if (e == hipSuccess) e = hipStreamSynchronize(G.st);
    if (e != hipSuccess) {
        free(t);
        return fail("tensor upload", e);
    }
    tensor_register(t);
    *out = t;
    return true;
}

}  // namespace coli

using namespace coli;

// c/backend_vulkan.h:37, c/backend_vulkan.c:596-994.  spv_path is ignored: the kernels
// are compiled into this library for gfx950.
COLI_API int coli_vk_init(const char *spv_path) {
    (void)spv_path;
    if (G.ready) return 1;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        fprintf(stderr, "[HIP] no GPU visible - staying on CPU\n");
        return 0;
    }
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return 0;
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        fprintf(stderr, "[HIP] device 0 is %s, this library is built for gfx950 only\n", p.gcnArchName);
        return 0;
    }
    if (hipSetDevice(0) != hipSuccess) return 0;
    if (hipStreamCreateWithFlags(&G.st, hipStreamNonBlocking) != hipSuccess) return 0;
    G.dev = 0;
    G.ncu = p.multiProcessorCount;
    (void)moe_noalloc_init(G.dev);   // a failure only disables coli_hip_moe_decode_noalloc
    const char *fa = getenv("COLI_HIP_FAIL_AFTER");
    G.fail_after = fa ? atol(fa) : -1;
    G.ready = 1;
    fprintf(stderr, "[HIP] %s (%s), %d CUs, %.1f GiB HBM\n", p.name, p.gcnArchName, G.ncu,
            p.totalGlobalMem / (1024.0 * 1024.0 * 1024.0));
    return 1;
}

// c/backend_vulkan.h:38, c/backend_vulkan.c:4139-4160.  Every file's state is dropped with
// the arena: tensors, the expert table, KV/GDN/norm state and scratch buffers.  Handles of
// the old generation are refused afterwards (coli_vk_tensor_free still releases them),
// and coli_vk_init can bring the device up again.
COLI_API void coli_vk_shutdown(void) {
    if (!G.st) return;
    (void)hipStreamSynchronize(G.st);
    gemv_shutdown();
    moe_shutdown();
    prefill_shutdown();
    layer_shutdown();
    container_shutdown();
    read_back_shutdown();
    scratch_free(&g_stage, &g_stage_cap);
    for (int i = 0; i < G.nblocks; i++) (void)hipFree(G.blocks[i].base);
    G.nblocks = 0;
    G.used_bytes = G.tensor_count = 0;
    (void)hipStreamDestroy(G.st);
    G.st = nullptr;
    G.gen++;
    G.ready = 0;
}

// c/backend_vulkan.h:39
COLI_API int coli_vk_available(void) { return G.ready ? 1 : 0; }

// c/backend_vulkan.h:40, c/backend_vulkan.c:998
COLI_API void coli_vk_mem_info(size_t *used_bytes, size_t *tensor_count) {
    if (used_bytes) *used_bytes = G.used_bytes;
    if (tensor_count) *tensor_count = G.tensor_count;
}

// c/backend_vulkan.h:50: eviction classes do not exist on HBM; every tensor stays resident.
COLI_API void coli_vk_alloc_priority(float p) { (void)p; }

// c/backend_vulkan.h:51, c/backend_vulkan.c:387
COLI_API int coli_vk_mem_budget(double *used_gb, double *budget_gb) {
    if (!G.ready) return 0;
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) != hipSuccess) return 0;
    if (used_gb) *used_gb = (double)(tot - fr) / 1e9;
    if (budget_gb) *budget_gb = (double)tot / 1e9;
    return 1;
}

// c/backend_vulkan.h:91, c/backend_vulkan.c:1089-1092
COLI_API int coli_vk_tensor_ensure(ColiVkTensor **tensor, const void *weights, const float *scales,
                                   int fmt, int I, int O, int grp) {
    if (!tensor || !ok()) return 0;
    return upload(tensor, weights, scales, fmt, I, O, grp) ? 1 : 0;
}

// c/backend_vulkan.h:137, c/backend_vulkan.c:4119-4135: the arena slice is not reclaimed;
// the counters drop weights + scales, as the upload added them (a handle of an earlier
// generation was already uncounted by the shutdown).
COLI_API void coli_vk_tensor_free(ColiVkTensor *t) {
    if (!t) return;
    stream_tensor_freed(t);
    if (t->gen == G.gen) {
        G.used_bytes -= t->bytes;
        G.tensor_count--;
    }
    free(t);
}

// c/backend_vulkan.h:138, c/backend_vulkan.c:4137: the weight bytes (scales not counted)
COLI_API size_t coli_vk_tensor_bytes(const ColiVkTensor *t) { return t ? t->wbytes : 0; }

// Device view of a tensor for callers that drive kernels on device pointers.
COLI_API int coli_hip_tensor_info(const ColiVkTensor *t, int *fmt, int *I, int *O, int *gs,
                                  int *row_bytes, void **d_w, void **d_sz) {
    if (!tensor_live(t)) return 0;
    if (fmt) *fmt = t->fmt;
    if (I) *I = t->I;
    if (O) *O = t->O;
    if (gs) *gs = t->gs;
    if (row_bytes) *row_bytes = t->row_bytes;
    if (d_w) *d_w = t->w;
    if (d_sz) *d_sz = t->sz;
    return 1;
}

// Wait for `stream` (NULL = the library's stream).
COLI_API int coli_hip_sync(void *stream_) {
    if (!G.ready) return 0;
    const hipError_t e = hipStreamSynchronize(stream_ ? (hipStream_t)stream_ : G.st);
    if (e != hipSuccess) return fail("hipStreamSynchronize", e) ? 1 : 0;
    return 1;
}

// Blocking copy between any host / device addresses (unified addressing).
COLI_API int coli_hip_memcpy(void *dst, const void *src, size_t bytes) {
    if (!G.ready) return 0;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, G.st);
    if (e == hipSuccess) e = hipStreamSynchronize(G.st);
    if (e != hipSuccess) return fail("hipMemcpy", e) ? 1 : 0;
    return 1;
}
