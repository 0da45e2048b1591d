// gemv.hip - fmt=6 grouped-asymmetric int4 GEMV (decode), fmt 1 / fmt 0 GEMVs, device
// top-k over the outputs, RMSNorm, and the matmul entry points of the drop-in ABI.
//
// Semantics: c/qwen.c:211-229 (matmul_q4g_asym), c/shaders/qmatmul.comp:112-126.
//
// Fast path (fmt 6, kLayoutLanes): lanes run along K; lane j of a row owns two 16-byte
// chunks (64 columns) of the row and keeps the digit planes of its 64 x columns in
// VGPRs for the whole launch (see fmt6_device.h for the arithmetic).  LPR = the next
// power of two >= nl lanes cover one row, a wave covers 64/LPR rows per step, and each
// load instruction reads nl consecutive 16-byte chunks of a row (coalesced).  Rows are
// strided over a persistent grid, U row-steps are loaded before any is reduced, and a
// segmented DPP reduction sums the LPR lanes.  Per row this is 24 DOT8 per 64 columns
// plus one scale recombination per lane, about 35 VALU wave-instructions per KiB of
// weights.
//
// Top-k (fused): each block reduces its rows' candidates and publishes its k best as
// epoch-tagged 64-bit keys; the last block of the grid merges them in the same launch,
// polling the tags (agent-scope atomics: no device-scope fences, no second launch).
#include "fmt6_device.h"

#include <stdio.h>
#include <string.h>

namespace coli {

struct TopkArgs {
    int k;                       // 0 = off
    float *part_v;               // topk_partial: [gridDim.x * kTopK] block partials
    int *part_i;
    unsigned long long *slots;   // argmax: kArgSlots keys; fused top-k: [gridDim.x * kTopK] keys
    uint32_t epoch;              // tag of this launch (8 bits used)
    int *out_i;                  // fused top-k: the k best (value desc, index asc)
    float *out_v;
};

// ---- argmax as a 64-bit key: [63:56] launch epoch, [55:24] order-preserving bits of the
// value, [23:0] 0xFFFFFF - row.  The maximum key is the best (value desc, row asc) of the
// launch; a stale key of an earlier launch (lower epoch) always loses.  Rows < 2^24.
constexpr int kArgSlots = 16;   // blocks spread their atomicMax over 16 slots (contention)
__device__ __forceinline__ unsigned long long arg_key(uint32_t epoch, float v, uint32_t row) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)(epoch & 0xFFu) << 56) | ((unsigned long long)ord << 24) |
           (unsigned long long)(0xFFFFFFu - row);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned lo = __shfl_xor((unsigned)k, off), hi = __shfl_xor((unsigned)(k >> 32), off);
        const unsigned long long o = ((unsigned long long)hi << 32) | lo;
        k = o > k ? o : k;
    }
    return k;
}

// merge this block's per-thread lists and publish its k best as partials
__device__ void topk_publish(float (&tv)[kTopK], int (&ti)[kTopK], const TopkArgs &tk) {
    block_topk_merge<kTopK>(tv, ti, tk.k, tk.part_v + blockIdx.x * kTopK, tk.part_i + blockIdx.x * kTopK);
}

__device__ __forceinline__ unsigned long long aload64(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kFusedGrid = 1024;           // largest grid of a fused top-k launch
constexpr int kFusedWaves = kFusedGrid * 4;   // wave maxima slots (kWaves waves per block)
constexpr int kFusedSlots = 64;             // largest per-wave candidate count
constexpr int kFusedPollLimit = 1 << 20;

// Selection works on keys without the tag: a real key keeps its 56 bits, the padding key
// (tag only) becomes 1 so that it ranks below every real key but above "no entry" (0).
__device__ __forceinline__ unsigned long long strip_tag(unsigned long long key) {
    const unsigned long long v = key & 0x00FFFFFFFFFFFFFFull;
    return v ? v : (key ? 1ull : 0ull);
}

// decode a (tag-stripped) key into (row, value); padding and "no entry" -> (INT_MAX, -inf)
__device__ __forceinline__ void key_decode(unsigned long long key, int *row, float *val) {
    const uint32_t low = (uint32_t)(key & 0xFFFFFFu);
    if (key <= 1ull || low == 0u) {
        *row = INT_MAX;
        *val = -INFINITY;
        return;
    }
    const uint32_t ord = (uint32_t)(key >> 24);
    const uint32_t u = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    *row = (int)(0xFFFFFFu - low);
    *val = __uint_as_float(u);
}

// The grid's last block: the k best keys of the launch.  Units are waves: every wave
// published its largest key (wmax) and one key per slot it owns (cand).  The global top k
// can only come from the k waves whose maxima rank in the top k (a key of any other wave
// is beaten by k maxima), so: (1) each of the 4 waves selects the k best maxima of a
// quarter of the units, (2) wave 0 selects the k best of those 4k, (3) wave 0 selects the
// k best of the <= k x 64 keys of the chosen waves.  Keys of another launch carry another
// tag and are polled until overwritten.
__device__ void topk_final_block(const TopkArgs &tk, int nunits, int per_wave) {
    __shared__ unsigned long long s_key[kWaves * kTopK];
    __shared__ int s_unit[kWaves * kTopK];
    constexpr int kQ = kFusedWaves / kThreads;   // 16 maxima per lane
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, k = tk.k;
    const unsigned long long tag = (unsigned long long)(tk.epoch & 0xFFu);
    const unsigned long long *wmax = tk.slots, *cand = tk.slots + kFusedWaves;
    unsigned long long top[kTopK];
    int src[kTopK];
    bool fine = true;
    {   // (1) wave w: units w * 1024 + lane + 64 q
        unsigned long long kv[kQ];
        for (int polls = 0;; polls++) {
            bool all = true;
#pragma unroll
            for (int q = 0; q < kQ; q++) {
                const int u = wave * (kFusedWaves / kWaves) + lane + 64 * q;
                kv[q] = u < nunits ? aload64(&wmax[u]) : 0ull;
                all &= u >= nunits || (kv[q] >> 56) == tag;
            }
            if (__all(all)) break;
            if (polls > kFusedPollLimit) {
                fine = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int q = 0; q < kQ; q++) kv[q] = strip_tag(kv[q]);
        wave_select<kQ>(kv, k, top, src);
#pragma unroll
        for (int r = 0; r < kTopK; r++)
            if (lane == r) {   // src = lane' * kQ + q  ->  unit w * 1024 + lane' + 64 q
                s_key[wave * kTopK + r] = top[r];
                s_unit[wave * kTopK + r] =
                    src[r] < 0 ? -1 : wave * (kFusedWaves / kWaves) + src[r] / kQ + 64 * (src[r] % kQ);
            }
    }
    __syncthreads();
    if (wave != 0) return;
    // (2) the k best of the 4k unit maxima (one per lane)
    unsigned long long k1[1] = {lane < kWaves * kTopK ? s_key[lane] : 0ull};
    wave_select<1>(k1, k, top, src);
    int sel[kTopK];
#pragma unroll
    for (int r = 0; r < kTopK; r++) sel[r] = src[r] < 0 ? -1 : s_unit[src[r]];
    // (3) the keys of the chosen units: entry q of lane = slot `lane` of unit sel[q]
    unsigned long long kc[kTopK];
    for (int polls = 0;; polls++) {
        bool all = true;
#pragma unroll
        for (int q = 0; q < kTopK; q++) {
            const bool on = sel[q] >= 0 && lane < per_wave;
            kc[q] = on ? aload64(&cand[(size_t)sel[q] * per_wave + lane]) : 0ull;
            all &= !on || (kc[q] >> 56) == tag;
        }
        if (__all(all)) break;
        if (polls > kFusedPollLimit) {
            fine = false;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int q = 0; q < kTopK; q++) kc[q] = strip_tag(kc[q]);
    wave_select<kTopK>(kc, k, top, src);
#pragma unroll
    for (int r = 0; r < kTopK; r++)
        if (lane == r && r < k) {
            int row;
            float v;
            key_decode(top[r], &row, &v);
            tk.out_i[r] = fine ? row : -1;
            tk.out_v[r] = v;
        }
}

// The k best of nblk sorted partial lists (k entries each).  The global top k can only
// come from the k blocks whose best entry (head) ranks in the top k: a candidate of any
// other block is beaten by k heads.  Phase 1 picks those blocks by k rounds of a
// block-wide 64-bit max over the heads; phase 2 rank-selects among their k*k entries.
constexpr int kFinalThreads = 1024;
constexpr int kFinalWaves = kFinalThreads / 64;
__global__ __launch_bounds__(kFinalThreads) void topk_final(const float *__restrict__ part_v,
                                                            const int *__restrict__ part_i, int nblk, int k,
                                                            float *out_v, int *out_i) {
    __shared__ unsigned long long s_w[kFinalWaves];
    __shared__ int s_sel[kTopK];
    __shared__ float2 s_cand[kTopK * kTopK];
    __shared__ float s_ov[kTopK];
    __shared__ int s_oi[kTopK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // heads: thread t owns blocks t, t + 1024, ... (keep the best key it owns per round)
    constexpr int kPer = 2;   // nblk <= kFinalThreads * kPer
    unsigned long long key[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int bb = tid + q * kFinalThreads;
        key[q] = bb < nblk ? arg_key(0, part_v[bb * kTopK], (uint32_t)part_i[bb * kTopK]) : 0ull;
    }
    if (tid < kTopK) s_sel[tid] = -1;
    for (int r = 0; r < k; r++) {
        unsigned long long m = key[0];
#pragma unroll
        for (int q = 1; q < kPer; q++) m = key[q] > m ? key[q] : m;
        m = wave_max_u64(m);
        if (lane == 0) s_w[wave] = m;
        __syncthreads();
        unsigned long long best = s_w[0];
#pragma unroll
        for (int w = 1; w < kFinalWaves; w++) best = s_w[w] > best ? s_w[w] : best;
#pragma unroll
        for (int q = 0; q < kPer; q++)
            if (best != 0ull && key[q] == best) {   // unique (the row index is in the key)
                s_sel[r] = tid + q * kFinalThreads;
                key[q] = 0ull;
            }
        __syncthreads();
    }
    if (tid < kTopK * kTopK) {
        const int r = tid / kTopK, j = tid % kTopK, bb = s_sel[r < k ? r : 0];
        const bool on = r < k && j < k && bb >= 0;
        s_cand[tid] = on ? make_float2(part_v[bb * kTopK + j], __int_as_float(part_i[bb * kTopK + j]))
                         : make_float2(-INFINITY, __int_as_float(INT_MAX));
    }
    if (tid < kTopK) {
        s_ov[tid] = -INFINITY;
        s_oi[tid] = INT_MAX;
    }
    __syncthreads();
    rank_select(s_cand, kTopK * kTopK, k, s_ov, s_oi, kFinalThreads);
    __syncthreads();
    if (tid < k) {
        out_v[tid] = s_ov[tid];
        out_i[tid] = s_oi[tid];
    }
}

// one wave: decode the argmax slots of `epoch` into (idx, val)
__global__ void argmax_decode(const unsigned long long *__restrict__ slots, uint32_t epoch, int *out_i,
                              float *out_v) {
    unsigned long long best = threadIdx.x < kArgSlots ? slots[threadIdx.x] : 0ull;
    best = wave_max_u64(best);
    if (threadIdx.x == 0) {
        const uint32_t ord = (uint32_t)(best >> 24);
        const uint32_t u = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
        const bool okk = (uint32_t)(best >> 56) == (epoch & 0xFFu);
        out_i[0] = okk ? (int)(0xFFFFFFu - (uint32_t)(best & 0xFFFFFFu)) : -1;
        out_v[0] = okk ? __uint_as_float(u) : -INFINITY;
    }
}

__global__ void argmax_reset(unsigned long long *slots) {
    if (threadIdx.x < kArgSlots) slots[threadIdx.x] = 0ull;
}

// ---------------------------------------------------------------------------------- fast
// Requires O * row_bytes < 2^31 (32-bit buffer offsets; tensor_alloc only picks the lanes
// layout when that holds).
//   MODE 0: y only.
//   MODE 1: also argmax: leader lanes keep their best key, the block reduces it and
//           atomicMax-es it into slot blockIdx % kArgSlots (no fences: atomics are
//           coherent, and the reader runs after the kernel).
//   MODE 2: also top-k, fused: leader lanes store one tagged key per row slot of their
//           wave (`per_wave` slots, padding keys for slots past the end) and keep the
//           wave's largest key, which lane 0 publishes; the grid's last block then
//           merges (topk_final_block).
template <int LPR, int CU, int U, int MODE>
__global__ __launch_bounds__(kThreads) void gemv6_lanes(const uint8_t *__restrict__ W, const float *__restrict__ SZ,
                                                        const float *__restrict__ x, float *__restrict__ y, int I,
                                                        int O, int gs, int ng, int nl, int row_bytes, TopkArgs tk,
                                                        int per_wave) {
    __shared__ XPrep P;
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane % LPR, seg = lane / LPR;
    const uint32_t wtot = (uint32_t)O * (uint32_t)row_bytes, srb = (uint32_t)ng * 8u, stot = (uint32_t)O * srb;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(W, wtot), rs = buf_rsrc(SZ, stot);
    const int ncols = nl * kLaneChunks * 32;
    XRegs xr;
    prep_load(x, I, ncols, xr);   // x first: in-order load counters then let the
    LaneX<CU> L;                  // weight prefetch stay in flight through the prologue
    lane_geo<CU>(j, nl, I, gs, L);

    // slot u of this wave walks rows r = (rg0 + u*nw + it*nw*U) * RPW + seg
    const int nw = gridDim.x * kWaves;
    const int rg0 = blockIdx.x * kWaves + wave;
    const uint32_t rstep = (uint32_t)nw * U * RPW;
    const uint32_t wstep = rstep * (uint32_t)row_bytes, sstep = rstep * srb;
    uint32_t rr[U], wro[U], sro[U];   // row index and unclamped byte offsets of each slot
    uint4 wq[U][kLaneChunks];
    float2 sv[U][LaneX<CU>::NU];
#pragma unroll
    for (int u = 0; u < U; u++) {   // first loads go out before the x prologue
        rr[u] = (uint32_t)((rg0 + u * nw) * RPW + seg);
        wro[u] = rr[u] * (uint32_t)row_bytes;
        sro[u] = rr[u] * srb;
        lane_load<CU>(rw, rs, min(wro[u], wtot), min(sro[u], stot), L, wq[u], sv[u]);
    }
    prep_x(xr, gs, ncols, P);
    lane_x<CU>(P, gs, L);

    const uint32_t rlim = (uint32_t)((O + RPW - 1) / RPW) * RPW;   // rows the grid walks
    int slot = 0;                    // MODE 2: next candidate slot of this wave
    // best key of this lane's rows (MODE 2 starts at the padding key: waves without
    // rows still publish a tagged maximum)
    unsigned long long best = MODE == 2 ? (unsigned long long)(tk.epoch & 0xFFu) << 56 : 0ull;
    unsigned long long *cand = tk.slots + kFusedWaves + (size_t)(blockIdx.x * kWaves + wave) * per_wave;
    for (uint32_t base = (uint32_t)rg0 * RPW; base < rlim; base += rstep) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float part = lane_row<CU>(wq[u], sv[u], L);
            const uint32_t r = rr[u];
            rr[u] += rstep;   // refill this slot with its next row while the others compute
            wro[u] += wstep;
            sro[u] += sstep;
            lane_load<CU>(rw, rs, min(wro[u], wtot), min(sro[u], stot), L, wq[u], sv[u]);
            const float acc = seg_sum<LPR>(part);
            if (j == LPR - 1) {
                const bool valid = r < (uint32_t)O;
                if (valid) y[r] = acc;
                if constexpr (MODE == 1) {
                    const unsigned long long key = valid ? arg_key(tk.epoch, acc, r) : 0ull;
                    best = key > best ? key : best;
                }
                if constexpr (MODE == 2) {
                    const unsigned long long key = valid ? arg_key(tk.epoch, acc, r) : best & (0xFFull << 56);
                    __hip_atomic_store(&cand[slot + seg], key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    best = key > best ? key : best;
                }
            }
            if constexpr (MODE == 2) slot += RPW;
        }
    }
    if constexpr (MODE == 1) {
        __shared__ unsigned long long s_best[kWaves];
        best = wave_max_u64(best);
        if (lane == 0) s_best[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = s_best[0];
#pragma unroll
            for (int w = 1; w < kWaves; w++) b = s_best[w] > b ? s_best[w] : b;
            atomicMax(&tk.slots[blockIdx.x % kArgSlots], b);
        }
    }
    if constexpr (MODE == 2) {
        const unsigned long long pad = (unsigned long long)(tk.epoch & 0xFFu) << 56;
        for (int e = slot + lane; e < per_wave; e += 64)   // slots this wave's rows did not reach
            __hip_atomic_store(&cand[e], pad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        best = wave_max_u64(best);
        if (lane == 0)
            __hip_atomic_store(&tk.slots[blockIdx.x * kWaves + wave], best, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (blockIdx.x == gridDim.x - 1) topk_final_block(tk, gridDim.x * kWaves, per_wave);
    }
}

// clear the fused top-k keys (all tags 0) when the 8-bit launch tag wraps
__global__ void keys_reset(unsigned long long *keys, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) keys[i] = 0ull;
}

// Top-k pass over a logit vector: each block keeps per-thread lists of a strided slice
// and publishes its k best; topk_final merges the blocks.  Re-reads 4 bytes per logit.
__global__ __launch_bounds__(kThreads) void topk_partial(const float *__restrict__ v, int n, TopkArgs tk) {
    float tv[kTopK];
    int ti[kTopK];
    topk_clear<kTopK>(tv, ti);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads)
        topk_insert<kTopK>(tv, ti, v[i], i);
    topk_publish(tv, ti, tk);
}

// ----------------------------------------------------------------------------------
// Generic fp32 path: fmt 6 with any gs % 8 == 0 (per-word group partials as in
// c/shaders/qmatmul.comp:112-126), fmt 1 int8 rows (c/qwen.c:230-238), fmt 0 f32 rows
// (c/qwen.c:178-189).  One wave per row, lanes over 16-byte chunks.
__global__ __launch_bounds__(kThreads) void gemv_generic(const uint8_t *__restrict__ W, const float *__restrict__ SZ,
                                                         const float *__restrict__ x, float *__restrict__ y, int fmt,
                                                         int I, int O, int gs, int ng, int nchunks, int row_bytes) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int r = blockIdx.x * kWaves + wave; r < O; r += gridDim.x * kWaves) {
        const uint8_t *row = W + (size_t)r * row_bytes;
        float acc = 0.f;
        for (int c = lane; c < nchunks; c += 64) {
            const uint4 q = ((const uint4 *)row)[c];
            const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
            if (fmt == 6) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int i0 = c * 32 + j * 8;
                    if (i0 >= I) break;
                    const int g = i0 / gs;
                    const float sc = SZ[((size_t)r * ng + g) * 2], zr = SZ[((size_t)r * ng + g) * 2 + 1];
                    float awn = 0.f, ax = 0.f;
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const int i = i0 + k;
                        if (i < I) {
                            const float xv = x[i];
                            awn = fmaf(xv, (float)((wv[j] >> (4 * k)) & 15u), awn);
                            ax += xv;
                        }
                    }
                    acc = fmaf(sc, awn - zr * ax, acc);
                }
            } else if (fmt == 1) {
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int i = c * 16 + j * 4 + k;
                        if (i < I) acc = fmaf(x[i], (float)(int8_t)(wv[j] >> (8 * k)), acc);
                    }
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int i = c * 4 + j;
                    if (i < I) acc = fmaf(x[i], __uint_as_float(wv[j]), acc);
                }
            }
        }
        acc = seg_sum<64>(acc);
        if (lane == 63) y[r] = fmt == 1 ? acc * SZ[r] : acc;
    }
}

// zero-centred RMSNorm, one block per row (c/qwen.c:326-330: double sum of squares)
__global__ __launch_bounds__(kThreads) void rmsnorm_zc_kernel(const float *__restrict__ x,
                                                              const float *__restrict__ w, float *__restrict__ y,
                                                              int D, float eps) {
    __shared__ double s_r[kWaves];
    const float *xr = x + (size_t)blockIdx.x * D;
    float *yr = y + (size_t)blockIdx.x * D;
    double ms = 0;
    for (int i = threadIdx.x; i < D; i += kThreads) ms += (double)xr[i] * xr[i];
    for (int off = 32; off > 0; off >>= 1) ms += __shfl_xor(ms, off);
    if ((threadIdx.x & 63) == 0) s_r[threadIdx.x >> 6] = ms;
    __syncthreads();
    ms = 0;
    for (int wv = 0; wv < kWaves; wv++) ms += s_r[wv];
    const float r = 1.f / sqrtf((float)(ms / D) + eps);
    for (int i = threadIdx.x; i < D; i += kThreads) yr[i] = xr[i] * r * (1.f + w[i]);
}

// ---------------------------------------------------------------------------------- launch
struct TopkScratch {
    void *buf = nullptr;
    size_t cap = 0;
};
static TopkScratch g_tk;

static int pow2_at_least(int n) {
    int l = 1;
    while (l < n) l <<= 1;
    return l;
}

constexpr int kU = 4;           // row steps in flight per wave
constexpr int kMaxBlocksPerCU = 8;

// Resident blocks per CU of one kernel instantiation (queried once).
template <typename Kern>
static int occupancy(Kern kern) {
    static int v = 0;
    if (!v) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kThreads, 0) != hipSuccess || n < 1) n = 1;
        v = n > kMaxBlocksPerCU ? kMaxBlocksPerCU : n;
    }
    return v;
}

// persistent grid: enough blocks for the work, at most one resident wave of blocks
static int grid_size(long work_blocks, int per_cu) {
    const long cap = (long)n_cu() * per_cu;
    const long nb = work_blocks < cap ? work_blocks : cap;
    return nb < 1 ? 1 : (int)nb;
}

// returns the grid size used, 0 on failure
template <int LPR, int CU, int MODE>
static int launch_lanes(const ColiVkTensor *t, const float *x, float *y, hipStream_t st, const TopkArgs &ta) {
    constexpr int rpw = 64 / LPR;
    const long nrg = (t->O + rpw - 1) / rpw;
    const long work = (nrg + (long)kWaves * kU - 1) / ((long)kWaves * kU);
    auto kern = gemv6_lanes<LPR, CU, kU, MODE>;
    int nb = grid_size(work, occupancy(kern));
    if (MODE == 2 && nb > kFusedGrid) nb = kFusedGrid;   // the fused merge reads at most kFusedGrid blocks
    int per_wave = 0;
    size_t lds = 0;
    if (MODE == 2) {
        const long nw = (long)nb * kWaves;
        per_wave = (int)((nrg + nw * kU - 1) / (nw * kU)) * kU * rpw;   // slots one wave fills
        if (per_wave > kFusedSlots) return 0;   // more rows than the fused merge reads per wave
    }
    hipLaunchKernelGGL(kern, dim3(nb), dim3(kThreads), lds, st, t->w, t->sz, x, y, t->I, t->O, t->gs, t->ng, t->nl,
                       t->row_bytes, ta, per_wave);
    return nb;
}

template <int CU, int MODE>
static int launch_lanes_cu(const ColiVkTensor *t, const float *x, float *y, hipStream_t st, const TopkArgs &ta) {
    switch (pow2_at_least(t->nl)) {
    case 1: return launch_lanes<1, CU, MODE>(t, x, y, st, ta);
    case 2: return launch_lanes<2, CU, MODE>(t, x, y, st, ta);
    case 4: return launch_lanes<4, CU, MODE>(t, x, y, st, ta);
    case 8: return launch_lanes<8, CU, MODE>(t, x, y, st, ta);
    case 16: return launch_lanes<16, CU, MODE>(t, x, y, st, ta);
    case 32: return launch_lanes<32, CU, MODE>(t, x, y, st, ta);
    case 64: return launch_lanes<64, CU, MODE>(t, x, y, st, ta);
    default: return 0;
    }
}

// fmt 6 lanes-layout GEMV in one of the modes; returns the grid size (0 = not launched)
template <int MODE>
static int launch_lanes_mode(const ColiVkTensor *t, const float *x, float *y, hipStream_t st, const TopkArgs &ta) {
    const int nb = t->gs >= 32 * kLaneChunks ? launch_lanes_cu<kLaneChunks, MODE>(t, x, y, st, ta)
                                             : launch_lanes_cu<1, MODE>(t, x, y, st, ta);
    if (nb) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("gemv launch", e) ? 1 : 0;
    }
    return nb;
}

static bool launch_one(const ColiVkTensor *t, const float *x, float *y, hipStream_t st) {
    int nb;
    if (t->layout == kLayoutLanes) {
        const TopkArgs none = {0, nullptr, nullptr, nullptr, 0, nullptr, nullptr};
        nb = launch_lanes_mode<0>(t, x, y, st, none);
    } else {
        nb = grid_size((t->O + kWaves - 1) / kWaves, occupancy(gemv_generic));
        hipLaunchKernelGGL(gemv_generic, dim3(nb), dim3(kThreads), 0, st, t->w, t->sz, x, y, t->fmt, t->I, t->O,
                           t->gs, t->ng, t->nchunks, t->row_bytes);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("gemv launch", e);
    }
    return nb != 0;
}

static void *g_logits = nullptr;   // logits of a top-k launch whose caller wants none
static size_t g_logits_cap = 0;
static void *g_slots = nullptr;    // argmax slots (kArgSlots keys)
static size_t g_slots_cap = 0;
static uint32_t g_epoch = 0;
static void *g_keys = nullptr;     // fused top-k keys: wave maxima, then per-slot candidates
static size_t g_keys_cap = 0;
static uint32_t g_tk_epoch = 0;

bool topk(const float *d_v, int n, int k, int *d_idx, float *d_val, hipStream_t st) {
    if (k < 1 || k > kTopK || n < 1) return false;
    long nbp = ((long)n + kThreads * 8 - 1) / (kThreads * 8);
    if (nbp > (long)n_cu() * 2) nbp = (long)n_cu() * 2;
    if (!scratch(&g_tk.buf, &g_tk.cap, (size_t)nbp * kTopK * 8)) return false;
    TopkArgs ta = {k, (float *)g_tk.buf, (int *)((float *)g_tk.buf + (size_t)nbp * kTopK), nullptr, 0, nullptr, nullptr};
    hipLaunchKernelGGL(topk_partial, dim3((unsigned)nbp), dim3(kThreads), 0, st, d_v, n, ta);
    hipLaunchKernelGGL(topk_final, dim3(1), dim3(kFinalThreads), 0, st, ta.part_v, ta.part_i, (int)nbp, k, d_val,
                       d_idx);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("topk launch", e);
    return true;
}

// GEMV whose blocks also fold their best row into the argmax slots (fmt 6 lanes layout,
// O < 2^24).  *epoch receives the launch tag; the slots hold the result after the kernel.
bool gemv_argmax(const ColiVkTensor *t, const float *d_x, float *d_y, hipStream_t st, uint32_t *epoch,
                 const unsigned long long **slots) {
    if (t->layout != kLayoutLanes || t->O >= (1 << 24)) return false;
    if (!d_y) {
        if (!scratch(&g_logits, &g_logits_cap, (size_t)t->O * 4)) return false;
        d_y = (float *)g_logits;
    }
    if (!scratch(&g_slots, &g_slots_cap, kArgSlots * 8)) return false;   // zeroed when allocated
    g_epoch = (g_epoch + 1) & 0xFFu;
    if (g_epoch == 0) {   // tags wrap: clear the slots so no old key outranks the new tag
        hipLaunchKernelGGL(argmax_reset, dim3(1), dim3(64), 0, st, (unsigned long long *)g_slots);
        g_epoch = 1;
    }
    const TopkArgs ta = {1, nullptr, nullptr, (unsigned long long *)g_slots, g_epoch, nullptr, nullptr};
    if (!launch_lanes_mode<1>(t, d_x, d_y, st, ta)) return false;
    *epoch = g_epoch;
    *slots = (const unsigned long long *)g_slots;
    return true;
}

bool gemv(const ColiVkTensor *t, const float *d_x, float *d_y, int S, hipStream_t st, const TopkOut *tk) {
    if (!t || S < 1) return false;
    const bool want_k = tk && tk->k > 0;
    if (want_k && (S != 1 || tk->k > kTopK)) return false;
    if (!d_y) {
        if (!scratch(&g_logits, &g_logits_cap, (size_t)S * t->O * 4)) return false;
        d_y = (float *)g_logits;
    }
    if (want_k && tk->k == 1 && t->layout == kLayoutLanes && t->O < (1 << 24)) {
        uint32_t ep;
        const unsigned long long *sl;
        if (!gemv_argmax(t, d_x, d_y, st, &ep, &sl)) return false;
        hipLaunchKernelGGL(argmax_decode, dim3(1), dim3(64), 0, st, sl, ep, tk->idx, tk->val);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("argmax decode", e);
        return true;
    }
    if (want_k && t->layout == kLayoutLanes && t->O < (1 << 24)) {   // fused: one launch
        const int n = kFusedWaves + kFusedGrid * kWaves * kFusedSlots;
        if (!scratch(&g_keys, &g_keys_cap, (size_t)n * 8)) return false;
        g_tk_epoch = (g_tk_epoch + 1) & 0xFFu;
        if (g_tk_epoch == 0) {   // tags wrap: clear the keys so no old key carries the new tag
            hipLaunchKernelGGL(keys_reset, dim3((n + 255) / 256), dim3(256), 0, st, (unsigned long long *)g_keys, n);
            g_tk_epoch = 1;
        }
        const TopkArgs ta = {tk->k, nullptr, nullptr, (unsigned long long *)g_keys, g_tk_epoch, tk->idx, tk->val};
        if (launch_lanes_mode<2>(t, d_x, d_y, st, ta)) return true;
        if (!ok()) return false;   // otherwise (LDS too small) fall through to separate passes
    }
    for (int s = 0; s < S; s++)
        if (!launch_one(t, d_x + (size_t)s * t->I, d_y + (size_t)s * t->O, st)) return false;
    return want_k ? topk(d_y, t->O, tk->k, tk->idx, tk->val, st) : true;
}

// host side of an argmax slot read-back: the best key of `epoch` -> (idx, val)
bool argmax_decode_host(const unsigned long long *keys, uint32_t epoch, int *idx, float *val) {
    unsigned long long best = 0;
    for (int i = 0; i < kArgSlots; i++) best = keys[i] > best ? keys[i] : best;
    if ((uint32_t)(best >> 56) != (epoch & 0xFFu)) return false;
    const uint32_t ord = (uint32_t)(best >> 24);
    const uint32_t u = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    *idx = (int)(0xFFFFFFu - (uint32_t)(best & 0xFFFFFFu));
    if (val) memcpy(val, &u, 4);
    return true;
}

bool rmsnorm_zc(const float *d_x, const float *d_w, float *d_y, int D, float eps, hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_zc_kernel, dim3(1), dim3(kThreads), 0, st, d_x, d_w, d_y, D, eps);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("rmsnorm launch", e);
    return true;
}

// ----------------------------------------------------------------------------------
// host-buffer entry points: stage through pinned buffers, one sync per call
struct Stage {
    void *hx = nullptr, *hy = nullptr, *dx = nullptr, *dy = nullptr, *dk = nullptr;
    size_t hxc = 0, hyc = 0, dxc = 0, dyc = 0, dkc = 0;
};
static Stage g_st;

static bool stage_x(const float *x, size_t xb) {
    if (!host_scratch(&g_st.hx, &g_st.hxc, xb) || !scratch(&g_st.dx, &g_st.dxc, xb)) return false;
    memcpy(g_st.hx, x, xb);
    const hipError_t e = hipMemcpyAsync(g_st.dx, g_st.hx, xb, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("x upload", e);
    return true;
}

static bool fetch(void *dst, const void *dsrc, size_t bytes, const char *who) {
    if (!host_scratch(&g_st.hy, &g_st.hyc, bytes)) return false;
    hipError_t e = hipMemcpyAsync(g_st.hy, dsrc, bytes, hipMemcpyDeviceToHost, stream());
    if (e == hipSuccess) e = hipStreamSynchronize(stream());
    if (e != hipSuccess) return fail(who, e);
    memcpy(dst, g_st.hy, bytes);
    return true;
}

}  // namespace coli

using namespace coli;

extern "C" int coli_vk_tensor_ensure(ColiVkTensor **, const void *, const float *, int, int, int, int);

// c/backend_vulkan.h:58-61, c/backend_vulkan.c:1215-1295
COLI_API int coli_vk_matmul(ColiVkTensor **tensor, float *y, const float *x, const void *weights,
                            const float *scales, int fmt, int S, int I, int O, int gs) {
    if (!tensor || !y || !x || S < 1) return 0;
    if (!coli_vk_tensor_ensure(tensor, weights, scales, fmt, I, O, gs)) return 0;
    const ColiVkTensor *t = *tensor;
    const size_t xb = (size_t)S * I * 4, yb = (size_t)S * O * 4;
    if (!stage_x(x, xb) || !scratch(&g_st.dy, &g_st.dyc, yb)) return 0;
    if (!gemv(t, (const float *)g_st.dx, (float *)g_st.dy, S, stream())) return 0;
    return fetch(y, g_st.dy, yb, "matmul") ? 1 : 0;
}

// c/backend_vulkan.h:128-130, c/backend_vulkan.c:3906-3955: two GEMVs sharing x, one sync
COLI_API int coli_vk_matmul_pair(ColiVkTensor **t1p, float *y1, const void *w1, const float *s1, int O1,
                                 ColiVkTensor **t2p, float *y2, const void *w2, const float *s2, int O2,
                                 int fmt, const float *x, int S, int I, int grp) {
    if (!t1p || !t2p || !y1 || !y2 || !x || S < 1) return 0;
    if (!coli_vk_tensor_ensure(t1p, w1, s1, fmt, I, O1, grp) || !coli_vk_tensor_ensure(t2p, w2, s2, fmt, I, O2, grp))
        return 0;
    const size_t xb = (size_t)S * I * 4, y1b = (size_t)S * O1 * 4, yb = y1b + (size_t)S * O2 * 4;
    if (!stage_x(x, xb) || !scratch(&g_st.dy, &g_st.dyc, yb)) return 0;
    float *dy = (float *)g_st.dy;
    if (!gemv(*t1p, (const float *)g_st.dx, dy, S, stream()) ||
        !gemv(*t2p, (const float *)g_st.dx, dy + (size_t)S * O1, S, stream()))
        return 0;
    if (!host_scratch(&g_st.hy, &g_st.hyc, yb)) return 0;
    hipError_t e = hipMemcpyAsync(g_st.hy, dy, yb, hipMemcpyDeviceToHost, stream());
    if (e == hipSuccess) e = hipStreamSynchronize(stream());
    if (e != hipSuccess) return fail("matmul_pair", e);
    memcpy(y1, g_st.hy, y1b);
    memcpy(y2, (uint8_t *)g_st.hy + y1b, yb - y1b);
    return 1;
}

// c/backend_vulkan.h:68-71, c/backend_vulkan.c:1355-1405: GEMV + device argmax; only the
// argmax slots (128 bytes) cross the bus and the host picks the winner (ties -> lowest
// index, c/shaders/argmax.comp:7-9).
COLI_API int coli_vk_matmul_argmax(ColiVkTensor **tensor, const void *weights, const float *scales, int fmt,
                                   int I, int O, int gs, const float *x, int *idx, float *val) {
    if (!tensor || !x || !idx || O < 1) return 0;
    if (!coli_vk_tensor_ensure(tensor, weights, scales, fmt, I, O, gs)) return 0;
    if (!stage_x(x, (size_t)I * 4)) return 0;
    uint32_t ep;
    const unsigned long long *sl;
    if (gemv_argmax(*tensor, (const float *)g_st.dx, nullptr, stream(), &ep, &sl)) {
        unsigned long long keys[kArgSlots];
        if (!fetch(keys, sl, sizeof(keys), "matmul_argmax")) return 0;
        return argmax_decode_host(keys, ep, idx, val) ? 1 : 0;
    }
    if (!ok() || !scratch(&g_st.dk, &g_st.dkc, 64)) return 0;   // other layouts: top-1 passes
    TopkOut tk = {1, (int *)g_st.dk, (float *)g_st.dk + 8};
    if (!gemv(*tensor, (const float *)g_st.dx, nullptr, 1, stream(), &tk)) return 0;
    int res[16];
    if (!fetch(res, g_st.dk, 64, "matmul_argmax")) return 0;
    *idx = res[0];
    if (val) memcpy(val, &res[8], 4);
    return 1;
}

// ---- device-pointer entry points (inputs already resident in HBM) ----------------
// y[S, O] = x[S, I] @ dequant(W)^T on `stream` (NULL = the library's stream).
COLI_API int coli_hip_gemv(const ColiVkTensor *t, const float *d_x, float *d_y, int S, void *stream_) {
    if (!ok() || !t) return 0;
    return gemv(t, d_x, d_y, S, stream_ ? (hipStream_t)stream_ : stream()) ? 1 : 0;
}

// GEMV fused with the top-k (k <= 8) of its outputs: d_idx/d_val receive the k best
// (value desc, index asc).  d_y may be NULL (outputs stay unwritten).  Top-k launches
// share one partials buffer: issue them on one stream.
COLI_API int coli_hip_gemv_topk(const ColiVkTensor *t, const float *d_x, float *d_y, int k, int *d_idx,
                                float *d_val, void *stream_) {
    if (!ok() || !t || k < 1 || k > kTopK || !d_idx || !d_val) return 0;
    TopkOut tk = {k, d_idx, d_val};
    return gemv(t, d_x, d_y, 1, stream_ ? (hipStream_t)stream_ : stream(), &tk) ? 1 : 0;
}

// the library's stream (for callers that time or order work against it)
COLI_API void *coli_hip_stream(void) { return (void *)stream(); }
