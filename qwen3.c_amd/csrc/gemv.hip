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
// Top-k (fused): each wave keeps the k best of its rows in registers and publishes them as
// epoch-tagged 64-bit keys; the first block of the grid to finish merges them in the same
// launch, polling the tags (agent-scope atomics: no device-scope fences, no second launch).
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
    int *err;                    // fused top-k: set to 1 when a bounded poll gives up
    const float *xw;             // argmax: x := zero-centred RMSNorm of x with weight xw (none if null)
    float eps;
};

// ---- argmax as a 64-bit key: [63:56] launch epoch, [55:24] order-preserving bits of the
// value, [23:0] 0xFFFFFF - row.  The maximum key is the best (value desc, row asc) of the
// launch; a stale key of an earlier launch (lower epoch) always loses.  Rows < 2^24.
static_assert(kArgSlots == 16, "blocks spread their atomicMax over 16 slots (contention)");
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
__device__ __forceinline__ void topk_publish(float (&tv)[kTopK], int (&ti)[kTopK], const TopkArgs &tk) {
    block_topk_merge<kTopK>(tv, ti, tk.k, tk.part_v + blockIdx.x * kTopK, tk.part_i + blockIdx.x * kTopK);
}

__device__ __forceinline__ unsigned long long aload64(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kFusedGrid = kThreads;       // largest grid of a fused top-k launch (one list per thread)
constexpr int kTkBuf = 256;                // row results a wave buffers between selections
constexpr int kFusedPollLimit = 1 << 20;

// decode a key into (row, value); the padding key (tag only) -> (INT_MAX, -inf)
__device__ __forceinline__ void key_decode(unsigned long long key, int *row, float *val) {
    const uint32_t low = (uint32_t)(key & 0xFFFFFFu);
    if ((key & 0x00FFFFFFFFFFFFFFull) == 0ull || low == 0u) {
        *row = INT_MAX;
        *val = -INFINITY;
        return;
    }
    const uint32_t ord = (uint32_t)(key >> 24);
    const uint32_t u = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    *row = (int)(0xFFFFFFu - low);
    *val = __uint_as_float(u);
}

// One wave ranks keys[0, n) in LDS (n <= 64; 16-byte aligned, zeros from n up to the next
// multiple of 8: zero is below every key, so the counting loop reads without conditions)
// by counting for each key the keys above it; out (LDS) gets the key of rank r < kTopK.
// Real keys are unique (the row is part of the key); equal padding keys share a rank, so
// out is filled with the padding key first.  The keys were written by the block before a
// barrier the caller has passed; only the calling wave's LDS operations touch out, and
// they complete in issue order, so no block barrier is needed.
__device__ __forceinline__ void rank_keys_wave(const unsigned long long *keys, int n, unsigned long long pad,
                                               unsigned long long *out) {
    const int lane = threadIdx.x & 63;
    if (lane < kTopK) out[lane] = pad;
    asm volatile("" ::: "memory");
    const ulonglong2 *k2 = (const ulonglong2 *)keys;
    const unsigned long long me = lane < n ? keys[lane] : 0ull;
    int r = 0;
    for (int o = 0; o < (n + 7) / 8 * 4; o += 4) {
        ulonglong2 q[4];
#pragma unroll
        for (int u = 0; u < 4; u++) q[u] = k2[o + u];
#pragma unroll
        for (int u = 0; u < 4; u++) r += (q[u].x > me ? 1 : 0) + (q[u].y > me ? 1 : 0);
    }
    if (lane < n && r < kTopK) out[r] = me;
    asm volatile("" ::: "memory");
}

// Arrival counter of a fused top-k launch: two, used by launch-tag parity, after the keys.
__device__ __forceinline__ unsigned *topk_counter(const TopkArgs &tk, uint32_t epoch) {
    return (unsigned *)(tk.slots + (size_t)kFusedGrid * kTopK) + (epoch & 1u);
}

// Poll the kTopK tagged keys at p until all carry the launch's tag (bounded).
__device__ __forceinline__ void poll_keys(const unsigned long long *p, unsigned long long tag,
                                          unsigned long long (&v)[kTopK], int *bad) {
    for (int polls = 0;; polls++) {
        bool all = true;
#pragma unroll
        for (int q = 0; q < kTopK; q++) {
            v[q] = aload64(p + q);
            all &= (v[q] >> 56) == tag;
        }
        if (all) return;
        if (polls > kFusedPollLimit) {
            *bad = 1;
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Wave-wide maximum of 64-bit keys by DPP (high words, then low words among the lanes
// holding the highest high word), broadcast to all lanes.
__device__ __forceinline__ uint32_t wave_umax32(uint32_t v) {
    v = COLI_DPP_UMAX(v, 0xB1, 0xF);    // quad_perm [1,0,3,2]
    v = COLI_DPP_UMAX(v, 0x4E, 0xF);    // quad_perm [2,3,0,1]
    v = COLI_DPP_UMAX(v, 0x141, 0xF);   // row_half_mirror
    v = COLI_DPP_UMAX(v, 0x140, 0xF);   // row_mirror
    v = COLI_DPP_UMAX(v, 0x142, 0xA);   // row_bcast15
    v = COLI_DPP_UMAX(v, 0x143, 0xC);   // row_bcast31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long k) {
    const uint32_t hi = (uint32_t)(k >> 32), mh = wave_umax32(hi);
    const uint32_t ml = wave_umax32(hi == mh ? (uint32_t)k : 0u);
    return ((unsigned long long)mh << 32) | ml;
}

// lane l's 64-bit value, wave uniform
__device__ __forceinline__ unsigned long long readlane64(unsigned long long v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((unsigned long long)hi << 32) | lo;
}

// compare-exchange of 64-bit keys: a gets the larger
__device__ __forceinline__ void cx_desc(unsigned long long &a, unsigned long long &b) {
    const unsigned long long hi = a > b ? a : b, lo = a > b ? b : a;
    a = hi;
    b = lo;
}

// kTopK rounds of a wave maximum over the lanes' sorted lists L (descending, 0 = none):
// the lane holding the winner moves to its next key.  Returns, in lane r < kTopK, the
// wave's key of rank r (pad when the lists ran out).
template <int N>
__device__ __forceinline__ unsigned long long wave_rounds(unsigned long long (&L)[N], unsigned long long pad) {
    const int lane = threadIdx.x & 63;
    unsigned long long out = pad;
#pragma unroll
    for (int r = 0; r < kTopK; r++) {
        // the head with the largest value bits (key bits 55:24) wins; only when several
        // heads share them does the full 64-bit maximum (row order) decide
        const uint32_t h = (uint32_t)(L[0] >> 24);
        const uint32_t mh = wave_umax32(h);
        const unsigned long long tied = __ballot(h == mh);
        int w;
        if (__popcll(tied) == 1) {
            w = __ffsll((long long)tied) - 1;
        } else {
            const unsigned long long mt = wave_max_key(h == mh ? L[0] : 0ull);
            w = __ffsll((long long)__ballot(L[0] == mt)) - 1;
        }
        const unsigned long long m = readlane64(L[0], w);
        if (lane == w) {
#pragma unroll
            for (int q = 0; q + 1 < N; q++) L[q] = L[q + 1];
            L[N - 1] = 0ull;
        }
        if (lane == r) out = m > pad ? m : pad;
    }
    return out;
}

// The block that arrives first: the k best keys of the launch from the blocks' sorted lists
// (cand[b * kTopK + e]; nblk <= kThreads).  Thread t polls block t's list until its keys
// carry the launch's tag, so the merge ends soon after the last block's keys land (a last
// block that merged would first wait for its arrival count to return); the other blocks
// wait on nothing, so every list arrives.  Each wave takes
// kTopK rounds of a wave maximum over its lanes' list heads (the lane whose head wins
// moves to its next key), and the 4 wave lists are ranked in LDS.  Keys of another launch
// carry another tag and are polled until overwritten.
__device__ __forceinline__ void topk_final_block(const TopkArgs &tk, int nblk) {
    __shared__ __attribute__((aligned(16))) unsigned long long s_wl[kWaves * kTopK];
    __shared__ unsigned long long s_top[kTopK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const unsigned long long tag = (unsigned long long)(tk.epoch & 0xFFu), pad = tag << 56;
    int bad = 0;
    unsigned long long L[kTopK];
    if (tid < nblk) {
        poll_keys(tk.slots + (size_t)tid * kTopK, tag, L, &bad);
    } else {
#pragma unroll
        for (int q = 0; q < kTopK; q++) L[q] = 0ull;
    }
    const unsigned long long wl = wave_rounds<kTopK>(L, pad);   // lane r: the wave's key of rank r
    if (lane < kTopK) s_wl[wave * kTopK + lane] = wl;
    bad = __syncthreads_or(bad);
    if (wave != 0) return;   // wave 0 ranks the 4 wave lists and writes the result
    rank_keys_wave(s_wl, kWaves * kTopK, pad, s_top);
    if (lane < tk.k) {
        int row;
        float v;
        key_decode(s_top[lane], &row, &v);
        tk.out_i[lane] = bad ? -1 : row;
        tk.out_v[lane] = v;
    }
    if (bad && lane == 0) __hip_atomic_store(tk.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
//   MODE 2: also top-k, fused: every wave keeps the kTopK best keys of its rows (value
//           desc, row asc) distributed over lanes 0..kTopK-1; its leader lanes park their
//           results in LDS, and every kTkBuf rows (and at the end) the wave selects the new
//           list from them and the old list by kTopK rounds of a wave maximum.  At the end
//           the block ranks its waves' lists into one list that it stores as tagged keys
//           and counts itself in; the block that arrives first merges the blocks' lists
//           as they land (topk_final_block).
// The grid is persistent with few waves per CU (COLI_GEMV_BPC blocks): with U row steps
// of every wave in flight that keeps ~8-10 MB of loads outstanding chip-wide, where HBM
// streams best (more outstanding requests only add DRAM page conflicts).
template <int LPR, int CU, int U, int MODE>
__global__ __launch_bounds__(kThreads) void gemv6_lanes(const uint8_t *__restrict__ W, const float *__restrict__ SZ,
                                                        const float *__restrict__ x, float *__restrict__ y, int I,
                                                        int O, int gs, int ng, int nl, int row_bytes, TopkArgs tk) {
    __shared__ XPrep P;
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane % LPR, seg = lane / LPR;
    const uint32_t wtot = (uint32_t)O * (uint32_t)row_bytes, srb = (uint32_t)ng * 8u, stot = (uint32_t)O * srb;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(W, wtot), rs = buf_rsrc(SZ, stot);
    const int ncols = nl * kLaneChunks * 32;
    XRegs xr, wr;
    prep_load(x, I, ncols, xr);   // x first: in-order load counters then let the
    if constexpr (MODE == 1)      // weight prefetch stay in flight through the prologue
        prep_load(tk.xw ? tk.xw : x, tk.xw ? I : 0, ncols, wr);   // no norm: reads 0, no memory access
    LaneX<CU> L;
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
    if constexpr (MODE == 1)
        if (tk.xw) {   // c/qwen.c:326-330 (the final norm before lm_head)
            __shared__ double s_red[kWaves];
            norm_apply(xr, wr, I, ncols, tk.eps, s_red);
        }
    prep_x(xr, gs, ncols, P);
    lane_x<CU>(P, gs, L);

    const uint32_t rlim = (uint32_t)((O + RPW - 1) / RPW) * RPW;   // rows the grid walks
    if (MODE == 2 && blockIdx.x == 0 && threadIdx.x == 0)   // the previous launch's counter is free now
        __hip_atomic_store(topk_counter(tk, tk.epoch + 1), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned long long best = 0ull;   // MODE 1: best key of this lane's rows
    // MODE 2: the wave's k best keys (lane q < kTopK: key q); the padding key is the tag
    // alone, below every real key of the launch
    const unsigned long long pad = (unsigned long long)(tk.epoch & 0xFFu) << 56;
    unsigned long long tl = pad;   // lane q < kTopK: the wave's key of rank q so far
    // MODE 2: leader lanes buffer their row results in LDS (row r of wave step s goes to
    // entry (s - s0) * RPW + seg); every kWin steps, and at the end, the wave turns them
    // into keys and offers them to its list, 64 at a time.
    constexpr int kBuf = RPW * U > kTkBuf ? RPW * U : kTkBuf;
    constexpr int kWin = kBuf / RPW / U * U;
    __shared__ float s_tk[MODE == 2 ? kWaves : 1][MODE == 2 ? kBuf : 1];
    int win = 0, s0 = 0;   // steps buffered, step of entry 0 (wave uniform)
    auto flush = [&]() {
        // A wave's LDS operations complete in issue order, so its lanes read what its
        // lanes wrote; only compiler reordering is fenced (a hardware fence here would wait
        // for the weight loads in flight).  Lane l takes entries l + 64 q and the list key
        // of rank l (lanes < kTopK), sorts its 5 keys, and kTopK wave rounds select.
        asm volatile("" ::: "memory");
        const int n = win * RPW;
        constexpr int NQ = kBuf / 64 > 0 ? kBuf / 64 : 1;
        unsigned long long L[NQ + 1];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int e = q * 64 + lane;
            L[q] = 0ull;
            if (e < n) {
                const uint32_t r = (uint32_t)((rg0 + (s0 + e / RPW) * nw) * RPW + e % RPW);
                if (r < (uint32_t)O) L[q] = arg_key(tk.epoch, s_tk[wave][e], r);
            }
        }
        L[NQ] = lane < kTopK ? tl : 0ull;
#pragma unroll
        for (int i = 0; i < NQ + 1; i++)   // odd-even transposition sort, descending
#pragma unroll
            for (int q = i & 1; q + 1 < NQ + 1; q += 2) cx_desc(L[q], L[q + 1]);
        tl = wave_rounds<NQ + 1>(L, pad);
        asm volatile("" ::: "memory");
        s0 += win;
        win = 0;
    };
    for (uint32_t base = (uint32_t)rg0 * RPW; base < rlim; base += rstep) {
        if constexpr (MODE == 2)
            if (win + U > kWin) flush();
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float part = lane_row<CU>(wq[u], sv[u], L);
            const uint32_t r = rr[u];
            rr[u] += rstep;   // refill this slot with its next row while the others compute
            wro[u] += wstep;
            sro[u] += sstep;
            lane_load<CU>(rw, rs, min(wro[u], wtot), min(sro[u], stot), L, wq[u], sv[u]);
            const float acc = seg_sum<LPR>(part);
            const bool lead = j == LPR - 1 && r < (uint32_t)O;
            if (lead) {
                y[r] = acc;
                if constexpr (MODE == 1) {
                    const unsigned long long key = arg_key(tk.epoch, acc, r);
                    best = key > best ? key : best;
                }
            }
            if constexpr (MODE == 2)
                if (j == LPR - 1) s_tk[wave][(win + u) * RPW + seg] = acc;
        }
        if constexpr (MODE == 2) win += U;
    }
    if constexpr (MODE == 2) flush();
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
    if constexpr (MODE == 2) {   // the block's list: rank the waves' lists in LDS
        __shared__ __attribute__((aligned(16))) unsigned long long s_wl[kWaves * kTopK];
        __shared__ unsigned long long s_bl[kTopK];
        __shared__ int s_merge;
        if (lane < kTopK) s_wl[wave * kTopK + lane] = tl;
        __syncthreads();
        if (wave == 0) {   // one wave ranks the block's list and stores it
            rank_keys_wave(s_wl, kWaves * kTopK, pad, s_bl);
            if (lane < kTopK)
                __hip_atomic_store(tk.slots + (size_t)blockIdx.x * kTopK + lane, s_bl[lane], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0)   // arrival count of this launch: the first block merges
                s_merge = __hip_atomic_fetch_add(topk_counter(tk, tk.epoch), 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) == 0;
        }
        __syncthreads();
        if (s_merge) topk_final_block(tk, gridDim.x);
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

// Launch shape of the fmt 6 GEMV (tuned on MI355X: 287 MB lm_head stream).
#ifndef COLI_GEMV_U
#define COLI_GEMV_U 4           // row steps in flight per wave
#endif
#ifndef COLI_GEMV_BPC
#define COLI_GEMV_BPC 1         // resident blocks per CU (4 waves each)
#endif
constexpr int kU = COLI_GEMV_U;
constexpr int kGemvBlocksPerCU = COLI_GEMV_BPC;
constexpr int kMaxBlocksPerCU = 8;

// Resident blocks per CU of one kernel instantiation, queried once per kernel (the cache is
// keyed by the kernel's address: every gemv6_lanes instantiation has the same type).
template <typename Kern>
static int occupancy(Kern kern) {
    static struct {
        const void *k;
        int v;
    } cache[64];
    static int n_cached = 0;
    const void *key = (const void *)kern;
    for (int i = 0; i < n_cached; i++)
        if (cache[i].k == key) return cache[i].v;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kThreads, 0) != hipSuccess || n < 1) n = 1;
    const int v = n > kMaxBlocksPerCU ? kMaxBlocksPerCU : n;
    if (n_cached < 64) cache[n_cached++] = {key, v};
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
    const int per = occupancy(kern);
    int nb = grid_size(work, per < kGemvBlocksPerCU ? per : kGemvBlocksPerCU);
    if (MODE == 2 && nb > kFusedGrid) nb = kFusedGrid;   // the fused merge reads at most kFusedGrid blocks
    hipLaunchKernelGGL(kern, dim3(nb), dim3(kThreads), 0, st, t->w, t->sz, x, y, t->I, t->O, t->gs, t->ng, t->nl,
                       t->row_bytes, ta);
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
    const int nb = t->gs % (32 * kLaneChunks) == 0 ? launch_lanes_cu<kLaneChunks, MODE>(t, x, y, st, ta)
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
        const TopkArgs none = {0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr};
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
static void *g_keys = nullptr;     // fused top-k: block lists [kFusedGrid][kTopK], then 2 counters
static size_t g_keys_cap = 0;
static uint32_t g_tk_epoch = 0;

bool topk(const float *d_v, int n, int k, int *d_idx, float *d_val, hipStream_t st) {
    if (k < 1 || k > kTopK || n < 1) return false;
    long nbp = ((long)n + kThreads * 8 - 1) / (kThreads * 8);
    if (nbp > (long)n_cu() * 2) nbp = (long)n_cu() * 2;
    if (!scratch(&g_tk.buf, &g_tk.cap, (size_t)nbp * kTopK * 8)) return false;
    TopkArgs ta = {k, (float *)g_tk.buf, (int *)((float *)g_tk.buf + (size_t)nbp * kTopK), nullptr, 0, nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(topk_partial, dim3((unsigned)nbp), dim3(kThreads), 0, st, d_v, n, ta);
    hipLaunchKernelGGL(topk_final, dim3(1), dim3(kFinalThreads), 0, st, ta.part_v, ta.part_i, (int)nbp, k, d_val,
                       d_idx);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("topk launch", e);
    return true;
}

// GEMV whose blocks also fold their best row into the argmax slots (fmt 6 lanes layout,
// O < 2^24).  *epoch receives the launch tag; the slots hold the result after the kernel.
// xw != NULL: x is normed first (zero-centred RMSNorm, weight xw, in each block's x
// prologue).  The kArgSpare words after the slots are the caller's.
bool gemv_argmax(const ColiVkTensor *t, const float *d_x, float *d_y, hipStream_t st, uint32_t *epoch,
                 unsigned long long **slots, const float *xw, float eps) {
    if (t->layout != kLayoutLanes || t->O >= (1 << 24)) return false;
    if (!d_y) {
        if (!scratch(&g_logits, &g_logits_cap, (size_t)t->O * 4)) return false;
        d_y = (float *)g_logits;
    }
    if (!scratch(&g_slots, &g_slots_cap, (kArgSlots + kArgSpare) * 8)) return false;   // zeroed when allocated
    g_epoch = (g_epoch + 1) & 0xFFu;
    if (g_epoch == 0) {   // tags wrap: clear the slots so no old key outranks the new tag
        hipLaunchKernelGGL(argmax_reset, dim3(1), dim3(64), 0, st, (unsigned long long *)g_slots);
        g_epoch = 1;
    }
    const TopkArgs ta = {1, nullptr, nullptr, (unsigned long long *)g_slots, g_epoch, nullptr, nullptr, nullptr, xw, eps};
    if (!launch_lanes_mode<1>(t, d_x, d_y, st, ta)) return false;
    *epoch = g_epoch;
    *slots = (unsigned long long *)g_slots;
    return true;
}

bool gemv(const ColiVkTensor *t, const float *d_x, float *d_y, int S, hipStream_t st, const TopkOut *tk) {
    if (!tensor_live(t) || S < 1) return false;
    const bool want_k = tk && tk->k > 0;
    if (want_k && (S != 1 || tk->k > kTopK)) return false;
    if (!d_y) {
        if (!scratch(&g_logits, &g_logits_cap, (size_t)S * t->O * 4)) return false;
        d_y = (float *)g_logits;
    }
    if (want_k && tk->k == 1 && t->layout == kLayoutLanes && t->O < (1 << 24)) {
        uint32_t ep;
        unsigned long long *sl;
        if (!gemv_argmax(t, d_x, d_y, st, &ep, &sl)) return false;
        hipLaunchKernelGGL(argmax_decode, dim3(1), dim3(64), 0, st, sl, ep, tk->idx, tk->val);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("argmax decode", e);
        return true;
    }
    if (want_k && t->layout == kLayoutLanes && t->O < (1 << 24)) {   // fused: one launch
        // block lists, then one word with the two counters, then the error word (not reset)
        const int n = kFusedGrid * kTopK + 1;
        if (!scratch(&g_keys, &g_keys_cap, (size_t)(n + 1) * 8)) return false;
        g_tk_epoch = (g_tk_epoch + 1) & 0xFFu;
        if (g_tk_epoch == 0) {   // tags wrap: clear keys and counters, no old key carries the new tag
            hipLaunchKernelGGL(keys_reset, dim3((n + 255) / 256), dim3(256), 0, st, (unsigned long long *)g_keys, n);
            g_tk_epoch = 1;
        }
        const TopkArgs ta = {tk->k,   nullptr, nullptr, (unsigned long long *)g_keys, g_tk_epoch, tk->idx, tk->val,
                             (int *)((unsigned long long *)g_keys + n)};
        return launch_lanes_mode<2>(t, d_x, d_y, st, ta) != 0;
    }
    if (S >= kGemmMinS && gemm6_ok(t)) return gemm6(&t, &d_y, 1, d_x, S, st);   // c/backend_vulkan.c:282-299
    if (S >= 2 && !want_k && gemm_f01_ok(t, d_x)) return gemm_f01(t, d_x, d_y, S, st);
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
// host-buffer entry points: x up through the pinned upload staging, y back through pinned
// buffers, one sync per call
struct Stage {
    void *hy = nullptr, *dx = nullptr, *dy = nullptr, *dk = nullptr;
    size_t hyc = 0, dxc = 0, dyc = 0, dkc = 0;
};
static Stage g_st;

static bool stage_x(const float *x, size_t xb) {
    if (!scratch(&g_st.dx, &g_st.dxc, xb)) return false;
    const Upload u = {g_st.dx, x, xb};
    return upload(&u, 1, stream(), "x upload");
}

static bool fetch(void *dst, const void *dsrc, size_t bytes, const char *who) {
    return read_back(dst, dsrc, bytes, stream(), who);
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
    const ColiVkTensor *tp[2] = {*t1p, *t2p};
    float *const yp[2] = {dy, dy + (size_t)S * O1};
    if (S >= kGemmMinS && gemm6_ok(tp[0]) && gemm6_ok(tp[1])) {   // one digit decomposition of x for both
        if (!gemm6(tp, yp, 2, (const float *)g_st.dx, S, stream())) return 0;
    } else if (!gemv(tp[0], (const float *)g_st.dx, yp[0], S, stream()) ||
               !gemv(tp[1], (const float *)g_st.dx, yp[1], S, stream())) {
        return 0;
    }
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
    unsigned long long *sl;
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
    if (res[0] < 0 || res[0] >= O) return 0;   // a selection that gave up: the caller's host scan
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

namespace coli {
// Error word of the fused top-k launches since the last call (synchronises the device):
// 0 none, 1 a bounded wait of the merge gave up (that launch wrote -1 to d_idx), -1 runtime error.
int gemv_error_take() {
    if (!g_keys) return 0;
    int *w = (int *)((unsigned long long *)g_keys + kFusedGrid * kTopK + 1);
    int e = 0;
    // the device, not the library stream: a fused top-k may have run on a caller's stream
    if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(&e, w, 4, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    if (e) {
        const int z = 0;
        if (hipMemcpy(w, &z, 4, hipMemcpyHostToDevice) != hipSuccess) return -1;
    }
    return e;
}

void gemv_shutdown() {
    scratch_free(&g_tk.buf, &g_tk.cap);
    scratch_free(&g_logits, &g_logits_cap);
    scratch_free(&g_slots, &g_slots_cap);
    scratch_free(&g_keys, &g_keys_cap);
    host_scratch_free(&g_st.hy, &g_st.hyc);
    scratch_free(&g_st.dx, &g_st.dxc);
    scratch_free(&g_st.dy, &g_st.dyc);
    scratch_free(&g_st.dk, &g_st.dkc);
    g_epoch = g_tk_epoch = 0;
}
}  // namespace coli

// the library's stream (for callers that time or order work against it)
COLI_API void *coli_hip_stream(void) { return (void *)stream(); }

COLI_API int coli_hip_gemv_error(void) { return gemv_error_take(); }
