// fmt6_device.h - device building blocks of the fmt=6 int4 matvec, shared by the GEMV
// and MoE kernels (gfx950, wave64).
//
// Arithmetic (c/qwen.c:211-229):  y[o] = sum_g s_g * (sum_{i in g} x_i n_i - z_g sum_{i in g} x_i)
//
// x is converted once per workgroup into block fixed point per group g: e_g is the
// smallest exponent with max|x_g| < 2^e_g, q_i = rint(x_i * 2^(22-e_g)) (|q_i| <= 2^22,
// i.e. 23 significant bits relative to the group maximum), and q_i = sum_{l<6} d_l 16^l
// with balanced digits d_l in [-8, 7].  Digit l of 8 consecutive columns is packed into
// one 32-bit "limb word"; the weights are stored XOR 0x88 (signed nibbles n - 8, see
// kLayoutLanes), so sum_i q_i (n_i - 8) over 8 columns is six v_dot8_i32_i4.  Integer
// sums are exact; one "unit" of chunks sharing a group is scaled back in fp32:
//   partial = s_g * (2^(e_g-22) * T  -  (z_g - 8) * sum_unit(x~)).
// The only rounding not present in exact arithmetic on the reference's inputs is x to 23
// bits relative to its group maximum, so results stay within fp32-accumulation accuracy.
#pragma once

#include "internal.h"

#include <limits.h>

namespace coli {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLimbs = 6;
constexpr int kTopK = 8;                           // largest fused top-k
constexpr int kLaneWords = kLaneChunks * 4;        // 32-bit weight words per lane and row

// ---------------------------------------------------------------- wave helpers
#define COLI_DPP_ADD(v, ctrl, rmask)                                                                  \
    ((v) + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), \
                                                                 (ctrl), (rmask), 0xF, false)))

// Sum over aligned segments of LPR lanes; the full sum is valid in the LAST lane of each
// segment (row_bcast15/31 only feed the upper DPP rows).
template <int LPR>
__device__ __forceinline__ float seg_sum(float v) {
    if constexpr (LPR >= 2) v = COLI_DPP_ADD(v, 0xB1, 0xF);    // quad_perm [1,0,3,2]
    if constexpr (LPR >= 4) v = COLI_DPP_ADD(v, 0x4E, 0xF);    // quad_perm [2,3,0,1]
    if constexpr (LPR >= 8) v = COLI_DPP_ADD(v, 0x141, 0xF);   // row_half_mirror
    if constexpr (LPR >= 16) v = COLI_DPP_ADD(v, 0x140, 0xF);  // row_mirror
    if constexpr (LPR >= 32) v = COLI_DPP_ADD(v, 0x142, 0xA);  // row_bcast15 -> rows 1,3
    if constexpr (LPR >= 64) v = COLI_DPP_ADD(v, 0x143, 0xC);  // row_bcast31 -> rows 2,3
    return v;
}

// Wave-wide sum of a double by DPP on its two halves; the sum is valid in lane 63 and
// is returned broadcast to all lanes.
template <int CTRL, int RMASK>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, RMASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, RMASK, 0xF, false);
    return __builtin_bit_cast(double, ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ double wave_sum_dpp(double v) {
    v += dpp_d<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v += dpp_d<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v += dpp_d<0x141, 0xF>(v);   // row_half_mirror
    v += dpp_d<0x140, 0xF>(v);   // row_mirror
    v += dpp_d<0x142, 0xA>(v);   // row_bcast15
    v += dpp_d<0x143, 0xC>(v);   // row_bcast31
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// max of an unsigned value and its DPP-moved copy (one step of a wave maximum)
#define COLI_DPP_UMAX(v, ctrl, rmask) \
    max((v), (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(v), (ctrl), (rmask), 0xF, false))

// Maximum over aligned runs of n lanes (n a power of two <= 16, wave uniform), in every
// lane of the run.  All lanes must be active.
__device__ __forceinline__ uint32_t run_umax(uint32_t v, int n) {
    if (n >= 2) v = COLI_DPP_UMAX(v, 0xB1, 0xF);    // quad_perm [1,0,3,2]
    if (n >= 4) v = COLI_DPP_UMAX(v, 0x4E, 0xF);    // quad_perm [2,3,0,1]
    if (n >= 8) v = COLI_DPP_UMAX(v, 0x141, 0xF);   // row_half_mirror
    if (n >= 16) v = COLI_DPP_UMAX(v, 0x140, 0xF);  // row_mirror
    return v;
}
// Sum over aligned quads of lanes, in every lane of the quad.  All lanes must be active.
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    return v;
}

// (value desc, index asc): the order of c/shaders/argmax.comp:28,41 and of the host scan
// c/qwen.c:1471-1472 (ties resolve to the lowest index).
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
    return a > b || (a == b && ia < ib);
}

template <int K>
__device__ __forceinline__ void topk_insert(float (&tv)[K], int (&ti)[K], float v, int i) {
    if (!better(v, i, tv[K - 1], ti[K - 1])) return;
#pragma unroll
    for (int j = 0; j < K; j++) {
        if (better(v, i, tv[j], ti[j])) {
            const float t = tv[j];
            const int u = ti[j];
            tv[j] = v;
            ti[j] = i;
            v = t;
            i = u;
        }
    }
}

template <int K>
__device__ __forceinline__ void topk_clear(float (&tv)[K], int (&ti)[K]) {
#pragma unroll
    for (int j = 0; j < K; j++) {
        tv[j] = -INFINITY;
        ti[j] = INT_MAX;
    }
}

// a := best K of (a U b), both sorted by `better`.  The elementwise best of a and
// reversed b is a bitonic sequence holding the top K; a bitonic merge sorts it.
template <int K>
__device__ __forceinline__ void topk_merge2(float (&av)[K], int (&ai)[K], const float (&bv)[K], const int (&bi)[K]) {
#pragma unroll
    for (int i = 0; i < K; i++)
        if (better(bv[K - 1 - i], bi[K - 1 - i], av[i], ai[i])) {
            av[i] = bv[K - 1 - i];
            ai[i] = bi[K - 1 - i];
        }
#pragma unroll
    for (int s = K / 2; s > 0; s >>= 1)
#pragma unroll
        for (int i = 0; i < K; i++)
            if ((i & s) == 0 && better(av[i + s], ai[i + s], av[i], ai[i])) {
                const float t = av[i];
                const int u = ai[i];
                av[i] = av[i + s];
                ai[i] = ai[i + s];
                av[i + s] = t;
                ai[i + s] = u;
            }
}

// merge the sorted lists of lanes l and l ^ off, for off = 1 .. LANES/2
template <int K, int LANES>
__device__ __forceinline__ void wave_topk_merge(float (&tv)[K], int (&ti)[K]) {
#pragma unroll
    for (int off = 1; off < LANES; off <<= 1) {
        float ov[K];
        int oi[K];
#pragma unroll
        for (int j = 0; j < K; j++) {
            ov[j] = __shfl_xor(tv[j], off);
            oi[j] = __shfl_xor(ti[j], off);
        }
        topk_merge2<K>(tv, ti, ov, oi);
    }
}

// Rank selection over n candidates in LDS (value, index-as-bits): each candidate counts
// the candidates that beat it; rank < k is its output position.  All comparisons are
// independent (no merge chain) and every thread reads the same LDS word (broadcast).
// Equal candidates (only the padding (-inf, INT_MAX)) share a rank and write the same.
__device__ __forceinline__ void rank_select(const float2 *cand, int n, int k, float *out_v, int *out_i,
                                            int nthreads) {
    for (int c = threadIdx.x; c < n; c += nthreads) {
        const float2 me = cand[c];
        const int mi = __float_as_int(me.y);
        int r = 0;
        for (int j = 0; j < n; j++) {
            const float2 o = cand[j];
            r += better(o.x, __float_as_int(o.y), me.x, mi) ? 1 : 0;
        }
        if (r < k) {
            out_v[r] = me.x;
            out_i[r] = mi;
        }
    }
}

// Block-wide best-k (k <= K) over per-thread sorted lists; result to out_v/out_i
// (written by thread 0).  All kThreads threads call.
template <int K>
__device__ __forceinline__ void block_topk_merge(float (&tv)[K], int (&ti)[K], int k, float *out_v, int *out_i) {
    __shared__ float s_v[kWaves][K];
    __shared__ int s_i[kWaves][K];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    wave_topk_merge<K, 64>(tv, ti);
    if (lane == 0)
#pragma unroll
        for (int j = 0; j < K; j++) {
            s_v[wave][j] = tv[j];
            s_i[wave][j] = ti[j];
        }
    __syncthreads();
    if (wave == 0) {
        const int w = lane < kWaves ? lane : 0;
#pragma unroll
        for (int j = 0; j < K; j++) {
            tv[j] = lane < kWaves ? s_v[w][j] : -INFINITY;
            ti[j] = lane < kWaves ? s_i[w][j] : INT_MAX;
        }
        wave_topk_merge<K, kWaves>(tv, ti);
        if (lane == 0)
            for (int j = 0; j < k; j++) {
                out_v[j] = tv[j];
                out_i[j] = ti[j];
            }
    }
    __syncthreads();
}

// ---------------------------------------------------------------- x -> digit planes
// Workgroup barrier for LDS traffic: orders this block's LDS accesses only.  A
// __syncthreads() carries a workgroup fence over all address spaces, which on gfx950 also
// waits for every global load in flight; the x preparation runs while the weight loads
// issued before it are still outstanding, so its barriers must not wait for them.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Digit plane l holds the digit-l nibbles of x word w (8 columns) at xprep_pos(w): the
// words of host chunk h (4 each) sit in slot h % kLaneChunks of lane h / kLaneChunks, the
// lanes of one slot side by side, so lane_x's 16-byte reads of consecutive lanes are
// consecutive in LDS (a word-major layout, 96 bytes per chunk, put 8-16 lanes on one bank).
constexpr int kXLanes = kLaneMaxI / (32 * kLaneChunks);   // lanes of a row, at most
__device__ __forceinline__ int xprep_pos(int w) {
    const int h = w >> 2;
    return ((h % kLaneChunks) * kXLanes + h / kLaneChunks) * 4 + (w & 3);
}
// The digit planes of 8 columns: u[c] holds the 6 nibbles of column c (nibble l = digit
// l + 8); plane l gets nibble l of u[c] at bits 4c, XOR 0x8 per nibble ((d + 8) ^ 8 == d mod
// 16).  Adjacent columns are paired into bytes (t: even digits, s: odd digits), then byte
// k of the four pairs is gathered with byte permutes: ~36 operations where the nibble-by-
// nibble form takes ~100.
static_assert(kLimbs == 6, "digit_planes packs 6 planes");
__device__ __forceinline__ void digit_planes(const uint32_t (&u)[8], uint32_t (&L)[kLimbs]) {
    uint32_t t[4], s[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        t[b] = ((u[2 * b + 1] << 4) & 0xF0F0F0F0u) | (u[2 * b] & 0x0F0F0F0Fu);   // byte k: digits 2k
        s[b] = (u[2 * b + 1] & 0xF0F0F0F0u) | ((u[2 * b] >> 4) & 0x0F0F0F0Fu);   // byte k: digits 2k+1
    }
    // v_perm_b32: selector byte i picks byte sel of {src0:src1} (0-3 src1, 4-7 src0, 12 zero)
    const uint32_t ta = __builtin_amdgcn_perm(t[1], t[0], 0x05010400u), tb = __builtin_amdgcn_perm(t[3], t[2], 0x05010400u);
    const uint32_t tc = __builtin_amdgcn_perm(t[1], t[0], 0x0C0C0602u), td = __builtin_amdgcn_perm(t[3], t[2], 0x0C0C0602u);
    const uint32_t sa = __builtin_amdgcn_perm(s[1], s[0], 0x05010400u), sb = __builtin_amdgcn_perm(s[3], s[2], 0x05010400u);
    const uint32_t sc = __builtin_amdgcn_perm(s[1], s[0], 0x0C0C0602u), sd = __builtin_amdgcn_perm(s[3], s[2], 0x0C0C0602u);
    L[0] = __builtin_amdgcn_perm(tb, ta, 0x05040100u) ^ 0x88888888u;
    L[2] = __builtin_amdgcn_perm(tb, ta, 0x07060302u) ^ 0x88888888u;
    L[4] = __builtin_amdgcn_perm(td, tc, 0x05040100u) ^ 0x88888888u;
    L[1] = __builtin_amdgcn_perm(sb, sa, 0x05040100u) ^ 0x88888888u;
    L[3] = __builtin_amdgcn_perm(sb, sa, 0x07060302u) ^ 0x88888888u;
    L[5] = __builtin_amdgcn_perm(sd, sc, 0x05040100u) ^ 0x88888888u;
}

struct XPrep {
    __attribute__((aligned(16))) uint32_t limb[kLimbs][kLaneMaxI / 8];   // [digit][xprep_pos(word)]
    int qsum[kLaneMaxI / 32];               // per 32-column chunk: sum of q
    unsigned gmax[kLaneMaxI / 32];          // per group (gs >= 32): bits of max |x|
};

// ncols: columns to prepare (a multiple of 32 covering every lane's chunks, <= kLaneMaxI);
// columns at or past I are zero.  Each thread owns whole 8-column words: it loads its
// x values once (all loads in flight together), publishes one max per word, then turns
// them into digit planes.  NT = threads of the block.  Ends with an LDS barrier.
// v[0..8) = the 8 floats at byte offset off of buffer r (two 16-byte loads; dwords out of
// the buffer's range read 0)
__device__ __forceinline__ void load8f(__amdgpu_buffer_rsrc_t r, int off, float (&v)[8]) {
    typedef int v4i_t __attribute__((ext_vector_type(4)));
    const v4i_t a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const v4i_t b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0);
    v[0] = __int_as_float(a.x);
    v[1] = __int_as_float(a.y);
    v[2] = __int_as_float(a.z);
    v[3] = __int_as_float(a.w);
    v[4] = __int_as_float(b.x);
    v[5] = __int_as_float(b.y);
    v[6] = __int_as_float(b.z);
    v[7] = __int_as_float(b.w);
}

template <int NT>
struct XRegsT {
    static constexpr int kWords = (kLaneMaxI / 8 + NT - 1) / NT;   // words per thread
    float v[kWords][8];
};
using XRegs = XRegsT<kThreads>;
// Issue the x loads (split from prep_x so that they can go out before other loads).
// Buffer loads with out-of-range offsets for the missing columns: no branches, so the
// compiler can wait for exactly these loads and not for the weight loads issued after.
// A thread's word is two 16-byte loads.  Raw buffer loads check the range per dword, so the
// columns at or past I read 0 also inside a partly covered load.
template <int NT = kThreads>
__device__ __forceinline__ void prep_load(const float *__restrict__ x, int I, int ncols, XRegsT<NT> &xr) {
    const int tid = threadIdx.x, nwords = ncols / 8;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(x), (short)0, I * 4, 0x00020000);
#pragma unroll
    for (int k = 0; k < XRegsT<NT>::kWords; k++) {
        const int w = tid + k * NT;
        const int off = w < nwords ? w * 32 : (int)0x80000000;
        load8f(r, off, xr.v[k]);
    }
}

// x := x r (1 + w) with r = 1 / sqrt(mean(x^2) + eps) over the I columns (zero-centred
// RMSNorm, c/qwen.c:326-330: double sum of squares; the multiplications in the reference's
// order).  xr, wr as loaded by prep_load; all threads call (two LDS barriers).
template <int NT = kThreads>
__device__ __forceinline__ void norm_apply(XRegsT<NT> &xr, const XRegsT<NT> &wr, int I, int ncols, float eps,
                                           double *s_red) {
    double ss = 0;
#pragma unroll
    for (int k = 0; k < XRegsT<NT>::kWords; k++)
#pragma unroll
        for (int c = 0; c < 8; c++) ss += (double)xr.v[k][c] * xr.v[k][c];   // zeros past I add 0
    ss = wave_sum_dpp(ss);
    lds_barrier();
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
    lds_barrier();
    double t = 0;
    for (int w = 0; w < NT / 64; w++) t += s_red[w];
    const float r = 1.f / sqrtf((float)((I & (I - 1)) ? t / I : t * (1.0 / I)) + eps);   // 1 / I exact for I = 2^k
#pragma unroll
    for (int k = 0; k < XRegsT<NT>::kWords; k++) {
        const int w = threadIdx.x + k * NT;
#pragma unroll
        for (int c = 0; c < 8; c++)
            if (w < ncols / 8 && w * 8 + c < I) xr.v[k][c] = xr.v[k][c] * r * (1.f + wr.v[k][c]);
    }
}

// 22 - e for a group maximum m: e = ilogb(m) + 1 (m < 2^e), the exponent frexp gives for
// finite m > 0 (denormals included); 0 for an all-zero group.
__device__ __forceinline__ int exp22_of(float m) { return 22 - (m > 0.f ? __builtin_amdgcn_frexp_expf(m) : 0); }

// The balanced digits of one 8-column word at scale 2^k (k = 22 - e, |v 2^k| < 2^22):
// u[c] = rint(v[c] 2^k) + 0x888888 (digit l + 8 in nibble l), and the sum of the
// rint(v[c] 2^k).  rint comes from adding 1.5 2^23 (round to nearest even, |v 2^k| < 2^22):
// the sum's bits are 0x4B400000 + rint(v 2^k).
__device__ __forceinline__ int word_digits(const float (&v)[8], int k, uint32_t (&u)[8]) {
    int qs = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const float t = ldexpf(v[c], k) + 12582912.f;
        const int q = (int)(__float_as_uint(t) - 0x4B400000u);
        qs += q;
        u[c] = (uint32_t)(q + 0x888888);
    }
    return qs;
}

template <int NT = kThreads>
__device__ __forceinline__ void prep_x(const XRegsT<NT> &xr, int gs, int ncols, XPrep &P) {
    const int tid = threadIdx.x;
    const int nwords = ncols / 8, ngrp = (ncols + gs - 1) / gs, wpg = gs / 8;
    // Word w sits in lane w % 64, so a group of wpg <= 16 words (a power of two) is an
    // aligned run of lanes: its maximum comes by DPP, and a chunk's q sum (4 words) by a
    // quad sum, with no LDS round trip.  Other group sizes use LDS atomics.
    const bool runs = wpg <= 16 && (wpg & (wpg - 1)) == 0;
    const int gsh = runs ? __builtin_ctz((unsigned)wpg) : 0;   // word -> group shift (runs)
    const auto &xv = xr.v;
    if (!runs) {
        for (int g = tid; g < ngrp; g += NT) P.gmax[g] = 0u;
        lds_barrier();
    }
    uint32_t mb[XRegsT<NT>::kWords];
#pragma unroll
    for (int k = 0; k < XRegsT<NT>::kWords; k++) {
        if (k > 0 && k * NT >= nwords) break;   // block uniform: no words left
        const int w = tid + k * NT;
        float m = 0.f;
#pragma unroll
        for (int c = 0; c < 8; c++) m = fmaxf(m, fabsf(xv[k][c]));   // words past ncols hold zeros
        mb[k] = __float_as_uint(m);
        if (runs) mb[k] = run_umax(mb[k], wpg);
        else if (w < nwords) atomicMax(&P.gmax[(w * 8) / gs], mb[k]);
    }
    if (!runs) lds_barrier();
#pragma unroll
    for (int k = 0; k < XRegsT<NT>::kWords; k++) {
        if (k > 0 && k * NT >= nwords) break;
        const int w = tid + k * NT;
        const bool on = w < nwords;
        const float m = runs ? __uint_as_float(mb[k]) : on ? __uint_as_float(P.gmax[(w * 8) / gs]) : 0.f;
        uint32_t u[8];
        int qs = word_digits(xv[k], exp22_of(m), u);
        if (on) {
            uint32_t lw[kLimbs];
            digit_planes(u, lw);
#pragma unroll
            for (int l = 0; l < kLimbs; l++) P.limb[l][xprep_pos(w)] = lw[l];
        }
        qs = quad_sum(qs);
        if (on && (w & 3) == 0) P.qsum[w >> 2] = qs;
        if (runs && on && (w & (wpg - 1)) == 0) P.gmax[w >> gsh] = mb[k];
    }
    lds_barrier();
}

__device__ __forceinline__ int group_exp22(const XPrep &P, int g) {
    const float m = __uint_as_float(P.gmax[g]);
    return -exp22_of(m);
}

// ---------------------------------------------------------------- per-lane state
// Buffer loads: out-of-range offsets read 0 (no predication), 32-bit offsets.  Weights are
// read once per launch, so by default they are loaded nontemporal (cache policy NT: the
// lines do not displace the activations and partials that are reused); callers whose
// blocks re-read the same weights pass kCached.
typedef int coli_v4i __attribute__((ext_vector_type(4)));
typedef int coli_v2i __attribute__((ext_vector_type(2)));
constexpr uint32_t kOOB = 0x80000000u;     // added to an offset <= 2^31: always out of range
constexpr int kStream = 2;                 // buffer-load cache policy: nt
constexpr int kCached = 0;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
template <int POL = kStream>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, POL);
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
template <int POL = kStream>
__device__ __forceinline__ float2 buf_load8f(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const coli_v2i v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, POL);
    return make_float2(__int_as_float(v.x), __int_as_float(v.y));
}

// One lane's share of a row: kLaneChunks host chunks, split into NU units of CU chunks
// that share a group (CU = min(gs/32, kLaneChunks)).
template <int CU>
struct LaneX {
    static constexpr int NU = kLaneChunks / CU;
    // geometry (independent of x)
    uint32_t woff[kLaneChunks];   // byte offset of the lane's chunk c within a row (or kOOB)
    uint32_t soff[NU];            // byte offset of the unit's [scale, zero] within a row (or kOOB)
    int ch0;                      // first host chunk of the lane
    bool on;                      // lane holds data (j < nl)
    // x digits of the lane's columns
    uint32_t lm[kLaneWords][kLimbs];
    int ue[NU];      // e_g - 22
    float ucs[NU];   // sum of x~ over the unit
};

template <int CU>
__device__ __forceinline__ void lane_geo(int j, int nl, int I, int gs, LaneX<CU> &L) {
    L.on = j < nl;
    L.ch0 = (L.on ? j : 0) * kLaneChunks;
#pragma unroll
    for (int c = 0; c < kLaneChunks; c++) L.woff[c] = L.on ? (uint32_t)((c * nl + j) * 16) : kOOB;
#pragma unroll
    for (int q = 0; q < LaneX<CU>::NU; q++) {
        const int col0 = (L.ch0 + q * CU) * 32;
        L.soff[q] = (L.on && col0 < I) ? (uint32_t)((col0 / gs) * 8) : kOOB;
    }
}

template <int CU>
__device__ __forceinline__ void lane_x(const XPrep &P, int gs, LaneX<CU> &L) {
    const int j = L.ch0 / kLaneChunks;
#pragma unroll
    for (int c = 0; c < kLaneChunks; c++)
#pragma unroll
        for (int l = 0; l < kLimbs; l++) {
            const uint4 v = *(const uint4 *)&P.limb[l][(c * kXLanes + j) * 4];
            L.lm[c * 4 + 0][l] = v.x;
            L.lm[c * 4 + 1][l] = v.y;
            L.lm[c * 4 + 2][l] = v.z;
            L.lm[c * 4 + 3][l] = v.w;
        }
#pragma unroll
    for (int q = 0; q < LaneX<CU>::NU; q++) {
        const int ch = L.ch0 + q * CU;
        L.ue[q] = group_exp22(P, (ch * 32) / gs);
        int qs = 0;
#pragma unroll
        for (int c = 0; c < CU; c++) qs += P.qsum[ch + c];
        L.ucs[q] = ldexpf((float)qs, L.ue[q]);
    }
}

// Lane partial of one row: wq = the lane's kLaneChunks chunks (device words), sv = the
// units' [scale, zero] (scale 0 for units without data).
template <int CU>
__device__ __forceinline__ float lane_row(const uint4 (&wq)[kLaneChunks], const float2 (&sv)[LaneX<CU>::NU],
                                          const LaneX<CU> &L) {
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < LaneX<CU>::NU; q++) {
        int t[kLimbs] = {0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int c = q * CU; c < (q + 1) * CU; c++) {
            const uint32_t wv[4] = {wq[c].x, wq[c].y, wq[c].z, wq[c].w};
#pragma unroll
            for (int w = 0; w < 4; w++)
#pragma unroll
                for (int l = 0; l < kLimbs; l++)
                    t[l] = __builtin_amdgcn_sdot8((int)wv[w], (int)L.lm[c * 4 + w][l], t[l], false);
        }
        const int lo = t[0] + 16 * t[1] + 256 * t[2];
        const int hi = t[3] + 16 * t[4] + 256 * t[5];
        const float T = fmaf((float)hi, 4096.f, (float)lo);
        const float v = fmaf(-(sv[q].y - 8.f), L.ucs[q], ldexpf(T, L.ue[q]));
        acc = fmaf(sv[q].x, v, acc);
    }
    return acc;
}

// Load the lane's chunks and unit scales of the row at byte offsets (wrow, srow), which
// are clamped by the caller to at most the buffer sizes: rows past the end, lanes without
// data and units without columns all read 0 and contribute 0.
template <int CU>
__device__ __forceinline__ void lane_load(__amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs, uint32_t wrow,
                                          uint32_t srow, const LaneX<CU> &L, uint4 (&wq)[kLaneChunks],
                                          float2 (&sv)[LaneX<CU>::NU]) {
#pragma unroll
    for (int c = 0; c < kLaneChunks; c++) wq[c] = buf_load16(rw, wrow + L.woff[c]);
#pragma unroll
    for (int q = 0; q < LaneX<CU>::NU; q++) sv[q] = buf_load8f(rs, srow + L.soff[q]);
}

}  // namespace coli
