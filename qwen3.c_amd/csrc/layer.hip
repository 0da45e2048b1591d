// layer.hip - the attention and GatedDeltaNet layer blocks of the decode step, the device
// residual stream and the route tail, on gfx950.
//
// Semantics (one token):
//   gated GQA block        c/qwen.c:581-667   (q|gate projection, per-head zero-centred
//                          q/k norm, partial RoPE, KV rows at pos, softmax attention,
//                          sigmoid output gate, o_proj)
//   GatedDeltaNet block    c/qwen.c:669-776   (qkv/z projections, causal conv1d ring +
//                          SiLU, l2norm, decay/beta from a/b, delta rule, gated RMSNorm,
//                          out_proj)
//   layer composition      c/qwen.c:1340-1352 (resid += block(in_ln(resid));
//                          resid += moe(post_ln(resid)))
//   stream / route tail    c/qwen.c:1228-1290 (device residual, device top-k, MoE)
//
// Kernels of a layer (all stream-ordered, no host synchronisation inside a layer):
//   proj_gemv   fmt 6 lanes-layout GEMV over up to 4 tensors that share the input row
//               (qkv | z | a | b of GDN, q | k | v of GQA), with the input transform fused
//               into the x prologue (in_ln RMSNorm of the residual, or the GDN per-head
//               gated RMSNorm) and the residual add fused into the store.
//   gdn_core    one block per (v-head, 16-column slice) of the recurrent state: decay/beta
//               from the a/b dots, conv + SiLU of the channels it needs (the conv ring is
//               circular: the owner of a channel stores this token's input in place), l2norm,
//               then the delta rule on its columns.  The state is kept transposed ([VH][VD][KD]) so that a column is
//               contiguous: each wave updates a column with one coalesced load and two
//               DPP reductions, and blocks own disjoint columns (in-place, race free).
//   attn_part   one block per (kv head, 32-position chunk): normalises and rotates the
//               q rows of its query group (and the new key row, which the chunk holding
//               pos writes to the cache), then scores, chunk softmax and P.V.
//   attn_merge  one block per query head: merges the chunks (max, sum of exp), applies
//               the sigmoid gate.
#include "fmt6_device.h"
#include "moe_common.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

namespace coli {

// ---------------------------------------------------------------- block reductions
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Block-wide double sum in a fixed order (deterministic); every thread gets the sum.
__device__ __forceinline__ double block_sum_d(double v, double *s_red) {
    v = wave_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) s += s_red[w];
    return s;
}

__device__ __forceinline__ float wave_sum_f(float v) {
    v = seg_sum<64>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }
// silu(z) of the gated norm, with a hardware reciprocal (< 2 ulp)
__device__ __forceinline__ float silu_gate(float z) { return z * __builtin_amdgcn_rcpf(1.f + expf(-z)); }

// ---------------------------------------------------------------- projections
constexpr int kMaxSeg = 4;
enum { XF_PLAIN = 0, XF_NORM = 1, XF_GATED = 2 };

struct ProjSeg {
    const uint8_t *w;
    const float *sz;
    float *y;
    int O;
    int g0;                  // first row group of the segment in the launch's row-group space
    unsigned long long *yt;  // fused layer kernel: the outputs as tagged words (epoch << 32 | bits)
    int act;                 // 1: the segment stores silu(row) (GDN's z, the gated norm's gate)
};

struct ProjArgs {
    ProjSeg seg[kMaxSeg];
    int nseg, ngroups;
    int I, gs, ng, nl, row_bytes;
    const float *x;    // XF_PLAIN: the input row; XF_NORM: the residual; XF_GATED: raw y
    const float *xw;   // XF_NORM: norm weight [I] (zero-centred); XF_GATED: gnorm [VD]
    const float *z;    // XF_GATED: silu of the z projection [I] (its in-projection segment has act)
    int VD;
    float eps;
    int add;           // 1: y[r] += acc (residual add), 0: y[r] = acc
    // fused layer kernel: x (and z) as tagged words, polled until they carry `epoch`
    const unsigned long long *xt, *zt;
    unsigned long long *err;
    uint32_t epoch;
    const unsigned long long *done;   // > 0 words: the producers of x mark their end (see proj_body)
    int ndone;
};

// Sum over aligned groups of n lanes (n a power of two <= 64, wave uniform), in every lane
// of the group: the xor butterfly's pairing, by DPP within rows of 16 lanes.
__device__ __forceinline__ double seg_sum_d(double v, int n) {
    if (n >= 2) v += dpp_d<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]: lane ^ 1
    if (n >= 4) v += dpp_d<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]: lane ^ 2
    if (n >= 8) v += dpp_d<0x141, 0xF>(v);   // row_half_mirror: the other quad of the 8
    if (n >= 16) v += dpp_d<0x140, 0xF>(v);  // row_mirror: the other 8 of the row
    for (int off = 16; off < n; off <<= 1) v += __shfl_xor(v, off);
    return v;
}

// XF_NORM: x[i] * r * (1 + w[i]), r = 1/sqrt(mean(x^2) + eps) over the I columns
// (c/qwen.c:326-330, double sum of squares).  XF_GATED: per head of VD columns,
// y * r_h * gnorm[d] * silu(z) (c/qwen.c:768-772).  Zero columns past I stay zero.  The
// operands (w; or silu(z) and gnorm) were loaded into ar / br together with x.  silu(z) is
// applied once, by the store of z's in-projection (silu_gate), not by every block here.
template <int XF>
__device__ __forceinline__ void xf_apply(XRegs &xr, const XRegs &ar, const XRegs &br, const ProjArgs &a, int ncols) {
    const int tid = threadIdx.x, nwords = ncols / 8;
    if constexpr (XF == XF_NORM) {
        __shared__ double s_red[kWaves];
        norm_apply(xr, ar, a.I, ncols, a.eps, s_red);
    } else if constexpr (XF == XF_GATED) {
        const int wph = a.VD / 8;   // words per head: a power of two <= 64, lane aligned
#pragma unroll
        for (int k = 0; k < XRegs::kWords; k++) {
            const int w = tid + k * kThreads;
            double ss = 0;
#pragma unroll
            for (int c = 0; c < 8; c++) ss += (double)xr.v[k][c] * xr.v[k][c];
            ss = seg_sum_d(ss, wph);
            const float r = 1.f / sqrtf((float)(ss * (1.0 / a.VD)) + a.eps);   // VD = 8 wph, a power of two: exact
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int i = w * 8 + c;
                if (w < nwords && i < a.I) xr.v[k][c] = xr.v[k][c] * r * br.v[k][c] * ar.v[k][c];
            }
        }
    }
}

// the transform operands of the thread's columns: XF_NORM w; XF_GATED z (ar) and the
// gated-norm weight of the column's head position (br)
template <int XF>
__device__ __forceinline__ void xf_load(XRegs &ar, XRegs &br, const ProjArgs &a, int ncols) {
    if constexpr (XF == XF_NORM) prep_load(a.xw, a.I, ncols, ar);
    if constexpr (XF == XF_GATED) {
        prep_load(a.z, a.I, ncols, ar);
        const int tid = threadIdx.x, nwords = ncols / 8;
        const __amdgpu_buffer_rsrc_t r = buf_rsrc(a.xw, (uint32_t)a.VD * 4);
#pragma unroll
        for (int k = 0; k < XRegs::kWords; k++) {   // unconditional loads, as prep_load; VD % 8 == 0,
            const int w = tid + k * kThreads;          // so a word lies within one head
            load8f(r, (w < nwords && w * 8 < a.I) ? ((w * 8) % a.VD) * 4 : (int)kOOB, br.v[k]);
        }
    }
}

// The segment holding row group g (g wave-uniform, so the selection is scalar).
struct SegSel {
    const uint8_t *w;
    const float *sz;
    float *y;
    int O, g0;
    unsigned long long *yt;
    int act;
};
__device__ __forceinline__ SegSel seg_of(const ProjArgs &a, int g) {
    SegSel s = {a.seg[0].w, a.seg[0].sz, a.seg[0].y, a.seg[0].O, a.seg[0].g0, a.seg[0].yt, a.seg[0].act};
#pragma unroll
    for (int t = 1; t < kMaxSeg; t++)
        if (t < a.nseg && g >= a.seg[t].g0)
            s = {a.seg[t].w, a.seg[t].sz, a.seg[t].y, a.seg[t].O, a.seg[t].g0, a.seg[t].yt, a.seg[t].act};
    return s;
}

// Two tagged rows (y and z of the gated norm) polled together.
__device__ __forceinline__ bool prep_load_tagged2(const unsigned long long *xt, const unsigned long long *zt, int I,
                                                  int ncols, XRegs &xr, XRegs &zr, uint32_t ep,
                                                  unsigned long long *err) {
    const int tid = threadIdx.x, nwords = ncols / 8;
    for (int polls = 0;; polls++) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < XRegs::kWords; k++) {
            const int w = tid + k * kThreads;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int i = w * 8 + c;
                const bool on = w < nwords && i < I;
                const unsigned long long v = on ? aload(xt + i) : 0ull, u = on ? aload(zt + i) : 0ull;
                all &= !on || ((uint32_t)(v >> 32) == ep && (uint32_t)(u >> 32) == ep);
                xr.v[k][c] = __uint_as_float((uint32_t)v);
                zr.v[k][c] = __uint_as_float((uint32_t)u);
            }
        }
        if (all) return true;
        if (poll_give_up(err, ep, polls)) return false;
    }
}

// prep_load from tagged words: every column's word is polled until it carries the epoch
// (bounded; false when the launch has failed).  Columns at or past I are zero.
__device__ __forceinline__ bool prep_load_tagged(const unsigned long long *xt, int I, int ncols, XRegs &xr, uint32_t ep,
                                                 unsigned long long *err) {
    const int tid = threadIdx.x, nwords = ncols / 8;
    for (int polls = 0;; polls++) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < XRegs::kWords; k++) {
            const int w = tid + k * kThreads;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int i = w * 8 + c;
                const bool on = w < nwords && i < I;
                const unsigned long long v = on ? aload(xt + i) : 0ull;
                all &= !on || (uint32_t)(v >> 32) == ep;
                xr.v[k][c] = __uint_as_float((uint32_t)v);
            }
        }
        if (all) return true;
        if (poll_give_up(err, ep, polls)) return false;
    }
}

// Row groups (RPW rows of one wave step) of all segments form one space; a segment
// starts on a group boundary, so a wave step never mixes tensors.  U row steps per wave
// are loaded before any is reduced (the loads of the next step go out while the current
// one computes), as in the single-tensor GEMV.
// kTagIn (fused layer kernel, XF_GATED): x and z come as tagged words from earlier tiles;
// the weights of the block's first row steps are then loaded before the wait.  kTagOut: the
// outputs go out as tagged words.  bid / nb: this block's index among the nb blocks of the
// projection.
template <int LPR, int CU, int U, int XF, bool kTagIn, bool kTagOut>
__device__ __forceinline__ void proj_body(const ProjArgs &a, int bid, int nb, XPrep &P) {
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane % LPR, sg = lane / LPR;
    const int ncols = a.nl * kLaneChunks * 32;
    const uint32_t srb = (uint32_t)a.ng * 8u;
    XRegs xr, ar, br;
    if constexpr (!kTagIn) {
        prep_load(a.x, a.I, ncols, xr);
        if constexpr (XF != XF_PLAIN) xf_load<XF>(ar, br, a, ncols);
    }
    LaneX<CU> L;
    lane_geo<CU>(j, a.nl, a.I, a.gs, L);
    const int nw = nb * kWaves;
    const int gbase = bid * kWaves + wave;
    uint4 wq[U][kLaneChunks];
    float2 sv[U][LaneX<CU>::NU];
    float yo[U];   // a.add: the output row's old value, loaded with the step's weights (a load
                   // issued after the dot would wait for every prefetched weight load)
    auto load = [&](int u, int g) {   // unconditional: out-of-range offsets past the last group
        const bool on = g < a.ngroups;
        const SegSel s = seg_of(a, on ? g : a.ngroups - 1);
        const uint32_t r = (uint32_t)((on ? g - s.g0 : 0) * RPW + sg);
        const uint32_t wtot = (uint32_t)s.O * (uint32_t)a.row_bytes, stot = (uint32_t)s.O * srb;
        lane_load<CU>(buf_rsrc(s.w, wtot), buf_rsrc(s.sz, stot), on ? min(r * (uint32_t)a.row_bytes, wtot) : kOOB,
                      on ? min(r * srb, stot) : kOOB, L, wq[u], sv[u]);
        if constexpr (!kTagOut)
            yo[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  buf_rsrc(s.y, (uint32_t)s.O * 4u),
                                                  on && a.add && j == LPR - 1 && r < (uint32_t)s.O ? r * 4 : kOOB, 0, 0));
    };
#pragma unroll
    for (int u = 0; u < U; u++) load(u, gbase + u * nw);
    if constexpr (kTagIn) {   // the weights are in flight; now the inputs
        // first the producers' done words, so that the block's many loads of x go out
        // once, when x is complete
        if (a.ndone > 0) {   // wave 0 waits for the producers' done words, then one pass of loads
            if (threadIdx.x < 64) {
                constexpr int kDone = 8;   // a.ndone <= 64 kDone
                for (int polls = 0;; polls++) {
                    bool all = true;
#pragma unroll
                    for (int k = 0; k < kDone; k++) {
                        const int i = threadIdx.x + 64 * k;
                        const unsigned long long v = i < a.ndone ? aload(a.done + i) : 0ull;
                        all &= i >= a.ndone || (uint32_t)(v >> 32) == a.epoch;
                    }
                    if (__ballot(!all) == 0ull || poll_give_up(a.err, a.epoch, polls)) break;
                }
            }
            __syncthreads();
        }
        if constexpr (XF == XF_GATED) {   // y and z in one pass of loads
            prep_load_tagged2(a.xt, a.zt, a.I, ncols, xr, ar, a.epoch, a.err);
            const int tid = threadIdx.x, nwords = ncols / 8;
            const __amdgpu_buffer_rsrc_t r = buf_rsrc(a.xw, (uint32_t)a.VD * 4);
#pragma unroll
            for (int k = 0; k < XRegs::kWords; k++) {   // gnorm of the column's head position
                const int w = tid + k * kThreads;
                load8f(r, (w < nwords && w * 8 < a.I) ? ((w * 8) % a.VD) * 4 : (int)kOOB, br.v[k]);
            }
        } else {
            prep_load_tagged(a.xt, a.I, ncols, xr, a.epoch, a.err);
        }
    }
    if constexpr (XF != XF_PLAIN) xf_apply<XF>(xr, ar, br, a, ncols);
    prep_x(xr, a.gs, ncols, P);
    lane_x<CU>(P, a.gs, L);
    for (int g0 = gbase; g0 < a.ngroups; g0 += nw * U) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int g = g0 + u * nw;
            if (g >= a.ngroups) break;
            const float part = lane_row<CU>(wq[u], sv[u], L);
            float old = 0.f;
            if constexpr (!kTagOut) old = yo[u];
            load(u, g + nw * U);
            const float acc = seg_sum<LPR>(part);
            const SegSel s = seg_of(a, g);
            const int r = (g - s.g0) * RPW + sg;
            if (j == LPR - 1 && r < s.O) {
                if constexpr (kTagOut) {
                    tag_put(&s.yt[r], a.epoch, s.act ? silu_gate(acc) : acc);
                } else {
                    const float v = a.add ? old + acc : acc;
                    s.y[r] = s.act ? silu_gate(v) : v;
                }
            }
        }
    }
}

template <int LPR, int CU, int U, int XF>
__global__ __launch_bounds__(kThreads) void proj_gemv(ProjArgs a) {
    __shared__ XPrep P;
    proj_body<LPR, CU, U, XF, false, false>(a, blockIdx.x, gridDim.x, P);
}

// ---------------------------------------------------------------- GatedDeltaNet core
constexpr int kGdnCols = 16;            // state columns per block (4 per wave)
constexpr int kGdnColsPerWave = kGdnCols / kWaves;
constexpr int kGdnMaxKD = 256;
constexpr int kGdnMaxK = 4;             // conv taps of the one-round-trip path (others loop)

// A small projection row (GDN a/b: [VH, D]) in any device layout: element i of row r.
struct RowMat {
    const uint8_t *w;
    const float *sz;
    int fmt, layout, I, gs, ng, nl, row_bytes;
};
__device__ __forceinline__ float rowmat_w(const RowMat &m, int r, int i) {
    const uint8_t *row = m.w + (size_t)r * m.row_bytes;
    if (m.fmt == 0) return ((const float *)row)[i];
    if (m.fmt == 1) return (float)(int8_t)row[i];   // times the row scale, applied by the caller
    int nib;
    if (m.layout == kLayoutLanes) {   // host chunk h = 2 jj + c at slot c * nl + jj, bytes ^ 0x88
        const int h = i >> 5, jj = h >> 1, c = h & 1;
        const uint8_t b = row[(c * m.nl + jj) * 16 + ((i & 31) >> 1)] ^ 0x88;
        nib = (i & 1) ? (b >> 4) : (b & 15);
    } else {
        const uint8_t b = row[i >> 1];
        nib = (i & 1) ? (b >> 4) : (b & 15);
    }
    const float *s = m.sz + ((size_t)r * m.ng + i / m.gs) * 2;
    return ((float)nib - s[1]) * s[0];
}

struct GdnArgs {
    const float *qkv;      // [CD] projection of this token (before the conv)
    float *ring;           // [K][CD] circular: the previous K - 1 inputs at slots head + 1 ..
                           // head + K - 1 (mod K), oldest first; this token's input goes to head
    int head;
    const float *convw;    // [CD][K]
    float *S;              // [VH][VD][KD]
    float *y;              // [VH * VD] recurrence output (before the gated norm)
    const float *params;   // host-packed [decay(VH) | beta(VH) | ...], or NULL: from a/b
    const float *ab;       // a/b dots [a(VH) | b(VH)] from the projection launch, or NULL
    const float *xin;      // a/b input: the normed row, or NULL: in_ln(resid) here
    const float *resid, *in_ln;
    RowMat a, b;
    const float *alog, *dtb;
    float eps;
    int D, KH, KD, VH, VD, K, CD;
    // fused layer kernel: qkv and the a/b dots as tagged words from the projection tiles,
    // y out as tagged words
    const unsigned long long *qkvt, *abt;
    unsigned long long *yt, *done, *err;   // done[block]: the block's y words are out
    uint32_t epoch;
};

// kTag (fused layer kernel): the inputs are polled from tagged words and y is published as
// tagged words (the a/b path only; conv taps K <= kGdnMaxK).  bid: the block's index.
template <int KPL, bool kTag>   // state elements per lane of a column (KD = 64 KPL)
__device__ __forceinline__ void gdn_core_body(const GdnArgs &g, int bid) {
    __shared__ double s_red[kWaves];
    __shared__ float s_q[kGdnMaxKD], s_k[kGdnMaxKD], s_v[kGdnCols];
    __shared__ float s_ab[2][kWaves], s_nrm[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nsl = g.VD / kGdnCols;
    const int h = bid / nsl, c0 = (bid % nsl) * kGdnCols;
    const int src = h / (g.VH / g.KH), KD = g.KD, key_dim = g.KH * KD;

    // the block's state columns: loads go out first
    float sv[kGdnColsPerWave][KPL];
#pragma unroll
    for (int q = 0; q < kGdnColsPerWave; q++) {
        const float *col = g.S + ((size_t)h * g.VD + c0 + wave * kGdnColsPerWave + q) * KD + lane * KPL;
#pragma unroll
        for (int e = 0; e < KPL; e++) sv[q][e] = col[e];
    }

    // the a/b dots and their parameters (c/qwen.c:722-728) load with the state; decay and
    // beta are computed after the conv, whose loads then go out without waiting for these
    float decay = 0.f, beta = 0.f;
    const bool abp = !kTag && !g.params && g.ab;
    float pa, pb, pdtb, palog;
    {
        const uint32_t nab = abp ? (uint32_t)g.VH * 8u : 0u, np = abp || kTag ? (uint32_t)g.VH * 4u : 0u;
        const __amdgpu_buffer_rsrc_t ra = buf_rsrc(abp ? g.ab : g.dtb, nab), rd = buf_rsrc(g.dtb, np),
                                     rl = buf_rsrc(g.alog, np);
        pa = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ra, h * 4, 0, 0));
        pb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ra, (g.VH + h) * 4, 0, 0));
        pdtb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, h * 4, 0, 0));
        palog = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, h * 4, 0, 0));
    }

    // conv1d + SiLU of the channels this block reads (c/qwen.c:697-707): q and k of the
    // source k-head, v of the block's columns; the block that owns a channel (the group's
    // first v-head, first column slice, for q and k; every block for its own v columns)
    // stores this token's input at the ring head, a slot no block reads for this token
    const bool owns_qk = h % (g.VH / g.KH) == 0 && c0 == 0;
    auto channel = [&](int t) {
        return t < KD ? src * KD + t : t < 2 * KD ? key_dim + src * KD + (t - KD) : 2 * key_dim + h * g.VD + c0 + (t - 2 * KD);
    };
    if (g.K <= kGdnMaxK) {   // every load of the conv first (one memory round trip), branch-free
        constexpr int kCh = (2 * kGdnMaxKD + kGdnCols + kThreads - 1) / kThreads;
        const int nch = 2 * KD + kGdnCols, K = g.K;
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(g.qkv, (uint32_t)g.CD * 4u);
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(g.convw, (uint32_t)g.CD * (uint32_t)K * 4u);
        const __amdgpu_buffer_rsrc_t rr = buf_rsrc(g.ring, (uint32_t)K * (uint32_t)g.CD * 4u);
        auto ld = [](__amdgpu_buffer_rsrc_t r, bool on, int i) {
            return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, on ? i * 4 : (int)kOOB, 0, 0));
        };
        float xin[kCh], wlast[kCh], cw[kCh][kGdnMaxK - 1], rg[kCh][kGdnMaxK - 1];
#pragma unroll
        for (int i = 0; i < kCh; i++) {
            const int t = tid + i * kThreads;
            const bool on = t < nch;
            const int ch = on ? channel(t) : 0;
            if (!kTag) xin[i] = ld(rx, on, ch);
            wlast[i] = ld(rw, on, ch * K + K - 1);
#pragma unroll
            for (int q = 0; q + 1 < kGdnMaxK; q++) {
                int slot = g.head + 1 + q;
                if (slot >= K) slot -= K;
                cw[i][q] = ld(rw, on && q + 1 < K, ch * K + q);
                rg[i][q] = ld(rr, on && q + 1 < K, slot * g.CD + ch);
            }
        }
        if (kTag) {   // this token's conv inputs and the a/b dots from the projection tiles
            float av = 0.f, bv = 0.f;
            for (int polls = 0;; polls++) {
                const unsigned long long wa = aload(g.abt + h), wb = aload(g.abt + g.VH + h);
                bool all = (uint32_t)(wa >> 32) == g.epoch && (uint32_t)(wb >> 32) == g.epoch;
                av = __uint_as_float((uint32_t)wa);
                bv = __uint_as_float((uint32_t)wb);
#pragma unroll
                for (int i = 0; i < kCh; i++) {
                    const int t = tid + i * kThreads;
                    const bool on = t < nch;
                    const unsigned long long v = on ? aload(g.qkvt + channel(t)) : 0ull;
                    all &= !on || (uint32_t)(v >> 32) == g.epoch;
                    xin[i] = __uint_as_float((uint32_t)v);
                }
                if (all || poll_give_up(g.err, g.epoch, polls)) break;
            }
            const float sp_in = av + pdtb;
            const float sp = sp_in > 20.f ? sp_in : log1pf(expf(sp_in));
            decay = expf(-expf(palog) * sp);
            beta = 1.f / (1.f + expf(-bv));
        }
#pragma unroll
        for (int i = 0; i < kCh; i++) {
            const int t = tid + i * kThreads;
            if (t >= nch) continue;
            const int ch = channel(t);
            float acc = 0.f;   // the reference's order: older inputs first, this token last
#pragma unroll
            for (int q = 0; q + 1 < kGdnMaxK; q++)
                if (q + 1 < K) acc += cw[i][q] * rg[i][q];
            acc += wlast[i] * xin[i];
            const float v = silu_f(acc);
            if (t < KD) s_q[t] = v;
            else if (t < 2 * KD) s_k[t - KD] = v;
            else s_v[t - 2 * KD] = v;
            if (t >= 2 * KD || owns_qk) g.ring[(size_t)g.head * g.CD + ch] = xin[i];
        }
    } else
    for (int t = tid; t < 2 * KD + kGdnCols; t += kThreads) {
        const int ch = t < KD ? src * KD + t : t < 2 * KD ? key_dim + src * KD + (t - KD)
                                                          : 2 * key_dim + h * g.VD + c0 + (t - 2 * KD);
        const float *w = g.convw + (size_t)ch * g.K;
        const float xn = g.qkv[ch];
        float acc = 0.f;
        for (int q = 0; q + 1 < g.K; q++) {
            int slot = g.head + 1 + q;
            if (slot >= g.K) slot -= g.K;
            acc += w[q] * g.ring[(size_t)slot * g.CD + ch];
        }
        acc += w[g.K - 1] * xn;
        const float v = silu_f(acc);
        if (t < KD) s_q[t] = v;
        else if (t < 2 * KD) s_k[t - KD] = v;
        else s_v[t - 2 * KD] = v;
        if (t >= 2 * KD || owns_qk) g.ring[(size_t)g.head * g.CD + ch] = xn;
    }
    __syncthreads();
    // decay / beta (c/qwen.c:722-728): host params, the a/b dots of the projection launch, or
    // a/b over in_ln(resid) here (the fused kernel's came with the conv inputs)
    if (kTag) {
    } else if (g.params) {
        decay = g.params[h];
        beta = g.params[g.VH + h];
    } else if (g.ab) {   // fmt 6 a/b: projected with qkv/z in one launch
        const float sp_in = pa + pdtb;
        const float sp = sp_in > 20.f ? sp_in : log1pf(expf(sp_in));
        decay = expf(-expf(palog) * sp);
        beta = 1.f / (1.f + expf(-pb));
    } else {
        float r = 0.f;
        if (!g.xin) {
            double ss = 0;
            for (int i = tid; i < g.D; i += kThreads) ss += (double)g.resid[i] * g.resid[i];
            ss = block_sum_d(ss, s_red);
            r = 1.f / sqrtf((float)(ss / g.D) + g.eps);
        }
        float da = 0.f, db = 0.f;
        for (int i = tid; i < g.D; i += kThreads) {
            const float xv = g.xin ? g.xin[i] : g.resid[i] * r * (1.f + g.in_ln[i]);
            da = fmaf(rowmat_w(g.a, h, i), xv, da);
            db = fmaf(rowmat_w(g.b, h, i), xv, db);
        }
        da = wave_sum_f(da);
        db = wave_sum_f(db);
        if (lane == 0) {
            s_ab[0][wave] = da;
            s_ab[1][wave] = db;
        }
        __syncthreads();
        float ta = 0.f, tb = 0.f;
        for (int w = 0; w < kWaves; w++) {
            ta += s_ab[0][w];
            tb += s_ab[1][w];
        }
        if (g.a.fmt == 1) ta *= g.a.sz[h];
        if (g.b.fmt == 1) tb *= g.b.sz[h];
        const float sp_in = ta + g.dtb[h];
        const float sp = sp_in > 20.f ? sp_in : log1pf(expf(sp_in));
        decay = expf(-expf(g.alog[h]) * sp);
        beta = 1.f / (1.f + expf(-tb));
    }

    // l2norm of q and k (c/qwen.c:713-721)
    float sq = 0.f, sk = 0.f;
    if (wave == 0) {
        for (int d = lane; d < KD; d += 64) {
            sq += s_q[d] * s_q[d];
            sk += s_k[d] * s_k[d];
        }
        sq = wave_sum_f(sq);
        sk = wave_sum_f(sk);
        if (lane == 0) {
            s_nrm[0] = sq;
            s_nrm[1] = sk;
        }
    }
    __syncthreads();
    const float rq = 1.f / sqrtf(s_nrm[0] + g.eps) / sqrtf((float)KD);
    const float rk = 1.f / sqrtf(s_nrm[1] + g.eps);
    float kq[KPL], qq[KPL];
#pragma unroll
    for (int e = 0; e < KPL; e++) {
        kq[e] = s_k[lane * KPL + e] * rk;
        qq[e] = s_q[lane * KPL + e] * rq;
    }
    // delta rule per column (c/qwen.c:749-767)
#pragma unroll
    for (int q = 0; q < kGdnColsPerWave; q++) {
        const int vd = c0 + wave * kGdnColsPerWave + q;
        float kv = 0.f;
#pragma unroll
        for (int e = 0; e < KPL; e++) {
            sv[q][e] *= decay;
            kv = fmaf(sv[q][e], kq[e], kv);
        }
        kv = wave_sum_f(kv);
        const float delta = (s_v[vd - c0] - kv) * beta;
        float yv = 0.f;
#pragma unroll
        for (int e = 0; e < KPL; e++) {
            sv[q][e] = fmaf(kq[e], delta, sv[q][e]);
            yv = fmaf(sv[q][e], qq[e], yv);
        }
        yv = wave_sum_f(yv);
        float *col = g.S + ((size_t)h * g.VD + vd) * KD + lane * KPL;
#pragma unroll
        for (int e = 0; e < KPL; e++) col[e] = sv[q][e];
        if (lane == 0) {
            if (kTag) tag_put(g.yt + (size_t)h * g.VD + vd, g.epoch, yv);
            else g.y[(size_t)h * g.VD + vd] = yv;
        }
    }
    if (kTag) {   // one word for the consumers to poll (they still check every y word's tag)
        __syncthreads();
        if (tid == 0) tag_put(g.done + bid, g.epoch, 0.f);
    }
}

template <int KPL>
__global__ __launch_bounds__(kThreads) void gdn_core(GdnArgs g) {
    gdn_core_body<KPL, false>(g, blockIdx.x);
}

// ---------------------------------------------------------------- GDN over a chunk of tokens
// The recurrence of n consecutive tokens in one launch (prefill, c/backend_vulkan.c:2018-
// 2157): the block keeps its (head, 16-column) slice of the state in registers across the
// tokens and walks them in order.  The conv inputs of all n tokens were projected at once
// (qkv [n][CD]); each thread keeps its channels' last K - 1 inputs in registers (from the
// ring for the chunk's first tokens) and prefetches the next token's input while the
// current one computes.  Per token the arithmetic is gdn_core's with host params: the
// same conv order, SiLU, l2 norms and delta rule.  The ring is not written here (other
// blocks still read it for their first tokens): gdn_ring_push stores the chunk's last
// inputs afterwards.
struct GdnSeqArgs {
    const float *qkv;      // [n][CD]
    const float *ring;     // [K][CD], previous inputs at head + 1 .. head + K - 1 (oldest first)
    int head, n;
    const float *convw;    // [CD][K]
    float *S;              // [VH][VD][KD]
    float *y;              // [n][VH * VD]
    const float *params;   // [n][prs]: decay(VH) | beta(VH) | gnorm
    int prs;
    float eps;
    int KH, KD, VH, VD, K, CD;
};

constexpr int kGdnAhead = 8;   // tokens per load group (inputs in flight one group ahead)

// kSeqCPW state columns per wave, kSeqCols per block.  Measured at configs[3] shapes over 512
// tokens: one column per wave (four blocks per CU, the conv and norms of q and k recomputed
// by four times as many blocks) made the whole coli_vk_gdn_full_seq call 1.47 ms against
// 1.30 ms with four.
constexpr int kSeqCPW = 4;
constexpr int kSeqCols = kWaves * kSeqCPW;
template <int KPL>
__global__ __launch_bounds__(kThreads) void gdn_seq(GdnSeqArgs g) {
    // conv outputs of a token, double buffered by token parity: a wave that starts token
    // t + 1 writes the other buffer, and none can start t + 2 before every wave has passed
    // t + 1's barrier, i.e. finished reading t's values: one barrier per token
    __shared__ float s_q[2][kGdnMaxKD], s_k[2][kGdnMaxKD], s_v[2][kSeqCols];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nsl = g.VD / kSeqCols;
    const int h = blockIdx.x / nsl, c0 = (blockIdx.x % nsl) * kSeqCols;
    const int src = h / (g.VH / g.KH), KD = g.KD, key_dim = g.KH * KD, K = g.K;
    float sv[kSeqCPW][KPL];
#pragma unroll
    for (int q = 0; q < kSeqCPW; q++) {
        const float *col = g.S + ((size_t)h * g.VD + c0 + wave * kSeqCPW + q) * KD + lane * KPL;
#pragma unroll
        for (int e = 0; e < KPL; e++) sv[q][e] = col[e];
    }
    constexpr int kCh = (2 * kGdnMaxKD + kSeqCols + kThreads - 1) / kThreads;
    const int nch = 2 * KD + kSeqCols;
    int chn[kCh];
    float cw[kCh][kGdnMaxK - 1], wl[kCh], win[kCh][kGdnMaxK - 1];
#pragma unroll
    for (int i = 0; i < kCh; i++) {
        const int t = tid + i * kThreads;
        const bool on = t < nch;
        chn[i] = !on ? 0
                 : t < KD ? src * KD + t
                 : t < 2 * KD ? key_dim + src * KD + (t - KD)
                              : 2 * key_dim + h * g.VD + c0 + (t - 2 * KD);
#pragma unroll
        for (int q = 0; q + 1 < kGdnMaxK; q++) cw[i][q] = on && q + 1 < K ? g.convw[(size_t)chn[i] * K + q] : 0.f;
        wl[i] = on ? g.convw[(size_t)chn[i] * K + K - 1] : 0.f;
#pragma unroll
        for (int q = 0; q + 1 < kGdnMaxK; q++) {
            int slot = g.head + 1 + q;
            if (slot >= K) slot -= K;
            win[i][q] = on && q + 1 < K ? g.ring[(size_t)slot * g.CD + chn[i]] : 0.f;
        }
    }
    // inputs and params by groups of kGdnAhead tokens: the next group's loads go out when a
    // group starts, so the one wait per group (at its start) finds them long arrived
    const __amdgpu_buffer_rsrc_t rq = buf_rsrc(g.qkv, (uint32_t)g.n * (uint32_t)g.CD * 4u);
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(g.params, (uint32_t)g.n * (uint32_t)g.prs * 4u);
    auto ldf = [](__amdgpu_buffer_rsrc_t r, bool on, uint32_t i) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, on ? (int)(i * 4u) : (int)kOOB, 0, 0));
    };
    float xn[kCh][kGdnAhead], dn[kGdnAhead], bn[kGdnAhead];
    auto group_load = [&](int t0) {
#pragma unroll
        for (int j = 0; j < kGdnAhead; j++) {
            const bool on = t0 + j < g.n;
            const uint32_t tk = (uint32_t)(t0 + j);
#pragma unroll
            for (int i = 0; i < kCh; i++) xn[i][j] = ldf(rq, on && tid + i * kThreads < nch, tk * g.CD + chn[i]);
            dn[j] = ldf(rp, on, tk * g.prs + h);
            bn[j] = ldf(rp, on, tk * g.prs + g.VH + h);
        }
    };
    group_load(0);
    for (int tok0 = 0; tok0 < g.n; tok0 += kGdnAhead) {
        float xg[kCh][kGdnAhead], dg[kGdnAhead], bg[kGdnAhead];
#pragma unroll
        for (int j = 0; j < kGdnAhead; j++) {
#pragma unroll
            for (int i = 0; i < kCh; i++) xg[i][j] = xn[i][j];
            dg[j] = dn[j];
            bg[j] = bn[j];
        }
        if (tok0 + kGdnAhead < g.n) group_load(tok0 + kGdnAhead);
#pragma unroll
        for (int j = 0; j < kGdnAhead; j++) {
            const int tok = tok0 + j;
            if (tok < g.n) {   // uniform
                const int pb = j & 1;   // kGdnAhead is even: parity of tok
                float xin[kCh];
                const float decay = dg[j], beta = bg[j];
#pragma unroll
                for (int i = 0; i < kCh; i++) xin[i] = xg[i][j];
                // conv1d + SiLU (c/qwen.c:697-707), older inputs first, this token last
#pragma unroll
                for (int i = 0; i < kCh; i++) {
                    const int t = tid + i * kThreads;
                    float acc = 0.f;
#pragma unroll
                    for (int q = 0; q + 1 < kGdnMaxK; q++)
                        if (q + 1 < K) acc += cw[i][q] * win[i][q];
                    acc += wl[i] * xin[i];
                    // the window moves on: the K - 1 newest inputs, oldest first
#pragma unroll
                    for (int q = 0; q + 1 < kGdnMaxK; q++) {
                        if (q + 2 < K) win[i][q] = win[i][q + 1];
                        else if (q + 2 == K) win[i][q] = xin[i];
                    }
                    if (t < nch) {
                        const float v = silu_f(acc);
                        if (t < KD) s_q[pb][t] = v;
                        else if (t < 2 * KD) s_k[pb][t - KD] = v;
                        else s_v[pb][t - 2 * KD] = v;
                    }
                }
                __syncthreads();
                // l2norm of q and k (c/qwen.c:713-721), each wave for itself
                float sq = 0.f, sk = 0.f;
                for (int d = lane; d < KD; d += 64) {
                    sq += s_q[pb][d] * s_q[pb][d];
                    sk += s_k[pb][d] * s_k[pb][d];
                }
                sq = wave_sum_f(sq);
                sk = wave_sum_f(sk);
                const float rqn = 1.f / sqrtf(sq + g.eps) / sqrtf((float)KD);
                const float rkn = 1.f / sqrtf(sk + g.eps);
                float kq[KPL], qq[KPL];
#pragma unroll
                for (int e = 0; e < KPL; e++) {
                    kq[e] = s_k[pb][lane * KPL + e] * rkn;
                    qq[e] = s_q[pb][lane * KPL + e] * rqn;
                }
                // delta rule per column (c/qwen.c:749-767)
#pragma unroll
                for (int q = 0; q < kSeqCPW; q++) {
                    const int vd = c0 + wave * kSeqCPW + q;
                    float kv = 0.f;
#pragma unroll
                    for (int e = 0; e < KPL; e++) {
                        sv[q][e] *= decay;
                        kv = fmaf(sv[q][e], kq[e], kv);
                    }
                    kv = wave_sum_f(kv);
                    const float delta = (s_v[pb][vd - c0] - kv) * beta;
                    float yv = 0.f;
#pragma unroll
                    for (int e = 0; e < KPL; e++) {
                        sv[q][e] = fmaf(kq[e], delta, sv[q][e]);
                        yv = fmaf(sv[q][e], qq[e], yv);
                    }
                    yv = wave_sum_f(yv);
                    if (lane == 0) g.y[(size_t)tok * g.VH * g.VD + (size_t)h * g.VD + vd] = yv;
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < kSeqCPW; q++) {
        float *col = g.S + ((size_t)h * g.VD + c0 + wave * kSeqCPW + q) * KD + lane * KPL;
#pragma unroll
        for (int e = 0; e < KPL; e++) col[e] = sv[q][e];
    }
}

// The chunk's inputs into the conv ring as if its tokens had been pushed one at a time:
// token t's input at slot (head + t) % K; only the last K tokens survive.
__global__ void gdn_ring_push(const float *__restrict__ qkv, int n, float *__restrict__ ring, int head, int K,
                              int CD) {
    const int t0 = n > K ? n - K : 0, cnt = n - t0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)cnt * CD;
         i += (size_t)gridDim.x * blockDim.x) {
        const int t = t0 + (int)(i / CD), c = (int)(i % CD);
        ring[(size_t)((head + t) % K) * CD + c] = qkv[(size_t)t * CD + c];
    }
}

// ---------------------------------------------------------------- chunked GatedDeltaNet recurrence
// The delta rule of c/qwen.c:749-767 (per value column: s = decay s; kv = s . k;
// delta = (v - kv) beta; s += k delta; y = s . q) over a chunk of kGc tokens from the state
// s_0, in closed form.  With G_t = sum over j <= t of log decay_j:
//   s_t = e^{G_t} s_0 + sum_{i <= t} e^{G_t - G_i} k_i delta_i
//   (I + L) delta = r,  L[t][i] = beta_t e^{G_t - G_i} (k_t . k_i) for i < t,
//                       r_t = beta_t (v_t - e^{G_t} (k_t . s_0))
//   y_t = e^{G_t} (q_t . s_0) + sum_{i <= t} e^{G_t - G_i} (q_t . k_i) delta_i
//   s_end = e^{G_end} s_0 + sum_i e^{G_end - G_i} k_i delta_i
// Each value column is independent, so a scan block takes kGcCols columns of one v-head
// through the chunks in order.  T = (I + L)^-1 and M[t][i] = e^{G_t - G_i} (q_t . k_i)
// (i <= t) depend only on the head and the chunk: gdn_chunk_mats forms them for all chunks
// at once.  The result equals gdn_seq's token-by-token recurrence up to fp32 rounding (the
// decays enter as exponentials of summed logs instead of repeated products).  Tokens past
// the end of the last chunk are padding: k = q = v = 0, beta = 0, decay = 1, so they change
// nothing and their outputs are not stored.
static int g_gdn_chunked = 1;  // prefill recurrence in closed form per chunk (0: gdn_seq)
typedef float coli_v4f __attribute__((ext_vector_type(4)));
constexpr int kGc = 64;        // tokens per chunk
constexpr int kGcCols = 16;    // value columns per scan block
constexpr int kGcConvT = 16;   // tokens per conv block
constexpr int kGcMaxKD = 128;  // key head dims of the chunked path
constexpr int kGcMat = 2 * kGc * kGc + 2 * kGc + 4;   // floats per (head, chunk): T, M, e^G, w, e^G_end
constexpr float kGcMinLog = -87.f;   // log decay clamp: e^-87 is still a normal float

struct GdnChunkArgs {
    const float *qkv;      // [n][CD] projected inputs of the call's tokens
    const float *ring;     // [K][CD] previous inputs (see GdnSeqArgs)
    int head, n;
    const float *convw;    // [CD][K]
    const float *params;   // [n][prs]: decay(VH) | beta(VH) | gnorm
    int prs;
    float eps;
    int KH, KD, VH, VD, K, CD, nchunk;
    float *qn, *kn;        // [n][KH][KD] normed q (times 1/sqrt(KD)) and k
    float *vv;             // [n][CD] conv + SiLU of every channel (q | k | v)
    float *mats;           // [VH][nchunk][kGcMat]
    float *S;              // [VH][VD][KD] state, updated in place
    float *y;              // [n][VH][VD]
};

// Conv1d + SiLU of every channel (c/qwen.c:697-707; the window's older inputs first, this
// token last, as gdn_seq): one thread per channel walks kGcConvT tokens with its K - 1 previous
// inputs in registers; the loads of a token row are one coalesced pass.
__global__ __launch_bounds__(kThreads) void gdn_chunk_conv(GdnChunkArgs g) {
    const int ch = blockIdx.x * kThreads + threadIdx.x, t0 = blockIdx.y * kGcConvT, K = g.K;
    if (ch >= g.CD) return;
    float cw[kGdnMaxK], win[kGdnMaxK - 1];
#pragma unroll
    for (int q = 0; q < kGdnMaxK; q++) cw[q] = q < K ? g.convw[(size_t)ch * K + q] : 0.f;
#pragma unroll
    for (int q = 0; q + 1 < kGdnMaxK; q++) {   // inputs t0 - (K - 1) + q: this call's rows or the ring
        const int tp = t0 - (K - 1) + q;
        win[q] = q + 1 >= K ? 0.f
                 : tp >= 0  ? g.qkv[(size_t)tp * g.CD + ch]
                            : g.ring[(size_t)((g.head + K + tp) % K) * g.CD + ch];
    }
    const int nt = min(kGcConvT, g.n - t0);
    constexpr int kU = 8;   // token rows loaded ahead
    for (int j0 = 0; j0 < nt; j0 += kU) {
        float xin[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) xin[u] = j0 + u < nt ? g.qkv[(size_t)(t0 + j0 + u) * g.CD + ch] : 0.f;
#pragma unroll
        for (int u = 0; u < kU; u++) {
            if (j0 + u >= nt) break;
            float acc = 0.f;
#pragma unroll
            for (int q = 0; q + 1 < kGdnMaxK; q++)
                if (q + 1 < K) acc += cw[q] * win[q];
            acc += cw[K - 1] * xin[u];
#pragma unroll
            for (int q = 0; q + 1 < kGdnMaxK; q++) {
                if (q + 2 < K) win[q] = win[q + 1];
                else if (q + 2 == K) win[q] = xin[u];
            }
            g.vv[(size_t)(t0 + j0 + u) * g.CD + ch] = silu_f(acc);
        }
    }
}

// l2 norms of q and k (c/qwen.c:713-721): one wave per (token, head), each lane's columns
// summed in order and the wave's sum by DPP, as gdn_seq does it.
__global__ __launch_bounds__(kThreads) void gdn_chunk_norm(GdnChunkArgs g) {
    const int w = blockIdx.x * kWaves + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int tok = w / (2 * g.KH), hh = w % (2 * g.KH);
    if (tok >= g.n) return;   // wave uniform
    const float *v = g.vv + (size_t)tok * g.CD + (size_t)hh * g.KD;
    float x[kGcMaxKD / 64];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kGcMaxKD / 64; i++) {
        const int d = lane + 64 * i;
        x[i] = d < g.KD ? v[d] : 0.f;
        if (d < g.KD) ss += x[i] * x[i];
    }
    ss = wave_sum_f(ss);
    const bool isq = hh < g.KH;
    const float r = isq ? 1.f / sqrtf(ss + g.eps) / sqrtf((float)g.KD) : 1.f / sqrtf(ss + g.eps);
    float *dst = isq ? g.qn + ((size_t)tok * g.KH + hh) * g.KD : g.kn + ((size_t)tok * g.KH + hh - g.KH) * g.KD;
#pragma unroll
    for (int i = 0; i < kGcMaxKD / 64; i++) {
        const int d = lane + 64 * i;
        if (d < g.KD) dst[d] = x[i] * r;
    }
}

// Rows [t0, t0 + kGc) of a [n][KH][KD] array for k-head src into s[kGc][ld] (zeros past n),
// 16-byte loads, all of a thread's loads issued before its stores.
template <int LD>
__device__ __forceinline__ void gc_rows(const float *a, int t0, int n, int KH, int src, int KD, float (*s)[LD]) {
    constexpr int kPer = kGc * kGcMaxKD / 4 / kThreads;   // float4 per thread at KD = kGcMaxKD (8)
    const int q4 = KD / 4;
    float4 v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int f = threadIdx.x + i * kThreads, t = f / q4, e = (f - t * q4) * 4;
        v[i] = t < kGc && t0 + t < n ? *(const float4 *)(a + ((size_t)(t0 + t) * KH + src) * KD + e)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int f = threadIdx.x + i * kThreads, t = f / q4, e = (f - t * q4) * 4;
        if (t < kGc) *(float4 *)&s[t][e] = v[i];
    }
}

// One block per (v-head, chunk): G, the Gram products, T = (I + L)^-1 and M, the products on
// fp32 MFMA in the lane layout of gdn_chunk_scan.  T by block forward substitution over its
// 16 x 16 blocks: wave w inverts diagonal block w by rows, one lane per column, then block
// (r, c) = -T[r][r] sum_{c <= m < r} L[r][m] T[m][c], one block distance at a time.
__global__ __launch_bounds__(kThreads) void gdn_chunk_mats(GdnChunkArgs g) {
    constexpr int LDK = kGcMaxKD + 4, LDT = kGc + 4, NB = kGc / 16;
    static_assert(NB == kWaves, "one diagonal block per wave");
    __shared__ __attribute__((aligned(16))) float sK[kGc][LDK], sQ[kGc][LDK];
    __shared__ __attribute__((aligned(16))) float sL[kGc][LDT], sT[kGc][LDT];
    __shared__ float sG[kGc], sBe[kGc];
    const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x, KD = g.KD;
    const int wave = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    const int src = h / (g.VH / g.KH), t0 = c * kGc, nt = min(kGc, g.n - t0);
    gc_rows<LDK>(g.kn, t0, g.n, g.KH, src, KD, sK);
    gc_rows<LDK>(g.qn, t0, g.n, g.KH, src, KD, sQ);
    for (int i = tid; i < kGc * LDT; i += kThreads) (&sT[0][0])[i] = 0.f;
    if (wave == 0) {   // G_t: the logs up to t, an inclusive scan across the wave (kGc = 64)
        const bool on = lane < nt;
        float a = on ? fmaxf(logf(g.params[(size_t)(t0 + lane) * g.prs + h]), kGcMinLog) : 0.f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float u = __shfl_up(a, o);
            if (lane >= o) a += u;
        }
        sG[lane] = a;
        sBe[lane] = on ? g.params[(size_t)(t0 + lane) * g.prs + g.VH + h] : 0.f;
    }
    __syncthreads();
    auto mfma = [](float a, float b, coli_v4f c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); };
    float *mat = g.mats + ((size_t)h * g.nchunk + c) * kGcMat;   // T [kGc][kGc] | M | e^G | w | e^G_end
    // Gram tiles (ti, tj <= ti): ten of K K^T (into L), then ten of Q K^T (into M)
    for (int u = wave; u < NB * (NB + 1); u += kWaves) {
        const bool isq = u >= NB * (NB + 1) / 2;
        const int v = isq ? u - NB * (NB + 1) / 2 : u;
        int ti = 0;
        while ((ti + 1) * (ti + 2) / 2 <= v) ti++;
        const int tj = v - ti * (ti + 1) / 2;
        const float(*A)[LDK] = isq ? sQ : sK;
        coli_v4f acc = {0.f, 0.f, 0.f, 0.f};
        for (int kb = 0; kb < KD; kb += 16) {
            const float4 a4 = *(const float4 *)&A[16 * ti + li][kb + 4 * lg];
            const float4 b4 = *(const float4 *)&sK[16 * tj + li][kb + 4 * lg];
            acc = mfma(a4.x, b4.x, acc);
            acc = mfma(a4.y, b4.y, acc);
            acc = mfma(a4.z, b4.z, acc);
            acc = mfma(a4.w, b4.w, acc);
        }
        const int i = 16 * tj + li;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = 16 * ti + 4 * lg + r;
            const float dec = expf(sG[t] - sG[min(i, t)]);
            if (!isq) sL[t][i] = i < t ? sBe[t] * dec * acc[r] : 0.f;
            else mat[kGc * kGc + t * kGc + i] = i <= t ? dec * acc[r] : 0.f;
        }
    }
    for (int idx = tid; idx < kGc * kGc; idx += kThreads) {   // M right of the diagonal blocks
        const int t = idx / kGc, i = idx % kGc;
        if (i / 16 > t / 16) mat[kGc * kGc + idx] = 0.f;
    }
    __syncthreads();
    {   // diagonal block wave: T[t][j] = [t == j] - sum_{i < t} L[t][i] T[i][j], column j = li
        const int o = 16 * wave;
        float col[16];
#pragma unroll
        for (int t = 0; t < 16; t++) {
            float acc = t == li ? 1.f : 0.f;
#pragma unroll
            for (int i = 0; i < t; i++) acc = fmaf(-sL[o + t][o + i], col[i], acc);
            col[t] = acc;
        }
        if (lg == 0) {
#pragma unroll
            for (int t = 0; t < 16; t++) sT[o + t][o + li] = col[t];
        }
    }
    __syncthreads();
    for (int dist = 1; dist < NB; dist++) {
        const int cb = wave, rb = wave + dist;
        if (rb < NB) {   // wave uniform
            coli_v4f x = {0.f, 0.f, 0.f, 0.f};
            for (int mb = cb; mb < rb; mb++) {   // X = sum_mb L[rb][mb] T[mb][cb]
                const float4 l4 = *(const float4 *)&sL[16 * rb + li][16 * mb + 4 * lg];
                x = mfma(l4.x, sT[16 * mb + 4 * lg][16 * cb + li], x);
                x = mfma(l4.y, sT[16 * mb + 4 * lg + 1][16 * cb + li], x);
                x = mfma(l4.z, sT[16 * mb + 4 * lg + 2][16 * cb + li], x);
                x = mfma(l4.w, sT[16 * mb + 4 * lg + 3][16 * cb + li], x);
            }
            // T[rb][cb] = -T[rb][rb] X, X as B in its D layout (register s holds k = 4 lg + s)
            const float4 d4 = *(const float4 *)&sT[16 * rb + li][16 * rb + 4 * lg];
            coli_v4f y = {0.f, 0.f, 0.f, 0.f};
            y = mfma(d4.x, x[0], y);
            y = mfma(d4.y, x[1], y);
            y = mfma(d4.z, x[2], y);
            y = mfma(d4.w, x[3], y);
#pragma unroll
            for (int r = 0; r < 4; r++) sT[16 * rb + 4 * lg + r][16 * cb + li] = -y[r];
        }
        __syncthreads();
    }
    for (int i = tid; i < kGc * kGc / 4; i += kThreads)
        ((float4 *)mat)[i] = *(const float4 *)&sT[4 * i / kGc][4 * i % kGc];
    if (tid < kGc) {
        mat[2 * kGc * kGc + tid] = expf(sG[tid]);
        mat[2 * kGc * kGc + kGc + tid] = expf(sG[kGc - 1] - sG[tid]);
    }
    if (tid == 0) mat[2 * kGc * kGc + 2 * kGc] = expf(sG[kGc - 1]);
}

// One block per (v-head, kGcCols value columns): the chunks in order, the columns' state
// slice in LDS, every product on fp32 MFMA (v_mfma_f32_16x16x4_f32: lane l gives A[l % 16]
// [l / 16] and B[l / 16][l % 16]; D[4 (l / 16) + r][l % 16] is its register r).  A lane
// gives the four k = kb + 4 (l / 16) + s of a 16-wide k block over four MFMAs (s = 0..3),
// so each operand is one 16-byte LDS read, and D's layout is B's for the next product.
// Wave w forms tokens 16 w .. + 15 of a = K s, b = Q s, r, delta = T r and y = e^G b + M delta
// and key tiles w, w + 4, .. of the state.  T and M are zero right of their diagonal blocks,
// so every wave takes all four token blocks of T r and M delta (wave 3 needs them all anyway)
// and issues its LDS reads before its MFMAs.  The next chunk's operands are loaded into
// registers in three parts between the k blocks of a and b, one load per two MFMAs (the
// scheduler's group barriers), while the MFMAs run.
template <int KD>
__global__ __launch_bounds__(kThreads) void gdn_chunk_scan(GdnChunkArgs g) {
    static_assert(KD % 64 == 0 && KD <= kGcMaxKD, "key tiles per wave");
    constexpr int LDK = KD + 4, LDT = kGc + 4, NTB = kGc / 16, kTW = KD / 16 / kWaves;
    constexpr int kKQ = kGc * KD / 4 / kThreads, kTM = kGc * kGc / 4 / kThreads, kSV = kGcCols * KD / 4 / kThreads;
    __shared__ __attribute__((aligned(16))) float sK[kGc][LDK], sQ[kGc][LDK];
    __shared__ __attribute__((aligned(16))) float sT[kGc][LDT], sM[kGc][LDT];
    __shared__ __attribute__((aligned(16))) float sS[kGcCols][LDK];   // state slice, [column][key]
    __shared__ __attribute__((aligned(16))) float sR[kGcCols][LDT], sD[kGcCols][LDT], sWD[kGcCols][LDT];
    const int nsl = g.VD / kGcCols, h = blockIdx.x / nsl, c0 = (blockIdx.x % nsl) * kGcCols;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    const int src = h / (g.VH / g.KH), key_dim = g.KH * KD;
    const int row0 = 16 * wave + 4 * lg, r16 = 16 * wave + li;   // D rows of this lane; A row
    // the slice's columns are adjacent in S ([VH][VD][KD]): one contiguous run of kGcCols KD floats
    coli_v4f *Sg = (coli_v4f *)(g.S + ((size_t)h * g.VD + c0) * KD);
    {
        coli_v4f sv[kSV];
#pragma unroll
        for (int i = 0; i < kSV; i++) sv[i] = Sg[tid + i * kThreads];
#pragma unroll
        for (int i = 0; i < kSV; i++) {
            const int f = 4 * (tid + i * kThreads);
            *(coli_v4f *)&sS[f / KD][f % KD] = sv[i];
        }
    }
    coli_v4f pk[kKQ], pq[kKQ], pt[kTM], pm[kTM];
    float4 pe, pw;
    float pv[4], pb[4], pend;
    // The loads of a chunk go through buffer descriptors bounded by the arrays' sizes, so rows
    // past n (and a chunk past the last) read as zeros without a branch; a chunk past the last
    // of head h reads head h + 1's first matrices or zeros, and is never stored.
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(g.kn, (uint32_t)g.n * g.KH * KD * 4u);
    const __amdgpu_buffer_rsrc_t rq = buf_rsrc(g.qn, (uint32_t)g.n * g.KH * KD * 4u);
    const __amdgpu_buffer_rsrc_t rm = buf_rsrc(g.mats, (uint32_t)g.VH * g.nchunk * kGcMat * 4u);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(g.vv, (uint32_t)g.n * g.CD * 4u);
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(g.params, (uint32_t)g.n * g.prs * 4u);
    auto ld4 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
        return __builtin_bit_cast(coli_v4f, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
    };
    auto ld1 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
    };
    auto fetch_kq = [&](int c, __amdgpu_buffer_rsrc_t r, coli_v4f *dst) {
        const uint32_t t0 = (uint32_t)c * kGc;
#pragma unroll
        for (int i = 0; i < kKQ; i++) {
            const int f = tid + i * kThreads, t = f / (KD / 4), e = (f % (KD / 4)) * 4;
            dst[i] = ld4(r, (((t0 + t) * g.KH + src) * KD + e) * 4u);
        }
    };
    auto fetch_rest = [&](int c) {
        const uint32_t t0 = (uint32_t)c * kGc, mo = ((uint32_t)h * g.nchunk + c) * kGcMat;
#pragma unroll
        for (int i = 0; i < kTM; i++) {
            pt[i] = ld4(rm, (mo + 4 * (tid + i * kThreads)) * 4u);
            pm[i] = ld4(rm, (mo + kGc * kGc + 4 * (tid + i * kThreads)) * 4u);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t t = t0 + row0 + r;
            pv[r] = ld1(rv, (t * g.CD + 2 * key_dim + h * g.VD + c0 + li) * 4u);
            pb[r] = ld1(rp, (t * g.prs + g.VH + h) * 4u);
        }
        const coli_v4f e4 = ld4(rm, (mo + 2 * kGc * kGc + row0) * 4u);
        const coli_v4f w4 = ld4(rm, (mo + 2 * kGc * kGc + kGc + row0) * 4u);
        pe = make_float4(e4[0], e4[1], e4[2], e4[3]);
        pw = make_float4(w4[0], w4[1], w4[2], w4[3]);
        pend = ld1(rm, (mo + 2 * kGc * kGc + 2 * kGc) * 4u);
    };
    auto mfma = [](float a, float b, coli_v4f c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); };
    fetch_kq(0, rk, pk);
    fetch_kq(0, rq, pq);
    fetch_rest(0);
    for (int c = 0; c < g.nchunk; c++) {
        const int t0 = c * kGc;
#pragma unroll
        for (int i = 0; i < kKQ; i++) {
            const int f = tid + i * kThreads, t = f / (KD / 4), e = (f % (KD / 4)) * 4;
            *(coli_v4f *)&sK[t][e] = pk[i];
            *(coli_v4f *)&sQ[t][e] = pq[i];
        }
#pragma unroll
        for (int i = 0; i < kTM; i++) {
            const int f = 4 * (tid + i * kThreads);
            *(coli_v4f *)&sT[f / kGc][f % kGc] = pt[i];
            *(coli_v4f *)&sM[f / kGc][f % kGc] = pm[i];
        }
        const float4 eg = pe, wt = pw;
        const float eend = pend;
        float v[4], be[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            v[r] = pv[r];
            be[r] = pb[r];
        }
        __syncthreads();   // the chunk's K, Q, T, M and the state slice in LDS
        // a = K s and b = Q s
        coli_v4f a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KD; kb += 16) {
            const coli_v4f k4 = *(const coli_v4f *)&sK[r16][kb + 4 * lg];
            const coli_v4f x4 = *(const coli_v4f *)&sQ[r16][kb + 4 * lg];
            const coli_v4f s4 = *(const coli_v4f *)&sS[li][kb + 4 * lg];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                a = mfma(k4[s], s4[s], a);
                b = mfma(x4[s], s4[s], b);
            }
            if (kb == 0) fetch_kq(c + 1, rk, pk);   // the next chunk's (zeros past the last)
            else if (kb == 16) fetch_kq(c + 1, rq, pq);
            else if (kb == 32) fetch_rest(c + 1);
            // per k block: its 3 LDS reads, then 2 MFMAs per global load of the next chunk
            __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
        }
        // r = beta (v - e^G a)
        *(float4 *)&sR[li][row0] = make_float4(be[0] * (v[0] - eg.x * a[0]), be[1] * (v[1] - eg.y * a[1]),
                                               be[2] * (v[2] - eg.z * a[2]), be[3] * (v[3] - eg.w * a[3]));
        __syncthreads();
        // delta = T r
        coli_v4f op[NTB], rv[NTB];
#pragma unroll
        for (int j = 0; j < NTB; j++) {
            op[j] = *(const coli_v4f *)&sT[r16][16 * j + 4 * lg];
            rv[j] = *(const coli_v4f *)&sR[li][16 * j + 4 * lg];
        }
        coli_v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NTB; j++)
#pragma unroll
            for (int s = 0; s < 4; s++) d = mfma(op[j][s], rv[j][s], d);
        *(float4 *)&sD[li][row0] = make_float4(d[0], d[1], d[2], d[3]);
        *(float4 *)&sWD[li][row0] = make_float4(wt.x * d[0], wt.y * d[1], wt.z * d[2], wt.w * d[3]);
        __syncthreads();
        // y = e^G b + M delta
#pragma unroll
        for (int j = 0; j < NTB; j++) {
            op[j] = *(const coli_v4f *)&sM[r16][16 * j + 4 * lg];
            rv[j] = *(const coli_v4f *)&sD[li][16 * j + 4 * lg];
        }
        coli_v4f y = {eg.x * b[0], eg.y * b[1], eg.z * b[2], eg.w * b[3]};
#pragma unroll
        for (int j = 0; j < NTB; j++)
#pragma unroll
            for (int s = 0; s < 4; s++) y = mfma(op[j][s], rv[j][s], y);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (t0 + row0 + r < g.n) g.y[((size_t)(t0 + row0 + r) * g.VH + h) * g.VD + c0 + li] = y[r];
        // s = e^G_end s + K^T (w delta), key tiles m = wave + kWaves j: A[e][t] = K[t][16 m + e]
        coli_v4f acc[kTW];
#pragma unroll
        for (int j = 0; j < kTW; j++) {
            const coli_v4f s4 = *(const coli_v4f *)&sS[li][16 * (wave + kWaves * j) + 4 * lg];
            acc[j] = eend * s4;
        }
#pragma unroll
        for (int tb = 0; tb < NTB; tb++) {
            const coli_v4f w4 = *(const coli_v4f *)&sWD[li][16 * tb + 4 * lg];
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int j = 0; j < kTW; j++)
                    acc[j] = mfma(sK[16 * tb + 4 * lg + s][16 * (wave + kWaves * j) + li], w4[s], acc[j]);
        }
#pragma unroll
        for (int j = 0; j < kTW; j++) *(coli_v4f *)&sS[li][16 * (wave + kWaves * j) + 4 * lg] = acc[j];
        __syncthreads();   // the chunk's operands are replaced by the next chunk's
    }
#pragma unroll
    for (int i = 0; i < kSV; i++) {
        const int f = 4 * (tid + i * kThreads);
        Sg[tid + i * kThreads] = *(const coli_v4f *)&sS[f / KD][f % KD];
    }
}

// ---------------------------------------------------------------- GQA attention
constexpr int kAttT = 32;       // positions per chunk (block)
constexpr int kAttW = 8;        // waves of an attn_part block
constexpr int kAttMaxG = 16;    // query heads per kv head
constexpr int kAttMaxHD = 512;
constexpr int kAttMaxHR = 64;   // rotary pairs (rot / 2)

struct AttnArgs {
    const float *q;      // [H][2 hd]: q | gate per head (projection output)
    const float *k, *v;  // [KH][hd] projections of this token
    const float *qn, *kn;
    float *Kc, *Vc;      // [KH][max_t][hd]
    float *part;         // [KH][nsplit][G][hd + 2]: ctx, then m, l
    float *ctx;          // [H * hd] merged, gated
    int H, KH, hd, rot, pos, max_t, nsplit;
    float eps, scale;
    float cs[kAttMaxHR], sn[kAttMaxHR];   // rotation at pos (host: c/qwen.c:570-579 in double)
};

// zero-centred RMSNorm over hd, then partial RoPE at pos (c/qwen.c:326-330, :570-579), of
// the row src into the LDS row x and, if gdst != NULL, into gdst.  One wave; every output
// element is written by the lane that computes it from src (no cross-lane LDS reads).
// The loads of one row (issued by row_load, consumed by row_finish): the row and its norm
// weight at lane + 64 q, and the lane's rotation pairs (jj, jj + hr) with their weights and
// cos/sin.  Splitting lets a wave issue several rows' loads before it waits for any.
struct RowLd {
    static constexpr int kPer = kAttMaxHD / 64, kPairs = (kAttMaxHR + 63) / 64;
    float v[kPer], wv[kPer], lo[kPairs], hi[kPairs], wl[kPairs], wh[kPairs], cs[kPairs], sn[kPairs];
};
// NQ: the 64-column slots to load (hd / 64, known to the caller at compile time; the others
// read as 0).  live = false: every load reads 0 without a memory access.  No branch sits
// around a load, so the compiler's wait counts stay exact and nothing waits early.
template <int NQ = RowLd::kPer>
__device__ __forceinline__ void row_load(RowLd &R, const float *src, const float *w, const AttnArgs &a,
                                         bool live = true) {
    static_assert(NQ >= 1 && NQ <= RowLd::kPer, "slots");
    const int lane = threadIdx.x & 63, hd = a.hd, hr = a.rot / 2;
    const uint32_t nb = live ? (uint32_t)hd * 4 : 0u;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(src, nb), rw = buf_rsrc(w, nb);
    auto ld = [](__amdgpu_buffer_rsrc_t r, bool on, int i) {   // unconditional: out of range reads 0
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, on ? i * 4 : (int)kOOB, 0, 0));
    };
#pragma unroll
    for (int q = 0; q < RowLd::kPer; q++) {
        const int d = lane + 64 * q;
        R.v[q] = q < NQ ? ld(rs, d < hd, d) : 0.f;
        R.wv[q] = q < NQ ? ld(rw, d < hd, d) : 0.f;
    }
#pragma unroll
    for (int p = 0; p < RowLd::kPairs; p++) {
        const int jj = lane + 64 * p, jc = jj < kAttMaxHR ? jj : kAttMaxHR - 1;
        const bool on = jj < hr;
        R.lo[p] = ld(rs, on, jj);
        R.hi[p] = ld(rs, on, jj + hr);
        R.wl[p] = ld(rw, on, jj);
        R.wh[p] = ld(rw, on, jj + hr);
        R.cs[p] = a.cs[jc];
        R.sn[p] = a.sn[jc];
    }
}
// zero-centred RMSNorm over hd, then partial RoPE at pos, of a loaded row into the LDS row x
// and, if gdst != NULL, into gdst.  One wave; every output element is written by the lane
// that computes it (no cross-lane LDS reads).
__device__ __forceinline__ void row_finish(float *x, float *gdst, const RowLd &R, const AttnArgs &a) {
    const int lane = threadIdx.x & 63, hd = a.hd, hr = a.rot / 2;
    double ss = 0;
#pragma unroll
    for (int q = 0; q < RowLd::kPer; q++) ss += (double)R.v[q] * R.v[q];   // zeros past hd add 0
    ss = wave_sum_d(ss);
    const float r = 1.f / sqrtf((float)(ss / hd) + a.eps);
#pragma unroll
    for (int q = 0; q < RowLd::kPer; q++) {
        const int d = lane + 64 * q;
        if (d >= a.rot && d < hd) {
            const float o = R.v[q] * r * (1.f + R.wv[q]);
            x[d] = o;
            if (gdst) gdst[d] = o;
        }
    }
#pragma unroll
    for (int p = 0; p < RowLd::kPairs; p++) {
        const int jj = lane + 64 * p;
        if (jj < hr) {
            const float l = R.lo[p] * r * (1.f + R.wl[p]), h = R.hi[p] * r * (1.f + R.wh[p]);
            const float o0 = l * R.cs[p] - h * R.sn[p], o1 = h * R.cs[p] + l * R.sn[p];
            x[jj] = o0;
            x[jj + hr] = o1;
            if (gdst) {
                gdst[jj] = o0;
                gdst[jj + hr] = o1;
            }
        }
    }
}
template <int NQ = RowLd::kPer>
__device__ __forceinline__ void norm_rope_row(float *x, float *gdst, const float *src, const float *w, const AttnArgs &a) {
    RowLd R;
    row_load<NQ>(R, src, w, a);
    row_finish(x, gdst, R, a);
}

// One block per (kv head, chunk of kAttT positions).  The q rows of the group (and the new
// key row, in the chunk holding pos) are loaded first, then every K and V element the block
// needs (one memory round trip); the q rows are normed and rotated while
// K and V arrive, scores computed, the chunk softmax taken and P.V accumulated.  The block
// barriers are LDS-only, so no phase waits for loads it does not use.
template <int DPL, int AW>
__global__ __launch_bounds__(64 * AW) void attn_part(AttnArgs a) {
    constexpr int kT = 64 * AW;                 // threads of the block (AW waves)
    constexpr int kSteps = kAttT / (AW * 4);   // position steps per wave (4 positions each)
    constexpr int kPV = kT > 256 ? 256 : kT;    // P.V threads per head half (AW 8: two halves of the heads)
    constexpr int kVPer = kAttMaxHD / kPV;      // head dims per thread in P.V
    __shared__ __attribute__((aligned(16))) float s_q[kAttMaxG][kAttMaxHD];
    __shared__ __attribute__((aligned(16))) float s_k[kAttMaxHD];
    __shared__ __attribute__((aligned(16))) float s_p[kAttMaxG][kAttT];
    __shared__ __attribute__((aligned(16))) float s_v[kAttT][kAttMaxHD];
    __shared__ float s_m[kAttMaxG], s_l[kAttMaxG];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.H / a.KH, hd = a.hd;
    const int kh = blockIdx.x / a.nsplit, sp = blockIdx.x % a.nsplit;
    const int t0 = sp * kAttT, t1 = min(t0 + kAttT, a.pos + 1), n = t1 - t0;
    const bool owns_pos = a.pos >= t0 && a.pos < t1;
    // K rows of the score steps (16 lanes per position, DPL dims each) and V columns of
    // P.V (thread pvt: dims pvt + kPV * i), all in flight together
    // (branch-free buffer loads: out-of-range offsets read 0, so no load waits behind a
    // data-dependent branch)
    // the wave's first q row and, in the chunk holding pos, the new key row: their loads go
    // out first (the norms need them first; no branch: absent rows read 0 without memory
    // access); rows past one per wave follow one by one.  A wave keeps under the 63 loads
    // the wait counter tracks, or issue stalls until the first ones return.
    const int g0 = wave;
    const bool own_k = owns_pos && wave == AW - 1;
    RowLd r0, rkr;
    constexpr int NQ = DPL / 4;   // hd = 16 DPL
    row_load<NQ>(r0, a.q + (size_t)(kh * G + min(g0, G - 1)) * 2 * hd, a.qn, a, g0 < G);
    row_load<NQ>(rkr, a.k + (size_t)kh * hd, a.kn, a, own_k);
    const int pl = lane >> 4, part = lane & 15;
    const uint32_t cache_b = (uint32_t)a.max_t * (uint32_t)hd * 4u;
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(a.Kc + (size_t)kh * a.max_t * hd, cache_b);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(a.Vc + (size_t)kh * a.max_t * hd, cache_b);
    float kv[kSteps][DPL];
#pragma unroll
    for (int st = 0; st < kSteps; st++) {
        const int t = t0 + (st * AW + wave) * 4 + pl;
        const bool ld = t < t1 && t != a.pos;
#pragma unroll
        for (int e = 0; e < DPL; e += 4) {
            const coli_v4i v4 = __builtin_amdgcn_raw_buffer_load_b128(
                rk, ld ? (t * hd + part * DPL + e) * 4 : (int)kOOB, 0, 0);
            kv[st][e] = __int_as_float(v4.x);
            kv[st][e + 1] = __int_as_float(v4.y);
            kv[st][e + 2] = __int_as_float(v4.z);
            kv[st][e + 3] = __int_as_float(v4.w);
        }
    }
    // V: the chunk's cached rows (this token's v for the position pos) as 16-byte loads,
    // written to LDS once the scores are done; P.V reads them from there
    constexpr int kV4 = kAttT * kAttMaxHD / 4 / kT;   // float4 slots per thread (kT % (hd / 4) == 0:
    const int hd4 = hd / 4;                             // a thread's dims are the same in every slot)
    const __amdgpu_buffer_rsrc_t rnv = buf_rsrc(a.v + (size_t)kh * hd, (uint32_t)hd * 4u);
    const int c4 = tid % hd4;
    const coli_v4i nv = __builtin_amdgcn_raw_buffer_load_b128(rnv, owns_pos ? 16 * c4 : (int)kOOB, 0, 0);
    float4 vq[kV4];
#pragma unroll
    for (int j = 0; j < kV4; j++) {
        if (j > 0 && j * kT >= kAttT * hd4) continue;   // uniform; a guarded body keeps the unroll
        const int t = (tid + j * kT) / hd4, tt = t0 + t;
        const int off = t < n && tt != a.pos ? (tt * hd + 4 * c4) * 4 : (int)kOOB;
        const coli_v4i c = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);   // pos: selected at the LDS write
        vq[j] = make_float4(__int_as_float(c.x), __int_as_float(c.y), __int_as_float(c.z), __int_as_float(c.w));
    }
    if (g0 < G) row_finish(s_q[g0], nullptr, r0, a);
    for (int gg = wave + AW; gg < G; gg += AW)
        norm_rope_row<NQ>(s_q[gg], nullptr, a.q + (size_t)(kh * G + gg) * 2 * hd, a.qn, a);
    if (own_k) {   // the new key row and value row (c/qwen.c:605-614)
        const size_t row = ((size_t)kh * a.max_t + a.pos) * hd;
        row_finish(s_k, a.Kc + row, rkr, a);
        for (int d = lane; d < hd; d += 64) a.Vc[row + d] = a.v[(size_t)kh * hd + d];
    }
    lds_barrier();
    // scores: 16 lanes per position, 4 positions per wave step; each q fragment is read
    // from LDS once for all the wave's steps
#pragma unroll
    for (int st = 0; st < kSteps; st++) {
        const int t = t0 + (st * AW + wave) * 4 + pl;
        if (t < t1 && t == a.pos)
#pragma unroll
            for (int e = 0; e < DPL; e++) kv[st][e] = s_k[part * DPL + e];
    }
    for (int gg = 0; gg < G; gg++) {
        float qf[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e += 4) {
            const float4 q4 = *(const float4 *)&s_q[gg][part * DPL + e];
            qf[e] = q4.x;
            qf[e + 1] = q4.y;
            qf[e + 2] = q4.z;
            qf[e + 3] = q4.w;
        }
#pragma unroll
        for (int st = 0; st < kSteps; st++) {
            const int t = t0 + (st * AW + wave) * 4 + pl;
            float sc = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; e++) sc = fmaf(qf[e], kv[st][e], sc);
            sc = seg_sum<16>(sc);
            if (part == 15 && t < t1) s_p[gg][t - t0] = sc * a.scale;
        }
    }
    lds_barrier();
    // chunk max and sum of exp per head: 32 lanes per head, lane = position; positions past
    // the chunk get p = 0
    static_assert(kAttT == 32, "one position per lane of a half wave");
    for (int gg = tid >> 5; gg < G; gg += kT / 32) {
        const int t = tid & 31;
        const float sc = t < n ? s_p[gg][t] : -INFINITY;
        float m = sc;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float pv = t < n ? expf(sc - m) : 0.f;
        float l = pv;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) l += __shfl_xor(l, o);
        s_p[gg][t] = pv;
        if (t == 0) {
            s_m[gg] = m;
            s_l[gg] = l;
        }
    }
#pragma unroll
    for (int j = 0; j < kV4; j++) {
        if (j > 0 && j * kT >= kAttT * hd4) continue;
        const int t = (tid + j * kT) / hd4;
        *(float4 *)&s_v[t][4 * c4] = t0 + t == a.pos ? make_float4(__int_as_float(nv.x), __int_as_float(nv.y),
                                                                     __int_as_float(nv.z), __int_as_float(nv.w))
                                                      : vq[j];
    }
    lds_barrier();
    // P.V: thread pvt of the head dims; with two halves, half h takes heads h G / 2 ..
    const int pvt = tid % kPV, half = tid / kPV;
    float *pb = a.part + ((size_t)kh * a.nsplit + sp) * G * (hd + 2);
    const int nh = kT > kPV ? (G + 1) / 2 : G, g_lo = half * nh, g_hi = min(G, g_lo + nh);
#pragma unroll
    for (int i = 0; i < kVPer; i++) {   // guarded bodies, no breaks: the loops unroll fully
        const int d = pvt + i * kPV;
        if (i * kPV >= hd) continue;   // uniform
        float vv[kAttT];
#pragma unroll
        for (int t = 0; t < kAttT; t++) vv[t] = d < hd ? s_v[t][d] : 0.f;
        for (int gg = g_lo; gg < g_hi; gg++) {   // p as float4 broadcasts, positions in order
            float acc = 0.f;
#pragma unroll
            for (int t4 = 0; t4 < kAttT; t4 += 4) {
                const float4 p = *(const float4 *)&s_p[gg][t4];
                acc = fmaf(p.x, vv[t4], acc);
                acc = fmaf(p.y, vv[t4 + 1], acc);
                acc = fmaf(p.z, vv[t4 + 2], acc);
                acc = fmaf(p.w, vv[t4 + 3], acc);
            }
            if (d < hd) pb[(size_t)gg * (hd + 2) + d] = acc;
        }
    }
    if (tid < G) {
        pb[(size_t)tid * (hd + 2) + hd] = s_m[tid];
        pb[(size_t)tid * (hd + 2) + hd + 1] = s_l[tid];
    }
}

constexpr int kAttMaxSplit = 4096;

// One block per query head: merges the chunks (max, rescaled sums) and applies the
// sigmoid gate.  kMW waves; wave w takes chunks w, w + kMW, ...; lane l takes dims
// 4 l .. 4 l + 3 (and + 256 for hd = 512); the wave partials are summed in LDS in wave order.
// Each chunk's (m, l) and the context rows of a wave's first kMPre chunks are loaded together
// (one memory round trip: the rows do not depend on the max), as branch-free buffer loads.
constexpr int kMW = 8, kMT = 64 * kMW, kMPre = 16;
__global__ __launch_bounds__(kMT) void attn_merge(AttnArgs a) {
    __shared__ float s_w[kAttMaxSplit];
    __shared__ float s_red[kMW];
    __shared__ __attribute__((aligned(16))) float s_acc[kMW][kAttMaxHD];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = blockIdx.x, G = a.H / a.KH, kh = h / G, gg = h % G, hd = a.hd;
    const int ns = (a.pos + 1 + kAttT - 1) / kAttT;
    const float *pb = a.part + ((size_t)kh * a.nsplit) * G * (hd + 2) + (size_t)gg * (hd + 2);
    const size_t stride = (size_t)G * (hd + 2);
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(pb, (uint32_t)(((size_t)(ns - 1) * stride + hd + 2) * 4));
    auto ldp = [&](size_t i, bool on) {   // float i of the partials (0 without memory access when !on)
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, on ? (int)(i * 4) : (int)kOOB, 0, 0));
    };
    // the gate row of the output, each chunk's (m, l) (ns <= kMT: one chunk per thread, kept
    // in registers for the weights) and the first kMPre chunk rows of the wave's first dims
    constexpr int kGPer = (kAttMaxHD + kMT - 1) / kMT;
    const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.q + (size_t)h * 2 * hd + hd, (uint32_t)hd * 4u);
    float gv[kGPer];
#pragma unroll
    for (int i = 0; i < kGPer; i++) {
        const int d = tid + i * kMT;
        gv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, d < hd ? d * 4 : (int)kOOB, 0, 0));
    }
    const bool one = ns <= kMT;
    const float mv = ldp((size_t)tid * stride + hd, one && tid < ns);
    const float lv = ldp((size_t)tid * stride + hd + 1, one && tid < ns);
    float4 pre[kMPre];
    {
        const int d0 = lane * 4;
#pragma unroll
        for (int u = 0; u < kMPre; u++) {
            const int s = wave + u * kMW;
            const bool on = s < ns && d0 < hd;
            const uint32_t o = on ? (uint32_t)(((size_t)s * stride + d0) * 4) : kOOB;
            const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rp, (int)o, 0, 0);
            pre[u] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
        }
    }
    float m = -INFINITY;
    if (one) {
        if (tid < ns) m = mv;
    } else {
        for (int s = tid; s < ns; s += kMT) m = fmaxf(m, pb[s * stride + hd]);
    }
    m = wave_max_f(m);
    if (lane == 0) s_red[wave] = m;
    lds_barrier();
    m = s_red[0];
    for (int w = 1; w < kMW; w++) m = fmaxf(m, s_red[w]);
    float l = 0.f;
    if (one) {
        if (tid < ns) {
            const float w = expf(mv - m);
            s_w[tid] = w;
            l = lv * w;
        }
    } else {
        for (int s = tid; s < ns; s += kMT) {
            const float w = expf(pb[s * stride + hd] - m);
            s_w[s] = w;
            l += pb[s * stride + hd + 1] * w;
        }
    }
    l = wave_sum_f(l);
    lds_barrier();
    if (lane == 0) s_red[wave] = l;
    lds_barrier();
    l = 0.f;
    for (int w = 0; w < kMW; w++) l += s_red[w];
    const float inv = 1.f / l;
    for (int d0 = lane * 4; d0 < hd; d0 += 256) {   // hd % 64 == 0: whole float4s
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        int s = wave;
        if (d0 == lane * 4) {   // the prefetched rows (uniform: the first dims pass)
#pragma unroll
            for (int u = 0; u < kMPre; u++, s += kMW) {
                const float w = s < ns ? s_w[s] : 0.f;
                acc.x = fmaf(pre[u].x, w, acc.x);
                acc.y = fmaf(pre[u].y, w, acc.y);
                acc.z = fmaf(pre[u].z, w, acc.z);
                acc.w = fmaf(pre[u].w, w, acc.w);
            }
        }
        for (; s + 15 * kMW < ns; s += 16 * kMW) {   // 16 chunks' loads in flight
            float4 v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = *(const float4 *)(pb + (size_t)(s + u * kMW) * stride + d0);
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const float w = s_w[s + u * kMW];
                acc.x = fmaf(v[u].x, w, acc.x);
                acc.y = fmaf(v[u].y, w, acc.y);
                acc.z = fmaf(v[u].z, w, acc.z);
                acc.w = fmaf(v[u].w, w, acc.w);
            }
        }
        for (; s < ns; s += kMW) {
            const float4 v = *(const float4 *)(pb + (size_t)s * stride + d0);
            const float w = s_w[s];
            acc.x = fmaf(v.x, w, acc.x);
            acc.y = fmaf(v.y, w, acc.y);
            acc.z = fmaf(v.z, w, acc.z);
            acc.w = fmaf(v.w, w, acc.w);
        }
        *(float4 *)&s_acc[wave][d0] = acc;
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < kGPer; i++) {
        const int d = tid + i * kMT;
        if (d < hd) {
            float acc = s_acc[0][d];
#pragma unroll
            for (int w = 1; w < kMW; w++) acc += s_acc[w][d];
            a.ctx[(size_t)h * hd + d] = acc * inv * (1.f / (1.f + expf(-gv[i])));
        }
    }
}

// The merge with a head's dims split over blocks (ns <= kMT chunks, hd % 64 == 0): block
// (h, q) takes dims 64 q .. 64 q + 63, so a head's partials are read by hd / 64 blocks
// (one block per head read ~130 KB at configs[3]).  Lane l holds dims 64 q + 4 (l % 16) ..
// + 3 of chunks (u kMW + wave) 4 + l / 16; those rows, each chunk's (m, l) (thread t: chunk
// t) and the gate go out in one round trip.  The chunk sums meet in LDS and are added in
// chunk order.
constexpr int kMDPre = kMT / (kMW * 4);   // chunk rows per lane
__global__ __launch_bounds__(kMT) void attn_merge_d(AttnArgs a) {
    __shared__ float s_w[kMT];
    __shared__ float s_red[kMW];
    __shared__ __attribute__((aligned(16))) float s_acc[kMT / 16][64];   // [chunk % 32][dim]
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hd = a.hd, nq = hd / 64, h = blockIdx.x / nq, q = blockIdx.x % nq;
    const int G = a.H / a.KH, kh = h / G, gg = h % G;
    const int ns = (a.pos + 1 + kAttT - 1) / kAttT;
    const float *pb = a.part + ((size_t)kh * a.nsplit) * G * (hd + 2) + (size_t)gg * (hd + 2);
    const size_t stride = (size_t)G * (hd + 2);
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(pb, (uint32_t)(((size_t)(ns - 1) * stride + hd + 2) * 4));
    auto ldp = [&](size_t i, bool on) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, on ? (int)(i * 4) : (int)kOOB, 0, 0));
    };
    const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.q + (size_t)h * 2 * hd + hd, (uint32_t)hd * 4u);
    const float gv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, tid < 64 ? (64 * q + tid) * 4 : (int)kOOB, 0, 0));
    const float mv = ldp((size_t)tid * stride + hd, tid < ns);
    const float lv = ldp((size_t)tid * stride + hd + 1, tid < ns);
    const int dq = lane & 15, cs = lane >> 4, d0 = 64 * q + 4 * dq;
    float4 pre[kMDPre];
#pragma unroll
    for (int u = 0; u < kMDPre; u++) {
        const int sc = (u * kMW + wave) * 4 + cs;
        const uint32_t o = sc < ns ? (uint32_t)(((size_t)sc * stride + d0) * 4) : kOOB;
        const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rp, (int)o, 0, 0);
        pre[u] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
    }
    float m = tid < ns ? mv : -INFINITY;
    m = wave_max_f(m);
    if (lane == 0) s_red[wave] = m;
    lds_barrier();
    m = s_red[0];
    for (int w = 1; w < kMW; w++) m = fmaxf(m, s_red[w]);
    const float wgt = tid < ns ? expf(mv - m) : 0.f;
    s_w[tid] = wgt;
    float l = wave_sum_f(tid < ns ? lv * wgt : 0.f);
    lds_barrier();
    if (lane == 0) s_red[wave] = l;
    lds_barrier();
    l = 0.f;
    for (int w = 0; w < kMW; w++) l += s_red[w];
    const float inv = 1.f / l;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < kMDPre; u++) {
        const int sc = (u * kMW + wave) * 4 + cs;
        const float w = sc < ns ? s_w[sc] : 0.f;
        acc.x = fmaf(pre[u].x, w, acc.x);
        acc.y = fmaf(pre[u].y, w, acc.y);
        acc.z = fmaf(pre[u].z, w, acc.z);
        acc.w = fmaf(pre[u].w, w, acc.w);
    }
    *(float4 *)&s_acc[wave * 4 + cs][4 * dq] = acc;
    lds_barrier();
    if (tid < 64) {
        float t = 0.f;
        for (int r = 0; r < kMT / 16; r++) t += s_acc[r][tid];
        a.ctx[(size_t)h * hd + 64 * q + tid] = t * inv * (1.f / (1.f + expf(-gv)));
    }
}

// ---------------------------------------------------------------- GQA over S query rows
// The block over S > 1 rows at positions pos_base .. pos_base + S - 1, causal (the prompt, or
// a continuation chunk; c/qwen.c:581-667 restated, batched as c/backend_vulkan.c:2280-2340):
// projections as GEMMs, qk_rows for the norms, RoPE and KV writes of all rows, attn_rows for
// the attention and its output gate, then the o-projection GEMM.

// q/k norm + partial RoPE of one head row of token s (c/qwen.c:598-614, the arithmetic of
// row_finish), block (s, j) of one wave: j < H is q head j into qn [S][H][hd]; j >= H is k
// head j - H into the cache row pos_base + s, with its v row.  rope [S][rot / 2] holds the
// (cos, sin) of each position, computed on the host as for the decode block.
__global__ __launch_bounds__(64) void qk_rows(const float *__restrict__ qraw, const float *__restrict__ kraw,
                                              const float *__restrict__ vraw, const float *__restrict__ qnw,
                                              const float *__restrict__ knw, const float2 *__restrict__ rope,
                                              float *__restrict__ qn, float *__restrict__ Kc, float *__restrict__ Vc,
                                              int H, int KH, int hd, int rot, int pos_base, int max_t, float eps) {
    __shared__ float s_row[kAttMaxHD];
    const int s = blockIdx.x, j = blockIdx.y, lane = threadIdx.x, hr = rot / 2;
    const bool isq = j < H;
    const int kh = j - H;
    const float *src = isq ? qraw + ((size_t)s * H + j) * 2 * hd : kraw + ((size_t)s * KH + kh) * hd;
    const float *w = isq ? qnw : knw;
    float *dst = isq ? qn + ((size_t)s * H + j) * hd : Kc + ((size_t)kh * max_t + pos_base + s) * hd;
    constexpr int kPer = kAttMaxHD / 64;
    float v[kPer];
    double ss = 0;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int d = lane + 64 * q;
        v[q] = d < hd ? src[d] : 0.f;
        ss += (double)v[q] * v[q];
    }
    ss = wave_sum_d(ss);
    const float r = 1.f / sqrtf((float)(ss / hd) + eps);
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int d = lane + 64 * q;
        if (d < hd) s_row[d] = v[q] * r * (1.f + w[d]);
    }
    __syncthreads();
    const float2 *cs = rope + (size_t)s * hr;
    for (int d = lane; d < hd; d += 64) {
        float o = s_row[d];
        if (d < hr) {
            const float2 c = cs[d];
            o = s_row[d] * c.x - s_row[d + hr] * c.y;
        } else if (d < rot) {
            const float2 c = cs[d - hr];
            o = s_row[d] * c.x + s_row[d - hr] * c.y;
        }
        dst[d] = o;
    }
    if (!isq) {
        const float *vs = vraw + ((size_t)s * KH + kh) * hd;
        float *vd = Vc + ((size_t)kh * max_t + pos_base + s) * hd;
        for (int d = lane; d < hd; d += 64) vd[d] = vs[d];
    }
}

// Causal attention of 16 query rows of one head on fp32 MFMA (v_mfma_f32_16x16x4_f32), one
// block of 4 waves per (head, 16-row query tile); wave w takes the key tiles w, w + 4, ...
// of 16 positions and keeps its own running max, sum and context; the block merges the
// four in wave order and applies the output gate (c/qwen.c:641-660).
//   scores^T = K Q^T: A = 16 keys x 4 dims, B = 4 dims x 16 queries; lane l, register r of
//     the product is (key 4 (l / 16) + r, query l % 16).  The K dimension is permuted: step
//     kk of lane group g = l / 16 is dim (hd / 4) g + kk, so each lane holds a contiguous
//     quarter of its query row (registers) and reads a contiguous quarter of its key row.
//   ctx^T += V^T P^T: A = 16 dims x 4 keys (V tile from LDS), B = the lane's own 4 scores
//     (step kk of group g is key 4 g + kk); lane l, register r of dim tile t is
//     (dim 16 t + 4 (l / 16) + r, query l % 16).  Every per-query value (max, sum, rescale)
//     stays in the lanes of its query.
constexpr int kPQ = 16, kPKey = 16;
struct AttnRowsArgs {
    const float *qraw;    // [S][H][2 hd]: q | gate per head
    const float *qn;      // [S][H][hd] normed, rotated
    const float *Kc, *Vc; // [KH][max_t][hd]
    float *ctx;           // [S][H hd] gated context
    int S, H, KH, pos_base, max_t, nqt;
    float scale;
};
template <int HD>
__global__ __launch_bounds__(256) void attn_rows(AttnRowsArgs a) {
    constexpr int NK = HD / 4, NDT = HD / 16, kVP = HD + 4;   // LDS pitch of a V row
    __shared__ __attribute__((aligned(16))) float s_v[4][kPKey][kVP];
    __shared__ float s_m[4][kPQ], s_l[4][kPQ];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = blockIdx.x % a.H, qt = a.nqt - 1 - blockIdx.x / a.H;   // the longest tiles first
    const int G = a.H / a.KH, kh = h / G, qi = lane & 15, grp = lane >> 4;
    const int s0 = qt * kPQ, sq = min(s0 + qi, a.S - 1), qpos = a.pos_base + sq;
    const int last = a.pos_base + min(s0 + kPQ, a.S) - 1, nkt = last / kPKey + 1;
    float qf[NK];
    {
        const float4 *qp = (const float4 *)(a.qn + ((size_t)sq * a.H + h) * HD + NK * grp);
#pragma unroll
        for (int i = 0; i < NK / 4; i++) {
            const float4 v = qp[i];
            qf[4 * i] = v.x, qf[4 * i + 1] = v.y, qf[4 * i + 2] = v.z, qf[4 * i + 3] = v.w;
        }
    }
    coli_v4f acc[NDT];
#pragma unroll
    for (int t = 0; t < NDT; t++) acc[t] = coli_v4f{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    const float *Kh = a.Kc + (size_t)kh * a.max_t * HD, *Vh = a.Vc + (size_t)kh * a.max_t * HD;
    constexpr int kV4 = kPKey * HD / 4 / 64;   // float4 of the V tile per lane
    for (int kt = wave; kt < nkt; kt += 4) {
        const int t0 = kt * kPKey;
        // key rows past the tile's last query position are masked; their loads stay inside
        // the rows written so far (K clamped, V read as zeros: 0 * stale data is not 0)
        float kf[NK];
        const float4 *kp = (const float4 *)(Kh + (size_t)min(t0 + qi, last) * HD + NK * grp);
#pragma unroll
        for (int i = 0; i < NK / 4; i++) {
            const float4 v = kp[i];
            kf[4 * i] = v.x, kf[4 * i + 1] = v.y, kf[4 * i + 2] = v.z, kf[4 * i + 3] = v.w;
        }
        float4 vt[kV4];
#pragma unroll
        for (int i = 0; i < kV4; i++) {
            const int f = lane + 64 * i, key = f / (HD / 4), c4 = f % (HD / 4);
            vt[i] = t0 + key <= last ? *(const float4 *)(Vh + (size_t)(t0 + key) * HD + 4 * c4)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        coli_v4f sc = coli_v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; kk++) sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kk], qf[kk], sc, 0, 0, 0);
        wave_lds_order();   // the previous tile's P.V reads of s_v come before these writes
#pragma unroll
        for (int i = 0; i < kV4; i++) {
            const int f = lane + 64 * i, key = f / (HD / 4), c4 = f % (HD / 4);
            *(float4 *)&s_v[wave][key][4 * c4] = vt[i];
        }
        // scale, causal mask, online softmax of the lane's query over the tile's 16 keys
        float p[4], mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int kpos = t0 + 4 * grp + r;
            p[r] = kpos <= qpos ? sc[r] * a.scale : -INFINITY;
            mx = fmaxf(mx, p[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const bool live = mn != -INFINITY;   // some key of the query seen so far
        const float al = live && m != -INFINITY ? expf(m - mn) : (live ? 0.f : 1.f);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            p[r] = live && p[r] != -INFINITY ? expf(p[r] - mn) : 0.f;
            ps += p[r];
        }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l = l * al + ps;
        m = mn;
#pragma unroll
        for (int t = 0; t < NDT; t++) acc[t] *= al;
        wave_lds_order();   // the V tile is in LDS before the P.V reads (one wave: in order)
#pragma unroll
        for (int t = 0; t < NDT; t++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(s_v[wave][4 * grp + kk][16 * t + qi], p[kk], acc[t], 0,
                                                              0, 0);
    }
    // merge the four waves (wave order), gate, store
    if (grp == 0) {
        s_m[wave][qi] = m;
        s_l[wave][qi] = l;
    }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; w++) M = fmaxf(M, s_m[w][qi]);
    const float fw = m == -INFINITY ? 0.f : expf(m - M);
    float (*s_c)[kPQ][HD] = (float (*)[kPQ][HD])&s_v[0][0][0];   // [4][16][HD] over the V tiles
    static_assert(sizeof(s_v) >= 4 * kPQ * HD * 4, "context staging fits the V tiles");
    __syncthreads();   // every wave is done with its V tile
#pragma unroll
    for (int t = 0; t < NDT; t++)
        *(float4 *)&s_c[wave][qi][16 * t + 4 * grp] =
            make_float4(acc[t][0] * fw, acc[t][1] * fw, acc[t][2] * fw, acc[t][3] * fw);
    __syncthreads();
    for (int o = tid; o < kPQ * HD; o += 256) {
        const int q = o / HD, d = o % HD, s = s0 + q;
        if (s >= a.S) continue;
        float L = 0.f, Mq = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) Mq = fmaxf(Mq, s_m[w][q]);
#pragma unroll
        for (int w = 0; w < 4; w++) L += s_m[w][q] == -INFINITY ? 0.f : s_l[w][q] * expf(s_m[w][q] - Mq);
        float c = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) c += s_c[w][q][d];
        const float gate = a.qraw[((size_t)s * a.H + h) * 2 * HD + HD + d];
        a.ctx[(size_t)s * a.H * HD + (size_t)h * HD + d] = c / L * (1.f / (1.f + expf(-gate)));
    }
}

// ---------------------------------------------------------------- small kernels
__global__ void rms_rows(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ y, int D,
                         float eps) {
    __shared__ double s_red[kWaves];
    double ss = 0;
    for (int i = threadIdx.x; i < D; i += kThreads) ss += (double)x[i] * x[i];
    ss = block_sum_d(ss, s_red);
    const float r = 1.f / sqrtf((float)(ss / D) + eps);
    for (int i = threadIdx.x; i < D; i += kThreads) y[i] = x[i] * r * (1.f + w[i]);
}

// Router logits of the route tail, one row per wave: lg[e] = the exact dot x . router row e
// rounded to fp32 (times the int8 row scale), bd[e] = its bound against the reference's
// sequential fp32 sum (router_row, c/qwen.c:178-189 / 230-238).  fmt 0 or 1 rows.
__global__ __launch_bounds__(kThreads) void router_lb(const float *__restrict__ x, const uint8_t *__restrict__ rw,
                                                      const float *__restrict__ rs, int rfmt, int rrb, int E, int D,
                                                      float *__restrict__ lg, float *__restrict__ bd) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= E) return;   // wave uniform
    const bool int8 = rfmt == 1;
    const __amdgpu_buffer_rsrc_t rr = buf_rsrc(rw + (size_t)r * rrb, int8 ? (uint32_t)D : (uint32_t)D * 4u);
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint32_t)D * 4u);
    float4 w[kRouterRC];
    auto load_row = [&](int c0, float4 (&wv)[kRouterRC]) {
#pragma unroll
        for (int c = 0; c < kRouterRC; c++) {
            const int col = c0 + (lane + c * 64) * 4;
            if (!int8) {
                const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rr, col * 4, 0, kStream);
                wv[c] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
            } else {
                const uint32_t q = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rr, col, 0, kStream);
                wv[c] = make_float4((float)(int8_t)q, (float)(int8_t)(q >> 8), (float)(int8_t)(q >> 16),
                                    (float)(int8_t)(q >> 24));
            }
        }
    };
    auto load_x = [&](int c0, float4 (&xq)[kRouterRC]) {
#pragma unroll
        for (int c = 0; c < kRouterRC; c++) {
            const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rx, (c0 + (lane + c * 64) * 4) * 4, 0, kCached);
            xq[c] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
        }
    };
    const float scale = int8 ? rs[r] : 1.f;
    const float B = router_row(D, scale, int8, w, false, load_row, load_x, [&](float L, float) {
        if (lane == 0) lg[r] = L;
    });
    if (lane == 0) bd[r] = B;
}

// softmax + K greedy picks + renorm of one router row (device top-k of the route tail),
// certified against the reference's sequential logits (route_certify); x = the router input.
__global__ __launch_bounds__(64) void route_row(const float *__restrict__ lb, const float *__restrict__ x,
                                                const uint8_t *__restrict__ rw, const float *__restrict__ rs,
                                                int rfmt, int rrb, int D, int E, int K, int *idx, float *val,
                                                int cert_all) {
    __shared__ RouteLds R;
    __shared__ CertLds C;
    for (int e = threadIdx.x; e < E; e += 64) {
        R.p[e] = lb[e];
        C.l[e] = lb[e];
        C.b[e] = lb[E + e];
    }
    wave_lds_order();
    route_wave(R, E, K, C.l, C.b);
    if (cert_all) {   // test hook: every candidate gets its reference logit
        if (threadIdx.x == 0) {
            R.amb = 1;
            R.thr = -INFINITY;
        }
        wave_lds_order();
    }
    route_certify_wave(
        R, C, K, D, rfmt == 1, rs, rw, rrb, E, [&](float *xn) { stage_input_wave(x, nullptr, D, 0.f, xn); });
    if (threadIdx.x < K) {
        idx[threadIdx.x] = R.idx[threadIdx.x];
        val[threadIdx.x] = R.val[threadIdx.x] / R.vsum;
    }
}

// ================================================================ host side
constexpr int kMaxLayers = 160;   // c/backend_vulkan.c:63 (VK_KV_LAYERS)

struct KvState {             // device KV mirror: row = kv_head * max_t + pos
    float *K = nullptr, *V = nullptr;
    int rows = 0, kd = 0, vd = 0, cap_rows = 0;
};
struct QkNorm {
    float *qn = nullptr, *kn = nullptr;
    int hd = 0;
};
struct GdnState {
    float *S = nullptr;      // [VH][VD][KD] (transposed from the reference's [VH][KD][VD])
    int VH = 0, KD = 0, VD = 0;
    float *ring = nullptr;   // [K][CD] circular (see GdnArgs)
    int head = 0;
    float *convw = nullptr;  // [CD][K]
    int K = 0, CD = 0, convw_set = 0;
    float *alog = nullptr, *dtb = nullptr, *gnorm = nullptr;
    int ba_VH = 0, ba_VD = 0;
};
struct LnState {
    float *in_ln = nullptr, *post_ln = nullptr;
    int D = 0;
};
static KvState g_kv[kMaxLayers];
static QkNorm g_qk[kMaxLayers];
static GdnState g_gdn[kMaxLayers];
static LnState g_ln[kMaxLayers];

// one-shot failures of the layer blocks: one stderr line per reason
static bool refuse(const char *why) {
    static const char *last = nullptr;
    if (why != last) fprintf(stderr, "[HIP] layer block refused: %s\n", why);
    last = why;
    return false;
}

static bool h2d(void *d, const void *h, size_t bytes, const char *who) {
    if (!bytes) return true;
    const hipError_t e = hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail(who, e);
    return sync_stream(who);
}

// arena copy of a host vector (re-uploaded in place when the size matches)
static bool put_vec(float **d, int *have, const float *h, int n, const char *who) {
    if (!h || n < 1) return false;
    if (!*d || *have != n) {
        float *p = (float *)arena_alloc((size_t)n * 4);
        if (!p) return false;
        *d = p;
        *have = n;
    }
    return h2d(*d, h, (size_t)n * 4, who);
}

// ---------------------------------------------------------------- work buffers
enum {
    W_Q, W_K, W_V, W_CTX, W_PART, W_QKV, W_Z, W_Y, W_AB, W_NRM, W_LOGIT, W_IDX, W_IO_X, W_IO_R, W_IO_P, W_IO_O,
    W_HIST, W_BND, W_SQKV, W_SZ, W_SY, W_ROPE, W_GQN, W_GKN, W_GVV, W_GMAT, W_COUNT
};
struct WorkBuf {
    void *p = nullptr;
    size_t cap = 0;
};
static WorkBuf g_w[W_COUNT];
static float *wbuf(int slot, size_t n) {
    return scratch(&g_w[slot].p, &g_w[slot].cap, n * 4 + 256) ? (float *)g_w[slot].p : nullptr;
}

// ---------------------------------------------------------------- projection launch
struct SegIn {
    const ColiVkTensor *t;
    float *y;
    int act;   // the segment stores silu(row)
};

// Row steps per wave, all loaded before the first is reduced: the smallest of 2..8 that
// covers the rows with up to kProjBPC blocks per CU (the kernel's occupancy holds 4-5
// waves per SIMD).  A launch is latency-bound, and more waves in flight per CU beat fewer
// waves with more steps each (decode step 1.73 against 1.77 ms per token with one block
// per CU, 1.75 with one step per wave).  Larger projections take 8 and loop.
constexpr int kProjBPC = 4;
static int proj_u(int ngroups) {
    const long per_step = (long)kWaves * n_cu() * kProjBPC;
    const long need = (ngroups + per_step - 1) / per_step;
    return need <= 2 ? 2 : need <= 3 ? 3 : need <= 4 ? 4 : need <= 5 ? 5 : need <= 6 ? 6 : need <= 7 ? 7 : 8;
}

template <int LPR, int CU, int U, int XF>
static bool launch_proj_u(ProjArgs &a, hipStream_t st) {
    auto kern = proj_gemv<LPR, CU, U, XF>;
    long nb = ((long)a.ngroups + kWaves * U - 1) / (kWaves * U);
    if (nb > (long)kProjBPC * n_cu()) nb = (long)kProjBPC * n_cu();
    // Blocks past a whole number per CU (up to a quarter of the CUs) share a CU with the
    // others and end last (measured: the GatedDeltaNet in-projection's 4 blocks past 768
    // ended ~1 us after the rest); without them, some waves take one more row step, whose
    // loads are prefetched.
    const long ncu = n_cu();
    if (nb > ncu && nb % ncu <= ncu / 4) nb -= nb % ncu;
    if (nb < 1) nb = 1;
    hipLaunchKernelGGL(kern, dim3((unsigned)nb), dim3(kThreads), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("projection launch", e);
    return true;
}

template <int LPR, int CU, int XF>
static bool launch_proj(ProjArgs &a, hipStream_t st) {
    switch (proj_u(a.ngroups)) {
    case 2: return launch_proj_u<LPR, CU, 2, XF>(a, st);
    case 3: return launch_proj_u<LPR, CU, 3, XF>(a, st);
    case 4: return launch_proj_u<LPR, CU, 4, XF>(a, st);
    case 5: return launch_proj_u<LPR, CU, 5, XF>(a, st);
    case 6: return launch_proj_u<LPR, CU, 6, XF>(a, st);
    case 7: return launch_proj_u<LPR, CU, 7, XF>(a, st);
    default: return launch_proj_u<LPR, CU, 8, XF>(a, st);
    }
}

template <int CU, int XF>
static bool proj_lpr(ProjArgs &a, int lpr, hipStream_t st) {
    switch (lpr) {
    case 2: return launch_proj<2, CU, XF>(a, st);
    case 4: return launch_proj<4, CU, XF>(a, st);
    case 8: return launch_proj<8, CU, XF>(a, st);
    case 16: return launch_proj<16, CU, XF>(a, st);
    case 32: return launch_proj<32, CU, XF>(a, st);
    case 64: return launch_proj<64, CU, XF>(a, st);
    default: return refuse("projection row too short for the lanes kernel");
    }
}

static int pow2_up(int n) {
    int l = 1;
    while (l < n) l <<= 1;
    return l;
}

// The arguments of a projection over the segments (same I, gs: they share the input row
// x' = XF(x)); *lpr the lanes per row.  False (with a message) for shapes it cannot run.
static bool proj_args(const SegIn *segs, int n, int xf, const float *x, const float *xw, const float *z, int VD,
                      float eps, bool add, ProjArgs &a, int *lpr) {
    if (n < 1 || n > kMaxSeg) return refuse("projection segment count");
    const ColiVkTensor *t0 = segs[0].t;
    for (int i = 0; i < n; i++) {
        const ColiVkTensor *t = segs[i].t;
        if (!tensor_live(t) || !segs[i].y) return refuse("NULL or stale projection tensor");
        if (t->fmt != 6 || t->layout != kLayoutLanes) return refuse("projection is not fmt 6 (gs % 32 == 0, I <= 4096)");
        if (t->I != t0->I || t->gs != t0->gs || t->nl != t0->nl || t->row_bytes != t0->row_bytes)
            return refuse("fused projections differ in input geometry");
    }
    memset(&a, 0, sizeof(a));
    const int l = pow2_up(t0->nl), rpw = 64 / (l < 2 ? 2 : l);
    int g = 0;
    for (int i = 0; i < n; i++) {
        a.seg[i] = {segs[i].t->w, segs[i].t->sz, segs[i].y, segs[i].t->O, g, nullptr, segs[i].act};
        g += (segs[i].t->O + rpw - 1) / rpw;
    }
    a.nseg = n;
    a.ngroups = g;
    a.I = t0->I;
    a.gs = t0->gs;
    a.ng = t0->ng;
    a.nl = t0->nl;
    a.row_bytes = t0->row_bytes;
    a.x = x;
    a.xw = xw;
    a.z = z;
    a.VD = VD;
    a.eps = eps;
    a.add = add ? 1 : 0;
    if (xf == XF_GATED) {
        const int wph = VD / 8;
        if (VD % 8 || wph < 1 || wph > 64 || (wph & (wph - 1)) || a.I % VD) return refuse("gated norm head size");
    }
    *lpr = l < 2 ? 2 : l;
    return true;
}

// y_s = W_s x' for the segments (same I, gs: they share the input row x' = XF(x)).
static bool proj(const SegIn *segs, int n, int xf, const float *x, const float *xw, const float *z, int VD, float eps,
                 bool add, hipStream_t st) {
    ProjArgs a;
    int l;
    if (!proj_args(segs, n, xf, x, xw, z, VD, eps, add, a, &l)) return false;
    const bool wide = segs[0].t->gs % (32 * kLaneChunks) == 0;   // a unit of kLaneChunks chunks lies in one group
    switch (xf) {
    case XF_PLAIN: return wide ? proj_lpr<kLaneChunks, XF_PLAIN>(a, l, st) : proj_lpr<1, XF_PLAIN>(a, l, st);
    case XF_NORM: return wide ? proj_lpr<kLaneChunks, XF_NORM>(a, l, st) : proj_lpr<1, XF_NORM>(a, l, st);
    default: return wide ? proj_lpr<kLaneChunks, XF_GATED>(a, l, st) : proj_lpr<1, XF_GATED>(a, l, st);
    }
}

// ---------------------------------------------------------------- fused GatedDeltaNet layer
// One launch for in-projection -> recurrence -> out-projection of a decode token (the
// reference records the same chain in one command buffer, c/backend_vulkan.c:1905-2017):
// tiles [0, n1) the in-projection (qkv | z | a | b, in_ln of the residual in the x
// prologue), [n1, n1 + nc) the recurrence blocks of gdn_core, then the out-projection
// (gated norm prologue, residual add).  Each stage's outputs are tagged words (epoch << 32 |
// bits) in one buffer, qkv | z | a,b | y | done, which the later tiles poll (the
// out-projection first one done word per recurrence block, by one wave, so that its many
// loads of y and z go out once); every wait is on tiles
// of lower index, so with workgroups dispatched in index order every wait ends.  The
// out-projection tiles issue their weight loads before they wait.  The residual the
// in-projection reads is rewritten only by out-projection tiles, which run after every
// in-projection tile has published (their prologues read it first).
constexpr int kFuseU = 8;    // row steps per wave of the fused in-projection
constexpr int kFuseU3 = 2;   // of the fused out-projection (short rows of work per tile after its wait)
struct GdnFusedArgs {
    ProjArgs p1, p3;
    GdnArgs g;
    int n1, nc;
};
template <int LPR1, int LPR3, int KPL>
__global__ __launch_bounds__(kThreads) void gdn_fused(GdnFusedArgs f) {
    __shared__ XPrep P;
    const int t = blockIdx.x;
    if (t < f.n1) proj_body<LPR1, kLaneChunks, kFuseU, XF_NORM, false, true>(f.p1, t, f.n1, P);
    else if (t < f.n1 + f.nc) gdn_core_body<KPL, true>(f.g, t - f.n1);
    else proj_body<LPR3, kLaneChunks, kFuseU3, XF_GATED, true, false>(f.p3, t - f.n1 - f.nc, (int)gridDim.x - f.n1 - f.nc, P);
}

// ---------------------------------------------------------------- GQA block
struct GqaDims {
    int H, KH, hd, rot, max_t;
    float eps, theta;
};

// One token at position pos.  ln != NULL: the input is the residual and the block applies
// in_ln itself; otherwise src is the normed row.  add: dst += block, else dst = block.
static bool gqa_block(int kvi, const float *src, const float *ln, ColiVkTensor *tq, ColiVkTensor *tk, ColiVkTensor *tv,
                      ColiVkTensor *to, float *dst, bool add, const GqaDims &d, int pos, hipStream_t st) {
    if (kvi < 0 || kvi >= kMaxLayers) return refuse("attention layer index");
    const KvState &kv = g_kv[kvi];
    const QkNorm &qk = g_qk[kvi];
    const int H = d.H, KH = d.KH, hd = d.hd;
    if (!kv.K || kv.kd != hd || kv.vd != hd || (long)KH * d.max_t > kv.rows) return refuse("KV mirror not ensured");
    if (!qk.qn || qk.hd != hd) return refuse("q/k norm weights not set");
    if (H < 1 || KH < 1 || H % KH || H / KH > kAttMaxG || hd % 64 || hd > kAttMaxHD || d.rot < 2 || d.rot > hd ||
        d.rot % 2 || d.rot / 2 > kAttMaxHR || pos < 0 || pos >= d.max_t)
        return refuse("attention shape");
    if (!tq || !tk || !tv || !to || tq->O != 2 * H * hd || tk->O != KH * hd || tv->O != KH * hd || to->I != H * hd)
        return refuse("attention projection shapes");
    const int nsplit = (pos + 1 + kAttT - 1) / kAttT, G = H / KH;
    if (nsplit > kAttMaxSplit) return refuse("attention window");
    float *q = wbuf(W_Q, (size_t)2 * H * hd), *k = wbuf(W_K, (size_t)KH * hd), *v = wbuf(W_V, (size_t)KH * hd);
    float *ctx = wbuf(W_CTX, (size_t)H * hd), *part = wbuf(W_PART, (size_t)KH * nsplit * G * (hd + 2));
    if (!q || !k || !v || !ctx || !part) return false;
    const SegIn in[3] = {{tq, q}, {tk, k}, {tv, v}};
    if (!proj(in, 3, ln ? XF_NORM : XF_PLAIN, src, ln, nullptr, 0, d.eps, false, st))
        return false;
    AttnArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.qn = qk.qn;
    a.kn = qk.kn;
    a.Kc = kv.K;
    a.Vc = kv.V;
    a.part = part;
    a.ctx = ctx;
    a.H = H;
    a.KH = KH;
    a.hd = hd;
    a.rot = d.rot;
    a.pos = pos;
    a.max_t = d.max_t;
    a.nsplit = nsplit;
    a.eps = d.eps;
    a.scale = 1.f / sqrtf((float)hd);
    for (int j = 0; j < d.rot / 2; j++) {   // c/qwen.c:572-574, in double, rounded to float
        const float inv = (float)pow((double)d.theta, (double)(-2.0f * j / d.rot));
        const float ang = (float)pos * inv;
        a.cs[j] = (float)cos((double)ang);
        a.sn[j] = (float)sin((double)ang);
    }
    switch (hd / 16) {
    case 4: hipLaunchKernelGGL((attn_part<4, kAttW>), dim3(KH * nsplit), dim3(64 * kAttW), 0, st, a); break;
    case 8: hipLaunchKernelGGL((attn_part<8, kAttW>), dim3(KH * nsplit), dim3(64 * kAttW), 0, st, a); break;
    case 16: hipLaunchKernelGGL((attn_part<16, kAttW>), dim3(KH * nsplit), dim3(64 * kAttW), 0, st, a); break;
    case 32: hipLaunchKernelGGL((attn_part<32, kAttW>), dim3(KH * nsplit), dim3(64 * kAttW), 0, st, a); break;
    default: return refuse("head dim not in {64, 128, 256, 512}");
    }
    if ((pos + kAttT) / kAttT <= kMT && hd % 64 == 0)   // ns chunks: one per thread
        hipLaunchKernelGGL(attn_merge_d, dim3(H * (hd / 64)), dim3(kMT), 0, st, a);
    else
        hipLaunchKernelGGL(attn_merge, dim3(H), dim3(kMT), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("attention launch", e);
    const SegIn o[1] = {{to, dst}};
    return proj(o, 1, XF_PLAIN, ctx, nullptr, nullptr, 0, d.eps, add, st);
}

// ---------------------------------------------------------------- GDN block
struct GdnDims {
    int KH, KD, VH, VD, CD, K;
    float eps;
};

static RowMat rowmat(const ColiVkTensor *t) {
    RowMat m;
    m.w = t->w;
    m.sz = t->sz;
    m.fmt = t->fmt;
    m.layout = t->layout;
    m.I = t->I;
    m.gs = t->gs;
    m.ng = t->ng;
    m.nl = t->nl;
    m.row_bytes = t->row_bytes;
    return m;
}

// One token.  params != NULL: host-packed [decay | beta | gnorm] (device copy); otherwise
// decay/beta from the a/b projections of in_ln(resid) and the layer's A_log/dt_bias/gnorm.
// ---------------------------------------------------------------- fused layer launches
// Tag buffer of the fused layer kernels (words qkv | z | a,b | y of one launch) and their
// error word: (epoch << 32) | code, code 1 when a bounded wait gave up.
struct LayerTags {
    void *tag = nullptr, *err = nullptr;
    size_t cap = 0, ecap = 0;
    uint32_t epoch = 0;
    uint64_t launches = 0;   // fused launches (they can set the error word)
};
static LayerTags g_lt;
// Off by default: on MI355X the one-launch layer measures slower than the three launches
// (about 24.5 us against 21 us per configs[3] layer; the out-projection tiles see their
// inputs some 6 us after the last recurrence tile ends).  COLI_HIP_FUSE=1 turns it on.
static int g_fuse = -1;   // -1: not read yet
static bool fuse_on() {
    if (g_fuse < 0) {
        const char *v = getenv("COLI_HIP_FUSE");
        g_fuse = v && *v == '1' ? 1 : 0;
    }
    return g_fuse == 1;
}

__global__ void zero_words(unsigned long long *w, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) w[i] = 0ull;
}

// The shapes the fused kernel is instantiated for: the configs[3] GatedDeltaNet layer
// (in-projection rows of 2048 columns, out-projection rows of 4096, key heads of 128, conv
// taps <= kGdnMaxK, group size a multiple of 64).  Other shapes take the three launches.
static bool gdn_fusable(const ColiVkTensor *tqkv, const ColiVkTensor *tout, const GdnDims &d) {
    return tout && tout->fmt == 6 && tout->layout == kLayoutLanes && tqkv->gs % (32 * kLaneChunks) == 0 &&
           tout->gs % (32 * kLaneChunks) == 0 && pow2_up(tqkv->nl) == 32 && pow2_up(tout->nl) == 64 && d.KD == 128 &&
           d.K <= kGdnMaxK;
}

static bool gdn_fused_launch(GdnState &G, const float *src, const float *ln, ColiVkTensor *tqkv, ColiVkTensor *tz,
                             ColiVkTensor *ta, ColiVkTensor *tb, ColiVkTensor *tout, float *dst, bool add, const GdnDims &d,
                             hipStream_t st) {
    const int VV = d.VH * d.VD;
    const size_t nwords = (size_t)d.CD + VV + 2 * d.VH + VV + (size_t)d.VH * (d.VD / kGdnCols);
    if (!scratch(&g_lt.tag, &g_lt.cap, nwords * 8) || !scratch(&g_lt.err, &g_lt.ecap, 256)) return false;
    unsigned long long *tags = (unsigned long long *)g_lt.tag, *err = (unsigned long long *)g_lt.err;
    unsigned long long *t_qkv = tags, *t_z = t_qkv + d.CD, *t_ab = t_z + VV, *t_y = t_ab + 2 * d.VH, *t_done = t_y + VV;
    if (++g_lt.epoch == 0) {   // tags wrap: no old word may carry the new epoch
        hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, st, tags, g_lt.cap / 8);
        hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, err, (size_t)1);
        g_lt.epoch = 1;
    }
    const uint32_t ep = g_lt.epoch;
    g_lt.launches++;
    GdnFusedArgs f;
    memset(&f, 0, sizeof(f));
    int l1, l3;
    float *placeholder = (float *)tags;   // proj_args checks a destination; the tagged words replace it
    const SegIn in[4] = {{tqkv, placeholder}, {tz, placeholder, 1}, {ta, placeholder}, {tb, placeholder}};
    if (!proj_args(in, 4, XF_NORM, src, ln, nullptr, 0, d.eps, false, f.p1, &l1)) return false;
    f.p1.seg[0].yt = t_qkv;
    f.p1.seg[1].yt = t_z;
    f.p1.seg[2].yt = t_ab;
    f.p1.seg[3].yt = t_ab + d.VH;
    f.p1.epoch = ep;
    f.p1.err = err;
    const SegIn o[1] = {{tout, dst}};
    if (!proj_args(o, 1, XF_GATED, nullptr, G.gnorm, nullptr, d.VD, d.eps, add, f.p3, &l3)) return false;
    f.p3.xt = t_y;
    f.p3.zt = t_z;
    f.p3.done = t_done;
    f.p3.ndone = d.VH * (d.VD / kGdnCols);
    f.p3.epoch = ep;
    f.p3.err = err;
    GdnArgs &g = f.g;
    g.ring = G.ring;
    g.head = G.head;
    g.convw = G.convw;
    g.S = G.S;
    g.alog = G.alog;
    g.dtb = G.dtb;
    g.eps = d.eps;
    g.D = tqkv->I;
    g.KH = d.KH;
    g.KD = d.KD;
    g.VH = d.VH;
    g.VD = d.VD;
    g.K = d.K;
    g.CD = d.CD;
    g.qkvt = t_qkv;
    g.abt = t_ab;
    g.yt = t_y;
    g.done = t_done;
    g.err = err;
    g.epoch = ep;
    f.n1 = (f.p1.ngroups + kWaves * kFuseU - 1) / (kWaves * kFuseU);
    f.nc = d.VH * (d.VD / kGdnCols);
    const int n3 = (f.p3.ngroups + kWaves * kFuseU3 - 1) / (kWaves * kFuseU3);
    if (l1 != 32 || l3 != 64 || f.p3.ndone > 64 * 8) return refuse("fused GDN shape");
    hipLaunchKernelGGL((gdn_fused<32, 64, 2>), dim3((unsigned)(f.n1 + f.nc + n3)), dim3(kThreads), 0, st, f);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("fused GDN launch", e);
    G.head = G.head + 1 == G.K ? 0 : G.head + 1;   // the ring advanced by this token
    return true;
}

// Error word of the fused layer launches since the last call (synchronizes): 0 none, 1 a
// bounded wait gave up, -1 runtime error.  Reading clears it.
static int layer_error_take() {
    if (!g_lt.err) return 0;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    unsigned long long v = 0;
    if (hipMemcpy(&v, g_lt.err, 8, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if ((uint32_t)v == 0) return 0;
    const unsigned long long z = 0;
    if (hipMemcpy(g_lt.err, &z, 8, hipMemcpyHostToDevice) != hipSuccess) return -1;
    return (int)(uint32_t)v;
}

static bool gdn_block(int gi, const float *src, const float *ln, const float *params, ColiVkTensor *tqkv,
                      ColiVkTensor *tz, ColiVkTensor *ta, ColiVkTensor *tb, ColiVkTensor *tout, float *dst, bool add,
                      const GdnDims &d, hipStream_t st) {
    if (gi < 0 || gi >= kMaxLayers) return refuse("GDN layer index");
    GdnState &G = g_gdn[gi];
    if (!G.S || G.VH != d.VH || G.KD != d.KD || G.VD != d.VD) return refuse("GDN state not ensured");
    if (!G.ring || !G.convw_set || G.K != d.K || G.CD != d.CD) return refuse("GDN conv ring/weights not set");
    if (d.KH < 1 || d.VH % d.KH || d.CD != 2 * d.KH * d.KD + d.VH * d.VD || d.KD % 64 || d.KD > kGdnMaxKD ||
        d.VD % kGdnCols || d.K < 1 || d.K > 16)
        return refuse("GDN shape");
    if (!tqkv || !tz || !tout || tqkv->O != d.CD || tz->O != d.VH * d.VD || tout->I != d.VH * d.VD)
        return refuse("GDN projection shapes");
    if (!params) {
        if (!G.alog || G.ba_VH != d.VH || G.ba_VD != d.VD) return refuse("GDN A_log/dt_bias/gnorm not set");
        if (!tensor_live(ta) || !tensor_live(tb) || ta->O != d.VH || tb->O != d.VH || ta->I != tqkv->I || tb->I != tqkv->I ||
            (ta->fmt != 0 && ta->fmt != 1 && ta->fmt != 6) || (tb->fmt != 0 && tb->fmt != 1 && tb->fmt != 6))
            return refuse("GDN a/b projections");
    }
    float *qkv = wbuf(W_QKV, d.CD), *z = wbuf(W_Z, (size_t)d.VH * d.VD), *y = wbuf(W_Y, (size_t)d.VH * d.VD);
    float *ab = wbuf(W_AB, (size_t)2 * d.VH);
    if (!qkv || !z || !y || !ab) return false;
    // fmt 6 a/b with the qkv geometry: two more segments of the same launch
    const auto lanes_like = [&](const ColiVkTensor *t) {
        return t && t->fmt == 6 && t->layout == kLayoutLanes && t->I == tqkv->I && t->gs == tqkv->gs &&
               t->nl == tqkv->nl && t->row_bytes == tqkv->row_bytes;
    };
    const bool ab_proj = !params && lanes_like(ta) && lanes_like(tb) && lanes_like(tz) && tqkv->fmt == 6;
    if (ab_proj && ln && fuse_on() && gdn_fusable(tqkv, tout, d))
        return gdn_fused_launch(G, src, ln, tqkv, tz, ta, tb, tout, dst, add, d, st);
    const SegIn in[4] = {{tqkv, qkv}, {tz, z, 1}, {ta, ab}, {tb, ab + d.VH}};   // z as silu(z)
    if (!proj(in, ab_proj ? 4 : 2, ln ? XF_NORM : XF_PLAIN, src, ln, nullptr, 0, d.eps, false, st))
        return false;
    GdnArgs g;
    memset(&g, 0, sizeof(g));
    g.qkv = qkv;
    g.ring = G.ring;
    g.head = G.head;
    g.ab = ab_proj ? ab : nullptr;
    g.convw = G.convw;
    g.S = G.S;
    g.y = y;
    g.params = params;
    g.xin = ln ? nullptr : src;
    g.resid = src;
    g.in_ln = ln;
    if (!params) {
        g.a = rowmat(ta);
        g.b = rowmat(tb);
    }
    g.alog = G.alog;
    g.dtb = G.dtb;
    g.eps = d.eps;
    g.D = tqkv->I;
    g.KH = d.KH;
    g.KD = d.KD;
    g.VH = d.VH;
    g.VD = d.VD;
    g.K = d.K;
    g.CD = d.CD;
    const dim3 grid(d.VH * (d.VD / kGdnCols));
    switch (d.KD / 64) {
    case 1: hipLaunchKernelGGL(gdn_core<1>, grid, dim3(kThreads), 0, st, g); break;
    case 2: hipLaunchKernelGGL(gdn_core<2>, grid, dim3(kThreads), 0, st, g); break;
    case 4: hipLaunchKernelGGL(gdn_core<4>, grid, dim3(kThreads), 0, st, g); break;
    default: return refuse("GDN key head dim not in {64, 128, 256}");
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("GDN launch", e);
    G.head = G.head + 1 == G.K ? 0 : G.head + 1;   // the ring advanced by this token
    const float *gnorm = params ? params + 2 * d.VH : G.gnorm;
    const SegIn o[1] = {{tout, dst}};
    return proj(o, 1, XF_GATED, y, gnorm, z, d.VD, d.eps, add, st);
}

// ---------------------------------------------------------------- residual stream state
struct StreamState {
    float *d_resid = nullptr;
    size_t resid_cap = 0;
    float *h_y = nullptr;         // pinned staging (stream_add, route read-back)
    size_t hy_cap = 0;
    float *d_y = nullptr;
    size_t dy_cap = 0;
    float *d_fnw = nullptr;       // final norm weight
    size_t fnw_cap = 0;
    int fn_D = 0;
    float *d_xn = nullptr;        // normed row + argmax result
    size_t xn_cap = 0;
    int D = 0, live = 0;
    int fused_last = 0;           // the last route_pipe ran the MoE on the device
    int pending = 0;              // top-k ids of fused layers await stream_end
    int hist_K[kMaxLayers];       // ids recorded per layer in this stream (0 = none)
    int hist_hi = 0;              // 1 + the highest layer with recorded ids
    int *h_rb = nullptr;          // pinned: stream_end's read-back, laid out as the device history
    size_t hrb_cap = 0;
    unsigned long long *h_am = nullptr;   // pinned: stream_norm_argmax's read-back (keys, error words)
    size_t ham_cap = 0;
    uint64_t chk_moe = ~0ull, chk_layer = ~0ull;   // launch counts at the last clean check
    float *h_nrm = nullptr;       // host copy of the last non-fused route's nrm
    size_t hnrm_cap = 0;
    float *h_x = nullptr;         // pinned staging of stream_begin's row (copied without a sync)
    size_t hx_cap = 0;
};
static StreamState g_str;
// stream_norm_argmax's work launched ahead by stream_end (see ahead_launch)
struct AheadArgmax {
    const ColiVkTensor *t = nullptr;   // the last stream_norm_argmax's tensor (NULL: none yet)
    const uint8_t *w = nullptr;
    int fmt = 0, I = 0, O = 0, gs = 0;
    float eps = 0.f;
    bool pending = false;              // launched by stream_end, not yet taken
    uint32_t ep = 0;                   // its launch tag
};
static AheadArgmax g_ahead;

float *stream_resid(int D) { return g_str.live && g_str.D == D ? g_str.d_resid : nullptr; }
const float *stream_nrm_dev(int D) {
    return g_str.live && g_str.D == D && !g_str.fused_last && g_w[W_NRM].p ? (const float *)g_w[W_NRM].p : nullptr;
}

// post_ln + router (+ device top-k) after the block has updated the residual `resid`.
// fused: the layer's MoE block runs on the device (expert table) and accumulates into
// resid; otherwise idx/val (route_pipe) or nothing is produced here.
static bool route_tail(int ln_layer, const float *resid, ColiVkTensor *router, int E, int topk, float eps,
                       float *nrm, float *logits, hipStream_t st, float *bounds = nullptr) {
    const LnState &ln = g_ln[ln_layer];
    hipLaunchKernelGGL(rms_rows, dim3(1), dim3(kThreads), 0, st, resid, ln.post_ln, nrm, ln.D, eps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("post norm launch", e);
    (void)topk;
    if (logits) {   // logits [E] (and their bounds [E] at `bounds`, or in work memory)
        if (router->fmt != 0 && router->fmt != 1) return gemv(router, nrm, logits, 1, st);
        if (!bounds && !(bounds = wbuf(W_BND, E))) return false;
        hipLaunchKernelGGL(router_lb, dim3((E + kWaves - 1) / kWaves), dim3(kThreads), 0, st, nrm, router->w,
                           router->sz, router->fmt, router->row_bytes, E, ln.D, logits, bounds);
        e = hipGetLastError();
        if (e != hipSuccess) return fail("router launch", e);
    }
    return true;
}

void layer_shutdown() {
    for (int i = 0; i < kMaxLayers; i++) {   // arena slices: gone with the arena
        g_kv[i] = KvState();
        g_qk[i] = QkNorm();
        g_gdn[i] = GdnState();
        g_ln[i] = LnState();
    }
    for (int i = 0; i < W_COUNT; i++) scratch_free(&g_w[i].p, &g_w[i].cap);
    scratch_free(&g_lt.tag, &g_lt.cap);
    scratch_free(&g_lt.err, &g_lt.ecap);
    g_lt.epoch = 0;
    scratch_free((void **)&g_str.d_resid, &g_str.resid_cap);
    scratch_free((void **)&g_str.d_y, &g_str.dy_cap);
    scratch_free((void **)&g_str.d_fnw, &g_str.fnw_cap);
    scratch_free((void **)&g_str.d_xn, &g_str.xn_cap);
    host_scratch_free((void **)&g_str.h_y, &g_str.hy_cap);
    host_scratch_free((void **)&g_str.h_nrm, &g_str.hnrm_cap);
    host_scratch_free((void **)&g_str.h_x, &g_str.hx_cap);
    host_scratch_free((void **)&g_str.h_rb, &g_str.hrb_cap);
    host_scratch_free((void **)&g_str.h_am, &g_str.ham_cap);
    g_str = StreamState();
    g_ahead = AheadArgmax();
}

}  // namespace coli

using namespace coli;

extern "C" int coli_vk_tensor_ensure(ColiVkTensor **, const void *, const float *, int, int, int, int);

static bool ln_ok(int ln_layer, int D) {
    return ln_layer >= 0 && ln_layer < kMaxLayers && g_ln[ln_layer].in_ln && g_ln[ln_layer].D == D;
}

// ---------------------------------------------------------------- ABI: KV mirror + GQA
// c/backend_vulkan.h:110-116, c/backend_vulkan.c:1705-1743
COLI_API int coli_vk_kv_ensure(int layer, int max_rows, int K, int Rd) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || max_rows < 1 || K < 1 || Rd < 1) return 0;
    KvState &v = g_kv[layer];
    if (v.K && v.rows) return v.rows >= max_rows && v.kd == K && v.vd == Rd;
    if (!v.K || v.cap_rows < max_rows || v.kd != K || v.vd != Rd) {   // kv_reset keeps the old arena slice
        v.K = (float *)arena_alloc((size_t)max_rows * K * 4);
        v.V = (float *)arena_alloc((size_t)max_rows * Rd * 4);
        if (!v.K || !v.V) {
            v = KvState();
            return 0;
        }
        v.cap_rows = max_rows;
    }
    v.rows = max_rows;
    v.kd = K;
    v.vd = Rd;
    hipError_t e = hipMemsetAsync(v.K, 0, (size_t)max_rows * K * 4, stream());
    if (e == hipSuccess) e = hipMemsetAsync(v.V, 0, (size_t)max_rows * Rd * 4, stream());
    if (e != hipSuccess) return fail("kv ensure", e) ? 1 : 0;
    return sync_stream("kv ensure") ? 1 : 0;
}

// one host cache row (normed + roped key, raw value) into the mirror
COLI_API int coli_vk_kv_row(int layer, int pos, const float *L, const float *R) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || !L || !R) return 0;
    KvState &v = g_kv[layer];
    if (!v.K || pos < 0 || pos >= v.rows) return 0;
    return h2d(v.K + (size_t)pos * v.kd, L, (size_t)v.kd * 4, "kv row") &&
                   h2d(v.V + (size_t)pos * v.vd, R, (size_t)v.vd * 4, "kv row")
               ? 1
               : 0;
}

// Rows [row0, row0 + n) of a layer's mirror from host arrays [n][kd] and [n][vd] (a bulk
// kv_row; used to seed a cache of a given length).
COLI_API int coli_hip_kv_load(int layer, int row0, int n, const float *L, const float *R) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || !L || !R || n < 0) return 0;
    KvState &v = g_kv[layer];
    if (!v.K || row0 < 0 || row0 + n > v.rows) return 0;
    return h2d(v.K + (size_t)row0 * v.kd, L, (size_t)n * v.kd * 4, "kv load") &&
                   h2d(v.V + (size_t)row0 * v.vd, R, (size_t)n * v.vd * 4, "kv load")
               ? 1
               : 0;
}

// Rows [row0, row0 + n) of the mirror back to the host (tests).
COLI_API int coli_hip_kv_read(int layer, int row0, int n, float *L, float *R) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || !L || !R || n < 0) return 0;
    KvState &v = g_kv[layer];
    if (!v.K || row0 < 0 || row0 + n > v.rows || !sync_stream("kv read")) return 0;
    return hipMemcpy(L, v.K + (size_t)row0 * v.kd, (size_t)n * v.kd * 4, hipMemcpyDeviceToHost) == hipSuccess &&
                   hipMemcpy(R, v.V + (size_t)row0 * v.vd, (size_t)n * v.vd * 4, hipMemcpyDeviceToHost) ==
                       hipSuccess
               ? 1
               : 0;
}

COLI_API void coli_vk_kv_reset(void) {
    for (int i = 0; i < kMaxLayers; i++) g_kv[i].rows = 0;   // slices stay for a later kv_ensure
}

COLI_API int coli_vk_gqa_available(void) { return ok() ? 1 : 0; }
COLI_API int coli_vk_gqa_full_available(void) { return ok() ? 1 : 0; }

COLI_API int coli_vk_gqa_norm_weight(int layer, const float *qnw, const float *knw, int hd) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || hd < 1) return 0;
    QkNorm &q = g_qk[layer];
    int h1 = q.hd, h2 = q.hd;
    if (!put_vec(&q.qn, &h1, qnw, hd, "q norm weight") || !put_vec(&q.kn, &h2, knw, hd, "k norm weight")) return 0;
    q.hd = hd;
    return 1;
}

// Host rows through the device block, S tokens in order (token s attends to the rows the
// earlier tokens of the call wrote).
static int gqa_rows(int layer, const float *x, int D, ColiVkTensor *tq, ColiVkTensor *tk, ColiVkTensor *tv,
                    ColiVkTensor *to, float *out, int S, const GqaDims &d, int pos_base, int Dout) {
    if (!ok() || !x || !out || S < 1 || D < 1 || !tq || tq->I != D || !to || to->O != Dout) return 0;
    float *dx = wbuf(W_IO_X, (size_t)S * D), *dout = wbuf(W_IO_O, (size_t)S * Dout);
    if (!dx || !dout || !h2d(dx, x, (size_t)S * D * 4, "gqa rows")) return 0;
    for (int s = 0; s < S; s++)
        if (!gqa_block(layer, dx + (size_t)s * D, nullptr, tq, tk, tv, to, dout + (size_t)s * Dout, false, d,
                       pos_base + s, stream()))
            return 0;
    return read_back(out, dout, (size_t)S * Dout * 4, stream(), "gqa rows") ? 1 : 0;
}

// S >= kGemmMinS rows in one pass (c/backend_vulkan.c:2280-2340): q/k/v as one digit
// decomposition and three GEMMs, qk_rows, attn_rows, the o-projection GEMM.  0 with no
// device work done when a shape is outside these kernels (the caller then takes gqa_rows).
enum { kSeqNo = -1 };
static int g_gqa_seq = 1;   // 0: every S takes the token loop (coli_hip_gqa_seq)
// The rotation rows [pos][rot / 2] of (cos, sin) per position, c/qwen.c:570-579 as the
// decode block computes them (in double, rounded to float), kept across calls: they depend
// only on (theta, rot, pos), so the GQA layers of a prompt and its later chunks share them.
// Rows are added as positions are first used.  nullptr when out of host memory.
static const float *rope_rows(float theta, int rot, int pos_end) {
    static float c_theta = 0.f;
    static int c_rot = 0, c_rows = 0;
    static std::vector<float> c_inv, c_tab;
    const int hr = rot / 2;
    try {
        if (c_theta != theta || c_rot != rot) {
            c_theta = theta, c_rot = rot, c_rows = 0;
            c_tab.clear();
            c_inv.resize(hr);
            for (int j = 0; j < hr; j++) c_inv[j] = (float)pow((double)theta, (double)(-2.0f * j / rot));
        }
        if (pos_end > c_rows) {
            c_tab.resize((size_t)pos_end * hr * 2);
            for (int s = c_rows; s < pos_end; s++)
                for (int j = 0; j < hr; j++) {
                    const float ang = (float)s * c_inv[j];
                    c_tab[((size_t)s * hr + j) * 2] = (float)cos((double)ang);
                    c_tab[((size_t)s * hr + j) * 2 + 1] = (float)sin((double)ang);
                }
            c_rows = pos_end;
        }
    } catch (...) {
        c_theta = 0.f, c_rot = 0, c_rows = 0;
        return nullptr;
    }
    return c_tab.data();
}

static int gqa_seq(int layer, const float *x, int D, ColiVkTensor *tq, ColiVkTensor *tk, ColiVkTensor *tv,
                   ColiVkTensor *to, float *out, int S, const GqaDims &d, int pos_base, int Dout) {
    const int H = d.H, KH = d.KH, hd = d.hd, hr = d.rot / 2;
    if (layer < 0 || layer >= kMaxLayers || S < kGemmMinS || (hd != 64 && hd != 128 && hd != 256)) return kSeqNo;
    const KvState &kv = g_kv[layer];
    const QkNorm &qk = g_qk[layer];
    if (!kv.K || kv.kd != hd || kv.vd != hd || (long)KH * d.max_t > kv.rows || !qk.qn || qk.hd != hd) return kSeqNo;
    if (H < 1 || KH < 1 || H % KH || d.rot < 2 || d.rot > hd || d.rot % 2 || pos_base < 0 ||
        (long)pos_base + S > d.max_t)
        return kSeqNo;
    if (!gemm6_ok(tq) || !gemm6_ok(tk) || !gemm6_ok(tv) || !gemm6_ok(to) || tq->I != D || tk->I != D ||
        tv->I != D || tq->O != 2 * H * hd || tk->O != KH * hd || tv->O != KH * hd || to->I != H * hd ||
        to->O != Dout)
        return kSeqNo;
    float *dx = wbuf(W_IO_X, (size_t)S * D), *dout = wbuf(W_IO_O, (size_t)S * Dout);
    float *qraw = wbuf(W_SQKV, (size_t)S * 2 * H * hd), *kr = wbuf(W_SZ, (size_t)S * 2 * KH * hd);
    float *qn = wbuf(W_SY, (size_t)S * H * hd), *ctx = wbuf(W_CTX, (size_t)S * H * hd);
    float *rope = wbuf(W_ROPE, (size_t)S * hr * 2);
    if (!dx || !dout || !qraw || !kr || !qn || !ctx || !rope) return 0;
    float *vr = kr + (size_t)S * KH * hd;
    const float *tab = rope_rows(d.theta, d.rot, pos_base + S);
    if (!tab) return 0;
    const Upload u[2] = {{dx, x, (size_t)S * D * 4}, {rope, tab + (size_t)pos_base * hr * 2, (size_t)S * hr * 8}};
    if (!upload(u, 2, stream(), "gqa seq upload")) return 0;
    const ColiVkTensor *tp[3] = {tq, tk, tv};
    float *const yp[3] = {qraw, kr, vr};
    if (!gemm6(tp, yp, 3, dx, S, stream())) return 0;
    hipLaunchKernelGGL(qk_rows, dim3(S, H + KH), dim3(64), 0, stream(), qraw, kr, vr, qk.qn, qk.kn,
                       (const float2 *)rope, qn, kv.K, kv.V, H, KH, hd, d.rot, pos_base, d.max_t, d.eps);
    AttnRowsArgs a;
    a.qraw = qraw;
    a.qn = qn;
    a.Kc = kv.K;
    a.Vc = kv.V;
    a.ctx = ctx;
    a.S = S;
    a.H = H;
    a.KH = KH;
    a.pos_base = pos_base;
    a.max_t = d.max_t;
    a.nqt = (S + kPQ - 1) / kPQ;
    a.scale = 1.f / sqrtf((float)hd);
    const dim3 ga((unsigned)(H * a.nqt));
    if (hd == 64) hipLaunchKernelGGL(attn_rows<64>, ga, dim3(256), 0, stream(), a);
    else if (hd == 128) hipLaunchKernelGGL(attn_rows<128>, ga, dim3(256), 0, stream(), a);
    else hipLaunchKernelGGL(attn_rows<256>, ga, dim3(256), 0, stream(), a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("attention rows launch", e) ? 1 : 0;
    const ColiVkTensor *op[1] = {to};
    float *const oy[1] = {dout};
    if (!gemm6(op, oy, 1, ctx, S, stream())) return 0;
    return read_back(out, dout, (size_t)S * Dout * 4, stream(), "gqa seq") ? 1 : 0;
}

// c/backend_vulkan.h:171-178: x is the normed input [S, D]; out [S, Dout] = block output
COLI_API int coli_vk_gqa_full(int layer, const float *x, int D, ColiVkTensor *gq_t, ColiVkTensor *gk_t,
                              ColiVkTensor *gv_t, ColiVkTensor *out_t, float *out, int S, int H, int KH, int hd,
                              int rot, int pos_base, int max_t, float eps, float theta, int Dout) {
    const GqaDims d = {H, KH, hd, rot, max_t, eps, theta};
    if (!ok() || !x || !out || S < 1 || D < 1) return 0;
    if (g_gqa_seq) {
        const int r = gqa_seq(layer, x, D, gq_t, gk_t, gv_t, out_t, out, S, d, pos_base, Dout);
        if (r != kSeqNo) return r;
    }
    return gqa_rows(layer, x, D, gq_t, gk_t, gv_t, out_t, out, S, d, pos_base, Dout);
}

// Test and bench hook: S > 1 rows of coli_vk_gqa_full in one batched pass (1, the default) or
// as the token loop (0); returns the previous setting.
COLI_API int coli_hip_gqa_seq(int on) {
    const int prev = g_gqa_seq;
    g_gqa_seq = on ? 1 : 0;
    return prev;
}

COLI_API int coli_hip_gdn_chunked(int on) {
    const int prev = g_gdn_chunked;
    g_gdn_chunked = on ? 1 : 0;
    return prev;
}

// The staged forms take host-computed q (already normed and rotated) and the host KV
// mirror rows; the engine only reaches them when the fused block is off.  Not provided:
// 0 makes the engine attend on the CPU (c/qwen.c:620-636).
COLI_API int coli_vk_gqa(int, const float *, float *, int, int, int, int, int, int, int, float) { return 0; }
COLI_API int coli_vk_gqa_project(int, const float *, ColiVkTensor *, float *, int, int, int, int, int, int, int,
                                 float, int) {
    return 0;
}

// ---------------------------------------------------------------- ABI: GDN state
// c/backend_vulkan.h:146-156, :258-279, c/backend_vulkan.c:1745-1790
COLI_API int coli_vk_gdn_available(void) { return ok() ? 1 : 0; }
COLI_API int coli_vk_gdn_full_available(void) { return ok() ? 1 : 0; }

COLI_API int coli_vk_gdn_state_ensure(int layer, int VH, int KD, int VD) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || VH < 1 || KD < 1 || VD < 1) return 0;
    GdnState &G = g_gdn[layer];
    if (G.S) return G.VH == VH && G.KD == KD && G.VD == VD;
    const size_t bytes = (size_t)VH * KD * VD * 4;
    G.S = (float *)arena_alloc(bytes);
    if (!G.S) return 0;
    G.VH = VH;
    G.KD = KD;
    G.VD = VD;
    const hipError_t e = hipMemsetAsync(G.S, 0, bytes, stream());
    if (e != hipSuccess) return fail("gdn state", e) ? 1 : 0;
    return sync_stream("gdn state") ? 1 : 0;
}

COLI_API void coli_vk_gdn_reset(void) {
    if (!ok()) return;
    for (int i = 0; i < kMaxLayers; i++) {
        GdnState &G = g_gdn[i];
        if (G.S) (void)hipMemsetAsync(G.S, 0, (size_t)G.VH * G.KD * G.VD * 4, stream());
        if (G.ring) (void)hipMemsetAsync(G.ring, 0, (size_t)G.K * G.CD * 4, stream());
        G.head = 0;
    }
    (void)sync_stream("gdn reset");
}

COLI_API int coli_vk_gdn_conv_ensure(int layer, int conv_k, int conv_dim) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || conv_k < 1 || conv_k > 16 || conv_dim < 1) return 0;
    GdnState &G = g_gdn[layer];
    if (G.ring) return G.K == conv_k && G.CD == conv_dim;
    const size_t n = (size_t)conv_k * conv_dim;
    G.ring = (float *)arena_alloc(n * 4);
    G.convw = (float *)arena_alloc(n * 4);
    if (!G.ring || !G.convw) {
        G.ring = G.convw = nullptr;
        return 0;
    }
    G.K = conv_k;
    G.CD = conv_dim;
    G.head = 0;
    const hipError_t e = hipMemsetAsync(G.ring, 0, n * 4, stream());
    if (e != hipSuccess) return fail("gdn conv ring", e) ? 1 : 0;
    return sync_stream("gdn conv ring") ? 1 : 0;
}

// cw [conv_dim][conv_k] (c/qwen.c:702: w = conv + ch * K)
COLI_API int coli_vk_gdn_conv_weight(int layer, const float *cw, int conv_k, int conv_dim) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || !cw) return 0;
    GdnState &G = g_gdn[layer];
    if (!G.ring || G.K != conv_k || G.CD != conv_dim) return 0;
    if (!h2d(G.convw, cw, (size_t)conv_k * conv_dim * 4, "gdn conv weight")) return 0;
    G.convw_set = 1;
    return 1;
}

// c/qwen.c:1525-1533: A_log [VH], dt_bias [VH], gated-norm weight [VD] of a GDN layer
COLI_API int coli_vk_gdn_ba_weight(int layer, const float *alog, const float *dtb, const float *gnorm, int VH,
                                   int VD) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || VH < 1 || VD < 1) return 0;
    GdnState &G = g_gdn[layer];
    int h1 = G.ba_VH, h2 = G.ba_VH, h3 = G.ba_VD;
    if (!put_vec(&G.alog, &h1, alog, VH, "A_log") || !put_vec(&G.dtb, &h2, dtb, VH, "dt_bias") ||
        !put_vec(&G.gnorm, &h3, gnorm, VD, "gdn norm weight"))
        return 0;
    G.ba_VH = VH;
    G.ba_VD = VD;
    return 1;
}

// GDN prefill over S >= kGemmMinS tokens with host params (c/backend_vulkan.c:2018-2157),
// per chunk of up to kGdnSeqChunk tokens: qkv and z of all the chunk's rows in one dense
// GEMM (one digit decomposition of x), the recurrence of the chunk (gdn_chunk_prep /
// _mats / _scan over 64-token pieces; gdn_seq token by token for other shapes or when
// coli_hip_gdn_chunked(0)), the ring push, then the gated norm and out-projection of all
// rows in one more GEMM.
// False with nothing launched when the shapes are not the GEMM's or the conv is longer than
// gdn_seq's register window (the caller then runs the tokens one at a time).
constexpr int kGdnSeqChunk = 1024;
static bool gdn_chunks(int gi, const float *dx, const float *dp, int S, const ColiVkTensor *tqkv,
                       const ColiVkTensor *tz, const ColiVkTensor *tout, float *dout, const GdnDims &d,
                       hipStream_t st, bool *ran) {
    *ran = false;
    if (gi < 0 || gi >= kMaxLayers || S < kGemmMinS) return true;
    GdnState &G = g_gdn[gi];
    const int VV = d.VH * d.VD, prs = 2 * d.VH + d.VD;
    if (!G.S || G.VH != d.VH || G.KD != d.KD || G.VD != d.VD || !G.ring || !G.convw_set || G.K != d.K ||
        G.CD != d.CD)
        return true;   // gdn_block refuses these with a message
    if (d.KH < 1 || d.VH % d.KH || d.CD != 2 * d.KH * d.KD + VV || d.KD % 64 || d.KD > kGdnMaxKD ||
        d.VD % kSeqCols || d.K < 1 || d.K > kGdnMaxK || d.VD > 512 || (d.VD & (d.VD - 1)))
        return true;
    if (!gemm6_ok(tqkv) || !gemm6_ok(tz) || !gemm6_ok(tout) || tqkv->O != d.CD || tz->O != VV || tz->I != tqkv->I ||
        tout->I != VV)
        return true;
    *ran = true;
    const int D = tqkv->I, Dout = tout->O;
    for (int s0 = 0; s0 < S; s0 += kGdnSeqChunk) {
        const int n = min(kGdnSeqChunk, S - s0);
        float *qkv = wbuf(W_SQKV, (size_t)n * d.CD), *z = wbuf(W_SZ, (size_t)n * VV), *y = wbuf(W_SY, (size_t)n * VV);
        if (!qkv || !z || !y) return false;
        const ColiVkTensor *tin[2] = {tqkv, tz};
        float *const yin[2] = {qkv, z};
        if (!gemm6(tin, yin, 2, dx + (size_t)s0 * D, n, st)) return false;
        GdnSeqArgs a;
        a.qkv = qkv;
        a.ring = G.ring;
        a.head = G.head;
        a.n = n;
        a.convw = G.convw;
        a.S = G.S;
        a.y = y;
        a.params = dp + (size_t)s0 * prs;
        a.prs = prs;
        a.eps = d.eps;
        a.KH = d.KH;
        a.KD = d.KD;
        a.VH = d.VH;
        a.VD = d.VD;
        a.K = d.K;
        a.CD = d.CD;
        if (g_gdn_chunked && (d.KD == 64 || d.KD == 128) && d.VD % kGcCols == 0) {
            const int nchunk = (n + kGc - 1) / kGc;
            GdnChunkArgs c;
            c.qkv = qkv;
            c.ring = G.ring;
            c.head = G.head;
            c.n = n;
            c.convw = G.convw;
            c.params = a.params;
            c.prs = prs;
            c.eps = d.eps;
            c.KH = d.KH;
            c.KD = d.KD;
            c.VH = d.VH;
            c.VD = d.VD;
            c.K = d.K;
            c.CD = d.CD;
            c.nchunk = nchunk;
            c.qn = wbuf(W_GQN, (size_t)n * d.KH * d.KD);
            c.kn = wbuf(W_GKN, (size_t)n * d.KH * d.KD);
            c.vv = wbuf(W_GVV, (size_t)n * d.CD);
            c.mats = wbuf(W_GMAT, (size_t)d.VH * nchunk * kGcMat);
            c.S = G.S;
            c.y = y;
            if (!c.qn || !c.kn || !c.vv || !c.mats) return false;
            hipLaunchKernelGGL(gdn_chunk_conv, dim3((d.CD + kThreads - 1) / kThreads, (n + kGcConvT - 1) / kGcConvT),
                               dim3(kThreads), 0, st, c);
            hipLaunchKernelGGL(gdn_chunk_norm, dim3((n * 2 * d.KH + kWaves - 1) / kWaves), dim3(kThreads), 0, st, c);
            hipLaunchKernelGGL(gdn_chunk_mats, dim3(d.VH, nchunk), dim3(kThreads), 0, st, c);
            if (d.KD == 128)
                hipLaunchKernelGGL(gdn_chunk_scan<128>, dim3(d.VH * (d.VD / kGcCols)), dim3(kThreads), 0, st, c);
            else
                hipLaunchKernelGGL(gdn_chunk_scan<64>, dim3(d.VH * (d.VD / kGcCols)), dim3(kThreads), 0, st, c);
        } else {
            const dim3 grid(d.VH * (d.VD / kSeqCols));
            switch (d.KD / 64) {
            case 1: hipLaunchKernelGGL(gdn_seq<1>, grid, dim3(kThreads), 0, st, a); break;
            case 2: hipLaunchKernelGGL(gdn_seq<2>, grid, dim3(kThreads), 0, st, a); break;
            case 4: hipLaunchKernelGGL(gdn_seq<4>, grid, dim3(kThreads), 0, st, a); break;
            default: return refuse("GDN key head dim not in {64, 128, 256}");
            }
        }
        const int pushed = min(n, d.K) * d.CD;
        hipLaunchKernelGGL(gdn_ring_push, dim3((pushed + 255) / 256), dim3(256), 0, st, qkv, n, G.ring, G.head, d.K,
                           d.CD);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("GDN chunk launch", e);
        G.head = (G.head + n) % d.K;
        const GatedX gx = {z, dp + (size_t)s0 * prs + 2 * d.VH, prs, d.VD, d.eps};
        const ColiVkTensor *to[1] = {tout};
        float *const yo[1] = {dout + (size_t)s0 * Dout};
        if (!gemm6(to, yo, 1, y, n, st, &gx)) return false;
    }
    return true;
}

static int gdn_rows(int layer, const float *x, int S, int D, ColiVkTensor *gqkv_t, ColiVkTensor *gz_t,
                    const float *params, ColiVkTensor *out_t, float *out, const GdnDims &d, int Dout) {
    if (!ok() || !x || !params || !out || S < 1 || !gqkv_t || gqkv_t->I != D || !out_t || out_t->O != Dout)
        return 0;
    const int prs = 2 * d.VH + d.VD;
    float *dx = wbuf(W_IO_X, (size_t)S * D), *dp = wbuf(W_IO_P, (size_t)S * prs),
          *dout = wbuf(W_IO_O, (size_t)S * Dout);
    const Upload u[2] = {{dx, x, (size_t)S * D * 4}, {dp, params, (size_t)S * prs * 4}};
    if (!dx || !dp || !dout || !upload(u, 2, stream(), "gdn rows upload")) return 0;
    bool ran;
    if (!gdn_chunks(layer, dx, dp, S, gqkv_t, gz_t, out_t, dout, d, stream(), &ran)) return 0;
    for (int s = 0; !ran && s < S; s++)
        if (!gdn_block(layer, dx + (size_t)s * D, nullptr, dp + (size_t)s * prs, gqkv_t, gz_t, nullptr, nullptr,
                       out_t, dout + (size_t)s * Dout, false, d, stream()))
            return 0;
    return read_back(out, dout, (size_t)S * Dout * 4, stream(), "gdn rows") ? 1 : 0;
}

// c/backend_vulkan.h:268-271: one token, x normed, params [decay | beta | gnorm]
COLI_API int coli_vk_gdn_full(int layer, const float *x, int D, ColiVkTensor *gqkv_t, ColiVkTensor *gz_t,
                              const float *params, ColiVkTensor *out_t, float *out, int KH, int KD, int VH, int VD,
                              int conv_dim, int conv_k, float eps, int Dout) {
    const GdnDims d = {KH, KD, VH, VD, conv_dim, conv_k, eps};
    return gdn_rows(layer, x, 1, D, gqkv_t, gz_t, params, out_t, out, d, Dout);
}

// c/backend_vulkan.h:272-279: S tokens in order (the state and ring advance per token)
COLI_API int coli_vk_gdn_full_seq(int layer, const float *x, int S, int D, ColiVkTensor *gqkv_t, ColiVkTensor *gz_t,
                                  const float *params, ColiVkTensor *out_t, float *out, int KH, int KD, int VH, int VD,
                                  int conv_dim, int conv_k, float eps, int Dout) {
    const GdnDims d = {KH, KD, VH, VD, conv_dim, conv_k, eps};
    return gdn_rows(layer, x, S, D, gqkv_t, gz_t, params, out_t, out, d, Dout);
}

// Staged forms (host qn/kn/v/z/decay/beta): reached only when the fused block is off; 0
// keeps that token's recurrence on the CPU (c/qwen.c:741-761).
COLI_API int coli_vk_gdn(int, const float *, const float *, const float *, const float *, const float *, const float *,
                         const float *, float *, int, int, int, int, float) {
    return 0;
}
COLI_API int coli_vk_gdn_project(int, const float *, const float *, const float *, const float *, const float *,
                                 const float *, const float *, ColiVkTensor *, float *, int, int, int, int, float,
                                 int) {
    return 0;
}

// GDN state of a layer back to the host in the reference's layouts (tests): conv ring
// [K][CD], recurrent state [VH][KD][VD].
COLI_API int coli_hip_gdn_state_read(int layer, float *ring, float *S) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || !ring || !S) return 0;
    GdnState &G = g_gdn[layer];
    if (!G.S || !G.ring || !sync_stream("gdn state read")) return 0;
    const size_t n = (size_t)G.VH * G.KD * G.VD;
    float *t = (float *)malloc(n * 4);
    if (!t) return 0;
    int r = hipMemcpy(t, G.S, n * 4, hipMemcpyDeviceToHost) == hipSuccess;
    for (int j = 0; r && j < G.K; j++) {   // logical slot j (0 = oldest) is physical head + j
        const int slot = (G.head + j) % G.K;
        r = hipMemcpy(ring + (size_t)j * G.CD, G.ring + (size_t)slot * G.CD, (size_t)G.CD * 4,
                      hipMemcpyDeviceToHost) == hipSuccess;
    }
    for (int h = 0; r && h < G.VH; h++)   // device [h][vd][kd] -> host [h][kd][vd]
        for (int kd = 0; kd < G.KD; kd++)
            for (int vd = 0; vd < G.VD; vd++)
                S[((size_t)h * G.KD + kd) * G.VD + vd] = t[((size_t)h * G.VD + vd) * G.KD + kd];
    free(t);
    return r;
}

// ---------------------------------------------------------------- ABI: route fusion
// c/backend_vulkan.h:179-198
COLI_API int coli_vk_moe_route_available(void) { return ok() ? 1 : 0; }

COLI_API int coli_vk_layer_norm_weight(int layer, const float *in_ln, const float *post_ln, int D) {
    if (!ok() || layer < 0 || layer >= kMaxLayers || D < 1) return 0;
    LnState &L = g_ln[layer];
    int h1 = L.D, h2 = L.D;
    if (!put_vec(&L.in_ln, &h1, in_ln, D, "in_ln") || !put_vec(&L.post_ln, &h2, post_ln, D, "post_ln")) return 0;
    L.D = D;
    return 1;
}

// the tail outputs of the *_full_route forms: resid_out, nrm_out [S, D], pr_out [S, E]
static bool full_route_out(const float *dres, const float *dnrm, const float *dlog, int S, int D, int E,
                           float *resid_out, float *nrm_out, float *pr_out) {
    if (!sync_stream("route read-back")) return false;
    bool r = true;
    if (resid_out) r &= read_back(resid_out, dres, (size_t)S * D * 4, stream(), "route read-back");
    if (nrm_out) r &= read_back(nrm_out, dnrm, (size_t)S * D * 4, stream(), "route read-back");
    if (pr_out) r &= read_back(pr_out, dlog, (size_t)S * E * 4, stream(), "route read-back");
    return r;
}

COLI_API int coli_vk_gqa_full_route(int layer, const float *resid, int D, ColiVkTensor *gq_t, ColiVkTensor *gk_t,
                                    ColiVkTensor *gv_t, ColiVkTensor *out_t, ColiVkTensor *router, int ln_layer,
                                    float *resid_out, float *nrm_out, float *pr_out, int S, int H, int KH, int hd,
                                    int rot, int pos_base, int max_t, float eps, float theta, int Dout, int E) {
    if (!ok() || !resid || S < 1 || D != Dout || !ln_ok(ln_layer, D) || !router || router->I != D || router->O != E)
        return 0;
    const GqaDims d = {H, KH, hd, rot, max_t, eps, theta};
    float *dr = wbuf(W_IO_R, (size_t)S * D), *dn = wbuf(W_IO_X, (size_t)S * D), *dl = wbuf(W_IO_P, (size_t)S * E);
    if (!dr || !dn || !dl || !h2d(dr, resid, (size_t)S * D * 4, "gqa route")) return 0;
    for (int s = 0; s < S; s++) {
        float *rs = dr + (size_t)s * D;
        if (!gqa_block(layer, rs, g_ln[ln_layer].in_ln, gq_t, gk_t, gv_t, out_t, rs, true, d, pos_base + s,
                       stream()) ||
            !route_tail(ln_layer, rs, router, E, 0, eps, dn + (size_t)s * D, dl + (size_t)s * E, stream()))
            return 0;
    }
    return full_route_out(dr, dn, dl, S, D, E, resid_out, nrm_out, pr_out) ? 1 : 0;
}

COLI_API int coli_vk_gdn_full_route(int layer, const float *x_in, const float *resid, int D, ColiVkTensor *gqkv_t,
                                    ColiVkTensor *gz_t, const float *params, ColiVkTensor *out_t, ColiVkTensor *router,
                                    int ln_layer, float *resid_out, float *nrm_out, float *pr_out, int KH, int KD,
                                    int VH, int VD, int conv_dim, int conv_k, float eps, int Dout, int E) {
    if (!ok() || !x_in || !resid || !params || D != Dout || !ln_ok(ln_layer, D) || !router || router->I != D ||
        router->O != E)
        return 0;
    const GdnDims d = {KH, KD, VH, VD, conv_dim, conv_k, eps};
    const int prs = 2 * VH + VD;
    float *dr = wbuf(W_IO_R, D), *dx = wbuf(W_IO_X, 2 * (size_t)D), *dp = wbuf(W_IO_P, (size_t)prs + E);
    if (!dr || !dx || !dp || !h2d(dr, resid, (size_t)D * 4, "gdn route") || !h2d(dx, x_in, (size_t)D * 4, "gdn route") ||
        !h2d(dp, params, (size_t)prs * 4, "gdn route"))
        return 0;
    float *dn = dx + D, *dl = dp + prs;
    if (!gdn_block(layer, dx, nullptr, dp, gqkv_t, gz_t, nullptr, nullptr, out_t, dr, true, d, stream()) ||
        !route_tail(ln_layer, dr, router, E, 0, eps, dn, dl, stream()))
        return 0;
    return full_route_out(dr, dn, dl, 1, D, E, resid_out, nrm_out, pr_out) ? 1 : 0;
}

// ---------------------------------------------------------------- ABI: residual stream
// c/backend_vulkan.h:199-252.  The decode stream keeps the residual on the device across
// layers; each *_full_route_pipe runs in_ln + block + residual add + post_ln + router, then
// either the layer's MoE block on the device (expert table set for the layer: fused, the
// top-k ids go to a device history read at stream_end) or the device top-k whose ids and
// weights the caller reads back (the engine then issues the experts, c/qwen.c:934-998).
COLI_API int coli_vk_stream_available(void) { return ok() ? 1 : 0; }

// The device history of the fused layers' top-k ids: kHistHead ints (3 error words, gathered
// there by stream_end), then kTopK ids per layer (fused layers have K <= kTopK).  stream_end
// reads back the words up to the highest recorded layer in one copy.
constexpr int kHistHead = 8;
static size_t hist_ints() { return kHistHead + (size_t)kMaxLayers * kTopK; }
static int *hist_dev() { return (int *)wbuf(W_HIST, hist_ints()); }

COLI_API int coli_vk_stream_begin(const float *x, int D) {
    g_ahead.pending = false;   // a new token: the lm_head launched ahead is not wanted
    if (!ok() || !x || D < 1) return 0;
    // the row goes through pinned staging and a copy kernel: the token's first launches
    // queue behind it at once (a hipMemcpyAsync held the host ~15 us while the device sat
    // idle).  The staging is rewritten only with the stream idle (a live stream is drained
    // first; a finished token was drained by its read-backs).
    if (g_str.live && !sync_stream("stream begin")) return 0;
    if (!scratch((void **)&g_str.d_resid, &g_str.resid_cap, (size_t)D * 4) ||
        !host_scratch((void **)&g_str.h_x, &g_str.hx_cap, (size_t)D * 4))
        return 0;
    memcpy(g_str.h_x, x, (size_t)D * 4);
    if (!pin_copy(g_str.d_resid, g_str.h_x, (size_t)D * 4, stream(), "stream begin")) return 0;
    g_str.D = D;
    g_str.live = 1;
    g_str.pending = 0;
    g_str.fused_last = 0;
    memset(g_str.hist_K, 0, sizeof(g_str.hist_K));
    g_str.hist_hi = 0;
    return 1;
}

// A fused MoE launch whose bounded wait gave up (or that met a bad expert id) leaves the
// residual wrong: like a failed fence wait in the reference (c/backend_vulkan.c:1094-1124,
// G.ready = 0), that disables the device and the call returns 0, so the engine takes its
// host path.  The launches that can fail so (the fused layer kernel, the MoE block in both
// entry points) leave a code in an error word.  A check is skipped when none of them ran
// since the last clean one; otherwise err_gather copies the words, stream-ordered after the
// launches, next to the data the caller reads back anyway, so one copy carries both.
static void err_mark() {
    g_str.chk_moe = moe_launches();
    g_str.chk_layer = g_lt.launches;
}
static bool err_clean() { return g_str.chk_moe == moe_launches() && g_str.chk_layer == g_lt.launches; }

__global__ void err_gather(const unsigned long long *l, const unsigned long long *m0, const unsigned long long *m1,
                           unsigned long long *out) {
    if (threadIdx.x == 0) {
        out[0] = l ? __hip_atomic_load(l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        out[1] = m0 ? __hip_atomic_load(m0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        out[2] = m1 ? __hip_atomic_load(m1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
    }
}

static bool err_gather_launch(unsigned long long *d_out) {
    const unsigned long long *m0, *m1;
    moe_error_words(&m0, &m1);
    hipLaunchKernelGGL(err_gather, dim3(1), dim3(64), 0, stream(), (const unsigned long long *)g_lt.err, m0, m1,
                       d_out);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess || fail("error word gather", e);
}

static bool err_report(const char *who, int le, int e) {
    if (le != 0) {
        fprintf(stderr, "[HIP] %s: fused layer kernel reported %s\n", who,
                le == 1 ? "a bounded wait that gave up" : "a runtime error");
        return fail(who, hipErrorLaunchFailure);
    }
    if (e == 0) {
        err_mark();
        return true;
    }
    fprintf(stderr, "[HIP] %s: fused MoE reported %s\n", who,
            e == 1 ? "a bounded wait that gave up" : e == 2 ? "an out-of-range expert id" : "a runtime error");
    return fail(who, hipErrorLaunchFailure);
}

// The check on words gathered by err_gather (v[0] the layer kernel's, v[1..2] the MoE's),
// read back with the stream idle; the words that hold a failure are cleared.
static bool stream_err_ok(const char *who, const unsigned long long v[3]) {
    int le = (int)(uint32_t)v[0];
    if (le != 0) {
        const unsigned long long z = 0;
        if (!g_lt.err || hipMemcpy(g_lt.err, &z, 8, hipMemcpyHostToDevice) != hipSuccess) le = -1;
    }
    return err_report(who, le, le != 0 ? 0 : moe_error_settle(v + 1));
}

// The same check reading the words itself (synchronises the device).
static bool stream_moe_ok(const char *who) {
    const int le = layer_error_take();
    return err_report(who, le, le != 0 ? 0 : moe_error_take());
}

// The lm_head launched ahead.  The engine follows stream_end(NULL) with stream_norm_argmax
// on its lm_head (c/qwen.c:1282, 1437-1441).  stream_end issues that call's work (the final
// norm in the GEMV's prologue, the argmax keys, their copy to pinned memory) before it
// waits, with the arguments of the last stream_norm_argmax, so the device goes on from the
// last layer into the lm_head while the host returns and calls again.  stream_norm_argmax
// then only waits and decodes when its arguments are those; otherwise the keys are
// dropped and it runs as usual.  The residual and the final norm weight cannot change in
// between (stream_begin and coli_vk_final_norm_weight drop the launch); a tensor's weights
// stay where they are (the arena frees nothing), and its handle, weights and shape are
// compared.
void coli::stream_tensor_freed(const ColiVkTensor *t) {
    if (t && t == g_ahead.t) g_ahead = AheadArgmax();   // a launch in flight reads arena memory, never freed
}
static bool ahead_match(const ColiVkTensor *t, int fmt, int I, int O, int gs, float eps) {
    return g_ahead.t && t == g_ahead.t && tensor_live(t) && t->w == g_ahead.w && t->layout == kLayoutLanes &&
           t->fmt == fmt && t->I == I && t->O == O && t->gs == gs && fmt == g_ahead.fmt && I == g_ahead.I &&
           O == g_ahead.O && gs == g_ahead.gs && eps == g_ahead.eps;
}
// stream_end's launch of the next stream_norm_argmax (false only on a runtime error)
static bool ahead_launch() {
    g_ahead.pending = false;
    const ColiVkTensor *t = g_ahead.t;
    if (!t || !ahead_match(t, g_ahead.fmt, g_ahead.I, g_ahead.O, g_ahead.gs, g_ahead.eps) || !g_str.d_fnw ||
        g_str.fn_D != t->I || g_str.D != t->I || t->O >= (1 << 24))
        return true;
    if (!host_scratch((void **)&g_str.h_am, &g_str.ham_cap, (kArgSlots + 3) * 8)) return false;
    uint32_t ep;
    unsigned long long *sl;
    if (!gemv_argmax(t, g_str.d_resid, nullptr, stream(), &ep, &sl, g_str.d_fnw, g_ahead.eps) ||
        !pin_copy(g_str.h_am, sl, kArgSlots * 8, stream(), "stream end (lm_head ahead)"))
        return false;
    g_ahead.pending = true;
    g_ahead.ep = ep;
    return true;
}

// stream_end's read-back as one launch into pinned memory: the error words (when checked)
// at the head, then the fused layers' id history from ints kHistHead .. n.
__global__ void stream_out(int *h, const int *dh, int n, const unsigned long long *l, const unsigned long long *m0,
                           const unsigned long long *m1, int chk) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0 && chk) {
        unsigned long long *hw = (unsigned long long *)h;
        hw[0] = l ? __hip_atomic_load(l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        hw[1] = m0 ? __hip_atomic_load(m0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        hw[2] = m1 ? __hip_atomic_load(m1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
    }
    for (int j = kHistHead + i; j < n; j += gridDim.x * blockDim.x) h[j] = dh[j];
}

COLI_API int coli_vk_stream_end(float *x, int D) {
    if (!g_str.live || D != g_str.D) return 0;
    if (!ok()) {   // disabled by an earlier failure: every later call returns 0
        g_str.live = 0;
        g_str.pending = 0;
        return 0;
    }
    // one read-back after the drain: the error words (when a launch could have set one since
    // the last check) and the id history of the fused layers (when pending)
    const bool chk = !err_clean();
    int *dh = hist_dev();
    if (!dh || !host_scratch((void **)&g_str.h_rb, &g_str.hrb_cap, hist_ints() * 4)) return 0;
    const int n = g_str.pending ? kHistHead + g_str.hist_hi * kTopK : 0;
    if (chk || n) {
        const unsigned long long *m0, *m1;
        moe_error_words(&m0, &m1);
        hipLaunchKernelGGL(stream_out, dim3(1), dim3(256), 0, stream(), g_str.h_rb, (const int *)dh, n,
                           (const unsigned long long *)g_lt.err, m0, m1, chk ? 1 : 0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("stream end read-back", e) ? 1 : 0;
    }
    if (!x && !ahead_launch()) return 0;        // the residual stays on the device: the lm_head next
    if (!sync_stream("stream end")) return 0;   // the drain and the read-back
    if (chk && !stream_err_ok("stream end", (const unsigned long long *)g_str.h_rb)) {
        g_str.live = 0;
        g_str.pending = 0;
        return 0;
    }
    if (x && hipMemcpy(x, g_str.d_resid, (size_t)D * 4, hipMemcpyDeviceToHost) != hipSuccess) return 0;
    g_str.live = 0;
    return 1;
}

__global__ void vec_add_kernel(float *r, const float *y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) r[i] = r[i] + y[i];
}

COLI_API int coli_vk_stream_add(const float *y, int D) {
    if (!g_str.live || !y || D != g_str.D) return 0;
    if (!host_scratch((void **)&g_str.h_y, &g_str.hy_cap, (size_t)D * 4) ||
        !scratch((void **)&g_str.d_y, &g_str.dy_cap, (size_t)D * 4))
        return 0;
    memcpy(g_str.h_y, y, (size_t)D * 4);
    const hipError_t e = hipMemcpyAsync(g_str.d_y, g_str.h_y, (size_t)D * 4, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("stream add", e) ? 1 : 0;
    hipLaunchKernelGGL(vec_add_kernel, dim3((D + 255) / 256), dim3(256), 0, stream(), g_str.d_resid, g_str.d_y, D);
    return sync_stream("stream add") ? 1 : 0;
}

// the last non-fused route's nrm (host copy), the expert input of c/qwen.c:936-940
COLI_API const float *coli_vk_stream_nrm(void) { return g_str.live && !g_str.fused_last ? g_str.h_nrm : nullptr; }

COLI_API int coli_vk_stream_copy_resid(float *x, int D) {
    if (!ok() || !x || !g_str.d_resid || D != g_str.D || D < 1) return 0;
    if (!sync_stream("copy resid") || (!err_clean() && !stream_moe_ok("copy resid"))) return 0;
    return hipMemcpy(x, g_str.d_resid, (size_t)D * 4, hipMemcpyDeviceToHost) == hipSuccess ? 1 : 0;
}

// c/backend_vulkan.c:2692-2711
COLI_API int coli_vk_final_norm_weight(const float *w, int D) {
    g_ahead.pending = false;
    if (!ok() || !w || D < 1) return 0;
    if (!scratch((void **)&g_str.d_fnw, &g_str.fnw_cap, (size_t)D * 4)) return 0;
    if (!h2d(g_str.d_fnw, w, (size_t)D * 4, "final norm weight")) return 0;
    g_str.fn_D = D;
    return 1;
}

// c/backend_vulkan.c:2713-2782: final RMSNorm of the device residual + lm_head + argmax,
// only the winner is read back
COLI_API int coli_vk_stream_norm_argmax(ColiVkTensor **tensor, const void *weights, const float *scales, int fmt,
                                        int I, int O, int gs, float eps, int *idx, float *val) {
    if (!ok() || !g_str.d_fnw || g_str.fn_D != I || !g_str.d_resid || g_str.D != I || O < 1 || !idx) return 0;
    if (!coli_vk_tensor_ensure(tensor, weights, scales, fmt, I, O, gs)) return 0;
    const bool ahead = g_ahead.pending && ahead_match(*tensor, fmt, I, O, gs, eps) && err_clean();
    g_ahead.pending = false;
    if (ahead) {   // stream_end launched this call's work: wait for its keys
        int i;
        float v;
        if (!sync_stream("stream_norm_argmax") || !argmax_decode_host(g_str.h_am, g_ahead.ep, &i, &v) || i < 0 ||
            i >= O)
            return 0;
        *idx = i;
        if (val) *val = v;
        return 1;
    }
    if ((*tensor)->layout == kLayoutLanes && O < (1 << 24)) {
        // one launch: the norm in the GEMV's x prologue, argmax keys, and the error words
        // gathered after the keys; the host decodes the keys from the one read-back
        uint32_t ep;
        unsigned long long *sl;
        if (!gemv_argmax(*tensor, g_str.d_resid, nullptr, stream(), &ep, &sl, g_str.d_fnw, eps)) return 0;
        g_ahead = AheadArgmax();   // the arguments for stream_end's next launch ahead
        g_ahead.t = *tensor;
        g_ahead.w = (*tensor)->w;
        g_ahead.fmt = fmt, g_ahead.I = I, g_ahead.O = O, g_ahead.gs = gs, g_ahead.eps = eps;
        const bool chk = !err_clean();
        if (chk && !err_gather_launch(sl + kArgSlots)) return 0;
        if (!host_scratch((void **)&g_str.h_am, &g_str.ham_cap, (kArgSlots + 3) * 8)) return 0;
        unsigned long long *hb = g_str.h_am;
        if (!pin_copy(hb, sl, (kArgSlots + (chk ? 3 : 0)) * 8, stream(), "stream_norm_argmax") ||
            !sync_stream("stream_norm_argmax"))
            return 0;
        if (chk && !stream_err_ok("stream_norm_argmax", hb + kArgSlots)) return 0;
        int i;
        float v;
        if (!argmax_decode_host(hb, ep, &i, &v) || i < 0 || i >= O) return 0;   // the engine's host scan decides
        *idx = i;
        if (val) *val = v;
        return 1;
    }
    // xn [I] | result: 16 ints (idx at 0, value bits at 8) | 3 error words (8-aligned)
    const size_t roff = ((size_t)I * 4 + 7) & ~(size_t)7;
    if (!scratch((void **)&g_str.d_xn, &g_str.xn_cap, roff + 64 + 24)) return 0;
    float *xn = g_str.d_xn;
    int *d_iv = (int *)((uint8_t *)xn + roff);
    unsigned long long *d_err = (unsigned long long *)(d_iv + 16);
    if (!rmsnorm_zc(g_str.d_resid, g_str.d_fnw, xn, I, eps, stream())) return 0;
    TopkOut tk = {1, d_iv, (float *)(d_iv + 8)};
    if (!gemv(*tensor, xn, nullptr, 1, stream(), &tk)) return 0;
    const bool chk = !err_clean();
    if (chk && !err_gather_launch(d_err)) return 0;
    struct {
        int res[16];
        unsigned long long err[3];
    } hb;
    if (!sync_stream("stream_norm_argmax") || hipMemcpy(&hb, d_iv, chk ? sizeof(hb) : 64, hipMemcpyDeviceToHost) != hipSuccess)
        return 0;
    if (chk && !stream_err_ok("stream_norm_argmax", hb.err)) return 0;
    const int *res = hb.res;
    if (res[0] < 0 || res[0] >= O) return 0;   // no valid winner: the engine's host scan decides
    *idx = res[0];
    if (val) memcpy(val, &res[8], 4);
    return 1;
}

COLI_API void coli_vk_route_cache_stats(void) {}
COLI_API void coli_vk_decode_prof(double decode_ms, int tokens) { (void)decode_ms, (void)tokens; }

// After the block: post_ln, then the fused MoE (device expert table) or the device top-k
// read back into idx_out / val_out (and nrm into the host cache for stream_nrm).
static int pipe_tail(int ln_layer, ColiVkTensor *router, int E, int topk, float eps, int *idx_out, float *val_out) {
    float *dn = wbuf(W_NRM, g_str.D), *dl = wbuf(W_LOGIT, (size_t)2 * E + 2 * kMaxK);
    int *dh = hist_dev();
    if (!dn || !dl || !dh || topk < 1 || topk > kTopK || E > kMaxE) return 0;   // device top-k: K <= 8
    if (ln_layer < 0 || ln_layer >= kMaxLayers) return 0;
    // fused: the MoE block norms the residual itself (post_ln) and adds into it
    if (moe_ready(ln_layer) && moe_decode(ln_layer, router, topk, g_str.d_resid, g_str.d_resid, 1,
                                          dh + kHistHead + (size_t)ln_layer * kTopK, nullptr, stream(), g_ln[ln_layer].post_ln,
                                          eps)) {
        g_str.fused_last = 1;
        g_str.pending = 1;
        g_str.hist_K[ln_layer] = topk;
        if (ln_layer >= g_str.hist_hi) g_str.hist_hi = ln_layer + 1;
        return 1;
    }
    if (!ok()) return 0;
    if (router->fmt != 0 && router->fmt != 1) return 0;   // routers are f32 or int8 rows
    if (!route_tail(ln_layer, g_str.d_resid, router, E, topk, eps, dn, dl, stream(), dl + E)) return 0;
    g_str.fused_last = 0;
    int *di = (int *)(dl + 2 * E);
    float *dv = dl + 2 * E + kMaxK;
    hipLaunchKernelGGL(route_row, dim3(1), dim3(64), 0, stream(), dl, dn, router->w, router->sz, router->fmt,
                       router->row_bytes, g_str.D, E, topk, di, dv, moe_cert_all());
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("route launch", e) ? 1 : 0;
    if (!host_scratch((void **)&g_str.h_nrm, &g_str.hnrm_cap, (size_t)(g_str.D + 2 * kMaxK) * 4)) return 0;
    if (!sync_stream("route read-back") ||
        hipMemcpy(g_str.h_nrm, dn, (size_t)g_str.D * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(idx_out, di, (size_t)topk * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(val_out, dv, (size_t)topk * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return 0;
    return 1;
}

COLI_API int coli_vk_gqa_full_route_pipe(int layer, int D, ColiVkTensor *gq_t, ColiVkTensor *gk_t, ColiVkTensor *gv_t,
                                         ColiVkTensor *out_t, ColiVkTensor *router, int ln_layer, int *idx_out,
                                         float *val_out, int topk, int H, int KH, int hd, int rot, int pos_base,
                                         int max_t, float eps, float theta, int Dout, int E) {
    if (!ok() || !g_str.live || D != g_str.D || Dout != D || !ln_ok(ln_layer, D) || !router || router->I != D ||
        router->O != E || !idx_out || !val_out)
        return 0;
    const GqaDims d = {H, KH, hd, rot, max_t, eps, theta};
    if (!gqa_block(layer, g_str.d_resid, g_ln[ln_layer].in_ln, gq_t, gk_t, gv_t, out_t, g_str.d_resid, true, d,
                   pos_base, stream()))
        return 0;
    return pipe_tail(ln_layer, router, E, topk, eps, idx_out, val_out);
}

COLI_API int coli_vk_gdn_full_route_pipe(int layer, int D, ColiVkTensor *gqkv_t, ColiVkTensor *gz_t,
                                         ColiVkTensor *gba_t, ColiVkTensor *gbb_t, ColiVkTensor *out_t,
                                         ColiVkTensor *router, int ln_layer, int *idx_out, float *val_out, int topk,
                                         int KH, int KD, int VH, int VD, int conv_dim, int conv_k, float eps, int Dout,
                                         int E) {
    if (!ok() || !g_str.live || D != g_str.D || Dout != D || !ln_ok(ln_layer, D) || !router || router->I != D ||
        router->O != E || !idx_out || !val_out)
        return 0;
    const GdnDims d = {KH, KD, VH, VD, conv_dim, conv_k, eps};
    if (!gdn_block(layer, g_str.d_resid, g_ln[ln_layer].in_ln, nullptr, gqkv_t, gz_t, gba_t, gbb_t, out_t,
                   g_str.d_resid, true, d, stream()))
        return 0;
    return pipe_tail(ln_layer, router, E, topk, eps, idx_out, val_out);
}

COLI_API int coli_vk_stream_moe_fused(void) { return g_str.live && g_str.fused_last ? 1 : 0; }
COLI_API int coli_vk_stream_ix_pending(void) { return g_str.pending ? 1 : 0; }

// ids of a fused layer of the last stream (valid after stream_end); returns the count
COLI_API int coli_vk_stream_ix_hist(int layer, int *idx_out, int K) {
    if (!g_str.pending || g_str.live || layer < 0 || layer >= kMaxLayers || !idx_out) return 0;
    const int n = g_str.hist_K[layer] < K ? g_str.hist_K[layer] : K;
    for (int k = 0; k < n; k++) idx_out[k] = g_str.h_rb[kHistHead + layer * kTopK + k];
    return n;
}

// Test hook: fused layer launches on (1) or off (0, the separate kernels); returns the
// previous setting.  Both give the same results bit for bit.
COLI_API int coli_hip_layer_fuse(int on) {
    const int prev = fuse_on() ? 1 : 0;
    g_fuse = on ? 1 : 0;
    return prev;
}
