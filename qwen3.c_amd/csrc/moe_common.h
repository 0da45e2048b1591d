// moe_common.h - types and the routing core shared by the decode MoE block (moe.hip)
// and the prefill MoE path (prefill.hip).
#pragma once

#include "fmt6_device.h"

namespace coli {

struct ExpertRec {
    const uint8_t *wg, *wu, *wd;
    const float *sg, *su, *sd;
};

// geometry shared by every expert of a table (fmt 6, lanes layout)
struct MoeGeom {
    int D, I, gs;
    int ngD, ngI;   // groups per gate/up row (over D) and per down row (over I)
    int nlG, nlD;   // lanes with data per gate/up row and per down row
    int rbG, rbD;   // device row bytes of gate/up and of down
};

constexpr int kMaxE = 1024;
constexpr int kMaxSlots = kTopK + 1;      // fused kernel: K <= 8 routed + the shared expert
constexpr int kMoeMaxI = 512;             // expert intermediate size (h staged in LDS)
constexpr int kMaxK = 64;                 // c/backend_vulkan.c:3298 (topk <= 64)

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// wave maximum of a float by DPP (no LDS traffic), broadcast to all lanes
#define COLI_DPP_FMAX(v, ctrl, rmask) \
    fmaxf((v), __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -INFINITY), \
                                                                      __builtin_bit_cast(int, (v)), (ctrl), (rmask), 0xF, false)))
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = COLI_DPP_FMAX(v, 0xB1, 0xF);    // quad_perm [1,0,3,2]
    v = COLI_DPP_FMAX(v, 0x4E, 0xF);    // quad_perm [2,3,0,1]
    v = COLI_DPP_FMAX(v, 0x141, 0xF);   // row_half_mirror
    v = COLI_DPP_FMAX(v, 0x140, 0xF);   // row_mirror
    v = COLI_DPP_FMAX(v, 0x142, 0xA);   // row_bcast15
    v = COLI_DPP_FMAX(v, 0x143, 0xC);   // row_bcast31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

struct RouteLds {
    float p[kMaxE + 64];               // logits in; exp(l - max), zero padded to a multiple of 64
    unsigned long long cand[kMaxE + 8];   // candidates: expert index, then keys (p bits << 24 | 0xFFFFFF - e)
    unsigned hmax[2 * kWaves];         // half-wave maxima of the exp bits
    float red[kWaves];
    float sum, gate, vsum;
    int ncand, tie;
    unsigned long long top[kTopK];     // the first K candidates in rank order
    int idx[kTopK];
    float val[kTopK];
};

// u32 maximum over each half wave (32 lanes): valid in lanes 31 and 63
__device__ __forceinline__ uint32_t half_wave_umax(uint32_t v) {
    v = COLI_DPP_UMAX(v, 0xB1, 0xF);    // quad_perm [1,0,3,2]
    v = COLI_DPP_UMAX(v, 0x4E, 0xF);    // quad_perm [2,3,0,1]
    v = COLI_DPP_UMAX(v, 0x141, 0xF);   // row_half_mirror
    v = COLI_DPP_UMAX(v, 0x140, 0xF);   // row_mirror: every lane holds its row's max
    v = COLI_DPP_UMAX(v, 0x142, 0xA);   // row_bcast15: rows 1 and 3 take rows 0 and 2
    return v;
}

__device__ __forceinline__ float wave_sum_dppf(float v) {
    v = seg_sum<64>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Routing of one token on the block (kThreads threads): R.p[0, E) holds the router
// logits.  c/qwen.c:332-336 softmax_row (max from -1e30, e = expf(l - max), s = sequential
// sum of e in index order, p = e / s), :807-817 the K greedy picks (strict '>' from the
// lowest index: the order (p desc, index asc)) and the renorm in rank order.  Leaves the
// picks in R.idx / R.val (rank order, val = p) and the renorm sum in R.vsum.
//
// p = fl(e / s) is monotone in e, so the order (e desc, index asc) is the reference's
// order (p desc, index asc) unless two distinct e round to the same p; that needs them
// within 2^-21 relative.  Candidates: the 8 half-wave maxima of e are 8 distinct experts,
// so with theta the least of them every expert that can reach the K-th p has
// e >= theta (1 - 2^-21).  They are ranked by (e desc, index asc).  A group of equal p is
// a run of that order; if it holds distinct e, two neighbours in the run are distinct and
// within 2^-21, so when any candidate and its successor are, the exact path runs: the
// sequential sum s of the reference and a re-rank by (p desc, index asc).  Otherwise the
// e order is the reference's and p = e / s with s from a parallel sum (it only scales the
// weights: relative error ~1e-7 against the reference's).  Starts and ends with
// __syncthreads().
__device__ inline void route_select(RouteLds &R, int E, int K) {
    constexpr int kPer = kMaxE / kThreads;   // experts per thread
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Epad = (E + 63) & ~63;
    __syncthreads();
    float lv[kPer];
    float m = -1e30f;   // the reference's initial max
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = tid + q * kThreads;
        lv[q] = e < E ? R.p[e] : -INFINITY;
        m = fmaxf(m, lv[q]);
    }
    m = wave_max_dpp(m);
    if (lane == 0) R.red[wave] = m;
    if (tid == 0) {
        R.ncand = 0;
        R.tie = 0;
    }
    __syncthreads();
    m = R.red[0];
#pragma unroll
    for (int w = 1; w < kWaves; w++) m = fmaxf(m, R.red[w]);
    uint32_t mx = 0u;
    float ps = 0.f;   // parallel partial sum
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = tid + q * kThreads;
        if (e < Epad) {
            const float ev = e < E ? expf(lv[q] - m) : 0.f;
            R.p[e] = ev;
            ps += ev;
            mx = max(mx, __float_as_uint(ev));   // ev >= 0: the bits order like the values
        }
    }
    ps = wave_sum_dppf(ps);
    mx = half_wave_umax(mx);
    if (lane == 31 || lane == 63) R.hmax[2 * wave + (lane >> 5)] = mx;
    __syncthreads();   // R.red is free again: reuse it for the partial sums
    if (lane == 0) R.red[wave] = ps;
    uint32_t theta = R.hmax[0];
#pragma unroll
    for (int i = 1; i < 2 * kWaves; i++) theta = min(theta, R.hmax[i]);
    const float lo = __uint_as_float(theta) * (1.f - 0x1p-21f);
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = tid + q * kThreads;
        if (e < E && R.p[e] >= lo) R.cand[atomicAdd(&R.ncand, 1)] = (unsigned long long)e;
    }
    __syncthreads();
    const int nc = R.ncand, nc8 = (nc + 7) & ~7;
    for (int c = tid; c < nc8; c += kThreads) {   // keys by e; zeros pad to a multiple of 8
        unsigned long long k = 0ull;
        if (c < nc) {
            const int e = (int)R.cand[c];
            k = ((unsigned long long)__float_as_uint(R.p[e]) << 24) | (0xFFFFFFu - (uint32_t)e);
        }
        R.cand[c] = k;
    }
    if (tid == 0) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) s += R.red[w];
        R.sum = s;
    }
    __syncthreads();
    // rank by counting (keys are unique); the first K go to R.top.  Each candidate also
    // finds its successor in that order (the largest key below its own): distinct but close
    // e there may round to one p, and then the exact path decides.
    for (int c = tid; c < nc; c += kThreads) {
        const unsigned long long me = R.cand[c];
        int rank = 0;
        unsigned long long succ = 0ull;
        for (int o0 = 0; o0 < nc8; o0 += 8) {   // 8 broadcast reads in flight, no conditions
            unsigned long long o8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) o8[u] = R.cand[o0 + u];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                rank += o8[u] > me ? 1 : 0;
                succ = o8[u] < me && o8[u] > succ ? o8[u] : succ;
            }
        }
        if (rank < K) R.top[rank] = me;
        const float a = __uint_as_float((uint32_t)(me >> 24)), b = __uint_as_float((uint32_t)(succ >> 24));
        if (succ && b < a && b >= a * (1.f - 0x1p-21f)) R.tie = 1;
    }
    __syncthreads();
    if (R.tie) {   // exact: the reference's sequential sum, then (p desc, index asc)
        if (tid == 0) {
            float s = 0.f;
            for (int e0 = 0; e0 < Epad; e0 += 64) {
                float4 v[16];
#pragma unroll
                for (int c = 0; c < 16; c++) v[c] = *(const float4 *)&R.p[e0 + 4 * c];
#pragma unroll
                for (int c = 0; c < 16; c++) {
                    s += v[c].x;
                    s += v[c].y;
                    s += v[c].z;
                    s += v[c].w;
                }
            }
            R.sum = s;
        }
        __syncthreads();
        const float s = R.sum;
        for (int c = tid; c < nc; c += kThreads) {
            const int e = (int)(0xFFFFFFu - (uint32_t)(R.cand[c] & 0xFFFFFFu));
            R.cand[c] = ((unsigned long long)__float_as_uint(R.p[e] / s) << 24) | (0xFFFFFFu - (uint32_t)e);
        }
        __syncthreads();
        for (int c = tid; c < nc; c += kThreads) {
            const unsigned long long me = R.cand[c];
            int rank = 0;
            for (int o0 = 0; o0 < nc8; o0 += 8) {
                unsigned long long o8[8];
#pragma unroll
                for (int u = 0; u < 8; u++) o8[u] = R.cand[o0 + u];
#pragma unroll
                for (int u = 0; u < 8; u++) rank += o8[u] > me ? 1 : 0;
            }
            if (rank < K) R.top[rank] = me;
        }
        __syncthreads();
        if (tid < K) {
            const unsigned long long me = R.top[tid];
            R.idx[tid] = (int)(0xFFFFFFu - (uint32_t)(me & 0xFFFFFFu));
            R.val[tid] = __uint_as_float((uint32_t)(me >> 24));
        }
    } else if (tid < K) {
        const unsigned long long me = R.top[tid];
        const int e = (int)(0xFFFFFFu - (uint32_t)(me & 0xFFFFFFu));
        R.idx[tid] = e;
        R.val[tid] = R.p[e] / R.sum;
    }
    __syncthreads();
    if (tid == 0) {   // the renorm sum in rank order (c/qwen.c:816; trailing +0 leaves it unchanged)
        float v8[kTopK], sm = 0.f;
#pragma unroll
        for (int j = 0; j < kTopK; j++) v8[j] = j < K ? R.val[j] : 0.f;
#pragma unroll
        for (int j = 0; j < kTopK; j++) sm += v8[j];
        R.vsum = sm;
    }
    __syncthreads();
}

// the expert table of a layer (moe.hip): false if it is not complete
bool moe_layer(int layer, const ExpertRec **d_rec, const float **d_shgate, MoeGeom *geom, int *E);

}  // namespace coli
