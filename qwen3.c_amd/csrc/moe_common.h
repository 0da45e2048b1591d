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

struct RouteLds {
    float p[kMaxE + 64];               // probabilities, zero padded to a multiple of 64
    unsigned long long cand[kMaxE];    // candidate keys (p bits << 24 | 0xFFFFFF - e)
    unsigned hmax[2 * kWaves];         // half-wave maxima of the p bits
    float red[kWaves];
    float sum, gate, vsum;
    int ncand;
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

// Routing of one token on the block (kThreads threads): R.p[0, E) holds the router
// logits.  c/qwen.c:332-336 softmax_row (max from -1e30, expf, sequential sum in index
// order, divide), :807-817 the K greedy picks (strict '>' from the lowest index: the order
// (p desc, index asc)) and the renorm sum in rank order.  Leaves p in R.p, the picks in
// R.idx / R.val (rank order) and the renorm sum in R.vsum.  Starts and ends with
// __syncthreads().
__device__ inline void route_select(RouteLds &R, int E, int K) {
    constexpr int kPer = kMaxE / kThreads;   // experts per thread
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Epad = (E + 63) & ~63;
    __syncthreads();
    float m = -1e30f;   // the reference's initial max
    for (int e = tid; e < E; e += kThreads) m = fmaxf(m, R.p[e]);
    if (tid == 0) R.ncand = 0;
    m = wave_max_f(m);
    if (lane == 0) R.red[wave] = m;
    __syncthreads();
    m = R.red[0];
#pragma unroll
    for (int w = 1; w < kWaves; w++) m = fmaxf(m, R.red[w]);
    for (int e = tid; e < Epad; e += kThreads) R.p[e] = e < E ? expf(R.p[e] - m) : 0.f;
    __syncthreads();
    if (tid == 0) {   // sequential sum in index order, as the reference (the padding adds 0)
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
    uint32_t pb[kPer], mx = 0u;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = tid + q * kThreads;
        pb[q] = 0u;
        if (e < E) {
            const float pv = R.p[e] / s;
            R.p[e] = pv;
            pb[q] = __float_as_uint(pv);   // p >= 0: the bits order like the values
            mx = max(mx, pb[q]);
        }
    }
    // Candidates: p >= theta = the least of the 8 half-wave maxima.  Those maxima are 8
    // distinct experts with p >= theta, so the K <= 8 best (p desc, index asc) and every
    // expert tied with the K-th are candidates.
    mx = half_wave_umax(mx);
    if (lane == 31 || lane == 63) R.hmax[2 * wave + (lane >> 5)] = mx;
    __syncthreads();
    uint32_t theta = R.hmax[0];
#pragma unroll
    for (int i = 1; i < 2 * kWaves; i++) theta = min(theta, R.hmax[i]);
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = tid + q * kThreads;
        if (e < E && pb[q] >= theta)
            R.cand[atomicAdd(&R.ncand, 1)] = ((unsigned long long)pb[q] << 24) | (0xFFFFFFu - (uint32_t)e);
    }
    __syncthreads();
    // rank among the candidates: (p desc, index asc) is the order of the reference's strict
    // '>' scan from the lowest index (c/qwen.c:810-815)
    const int nc = R.ncand;
    for (int c = tid; c < nc; c += kThreads) {
        const unsigned long long me = R.cand[c];
        int rank = 0;
        for (int o0 = 0; o0 < nc; o0 += 8) {   // 8 LDS reads in flight
            unsigned long long o8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) o8[u] = o0 + u < nc ? R.cand[o0 + u] : 0ull;
#pragma unroll
            for (int u = 0; u < 8; u++) rank += o8[u] > me ? 1 : 0;
        }
        if (rank < K) {
            R.idx[rank] = (int)(0xFFFFFFu - (uint32_t)(me & 0xFFFFFFu));
            R.val[rank] = __uint_as_float((uint32_t)(me >> 24));
        }
    }
    __syncthreads();
    // renorm (c/qwen.c:816-817): the sum in rank order
    if (tid == 0) {   // the renorm sum in rank order (trailing +0 leaves it unchanged)
        float v8[kTopK], sm = 0.f;
#pragma unroll
        for (int j = 0; j < kTopK; j++) v8[j] = j < K ? R.val[j] : 0.f;
#pragma unroll
        for (int j = 0; j < kTopK; j++) sm += v8[j];
        R.vsum = sm;
    }
    __syncthreads();
    if (tid == 0) {   // the renorm sum in rank order (trailing +0 leaves it unchanged)
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
