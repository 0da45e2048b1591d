// moe_common.h - types and the routing core shared by the decode MoE block (moe.hip)
// and the prefill MoE path (prefill.hip).
#pragma once

#include "fmt6_device.h"

namespace coli {

struct ExpertRec {
    const uint8_t *wg, *wu, *wd;
    const float *sg, *su, *sd;
};

// A unit of the host-routed expert group on MFMA: <= 32 consecutive positions (rows of h
// and y) of one expert.
struct PfUnit {
    ExpertRec rec;
    int pos0, n, pad[2];
};

// geometry shared by every expert of a table (fmt 6, lanes layout)
struct MoeGeom {
    int D, I, gs;
    int ngD, ngI;   // groups per gate/up row (over D) and per down row (over I)
    int nlG, nlD;   // lanes with data per gate/up row and per down row
    int rbG, rbD;   // device row bytes of gate/up and of down
};

// The host-routed expert group (coli_vk_expert_group_issue{,_id} with rows > 1) on the
// prefill MFMA kernels (prefill.hip): nunits units over P positions, position p taking x
// row xrow[p] of d_x [Sx][D]; y [P][D].  key != 0 names the contents of d_x: the digit
// planes of the last call with the same (d_x, Sx, key) are reused.  eg_unit_rows: the
// positions per unit (32, or 16 when 32-row units would leave the CUs short of blocks).
bool eg_mfma_ok(const MoeGeom &m);
int eg_unit_rows(int count, const int *rows, const MoeGeom &m);
bool eg_mfma(const PfUnit *d_units, int nunits, const int *d_xrow, int P, const MoeGeom &m, const float *d_x, int Sx,
             uint64_t key, float *d_y, hipStream_t st);

// The resident expert table (moe.hip): would slot (layer, eid) take these tensors (no
// change made; *out their geometry), and are (layer, E, D, I, gs) within the table's shape.
bool eg_table_check(int layer, int eid, const ColiVkTensor *g, const ColiVkTensor *u, const ColiVkTensor *d,
                    MoeGeom *out);
bool eg_table_dims(int layer, int E, int D, int I, int gs);

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
    float red[kWaves], bred[kWaves];
    float sum, gate, vsum;
    int ncand, tie;
    unsigned long long top[kTopK];     // the first K candidates in rank order
    int idx[kTopK];
    float val[kTopK];
    // certification (route_wave with bounds): the candidates by rank, their expert ids and
    // logit intervals [lo, hi]; the lowest pick's lower end; 1 if a decision is ambiguous
    int cid[kMaxE + 8];
    float clo[kMaxE + 8], chi[kMaxE + 8];
    float thr;
    int amb;
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

constexpr int kPollLimit = 1 << 16;       // bounded polls (each ~0.3-2 us)

// ---------------------------------------------------------------- tagged words
__device__ __forceinline__ unsigned long long aload(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tag_put(unsigned long long *p, uint32_t epoch, float v) {
    __hip_atomic_store(p, ((unsigned long long)epoch << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// The error word holds (epoch << 32) | code of a launch that failed (code 1: a bounded wait
// gave up, 2: a route held an out-of-range expert id).  A wait gives up past kPollLimit
// polls, or at its 16th poll once its own launch has failed; the word is read on every 16th
// poll only (each read is one more memory round trip between a poll and the next).  The
// epoch stamp means no launch has to clear the word: an earlier launch's failure never
// matches.
__device__ __forceinline__ void err_set(unsigned long long *err, uint32_t epoch, int code) {
    __hip_atomic_store(err, ((unsigned long long)epoch << 32) | (uint32_t)code, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool poll_give_up(unsigned long long *err, uint32_t epoch, int polls) {
    if (polls > kPollLimit ||
        ((polls & 15) == 15 &&
         (uint32_t)(__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 32) == epoch)) {
        err_set(err, epoch, 1);
        return true;
    }
    if (polls < 8) __builtin_amdgcn_s_sleep(1);   // back off: the line may be in demand
    else __builtin_amdgcn_s_sleep(8);
    return false;
}

// ---------------------------------------------------------------- certified routing
// The reference computes a router logit as a sequential fp32 sum of rounded products
// (c/qwen.c:178-189; int8 rows :230-238, acc * scale after the sum).  The device's logit L
// is the exact dot rounded once (fp64 accumulation of exact products), and B bounds
// |L - l_ref| rigorously (running-error analysis of recursive summation, Higham 2002,
// "Accuracy and Stability of Numerical Algorithms", sec. 4.2): with u = 2^-24, exact
// products p_i, exact prefix sums S_k and A = sum |p_i|,
//   |l_ref - sum p_i| <= s (u sum_k |S_k| + u A (1 + u + n gamma_n))      (s: int8 row scale, else 1)
// and |L - sum p_i s| <= 3.2 u |L| (two roundings).  sum_k |S_k| is bounded from above per
// block of 4 columns: |S_k| <= |S_b| + (sum of the block's |p|), S_b the prefix before the
// block, computed in fp32 (its rounding, < 32 n u A over all blocks, is added).  A routing
// decision between experts whose intervals [L - B, L + B] do not overlap is the
// reference's; route_certify_wave recomputes l_ref exactly for every candidate whose
// interval meets the decision boundary.
__device__ __forceinline__ float router_bound(float L, float sum_abs_prefix, float A, int n, float scale) {
    const float u = 0x1p-24f, nu = (float)n * u;
    const float gam = nu / (1.f - nu);
    const float sum = sum_abs_prefix + A * (2.f + u + (float)n * gam + 32.f * nu);
    return (scale * u * sum + 3.2f * u * fabsf(L)) * (1.f + 0x1p-12f) + 0x1p-126f;
}
// The same bound with sum_k |S_k| <= sum_k sum_{i<=k} |p_i| = sum_i (n - i) |p_i| (no prefix
// sums: the router has it when L is ready; about 20x looser).  wsum = sum_i (n - i) |p_i|
// bounded from above per block of 4 columns by (n - first column) * (the block's sum |p|).

// Inclusive prefix sum over the wave (lane order), fp32, by DPP: row_shr 1/2/4/8 within
// rows of 16, then row_bcast15 / row_bcast31 across rows.
__device__ __forceinline__ float wave_scan_incl(float v) {
#define COLI_SCAN_STEP(ctrl, rmask) \
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), (ctrl), (rmask), 0xF, false))
    COLI_SCAN_STEP(0x111, 0xF);   // row_shr:1
    COLI_SCAN_STEP(0x112, 0xF);   // row_shr:2
    COLI_SCAN_STEP(0x114, 0xF);   // row_shr:4
    COLI_SCAN_STEP(0x118, 0xF);   // row_shr:8
    COLI_SCAN_STEP(0x142, 0xA);   // row_bcast15 -> rows 1, 3
    COLI_SCAN_STEP(0x143, 0xC);   // row_bcast31 -> rows 2, 3
#undef COLI_SCAN_STEP
    return v;
}

// One router row on one wave: L (exact dot rounded to fp32, times the int8 row scale) and
// its bound B.  The row and x are read in passes of 2048 columns, lane l holding columns
// c0 + 4 (l + 64 c) .. + 3 for c < 8.  rload(c0, w) fills the lane's 8 float4 weights of a
// pass (int8 rows converted), xload(c0, xq) its 8 float4 x values; the first pass's weights
// may be loaded by the caller before (prefetch), pass `w0_loaded`.  publish(L, Bc) is called
// (on every lane) with the crude bound Bc before the prefix sums of the tight bound (the
// return value) are computed, so a consumer waiting for L is not delayed by them.
constexpr int kRouterRC = 8;
template <typename RLoad, typename XLoad, typename Publish>
__device__ __forceinline__ float router_row(int D, float scale, bool int8, float4 (&w)[kRouterRC], bool w0_loaded,
                                            RLoad rload, XLoad xload, Publish publish) {
    constexpr int kPass = kRouterRC * 256, kMaxPass = (kLaneMaxI + kPass - 1) / kPass;
    const int lane = threadIdx.x & 63;
    double acc = 0.0;
    float T[kMaxPass][kRouterRC];   // per chunk: the lane's 4-column sum of products (fp32)
    float A = 0.f;                  // the lane's sum of |p|
    float Wt = 0.f;                 // the lane's sum of (n - i) |p_i| (blocks of 4 from above)
    float4 xq[kRouterRC];
    // fp32 estimates for the bound (their rounding is covered by its slack terms)
    auto terms = [&](int ps) {
#pragma unroll
        for (int c = 0; c < kRouterRC; c++)
            T[ps][c] = fmaf(xq[c].w, w[c].w, fmaf(xq[c].z, w[c].z, fmaf(xq[c].y, w[c].y, xq[c].x * w[c].x)));
    };
    const int np = (D + kPass - 1) / kPass;
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ps++) {
        if (ps >= np) break;
        const int c0 = ps * kPass;
        if (c0 || !w0_loaded) rload(c0, w);
        xload(c0, xq);
#pragma unroll
        for (int c = 0; c < kRouterRC; c++) {
            acc = fma((double)xq[c].x, (double)w[c].x, acc);
            acc = fma((double)xq[c].y, (double)w[c].y, acc);
            acc = fma((double)xq[c].z, (double)w[c].z, acc);
            acc = fma((double)xq[c].w, (double)w[c].w, acc);
            const float a = fmaf(fabsf(xq[c].w), fabsf(w[c].w),
                                 fmaf(fabsf(xq[c].z), fabsf(w[c].z),
                                      fmaf(fabsf(xq[c].y), fabsf(w[c].y), fabsf(xq[c].x) * fabsf(w[c].x))));
            A += a;
            Wt = fmaf((float)(D - (c0 + 4 * (lane + 64 * c))), a, Wt);
        }
        if (ps + 1 < np) terms(ps);   // the last pass's terms after the logit is out
    }
    acc = wave_sum_dpp(acc);
    float L = (float)acc;
    if (int8) L *= scale;   // c/qwen.c:237: acc * scale[o]
    A = wave_sum_dppf(A);
    publish(L, router_bound(L, wave_sum_dppf(Wt), A, D, int8 ? scale : 1.f));
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ps++)
        if (ps == np - 1) terms(ps);
    // prefix before each lane block: the chunk scans are independent, then the chunk bases
    float inc[kMaxPass][kRouterRC];
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ps++)
#pragma unroll
        for (int c = 0; c < kRouterRC; c++) inc[ps][c] = ps < np ? wave_scan_incl(T[ps][c]) : 0.f;
    float base = 0.f, pre = 0.f;   // prefix before the chunk; sum over blocks of |S_b|
#pragma unroll
    for (int ps = 0; ps < kMaxPass; ps++)
#pragma unroll
        for (int c = 0; c < kRouterRC; c++) {
            if (ps >= np) continue;
            pre += fabsf(base + (inc[ps][c] - T[ps][c]));
            base += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inc[ps][c]), 63));
        }
    pre = 4.f * wave_sum_dppf(pre);
    return router_bound(L, pre + 4.f * A, A, D, int8 ? scale : 1.f);
}

struct CertLds {
    float l[kMaxE], b[kMaxE];                      // device logits and their bounds
    __attribute__((aligned(16))) float x[kLaneMaxI];   // the router's input row (exact path only)
};

// ---------------------------------------------------------------- routing on one wave
// Orders this wave's LDS accesses for the compiler: a wave's LDS operations complete in
// issue order, so what a lane writes is visible to the wave's later reads.
__device__ __forceinline__ void wave_lds_order() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ float wave_min_dpp(float v) { return -wave_max_dpp(-v); }

// Maximum over each aligned run of 8 lanes, in every lane of the run (all lanes active).
__device__ __forceinline__ uint32_t run8_umax(uint32_t v) {
    v = COLI_DPP_UMAX(v, 0xB1, 0xF);    // quad_perm [1,0,3,2]
    v = COLI_DPP_UMAX(v, 0x4E, 0xF);    // quad_perm [2,3,0,1]
    v = COLI_DPP_UMAX(v, 0x141, 0xF);   // row_half_mirror
    return v;
}

// The certainty check over the candidates by rank (R.clo / R.chi, nc of them, the first K
// the picks): 1 when two consecutive picks' intervals meet or a later candidate's interval
// reaches the lowest pick's lower end (*thr).  One wave.
__device__ __forceinline__ int cert_check(const RouteLds &R, int K, int nc, float *thr) {
    const int lane = threadIdx.x & 63;
    float t = INFINITY;
    for (int r = lane; r < K; r += 64) t = fminf(t, R.clo[r]);
    *thr = wave_min_dpp(t);
    bool a = false;
    for (int r = lane; r < nc; r += 64) {
        if (r >= 1 && r < K) a |= !(R.clo[r - 1] > R.chi[r]);
        if (r >= K) a |= R.chi[r] >= *thr;
    }
    return __ballot(a) != 0ull;
}

__device__ __forceinline__ int key_expert(unsigned long long k) { return (int)(0xFFFFFFu - (uint32_t)(k & 0xFFFFFFu)); }
__device__ __forceinline__ float key_value(unsigned long long k) { return __uint_as_float((uint32_t)(k >> 24)); }

// Rank of key `me` among keys[0, n8) (n8 a multiple of 8, zero padded; keys unique).
__device__ __forceinline__ int key_rank(const unsigned long long *keys, int n8, unsigned long long me) {
    int rank = 0;
    for (int o0 = 0; o0 < n8; o0 += 8) {   // 8 broadcast reads in flight, no conditions
        unsigned long long o8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) o8[u] = keys[o0 + u];
#pragma unroll
        for (int u = 0; u < 8; u++) rank += o8[u] > me ? 1 : 0;
    }
    return rank;
}

// Routing of one token by ONE wave (no block barriers; the block's other waves may do
// other work or exit).  R.p[0, E) holds the router logits.  c/qwen.c:332-336 softmax_row
// (max from -1e30, e = expf(l - max), s = sequential sum of e in index order, p = e / s),
// :807-817 the K greedy picks (strict '>' from the lowest index: the order (p desc, index
// asc)) and the renorm in rank order.  Leaves the picks in R.idx / R.val (rank order,
// val = p), the renorm sum in R.vsum, e in R.p and s in R.sum.
//
// p = fl(e / s) is monotone in e, so the order (e desc, index asc) is the reference's order
// (p desc, index asc) unless two distinct e round to the same p; that needs them within
// 2^-21 relative.  Candidates: each aligned run of 8 lanes holds 8 kMaxE / 64 experts; the
// 8 runs' maxima of e are 8 distinct experts, so with theta the least of them every expert
// that can reach the K-th p has e >= theta (1 - 2^-21).  They are ranked by (e desc, index
// asc).  A group of equal p is a run of that order; if it holds distinct e, two neighbours
// in the run are distinct and within 2^-21, so when any candidate and its successor are,
// the exact path runs: the reference's sequential sum s and a re-rank by (p desc, index
// asc).  Otherwise the e order is the reference's and p = e / s with s from a parallel sum
// (it only scales the weights: relative error ~1e-7 against the reference's).
//
// With bounds (lg, bd: LDS arrays of the device logits and of bounds on their distance to
// the reference's logits, router_row) the candidate set widens to every expert whose
// interval [l - b, l + b] can reach a pick's (e >= theta (1 - 2 Bmax - 2^-19), Bmax the
// largest bound: exp(-2 Bmax) >= 1 - 2 Bmax), and R.amb = 1 when two consecutive picks'
// intervals meet or another candidate's interval reaches the lowest pick's lower end
// (R.thr): then route_certify_wave decides with the reference's logits.  The candidates
// by rank go to R.cid / R.clo / R.chi.
// Where route_wave publishes its provisional picks: the K expert ids by (e desc, index asc),
// before the exact tie path and the certification may change them, as tagged words
// w[c * stride + k] for copies c < reps.  w == nullptr: none.
struct RouteProv {
    unsigned long long *w;
    int stride, reps;
    uint32_t epoch;
};

template <int kPer>   // experts per lane: E <= 64 kPer
__device__ __forceinline__ void route_wave_n(RouteLds &R, int E, int K, const float *lg, const float *bd,
                                             const RouteProv &pv) {
    const int lane = threadIdx.x & 63;
    float ev[kPer];
    float m = -1e30f;   // the reference's initial max
    float bm = 0.f;     // largest bound
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = lane + 64 * q;
        ev[q] = e < E ? R.p[e] : -INFINITY;
        m = fmaxf(m, ev[q]);
        if (bd && e < E) bm = fmaxf(bm, bd[e]);
    }
    m = wave_max_dpp(m);
    if (bd) bm = wave_max_dpp(bm);
    float ps = 0.f;     // parallel partial sum
    uint32_t gm = 0u;   // the lane's largest e (bits order like the values: e >= 0)
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = lane + 64 * q;
        ev[q] = e < E ? expf(ev[q] - m) : 0.f;
        if (e < E) R.p[e] = ev[q];
        ps += ev[q];
        gm = max(gm, __float_as_uint(ev[q]));
    }
    const float s = wave_sum_dppf(ps);
    gm = run8_umax(gm);   // the maximum of the lane's run of 8
    uint32_t theta = 0xFFFFFFFFu;
#pragma unroll
    for (int g = 0; g < 8; g++) theta = min(theta, (uint32_t)__builtin_amdgcn_readlane((int)gm, 8 * g));
    const float lo = __uint_as_float(theta) * (bd ? fmaxf(0.f, 1.f - 2.f * bm - 0x1p-19f) : 1.f - 0x1p-21f);
    // candidates: compacted into R.cand as keys (e bits << 24 | 0xFFFFFF - index)
    int nc = 0;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = lane + 64 * q;
        const bool f = e < E && ev[q] >= lo;
        const unsigned long long mk = __ballot(f);
        if (f) {
            const int pos = nc + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
            R.cand[pos] = ((unsigned long long)__float_as_uint(ev[q]) << 24) | (0xFFFFFFu - (uint32_t)e);
        }
        nc += __popcll(mk);
    }
    const int nc8 = (nc + 7) & ~7;
    if (nc + lane < nc8) R.cand[nc + lane] = 0ull;   // pad to a multiple of 8 (zero is below every key)
    wave_lds_order();
    // rank by counting; the first K go to R.top, every candidate's expert to R.cid by rank
    for (int c = lane; c < nc; c += 64) {
        const unsigned long long me = R.cand[c];
        const int rank = key_rank(R.cand, nc8, me);
        if (rank < K) R.top[rank] = me;
        R.cid[rank] = key_expert(me);
    }
    wave_lds_order();
    if (pv.w)   // nc >= 8 >= K: R.top[0, K) is filled
        for (int q = lane; q < pv.reps * K; q += 64)
            tag_put(pv.w + (size_t)(q / K) * pv.stride + q % K, pv.epoch, __int_as_float(key_expert(R.top[q % K])));
    // Two candidates of consecutive ranks that are distinct but within 2^-21 may share their
    // p: then the exact path decides.  Their logit intervals by rank for the certification.
    bool tie = false;
    for (int r = lane; r < nc; r += 64) {
        const int e = R.cid[r];
        if (r + 1 < nc) {
            const float a = R.p[e], b = R.p[R.cid[r + 1]];
            tie |= b < a && b >= a * (1.f - 0x1p-21f);
        }
        if (bd) {
            R.clo[r] = lg[e] - bd[e];
            R.chi[r] = lg[e] + bd[e];
        }
    }
    wave_lds_order();
    int amb = 0;
    float thr = -INFINITY;
    if (bd) amb = cert_check(R, K, nc, &thr);
    float sum = s;
    if (__ballot(tie)) {   // exact: the reference's sequential sum, then (p desc, index asc)
        float ss = 0.f;
        if (lane == 0)
            for (int e = 0; e < E; e++) ss += R.p[e];
        sum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 0));
        for (int c = lane; c < nc; c += 64) {
            const int e = key_expert(R.cand[c]);
            R.cand[c] = ((unsigned long long)__float_as_uint(R.p[e] / sum) << 24) | (0xFFFFFFu - (uint32_t)e);
        }
        wave_lds_order();
        for (int c = lane; c < nc; c += 64) {
            const unsigned long long me = R.cand[c];
            const int rank = key_rank(R.cand, nc8, me);
            if (rank < K) R.top[rank] = me;
        }
        wave_lds_order();
        if (lane < K) {
            const unsigned long long me = R.top[lane];
            R.idx[lane] = key_expert(me);
            R.val[lane] = key_value(me);
        }
    } else if (lane < K) {
        const unsigned long long me = R.top[lane];
        R.idx[lane] = key_expert(me);
        R.val[lane] = key_value(me) / sum;
    }
    wave_lds_order();
    if (lane == 0) {   // the renorm sum in rank order (c/qwen.c:816)
        float sm = 0.f;
        for (int j = 0; j < K; j++) sm += R.val[j];
        R.vsum = sm;
        R.sum = sum;
        R.ncand = nc;
        R.amb = amb;
        R.thr = thr;
    }
    wave_lds_order();
}

// route_wave_n for the number of experts per lane that E needs (E <= kMaxE)
__device__ __forceinline__ void route_wave(RouteLds &R, int E, int K, const float *lg = nullptr, const float *bd = nullptr,
                                           const RouteProv &pv = RouteProv{nullptr, 0, 0, 0u}) {
    if (E <= 256) route_wave_n<4>(R, E, K, lg, bd, pv);
    else if (E <= 512) route_wave_n<8>(R, E, K, lg, bd, pv);
    else route_wave_n<16>(R, E, K, lg, bd, pv);
}

// The router's input row into LDS by one wave, bit for bit what the block form stage_input
// (moe.hip, norm_apply over XRegs) stages: x itself, or the zero-centred RMSNorm of x with
// weight xw (c/qwen.c:326-330).  The block form's thread t sums the squares of its words
// t + kThreads k (8 columns each, k ascending), per wave by wave_sum_dpp, then the 4 wave
// sums in order; lane l here plays threads l + 64 w of the 4 waves w, so every addition
// happens in the same order.  All loads are issued before the first use.
__device__ __forceinline__ void stage_input_wave(const float *x, const float *xw, int D, float eps, float *xn) {
    const int lane = threadIdx.x & 63;
    if (!xw) {
        for (int i = lane; i < D; i += 64) xn[i] = x[i];
        wave_lds_order();
        return;
    }
    constexpr int kW = XRegs::kWords;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(x), (short)0, D * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(xw), (short)0, D * 4, 0x00020000);
    // x: the squares summed, x kept in xn; then the norm weights (two round trips, few registers)
    double ws[kWaves];
    {
        float xv[kWaves][kW][8];
#pragma unroll
        for (int w = 0; w < kWaves; w++)
#pragma unroll
            for (int k = 0; k < kW; k++) {
                const int wd = lane + 64 * w + kThreads * k;
                load8f(rx, wd < D / 8 ? wd * 32 : (int)0x80000000, xv[w][k]);
            }
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            double ss = 0;
#pragma unroll
            for (int k = 0; k < kW; k++) {
#pragma unroll
                for (int c = 0; c < 8; c++) ss += (double)xv[w][k][c] * xv[w][k][c];   // zeros past D add 0
                const int wd = lane + 64 * w + kThreads * k;
                if (wd < D / 8) {   // xn: 16-byte aligned
                    *(float4 *)(xn + 8 * wd) = make_float4(xv[w][k][0], xv[w][k][1], xv[w][k][2], xv[w][k][3]);
                    *(float4 *)(xn + 8 * wd + 4) = make_float4(xv[w][k][4], xv[w][k][5], xv[w][k][6], xv[w][k][7]);
                }
            }
            ws[w] = wave_sum_dpp(ss);
        }
    }
    double t = 0;
#pragma unroll
    for (int w = 0; w < kWaves; w++) t += ws[w];
    const float rs = 1.f / sqrtf((float)(t / D) + eps);
    float wv[kWaves][kW][8];
#pragma unroll
    for (int w = 0; w < kWaves; w++)
#pragma unroll
        for (int k = 0; k < kW; k++) {
            const int wd = lane + 64 * w + kThreads * k;
            load8f(rw, wd < D / 8 ? wd * 32 : (int)0x80000000, wv[w][k]);
        }
    wave_lds_order();
#pragma unroll
    for (int w = 0; w < kWaves; w++)
#pragma unroll
        for (int k = 0; k < kW; k++) {
            const int wd = lane + 64 * w + kThreads * k;
            if (wd < D / 8) {
                float4 *o = (float4 *)(xn + 8 * wd);
                const float4 a = o[0], b = o[1];
                o[0] = make_float4(a.x * rs * (1.f + wv[w][k][0]), a.y * rs * (1.f + wv[w][k][1]),
                                   a.z * rs * (1.f + wv[w][k][2]), a.w * rs * (1.f + wv[w][k][3]));
                o[1] = make_float4(b.x * rs * (1.f + wv[w][k][4]), b.y * rs * (1.f + wv[w][k][5]),
                                   b.z * rs * (1.f + wv[w][k][6]), b.w * rs * (1.f + wv[w][k][7]));
            }
        }
    wave_lds_order();
}

// After route_wave with bounds, on the same wave: when a decision was ambiguous (R.amb),
// every candidate whose interval reaches the lowest pick's lower end (the picks among them)
// gets its reference logit, and the K best of those by (l_ref desc, index asc) are the picks:
// an expert outside that set is below all K current picks in exact arithmetic too.  Equal
// reference logits give equal p, so the reference's tie rule (lower index) holds; distinct
// logits whose p round equal are the documented exact-tie class.  The weights stay p / sum p
// from the device logits.  stage_x(C.x) fills the input row (this wave only); router row e
// is rw + e rrb (E rows, f32 or int8).  Returns at once when nothing was ambiguous.
//
// The reference logit (c/qwen.c:178-189, int8 :230-238) is the sequential fp32 sum of the
// rounded products x[i] w[i] in index order, then times the int8 row scale.  The rows go in
// groups of kCertRows: per chunk of kCertCols columns the wave loads the group's weights
// (kCertPF chunks ahead, one buffer descriptor over the router matrix), writes the rounded
// products to LDS (R.cand, free after route_wave) and lane j adds row j's in index order.
constexpr int kCertRows = 16, kCertCols = 64, kCertPF = 4, kCertPS = kCertCols + 4;
// The reference logits of S's rows [g0, g0 + ng) (S = sl, ranks into R.cid) into R.clo.  I8:
// int8 rows (times scales[e] after the sum), else f32; a template parameter so that the
// loads carry no per-load branch and the prefetched chunks stay in flight.
template <bool I8>
__device__ __forceinline__ void cert_group(RouteLds &R, const CertLds &C, const int *sl, int g0, int ng, int D,
                                           const float *scales, __amdgpu_buffer_rsrc_t rr, int rrb) {
    const int lane = threadIdx.x & 63;
    const int cl = 4 * (lane & 15);   // the lane's 4 columns of a chunk; rows 4 q + lane / 16
    float *P = (float *)R.cand;
    int base[4];                      // byte offset of the lane's row q, -1 past the group
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int j = 4 * q + (lane >> 4);
        base[q] = j < ng ? R.cid[sl[g0 + j]] * rrb : -1;
    }
    // chunk c0's weights of the lane's 4 rows; columns past D read 0 without memory access
    auto load_chunk = [&](int c0, float4 (&wv)[4]) {
        const int col = c0 + cl;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int off = base[q] >= 0 && col < D ? base[q] + (I8 ? col : 4 * col) : (int)0x80000000;
            if constexpr (I8) {
                const uint32_t v = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rr, off, 0, 0);
                wv[q] = make_float4(__int_as_float(v), 0.f, 0.f, 0.f);   // converted at use
            } else {
                const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 0);
                wv[q] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
            }
        }
    };
    // chunk c0 (n columns): the products into P, then lane j < ng adds row j's in order;
    // `next` (a chunk kCertPF ahead, or past D) is loaded into wv once wv is consumed
    float acc = 0.f;
    auto step = [&](float4 (&wv)[4], int c0, int n, bool next) {
        const float4 xv = *(const float4 *)(C.x + c0 + cl);   // past D: not summed below
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float4 w = wv[q];
            if constexpr (I8) {
                const uint32_t v = __float_as_uint(w.x);
                w = make_float4((float)(int8_t)v, (float)(int8_t)(v >> 8), (float)(int8_t)(v >> 16), (float)(int8_t)(v >> 24));
            }
            *(float4 *)(P + (4 * q + (lane >> 4)) * kCertPS + cl) =
                make_float4(__fmul_rn(xv.x, w.x), __fmul_rn(xv.y, w.y), __fmul_rn(xv.z, w.z), __fmul_rn(xv.w, w.w));
        }
        if (next) load_chunk(c0 + kCertPF * kCertCols, wv);
        wave_lds_order();
        if (lane < ng) {
            const float *pr = P + lane * kCertPS;
            if (n == kCertCols) {   // each half's reads issued before its first add
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float4 p[kCertCols / 8];
#pragma unroll
                    for (int i = 0; i < kCertCols / 8; i++) p[i] = *(const float4 *)(pr + h * (kCertCols / 2) + 4 * i);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < kCertCols / 8; i++)
                        acc = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(acc, p[i].x), p[i].y), p[i].z), p[i].w);
                }
            } else {
                for (int i = 0; i < n; i++) acc = __fadd_rn(acc, pr[i]);
            }
        }
        wave_lds_order();
    };
    static_assert(kCertPF == 4, "four named chunk buffers");
    float4 w0[4], w1[4], w2[4], w3[4];
    load_chunk(0, w0);
    load_chunk(kCertCols, w1);
    load_chunk(2 * kCertCols, w2);
    load_chunk(3 * kCertCols, w3);
    int c0 = 0;
    for (; c0 + 4 * kCertCols <= D; c0 += 4 * kCertCols) {   // full rounds: no conditions
        step(w0, c0, kCertCols, true);
        step(w1, c0 + kCertCols, kCertCols, true);
        step(w2, c0 + 2 * kCertCols, kCertCols, true);
        step(w3, c0 + 3 * kCertCols, kCertCols, true);
    }
    // the last < 4 chunks are in w0, w1, w2 (wave-uniform conditions)
    if (c0 < D) step(w0, c0, min(kCertCols, D - c0), false);
    if (c0 + kCertCols < D) step(w1, c0 + kCertCols, min(kCertCols, D - c0 - kCertCols), false);
    if (c0 + 2 * kCertCols < D) step(w2, c0 + 2 * kCertCols, min(kCertCols, D - c0 - 2 * kCertCols), false);
    if (lane < ng) {
        const int r = sl[g0 + lane];
        R.clo[r] = I8 ? __fmul_rn(acc, scales[R.cid[r]]) : acc;
    }
}

template <typename StageX>
__device__ __forceinline__ void route_certify_wave(RouteLds &R, CertLds &C, int K, int D, bool int8, const float *scales,
                                                   const uint8_t *rw, int rrb, int E, StageX stage_x) {
    static_assert(sizeof(float) * kCertRows * kCertPS <= sizeof(R.cand), "product chunk fits R.cand");
    if (!R.amb) return;
    const int lane = threadIdx.x & 63, nc = R.ncand;
    const float thr = R.thr;
    stage_x(C.x);
    // S: the ranks r < nc whose interval reaches thr, in rank order, into C.b (free now)
    int *sl = (int *)C.b;
    int ns = 0;
    for (int r0 = 0; r0 < nc; r0 += 64) {
        const int r = r0 + lane;
        const bool f = r < nc && R.chi[r] >= thr;
        const unsigned long long mk = __ballot(f);
        if (f) sl[ns + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u))] = r;
        ns += __popcll(mk);
    }
    wave_lds_order();
    const __amdgpu_buffer_rsrc_t rr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(rw), (short)0, E * rrb, 0x00020000);
    for (int g0 = 0; g0 < ns; g0 += kCertRows) {
        const int ng = min(kCertRows, ns - g0);
        if (int8) cert_group<true>(R, C, sl, g0, ng, D, scales, rr, rrb);
        else cert_group<false>(R, C, sl, g0, ng, D, scales, rr, rrb);
    }
    wave_lds_order();
    for (int r = lane; r < nc; r += 64) {
        if (!(R.chi[r] >= thr)) continue;
        const float v = R.clo[r];
        const int e = R.cid[r];
        int rank = 0;
        for (int j = 0; j < nc; j++) {
            const float o = R.clo[j];
            rank += (R.chi[j] >= thr && (o > v || (o == v && R.cid[j] < e))) ? 1 : 0;
        }
        if (rank < K) R.idx[rank] = e;
    }
    wave_lds_order();
    if (lane < K) R.val[lane] = R.p[R.idx[lane]] / R.sum;
    wave_lds_order();
    if (lane == 0) {   // the renorm sum in rank order (c/qwen.c:816)
        float sm = 0.f;
        for (int j = 0; j < K; j++) sm += R.val[j];
        R.vsum = sm;
    }
    wave_lds_order();
}

// the expert table of a layer (moe.hip): false if it is not complete
// the certification test hook's setting (coli_hip_moe_cert_all)
int moe_cert_all();
bool moe_layer(int layer, const ExpertRec **d_rec, const float **d_shgate, MoeGeom *geom, int *E);

}  // namespace coli
