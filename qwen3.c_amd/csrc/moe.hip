// moe.hip - the device-indexed top-k MoE block, the expert-group entry points (host
// rows, and the stream form that accumulates into the device residual) and the expert
// table of the drop-in ABI.
//
// Semantics (c/qwen.c:804-928, the --no-vulkan path):
//   logits = router @ x                                  (f32 router, c/qwen.c:178-189)
//   p = softmax(logits); idx/val = K greedy picks of p (ties -> lower index), val /= sum(val)
//   shgt = sigmoid(sh_gate . x)
//   out[d] = sum_k val_k * down_k(silu(gate_k x) * up_k x)[d]   (rank order), then
//   out[d] += shgt * down_sh(silu(gate_sh x) * up_sh x)[d]
//
// One persistent launch (moe_block_kernel) over a list of tiles in dependency order:
//   R  router rows          -> logits (tagged)
//   Gs shared gate/up rows  -> h[K]   (independent of routing: overlaps R and T)
//   T  softmax / top-k / renorm / shared gate -> route (tagged)
//   Gk routed gate/up rows  -> h[k]   (wait for route)
//   D  down rows of one slot -> y[k]   (wait for route, then h)
//   C  weighted combine of the K+1 y rows -> out   (wait for y)
// Block b runs tile b, one block per tile.  A tile only waits for tiles of smaller index,
// which blocks of smaller index hold (workgroups are dispatched in index order), so the
// launch makes progress however many blocks are resident at once.
//
// Cross-block data are 64-bit words {epoch, value} written and read with agent-scope
// atomics (single-copy atomic, coherent across the XCDs' L2s): a consumer polls until the
// tag equals the launch epoch.  There are no counters to order, so no device-scope fences
// (an L2 write-back each on gfx950) are issued.  Polls are bounded: past the limit they set an
// error word stamped with the launch's epoch and give up, so every wave always exits.
#include "moe_common.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

namespace coli {

constexpr int kRRows = kWaves;            // router rows per tile (one per wave)
constexpr int kGSteps = 1;                // gate/up row steps per tile
constexpr int kRouteReps = 4;             // copies of the route block (readers spread over them)
constexpr int kRouteStride = 32;          // words per copy: idx [K] | w [K + 1] | ... | prov [K], K <= 8
constexpr int kProvOff = 24;              // the provisional ids' words within a copy

struct MoeArgs {
    const float *x;                       // [D] expert input (post-attention RMSNorm), or the
                                          // residual when xw != NULL
    const float *xw;                      // post-attention norm weight [D] (zero-centred), or NULL
    float eps;
    const uint8_t *rw;                    // router rows (fmt 0 f32 or fmt 1 int8)
    const float *rs;                      // fmt 1: per-row scales
    int rfmt, rrb, E;
    const ExpertRec *rec;                 // [E + 1], shared expert at E
    const float *sh_gate;                 // [D]
    int K;
    float *out;                           // [D]
    int accumulate;                       // out += (residual stream) instead of out =
    int cert_all;                         // test hook: certify every route (all candidates)
    int *idx_out;                         // optional [K]
    float *val_out;                       // optional [K + 1] (renormed weights, then shgt)
    unsigned long long *tagv;             // logits [E + 1] | crude / tight bounds [E + 1] each |
                                          // route [kRouteReps][kRouteStride] |
                                          // h [(K + 1) * I] | y [(K + 1) * D]
                                          // (logit E = the shared-expert gate dot)
    unsigned long long *err;              // error word: (epoch << 32) | code of a failing launch
    uint32_t epoch;
    int gRows, nG;                        // gate/up rows per tile, tiles per expert
    int nD, nC;                           // down tiles per slot (kDRows rows), combine tiles
    MoeGeom g;
};

// tag-buffer regions
__device__ __forceinline__ unsigned long long *route_of(const MoeArgs &a, int rep) {
    return a.tagv + 3 * (a.E + 1) + (size_t)rep * kRouteStride;
}
__device__ __forceinline__ unsigned long long *h_of(const MoeArgs &a, int slot) {
    return a.tagv + 3 * (a.E + 1) + kRouteReps * kRouteStride + (size_t)slot * a.g.I;
}
__device__ __forceinline__ unsigned long long *y_of(const MoeArgs &a, int slot) {
    return h_of(a, a.K + 1) + (size_t)slot * a.g.D;
}
__device__ __forceinline__ float tag_get(const unsigned long long *p, uint32_t epoch, unsigned long long *err) {
    for (int polls = 0;; polls++) {
        const unsigned long long v = aload(p);
        if ((uint32_t)(v >> 32) == epoch) return __uint_as_float((uint32_t)v);
        if (poll_give_up(err, epoch, polls)) return 0.f;
    }
}

// ---------------------------------------------------------------- h -> digit planes
// The down projection uses the same integer-dot arithmetic as the GEMV (fmt6_device.h)
// with h (one slot) in place of x: digit planes limb[digit][hprep_pos(word)], qsum[chunk],
// gmax[group].  hprep_pos puts host chunk h = 2 jj + c (the chunk a down thread reads, see
// down_thread) at slot c, lane jj, lanes of a slot side by side: the 16-byte reads of a
// row's threads are consecutive in LDS.
constexpr int kHLanes = kMoeMaxI / 64;
__device__ __forceinline__ int hprep_pos(int w) {
    const int h = w >> 2;
    return ((h & 1) * kHLanes + (h >> 1)) * 4 + (w & 3);
}
struct HPrep {
    __attribute__((aligned(16))) uint32_t limb[kLimbs][kMoeMaxI / 8];
    int qsum[kMoeMaxI / 32];
    unsigned gmax[kMoeMaxI / 64];
};
constexpr int kHWords = (kMoeMaxI / 8 + kThreads - 1) / kThreads;

// v: the thread's words q = tid + k * kThreads (8 columns each) of the I values (zeros
// past I).  Group maxima and chunk q sums as in prep_x.  Ends with __syncthreads().
__device__ __forceinline__ void prep_h(const float (&v)[kHWords][8], int I, int gs, HPrep &H) {
    const int tid = threadIdx.x, nw = I / 8, wpg = gs / 8;
    const bool runs = wpg <= 16 && (wpg & (wpg - 1)) == 0;
    if (!runs) {
        for (int i = tid; i < I / gs; i += kThreads) H.gmax[i] = 0u;
        __syncthreads();
    }
    uint32_t mb[kHWords];
#pragma unroll
    for (int k = 0; k < kHWords; k++) {
        const int q = tid + k * kThreads;
        float m = 0.f;
#pragma unroll
        for (int c = 0; c < 8; c++) m = fmaxf(m, fabsf(v[k][c]));
        mb[k] = __float_as_uint(m);
        if (runs) mb[k] = run_umax(mb[k], wpg);
        else if (q < nw) atomicMax(&H.gmax[(q * 8) / gs], mb[k]);
    }
    if (!runs) __syncthreads();
#pragma unroll
    for (int k = 0; k < kHWords; k++) {
        const int q = tid + k * kThreads;
        const bool on = q < nw;
        const float m = runs ? __uint_as_float(mb[k]) : on ? __uint_as_float(H.gmax[(q * 8) / gs]) : 0.f;
        uint32_t u[8];
        int qs = word_digits(v[k], exp22_of(m), u);
        if (on) {
            uint32_t lw[kLimbs];
            digit_planes(u, lw);
#pragma unroll
            for (int l = 0; l < kLimbs; l++) H.limb[l][hprep_pos(q)] = lw[l];
        }
        qs = quad_sum(qs);
        if (on && (q & 3) == 0) H.qsum[q / 4] = qs;
        if (runs && on && (q & (wpg - 1)) == 0) H.gmax[(q * 8) / gs] = mb[k];
    }
    __syncthreads();
}

// ---------------------------------------------------------------- down rows
// One thread per 16-byte chunk of a down row: TPR = 2 * (lanes of the lanes layout,
// rounded up to a power of two); thread t < TPR/2 reads chunk slot 0 of lane t, thread
// TPR/2 + t chunk slot 1 of lane t, so one load instruction covers whole rows.  The
// thread's host chunk is h = 2 * lane + slot (columns 32h .. 32h + 31, one group).
struct DownThread {
    uint32_t woff, soff;   // byte offsets within a row (kOOB: no data)
    int h;                 // host chunk
};

template <int TPR>
__device__ __forceinline__ DownThread down_thread(const MoeGeom &g) {
    const int t = (threadIdx.x & 63) % TPR, c = t >= TPR / 2 ? 1 : 0, jj = t - c * (TPR / 2);
    const bool on = jj < g.nlD && 2 * jj + c < g.I / 32;
    DownThread d;
    d.h = on ? 2 * jj + c : 0;
    d.woff = on ? (uint32_t)((c * g.nlD + jj) * 16) : kOOB;
    d.soff = on ? (uint32_t)(((d.h * 32) / g.gs) * 8) : kOOB;
    return d;
}

// partial of one chunk: s * (2^(e-22) T - (z - 8) sum(h~)) over its 32 columns
__device__ __forceinline__ float down_chunk(const HPrep &H, int gs, const DownThread &d, const uint4 &w,
                                            const float2 &sz) {
    const int pos = ((d.h & 1) * kHLanes + (d.h >> 1)) * 4;
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    int t[kLimbs] = {0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int l = 0; l < kLimbs; l++) {
        const uint4 hv = *(const uint4 *)&H.limb[l][pos];
        t[l] = __builtin_amdgcn_sdot8((int)wv[0], (int)hv.x, t[l], false);
        t[l] = __builtin_amdgcn_sdot8((int)wv[1], (int)hv.y, t[l], false);
        t[l] = __builtin_amdgcn_sdot8((int)wv[2], (int)hv.z, t[l], false);
        t[l] = __builtin_amdgcn_sdot8((int)wv[3], (int)hv.w, t[l], false);
    }
    const int lo = t[0] + 16 * t[1] + 256 * t[2];
    const int hi = t[3] + 16 * t[4] + 256 * t[5];
    const float T = fmaf((float)hi, 4096.f, (float)lo);
    const float m = __uint_as_float(H.gmax[(d.h * 32) / gs]);
    const int ue = -exp22_of(m);
    const float ucs = ldexpf((float)H.qsum[d.h], ue);
    return sz.x * fmaf(-(sz.y - 8.f), ucs, ldexpf(T, ue));
}

// Down projection of one slot for kDRows rows r0 ..: y[r] = down row r . h.  Wave w takes
// rows r0 + (p * kWaves + w) * RPW + seg for passes p; every pass's weight loads are
// issued before gather(hv) fills the thread's h words (see prep_h).  emit(r, y) per row.
constexpr int kDRows = 64;
template <int TPR, typename Gather, typename Emit>
__device__ __forceinline__ void down_slot(const MoeGeom &g, const ExpertRec &rec, HPrep &H, int r0, Gather gather,
                                          Emit emit) {
    constexpr int RPW = 64 / TPR, P = kDRows / (kWaves * RPW);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = lane % TPR, seg = lane / TPR;
    const DownThread d = down_thread<TPR>(g);
    const uint32_t wtot = (uint32_t)g.D * g.rbD, stot = (uint32_t)g.D * g.ngI * 8;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(rec.wd, wtot), rs = buf_rsrc(rec.sd, stot);
    uint4 wq[P];
    float2 sv[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int r = r0 + (p * kWaves + wave) * RPW + seg;
        const uint32_t rc = (uint32_t)(r < g.D ? r : g.D);   // row D reads 0 (past the end)
        wq[p] = buf_load16(rw, rc * g.rbD + d.woff);
        sv[p] = buf_load8f(rs, rc * g.ngI * 8 + d.soff);
    }
    float hv[kHWords][8];
    gather(hv);
    prep_h(hv, g.I, g.gs, H);
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int r = r0 + (p * kWaves + wave) * RPW + seg;
        const float y = seg_sum<TPR>(down_chunk(H, g.gs, d, wq[p], sv[p]));
        if (t == TPR - 1 && r < g.D) emit(r, y);
    }
}

// ---------------------------------------------------------------- gate/up rows
// h[r] = silu(gate r . x) * (up r . x) for the tile's rows (c/qwen.c:780-786, silu :173).
// All of the tile's weight loads are issued before the first row is reduced.
// gateup_load issues the tile's loads, gateup_dot reduces them (split so that a tile can
// check its expert while the loads are in flight).
template <int CU>
struct GateUpW {
    uint4 wg[kGSteps][kLaneChunks], wu[kGSteps][kLaneChunks];
    float2 sg[kGSteps][LaneX<CU>::NU], su[kGSteps][LaneX<CU>::NU];
};
template <int LPR, int CU>
__device__ __forceinline__ void gateup_load(const LaneX<CU> &L, const ExpertRec &rec, const MoeGeom &g, int r0,
                                            GateUpW<CU> &W) {
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, seg = lane / LPR;
    const uint32_t wtot = (uint32_t)g.I * g.rbG, stot = (uint32_t)g.I * g.ngD * 8;
    const __amdgpu_buffer_rsrc_t rgw = buf_rsrc(rec.wg, wtot), rgs = buf_rsrc(rec.sg, stot);
    const __amdgpu_buffer_rsrc_t ruw = buf_rsrc(rec.wu, wtot), rus = buf_rsrc(rec.su, stot);
#pragma unroll
    for (int st = 0; st < kGSteps; st++) {
        const int r = r0 + (st * kWaves + wave) * RPW + seg;
        const uint32_t rc = (uint32_t)(r < g.I ? r : g.I);   // row I reads 0 (past the end)
        lane_load<CU>(rgw, rgs, rc * g.rbG, rc * g.ngD * 8, L, W.wg[st], W.sg[st]);
        lane_load<CU>(ruw, rus, rc * g.rbG, rc * g.ngD * 8, L, W.wu[st], W.su[st]);
    }
}
template <int LPR, int CU, typename Emit>
__device__ __forceinline__ void gateup_dot(const LaneX<CU> &L, const MoeGeom &g, int r0, const GateUpW<CU> &W,
                                           Emit emit) {
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane % LPR, seg = lane / LPR;
#pragma unroll
    for (int st = 0; st < kGSteps; st++) {
        const int r = r0 + (st * kWaves + wave) * RPW + seg;
        const float gv = seg_sum<LPR>(lane_row<CU>(W.wg[st], W.sg[st], L));
        const float uv = seg_sum<LPR>(lane_row<CU>(W.wu[st], W.su[st], L));
        if (j == LPR - 1 && r < g.I) emit(r, gv / (1.f + expf(-gv)) * uv);
    }
}
template <int LPR, int CU, typename Emit>
__device__ __forceinline__ void gateup_rows(const LaneX<CU> &L, const ExpertRec &rec, const MoeGeom &g, int r0,
                                            Emit emit) {
    GateUpW<CU> W;
    gateup_load<LPR, CU>(L, rec, g, r0, W);
    gateup_dot<LPR, CU>(L, g, r0, W, emit);
}

// ---------------------------------------------------------------- R: router rows
// One row per wave: rows r < E are the router (c/qwen.c:178-189 f32, :230-238 int8), row
// E is the shared-expert gate vector (c/qwen.c:833).  Dot products accumulate in fp64 from
// exact fp64 products, so each logit is the correctly rounded value of the exact sum (the
// reference sums sequentially in fp32).
__device__ __forceinline__ float4 int8x4(uint32_t q) {
    return make_float4((float)(int8_t)q, (float)(int8_t)(q >> 8), (float)(int8_t)(q >> 16), (float)(int8_t)(q >> 24));
}

// The normed input row into LDS (xn[0, D)) from x and the norm weights as loaded by prep_load
// (issued before any other load of the tile, so only these are waited for): norm_apply,
// the G tiles' staging, so the router's input and the experts' are the same bits.
__device__ __forceinline__ void stage_input(XRegs &xr, const XRegs &wr, int D, float eps, float *xn, double *s_red) {
    norm_apply(xr, wr, D, D, eps, s_red);
#pragma unroll
    for (int k = 0; k < XRegs::kWords; k++) {
        const int w = threadIdx.x + k * kThreads;
        if (w < D / 8) {
            *(float4 *)(xn + 8 * w) = make_float4(xr.v[k][0], xr.v[k][1], xr.v[k][2], xr.v[k][3]);
            *(float4 *)(xn + 8 * w + 4) = make_float4(xr.v[k][4], xr.v[k][5], xr.v[k][6], xr.v[k][7]);
        }
    }
    lds_barrier();
}

// Bounds of the logits: crude (published with the logits) and tight (published later), the
// words after the logits (E + 1 each; the shared gate's are not used).
__device__ __forceinline__ unsigned long long *bounds_of(const MoeArgs &a) { return a.tagv + a.E + 1; }
__device__ __forceinline__ unsigned long long *tight_of(const MoeArgs &a) { return a.tagv + 2 * (a.E + 1); }

// xn: an LDS row of D floats.  The tile's router rows are loaded first (in flight while the
// block stages the input row, normed when a.xw != NULL, into xn); then every wave reads x
// from LDS or global.  Each router row publishes its logit, then its bound (router_row).
__device__ __forceinline__ void tile_router(const MoeArgs &a, int r0, double *s_red, float *xn) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), D = a.g.D;
    const int r = r0 + wave;
    const bool live = r <= a.E, gate = r == a.E;   // wave-uniform
    const uint8_t *row = gate ? (const uint8_t *)a.sh_gate : a.rw + (size_t)r * a.rrb;
    const bool f32 = gate || a.rfmt == 0;
    // buffer loads: columns past D (and rows past E) read 0, no per-lane conditions
    const __amdgpu_buffer_rsrc_t rr = buf_rsrc(row, !live ? 0u : f32 ? (uint32_t)D * 4u : (uint32_t)D);
    float4 w[kRouterRC];
    auto load_row = [&](int c0, float4 (&wv)[kRouterRC]) {
        if (f32) {
#pragma unroll
            for (int c = 0; c < kRouterRC; c++) {
                const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rr, (c0 + (lane + c * 64) * 4) * 4, 0, kStream);
                wv[c] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
            }
        } else {
#pragma unroll
            for (int c = 0; c < kRouterRC; c++)
                wv[c] = int8x4((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rr, c0 + (lane + c * 64) * 4, 0, kStream));
        }
    };
    // x and the norm weights first (range 0 without a norm: no memory access), then the row
    XRegs xr, wr;
    const int nI = a.xw ? D : 0;
    prep_load(a.x, nI, D, xr);
    prep_load(a.xw ? a.xw : a.x, nI, D, wr);
    load_row(0, w);
    if (a.xw) stage_input(xr, wr, D, a.eps, xn, s_red);
    if (!live) return;
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x, (uint32_t)D * 4u);
    auto load_x = [&](int c0, float4 (&xq)[kRouterRC]) {
#pragma unroll
        for (int c = 0; c < kRouterRC; c++) {
            const int col = c0 + (lane + c * 64) * 4;
            if (a.xw) {
                xq[c] = col < D ? *(const float4 *)(xn + col) : make_float4(0.f, 0.f, 0.f, 0.f);   // LDS
            } else {
                const coli_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rx, col * 4, 0, kCached);
                xq[c] = make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
            }
        }
    };
    const bool int8 = !gate && a.rfmt == 1;
    const float scale = int8 ? a.rs[r] : 1.f;
    const uint32_t ep = a.epoch;
    const float B = router_row(D, scale, int8, w, true, load_row, load_x, [&](float L, float Bc) {
        if (lane == 0) {
            tag_put(&a.tagv[r], ep, L);
            if (!gate) tag_put(&bounds_of(a)[r], ep, Bc);
        }
    });
    if (lane == 0 && !gate) tag_put(&tight_of(a)[r], ep, B);
}

// ---------------------------------------------------------------- T: route
// c/qwen.c:332-336 softmax_row, :807-817 top-k and renorm, :833-834 shared gate, on one wave
// of the tile (route_wave, no block barriers); the picks certified against the reference's
// sequential fp32 logits (route_certify_wave).
template <int kPer>   // words per lane: E + 1 <= 64 kPer
__device__ __forceinline__ void tile_route_n(const MoeArgs &a, RouteLds &R, CertLds &C) {
    const int lane = threadIdx.x, E = a.E, K = a.K;
    // the lane's logits e = lane + 64 q <= E (logit E is the shared-expert gate dot) and their
    // bounds, all polled together: one round trip per poll however many a lane holds
    unsigned long long v[kPer], vb[kPer];
    for (int polls = 0;; polls++) {
        bool all = true;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int e = lane + 64 * q;
            v[q] = aload(&a.tagv[e <= E ? e : E]);
            vb[q] = aload(&bounds_of(a)[e < E ? e : E - 1]);
            all &= e > E || (uint32_t)(v[q] >> 32) == a.epoch;
            all &= e >= E || (uint32_t)(vb[q] >> 32) == a.epoch;
        }
        if (__ballot(!all) == 0ull || poll_give_up(a.err, a.epoch, polls)) break;
    }
    float gate = 0.f;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = lane + 64 * q;
        const float l = __uint_as_float((uint32_t)v[q]);
        if (e < E) {
            R.p[e] = l;
            C.l[e] = l;
            C.b[e] = __uint_as_float((uint32_t)vb[q]);
        } else if (e == E) {
            gate = l;
        }
    }
    gate = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gate), E & 63));
    wave_lds_order();
    route_wave(R, E, K, C.l, C.b, RouteProv{route_of(a, 0) + kProvOff, kRouteStride, kRouteReps, a.epoch});   // crude bounds
    if (R.amb) {   // the tight bounds of the candidates (published by now), and the check again
        const int nc = R.ncand;
        for (int r = lane; r < nc; r += 64) {
            const int e = R.cid[r];
            const float b = tag_get(&tight_of(a)[e], a.epoch, a.err);
            R.clo[r] = C.l[e] - b;
            R.chi[r] = C.l[e] + b;
        }
        wave_lds_order();
        float thr;
        const int amb = cert_check(R, K, nc, &thr);
        if (lane == 0) {
            R.amb = amb;
            R.thr = thr;
        }
        wave_lds_order();
    }
    if (a.cert_all) {   // test hook: every candidate gets its reference logit
        if (lane == 0) {
            R.amb = 1;
            R.thr = -INFINITY;
        }
        wave_lds_order();
    }
    route_certify_wave(
        R, C, K, a.g.D, a.rfmt == 1, a.rs, a.rw, a.rrb, a.E,
        [&](float *xn) { stage_input_wave(a.x, a.xw, a.g.D, a.eps, xn); });
    // lane (copy c, word k) writes word k of copy c: words [0, K) expert ids, [K, 2K)
    // renormed weights, 2K the shared gate
    const float sm = R.vsum;
    for (int q = lane; q < kRouteReps * kRouteStride; q += 64) {
        const int c = q / kRouteStride, k = q % kRouteStride;
        if (k > 2 * K) continue;
        float w;
        if (k < K) w = __int_as_float(R.idx[k]);
        else if (k < 2 * K) w = R.val[k - K] / sm;
        else w = 1.f / (1.f + expf(-gate));
        tag_put(&route_of(a, c)[k], a.epoch, w);
        if (c == 0) {
            if (k < K && a.idx_out) a.idx_out[k] = R.idx[k];
            if (k >= K && a.val_out) a.val_out[k - K] = w;
        }
    }
}

__device__ __forceinline__ void tile_route(const MoeArgs &a, RouteLds &R, CertLds &C) {
    if (threadIdx.x >= 64) return;
    if (a.E + 1 <= 320) tile_route_n<5>(a, R, C);
    else if (a.E + 1 <= 576) tile_route_n<9>(a, R, C);
    else tile_route_n<17>(a, R, C);
}

// ---------------------------------------------------------------- LDS of the kernel
struct RouterLds {
    __attribute__((aligned(16))) float xn[kLaneMaxI];   // the (normed) input row
};
struct RouteTileLds {
    RouteLds r;
    CertLds c;
};
union MoeLds {
    RouterLds n;      // R tiles
    XPrep x;          // G tiles
    HPrep h;          // D tiles
    RouteTileLds t;   // T tile
};

// ---------------------------------------------------------------- G tile
template <int LPR, int CU>
__device__ __forceinline__ void tile_gateup(const MoeArgs &a, const XPrep &P, int slot, int r0, int *s_e) {
    const MoeGeom &g = a.g;
    const int j = (threadIdx.x & 63) % LPR;
    LaneX<CU> L;   // x digits of the lane first: they do not depend on the route
    lane_geo<CU>(j, g.nlG, g.D, g.gs, L);
    lane_x<CU>(P, g.gs, L);
    // A routed tile starts its loads on the route tile's provisional pick, then checks the
    // final route (published later, after the certification) while they are in flight; only
    // when the certification changed this slot's pick does it load again.
    const unsigned long long *route = route_of(a, blockIdx.x % kRouteReps);
    auto pick = [&](int w) {
        int e = __float_as_int(tag_get(&route[w], a.epoch, a.err));
        if (e < 0 || e > a.E) {
            err_set(a.err, a.epoch, 2);
            e = a.E;
        }
        return e;
    };
    if (threadIdx.x == 0) s_e[0] = slot < a.K ? pick(kProvOff + slot) : a.E;
    __syncthreads();
    const int e0 = s_e[0];
    GateUpW<CU> W;
    gateup_load<LPR, CU>(L, a.rec[e0], g, r0, W);
    if (slot < a.K) {   // block uniform
        if (threadIdx.x == 0) s_e[1] = pick(slot);
        __syncthreads();
        if (s_e[1] != e0) gateup_load<LPR, CU>(L, a.rec[s_e[1]], g, r0, W);
    }
    unsigned long long *hs = h_of(a, slot);
    const uint32_t ep = a.epoch;
    gateup_dot<LPR, CU>(L, g, r0, W, [&](int r, float h) { tag_put(&hs[r], ep, h); });
}

// ---------------------------------------------------------------- D and C tiles
// D: y_s[r] = down_s row r . h_s for one slot and kDRows rows.  The tile polls one h word
// of each of the slot's G tiles (its last row) until all carry the launch's tag, then reads
// the whole tagged h (words not yet of this launch are read again): a cheap wait without
// counters, whose read-modify-writes and polls each added a memory round trip.  C:
// out[r] = ((0 + w_0 y_0) + w_1 y_1 ...) + shgt y_sh, the reference's order
// (c/qwen.c:870-877, :917), polling its rows' tagged y of every slot directly.
template <int TPR>
__device__ __forceinline__ void tile_dslot(const MoeArgs &a, HPrep &H, int slot, int r0, ExpertRec *s_rec) {
    const int tid = threadIdx.x, K = a.K;
    const unsigned long long *route = route_of(a, blockIdx.x % kRouteReps);
    if (tid == 0) {
        int e = a.E;
        if (slot < K) e = __float_as_int(tag_get(&route[slot], a.epoch, a.err));
        if (e < 0 || e > a.E) {
            err_set(a.err, a.epoch, 2);
            e = a.E;
        }
        s_rec[0] = a.rec[e];
    }
    __syncthreads();
    const unsigned long long *hs = h_of(a, slot);
    unsigned long long *ys = y_of(a, slot);
    const int nw = a.g.I / 8;
    const uint32_t ep = a.epoch;
    unsigned long long *err = a.err;
    auto gather = [&](float (&hv)[kHWords][8]) {
        if (tid < a.nG) {   // one word per G tile: the tile's last row
            const int r = min((tid + 1) * a.gRows, a.g.I) - 1;
            for (int polls = 0;; polls++)
                if ((uint32_t)(aload(hs + r) >> 32) == ep || poll_give_up(err, ep, polls)) break;
        }
        lds_barrier();   // no wait for the weight loads in flight
        for (int polls = 0;; polls++) {
            bool all = true;
#pragma unroll
            for (int k = 0; k < kHWords; k++) {
                const int q = tid + k * kThreads;
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const unsigned long long v = q < nw ? aload(hs + (size_t)q * 8 + c) : 0ull;
                    all &= q >= nw || (uint32_t)(v >> 32) == ep;
                    hv[k][c] = __uint_as_float((uint32_t)v);
                }
            }
            if (all || poll_give_up(err, ep, polls)) break;
        }
    };
    down_slot<TPR>(a.g, s_rec[0], H, r0, gather, [&](int r, float y) { tag_put(&ys[r], ep, y); });
}

constexpr int kCRows = 256;  // combine tile rows (one thread each)
__device__ __forceinline__ void tile_combine(const MoeArgs &a, int r0, float *s_w) {
    const int tid = threadIdx.x, K = a.K, NS = K + 1, D = a.g.D;
    const unsigned long long *route = route_of(a, blockIdx.x % kRouteReps);
    const unsigned long long *ys = y_of(a, 0);
    if (tid < NS) s_w[tid] = tag_get(&route[K + tid], a.epoch, a.err);   // val[0..K), then shgt at K
    __syncthreads();
    const int r = r0 + tid;
    if (tid >= kCRows || r >= D) return;
    float y[kMaxSlots];
    for (int polls = 0;; polls++) {
        bool all = true;
#pragma unroll
        for (int s = 0; s < kMaxSlots; s++) {
            const unsigned long long v = s < NS ? aload(ys + (size_t)s * D + r) : 0ull;
            all &= s >= NS || (uint32_t)(v >> 32) == a.epoch;
            y[s] = __uint_as_float((uint32_t)v);
        }
        if (all || poll_give_up(a.err, a.epoch, polls)) break;
    }
    float accum = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxSlots; s++)
        if (s < NS) accum = accum + s_w[s] * y[s];
    a.out[r] = a.accumulate ? a.out[r] + accum : accum;
}

// ---------------------------------------------------------------- the persistent kernel
template <int LPRG, int TPRD>
__global__ __launch_bounds__(kThreads, 3) void moe_block_kernel(MoeArgs a) {
    __shared__ MoeLds S;
    __shared__ int s_e[2];
    __shared__ ExpertRec s_rec[1];
    __shared__ float s_w[kMaxSlots];
    __shared__ double s_red[kWaves];
    const MoeGeom &g = a.g;
    const int K = a.K;
    // tile list: R router rows | Gs shared gate/up | Dsh shared down | T route |
    //            Gk routed gate/up | Dk routed down | C combine
    const int nR = (a.E + 1 + kRRows - 1) / kRRows;
    const int tGs = nR, tDsh = tGs + a.nG, tT = tDsh + a.nD, tGk = tT + 1, tDk = tGk + K * a.nG;
    const int tC = tDk + K * a.nD, total = tC + a.nC;
    // One block per tile (the host launches exactly that many): straight-line code, so
    // nothing tile-specific is computed up front and kept live across the other tile kinds.
    const int t = blockIdx.x;
    if (t >= total) return;
    const bool gtile = (t >= tGs && t < tDsh) || (t >= tGk && t < tDk);
    if (gtile) {   // x digits for the G tiles
        XRegs xr, wr;
        const int ncols = g.nlG * kLaneChunks * 32;
        prep_load(a.x, g.D, ncols, xr);
        if (a.xw) {   // post-attention norm of the residual (c/qwen.c:326-330)
            prep_load(a.xw, g.D, ncols, wr);
            norm_apply(xr, wr, g.D, ncols, a.eps, s_red);
        }
        prep_x(xr, g.gs, ncols, S.x);
    }
    if (t < tGs) tile_router(a, t * kRRows, s_red, S.n.xn);
    else if (t < tDsh) tile_gateup<LPRG, kLaneChunks>(a, S.x, K, (t - tGs) * a.gRows, s_e);
    else if (t < tT) tile_dslot<TPRD>(a, S.h, K, (t - tDsh) * kDRows, s_rec);
    else if (t == tT) tile_route(a, S.t.r, S.t.c);
    else if (t < tDk) tile_gateup<LPRG, kLaneChunks>(a, S.x, (t - tGk) / a.nG, ((t - tGk) % a.nG) * a.gRows, s_e);
    else if (t < tC) tile_dslot<TPRD>(a, S.h, (t - tDk) / a.nD, ((t - tDk) % a.nD) * kDRows, s_rec);
    else tile_combine(a, (t - tC) * kCRows, s_w);
}

// ---------------------------------------------------------------- expert table
struct EgTable {
    int n_layers = 0, E = 0, D = 0, I = 0, gs = 0;
    ExpertRec *d_rec = nullptr;   // device [n_layers][E + 1]
    ExpertRec *h_rec = nullptr;   // host mirror
    uint8_t *valid = nullptr;     // host [n_layers][E + 1]
    float *d_shgate = nullptr;    // device [n_layers][D]
    size_t rec_cap = 0, sg_cap = 0;
    MoeGeom geom;
    int geom_set = 0;
};
static EgTable g_eg;

// launches that can set an error word (both entry points), for the callers that skip a
// check when none ran since the last one
static uint64_t g_moe_launches = 0;
uint64_t moe_launches() { return g_moe_launches; }

struct MoeScratch {
    void *tag = nullptr;
    size_t tag_cap = 0;
    void *misc = nullptr;         // err at 64
    size_t misc_cap = 0;
    uint32_t epoch = 0;
};
static MoeScratch g_ms;

static bool geom_of(const ColiVkTensor *gt, const ColiVkTensor *dt, MoeGeom &m) {
    if (!tensor_live(gt) || !tensor_live(dt) || gt->fmt != 6 || dt->fmt != 6 || gt->layout != kLayoutLanes || dt->layout != kLayoutLanes)
        return false;
    memset(&m, 0, sizeof(m));
    m.D = gt->I;
    m.I = gt->O;
    m.gs = gt->gs;
    m.ngD = gt->ng;
    m.ngI = dt->ng;
    m.nlG = gt->nl;
    m.nlD = dt->nl;
    m.rbG = gt->row_bytes;
    m.rbD = dt->row_bytes;
    return dt->I == m.I && dt->O == m.D && dt->gs == m.gs;
}

static bool same_geom(const MoeGeom &a, const MoeGeom &b) { return memcmp(&a, &b, sizeof(a)) == 0; }

// every lane's 64 columns of a down row lie in one group; h fits the kernel's LDS
static bool geom_supported(const MoeGeom &m) {
    return m.gs % 64 == 0 && m.I % 64 == 0 && m.I >= 128 && m.I <= kMoeMaxI && m.D >= 192 && m.D <= kLaneMaxI &&
           m.D % 64 == 0;
}

static int pow2_ceil(int n) {
    int l = 1;
    while (l < n) l <<= 1;
    return l;
}

// Dispatch over the compiled shapes: LPRG = lanes per gate/up row (D / 64 rounded up to a
// power of two, 4..64), TPRD = threads per down row (2 x I / 64 likewise, 4..16).
template <template <int, int> class F, typename A>
static bool dispatch_shape(const MoeGeom &m, A &arg, hipStream_t st) {
    const int lg = pow2_ceil(m.nlG), td = 2 * pow2_ceil(m.nlD);
#define COLI_MOE_CASE(LG, TD) \
    if (lg == LG && td == TD) return F<LG, TD>::run(arg, st);
#define COLI_MOE_ROW(LG) COLI_MOE_CASE(LG, 4) COLI_MOE_CASE(LG, 8) COLI_MOE_CASE(LG, 16)
    COLI_MOE_ROW(4) COLI_MOE_ROW(8) COLI_MOE_ROW(16) COLI_MOE_ROW(32) COLI_MOE_ROW(64)
#undef COLI_MOE_ROW
#undef COLI_MOE_CASE
    return false;
}

template <int LPRG, int TPRD>
struct LaunchMoe {
    static bool run(MoeArgs &a, hipStream_t st) {
        auto kern = moe_block_kernel<LPRG, TPRD>;
        a.gRows = kGSteps * kWaves * (64 / LPRG);
        a.nG = (a.g.I + a.gRows - 1) / a.gRows;
        a.nD = (a.g.D + kDRows - 1) / kDRows;
        a.nC = (a.g.D + kCRows - 1) / kCRows;
        const int nR = (a.E + 1 + kRRows - 1) / kRRows;
        const long tiles = nR + (long)(a.K + 1) * (a.nG + a.nD) + 1 + a.nC;
        hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(kThreads), 0, st, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("moe launch", e);
        return true;
    }
};

// A refused call returns false with one line on stderr (once per reason).
static bool reject(const char *why) {
    static const char *last = nullptr;
    if (why != last) fprintf(stderr, "[HIP] moe block refused: %s\n", why);
    last = why;
    return false;
}

// Tag words a launch uses: logits [E + 1] | crude bounds [E + 1] | tight bounds [E + 1] |
// route copies | h [(K + 1) I] | y [(K + 1) D]
static size_t moe_tag_words(int E, int K, const MoeGeom &m) {
    return 3 * ((size_t)E + 1) + kRouteReps * kRouteStride + (size_t)(K + 1) * (m.I + m.D);
}

// clear n 64-bit words (a fill kernel rather than a memset, so the launch can be captured)
__global__ void clear_words(unsigned long long *w, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) w[i] = 0ull;
}

// The next launch epoch of a tag buffer.  Tags are 32-bit epochs and a consumer accepts a
// word whose tag equals its launch's, so when the counter wraps, the tag words and the error
// word are cleared first: no word written 2^32 launches ago can pass for a new one.  (A
// fresh buffer holds zeros, and epoch 0 is never used.)
static uint32_t next_epoch(uint32_t *epoch, unsigned long long *tags, size_t nwords, unsigned long long *err,
                           hipStream_t st) {
    if (++*epoch == 0) {
        hipLaunchKernelGGL(clear_words, dim3(64), dim3(256), 0, st, tags, nwords);
        hipLaunchKernelGGL(clear_words, dim3(1), dim3(64), 0, st, err, (size_t)1);
        *epoch = 1;
    }
    return *epoch;
}

// Validate a launch against the expert table and fill its arguments (everything but the
// tag buffer, error word and epoch).
static bool moe_args(int layer, const ColiVkTensor *router, int K, const float *d_x, float *d_out, int accumulate,
                     int *d_idx, float *d_val, const float *d_xw, float eps, MoeArgs &a) {
    EgTable &T = g_eg;
    if (!ok()) return false;
    if (!T.d_rec || layer < 0 || layer >= T.n_layers || !T.geom_set) return reject("no expert table for the layer");
    if (!tensor_live(router) || !d_x || !d_out) return reject("NULL argument or stale router handle");
    if (K < 1 || K > kTopK || K > T.E || T.E > kMaxE) return reject("K outside 1..8 or E above 1024");
    if (router->I != T.D || router->O != T.E || (router->fmt != 0 && router->fmt != 1) ||
        router->layout != kLayoutRows)
        return reject("router is not [E, D] fmt 0 or 1");
    for (int e = 0; e <= T.E; e++)
        if (!T.valid[(size_t)layer * (T.E + 1) + e]) return reject("expert table slot not set");
    memset(&a, 0, sizeof(a));
    a.x = d_x;
    a.xw = d_xw;
    a.eps = eps;
    a.rw = router->w;
    a.rs = router->sz;
    a.rfmt = router->fmt;
    a.rrb = router->row_bytes;
    a.E = T.E;
    a.rec = T.d_rec + (size_t)layer * (T.E + 1);
    a.sh_gate = T.d_shgate + (size_t)layer * T.D;
    a.K = K;
    a.out = d_out;
    a.accumulate = accumulate;
    a.cert_all = moe_cert_all();
    a.idx_out = d_idx;
    a.val_out = d_val;
    a.g = T.geom;
    return true;
}

// The layer's MoE block on device pointers (stream-ordered, no sync).  Launches share one
// scratch area: issue them on one stream.
bool moe_decode(int layer, const ColiVkTensor *router, int K, const float *d_x, float *d_out, int accumulate,
                int *d_idx, float *d_val, hipStream_t st, const float *d_xw, float eps) {
    MoeArgs a;
    if (!moe_args(layer, router, K, d_x, d_out, accumulate, d_idx, d_val, d_xw, eps, a)) return false;
    const size_t ntag = moe_tag_words(a.E, K, a.g);
    if (!scratch(&g_ms.tag, &g_ms.tag_cap, ntag * 8) || !scratch(&g_ms.misc, &g_ms.misc_cap, 256)) return false;
    a.tagv = (unsigned long long *)g_ms.tag;
    a.err = (unsigned long long *)((uint8_t *)g_ms.misc + 64);
    a.epoch = next_epoch(&g_ms.epoch, a.tagv, g_ms.tag_cap / 8, a.err, st);
    g_moe_launches++;
    return dispatch_shape<LaunchMoe>(a.g, a, st) || (ok() && reject("expert shape not compiled"));
}

static int g_cert_all = 0;
int moe_cert_all() { return g_cert_all; }

// Test hook: every route certified (each candidate's reference logit computed and ranked) on
// (1) or only the ambiguous ones (0, the default); returns the previous setting.  Both give
// the reference's picks.
COLI_API int coli_hip_moe_cert_all(int on) {
    const int prev = g_cert_all;
    g_cert_all = on ? 1 : 0;
    return prev;
}

bool moe_ready(int layer) {
    const EgTable &T = g_eg;
    if (!T.d_rec || layer < 0 || layer >= T.n_layers || !T.geom_set) return false;
    for (int e = 0; e <= T.E; e++)
        if (!T.valid[(size_t)layer * (T.E + 1) + e]) return false;
    return true;
}

bool moe_layer(int layer, const ExpertRec **d_rec, const float **d_shgate, MoeGeom *geom, int *E) {
    EgTable &T = g_eg;
    if (!moe_ready(layer)) return false;
    *d_rec = T.d_rec + (size_t)layer * (T.E + 1);
    *d_shgate = T.d_shgate + (size_t)layer * T.D;
    *geom = T.geom;
    *E = T.E;
    return true;
}

// ---------------------------------------------------------------- allocation-free variant
// coli_hip_moe_decode_noalloc runs the same launch with its cross-block words in a static
// device array instead of library scratch, for callers that cannot allocate (HIP graph
// capture, serving loops).  The array's first 256-byte line holds the error word, the rest
// the tag words; every device holds its own copy at its own address, looked up once per
// device at init (hipGetSymbolAddress), and each device keeps its own launch epoch.  Calls
// on one device share the array: calls that overlap on one device race.
namespace noalloc {
constexpr size_t kScratchBytes = (size_t)256 << 10;   // 32736 tag words after the error line
static __device__ __align__(256) unsigned long long scratch[kScratchBytes / 8];
}  // namespace noalloc

constexpr int kMaxDevices = 16;
struct NoAllocDev {
    unsigned long long *ptr = nullptr;   // device address of noalloc::scratch (never the host symbol)
    uint32_t epoch = 0;                  // kept across shutdown: the array outlives it
};
static NoAllocDev g_na[kMaxDevices];

bool moe_noalloc_init(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return false;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc::scratch));
    if (e != hipSuccess || !p) {
        fprintf(stderr, "[HIP] no-alloc MoE scratch: hipGetSymbolAddress failed: %s\n", hipGetErrorString(e));
        g_na[dev].ptr = nullptr;
        return false;
    }
    g_na[dev].ptr = (unsigned long long *)p;
    return true;
}

static bool moe_decode_noalloc(int layer, const ColiVkTensor *router, int K, const float *d_x, float *d_out,
                               int accumulate, int *d_idx, float *d_val, hipStream_t st) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices || !g_na[dev].ptr)
        return reject("no-alloc scratch not set up on this device");
    MoeArgs a;
    if (!moe_args(layer, router, K, d_x, d_out, accumulate, d_idx, d_val, nullptr, 0.f, a)) return false;
    constexpr size_t kErrWords = 256 / 8, kTagWords = noalloc::kScratchBytes / 8 - kErrWords;
    const size_t ntag = moe_tag_words(a.E, K, a.g);
    if (ntag > kTagWords) {
        fprintf(stderr, "[HIP] moe block (no-alloc) refused: needs %zu bytes of tag words, the static scratch holds %zu\n",
                ntag * 8, kTagWords * 8);
        return false;
    }
    NoAllocDev &n = g_na[dev];
    a.err = n.ptr;
    a.tagv = n.ptr + kErrWords;
    a.epoch = next_epoch(&n.epoch, a.tagv, kTagWords, a.err, st);
    g_moe_launches++;
    return dispatch_shape<LaunchMoe>(a.g, a, st) || (ok() && reject("expert shape not compiled"));
}

// The failure code a word holds (its low 32 bits), or 0.
static int err_code(unsigned long long w) { return (int)(uint32_t)w; }

// The error words of the current device: the scratch launches' and the no-alloc launches'
// (NULL where not allocated).
void moe_error_words(const unsigned long long **w0, const unsigned long long **w1) {
    *w0 = g_ms.misc ? (const unsigned long long *)((uint8_t *)g_ms.misc + 64) : nullptr;
    *w1 = nullptr;
    int dev = -1;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices) *w1 = g_na[dev].ptr;
}

// The code of the words' values v[0..1] (read with the launches finished): the first failure,
// each word that holds one cleared; -1 on a runtime error.
int moe_error_settle(const unsigned long long v[2]) {
    const unsigned long long *w[2];
    moe_error_words(&w[0], &w[1]);
    int code = 0;
    for (int i = 0; i < 2; i++) {
        if (!w[i] || !err_code(v[i])) continue;
        if (!code) code = err_code(v[i]);
        const unsigned long long z = 0;
        if (hipMemcpy(const_cast<unsigned long long *>(w[i]), &z, 8, hipMemcpyHostToDevice) != hipSuccess) return -1;
    }
    return code;
}

// 0 = no error since the last call; 1 = a poll gave up; 2 = a route held a bad expert id.
// Covers the scratch launches and the no-alloc launches of the current device.
int moe_error_take() {
    const unsigned long long *w[2];
    moe_error_words(&w[0], &w[1]);
    if (!w[0] && !w[1]) return 0;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    unsigned long long v[2] = {0, 0};
    for (int i = 0; i < 2; i++)
        if (w[i] && hipMemcpy(&v[i], w[i], 8, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    return moe_error_settle(v);
}

// Host-forced failure for tests: the error word is stamped with the next scratch launch's
// epoch, so that launch's bounded waits give up at their 16th poll (the kernels still exit
// normally) and the word reports the failure.
static bool moe_error_force(int code) {
    if (!ok() || !scratch(&g_ms.misc, &g_ms.misc_cap, 256) || code < 1 || code > 2) return false;
    uint32_t next = g_ms.epoch + 1;
    if (next == 0) next = 1;
    const unsigned long long v = ((unsigned long long)next << 32) | (uint32_t)code;
    const hipError_t e = hipMemcpyAsync((uint8_t *)g_ms.misc + 64, &v, 8, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("moe error word", e);
    return sync_stream("moe error word");
}

// ---------------------------------------------------------------- expert group kernels
// Items (expert record, input row) of the host-routed ABI path: h = silu(g x) * (u x),
// then y = d h, one launch each; nothing is combined (the caller weighs and accumulates).
struct EgItems {
    const ExpertRec *rec;     // [n] per item
    const float *x;           // rows [n_x, D]
    const int *xrow;          // [n] row of x per item
    float *h;                 // [n, I]
    float *y;                 // [n, D]
    int n;
    int gRows, nG, nD;
    MoeGeom g;
};

template <int LPR>
__global__ __launch_bounds__(kThreads) void eg_gateup_kernel(EgItems it) {
    __shared__ XPrep P;
    const MoeGeom &g = it.g;
    const int item = blockIdx.x / it.nG, r0 = (blockIdx.x % it.nG) * it.gRows;
    const int j = (threadIdx.x & 63) % LPR;
    XRegs xr;
    prep_load(it.x + (size_t)it.xrow[item] * g.D, g.D, g.nlG * kLaneChunks * 32, xr);
    prep_x(xr, g.gs, g.nlG * kLaneChunks * 32, P);
    LaneX<kLaneChunks> L;
    lane_geo<kLaneChunks>(j, g.nlG, g.D, g.gs, L);
    lane_x<kLaneChunks>(P, g.gs, L);
    float *h = it.h + (size_t)item * g.I;
    gateup_rows<LPR, kLaneChunks>(L, it.rec[item], g, r0, [&](int r, float v) { h[r] = v; });
}

template <int TPR>
__global__ __launch_bounds__(kThreads) void eg_down_kernel(EgItems it) {
    __shared__ HPrep H;
    const int item = blockIdx.x / it.nD, r0 = (blockIdx.x % it.nD) * kDRows;
    const float *hsrc = it.h + (size_t)item * it.g.I;
    float *y = it.y + (size_t)item * it.g.D;
    const int nw = it.g.I / 8;
    down_slot<TPR>(it.g, it.rec[item], H, r0,
                   [&](float (&hv)[kHWords][8]) {
#pragma unroll
                       for (int k = 0; k < kHWords; k++) {
                           const int q = threadIdx.x + k * kThreads;
#pragma unroll
                           for (int c = 0; c < 8; c++) hv[k][c] = q < nw ? hsrc[q * 8 + c] : 0.f;
                       }
                   },
                   [&](int r, float v) { y[r] = v; });
}

template <int LPRG, int TPRD>
struct LaunchEg {
    static bool run(EgItems &it, hipStream_t st) {
        it.gRows = kGSteps * kWaves * (64 / LPRG);
        it.nG = (it.g.I + it.gRows - 1) / it.gRows;
        it.nD = (it.g.D + kDRows - 1) / kDRows;
        hipLaunchKernelGGL(eg_gateup_kernel<LPRG>, dim3(it.n * it.nG), dim3(kThreads), 0, st, it);
        hipLaunchKernelGGL(eg_down_kernel<TPRD>, dim3(it.n * it.nD), dim3(kThreads), 0, st, it);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail("expert group launch", e);
        return true;
    }
};

// ---------------------------------------------------------------- expert group state
// One group in flight (c/backend_vulkan.c:1648).  Pinned staging holds rec | xrow | x | y.
struct EgGroup {
    int inflight = 0;
    size_t y_off = 0;
    PieceEvents y;            // the rows' read-back, in pieces
    void *d_buf = nullptr;
    size_t d_cap = 0;
    void *h_buf = nullptr;
    size_t h_cap = 0;
    void *d_xs = nullptr;     // bound prefill rows (coli_vk_eg_xs_bind)
    size_t d_xs_cap = 0;
    int xs_S = 0, xs_D = 0;
    uint64_t xs_key = 0;      // changes with every bind (names the bound rows' contents)
};
static EgGroup g_grp;

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// Rows > 1 (the engine's prefill: c/qwen.c:1099-1125, the shared expert over all rows
// :1149-1161) go to the grouped MFMA GEMMs, as the reference switches to its multi-row
// kernels there (c/backend_vulkan.c:1462-1466,1575-1585): each expert's weights stream once
// per unit of up to 32 rows instead of once per row.  Pinned staging holds
// units | xrow | x | y.
static bool eg_submit_mfma(ColiVkTensor *const *gates, ColiVkTensor *const *ups, ColiVkTensor *const *downs,
                           const int *rows, int count, int total, const MoeGeom &m, const float *x,
                           const int *tok_ids) {
    const int ur = eg_unit_rows(count, rows, m);
    int nunits = 0;
    for (int c = 0; c < count; c++) nunits += (rows[c] + ur - 1) / ur;
    const size_t un_b = al256((size_t)nunits * sizeof(PfUnit)), xrow_b = al256((size_t)total * 4);
    const size_t x_b = tok_ids ? 0 : al256((size_t)total * m.D * 4), y_b = (size_t)total * m.D * 4;
    if (!scratch(&g_grp.d_buf, &g_grp.d_cap, un_b + xrow_b + x_b + al256(y_b))) return false;
    if (!host_scratch(&g_grp.h_buf, &g_grp.h_cap, un_b + xrow_b + x_b + y_b)) return false;
    uint8_t *hb = (uint8_t *)g_grp.h_buf;
    PfUnit *hu = (PfUnit *)hb;
    int *hrow = (int *)(hb + un_b);
    for (int c = 0, p = 0, k = 0; c < count; c++) {
        const ExpertRec rec = {gates[c]->w, ups[c]->w, downs[c]->w, gates[c]->sz, ups[c]->sz, downs[c]->sz};
        for (int r = 0; r < rows[c]; r += ur, k++) {
            memset(&hu[k], 0, sizeof(PfUnit));
            hu[k].rec = rec;
            hu[k].pos0 = p + r;
            hu[k].n = rows[c] - r < ur ? rows[c] - r : ur;
        }
        for (int r = 0; r < rows[c]; r++, p++) {
            hrow[p] = tok_ids ? tok_ids[p] : p;
            if (hrow[p] < 0 || (tok_ids && hrow[p] >= g_grp.xs_S)) return false;
        }
    }
    if (!tok_ids) memcpy(hb + un_b + xrow_b, x, (size_t)total * m.D * 4);
    uint8_t *db = (uint8_t *)g_grp.d_buf;
    float *d_y = (float *)(db + un_b + xrow_b + x_b);
    hipError_t e = hipMemcpyAsync(db, hb, un_b + xrow_b + x_b, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("expert group upload", e);
    const float *src = tok_ids ? (const float *)g_grp.d_xs : (const float *)(db + un_b + xrow_b);
    if (!eg_mfma((const PfUnit *)db, nunits, (const int *)(db + un_b), total, m, src, tok_ids ? g_grp.xs_S : total,
                 tok_ids ? g_grp.xs_key : 0, d_y, stream()))
        return false;
    g_grp.y_off = un_b + xrow_b + x_b;
    if (!issue_pieces(g_grp.y, hb + g_grp.y_off, d_y, y_b, stream())) return false;
    g_grp.inflight = 1;
    return true;
}

// Validate a group (c/backend_vulkan.c:1418-1440) and issue it.  tok_ids != NULL: rows
// come from the bound xs; otherwise x is packed [sum(rows), D].  Groups of one row per
// expert run the GEMV kernels (batch-1 decode arithmetic); any expert with more rows sends
// the whole group to the MFMA path (eg_submit_mfma), unless coli_hip_eg_path forced GEMV.
static int g_eg_force_gemv = 0;
static bool eg_submit(ColiVkTensor *const *gates, ColiVkTensor *const *ups, ColiVkTensor *const *downs,
                      const int *rows, int count, const float *x, const int *tok_ids) {
    if (!ok() || count < 1 || count > 64 || !gates || !ups || !downs || !rows) return false;
    MoeGeom m;
    if (!geom_of(gates[0], downs[0], m)) return false;
    int total = 0, max_rows = 0;
    for (int c = 0; c < count; c++) {
        MoeGeom mc, mu;
        if (rows[c] < 1 || !geom_of(gates[c], downs[c], mc) || !same_geom(mc, m) || !ups[c] ||
            !geom_of(ups[c], downs[c], mu) || !same_geom(mu, m))
            return false;
        if (rows[c] > (1 << 24) - total) return false;
        total += rows[c];
        max_rows = rows[c] > max_rows ? rows[c] : max_rows;
    }
    if (tok_ids && (!g_grp.d_xs || g_grp.xs_D != m.D)) return false;
    if (max_rows > 1 && !g_eg_force_gemv && eg_mfma_ok(m))
        return eg_submit_mfma(gates, ups, downs, rows, count, total, m, x, tok_ids);
    if (!geom_supported(m)) return false;
    const size_t rec_b = al256((size_t)total * sizeof(ExpertRec)), xrow_b = al256((size_t)total * 4);
    const size_t x_b = tok_ids ? 0 : al256((size_t)total * m.D * 4);
    const size_t h_b = al256((size_t)total * m.I * 4), y_b = (size_t)total * m.D * 4;
    if (!scratch(&g_grp.d_buf, &g_grp.d_cap, rec_b + xrow_b + x_b + h_b + al256(y_b))) return false;
    if (!host_scratch(&g_grp.h_buf, &g_grp.h_cap, rec_b + xrow_b + x_b + y_b)) return false;
    uint8_t *hb = (uint8_t *)g_grp.h_buf;
    ExpertRec *hrec = (ExpertRec *)hb;
    int *hrow = (int *)(hb + rec_b);
    for (int c = 0, p = 0; c < count; c++)
        for (int r = 0; r < rows[c]; r++, p++) {
            hrec[p] = {gates[c]->w, ups[c]->w, downs[c]->w, gates[c]->sz, ups[c]->sz, downs[c]->sz};
            hrow[p] = tok_ids ? tok_ids[p] : p;
            if (hrow[p] < 0 || (tok_ids && hrow[p] >= g_grp.xs_S)) return false;
        }
    if (!tok_ids) memcpy(hb + rec_b + xrow_b, x, (size_t)total * m.D * 4);
    uint8_t *db = (uint8_t *)g_grp.d_buf;
    EgItems it;
    memset(&it, 0, sizeof(it));
    it.rec = (const ExpertRec *)db;
    it.xrow = (const int *)(db + rec_b);
    it.x = tok_ids ? (const float *)g_grp.d_xs : (const float *)(db + rec_b + xrow_b);
    it.h = (float *)(db + rec_b + xrow_b + x_b);
    it.y = (float *)(db + rec_b + xrow_b + x_b + h_b);
    it.n = total;
    it.g = m;
    hipError_t e = hipMemcpyAsync(db, hb, rec_b + xrow_b + x_b, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("expert group upload", e);
    if (!dispatch_shape<LaunchEg>(m, it, stream())) return false;
    g_grp.y_off = rec_b + xrow_b + x_b;
    if (!issue_pieces(g_grp.y, hb + g_grp.y_off, it.y, y_b, stream())) return false;
    g_grp.inflight = 1;
    return true;
}

// The rows come back in pieces (issue_pieces at issue time); each is copied out as soon as
// it has arrived.
static bool eg_take(float *y) {
    if (!g_grp.inflight) return false;
    g_grp.inflight = 0;
    return copy_out(g_grp.y, y, (uint8_t *)g_grp.h_buf + g_grp.y_off, "expert group take");
}

__global__ void silu_mul_kernel(const float *g, const float *u, float *h, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float gv = g[i];
        h[i] = gv / (1.f + expf(-gv)) * u[i];
    }
}

static void *g_gu_d = nullptr, *g_gu_h = nullptr;
static size_t g_gu_dc = 0, g_gu_hc = 0;

void moe_shutdown() {
    free(g_eg.h_rec);
    free(g_eg.valid);
    g_eg = EgTable();   // the device table lived in the arena
    scratch_free(&g_ms.tag, &g_ms.tag_cap);
    scratch_free(&g_ms.misc, &g_ms.misc_cap);
    g_ms.epoch = 0;
    scratch_free(&g_grp.d_buf, &g_grp.d_cap);
    host_scratch_free(&g_grp.h_buf, &g_grp.h_cap);
    scratch_free(&g_grp.d_xs, &g_grp.d_xs_cap);
    piece_events_free(g_grp.y);
    g_grp = EgGroup();
    scratch_free(&g_gu_d, &g_gu_dc);
    host_scratch_free(&g_gu_h, &g_gu_hc);
}

}  // namespace coli

using namespace coli;

extern "C" int coli_vk_tensor_ensure(ColiVkTensor **, const void *, const float *, int, int, int, int);

// ---------------------------------------------------------------- ABI: expert group
// c/backend_vulkan.h:85-101, c/backend_vulkan.c:1645-1697.  Gate/up/down must be fmt 6
// in the lanes layout (D <= 4096, I <= 1024, gs % 64 == 0); otherwise 0 (the caller
// computes on the CPU, as it does when the reference rejects a group).
COLI_API int coli_vk_expert_group_issue(ColiVkTensor *const *gates, ColiVkTensor *const *ups,
                                        ColiVkTensor *const *downs, const int *rows, int count, const float *x) {
    if (g_grp.inflight || !x) return 0;
    return eg_submit(gates, ups, downs, rows, count, x, nullptr) ? 1 : 0;
}

COLI_API int coli_vk_expert_group_take(float *y) { return y && eg_take(y) ? 1 : 0; }

COLI_API int coli_hip_eg_force_gemv(int force_gemv) {
    const int prev = g_eg_force_gemv;
    g_eg_force_gemv = force_gemv ? 1 : 0;
    return prev;
}

COLI_API int coli_vk_expert_group(ColiVkTensor *const *gates, ColiVkTensor *const *ups, ColiVkTensor *const *downs,
                                  const int *rows, int count, float *y, const float *x) {
    if (g_grp.inflight || !x || !y) return 0;
    if (!eg_submit(gates, ups, downs, rows, count, x, nullptr)) return 0;
    return eg_take(y) ? 1 : 0;
}

COLI_API int coli_vk_eg_gather_available(void) { return ok() ? 1 : 0; }

// c/backend_vulkan.c:1656-1666: bind the prefill rows once; issue_id then names rows
COLI_API int coli_vk_eg_xs_bind(const float *xs, int S, int D) {
    if (!ok() || !xs || S < 1 || D < 1 || g_grp.inflight) return 0;
    const size_t xb = (size_t)S * D * 4;
    if (!scratch(&g_grp.d_xs, &g_grp.d_xs_cap, xb)) return 0;
    const Upload u = {g_grp.d_xs, xs, xb};
    if (!upload(&u, 1, stream(), "xs bind")) return 0;
    g_grp.xs_S = S;
    g_grp.xs_D = D;
    static uint64_t binds = 0;
    g_grp.xs_key = ++binds;
    return 1;
}

COLI_API int coli_vk_expert_group_issue_id(ColiVkTensor *const *gates, ColiVkTensor *const *ups,
                                           ColiVkTensor *const *downs, const int *rows, int count,
                                           const int *tok_ids) {
    if (g_grp.inflight || !tok_ids) return 0;
    return eg_submit(gates, ups, downs, rows, count, nullptr, tok_ids) ? 1 : 0;
}

// c/backend_vulkan.h:75-79, c/backend_vulkan.c:1300-1344: hidden[s, o] = silu(gate x_s) * up x_s
COLI_API int coli_vk_gate_up(ColiVkTensor **gate, ColiVkTensor **up, float *hidden, const float *x, const void *gw,
                             const float *gsc, const void *uw, const float *usc, int fmt, int S, int D, int I,
                             int grp) {
    if (!gate || !up || !hidden || !x || S < 1 || D < 1 || I < 1) return 0;
    if (!coli_vk_tensor_ensure(gate, gw, gsc, fmt, D, I, grp) || !coli_vk_tensor_ensure(up, uw, usc, fmt, D, I, grp))
        return 0;
    const size_t xb = (size_t)S * D * 4, hb = (size_t)S * I * 4;
    if (!scratch(&g_gu_d, &g_gu_dc, al256(xb) + 3 * al256(hb)) || !host_scratch(&g_gu_h, &g_gu_hc, xb > hb ? xb : hb))
        return 0;
    uint8_t *db = (uint8_t *)g_gu_d;
    float *dx = (float *)db, *dg = (float *)(db + al256(xb)), *du = (float *)(db + al256(xb) + al256(hb));
    float *dh = (float *)(db + al256(xb) + 2 * al256(hb));
    memcpy(g_gu_h, x, xb);
    hipError_t e = hipMemcpyAsync(dx, g_gu_h, xb, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("gate_up upload", e) ? 1 : 0;
    if (!gemv(*gate, dx, dg, S, stream()) || !gemv(*up, dx, du, S, stream())) return 0;
    const size_t n = (size_t)S * I;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream(), dg, du, dh, n);
    e = hipMemcpyAsync(g_gu_h, dh, hb, hipMemcpyDeviceToHost, stream());
    if (e == hipSuccess) e = hipStreamSynchronize(stream());
    if (e != hipSuccess) return fail("gate_up", e) ? 1 : 0;
    memcpy(hidden, g_gu_h, hb);
    return 1;
}

// ---------------------------------------------------------------- ABI: expert table
// c/backend_vulkan.h:243-252, c/backend_vulkan.c:3019-3091: slot [layer][eid], the shared
// expert at eid = E, plus the layer's shared-expert gate vector.  All experts of a layer
// must be set before the layer's indexed MoE runs (every expert stays resident in HBM).
COLI_API int coli_vk_moe_ix_available(void) { return ok() ? 1 : 0; }

// Calling init again re-dimensions the table and clears every slot (as the reference,
// :3028-3049); the old device arrays are kept when they are large enough.
COLI_API int coli_vk_eg_table_init(int n_layers, int E, int D, int I, int gs) {
    EgTable &T = g_eg;
    if (!ok() || n_layers < 1 || E < 1 || E > kMaxE || D < 1 || I < 1 || gs < 8) return 0;
    const size_t nrec = (size_t)n_layers * (E + 1), nsg = (size_t)n_layers * D;
    if (!sync_stream("expert table")) return 0;   // launches in flight may read the table
    if (nrec > T.rec_cap) {
        ExpertRec *d_rec = (ExpertRec *)arena_alloc(nrec * sizeof(ExpertRec));
        ExpertRec *h_rec = (ExpertRec *)calloc(nrec, sizeof(ExpertRec));
        uint8_t *valid = (uint8_t *)calloc(nrec, 1);
        if (!d_rec || !h_rec || !valid) {
            free(h_rec);
            free(valid);
            return 0;
        }
        free(T.h_rec);
        free(T.valid);
        T.d_rec = d_rec;
        T.h_rec = h_rec;
        T.valid = valid;
        T.rec_cap = nrec;
    }
    if (nsg > T.sg_cap) {
        float *d_sg = (float *)arena_alloc(nsg * 4);
        if (!d_sg) return 0;
        T.d_shgate = d_sg;
        T.sg_cap = nsg;
    }
    memset(T.valid, 0, T.rec_cap);
    T.geom_set = 0;
    T.n_layers = n_layers;
    T.E = E;
    T.D = D;
    T.I = I;
    T.gs = gs;
    return 1;
}

namespace coli {
// Would slot (layer, eid) of the current table take these tensors (eid == E: the shared
// expert)?  The table's dimensions, the fmt 6 lanes layout and the geometry of the slots
// already set must match.
bool eg_table_check(int layer, int eid, const ColiVkTensor *g, const ColiVkTensor *u, const ColiVkTensor *d,
                    MoeGeom *out) {
    const EgTable &T = g_eg;
    if (!ok() || !T.d_rec || layer < 0 || layer >= T.n_layers || eid < 0 || eid > T.E || !g || !u || !d) return false;
    MoeGeom m, mu;
    if (!geom_of(g, d, m) || !geom_of(u, d, mu) || !same_geom(m, mu) || !geom_supported(m)) return false;
    if (m.D != T.D || m.I != T.I || m.gs != T.gs) return false;
    if (T.geom_set && !same_geom(m, T.geom)) return false;
    if (out) *out = m;
    return true;
}

bool eg_table_dims(int layer, int E, int D, int I, int gs) {
    const EgTable &T = g_eg;
    return ok() && T.d_rec && layer >= 0 && layer < T.n_layers && E >= 1 && E <= T.E && D == T.D && I == T.I &&
           gs == T.gs;
}
}  // namespace coli

static int eg_table_put(int layer, int eid, ColiVkTensor *g, ColiVkTensor *u, ColiVkTensor *d) {
    EgTable &T = g_eg;
    MoeGeom m;
    if (!eg_table_check(layer, eid, g, u, d, &m)) return 0;
    T.geom = m;
    T.geom_set = 1;
    const size_t i = (size_t)layer * (T.E + 1) + eid;
    T.h_rec[i] = {g->w, u->w, d->w, g->sz, u->sz, d->sz};
    // stream-ordered after any launch that still reads the table
    const hipError_t e = hipMemcpyAsync(T.d_rec + i, &T.h_rec[i], sizeof(ExpertRec), hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("expert table", e) ? 1 : 0;
    if (!sync_stream("expert table")) return 0;
    T.valid[i] = 1;
    return 1;
}

COLI_API int coli_vk_eg_table_set(int layer, int eid, ColiVkTensor *g, ColiVkTensor *u, ColiVkTensor *d) {
    if (eid < 0 || eid >= g_eg.E) return 0;
    return eg_table_put(layer, eid, g, u, d);
}

COLI_API int coli_vk_eg_table_set_shared(int layer, ColiVkTensor *g, ColiVkTensor *u, ColiVkTensor *d,
                                         const float *sh_gate, int D) {
    EgTable &T = g_eg;
    if (!sh_gate || D != T.D || !eg_table_put(layer, T.E, g, u, d)) return 0;
    const hipError_t e =
        hipMemcpyAsync(T.d_shgate + (size_t)layer * T.D, sh_gate, (size_t)D * 4, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("shared gate upload", e) ? 1 : 0;
    return sync_stream("shared gate upload") ? 1 : 0;
}

// ---------------------------------------------------------------- ABI: expert group (pipe)
// c/backend_vulkan.h:237-240, c/backend_vulkan.c:3696-3783: the stream-routed expert group
// of c/qwen.c:934-998.  Every row takes the last route's device nrm as input; the
// outputs are weighted and added to the device residual in item order:
//   resid[d] += sum_c weights[c] * y_c[d]
// (c/shaders/moe_accumulate.comp; the engine lists the routed experts in rank order and
// the shared expert last, as the CPU path sums them, c/qwen.c:870-877).  Stream-ordered:
// take_pipe has nothing left to wait for.
__global__ void eg_accumulate(float *resid, const float *y, const float *w, int n, int D) {
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    float acc = 0.f;
    for (int c = 0; c < n; c++) acc += w[c] * y[(size_t)c * D + d];
    resid[d] = resid[d] + acc;
}

COLI_API int coli_vk_expert_group_issue_pipe(ColiVkTensor *const *gates, ColiVkTensor *const *ups,
                                             ColiVkTensor *const *downs, const int *rows, const float *weights,
                                             int count, int D) {
    float *resid = stream_resid(D);
    const float *x = stream_nrm_dev(D);
    if (!ok() || !resid || !x || !weights || g_grp.inflight || count < 1 || count > 64 || !gates || !ups || !downs ||
        !rows)
        return 0;
    MoeGeom m;
    if (!geom_of(gates[0], downs[0], m) || !geom_supported(m) || m.D != D) return 0;
    int total = 0;
    for (int c = 0; c < count; c++) {
        MoeGeom mc, mu;
        if (rows[c] < 1 || !geom_of(gates[c], downs[c], mc) || !same_geom(mc, m) || !ups[c] ||
            !geom_of(ups[c], downs[c], mu) || !same_geom(mu, m))
            return 0;
        total += rows[c];
    }
    const size_t rec_b = al256((size_t)total * sizeof(ExpertRec)), xrow_b = al256((size_t)total * 4);
    const size_t w_b = al256((size_t)total * 4), h_b = al256((size_t)total * m.I * 4), y_b = (size_t)total * m.D * 4;
    if (!scratch(&g_grp.d_buf, &g_grp.d_cap, rec_b + xrow_b + w_b + h_b + al256(y_b))) return 0;
    if (!host_scratch(&g_grp.h_buf, &g_grp.h_cap, rec_b + xrow_b + w_b)) return 0;
    if (!sync_stream("expert group pipe")) return 0;   // the pinned staging may still feed a copy
    uint8_t *hb = (uint8_t *)g_grp.h_buf;
    ExpertRec *hrec = (ExpertRec *)hb;
    int *hrow = (int *)(hb + rec_b);
    float *hw = (float *)(hb + rec_b + xrow_b);
    for (int c = 0, p = 0; c < count; c++)
        for (int r = 0; r < rows[c]; r++, p++) {
            hrec[p] = {gates[c]->w, ups[c]->w, downs[c]->w, gates[c]->sz, ups[c]->sz, downs[c]->sz};
            hrow[p] = 0;
            hw[p] = weights[c];
        }
    uint8_t *db = (uint8_t *)g_grp.d_buf;
    EgItems it;
    memset(&it, 0, sizeof(it));
    it.rec = (const ExpertRec *)db;
    it.xrow = (const int *)(db + rec_b);
    it.x = x;
    it.h = (float *)(db + rec_b + xrow_b + w_b);
    it.y = (float *)(db + rec_b + xrow_b + w_b + h_b);
    it.n = total;
    it.g = m;
    hipError_t e = hipMemcpyAsync(db, hb, rec_b + xrow_b + w_b, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail("expert group pipe upload", e) ? 1 : 0;
    if (!dispatch_shape<LaunchEg>(m, it, stream())) return 0;
    hipLaunchKernelGGL(eg_accumulate, dim3((D + 255) / 256), dim3(256), 0, stream(), resid, it.y,
                       (const float *)(db + rec_b + xrow_b), total, D);
    e = hipGetLastError();
    if (e != hipSuccess) return fail("expert group pipe", e) ? 1 : 0;
    return 1;
}

COLI_API int coli_vk_expert_group_take_pipe(void) { return ok() ? 1 : 0; }


// ---------------------------------------------------------------- device-pointer MoE
// The layer's whole MoE block in one launch on `stream` (NULL = the library's stream):
// out = sum_k val_k y_k + shgt y_sh (accumulate != 0: out += that).  d_idx [K] and d_val
// [K + 1] (renormed weights, then shgt) are optional.  Launches share one scratch area:
// issue them on one stream.
COLI_API int coli_hip_moe_decode(int layer, const ColiVkTensor *router, int K, const float *d_x, float *d_out,
                                 int accumulate, int *d_idx, float *d_val, void *stream_) {
    return moe_decode(layer, router, K, d_x, d_out, accumulate, d_idx, d_val,
                      stream_ ? (hipStream_t)stream_ : stream())
               ? 1
               : 0;
}

// Error flag of the MoE launches since the last call (synchronizes the device):
// 0 none, 1 a poll gave up, 2 a route held an out-of-range expert id, -1 runtime error.
COLI_API int coli_hip_moe_error(void) { return moe_error_take(); }

// The same block with no allocation: cross-block words in a static device array.
COLI_API int coli_hip_moe_decode_noalloc(int layer, const ColiVkTensor *router, int K, const float *d_x,
                                         float *d_out, int accumulate, int *d_idx, float *d_val, void *stream_) {
    return moe_decode_noalloc(layer, router, K, d_x, d_out, accumulate, d_idx, d_val,
                              stream_ ? (hipStream_t)stream_ : stream())
               ? 1
               : 0;
}

// Test hook: set the error word from the host (see moe_error_force).
COLI_API int coli_hip_moe_force_error(int code) { return moe_error_force(code) ? 1 : 0; }
