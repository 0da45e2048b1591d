// prefill.hip - the MoE block over S tokens at once (prefill / ragged batch), with the
// expert projections as grouped GEMMs on MFMA.
//
// Semantics: c/qwen.c:1050-1183 (moe_batch_from_logits): route every token (softmax,
// top-K, renorm; c/qwen.c:1057-1072), group the (token, slot) pairs by expert
// (c/qwen.c:1076-1083), run each expert's MLP over its rows, then
//   out[t] = sum over t's experts in ascending expert id of w * y   (c/qwen.c:1144)
//   out[t] += shgt[t] * y_shared[t]                                  (c/qwen.c:1159-1161)
//
// Arithmetic of the projections: the same grouped form as the decode GEMV,
//   y[r] = sum_g s_g * (sum_{i in g} x_i n'_i - (z_g - 8) * sum_{i in g} x_i),  n' = n - 8,
// with x in block fixed point per (row of x, group): q = rint(x 2^(22-e)), split into
// three balanced base-256 digits.  n' (int8) times each digit plane is an exact integer
// product on v_mfma_i32_16x16x64_i8; the three sums recombine in fp32 per group.
//
// MFMA mapping (v_mfma_i32_16x16x64_i8): A = 16 weight rows x 64 K (int8), B = 64 K x 16
// rows of x (int8 digits), D = 16 x 16 int32 with lane l, register r holding
// D[4 (l / 16) + r][l % 16].  Any permutation of K shared by A and B gives the same
// product: lane l carries the 16 K positions 16 (l / 16) .. + 15 of the 64-column chunk
// in the order [0 2 4 6 1 3 5 7 8 10 12 14 9 11 13 15], which is how the weight nibbles
// fall out of a 32-bit word after masking even and odd nibbles.  The x digit planes are
// stored in that order (perm16).
//
// Launches: pf_logits (router logits, the reference's bits) -> pf_route (per token: logits,
// routing, shared gate, x digit planes) -> pf_group (positions per expert) -> pf_gateup
// (gate/up + SwiGLU) -> pf_digits (h as digit planes) -> pf_down -> pf_combine.
#include "moe_common.h"

#include <stdio.h>
#include <string.h>

#include <type_traits>

namespace coli {

typedef int pf_v4i __attribute__((ext_vector_type(4)));

constexpr int kGS = 128;               // group size of the MFMA path
constexpr int kPT = 256;               // threads of the projection kernels (4 waves)
constexpr int kPW = kPT / 64;
constexpr int kPR = 32;                // x rows per pass (two 16-row MFMA tiles)
constexpr int kPitch = kGS + 16;       // LDS bytes per staged row of one group (conflict-free B reads)
constexpr int kGU = kPW * 16;          // gate/up: h columns per block (64)
constexpr int kDT = 4;                 // down: 16-row tiles per wave
constexpr int kDR = kPW * kDT * 16;    // down: output rows per block (256)
constexpr int kDG = 4;                 // down: groups of h staged at a time (one weight superstep)
constexpr int kDPitch = kDG * kGS + 16;

// byte position of K offset o (0..15) inside a 16-byte block of digit plane
__device__ __forceinline__ int perm16(int o) {
    const int h = o & 8, r = o & 7;
    return h + ((r & 1) ? 4 + (r >> 1) : (r >> 1));
}

// A operand of one MFMA from 16 nibbles (two words).  A stored nibble (n XOR 8) is the
// 4-bit two's complement of n' = n - 8, so a nibble in the high half of its byte reads as
// the int8 16 n'.  Bytes: the low nibbles of w0 (K order 0 2 4 6), its high nibbles
// (1 3 5 7), then w1's (8 10 12 14, 9 11 13 15).  Products and sums carry the factor 16,
// which the fold removes exactly through the exponent.
__device__ __forceinline__ pf_v4i pf_a16(uint32_t w0, uint32_t w1) {
    return pf_v4i{(int)((w0 << 4) & 0xF0F0F0F0u), (int)(w0 & 0xF0F0F0F0u), (int)((w1 << 4) & 0xF0F0F0F0u),
                  (int)(w1 & 0xF0F0F0F0u)};
}

// Block fixed point of 8 consecutive columns (col % 8 == 0) of one row.  The 16 aligned
// consecutive lanes holding one 128-column group agree on its exponent by shuffles:
// e = ilogb(max |v|) + 1 (0 for an all-zero group), q = rint(v 2^(22-e)) in balanced
// base-256 digits d0 + 256 d1 + 65536 d2.  Writes the 8 bytes of each plane at
// dst + d * pstride (perm16 order) and, from the group's first lane, ge = e - 22 and
// gsum = 2^(e-22) sum q.  Lanes with valid = false join the shuffles and write nothing.
__device__ __forceinline__ void digit8(const float (&v)[8], bool valid, int col, int8_t *dst, size_t pstride,
                                       int *ge, float *gsum) {
    float m = 0.f;
#pragma unroll
    for (int c = 0; c < 8; c++) m = fmaxf(m, fabsf(v[c]));
    uint32_t mu = __float_as_uint(m);
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mu = max(mu, (uint32_t)__shfl_xor((int)mu, o));
    const float mf = __uint_as_float(mu);
    const int e = mf > 0.f ? ilogbf(mf) + 1 : 0;
    int qs = 0;
    uint32_t pl[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const int q = (int)rintf(ldexpf(v[c], 22 - e));
        qs += q;
        const uint32_t u = (uint32_t)(q + 0x808080);   // digits d + 128
        const int pos = perm16((col + c) & 15) & 7;     // within this 8-byte half
#pragma unroll
        for (int d = 0; d < 3; d++) pl[d][pos >> 2] |= ((((u >> (8 * d)) & 255u) ^ 0x80u)) << (8 * (pos & 3));
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) qs += __shfl_xor(qs, o);
    if (valid) {
#pragma unroll
        for (int d = 0; d < 3; d++) *(uint2 *)(dst + d * pstride) = make_uint2(pl[d][0], pl[d][1]);
        if ((col & (kGS - 1)) == 0) {
            *ge = e - 22;
            *gsum = ldexpf((float)qs, e - 22);
        }
    }
}

// ---------------------------------------------------------------- router logits
// lg[t][e] = the reference's router logit of token t, bit for bit: acc += x[t][k] w[e][k]
// for k in index order, fp32 products and sums, no contraction (c/qwen.c:178-189); int8
// rows (rfmt 1) convert each weight and multiply acc by the row scale after the sum
// (c/qwen.c:230-238).  One output per thread, 16 tokens x 16 experts per block of 256
// threads; x and w tiles of kLC columns staged in LDS (double buffered), read as float4
// (4 k per read, each lane's k order unchanged).  A tile's global loads go out when the
// tile before it starts, so they have its kLC steps of adds to arrive in (64-column tiles
// waited on their loads at every tile: 34 against 29.5 us at configs[4]).
constexpr int kLT = 16, kLE = 16, kLC = 256, kLS = kLC / 4 / 16;   // float4 per staged row and thread
__global__ __launch_bounds__(256) void pf_logits(const float *__restrict__ xs, int S, int D,
                                                 const uint8_t *__restrict__ rw, const float *__restrict__ rs,
                                                 int rfmt, int rrb, int E, float *__restrict__ lg) {
    __shared__ __attribute__((aligned(16))) float s_x[2][kLT][kLC + 4];
    __shared__ __attribute__((aligned(16))) float s_w[2][kLE][kLC + 4];
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
    const int t0 = blockIdx.x * kLT, e0 = blockIdx.y * kLE;
    // staging: thread tid stages float4 (tid & 15) + 16 j of row tid >> 4 for x and for w
    const int sr = tid >> 4, sc = 4 * (tid & 15);
    float4 rx[kLS], rv[kLS];
    auto load = [&](int kc) {
        const int t = t0 + sr, e = e0 + sr;
#pragma unroll
        for (int j = 0; j < kLS; j++) {
            const int k = kc + sc + 64 * j;
            rx[j] = (t < S && k < D) ? *(const float4 *)(xs + (size_t)t * D + k) : make_float4(0.f, 0.f, 0.f, 0.f);
            if (e >= E || k >= D) {
                rv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            } else if (rfmt == 0) {
                rv[j] = *(const float4 *)(rw + (size_t)e * rrb + 4 * (size_t)k);
            } else {
                const char4 c = *(const char4 *)(rw + (size_t)e * rrb + k);
                rv[j] = make_float4((float)c.x, (float)c.y, (float)c.z, (float)c.w);
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < kLS; j++) {
            *(float4 *)&s_x[buf][sr][sc + 64 * j] = rx[j];
            *(float4 *)&s_w[buf][sr][sc + 64 * j] = rv[j];
        }
    };
    float acc = 0.f;
    load(0);
    store(0);
    __syncthreads();
    for (int kc = 0, buf = 0; kc < D; kc += kLC, buf ^= 1) {
        const bool more = kc + kLC < D;
        if (more) load(kc + kLC);
        const int n = D - kc < kLC ? D - kc : kLC;   // D % 4 == 0
#pragma unroll 8
        for (int k = 0; k < n; k += 4) {
            const float4 a = *(const float4 *)&s_x[buf][ty][k];
            const float4 w = *(const float4 *)&s_w[buf][tx][k];
            acc = __fadd_rn(acc, __fmul_rn(a.x, w.x));
            acc = __fadd_rn(acc, __fmul_rn(a.y, w.y));
            acc = __fadd_rn(acc, __fmul_rn(a.z, w.z));
            acc = __fadd_rn(acc, __fmul_rn(a.w, w.w));
        }
        if (more) store(buf ^ 1);
        __syncthreads();
    }
    const int t = t0 + ty, e = e0 + tx;
    if (t < S && e < E) lg[(size_t)t * E + e] = rfmt == 1 ? __fmul_rn(acc, rs[e]) : acc;
}

// ---------------------------------------------------------------- route per token
// One block per token: the routing (route_wave) of the token's reference logits, the
// shared expert's gate sigmoid(x . sh_gate) (fp64 dot; c/qwen.c:1159), and x's digit
// planes for the projections ([3][S][D] planes, [S][D/128] exponents and sums).
__global__ __launch_bounds__(kThreads) void pf_route(const float *__restrict__ lg, const float *__restrict__ xs,
                                                    int S, int D, const float *__restrict__ sh_gate, int E, int K,
                                                    int *tidx, float *tval, float *tshg, int8_t *__restrict__ xd,
                                                    int *__restrict__ xe, float *__restrict__ xsum) {
    __shared__ RouteLds R;
    __shared__ double s_red[kWaves];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (wave == 0) {   // one wave routes while the others start on the digit planes
        for (int e = lane; e < E; e += 64) R.p[e] = lg[(size_t)t * E + e];
        wave_lds_order();
        route_wave(R, E, K);
        if (lane < K) {
            tidx[t * K + lane] = R.idx[lane];
            tval[t * K + lane] = R.val[lane] / R.vsum;
        }
    }
    const float *x = xs + (size_t)t * D;
    const int ngD = D / kGS;
    double g = 0.0;
    for (int c8 = tid; c8 < D / 8; c8 += kThreads) {   // D / 8 is a multiple of 16: whole groups
        float v[8];
        const float4 a = *(const float4 *)(x + 8 * c8), b = *(const float4 *)(x + 8 * c8 + 4);
        const float4 sa = *(const float4 *)(sh_gate + 8 * c8), sb = *(const float4 *)(sh_gate + 8 * c8 + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        const float sg[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
#pragma unroll
        for (int c = 0; c < 8; c++) g = fma((double)v[c], (double)sg[c], g);
        const int gi = (8 * c8) / kGS;
        digit8(v, true, 8 * c8, xd + (size_t)t * D + 8 * c8, (size_t)S * D, xe + (size_t)t * ngD + gi,
               xsum + (size_t)t * ngD + gi);
    }
    g = wave_sum_dpp(g);
    if (lane == 0) s_red[wave] = g;
    __syncthreads();
    if (tid == 0) {
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) s += s_red[w];
        R.gate = (float)s;
    }
    if (tid == 0) tshg[t] = 1.f / (1.f + expf(-R.gate));
}

// ---------------------------------------------------------------- grouping
// off[e] = first position of expert e's rows, off[E] = S*K; plist[p] = pair index
// (token * K + slot) at position p; ppos[pair] = its position.  Rows of one expert are
// independent, so their order within the expert does not change any result.  E <= 1024.
__global__ __launch_bounds__(1024) void pf_group(const int *tidx, int npairs, int E, int *off, int *plist,
                                                 int *ppos, int *rank) {
    __shared__ int s_cnt[kMaxE];
    __shared__ int s_wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < E; e += 1024) s_cnt[e] = 0;
    __syncthreads();
    constexpr int kB = 4;   // pairs per thread and batch, their loads in flight together
    for (int i0 = tid; i0 < npairs; i0 += 1024 * kB) {
        int e[kB];
#pragma unroll
        for (int k = 0; k < kB; k++) e[k] = i0 + 1024 * k < npairs ? tidx[i0 + 1024 * k] : 0;
#pragma unroll
        for (int k = 0; k < kB; k++)
            if (i0 + 1024 * k < npairs) rank[i0 + 1024 * k] = atomicAdd(&s_cnt[e[k]], 1);
    }
    __syncthreads();
    // exclusive scan of the counts: inclusive per wave, then the wave totals
    const int c = tid < E ? s_cnt[tid] : 0;
    int inc = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o);
        if (lane >= o) inc += v;
    }
    if (lane == 63) s_wsum[wave] = inc;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; w++) base += s_wsum[w];
    const int excl = base + inc - c;
    if (tid < E) {
        off[tid] = excl;
        s_cnt[tid] = excl;
    }
    if (tid == 1023) off[E] = base + inc;   // the last thread's inclusive sum is the total
    __syncthreads();
    for (int i0 = tid; i0 < npairs; i0 += 1024 * kB) {
        int e[kB], rk[kB];
#pragma unroll
        for (int k = 0; k < kB; k++) {
            const bool on = i0 + 1024 * k < npairs;
            e[k] = on ? tidx[i0 + 1024 * k] : 0;
            rk[k] = on ? rank[i0 + 1024 * k] : 0;
        }
#pragma unroll
        for (int k = 0; k < kB; k++) {
            const int i = i0 + 1024 * k;
            if (i >= npairs) continue;
            const int p = s_cnt[e[k]] + rk[k];
            plist[p] = i;
            ppos[i] = p;
        }
    }
}

// ---------------------------------------------------------------- projections
struct PfArgs {
    const ExpertRec *rec;   // [E + 1], the shared expert last
    const int *off;         // [E + 1] first position per expert (routed)
    const int *plist;       // position -> pair (token = pair / K)
    const PfUnit *units;    // host-routed form: [nunits] units (rec, off and the shared expert unused)
    int nunits;
    int E, S, K, D, I;
    int P;                  // positions (rows of h and y)
    int nlG, rbG, nlD, rbD;   // lanes layout: lanes per row, row bytes (gate/up, down)
    int nsp;                  // shared-expert passes: ceil(S / kPR)
    const int8_t *xd;         // x digit planes [3][S][D]
    const int *xe;            // [S][D / 128]
    const float *xsum;
    float *h;                 // [P][I] SwiGLU output per position, P = S K + S
    const int8_t *hd;         // h digit planes [3][P][I]
    const int *he;            // [P][I / 128]
    const float *hsum;
    float *y;                 // [P][D] expert outputs per position
};

// Block b of a projection launch -> (expert e, unit u, passes [p0, p1)).  Blocks
// [0, nu nsp) are the shared expert's units, one pass each (u = b % nu); the count is
// rounded up to a multiple of 8 with idle blocks; the rest are routed (e, u) with all of
// e's passes, placed so that the nu units of one expert run on one XCD (workgroups are
// dealt to the 8 XCDs round-robin by index) and share its rows of x in that L2.
// False for an idle block (or a routed expert without rows).
// Host-routed form: block b -> unit 8 (b / 8 / nu) + b % 8, u = (b / 8) % nu, one pass.
__device__ __forceinline__ bool pf_unit(const PfArgs &a, int nu, int &e, int &u, int &p0, int &p1, int &pos0,
                                        int &n, ExpertRec &rec) {
    if (a.units) {
        const int b = blockIdx.x, rest = b >> 3, ui = 8 * (rest / nu) + (b & 7);
        u = rest % nu;
        if (ui >= a.nunits) return false;
        const PfUnit &un = a.units[ui];
        rec = un.rec;
        pos0 = un.pos0;
        n = un.n;
        e = 0;
        p0 = 0;
        p1 = 1;
        return n > 0;
    }
    const int b = blockIdx.x, nsu = nu * a.nsp, nsu8 = (nsu + 7) & ~7;
    if (b < nsu) {
        e = a.E;
        u = b % nu;
        p0 = b / nu;
        p1 = p0 + 1;
        pos0 = a.S * a.K;
        n = a.S;
        rec = a.rec[e];
        return true;
    }
    if (b < nsu8) return false;
    const int r = b - nsu8, xcd = r & 7, rest = r >> 3;
    u = rest % nu;
    e = 8 * (rest / nu) + xcd;
    if (e >= a.E) return false;
    rec = a.rec[e];   // loaded with the offsets: one round trip
    pos0 = a.off[e];
    n = a.off[e + 1] - pos0;
    p0 = 0;
    p1 = (n + kPR - 1) / kPR;
    return n > 0;
}

// The fold of one group's three digit sums into the fp32 accumulator of 4 outputs:
// T = t0 + 256 t1 + 65536 t2 (t0 + 256 t1 exact in int32, t2 * 65536 exact in fp32),
// v = 2^xe T - (z - 8) xsum, acc += s v.  The sums are 16 times the integer products
// (pf_a16), so xe is the group's exponent e - 22 minus 4: every step is scaled by an
// exact power of two and the result is that of the unscaled sums.
__device__ __forceinline__ void pf_fold(const pf_v4i (&iacc)[3], const float2 (&sz)[4], int xe, float xs,
                                        float (&acc)[4]) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float lo = (float)(iacc[0][r] + 256 * iacc[1][r]);
        const float T = fmaf((float)iacc[2][r], 65536.f, lo);
        const float v = fmaf(-(sz[r].y - 8.f), xs, ldexpf(T, xe));
        acc[r] = fmaf(sz[r].x, v, acc[r]);
    }
}

// Weight slots of 4 consecutive groups (a superstep) for the MFMA A operand.  Lane (q, j)
// reads 16 bytes at slot 8 S + q and 8 S + 4 + q of each half of row j (lanes layout:
// even host chunks, then odd), so one load covers 64 contiguous bytes of each of 16 rows;
// a permlane32 swap of (even, odd) pairs then leaves one group per register across the 4
// q lanes: register i holds group 4 S + i, lane q host chunk 4 g + kq, kq = [0 2 1 3][q].
__device__ __forceinline__ void pf_swap(uint4 &a, uint4 &b) {
    const auto x = __builtin_amdgcn_permlane32_swap(a.x, b.x, false, false);
    const auto y = __builtin_amdgcn_permlane32_swap(a.y, b.y, false, false);
    const auto z = __builtin_amdgcn_permlane32_swap(a.z, b.z, false, false);
    const auto w = __builtin_amdgcn_permlane32_swap(a.w, b.w, false, false);
    a = make_uint4(x[0], y[0], z[0], w[0]);
    b = make_uint4(x[1], y[1], z[1], w[1]);
}
__device__ __forceinline__ void pf_wload(__amdgpu_buffer_rsrc_t r, uint32_t o, uint32_t half, uint4 (&d)[4]) {
    d[0] = buf_load16<kCached>(r, o);
    d[1] = buf_load16<kCached>(r, o + half);
    d[2] = buf_load16<kCached>(r, o + 64);
    d[3] = buf_load16<kCached>(r, o + half + 64);
}
__device__ __forceinline__ void pf_wgroups(uint4 (&d)[4]) {
    pf_swap(d[0], d[1]);   // groups 4 S, 4 S + 1
    pf_swap(d[2], d[3]);   // groups 4 S + 2, 4 S + 3
}

// Dense GEMM over S rows of x (prefill projections, c/shaders/qmatmul_mm.comp): Y[s][o] =
// sum_i x[s][i] W[o][i] for an fmt6 tensor of group size 128.  A unit is 128 output rows
// (two 16-row tiles per wave) and one pass of <= 32 rows of x; the units of one row block
// run on one XCD (workgroups go to the 8 XCDs round-robin), where their weights stay in L2.
struct GemmArgs {
    const uint8_t *w;       // lanes layout
    const float *sz;        // [O][I / 128] [scale, zero]
    int O, I, rb, nl;
    const int8_t *xd;       // x digit planes [3][S][I]
    const int *xe;          // [S][I / 128]
    const float *xsum;
    int S, nu, npass;       // rows of x; row blocks ceil(O / 128); passes ceil(S / 32)
    float *y;               // [S][O]
};
constexpr int kGR = 2 * kGU;   // dense: output rows per unit

// Gate/up + SwiGLU (kDense false) and the dense GEMM (kDense true) share one body.
// MoE unit = 64 columns of h: wave w owns gate and up rows 64 u + 16 w .. + 15.  Dense unit
// = 128 rows: wave w owns rows 128 u + 16 w + 64 m .. + 15 (m = 0, 1) in place of gate and up.
// Per pass of <= 32 rows of x, supersteps of 4 groups: the x digit planes of the pass's rows
// for the superstep sit in LDS (each thread stages its row's 12 x 16 bytes), the next
// superstep's x digits and then its weight slots are loaded while this one computes, so the
// in-order wait for those x digits never covers the weights.  Each (matrix, digit, 16-row
// tile) is two MFMAs per group, folded in fp32 with the group's scale.  MoE: h = silu(gate) *
// up (c/qwen.c:780-786, silu c/qwen.c:173) goes out as fp32 rows; dense: the two row tiles.
template <bool kDense>
__device__ __forceinline__ void gu_body(const PfArgs &a, const GemmArgs &g) {
    __shared__ __attribute__((aligned(16))) int8_t sB[4][3][kPR][kPitch];
    __shared__ int sE[4][kPR];
    __shared__ float sQ[4][kPR];
    extern __shared__ float4 sS4[];   // [ngD][2][kGU] float2: scales of the unit's rows
    float2 *sS = (float2 *)sS4;
    const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, j = lane & 15, kq = ((q & 1) << 1) | (q >> 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int e = 0, u, p0, p1, pos0, n, ngD, xD, xS;
    __amdgpu_buffer_rsrc_t wr[2], xr;
    uint32_t abase, a1off, whalf;   // matrix 1's slots at abase + a1off
    const float2 *sgp, *sup;
    int nv[2];   // valid scale entries of the two matrices' unit rows
    if constexpr (kDense) {
        const int b = blockIdx.x, r = b >> 3;
        u = 8 * (r / g.npass) + (b & 7);
        if (u >= g.nu) return;
        p0 = r % g.npass;
        p1 = p0 + 1;
        pos0 = 0;
        n = g.S;
        ngD = g.I / kGS;
        xD = g.I;
        xS = g.S;
        const __amdgpu_buffer_rsrc_t w = buf_rsrc(g.w, (uint32_t)g.O * g.rb);
        wr[0] = wr[1] = w;
        const int row0 = u * kGR + wave * 16 + j;
        abase = (uint32_t)(row0 * g.rb + q * 16);
        a1off = (uint32_t)(kGU * g.rb);
        whalf = (uint32_t)g.nl * 16;
        sgp = (const float2 *)g.sz + (size_t)u * kGR * ngD;
        sup = sgp + (size_t)kGU * ngD;
        nv[0] = min(max(g.O - u * kGR, 0), kGU) * ngD;
        nv[1] = min(max(g.O - u * kGR - kGU, 0), kGU) * ngD;
        xr = buf_rsrc(g.xd, (uint32_t)(3u * g.S * g.I));
    } else {
        ExpertRec rec;
        if (!pf_unit(a, a.I / kGU, e, u, p0, p1, pos0, n, rec)) return;
        ngD = a.D / kGS;
        xD = a.D;
        xS = a.S;
        wr[0] = buf_rsrc(rec.wg, (uint32_t)a.I * a.rbG);
        wr[1] = buf_rsrc(rec.wu, (uint32_t)a.I * a.rbG);
        abase = (uint32_t)((u * kGU + wave * 16 + j) * a.rbG + q * 16);
        a1off = 0;
        whalf = (uint32_t)a.nlG * 16;
        sgp = (const float2 *)rec.sg + (size_t)u * kGU * ngD;
        sup = (const float2 *)rec.su + (size_t)u * kGU * ngD;
        nv[0] = nv[1] = kGU * ngD;
        xr = buf_rsrc(a.xd, (uint32_t)(3u * a.S * a.D));
    }
    const int nss = (ngD + 3) / 4;
    const int *xe = kDense ? g.xe : a.xe;
    const float *xsum = kDense ? g.xsum : a.xsum;
    // scales of the unit's rows of the two matrices, regrouped by group in LDS: the first kSV
    // entries per thread are loaded with the first pass's x row and weights
    constexpr int kSV = 2;
    auto s_store = [&](int v, float2 gv, float2 uv) {
        const int r = v / ngD, gi = v - r * ngD;
        sS[(2 * gi) * kGU + r] = gv;
        sS[(2 * gi + 1) * kGU + r] = uv;
    };
    auto w_load = [&](int S, uint4 (&d)[2][4]) {
        pf_wload(wr[0], S < nss ? abase + 128u * S : kOOB, whalf, d[0]);
        pf_wload(wr[1], S < nss ? abase + a1off + 128u * S : kOOB, whalf, d[1]);
    };
    const uint32_t plane = (uint32_t)xS * xD;
    // staging thread: row sr of the pass, 16 columns at sc of every group and plane; the
    // threads with tid % 8 < 4 also carry exponent and sum of group tid % 8
    const int sr = tid >> 3, sc = (tid & 7) * 16, sg4 = tid & 7;
    struct XStage {
        uint4 v[4][3];
        int e;
        float s;
    };
    for (int pass = p0; pass < p1; pass++) {
        const int r0 = pass * kPR, nr = min(kPR, n - r0), ntt = nr > 16 ? 2 : 1;
        // issue order: this thread's row of x (the dependent chain), the first weights,
        // the scales (first pass), then the x digits once the row is known
        const int xi = r0 + min(sr, nr - 1);
        int xrow;
        if constexpr (kDense) xrow = xi;
        else xrow = a.units ? a.plist[pos0 + xi] : e == a.E ? xi : a.plist[pos0 + xi] / a.K;
        uint4 W[2][4];
        w_load(0, W);
        float2 sv[kSV][2];
        if (pass == p0)
#pragma unroll
            for (int i = 0; i < kSV; i++) {
                const int v = tid + kPT * i;
                sv[i][0] = v < nv[0] ? sgp[v] : make_float2(0.f, 0.f);
                sv[i][1] = v < nv[1] ? sup[v] : make_float2(0.f, 0.f);
            }
        auto x_load = [&](int S, XStage &st) {
#pragma unroll
            for (int gl = 0; gl < 4; gl++) {
                const int gi = 4 * S + gl;
                const uint32_t o = gi < ngD ? (uint32_t)xrow * xD + gi * kGS + sc : kOOB;
#pragma unroll
                for (int d = 0; d < 3; d++) st.v[gl][d] = buf_load16<kCached>(xr, o + d * plane);
            }
            const int gc = min(4 * S + (sg4 & 3), ngD - 1);
            st.e = xe[(size_t)xrow * ngD + gc];
            st.s = xsum[(size_t)xrow * ngD + gc];
        };
        auto x_store = [&](const XStage &st) {
#pragma unroll
            for (int gl = 0; gl < 4; gl++)
#pragma unroll
                for (int d = 0; d < 3; d++) *(uint4 *)&sB[gl][d][sr][sc] = st.v[gl][d];
            if (sg4 < 4) {
                sE[sg4][sr] = st.e - 4;   // the sums carry 16 (pf_a16)
                sQ[sg4][sr] = st.s;
            }
        };
        if (pass == p0) {   // the scales arrive with the x row: storing them first costs no wait
#pragma unroll
            for (int i = 0; i < kSV; i++)
                if (tid + kPT * i < kGU * ngD) s_store(tid + kPT * i, sv[i][0], sv[i][1]);
            for (int v = tid + kPT * kSV; v < kGU * ngD; v += kPT)   // I > 2048
                s_store(v, v < nv[0] ? sgp[v] : make_float2(0.f, 0.f), v < nv[1] ? sup[v] : make_float2(0.f, 0.f));
        }
        XStage xst;
        x_load(0, xst);
        x_store(xst);
        __syncthreads();
        // the tile count as a compile-time constant: no branches between the LDS reads
        // and the MFMAs of a group, so the scheduler can batch them
        auto run = [&](auto ntc) {
            constexpr int NT = decltype(ntc)::value;
            float facc[2][2][4];
#pragma unroll
            for (int m = 0; m < 2; m++)
#pragma unroll
                for (int tt = 0; tt < 2; tt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) facc[m][tt][r] = 0.f;
            for (int S = 0; S < nss; S++) {
                x_load(S + 1, xst);   // zeros past the end
                uint4 C[2][4];
#pragma unroll
                for (int m = 0; m < 2; m++)
#pragma unroll
                    for (int i = 0; i < 4; i++) C[m][i] = W[m][i];
                w_load(S + 1, W);
                pf_wgroups(C[0]);
                pf_wgroups(C[1]);
#pragma unroll
                for (int gl = 0; gl < 4; gl++) {
                    const int gi = 4 * S + gl;
                    if (gi >= ngD) continue;   // uniform
                    pf_v4i av[2][2];   // [matrix][half]
#pragma unroll
                    for (int m = 0; m < 2; m++) {
                        av[m][0] = pf_a16(C[m][gl].x, C[m][gl].y);
                        av[m][1] = pf_a16(C[m][gl].z, C[m][gl].w);
                    }
                    pf_v4i iacc[2][2][3];   // [matrix][tile][digit]; one B read serves both matrices
#pragma unroll
                    for (int hh = 0; hh < 2; hh++)
#pragma unroll
                        for (int d = 0; d < 3; d++)
#pragma unroll
                            for (int tt = 0; tt < 2; tt++)
                                if (tt < NT) {
                                    const pf_v4i bv = *(const pf_v4i *)&sB[gl][d][tt * 16 + j][32 * kq + 16 * hh];
#pragma unroll
                                    for (int m = 0; m < 2; m++)
                                        iacc[m][tt][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                            av[m][hh], bv, hh ? iacc[m][tt][d] : pf_v4i{0, 0, 0, 0}, 0, 0, 0);
                                }
                    float2 sz[2][4];
#pragma unroll
                    for (int m = 0; m < 2; m++) {
                        const float4 *sz4 = (const float4 *)&sS[(2 * gi + m) * kGU + wave * 16 + 4 * q];
                        const float4 za = sz4[0], zb = sz4[1];
                        sz[m][0] = make_float2(za.x, za.y);
                        sz[m][1] = make_float2(za.z, za.w);
                        sz[m][2] = make_float2(zb.x, zb.y);
                        sz[m][3] = make_float2(zb.z, zb.w);
                    }
#pragma unroll
                    for (int tt = 0; tt < 2; tt++)
                        if (tt < NT) {
                            const int xe_ = sE[gl][tt * 16 + j];
                            const float xs = sQ[gl][tt * 16 + j];
#pragma unroll
                            for (int m = 0; m < 2; m++) pf_fold(iacc[m][tt], sz[m], xe_, xs, facc[m][tt]);
                        }
                }
                if (S + 1 < nss) {   // uniform
                    __syncthreads();   // every wave is done with this superstep's x digits
                    x_store(xst);
                    __syncthreads();
                }
            }
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                const int x = tt * 16 + j;
                if (tt >= NT || x >= nr) continue;
                if constexpr (kDense) {
                    // rows 128 u + 64 m + 16 w + 4 q .. + 3 of x row r0 + x
#pragma unroll
                    for (int m = 0; m < 2; m++) {
                        const int row = u * kGR + m * kGU + wave * 16 + 4 * q;
                        float *yr = g.y + (size_t)(r0 + x) * g.O + row;
                        if (row + 3 < g.O && (g.O & 3) == 0)
                            *(float4 *)yr = make_float4(facc[m][tt][0], facc[m][tt][1], facc[m][tt][2], facc[m][tt][3]);
                        else
#pragma unroll
                            for (int r = 0; r < 4; r++)
                                if (row + r < g.O) yr[r] = facc[m][tt][r];
                    }
                } else {
                    // h columns kGU u + 16 w + 4 q .. + 3 of x row tt * 16 + j
                    float hv[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float gv = facc[0][tt][r];
                        hv[r] = gv / (1.f + expf(-gv)) * facc[1][tt][r];
                    }
                    *(float4 *)&a.h[(size_t)(pos0 + r0 + x) * a.I + u * kGU + wave * 16 + 4 * q] =
                        make_float4(hv[0], hv[1], hv[2], hv[3]);
                }
            }
        };
        if (ntt == 2) run(std::integral_constant<int, 2>{});
        else run(std::integral_constant<int, 1>{});
        __syncthreads();   // the next pass restages sB
    }
}

__global__ __launch_bounds__(kPT, 2) void pf_gateup(PfArgs a) { gu_body<false>(a, GemmArgs{}); }
__global__ __launch_bounds__(kPT, 2) void gemm6_mfma(GemmArgs g) { gu_body<true>(PfArgs{}, g); }

// Rows of n values (n % 128 == 0) -> digit planes [3][rows][n], ge / gsum [rows][n / 128]:
// one thread per 8 columns.  kGated: the row is first put through the GatedDeltaNet output
// norm, per head of VD columns y * r_h * gnorm[d] * silu(z) with r_h = 1 / sqrt(mean(y^2)
// + eps), the sum of squares in double (c/qwen.c:768-772); gnorm has a row stride (the
// host packs it into each token's parameter row).  VD / 8 consecutive lanes hold one head
// (VD a power of two, 8 <= VD <= 512), so the head sum is a butterfly over them.
template <bool kGated>
__global__ __launch_bounds__(256) void pf_digits_t(const float *__restrict__ src, int rows, int n,
                                                   int8_t *__restrict__ planes, int *__restrict__ ge,
                                                   float *__restrict__ gsum, const float *__restrict__ z,
                                                   const float *__restrict__ gnorm, int gstride, int VD, float eps) {
    const int per = n / 8, i = blockIdx.x * 256 + threadIdx.x, row = i / per, c8 = i - row * per;
    const bool valid = row < rows;
    float v[8];
    if (valid) {
        const float4 a = *(const float4 *)(src + (size_t)row * n + 8 * c8),
                     b = *(const float4 *)(src + (size_t)row * n + 8 * c8 + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
#pragma unroll
        for (int c = 0; c < 8; c++) v[c] = 0.f;
    }
    if constexpr (kGated) {
        double ss = 0;
#pragma unroll
        for (int c = 0; c < 8; c++) ss += (double)v[c] * v[c];
        for (int o = 1; o < VD / 8; o <<= 1) ss += __shfl_xor(ss, o);
        const float r = 1.f / sqrtf((float)(ss / VD) + eps);
        if (valid) {
            const float *zr = z + (size_t)row * n + 8 * c8;
            const float *gw = gnorm + (size_t)row * gstride + (8 * c8) % VD;
#pragma unroll
            for (int c = 0; c < 8; c++) {   // silu(z) with a hardware reciprocal (< 2 ulp)
                const float zv = zr[c], sz = zv * __builtin_amdgcn_rcpf(1.f + expf(-zv));
                v[c] = v[c] * r * gw[c] * sz;
            }
        }
    }
    const int ng = n / kGS, gi = (8 * c8) / kGS;
    const size_t r = valid ? row : 0;
    digit8(v, valid, 8 * c8, planes + r * n + 8 * c8, (size_t)rows * n, ge + r * ng + gi, gsum + r * ng + gi);
}

// Down projection.  Unit = 256 output rows: wave w owns rows 256 u + 64 w + 16 t .. + 15
// (t < 4).  Per pass of <= 32 positions, h's digit planes are staged in LDS 4 groups
// (512 columns) at a time with the matching scales; the lane's weight slots of those
// groups (one superstep per tile) are loaded at once and kept across passes when one
// chunk covers I.
__global__ __launch_bounds__(kPT, 2) void pf_down(PfArgs a) {
    __shared__ __attribute__((aligned(16))) int8_t sH[3][kPR][kDPitch];
    __shared__ int sE[kPR][kDG];
    __shared__ float sQ[kPR][kDG];
    __shared__ __attribute__((aligned(16))) float2 sS[kDG][kDR];
    const int nq = (a.D + kDR - 1) / kDR, ngI = a.I / kGS, nch = (ngI + kDG - 1) / kDG;
    int e, u, p0, p1, pos0, n;
    ExpertRec rec;
    if (!pf_unit(a, nq, e, u, p0, p1, pos0, n, rec)) return;
    const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, j = lane & 15, kq = ((q & 1) << 1) | (q >> 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(rec.wd, (uint32_t)a.D * a.rbD);
    const int P = a.P;
    const __amdgpu_buffer_rsrc_t hr = buf_rsrc(a.hd, (uint32_t)(3u * P * a.I));
    const int rbase = u * kDR + wave * 64;   // first row of the wave
    constexpr int kHS = 3 * kPR * kDG * kGS / 16 / kPT;   // 16-byte staging chunks per thread (12)
    uint4 wv[kDT][kDG];
    for (int pass = p0; pass < p1; pass++) {
        const int r0 = pass * kPR, nr = min(kPR, n - r0), ntt = nr > 16 ? 2 : 1;
        // staging chunk k = tid + kPT i of the 3 x 32 x 32 16-byte chunks: plane k / 1024,
        // row (k / 32) % 32 = (tid / 32 + 8 i) % 32, columns 16 (k % 32)
        int hrow[4];
#pragma unroll
        for (int i = 0; i < 4; i++) hrow[i] = pos0 + r0 + min(((tid >> 5) + 8 * i) & 31, nr - 1);
        float facc[kDT][2][4];
#pragma unroll
        for (int t = 0; t < kDT; t++)
#pragma unroll
            for (int tt = 0; tt < 2; tt++)
#pragma unroll
                for (int r = 0; r < 4; r++) facc[t][tt][r] = 0.f;
        for (int ch = 0; ch < nch; ch++) {
            const int gb = ch * kDG;
            uint4 hv[kHS];
#pragma unroll
            for (int i = 0; i < kHS; i++) {
                const int k = tid + kPT * i, col = gb * kGS + 16 * (k & 31);
                hv[i] = buf_load16<kCached>(hr, col < a.I ? (uint32_t)((k >> 10) * P + hrow[i & 3]) * a.I + col : kOOB);
            }
            int re = 0;
            float rq = 0.f;
            if (tid < kPR * kDG) {
                const int g = min(gb + (tid & 3), ngI - 1);
                const size_t o = (size_t)(pos0 + r0 + min(tid >> 2, nr - 1)) * ngI + g;
                re = a.he[o];
                rq = a.hsum[o];
            }
            float2 sv[kDG];
#pragma unroll
            for (int i = 0; i < kDG; i++) {   // scales: entry v = tid + kPT i -> row v / 4, group v % 4
                const int v = tid + kPT * i, row = u * kDR + (v >> 2), g = gb + (v & 3);
                sv[i] = row < a.D && g < ngI ? ((const float2 *)rec.sd)[(size_t)row * ngI + g] : make_float2(0.f, 0.f);
            }
            if (nch > 1 || pass == p0) {   // the superstep ch of each tile's rows
#pragma unroll
                for (int t = 0; t < kDT; t++) {
                    const int row = rbase + 16 * t + j;
                    pf_wload(wr, row < a.D ? (uint32_t)(row * a.rbD + q * 16 + 128 * ch) : kOOB, (uint32_t)a.nlD * 16, wv[t]);
                }
            }
#pragma unroll
            for (int i = 0; i < kHS; i++) {
                const int k = tid + kPT * i;
                *(uint4 *)&sH[k >> 10][(k >> 5) & 31][16 * (k & 31)] = hv[i];
            }
            if (tid < kPR * kDG) {
                sE[tid >> 2][tid & 3] = re - 4;   // the sums carry 16 (pf_a16)
                sQ[tid >> 2][tid & 3] = rq;
            }
#pragma unroll
            for (int i = 0; i < kDG; i++) {
                const int v = tid + kPT * i;
                sS[v & 3][v >> 2] = sv[i];
            }
            __syncthreads();
            if (nch > 1 || pass == p0)
#pragma unroll
                for (int t = 0; t < kDT; t++) pf_wgroups(wv[t]);   // once per load; kept for later passes
            constexpr int TP = 2;   // two row tiles share each B read
#pragma unroll
            for (int tp = 0; tp < kDT / TP; tp++) {
#pragma unroll
                for (int gl = 0; gl < kDG; gl++) {
                    if (gb + gl >= ngI) continue;   // uniform
                    pf_v4i av[TP][2];   // [tile][half]
#pragma unroll
                    for (int i = 0; i < TP; i++) {
                        av[i][0] = pf_a16(wv[TP * tp + i][gl].x, wv[TP * tp + i][gl].y);
                        av[i][1] = pf_a16(wv[TP * tp + i][gl].z, wv[TP * tp + i][gl].w);
                    }
                    pf_v4i iacc[TP][2][3];   // [tile][x tile][digit]
#pragma unroll
                    for (int hh = 0; hh < 2; hh++)
#pragma unroll
                        for (int d = 0; d < 3; d++)
#pragma unroll
                            for (int tt = 0; tt < 2; tt++) {
                                if (tt >= ntt) continue;   // uniform
                                const pf_v4i bv =
                                    *(const pf_v4i *)&sH[d][tt * 16 + j][gl * kGS + 32 * kq + 16 * hh];
#pragma unroll
                                for (int i = 0; i < TP; i++)
                                    iacc[i][tt][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                        av[i][hh], bv, hh ? iacc[i][tt][d] : pf_v4i{0, 0, 0, 0}, 0, 0, 0);
                            }
                    float2 sz[TP][4];
#pragma unroll
                    for (int i = 0; i < TP; i++) {
                        const float4 *sz4 = (const float4 *)&sS[gl][wave * 64 + 16 * (TP * tp + i) + 4 * q];
                        const float4 za = sz4[0], zb = sz4[1];
                        sz[i][0] = make_float2(za.x, za.y);
                        sz[i][1] = make_float2(za.z, za.w);
                        sz[i][2] = make_float2(zb.x, zb.y);
                        sz[i][3] = make_float2(zb.z, zb.w);
                    }
#pragma unroll
                    for (int tt = 0; tt < 2; tt++) {
                        if (tt >= ntt) continue;
                        const int xe = sE[tt * 16 + j][gl];
                        const float xs = sQ[tt * 16 + j][gl];
#pragma unroll
                        for (int i = 0; i < TP; i++) pf_fold(iacc[i][tt], sz[i], xe, xs, facc[TP * tp + i][tt]);
                    }
                }
            }
            __syncthreads();   // the staging buffers are refilled by the next chunk or pass
        }
        // y rows rbase + 16 t + 4 q .. + 3 of position r0 + 16 tt + j
#pragma unroll
        for (int t = 0; t < kDT; t++) {
            const int row = rbase + 16 * t + 4 * q;
            if (row >= a.D) continue;
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                const int x = tt * 16 + j;
                if (tt < ntt && x < nr)
                    *(float4 *)&a.y[(size_t)(pos0 + r0 + x) * a.D + row] =
                        make_float4(facc[t][tt][0], facc[t][tt][1], facc[t][tt][2], facc[t][tt][3]);
            }
        }
    }
}

// ---------------------------------------------------------------- combine
// out[t] = sum over t's K experts in ascending expert id of w * y[pos] + shgt * y_sh[t]
// (c/qwen.c:1144, 1159-1161).  The token's ids, positions and weights come in one round of
// loads and are put in expert order in registers (an odd-even transposition network: ids
// are distinct); then every float4 of the thread's columns and all K + 1 rows are loaded
// before the sums, which keep the order above.
constexpr int kCbCols = 2;   // float4 columns per thread and pass of 4 * 256 * kCbCols columns
__global__ __launch_bounds__(256) void pf_combine(const float *__restrict__ y, const int *tidx, const float *tval,
                                                  const float *tshg, const int *ppos, int S, int K, int D,
                                                  float *__restrict__ out) {
    const int t = blockIdx.x;
    int id[kTopK], pp[kTopK];
    float w[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; k++) {
        id[k] = k < K ? tidx[t * K + k] : 0x7FFFFFFF;   // absent slots sort last
        pp[k] = k < K ? ppos[t * K + k] : 0;
        w[k] = k < K ? tval[t * K + k] : 0.f;
    }
    const float shg = tshg[t];
#pragma unroll
    for (int i = 0; i < kTopK; i++)
#pragma unroll
        for (int k = i & 1; k + 1 < kTopK; k += 2)
            if (id[k] > id[k + 1]) {
                const int a = id[k], b = pp[k];
                const float c = w[k];
                id[k] = id[k + 1], pp[k] = pp[k + 1], w[k] = w[k + 1];
                id[k + 1] = a, pp[k + 1] = b, w[k + 1] = c;
            }
    const float *ysh = y + (size_t)(S * K + t) * D;
    for (int c0 = 0; c0 < D; c0 += 4 * 256 * kCbCols) {
        float4 v[kCbCols][kTopK], sv[kCbCols];
#pragma unroll
        for (int q = 0; q < kCbCols; q++) {
            const int c = c0 + 4 * threadIdx.x + 4 * 256 * q;
            const bool on = c < D;
#pragma unroll
            for (int i = 0; i < kTopK; i++)
                v[q][i] = on && i < K ? *(const float4 *)(y + (size_t)pp[i] * D + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            sv[q] = on ? *(const float4 *)(ysh + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int q = 0; q < kCbCols; q++) {
            const int c = c0 + 4 * threadIdx.x + 4 * 256 * q;
            if (c >= D) continue;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int i = 0; i < kTopK; i++)
                if (i < K) {
                    acc.x = acc.x + w[i] * v[q][i].x;
                    acc.y = acc.y + w[i] * v[q][i].y;
                    acc.z = acc.z + w[i] * v[q][i].z;
                    acc.w = acc.w + w[i] * v[q][i].w;
                }
            *(float4 *)(out + (size_t)t * D + c) = make_float4(acc.x + shg * sv[q].x, acc.y + shg * sv[q].y,
                                                               acc.z + shg * sv[q].z, acc.w + shg * sv[q].w);
        }
    }
}

// ---------------------------------------------------------------- host
struct PfScratch {
    void *buf = nullptr;
    size_t cap = 0;
};
static PfScratch g_pf;

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

bool moe_prefill(int layer, const ColiVkTensor *router, int K, const float *d_xs, int S, float *d_out, int *d_idx,
                 float *d_val, hipStream_t st) {
    const ExpertRec *rec;
    const float *shg;
    MoeGeom m;
    int E;
    if (!ok() || !tensor_live(router) || !d_xs || !d_out || S < 1) return false;
    if (!moe_layer(layer, &rec, &shg, &m, &E)) return false;
    if (K < 1 || K > kTopK || K > E || E > kMaxE) return false;
    if (router->I != m.D || router->O != E || (router->fmt != 0 && router->fmt != 1) || router->layout != kLayoutRows)
        return false;
    if (router->row_bytes % (router->fmt == 0 ? 16 : 4)) return false;
    if (m.gs != kGS || m.D % kGS || m.I % kGS || m.D > 4096 || m.I > 4096) return false;
    const int D = m.D, I = m.I, np = S * K, P = np + S, ngD = D / kGS, ngI = I / kGS;
    if ((size_t)3 * S * D >= (1u << 31) || (size_t)3 * P * I >= (1u << 31) || (size_t)P * D >= (1u << 31)) return false;
    // scratch layout
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += al256(bytes);
        return at;
    };
    const size_t o_pt = take((size_t)S * E * 4), o_ti = take((size_t)np * 4), o_tv = take((size_t)np * 4),
                 o_sh = take((size_t)S * 4), o_off = take((size_t)(E + 1) * 4), o_pl = take((size_t)np * 4),
                 o_pp = take((size_t)np * 4), o_rk = take((size_t)np * 4), o_xd = take((size_t)3 * S * D),
                 o_xe = take((size_t)S * ngD * 4), o_xs = take((size_t)S * ngD * 4), o_h = take((size_t)P * I * 4),
                 o_hd = take((size_t)3 * P * I),
                 o_he = take((size_t)P * ngI * 4), o_hs = take((size_t)P * ngI * 4), o_y = take((size_t)P * D * 4);
    if (!scratch(&g_pf.buf, &g_pf.cap, o)) return false;
    uint8_t *b = (uint8_t *)g_pf.buf;
    float *lg = (float *)(b + o_pt);
    float *tv = d_val ? d_val : (float *)(b + o_tv), *tsh = (float *)(b + o_sh);
    int *ti = d_idx ? d_idx : (int *)(b + o_ti), *off = (int *)(b + o_off);
    int *pl = (int *)(b + o_pl), *pp = (int *)(b + o_pp), *rk = (int *)(b + o_rk);

    hipLaunchKernelGGL(pf_logits, dim3((S + kLT - 1) / kLT, (E + kLE - 1) / kLE), dim3(256), 0, st, d_xs, S, D,
                       router->w, router->sz, router->fmt, router->row_bytes, E, lg);
    PfArgs a;
    memset(&a, 0, sizeof(a));
    a.rec = rec;
    a.off = off;
    a.plist = pl;
    a.E = E;
    a.S = S;
    a.K = K;
    a.D = D;
    a.I = I;
    a.nlG = m.nlG;
    a.rbG = m.rbG;
    a.nlD = m.nlD;
    a.rbD = m.rbD;
    a.P = P;
    a.nsp = (S + kPR - 1) / kPR;
    a.xd = (const int8_t *)(b + o_xd);
    a.xe = (const int *)(b + o_xe);
    a.xsum = (const float *)(b + o_xs);
    a.h = (float *)(b + o_h);
    a.hd = (const int8_t *)(b + o_hd);
    a.he = (const int *)(b + o_he);
    a.hsum = (const float *)(b + o_hs);
    a.y = (float *)(b + o_y);
    hipLaunchKernelGGL(pf_route, dim3(S), dim3(kThreads), 0, st, lg, d_xs, S, D, shg, E, K, ti, tv, tsh,
                       (int8_t *)(b + o_xd), (int *)(b + o_xe), (float *)(b + o_xs));
    hipLaunchKernelGGL(pf_group, dim3(1), dim3(1024), 0, st, ti, np, E, off, pl, pp, rk);
    const int E8 = (E + 7) & ~7;
    auto blocks = [&](int nu) { return ((nu * a.nsp + 7) & ~7) + nu * E8; };
    const int nh = I / kGU, nq = (D + kDR - 1) / kDR;
    hipLaunchKernelGGL(pf_gateup, dim3(blocks(nh)), dim3(kPT), (size_t)ngD * 2 * kGU * sizeof(float2), st, a);
    hipLaunchKernelGGL(pf_digits_t<false>, dim3((P * (I / 8) + 255) / 256), dim3(256), 0, st, a.h, P, I,
                       (int8_t *)(b + o_hd), (int *)(b + o_he), (float *)(b + o_hs), nullptr, nullptr, 0, 0, 0.f);
    hipLaunchKernelGGL(pf_down, dim3(blocks(nq)), dim3(kPT), 0, st, a);
    hipLaunchKernelGGL(pf_combine, dim3(S), dim3(256), 0, st, a.y, ti, tv, tsh, pp, S, K, D, d_out);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail("moe prefill launch", err);
    return true;
}

// ---------------------------------------------------------------- dense GEMM (host)
static PfScratch g_gm;

bool gemm6_ok(const ColiVkTensor *t) {
    return tensor_live(t) && t->fmt == 6 && t->layout == kLayoutLanes && t->gs == kGS && t->I % kGS == 0 &&
           t->I <= kGemmMaxI && t->O >= 1 && (size_t)(t->O + kGR) * t->row_bytes < (1ull << 32);
}

bool gemm6(const ColiVkTensor *const *t, float *const *d_y, int nt, const float *d_x, int S, hipStream_t st,
           const GatedX *gx) {
    if (nt < 1 || !d_x || S < 1) return false;
    const int I = t[0]->I, ng = I / kGS;
    for (int i = 0; i < nt; i++)
        if (!gemm6_ok(t[i]) || t[i]->I != I || !d_y[i]) return false;
    if ((size_t)3 * S * I >= (1u << 31)) return false;
    if (gx && (!gx->z || !gx->gnorm || gx->VD < 8 || gx->VD > 512 || (gx->VD & (gx->VD - 1)) || I % gx->VD))
        return false;
    const size_t o_xe = al256((size_t)3 * S * I), o_xs = o_xe + al256((size_t)S * ng * 4),
                 total = o_xs + al256((size_t)S * ng * 4);
    if (!scratch(&g_gm.buf, &g_gm.cap, total)) return false;
    uint8_t *b = (uint8_t *)g_gm.buf;
    const dim3 dg((unsigned)(((size_t)S * (I / 8) + 255) / 256));
    if (gx)
        hipLaunchKernelGGL(pf_digits_t<true>, dg, dim3(256), 0, st, d_x, S, I, (int8_t *)b, (int *)(b + o_xe),
                           (float *)(b + o_xs), gx->z, gx->gnorm, gx->gstride, gx->VD, gx->eps);
    else
        hipLaunchKernelGGL(pf_digits_t<false>, dg, dim3(256), 0, st, d_x, S, I, (int8_t *)b, (int *)(b + o_xe),
                           (float *)(b + o_xs), nullptr, nullptr, 0, 0, 0.f);
    for (int i = 0; i < nt; i++) {
        GemmArgs g;
        g.w = t[i]->w;
        g.sz = t[i]->sz;
        g.O = t[i]->O;
        g.I = I;
        g.rb = t[i]->row_bytes;
        g.nl = t[i]->nl;
        g.xd = (const int8_t *)b;
        g.xe = (const int *)(b + o_xe);
        g.xsum = (const float *)(b + o_xs);
        g.S = S;
        g.nu = (g.O + kGR - 1) / kGR;
        g.npass = (S + kPR - 1) / kPR;
        g.y = d_y[i];
        const int blocks = 8 * ((g.nu + 7) / 8) * g.npass;
        hipLaunchKernelGGL(gemm6_mfma, dim3(blocks), dim3(kPT), (size_t)ng * 2 * kGU * sizeof(float2), st, g);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail("dense gemm launch", err);
    return true;
}

// ---------------------------------------------------------------- fmt 0 / fmt 1 over S rows
// The engine's router (c/qwen.c:1189) and GatedDeltaNet a/b (:1359) over S prefill rows are
// fmt 1 (int8 rows, c/qwen.c:1876-1878) or fmt 0: one pf_logits launch for all rows, the
// reference's sequential fp32 sums (c/qwen.c:178-189, 230-238) bit for bit.
bool gemm_f01_ok(const ColiVkTensor *t, const float *d_x) {
    return tensor_live(t) && (t->fmt == 0 || t->fmt == 1) && t->layout == kLayoutRows && t->I % 4 == 0 &&
           t->row_bytes % (t->fmt == 0 ? 16 : 4) == 0 && ((uintptr_t)d_x & 15) == 0 &&
           (t->O + kLE - 1) / kLE <= 65535;
}

bool gemm_f01(const ColiVkTensor *t, const float *d_x, float *d_y, int S, hipStream_t st) {
    if (!gemm_f01_ok(t, d_x) || S < 1 || !d_y) return false;
    hipLaunchKernelGGL(pf_logits, dim3((S + kLT - 1) / kLT, (t->O + kLE - 1) / kLE), dim3(256), 0, st, d_x, S, t->I,
                       t->w, t->sz, t->fmt, t->row_bytes, t->O, d_y);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail("fmt 0/1 rows launch", err);
    return true;
}

// ---------------------------------------------------------------- host-routed expert group
// x digit planes of the group's source rows, kept while (rows, key) stay the same: the rows
// bound once per prefill layer (coli_vk_eg_xs_bind) serve every chunk of that layer.
static PfScratch g_egx, g_egh;
static const float *g_egx_src = nullptr;
static int g_egx_rows = 0, g_egx_n = 0;
static uint64_t g_egx_key = 0;

bool eg_mfma_ok(const MoeGeom &m) {
    return m.gs == kGS && m.D % kGS == 0 && m.I % kGS == 0 && m.D >= kGS && m.I >= kGS && m.D <= kGemmMaxI &&
           m.I <= kGemmMaxI;
}

int eg_unit_rows(int count, const int *rows, const MoeGeom &m) {
    long units32 = 0;
    for (int c = 0; c < count; c++) units32 += (rows[c] + kPR - 1) / kPR;
    const long blocks = units32 * (m.I / kGU);   // gate/up blocks with 32-row units
    return blocks >= 2L * n_cu() ? kPR : kPR / 2;
}

bool eg_mfma(const PfUnit *d_units, int nunits, const int *d_xrow, int P, const MoeGeom &m, const float *d_x,
             int Sx, uint64_t key, float *d_y, hipStream_t st) {
    if (!eg_mfma_ok(m) || nunits < 1 || P < 1 || Sx < 1 || !d_units || !d_xrow || !d_x || !d_y) return false;
    const int D = m.D, I = m.I, ngD = D / kGS, ngI = I / kGS;
    if ((size_t)3 * Sx * D >= (1u << 31) || (size_t)3 * P * I >= (1u << 31) || (size_t)P * D >= (1u << 31))
        return false;
    const size_t ox_e = al256((size_t)3 * Sx * D), ox_s = ox_e + al256((size_t)Sx * ngD * 4),
                 ox_end = ox_s + al256((size_t)Sx * ngD * 4);
    void *old = g_egx.buf;
    if (!scratch(&g_egx.buf, &g_egx.cap, ox_end)) return false;
    uint8_t *xb = (uint8_t *)g_egx.buf;
    if (key == 0 || key != g_egx_key || d_x != g_egx_src || Sx != g_egx_rows || D != g_egx_n || old != g_egx.buf) {
        hipLaunchKernelGGL(pf_digits_t<false>, dim3((unsigned)(((size_t)Sx * (D / 8) + 255) / 256)), dim3(256), 0, st,
                           d_x, Sx, D, (int8_t *)xb, (int *)(xb + ox_e), (float *)(xb + ox_s), nullptr, nullptr, 0, 0,
                           0.f);
        g_egx_key = key;
        g_egx_src = d_x;
        g_egx_rows = Sx;
        g_egx_n = D;
    }
    const size_t oh_d = al256((size_t)P * I * 4), oh_e = oh_d + al256((size_t)3 * P * I),
                 oh_s = oh_e + al256((size_t)P * ngI * 4), oh_end = oh_s + al256((size_t)P * ngI * 4);
    if (!scratch(&g_egh.buf, &g_egh.cap, oh_end)) return false;
    uint8_t *hb = (uint8_t *)g_egh.buf;
    PfArgs a;
    memset(&a, 0, sizeof(a));
    a.units = d_units;
    a.nunits = nunits;
    a.plist = d_xrow;
    a.S = Sx;
    a.K = 1;
    a.D = D;
    a.I = I;
    a.P = P;
    a.nlG = m.nlG;
    a.rbG = m.rbG;
    a.nlD = m.nlD;
    a.rbD = m.rbD;
    a.xd = (const int8_t *)xb;
    a.xe = (const int *)(xb + ox_e);
    a.xsum = (const float *)(xb + ox_s);
    a.h = (float *)hb;
    a.hd = (const int8_t *)(hb + oh_d);
    a.he = (const int *)(hb + oh_e);
    a.hsum = (const float *)(hb + oh_s);
    a.y = d_y;
    const int n8 = 8 * ((nunits + 7) / 8), nh = I / kGU, nq = (D + kDR - 1) / kDR;
    hipLaunchKernelGGL(pf_gateup, dim3(n8 * nh), dim3(kPT), (size_t)ngD * 2 * kGU * sizeof(float2), st, a);
    hipLaunchKernelGGL(pf_digits_t<false>, dim3((unsigned)(((size_t)P * (I / 8) + 255) / 256)), dim3(256), 0, st, a.h,
                       P, I, (int8_t *)(hb + oh_d), (int *)(hb + oh_e), (float *)(hb + oh_s), nullptr, nullptr, 0, 0,
                       0.f);
    hipLaunchKernelGGL(pf_down, dim3(n8 * nq), dim3(kPT), 0, st, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail("expert group mfma launch", err);
    return true;
}

void prefill_shutdown() {
    scratch_free(&g_pf.buf, &g_pf.cap);
    scratch_free(&g_gm.buf, &g_gm.cap);
    scratch_free(&g_egx.buf, &g_egx.cap);
    scratch_free(&g_egh.buf, &g_egh.cap);
    g_egx_src = nullptr;
    g_egx_rows = g_egx_n = 0;
    g_egx_key = 0;
}

}  // namespace coli

using namespace coli;

// The layer's MoE block over S token rows d_xs [S, D] (prefill), expert projections on
// MFMA: d_out [S, D]; d_idx / d_val [S, K] (routing, rank order) may be NULL.
COLI_API int coli_hip_moe_prefill(int layer, const ColiVkTensor *router, int K, const float *d_xs, int S,
                                  float *d_out, int *d_idx, float *d_val, void *stream_) {
    return moe_prefill(layer, router, K, d_xs, S, d_out, d_idx, d_val, stream_ ? (hipStream_t)stream_ : stream())
               ? 1
               : 0;
}
