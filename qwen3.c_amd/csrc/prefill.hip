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
// stored in that order (kPerm16).
#include "moe_common.h"

#include <stdio.h>
#include <string.h>

namespace coli {

typedef int pf_v4i __attribute__((ext_vector_type(4)));

constexpr int kTT = 2;          // 16-row tiles of x per pass (32 rows)
constexpr int kRowBlk = 64;     // weight rows per block (4 waves x 16)

// byte position of K offset o (0..15) inside a 16-byte block of digit plane
__device__ __forceinline__ int perm16(int o) {
    const int h = o & 8, r = o & 7;
    return h + ((r & 1) ? 4 + (r >> 1) : (r >> 1));
}

// signed nibbles (stored XOR 8, i.e. the 4-bit two's complement of n - 8) of the 8
// nibbles of w as int8: even nibbles, then odd nibbles
__device__ __forceinline__ void nib8(uint32_t w, uint32_t &ev, uint32_t &od) {
    uint32_t a = w & 0x0F0F0F0Fu, b = (w >> 4) & 0x0F0F0F0Fu;
    ev = a | ((a & 0x08080808u) * 0x1Eu);   // sign-extend 4 -> 8 bits per byte (no carries)
    od = b | ((b & 0x08080808u) * 0x1Eu);
}

// ---------------------------------------------------------------- router
// logits[t][e] for e < E (router rows, f32 or int8 * scale) and e = E (shared gate):
// fp64 accumulation of exact products, rounded once (the reference sums in fp32).
constexpr int kLT = 8, kLE = 32, kLK = 64;
__global__ __launch_bounds__(256) void pf_logits(const float *__restrict__ xs, int S, int D, const uint8_t *rw,
                                                 const float *rs, int rfmt, int rrb, int E,
                                                 const float *__restrict__ sh_gate, float *__restrict__ logits) {
    __shared__ float s_x[kLT][kLK];
    __shared__ float s_w[kLE][kLK + 1];
    const int tid = threadIdx.x, tt = tid / kLE, ee = tid % kLE;
    const int t0 = blockIdx.x * kLT, e0 = blockIdx.y * kLE;
    double acc = 0.0;
    for (int k0 = 0; k0 < D; k0 += kLK) {
        for (int q = tid; q < kLT * kLK; q += 256) {
            const int r = q / kLK, c = q % kLK, t = t0 + r;
            s_x[r][c] = (t < S && k0 + c < D) ? xs[(size_t)t * D + k0 + c] : 0.f;
        }
        for (int q = tid; q < kLE * kLK; q += 256) {
            const int r = q / kLK, c = q % kLK, e = e0 + r, k = k0 + c;
            float v = 0.f;
            if (e < E && k < D) v = rfmt == 0 ? ((const float *)(rw + (size_t)e * rrb))[k] : (float)(int8_t)rw[(size_t)e * rrb + k];
            else if (e == E && k < D) v = sh_gate[k];
            s_w[r][c] = v;
        }
        __syncthreads();
#pragma unroll 8
        for (int c = 0; c < kLK; c++) acc = fma((double)s_x[tt][c], (double)s_w[ee][c], acc);
        __syncthreads();
    }
    const int t = t0 + tt, e = e0 + ee;
    if (t < S && e <= E) {
        float l = (float)acc;
        if (e < E && rfmt == 1) l *= rs[e];   // c/qwen.c:237: acc * scale[o]
        logits[(size_t)t * (E + 1) + e] = l;
    }
}

// ---------------------------------------------------------------- route per token
__global__ __launch_bounds__(kThreads) void pf_route(const float *__restrict__ logits, int E, int K, int *tidx,
                                                    float *tval, float *tshg) {
    __shared__ RouteLds R;
    const int t = blockIdx.x;
    const float *lg = logits + (size_t)t * (E + 1);
    for (int e = threadIdx.x; e <= E; e += kThreads) {
        if (e < E) R.p[e] = lg[e];
        else R.gate = lg[e];
    }
    route_select(R, E, K);
    if (threadIdx.x < K) {
        tidx[t * K + threadIdx.x] = R.idx[threadIdx.x];
        tval[t * K + threadIdx.x] = R.val[threadIdx.x] / R.vsum;
    }
    if (threadIdx.x == 0) tshg[t] = 1.f / (1.f + expf(-R.gate));
}

// ---------------------------------------------------------------- grouping
// off[e] = first position of expert e's rows, off[E] = S*K; plist[p] = pair index
// (token * K + slot) at position p; ppos[pair] = its position.  Rows of one expert are
// independent, so their order within the expert does not change any result.
__global__ __launch_bounds__(1024) void pf_group(const int *tidx, int npairs, int E, int *cnt, int *off, int *plist,
                                                 int *ppos, int *rank) {
    extern __shared__ int s_cnt[];   // [E + 1]
    for (int e = threadIdx.x; e <= E; e += 1024) s_cnt[e] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < npairs; i += 1024) rank[i] = atomicAdd(&s_cnt[tidx[i]], 1);
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int e = 0; e < E; e++) {
            const int n = s_cnt[e];
            cnt[e] = n;
            s_cnt[e] = acc;
            off[e] = acc;
            acc += n;
        }
        off[E] = acc;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < npairs; i += 1024) {
        const int p = s_cnt[tidx[i]] + rank[i];
        plist[p] = i;
        ppos[i] = p;
    }
}

// ---------------------------------------------------------------- digit planes
// Rows of n values (x or h) -> planes[3][rows][n] (int8, kPerm16 order inside each
// 16-column block), ge[rows][ng] = e - 22 and gs_[rows][ng] = 2^(e-22) * sum of q, per
// group of gs columns: the block fixed point of fmt6_device.h in base 256.  One block of
// 256 threads per 4 rows; n <= 4096, n % 64 == 0, gs % 64 == 0.
__global__ __launch_bounds__(256) void pf_digits(const float *__restrict__ src, int rows, int n, int gs,
                                                 int8_t *__restrict__ planes, int *__restrict__ ge,
                                                 float *__restrict__ gsum) {
    __shared__ unsigned s_max[4][64];
    __shared__ int s_q[4][64];
    const int sub = threadIdx.x >> 6, lane = threadIdx.x & 63, row = blockIdx.x * 4 + sub;
    const int ng = n / gs;
    if (lane < 64) {
        s_max[sub][lane] = 0u;
        s_q[sub][lane] = 0;
    }
    __syncthreads();
    constexpr int kW = 4096 / 8 / 64;   // 8-column words per lane
    float v[kW][8];
#pragma unroll
    for (int k = 0; k < kW; k++) {
        const int w = lane + 64 * k;
#pragma unroll
        for (int c = 0; c < 8; c++) v[k][c] = (row < rows && w * 8 < n) ? src[(size_t)row * n + w * 8 + c] : 0.f;
        float m = 0.f;
#pragma unroll
        for (int c = 0; c < 8; c++) m = fmaxf(m, fabsf(v[k][c]));
        if (w * 8 < n) atomicMax(&s_max[sub][(w * 8) / gs], __float_as_uint(m));
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kW; k++) {
        const int w = lane + 64 * k;
        if (row >= rows || w * 8 >= n) continue;
        const int g = (w * 8) / gs;
        const float m = __uint_as_float(s_max[sub][g]);
        const int e = m > 0.f ? ilogbf(m) + 1 : 0;
        int qs = 0;
        uint32_t pl[3][2] = {{0, 0}, {0, 0}, {0, 0}};   // 8 bytes per plane
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int q = (int)rintf(ldexpf(v[k][c], 22 - e));
            qs += q;
            const uint32_t u = (uint32_t)(q + 0x808080);   // balanced base-256 digits d + 128
            const int pos = perm16((w * 8 + c) & 15) & 7;  // within this 8-byte half
#pragma unroll
            for (int d = 0; d < 3; d++) {
                const uint32_t byte = (((u >> (8 * d)) & 255u) ^ 0x80u);   // d as int8
                pl[d][pos >> 2] |= byte << (8 * (pos & 3));
            }
        }
#pragma unroll
        for (int d = 0; d < 3; d++)
            *(uint2 *)(planes + ((size_t)d * rows + row) * n + w * 8) = make_uint2(pl[d][0], pl[d][1]);
        atomicAdd(&s_q[sub][g], qs);
    }
    __syncthreads();
    if (row < rows && lane < ng) {
        const float m = __uint_as_float(s_max[sub][lane]);
        const int e = m > 0.f ? ilogbf(m) + 1 : 0;
        ge[(size_t)row * ng + lane] = e - 22;
        gsum[(size_t)row * ng + lane] = ldexpf((float)s_q[sub][lane], e - 22);
    }
}

// ---------------------------------------------------------------- grouped GEMM
// One block (4 waves) per (expert, 64 weight rows, pass of kXRows x-rows); gs = 128.
// Per group of 128 columns: lane (row i = l % 16, q = l / 16) loads the 16-byte lanes-
// layout slot of host chunk 4 g + q (32 nibbles: the first 16 feed MFMA half 0, the next
// 16 half 1); the x digits of the pass's rows for the group are staged in LDS once per
// block (double buffered) and read as B fragments; weight slots are loaded kGA groups
// ahead into a register ring.  Scales of the block's rows sit in LDS for the whole pass.
struct PfGemm {
    const ExpertRec *rec;   // [E + 1]
    const int *off;         // [E + 1] first position per expert (routed)
    int E, S, K;            // experts, tokens, slots
    int Kdim, O, ng;        // contraction length, weight rows, groups per row (gs = 128)
    int nl, rb;             // lanes layout: lanes per row, row bytes
    const int8_t *planes;   // digit planes [3][rows][Kdim]
    const int *ge;          // [rows][ng]
    const float *gsum;      // [rows][ng]
    int prow;               // rows of the planes (tokens for gate/up, positions for down)
    const int *plist;       // position -> pair (gate/up: row of planes = pair / K)
    float *out;             // [positions][O] (h for gate/up, y for down)
    int shared;             // 1: the shared expert over all S tokens (positions S*K + t)
};

constexpr int kGS = 128;              // group size of the MFMA path
constexpr int kXRows = 16 * kTT;      // x rows per pass
constexpr int kXPitch = kGS + 16;     // LDS bytes per staged row (bank-conflict-free B reads)
constexpr int kGA = 3;                // weight groups loaded ahead

template <int GU>
__global__ __launch_bounds__(256) void pf_gemm(PfGemm a) {
    constexpr int NM = GU ? 2 : 1;   // weight matrices: (gate, up) or (down)
    __shared__ __attribute__((aligned(16))) int8_t sB[2][3][kXRows][kXPitch];
    __shared__ int sE[2][kXRows];
    __shared__ float sQ[2][kXRows];
    extern __shared__ float2 sS[];   // [NM][kRowBlk][ng] scales of the block's rows
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, j = lane & 15;
    const int nblk = (a.O + kRowBlk - 1) / kRowBlk;
    const int e = a.shared ? a.E : (int)(blockIdx.x / nblk);
    const int rbk = blockIdx.x % nblk;
    const int pos0 = a.shared ? a.S * a.K : a.off[e];
    const int n = a.shared ? a.S : a.off[e + 1] - a.off[e];
    if (blockIdx.y * kXRows >= n) return;   // (uniform) no pass for this block
    const ExpertRec rec = a.rec[e];
    const uint8_t *W[2] = {GU ? rec.wg : rec.wd, rec.wu};
    const float *SZ[2] = {GU ? rec.sg : rec.sd, rec.su};
    const int ng = a.ng;
    const uint32_t wtot = (uint32_t)a.O * a.rb;
    // scales of the block's 64 rows
    for (int m = 0; m < NM; m++)
        for (int v = tid; v < kRowBlk * ng; v += 256) {
            const int r = rbk * kRowBlk + v / ng;
            sS[(m * kRowBlk) * ng + v] = r < a.O ? ((const float2 *)SZ[m])[(size_t)r * ng + v % ng] : make_float2(0.f, 0.f);
        }
    const int arow = rbk * kRowBlk + wave * 16 + j;   // weight row of this lane's A fragment
    // staging thread: x row sr = tid / 8 of the pass, 16 columns at 16 * (tid % 8)
    const int sr = tid >> 3, sc = (tid & 7) * 16;
    for (int pass = blockIdx.y; pass * kXRows < n; pass += gridDim.y) {
        int srow;   // planes row staged by this thread
        {
            const int i = pass * kXRows + sr;
            const int p = pos0 + (i < n ? i : 0);
            srow = GU ? (a.shared ? p - a.S * a.K : a.plist[p] / a.K) : p;
        }
        auto stage_load = [&](int g, uint4 (&rv)[3], int &re, float &rq) {
#pragma unroll
            for (int d = 0; d < 3; d++)
                rv[d] = *(const uint4 *)(a.planes + ((size_t)d * a.prow + srow) * a.Kdim + g * kGS + sc);
            if ((tid & 7) == 0) {
                re = a.ge[(size_t)srow * ng + g];
                rq = a.gsum[(size_t)srow * ng + g];
            }
        };
        auto stage_store = [&](int buf, const uint4 (&rv)[3], int re, float rq) {
#pragma unroll
            for (int d = 0; d < 3; d++) *(uint4 *)&sB[buf][d][sr][sc] = rv[d];
            if ((tid & 7) == 0) {
                sE[buf][sr] = re;
                sQ[buf][sr] = rq;
            }
        };
        uint4 ring[kGA][NM];
        auto a_load = [&](int g, uint4 (&dst)[NM]) {
            const int h = 4 * g + q;   // host chunk of this lane
            const uint32_t off = arow < a.O ? (uint32_t)(arow * a.rb + ((h & 1) * a.nl + (h >> 1)) * 16) : kOOB;
#pragma unroll
            for (int m = 0; m < NM; m++) dst[m] = buf_load16<kCached>(buf_rsrc(W[m], wtot), g < ng ? off : kOOB);
        };
#pragma unroll
        for (int g = 0; g < kGA; g++) a_load(g, ring[g]);
        {
            uint4 rv[3];
            int re = 0;
            float rq = 0.f;
            stage_load(0, rv, re, rq);
            stage_store(0, rv, re, rq);
        }
        __syncthreads();
        float facc[NM][kTT][4];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int tt = 0; tt < kTT; tt++)
#pragma unroll
                for (int r = 0; r < 4; r++) facc[m][tt][r] = 0.f;
        for (int g = 0; g < ng; g++) {
            const int buf = g & 1;
            uint4 rv[3];
            int re = 0;
            float rq = 0.f;
            if (g + 1 < ng) stage_load(g + 1, rv, re, rq);   // next group's x digits, in flight
            uint4 wcur[NM];
#pragma unroll
            for (int u = 0; u < kGA; u++)
                if (u == g % kGA)
#pragma unroll
                    for (int m = 0; m < NM; m++) wcur[m] = ring[u][m];
#pragma unroll
            for (int u = 0; u < kGA; u++)   // refill the slot with group g + kGA
                if (u == g % kGA) a_load(g + kGA, ring[u]);
            pf_v4i iacc[NM][3][kTT];
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int d = 0; d < 3; d++)
#pragma unroll
                    for (int tt = 0; tt < kTT; tt++) iacc[m][d][tt] = pf_v4i{0, 0, 0, 0};
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                pf_v4i av[NM];
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    uint32_t e0, o0, e1, o1;
                    nib8(hh ? wcur[m].z : wcur[m].x, e0, o0);
                    nib8(hh ? wcur[m].w : wcur[m].y, e1, o1);
                    av[m] = pf_v4i{(int)e0, (int)o0, (int)e1, (int)o1};
                }
#pragma unroll
                for (int d = 0; d < 3; d++)
#pragma unroll
                    for (int tt = 0; tt < kTT; tt++) {
                        const pf_v4i bv = *(const pf_v4i *)&sB[buf][d][tt * 16 + j][32 * q + 16 * hh];
#pragma unroll
                        for (int m = 0; m < NM; m++)
                            iacc[m][d][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[m], bv, iacc[m][d][tt], 0, 0, 0);
                    }
            }
            // fold the group: T = t0 + 256 t1 + 65536 t2 (t2 * 65536 exact in fp32)
#pragma unroll
            for (int tt = 0; tt < kTT; tt++) {
                const int xe = sE[buf][tt * 16 + j];
                const float xs = sQ[buf][tt * 16 + j];
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float2 sz = sS[(m * kRowBlk + wave * 16 + 4 * q + r) * ng + g];
                        const float lo = (float)(iacc[m][0][tt][r] + 256 * iacc[m][1][tt][r]);
                        const float T = fmaf((float)iacc[m][2][tt][r], 65536.f, lo);
                        const float v = fmaf(-(sz.y - 8.f), xs, ldexpf(T, xe));
                        facc[m][tt][r] = fmaf(sz.x, v, facc[m][tt][r]);
                    }
            }
            if (g + 1 < ng) stage_store(buf ^ 1, rv, re, rq);
            __syncthreads();
        }
        // epilogue: lane holds rows 4 q + r of the wave tile for x row j of each tile
#pragma unroll
        for (int tt = 0; tt < kTT; tt++) {
            const int i = pass * kXRows + tt * 16 + j;
            if (i >= n) continue;
            const size_t p = (size_t)pos0 + i;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int orow = rbk * kRowBlk + wave * 16 + 4 * q + r;
                if (orow >= a.O) continue;
                float v;
                if (GU) {   // c/qwen.c:780-786, silu c/qwen.c:173
                    const float gv = facc[0][tt][r];
                    v = gv / (1.f + expf(-gv)) * facc[NM - 1][tt][r];
                } else {
                    v = facc[0][tt][r];
                }
                a.out[p * a.O + orow] = v;
            }
        }
    }
}

// ---------------------------------------------------------------- combine
// out[t] = sum over t's K experts in ascending expert id of w * y[pos] + shgt * y_sh[t]
__global__ __launch_bounds__(256) void pf_combine(const float *__restrict__ y, const int *tidx, const float *tval,
                                                  const float *tshg, const int *ppos, int S, int K, int D,
                                                  float *out) {
    const int t = blockIdx.x;
    int ord[kTopK];
    int nk = 0;
    for (int k = 0; k < K; k++) {   // slots sorted by expert id (insertion; K <= 8 here)
        int j = nk++;
        while (j > 0 && tidx[t * K + ord[j - 1]] > tidx[t * K + k]) {
            ord[j] = ord[j - 1];
            j--;
        }
        ord[j] = k;
    }
    const float shg = tshg[t];
    const float *ysh = y + (size_t)(S * K + t) * D;
    for (int c = threadIdx.x; c < D; c += 256) {
        float acc = 0.f;
        for (int i = 0; i < K; i++) {
            const int k = ord[i];
            acc = acc + tval[t * K + k] * y[(size_t)ppos[t * K + k] * D + c];
        }
        out[(size_t)t * D + c] = acc + shg * ysh[c];
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
    if (!ok() || !router || !d_xs || !d_out || S < 1) return false;
    if (!moe_layer(layer, &rec, &shg, &m, &E)) return false;
    if (K < 1 || K > kTopK || K > E || E > kMaxE) return false;
    if (router->I != m.D || router->O != E || (router->fmt != 0 && router->fmt != 1) || router->layout != kLayoutRows)
        return false;
    if (m.gs != kGS || m.D % kGS || m.I % kGS || m.D > 4096 || m.I > 4096) return false;
    const int D = m.D, I = m.I, np = S * K, P = np + S, ngD = D / m.gs, ngI = I / m.gs;
    // scratch layout
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += al256(bytes);
        return at;
    };
    const size_t o_lg = take((size_t)S * (E + 1) * 4), o_ti = take((size_t)np * 4), o_tv = take((size_t)np * 4),
                 o_sh = take((size_t)S * 4), o_cnt = take((size_t)(E + 1) * 4), o_off = take((size_t)(E + 1) * 4),
                 o_pl = take((size_t)np * 4), o_pp = take((size_t)np * 4), o_rk = take((size_t)np * 4),
                 o_xd = take((size_t)3 * S * D), o_xe = take((size_t)S * ngD * 4), o_xs = take((size_t)S * ngD * 4),
                 o_h = take((size_t)P * I * 4), o_hd = take((size_t)3 * P * I), o_he = take((size_t)P * ngI * 4),
                 o_hs = take((size_t)P * ngI * 4), o_y = take((size_t)P * D * 4);
    if (!scratch(&g_pf.buf, &g_pf.cap, o)) return false;
    uint8_t *b = (uint8_t *)g_pf.buf;
    float *lg = (float *)(b + o_lg), *tv = d_val ? d_val : (float *)(b + o_tv), *tsh = (float *)(b + o_sh);
    int *ti = d_idx ? d_idx : (int *)(b + o_ti), *cnt = (int *)(b + o_cnt), *off = (int *)(b + o_off);
    int *pl = (int *)(b + o_pl), *pp = (int *)(b + o_pp), *rk = (int *)(b + o_rk);
    int8_t *xd = (int8_t *)(b + o_xd), *hd = (int8_t *)(b + o_hd);
    int *xe = (int *)(b + o_xe), *he = (int *)(b + o_he);
    float *xsum = (float *)(b + o_xs), *hsum = (float *)(b + o_hs), *h = (float *)(b + o_h), *y = (float *)(b + o_y);

    hipLaunchKernelGGL(pf_logits, dim3((S + kLT - 1) / kLT, (E + 1 + kLE - 1) / kLE), dim3(256), 0, st, d_xs, S, D,
                       router->w, router->sz, router->fmt, router->row_bytes, E, shg, lg);
    hipLaunchKernelGGL(pf_route, dim3(S), dim3(kThreads), 0, st, lg, E, K, ti, tv, tsh);
    hipLaunchKernelGGL(pf_group, dim3(1), dim3(1024), (size_t)(E + 1) * 4, st, ti, np, E, cnt, off, pl, pp, rk);
    hipLaunchKernelGGL(pf_digits, dim3((S + 3) / 4), dim3(256), 0, st, d_xs, S, D, m.gs, xd, xe, xsum);
    PfGemm gu;
    memset(&gu, 0, sizeof(gu));
    gu.rec = rec;
    gu.off = off;
    gu.E = E;
    gu.S = S;
    gu.K = K;
    gu.Kdim = D;
    gu.O = I;
    gu.ng = ngD;
    gu.nl = m.nlG;
    gu.rb = m.rbG;
    gu.planes = xd;
    gu.ge = xe;
    gu.gsum = xsum;
    gu.prow = S;
    gu.plist = pl;
    gu.out = h;
    const int nbu = (I + kRowBlk - 1) / kRowBlk, nbd = (D + kRowBlk - 1) / kRowBlk;
    const int passes_sh = (S + 16 * kTT - 1) / (16 * kTT);
    const size_t lds_gu = (size_t)2 * kRowBlk * ngD * sizeof(float2), lds_dn = (size_t)kRowBlk * ngI * sizeof(float2);
    hipLaunchKernelGGL(pf_gemm<1>, dim3(E * nbu, 2), dim3(256), lds_gu, st, gu);
    gu.shared = 1;
    hipLaunchKernelGGL(pf_gemm<1>, dim3(nbu, passes_sh), dim3(256), lds_gu, st, gu);
    hipLaunchKernelGGL(pf_digits, dim3((P + 3) / 4), dim3(256), 0, st, h, P, I, m.gs, hd, he, hsum);
    PfGemm dn = gu;
    dn.shared = 0;
    dn.Kdim = I;
    dn.O = D;
    dn.ng = ngI;
    dn.nl = m.nlD;
    dn.rb = m.rbD;
    dn.planes = hd;
    dn.ge = he;
    dn.gsum = hsum;
    dn.prow = P;
    dn.out = y;
    hipLaunchKernelGGL(pf_gemm<0>, dim3(E * nbd, 2), dim3(256), lds_dn, st, dn);
    dn.shared = 1;
    hipLaunchKernelGGL(pf_gemm<0>, dim3(nbd, passes_sh), dim3(256), lds_dn, st, dn);
    hipLaunchKernelGGL(pf_combine, dim3(S), dim3(256), 0, st, y, ti, tv, tsh, pp, S, K, D, d_out);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail("moe prefill launch", err);
    return true;
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
