/*
 * oracle.h - CPU restatement of qwen3.c's fmt=6 int4 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product library (qwen3.c_amd/) never links, loads or calls it, and has no CPU
 * fallback that could route through it.
 *
 * Every function restates the reference CPU semantics of zhaohb/qwen3.c (the
 * `--no-vulkan` path) and cites the file:line it follows.  Build flags match the
 * reference's stock build (c/Makefile:22-30: gcc -O2 -std=c11); -std=c11 keeps
 * GCC from contracting a*b+c into FMA, which the bit-exact comparison needs.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   orc_matmul_q4g_asym    golden vectors from the compiled reference; f64 brute force;
 *                          closed forms (z=0,s=1 integer dot; constant nibbles; gs=K)
 *   orc_matmul_f32/_q8     golden vectors from the compiled reference; f64 brute force
 *   orc_quant_rows         golden vectors from the compiled reference; round-trip bound
 *   orc_rmsnorm_zc         golden vectors from the compiled reference; closed form
 *   orc_route_topk         golden (through moe outputs); invariants; forced ties
 *   orc_expert_mlp_fmt6    golden vectors from the compiled reference
 *   orc_moe_decode         golden vectors from the compiled reference (moe_token)
 *   orc_moe_prefill        golden vectors from the compiled reference (moe_batch);
 *                          per-token brute force
 *   orc_argmax/_topk_logits  full sort on random and forced-tie inputs
 *   orc_gqa_decode         golden vectors from the compiled reference (attention);
 *                          closed forms (pos 0 attends to itself; rope identities)
 *   orc_gdn_step           golden vectors from the compiled reference (gdn_step);
 *                          f64 brute force of the recurrence
 *   orc_gen_*              hash / stream known-answer values; distribution moments
 */
#ifndef QWEN_HIP_ORACLE_H
#define QWEN_HIP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fmt=6 layout (c/qwen.c:207-229, c/tools/convert_qwen35_moe.py:124-144) ----
 * W is U8 [O, (I+1)/2] row-major; element i of a row sits in byte i>>1, low nibble
 * when i is even.  sz is f32 [O, ng, 2] with ng = ceil(I/gs), interleaved
 * [scale_g, zero_g]; weight = (nibble - zero_g) * scale_g. */

/* c/qwen.c:211-229 matmul_q4g_asym */
void orc_matmul_q4g_asym(float *y, const float *x, const uint8_t *q, const float *sz,
                         int I, int O, int gs);
/* c/qwen.c:178-189 matmul (f32, S rows) */
void orc_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O);
/* c/qwen.c:230-238 matmul_q8 (fmt 1: int8 rows, per-row scale) */
void orc_matmul_q8(float *y, const float *x, const uint8_t *q, const float *scale, int I, int O);
/* c/qwen.c:242-292 quant_rows (fmt 6 grouped-asym int4, fmt 1 int8) */
void orc_quant_rows(const float *W, int I, int O, int fmt, int gs, uint8_t *q, float *s);
/* c/qwen.c:326-330 rmsnorm_zc (double accumulator) */
void orc_rmsnorm_zc(float *out, const float *x, const float *w, int D, float eps);
/* c/qwen.c:332-336 softmax_row */
void orc_softmax_row(float *x, int n);
/* c/qwen.c:172-173 */
float orc_sigmoid(float x);
float orc_silu(float x);

/* c/qwen.c:806-817: softmax over all E logits (pr is overwritten with the
 * probabilities), K greedy picks with strict '>' from bv=-1 (ties -> lower index),
 * then val /= sum(val). idx/val in rank order. */
void orc_route_topk(float *pr, int E, int K, int *idx, float *val);

/* One fmt=6 expert: gate/up [I, D] and down [D, I]. */
typedef struct {
    const uint8_t *g, *u, *d;
    const float *gs, *us, *ds;
} OrcExpert;

/* c/qwen.c:780-786 expert_mlp_cpu, fmt 6 branch. h (optional scratch [I]) */
void orc_expert_mlp_fmt6(const OrcExpert *e, const float *x, int D, int I, int gs, float *y);

/* c/qwen.c:922-928 moe_token -> :804-920 moe_from_logits, pure-CPU branch, with the
 * shared expert quantized (mm_dense's quantized fallback :300-305 for gsg/gsu/gsd).
 *   out[d] = sum_k val_k * y_k[d] (rank order), then out[d] += shgt * y_sh[d].
 * router f32 [E, D]; experts[E]; idx/val/shgt/logits outputs may be NULL. */
void orc_moe_decode(const float *x, const float *router, const OrcExpert *experts,
                    const OrcExpert *shared, const float *sh_gate,
                    int D, int I, int E, int K, int gs,
                    float *out, int *idx, float *val, float *shgt, float *logits);

/* c/qwen.c:1185-1190 moe_batch -> :1050-1183 moe_batch_from_logits, pure-CPU branch:
 * route all S tokens, bucket (token,slot) pairs by expert (counting sort), then
 * out[tok] += w * y in ascending expert id, pair order within an expert; shared
 * expert over all rows last.  tidx/tval [S*K] outputs may be NULL. */
void orc_moe_prefill(const float *xs, int S, const float *router, const OrcExpert *experts,
                     const OrcExpert *shared, const float *sh_gate,
                     int D, int I, int E, int K, int gs,
                     float *out, int *tidx, float *tval);

/* ---- attention / GatedDeltaNet layer blocks (decode, one token) ----
 * A dense projection as c/qwen.c:296-309 mm_dense evaluates it on the CPU: fmt 6 = the
 * quantized host copy through matmul_q4g_asym, fmt 0 = f32 rows [O, I] through matmul. */
typedef struct {
    int fmt;
    const void *w;
    const float *sz;
    int I, O, gs;
} OrcMat;
void orc_proj(const OrcMat *m, const float *x, float *y);

/* c/qwen.c:570-579 rope_partial: half-half rotation of the first rot dims. */
void orc_rope_partial(float *x, int pos, int rot, float theta);

/* Gated GQA layer (c/qwen.c:581-667, S = 1): q_proj emits [q | gate] per head; per-head
 * zero-centred q/k norm, partial RoPE at pos, K/V rows written to the caches
 * ([KH][max_t][hd]), softmax attention over positions 0..pos, output gate
 * sigmoid(gate), o_proj. */
typedef struct {
    OrcMat q, k, v, o;
    const float *qn, *kn;
    int H, KH, hd, rot;
    float theta, eps;
} OrcGqa;
void orc_gqa_decode(const OrcGqa *L, float *Kc, float *Vc, int max_t, int pos, const float *x, float *out);

/* GatedDeltaNet layer, one token (c/qwen.c:669-776, CPU branch): qkv/z projections,
 * causal conv1d over the ring convst [K][CD] (slot K-1 newest) + SiLU, per-k-head l2norm
 * (q also / sqrt(KD)), decay = exp(-exp(alog) softplus(a + dtb)), beta = sigmoid(b),
 * delta rule on S [VH][KD][VD], gated RMSNorm (gnorm, SiLU(z)), out projection. */
typedef struct {
    OrcMat qkv, z, a, b, out;
    const float *conv;
    const float *alog, *dtb, *gnorm;
    int KH, KD, VH, VD, K;
    float eps;
} OrcGdn;
void orc_gdn_step(const OrcGdn *L, float *convst, float *S, const float *x, float *out);

/* c/qwen.c:1471-1472: ascending scan, strict '>' (ties -> lowest index). */
int orc_argmax(const float *v, int n);
/* Top-k over a logit vector.  The reference has no such routine; this is defined
 * as k rounds of the c/qwen.c:1471-1472 scan without replacement (descending value,
 * ties -> lower index), i.e. a stable descending sort's first k entries. */
void orc_topk_logits(const float *v, int n, int k, int *idx, float *val);

/* ---- deterministic synthetic data (shared spec with the device generator) ----
 * h(seed, i) = mix64(seed + (i+1) * 0x9E3779B97F4A7C15): the i-th output of a
 * splitmix64 stream started at `seed` (Steele, Lea, Flood 2014).
 * u01(seed, i) = ((h >> 11) + 0.5) * 2^-53 in (0,1)
 * normal(seed, i) = sqrt(-2 ln u01(seed,2i)) * cos(2 pi u01(seed,2i+1))  (Box-Muller)
 * stream(base, tag) = mix64(base ^ mix64(tag + 1)) gives each tensor its own seed. */
uint64_t orc_mix64(uint64_t z);
uint64_t orc_hash(uint64_t seed, uint64_t i);
uint64_t orc_stream(uint64_t base, uint64_t tag);
double   orc_normal(uint64_t seed, uint64_t i);
/* round-to-nearest-even to IEEE binary16 precision, returned as float */
float    orc_f16_round(double v);
/* byte j = bits [8*(j&7), 8*(j&7)+8) of h(seed, j>>3) */
void orc_gen_bytes(uint8_t *dst, size_t n, uint64_t seed);
/* [scale, zero] pairs for ng groups: scale = f16(|sigma*normal(seed, g)|),
 * zero = h(seed ^ 0x5A5A5A5A5A5A5A5A, g) >> 60 (uniform 0..15), stored as f32 */
void orc_gen_sz(float *sz, size_t ngroups, uint64_t seed, double sigma);
/* dst[i] = (float)(sigma * normal(seed, i)) */
void orc_gen_normal(float *dst, size_t n, uint64_t seed, double sigma);

#ifdef __cplusplus
}
#endif
#endif
