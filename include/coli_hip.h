/*
 * coli_hip.h - C ABI of libcoli_hip.so, the MI355X (gfx950) replacement for the
 * Vulkan backend of zhaohb/qwen3.c.
 *
 * Part 1 declares every entry point of the reference's c/backend_vulkan.h with the same
 * name, signature and return convention, so c/qwen.c builds and links against this
 * library unchanged (backend_vulkan.h in this directory forwards here).  Each comment
 * cites the reference declaration it replaces.  Conventions kept from the reference:
 *   - int 1 = success, 0 = unavailable / failed -> the caller computes on the CPU
 *     (c/backend_vulkan.h:55-57, c/qwen.c:296-308);
 *   - a device failure is sticky: every later call returns 0 (c/backend_vulkan.c:1280);
 *   - tensors are created lazily through the in/out ColiVkTensor** handle and own a
 *     device copy of the caller's host weights (c/backend_vulkan.c:1055-1085);
 *   - one host thread; at most one expert group in flight (c/backend_vulkan.c:1648).
 * Entry points that always return 0 (the caller then computes that step on the CPU):
 *   - the GLM MLA paths, which c/qwen.c never calls: coli_vk_attention_absorb,
 *     coli_vk_attn_qprep, coli_vk_attention_absorb_project;
 *   - the staged attention/GDN forms that take host-computed q or recurrence inputs:
 *     coli_vk_gqa, coli_vk_gqa_project, coli_vk_gdn, coli_vk_gdn_project.  The engine
 *     reaches them only when a fused block (coli_vk_gqa_full*, coli_vk_gdn_full*) is off,
 *     and falls back per call (c/qwen.c:620-636, 732-745).  coli_vk_gqa_available and
 *     coli_vk_gdn_available still report 1: they also gate the KV mirror, the GDN state
 *     and the fused blocks, which are implemented.
 *
 * Part 2 (coli_hip_*) has no counterpart in the reference: device-pointer forms of the
 * hot path for callers whose inputs already live in HBM (the benchmark, the parity
 * tests, a device-resident engine), plus the device synthetic-data generator.
 *
 * Plain pointers and sizes only.  `void *stream` is a hipStream_t (NULL = the
 * library's own stream); work issued on it is stream-ordered and not synchronised.
 */
#ifndef COLI_HIP_H
#define COLI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* c/backend_vulkan.h:33 - opaque device copy of one quantized tensor.  fmt 6 (grouped
 * asymmetric int4, [scale, zero] f32 per group) and fmt 1 (int8, f32 per-row scale) as
 * in the reference; fmt 0 (plain f32 rows, scales NULL) is an addition used for the f32
 * MoE router. */
typedef struct ColiVkTensor ColiVkTensor;

/* ======================= Part 1: the drop-in ABI ======================= */

/* c/backend_vulkan.h:37-40 */
int  coli_vk_init(const char *spv_path);            /* spv_path ignored (kernels are built in) */
void coli_vk_shutdown(void);
int  coli_vk_available(void);
void coli_vk_mem_info(size_t *used_bytes, size_t *tensor_count);
/* c/backend_vulkan.h:49-50 (no eviction classes on HBM: alloc_priority is a no-op) */
void coli_vk_alloc_priority(float p);
int  coli_vk_mem_budget(double *used_gb, double *budget_gb);

/* c/backend_vulkan.h:56-59: y[S,O] = x[S,I] @ dequant(W)^T */
int  coli_vk_matmul(ColiVkTensor **tensor, float *y, const float *x,
                    const void *weights, const float *scales,
                    int fmt, int S, int I, int O, int gs);
/* c/backend_vulkan.h:66-68: lm_head GEMV + device argmax, ties -> lowest index */
int  coli_vk_matmul_argmax(ColiVkTensor **tensor, const void *weights, const float *scales,
                           int fmt, int I, int O, int gs,
                           const float *x, int *idx, float *val);
/* c/backend_vulkan.h:75-79: hidden[s,o] = silu(gate(x)) * up(x) */
int  coli_vk_gate_up(ColiVkTensor **gate, ColiVkTensor **up, float *hidden, const float *x,
                     const void *gw, const float *gs, const void *uw, const float *us,
                     int fmt, int S, int D, int I, int grp);
/* c/backend_vulkan.h:85-101: batched expert MLP y_c = down_c(silu(gate_c x_c) * up_c x_c) */
int  coli_vk_expert_group(ColiVkTensor *const *gates, ColiVkTensor *const *ups,
                          ColiVkTensor *const *downs, const int *rows, int count,
                          float *y, const float *x);
int  coli_vk_expert_group_issue(ColiVkTensor *const *gates, ColiVkTensor *const *ups,
                                ColiVkTensor *const *downs, const int *rows, int count,
                                const float *x);
int  coli_vk_expert_group_take(float *y);
int  coli_vk_eg_gather_available(void);
int  coli_vk_eg_xs_bind(const float *xs, int S, int D);
int  coli_vk_expert_group_issue_id(ColiVkTensor *const *gates, ColiVkTensor *const *ups,
                                   ColiVkTensor *const *downs, const int *rows, int count,
                                   const int *tok_ids);
/* c/backend_vulkan.h:105 */
int  coli_vk_tensor_ensure(ColiVkTensor **tensor, const void *weights, const float *scales,
                           int fmt, int I, int O, int grp);
/* c/backend_vulkan.h:114-116: device KV mirror (rows kv_head * max_t + pos; also the GQA cache) */
int  coli_vk_kv_ensure(int layer, int max_rows, int K, int Rd);
int  coli_vk_kv_row(int layer, int pos, const float *L, const float *R);
void coli_vk_kv_reset(void);
/* c/backend_vulkan.h:117-119, 125-131, 138-141: GLM MLA paths (unused by c/qwen.c): return 0 */
int  coli_vk_attention_absorb(ColiVkTensor **kvb, const void *w, const float *sc, int fmt, int grp,
                              float *ctx, const float *q, int layer, int S, int H,
                              int Q, int R, int V, int K, int st0, int T, float scale);
int  coli_vk_attn_qprep(int layer,
                        ColiVkTensor **qa,  const void *wqa,  const float *sqa,  int Oqa,
                        ColiVkTensor **kva, const void *wkva, const float *skva, int Okva,
                        ColiVkTensor **qb,  const void *wqb,  const float *sqb,  int Oqb,
                        int fmt, int grp, const float *lnw, float eps,
                        const float *x, int S, int I, float *q_out, float *kv_out,
                        float *lat_out);
/* c/backend_vulkan.h:132-134: two GEMVs sharing x, one synchronisation */
int  coli_vk_matmul_pair(ColiVkTensor **t1p, float *y1, const void *w1, const float *s1, int O1,
                         ColiVkTensor **t2p, float *y2, const void *w2, const float *s2, int O2,
                         int fmt, const float *x, int S, int I, int grp);
int  coli_vk_attention_absorb_project(ColiVkTensor **kvb, const void *w, const float *sc, int fmt, int grp,
                              ColiVkTensor **ot, const void *ow, const float *osc, int ofmt, int ogrp,
                              float *out, const float *q, int layer, int S, int H,
                              int Q, int R, int V, int K, int st0, int T, float scale, int Dout);
/* c/backend_vulkan.h:143-144 (arena slices are not reclaimed, as in the reference) */
void   coli_vk_tensor_free(ColiVkTensor *t);
size_t coli_vk_tensor_bytes(const ColiVkTensor *t);

/* c/backend_vulkan.h:151-157: GatedDeltaNet recurrence */
int  coli_vk_gdn_available(void);
int  coli_vk_gdn_state_ensure(int layer, int VH, int KD, int VD);
void coli_vk_gdn_reset(void);
int  coli_vk_gdn(int layer, const float *qn, const float *kn, const float *v, const float *z,
                 const float *decay, const float *beta, const float *gnorm, float *y,
                 int KH, int KD, int VH, int VD, float eps);
/* c/backend_vulkan.h:162-180: GQA decode attention */
int  coli_vk_gqa_available(void);
int  coli_vk_gqa(int layer, const float *q, float *ctx, int S, int H, int KH, int hd,
                 int max_t, int st0, int T, float scale);
int  coli_vk_gqa_project(int layer, const float *q, ColiVkTensor *ot, float *out,
                         int S, int H, int KH, int hd, int max_t, int st0, int T,
                         float scale, int Dout);
int  coli_vk_gqa_full_available(void);
int  coli_vk_gqa_norm_weight(int layer, const float *qnw, const float *knw, int hd);
int  coli_vk_gqa_full(int layer, const float *x, int D, ColiVkTensor *gq_t, ColiVkTensor *gk_t,
                      ColiVkTensor *gv_t, ColiVkTensor *out_t, float *out, int S, int H, int KH,
                      int hd, int rot, int pos_base, int max_t, float eps, float theta, int Dout);
/* c/backend_vulkan.h:185-198: MoE route prep fused after the attention/GDN block */
int  coli_vk_moe_route_available(void);
int  coli_vk_layer_norm_weight(int layer, const float *in_ln, const float *post_ln, int D);
int  coli_vk_gqa_full_route(int layer, const float *resid, int D,
                            ColiVkTensor *gq_t, ColiVkTensor *gk_t, ColiVkTensor *gv_t, ColiVkTensor *out_t,
                            ColiVkTensor *router, int ln_layer,
                            float *resid_out, float *nrm_out, float *pr_out,
                            int S, int H, int KH, int hd, int rot, int pos_base, int max_t,
                            float eps, float theta, int Dout, int E);
int  coli_vk_gdn_full_route(int layer, const float *x_in, const float *resid, int D,
                            ColiVkTensor *gqkv_t, ColiVkTensor *gz_t, const float *params,
                            ColiVkTensor *out_t, ColiVkTensor *router, int ln_layer,
                            float *resid_out, float *nrm_out, float *pr_out,
                            int KH, int KD, int VH, int VD, int conv_dim, int conv_k,
                            float eps, int Dout, int E);
/* c/backend_vulkan.h:206-221: device-resident residual stream */
int  coli_vk_stream_available(void);
int  coli_vk_stream_begin(const float *x, int D);
int  coli_vk_stream_end(float *x, int D);
int  coli_vk_stream_add(const float *y, int D);
const float *coli_vk_stream_nrm(void);
int  coli_vk_final_norm_weight(const float *w, int D);
int  coli_vk_stream_norm_argmax(ColiVkTensor **tensor, const void *weights, const float *scales,
                                int fmt, int I, int O, int gs, float eps, int *idx, float *val);
int  coli_vk_stream_copy_resid(float *x, int D);
void coli_vk_route_cache_stats(void);
void coli_vk_decode_prof(double decode_ms, int tokens);
/* c/backend_vulkan.h:222-241: layer blocks with device routing (stream path) */
int  coli_vk_gdn_ba_weight(int layer, const float *alog, const float *dtb,
                           const float *gnorm, int VH, int VD);
int  coli_vk_gqa_full_route_pipe(int layer, int D,
                                 ColiVkTensor *gq_t, ColiVkTensor *gk_t, ColiVkTensor *gv_t, ColiVkTensor *out_t,
                                 ColiVkTensor *router, int ln_layer,
                                 int *idx_out, float *val_out, int topk,
                                 int H, int KH, int hd, int rot, int pos_base, int max_t,
                                 float eps, float theta, int Dout, int E);
int  coli_vk_gdn_full_route_pipe(int layer, int D,
                                 ColiVkTensor *gqkv_t, ColiVkTensor *gz_t,
                                 ColiVkTensor *gba_t, ColiVkTensor *gbb_t,
                                 ColiVkTensor *out_t, ColiVkTensor *router, int ln_layer,
                                 int *idx_out, float *val_out, int topk,
                                 int KH, int KD, int VH, int VD, int conv_dim, int conv_k,
                                 float eps, int Dout, int E);
int  coli_vk_expert_group_issue_pipe(ColiVkTensor *const *gates, ColiVkTensor *const *ups,
                                     ColiVkTensor *const *downs, const int *rows,
                                     const float *weights, int count, int D);
int  coli_vk_expert_group_take_pipe(void);
/* c/backend_vulkan.h:243-252: device-indexed MoE over a per-layer expert table */
int  coli_vk_moe_ix_available(void);
int  coli_vk_eg_table_init(int n_layers, int E, int D, int I, int gs);
int  coli_vk_eg_table_set(int layer, int eid, ColiVkTensor *g, ColiVkTensor *u, ColiVkTensor *d);
int  coli_vk_eg_table_set_shared(int layer, ColiVkTensor *g, ColiVkTensor *u, ColiVkTensor *d,
                                 const float *sh_gate, int D);
int  coli_vk_stream_moe_fused(void);
int  coli_vk_stream_ix_pending(void);
int  coli_vk_stream_ix_hist(int layer, int *idx_out, int K);
/* c/backend_vulkan.h:258-279: GDN block forms */
int  coli_vk_gdn_project(int layer, const float *qn, const float *kn, const float *v, const float *z,
                         const float *decay, const float *beta, const float *gnorm,
                         ColiVkTensor *ot, float *out, int KH, int KD, int VH, int VD,
                         float eps, int Dout);
int  coli_vk_gdn_full_available(void);
int  coli_vk_gdn_conv_ensure(int layer, int conv_k, int conv_dim);
int  coli_vk_gdn_conv_weight(int layer, const float *cw, int conv_k, int conv_dim);
int  coli_vk_gdn_full(int layer, const float *x, int D, ColiVkTensor *gqkv_t, ColiVkTensor *gz_t,
                      const float *params, ColiVkTensor *out_t, float *out,
                      int KH, int KD, int VH, int VD, int conv_dim, int conv_k, float eps, int Dout);
int  coli_vk_gdn_full_seq(int layer, const float *x, int S, int D,
                          ColiVkTensor *gqkv_t, ColiVkTensor *gz_t, const float *params,
                          ColiVkTensor *out_t, float *out,
                          int KH, int KD, int VH, int VD, int conv_dim, int conv_k,
                          float eps, int Dout);

/* ============ Part 2: device-pointer extensions (no reference counterpart) ============ */

/* Device view of a tensor: weights d_w [O, row_bytes] (row_bytes a multiple of 16,
 * zero padded), d_sz as uploaded.  Returns 0 for NULL. */
int   coli_hip_tensor_info(const ColiVkTensor *t, int *fmt, int *I, int *O, int *gs,
                           int *row_bytes, void **d_w, void **d_sz);
/* The library's stream (hipStream_t); wait for a stream; blocking copy between any
 * host / device addresses. */
void *coli_hip_stream(void);
int   coli_hip_sync(void *stream);
int   coli_hip_memcpy(void *dst, const void *src, size_t bytes);
/* y[S,O] = x[S,I] @ dequant(W)^T on device pointers. */
int   coli_hip_gemv(const ColiVkTensor *t, const float *d_x, float *d_y, int S, void *stream);
/* GEMV fused with the k best outputs (k <= 8; value desc, index asc); d_y may be NULL.
 * If the in-launch merge's bounded wait gives up, that launch writes -1 to d_idx[0..k)
 * and sets the error word that coli_hip_gemv_error reports. */
int   coli_hip_gemv_topk(const ColiVkTensor *t, const float *d_x, float *d_y, int k,
                         int *d_idx, float *d_val, void *stream);
/* Error word of the fused top-k launches since the last call (synchronises the device):
 * 0 none, 1 a bounded wait gave up, -1 runtime error.  Reading clears it. */
int   coli_hip_gemv_error(void);
/* Create a tensor whose contents are generated on the device with the synthetic-data
 * spec (fmt 6: bytes = stream(seed,1), [scale,zero] = stream(seed,2) with scale sigma;
 * fmt 0: rows = sigma * normal(stream(seed,3))); equal to uploading the host-generated
 * buffers.  Returns 0 on failure. */
int   coli_hip_tensor_synth(ColiVkTensor **t, int fmt, int I, int O, int gs,
                            uint64_t seed, double sigma);
/* d_dst[i] = (float)(sigma * normal(seed, i)) for i < n. */
int   coli_hip_synth_normal(float *d_dst, size_t n, uint64_t seed, double sigma, void *stream);
/* One layer's MoE block (router -> softmax/top-K -> K routed + shared expert -> weighted
 * combine, c/qwen.c:804-920) in one launch over the expert table of coli_vk_eg_table_*.
 * K <= 8; router fmt 0 (f32) or 1 (int8), [E, D].  d_out[D] = the block output
 * (accumulate != 0: d_out += it).  d_idx[K] (rank order) and d_val[K + 1] (renormed
 * weights, then the shared gate) may be NULL.  Launches share one scratch area: issue
 * them on one stream. */
int   coli_hip_moe_decode(int layer, const ColiVkTensor *router, int K, const float *d_x,
                          float *d_out, int accumulate, int *d_idx, float *d_val, void *stream);
/* coli_hip_moe_decode without any allocation: same arguments, same kernel and results.  No
 * counterpart in the reference; it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops).  The cross-block words live in a static device
 * array of 256 KiB per device (error line + 32736 tag words), held until the process
 * ends: a call needing more tag words (3 (E + 1) + 128 + (K + 1)(I + D)) is refused with a
 * message and returns 0.  Nothing needs clearing between calls (words carry the call's
 * epoch); calls that overlap on one device race on the array.  Errors are reported by
 * coli_hip_moe_error. */
int   coli_hip_moe_decode_noalloc(int layer, const ColiVkTensor *router, int K, const float *d_x,
                                  float *d_out, int accumulate, int *d_idx, float *d_val, void *stream);
/* Error word of the MoE launches since the last call, coli_hip_moe_decode_noalloc's
 * included (synchronizes the device): 0 none, 1 a bounded wait gave up, 2 an out-of-range
 * expert id, -1 runtime error.  Reading clears it. */
int   coli_hip_moe_error(void);
/* Test hook for the failure path: sets the MoE error word from the host (code 1 or 2), so
 * the next MoE launches' bounded waits give up at their 16th poll (every kernel still
 * exits normally) and the stream entry points report the failure (return 0, device
 * disabled) as after a real give-up.  Returns 1 when the word was written. */
int   coli_hip_moe_force_error(int code);
/* The layer's MoE block over S token rows d_xs[S, D] (prefill / ragged batch,
 * c/qwen.c:1050-1183): per-token routing, rows grouped by expert, expert projections as
 * grouped GEMMs on MFMA (int8 digits of the activations x int4 weights, exact integer
 * group sums), out[t] = sum in ascending expert id of w * y + shgt * y_shared.  K <= 8.
 * d_idx / d_val [S, K] (routing, rank order) may be NULL. */
int   coli_hip_moe_prefill(int layer, const ColiVkTensor *router, int K, const float *d_xs, int S,
                           float *d_out, int *d_idx, float *d_val, void *stream);
/* Bulk form of coli_vk_kv_row: mirror rows [row0, row0 + n) of an attention layer from
 * host arrays K [n][kd] and V [n][vd] (seeds a cache of a given length).  _read copies
 * them back. */
int   coli_hip_kv_load(int layer, int row0, int n, const float *K, const float *V);
int   coli_hip_kv_read(int layer, int row0, int n, float *K, float *V);
/* A GDN layer's state in the reference's host layouts: conv ring [conv_k][conv_dim]
 * (slot conv_k - 1 newest) and recurrent state [VH][KD][VD] (c/qwen.c:749-767). */
int   coli_hip_gdn_state_read(int layer, float *ring, float *S);
/* Fused layer launches (one kernel for a decode token's GatedDeltaNet in-projection,
 * recurrence and out-projection, where the shapes allow) on (1) or off (0: the separate
 * kernels); returns the previous setting.  Both give the same results bit for bit.  No
 * counterpart in the reference (its layer is separate dispatches).  Off by default (slower on
 * MI355X at configs[3]); the environment variable COLI_HIP_FUSE=1 starts with it on. */
int   coli_hip_layer_fuse(int on);
/* Routing certification of every decode route (each top-k candidate's logit recomputed as
 * the reference's sequential fp32 sum and ranked by it) on (1), or only of routes whose
 * device logits leave the order ambiguous (0, the default); returns the previous setting.
 * Both give the reference's picks.  A test hook with no counterpart in the reference (it
 * computes only the sequential logits). */
int   coli_hip_moe_cert_all(int on);
/* Host-routed expert groups (coli_vk_expert_group*) with more than one row per expert run
 * as grouped GEMMs on MFMA (0, the default) or, with force_gemv = 1, one GEMV item per
 * (expert, row) as for single rows; returns the previous setting.  A test and bench hook
 * with no counterpart in the reference (its multi-row switch is automatic). */
int   coli_hip_eg_force_gemv(int force_gemv);
/* coli_vk_gqa_full with S >= 4 rows runs them in one batched pass (1, the default: q/k/v
 * and o-projection GEMMs on MFMA, causal attention over all rows) or token by token through
 * the decode block (0); returns the previous setting.  A test and bench hook with no
 * counterpart in the reference. */
int   coli_hip_gqa_seq(int on);
/* coli_vk_gdn_full_seq's recurrence in closed form per 64-token chunk (1, the default) or
 * token by token (0); returns the previous setting.  A test and bench hook with no
 * counterpart in the reference. */
int   coli_hip_gdn_chunked(int on);

/* ---- fmt=6 container reader (c/st.h:120-456, c/qwen.c:509-536) ----
 * The safetensors shards c/tools/convert_qwen35_moe.py writes (U8 int4 nibbles plus an F32
 * ".qs" tensor of [scale, zero] pairs per group) read straight into device tensors.
 * coli_hip_st_open indexes every *.safetensors file of dir in name order and checks each
 * header as c/st.h:241-331 does (length within the file and under 512 MiB, a JSON object,
 * dtype / data_offsets / shape present and well-typed, offsets inside the file, no shape
 * overflow, element count equal to the byte span for F32/BF16/F16); a bad shard makes it
 * return NULL with a message, where the reference exits.  Host-only: open, count, find
 * and the two reads need no device. */
typedef struct ColiHipSt ColiHipSt;
ColiHipSt *coli_hip_st_open(const char *dir);
void  coli_hip_st_close(ColiHipSt *st);
int   coli_hip_st_count(const ColiHipSt *st);
/* dtype 0 BF16, 1 F16, 2 F32, 3 U8/I8; shape holds up to 8 sizes.  0 when absent. */
int   coli_hip_st_find(const ColiHipSt *st, const char *name, int *dtype, int64_t *numel, int64_t *nbytes,
                       int *ndim, int64_t *shape);
/* c/st.h:399-442: a float tensor as f32, at most cap elements; the count or -1. */
int64_t coli_hip_st_read_f32(const ColiHipSt *st, const char *name, float *out, int64_t cap);
/* c/st.h:445-452: raw bytes, at most cap; the count or -1. */
int64_t coli_hip_st_read_raw(const ColiHipSt *st, const char *name, void *out, int64_t cap);
/* In place of reading a tensor to host memory and calling coli_vk_tensor_ensure
 * (c/qwen.c:509-536, 1786-1789): fmt 6 reads name (U8 [O, ceil(I/2)]) and name.qs (F32
 * [O, 2 ceil(I/gs)]), fmt 0 an F32/BF16/F16 [O, I] tensor as f32 rows; *tensor must be
 * NULL.  1 on success. */
int   coli_hip_st_tensor(const ColiHipSt *st, const char *name, ColiVkTensor **tensor, int fmt, int I, int O,
                         int gs);
/* The E routed experts of model layer `layer` (converter names
 * model.layers.L.mlp.experts.E.{gate,up,down}_proj.weight[.qs], gate/up [I, D], down
 * [D, I]) into slots (layer, 0..E-1) of the resident expert table, which
 * coli_vk_eg_table_init must have sized; replaces c/qwen.c:1743-1805's per-expert
 * expert_read + three coli_vk_tensor_ensure calls.  Every tensor is checked before any
 * upload; batches are read by several threads (COLI_HIP_READ_THREADS, default the
 * hardware threads, at most 16) into pinned buffers while the device converts the previous
 * batch.  1 when every expert is resident. */
int   coli_hip_st_experts(const ColiHipSt *st, int layer, int E, int D, int I, int gs);

#ifdef __cplusplus
}
#endif
#endif
