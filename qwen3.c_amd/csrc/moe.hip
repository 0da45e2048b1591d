// moe.hip - expert group, device-indexed MoE and residual stream entry points.
// (first cut: unavailable; filled in by the MoE kernels)
#include "internal.h"

COLI_API int coli_vk_gate_up(ColiVkTensor **, ColiVkTensor **, float *, const float *, const void *,
                             const float *, const void *, const float *, int, int, int, int, int) { return 0; }
COLI_API int coli_vk_expert_group(ColiVkTensor *const *, ColiVkTensor *const *, ColiVkTensor *const *,
                                  const int *, int, float *, const float *) { return 0; }
COLI_API int coli_vk_expert_group_issue(ColiVkTensor *const *, ColiVkTensor *const *, ColiVkTensor *const *,
                                        const int *, int, const float *) { return 0; }
COLI_API int coli_vk_expert_group_take(float *) { return 0; }
COLI_API int coli_vk_eg_gather_available(void) { return 0; }
COLI_API int coli_vk_eg_xs_bind(const float *, int, int) { return 0; }
COLI_API int coli_vk_expert_group_issue_id(ColiVkTensor *const *, ColiVkTensor *const *, ColiVkTensor *const *,
                                           const int *, int, const int *) { return 0; }
COLI_API int coli_vk_stream_available(void) { return 0; }
COLI_API int coli_vk_stream_begin(const float *, int) { return 0; }
COLI_API int coli_vk_stream_end(float *, int) { return 0; }
COLI_API int coli_vk_stream_add(const float *, int) { return 0; }
COLI_API const float *coli_vk_stream_nrm(void) { return nullptr; }
COLI_API int coli_vk_final_norm_weight(const float *, int) { return 0; }
COLI_API int coli_vk_stream_norm_argmax(ColiVkTensor **, const void *, const float *, int, int, int, int, float,
                                        int *, float *) { return 0; }
COLI_API int coli_vk_stream_copy_resid(float *, int) { return 0; }
COLI_API void coli_vk_route_cache_stats(void) {}
COLI_API void coli_vk_decode_prof(double, int) {}
COLI_API int coli_vk_expert_group_issue_pipe(ColiVkTensor *const *, ColiVkTensor *const *, ColiVkTensor *const *,
                                             const int *, const float *, int, int) { return 0; }
COLI_API int coli_vk_expert_group_take_pipe(void) { return 0; }
COLI_API int coli_vk_moe_ix_available(void) { return 0; }
COLI_API int coli_vk_eg_table_init(int, int, int, int, int) { return 0; }
COLI_API int coli_vk_eg_table_set(int, int, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *) { return 0; }
COLI_API int coli_vk_eg_table_set_shared(int, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *, const float *, int) {
    return 0;
}
COLI_API int coli_vk_stream_moe_fused(void) { return 0; }
COLI_API int coli_vk_stream_ix_pending(void) { return 0; }
COLI_API int coli_vk_stream_ix_hist(int, int *, int) { return 0; }
