// unsupported.hip - drop-in ABI entry points this library does not implement.  Each
// returns the reference's "unavailable" answer (0 / no-op), which makes c/qwen.c keep
// the corresponding work on its CPU path (c/qwen.c:592,635,691,745 and the
// *_available() probes at :1704-1736).
//
// GLM MLA absorb attention and q-prep (c/backend_vulkan.h:114-141) are never called by
// c/qwen.c.  The attention / GatedDeltaNet layer blocks (c/backend_vulkan.h:151-198,
// 222-236, 258-279) are outside the int4 GEMV + MoE hot path this library accelerates.
#include "internal.h"

#define UNAVAILABLE return 0

COLI_API int coli_vk_kv_ensure(int, int, int, int) { UNAVAILABLE; }
COLI_API int coli_vk_kv_row(int, int, const float *, const float *) { UNAVAILABLE; }
COLI_API void coli_vk_kv_reset(void) {}
COLI_API int coli_vk_attention_absorb(ColiVkTensor **, const void *, const float *, int, int, float *,
                                      const float *, int, int, int, int, int, int, int, int, int, float) {
    UNAVAILABLE;
}
COLI_API int coli_vk_attn_qprep(int, ColiVkTensor **, const void *, const float *, int, ColiVkTensor **,
                                const void *, const float *, int, ColiVkTensor **, const void *,
                                const float *, int, int, int, const float *, float, const float *, int, int,
                                float *, float *, float *) {
    UNAVAILABLE;
}
COLI_API int coli_vk_attention_absorb_project(ColiVkTensor **, const void *, const float *, int, int,
                                              ColiVkTensor **, const void *, const float *, int, int, float *,
                                              const float *, int, int, int, int, int, int, int, int, int,
                                              float, int) {
    UNAVAILABLE;
}

COLI_API int coli_vk_gdn_available(void) { UNAVAILABLE; }
COLI_API int coli_vk_gdn_state_ensure(int, int, int, int) { UNAVAILABLE; }
COLI_API void coli_vk_gdn_reset(void) {}
COLI_API int coli_vk_gdn(int, const float *, const float *, const float *, const float *, const float *,
                         const float *, const float *, float *, int, int, int, int, float) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gqa_available(void) { UNAVAILABLE; }
COLI_API int coli_vk_gqa(int, const float *, float *, int, int, int, int, int, int, int, float) { UNAVAILABLE; }
COLI_API int coli_vk_gqa_project(int, const float *, ColiVkTensor *, float *, int, int, int, int, int, int, int,
                                 float, int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gqa_full_available(void) { UNAVAILABLE; }
COLI_API int coli_vk_gqa_norm_weight(int, const float *, const float *, int) { UNAVAILABLE; }
COLI_API int coli_vk_gqa_full(int, const float *, int, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *,
                              ColiVkTensor *, float *, int, int, int, int, int, int, int, float, float, int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_moe_route_available(void) { UNAVAILABLE; }
COLI_API int coli_vk_layer_norm_weight(int, const float *, const float *, int) { UNAVAILABLE; }
COLI_API int coli_vk_gqa_full_route(int, const float *, int, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *,
                                    ColiVkTensor *, ColiVkTensor *, int, float *, float *, float *, int, int, int,
                                    int, int, int, int, float, float, int, int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gdn_full_route(int, const float *, const float *, int, ColiVkTensor *, ColiVkTensor *,
                                    const float *, ColiVkTensor *, ColiVkTensor *, int, float *, float *, float *,
                                    int, int, int, int, int, int, float, int, int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gdn_ba_weight(int, const float *, const float *, const float *, int, int) { UNAVAILABLE; }
COLI_API int coli_vk_gqa_full_route_pipe(int, int, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *,
                                         ColiVkTensor *, int, int *, float *, int, int, int, int, int, int, int,
                                         float, float, int, int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gdn_full_route_pipe(int, int, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *, ColiVkTensor *,
                                         ColiVkTensor *, ColiVkTensor *, int, int *, float *, int, int, int, int,
                                         int, int, int, float, int, int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gdn_project(int, const float *, const float *, const float *, const float *, const float *,
                                 const float *, const float *, ColiVkTensor *, float *, int, int, int, int, float,
                                 int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gdn_full_available(void) { UNAVAILABLE; }
COLI_API int coli_vk_gdn_conv_ensure(int, int, int) { UNAVAILABLE; }
COLI_API int coli_vk_gdn_conv_weight(int, const float *, int, int) { UNAVAILABLE; }
COLI_API int coli_vk_gdn_full(int, const float *, int, ColiVkTensor *, ColiVkTensor *, const float *,
                              ColiVkTensor *, float *, int, int, int, int, int, int, float, int) {
    UNAVAILABLE;
}
COLI_API int coli_vk_gdn_full_seq(int, const float *, int, int, ColiVkTensor *, ColiVkTensor *, const float *,
                                  ColiVkTensor *, float *, int, int, int, int, int, int, float, int) {
    UNAVAILABLE;
}
