// unsupported.hip - drop-in ABI entry points this library does not implement.  Each
// returns the reference's "unavailable" answer (0), which makes a caller keep the work
// on its CPU path.
//
// GLM MLA absorb attention and q-prep (c/backend_vulkan.h:117-141) are never called by
// c/qwen.c.
#include "internal.h"

#define UNAVAILABLE return 0

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
