// internal.h - shared declarations of libcoli_hip (MI355X / gfx950 only).
//
// One process, one GPU, one host thread (the reference engine is single-threaded
// and keeps a global singleton too: c/backend_vulkan.c:69-278).  All device work is
// issued on one non-blocking HIP stream at default priority.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define COLI_API extern "C" __attribute__((visibility("default")))

// Opaque handle of the drop-in ABI (c/backend_vulkan.h:33).  Device layouts:
//   kLayoutRows  (fmt 0/1, and fmt 6 outside the fast path): row o of the host copy,
//                zero-padded to row_bytes (a 16-byte multiple).  fmt 6: U8 nibbles,
//                fmt 1: I8, fmt 0: F32.
//   kLayoutLanes (fmt 6 with gs % 32 == 0 and I <= kLaneMaxI): each row is cut into
//                16-byte chunks (32 nibbles); lane j of a row owns host chunks 2j, 2j+1,
//                and host chunk h = 2j + c is stored at chunk slot c * nl + j (nl = lanes
//                with data = ceil(nchunks / 2)), so one load instruction per c reads nl
//                consecutive 16-byte chunks.  Every byte is stored XOR 0x88, which turns
//                the unsigned nibble n into the signed nibble n - 8 for v_dot8_i32_i4.
//                Bytes past the host row read as 0 (stored as 0x88).
//   sz: fmt 6 f32 [O, ng, 2] verbatim, fmt 1 f32 [O], fmt 0 none.
enum { kLayoutRows = 0, kLayoutLanes = 1 };
struct ColiVkTensor {
    int fmt, I, O, gs, ng;
    int layout;
    int nchunks;       // 16-byte host chunks per row: ceil(host row bytes / 16)
    int nl;            // kLayoutLanes: lanes with data per row
    int row_bytes;     // device row stride
    uint8_t *w;        // device weights
    float *sz;         // device scales (+zeros)
    size_t bytes;      // device bytes held (weights + scales)
    size_t wbytes;     // device weight bytes (row_bytes * O), what coli_vk_tensor_bytes reports
    unsigned gen;      // runtime generation that allocated it (a shutdown invalidates the handle)
};

namespace coli {

struct Runtime;
extern Runtime G;

// sticky failure: print and disable the device for the rest of the process
bool fail(const char *what, hipError_t e);
bool ok();                               // device usable (init done, no sticky failure)
hipStream_t stream();
int n_cu();

// device memory
void *arena_alloc(size_t bytes);          // weights: 256-byte aligned slices, never freed
bool scratch(void **p, size_t *cap, size_t need);   // grow-only device scratch
bool host_scratch(void **p, size_t *cap, size_t need);  // grow-only pinned host scratch
bool sync_stream(const char *who);

// device -> pageable host read-back through pinned staging, copied out piece by piece as
// the pieces arrive (runtime.hip); read_back synchronises with every piece on `st`.
bool read_back(void *dst, const void *dsrc, size_t n, hipStream_t st, const char *who);
// Host buffers to device memory on `st` through pinned staging in pieces (runtime.hip); the
// host buffers may be reused on return.
struct Upload {
    void *d;
    const void *h;
    size_t n;
};
bool upload(const Upload *u, int nu, hipStream_t st, const char *who);
// a tensor handle is about to be freed: the decode stream drops what it kept of it (layer.hip)
void stream_tensor_freed(const ColiVkTensor *t);
// n bytes between device memory and pinned host memory (host_scratch) as a copy kernel on
// `st`: the launch returns at once (runtime.hip)
bool pin_copy(void *dst, const void *src, size_t n, hipStream_t st, const char *who);
// The pieces of a read-back already issued into pinned memory: record one event per piece
// after issuing it, then copy_out waits for each in turn and copies it out.
struct PieceEvents {
    static constexpr int kMax = 8;
    hipEvent_t ev[kMax] = {};
    size_t piece = 0, n = 0;
    int count = 0;
};
bool issue_pieces(PieceEvents &pe, void *hdst, const void *dsrc, size_t n, hipStream_t st);
bool copy_out(PieceEvents &pe, void *dst, const void *hsrc, const char *who);
void piece_events_free(PieceEvents &pe);
void read_back_shutdown();

// tensors
bool tensor_live(const ColiVkTensor *t);  // non-NULL and allocated since the last shutdown
constexpr int kLaneMaxI = 4096;          // fmt 6 lanes layout / fast GEMV path: nl <= 64
constexpr int kLaneChunks = 2;           // 16-byte chunks owned by one lane of a row
ColiVkTensor *tensor_alloc(int fmt, int I, int O, int gs);   // not yet filled or counted
size_t tensor_host_row_bytes(const ColiVkTensor *t);
void tensor_register(ColiVkTensor *t);                       // count it in mem_info
// Fill t->w from `rows` host-layout rows [r0, r0+rows) already in device memory
// (d_src, stride tensor_host_row_bytes), converting to t's device layout.
bool tensor_fill_rows(ColiVkTensor *t, const uint8_t *d_src, int r0, int rows, hipStream_t st);
// Shared device staging buffer for host-layout rows: *cap_rows rows of host_rb bytes.
bool stage_buffer(void **p, size_t *cap_rows, size_t host_rb);

// GEMV launchers on device pointers (stream-ordered, no sync)
struct TopkOut {       // fused top-k over the GEMV outputs (rows of one launch)
    int k;             // 1..8 (0 = none)
    int *idx;          // device [k]
    float *val;        // device [k]
};
bool gemv(const ColiVkTensor *t, const float *d_x, float *d_y, int S, hipStream_t st,
          const TopkOut *tk = nullptr);
// k best (value desc, index asc) of d_v[0, n), k <= 8
bool topk(const float *d_v, int n, int k, int *d_idx, float *d_val, hipStream_t st);
bool rmsnorm_zc(const float *d_x, const float *d_w, float *d_y, int D, float eps, hipStream_t st);
// GEMV (fmt 6 lanes layout, O < 2^24) whose blocks fold their best row into kArgSlots
// tagged keys (*slots, the launch tag in *epoch); with xw, x is first normed (zero-centred
// RMSNorm, weight xw) in the kernel's x prologue.  The kArgSpare words after the keys are
// the caller's (read back with them).  argmax_decode_host: the keys -> (idx, val), false
// when no key of the launch is there.
constexpr int kArgSlots = 16, kArgSpare = 8;
bool gemv_argmax(const ColiVkTensor *t, const float *d_x, float *d_y, hipStream_t st, uint32_t *epoch,
                 unsigned long long **slots, const float *xw = nullptr, float eps = 0.f);
bool argmax_decode_host(const unsigned long long *keys, uint32_t epoch, int *idx, float *val);

// Dense GEMM on MFMA over S rows of x (prefill.hip): d_y[i] [S][O_i] = x . t[i]^T for nt
// fmt6 tensors of group size 128 sharing I (one digit decomposition of x serves all).  gx:
// x is the GatedDeltaNet recurrence output and goes through its gated output norm first.
constexpr int kGemmMaxI = kLaneMaxI;
constexpr int kGemmMinS = 4;            // fewer rows of x: one GEMV launch per row
struct GatedX {
    const float *z;        // [S][I] z projection rows
    const float *gnorm;    // norm weight [VD] of row s at gnorm + s * gstride
    int gstride, VD;
    float eps;
};
bool gemm6_ok(const ColiVkTensor *t);
// fmt 0 / fmt 1 rows over S >= 2 rows of x in one launch, the reference's sequential fp32
// sums bit for bit (d_x 16-byte aligned)
bool gemm_f01_ok(const ColiVkTensor *t, const float *d_x);
bool gemm_f01(const ColiVkTensor *t, const float *d_x, float *d_y, int S, hipStream_t st);
bool gemm6(const ColiVkTensor *const *t, float *const *d_y, int nt, const float *d_x, int S, hipStream_t st,
           const GatedX *gx = nullptr);

// the layer's MoE block in one launch (moe.hip): out (+)= sum_k val_k y_k + shgt y_sh.
// d_xw != NULL: d_x is the residual and the block applies the post-attention RMSNorm
// (weight d_xw, eps) itself.
bool moe_decode(int layer, const ColiVkTensor *router, int K, const float *d_x, float *d_out, int accumulate,
                int *d_idx, float *d_val, hipStream_t st, const float *d_xw = nullptr, float eps = 0.f);
// expert table complete for the layer
bool moe_ready(int layer);

// MoE error word of the decode launches: 0 none, 1 a bounded wait gave up, 2 a route held
// an out-of-range expert id.  moe_error_take reads and clears it (synchronises the device);
// -1 on a runtime error.
int moe_error_take();
// The MoE error words of the current device (NULL where absent), the decision on values read
// from them once the launches finished (moe_error_take's, without its synchronisation and
// reads), and the count of launches that can set them.
void moe_error_words(const unsigned long long **w0, const unsigned long long **w1);
int moe_error_settle(const unsigned long long v[2]);
uint64_t moe_launches();
// Device address of the no-alloc MoE scratch array, looked up once per device with that
// device current (coli_vk_init).  false: the no-alloc entry point refuses on that device.
bool moe_noalloc_init(int dev);

// Teardown of each source file's state at coli_vk_shutdown: scratch buffers are freed and
// every device pointer into the weight arena is forgotten, so calls after a shutdown
// refuse instead of running kernels on freed memory.
void gemv_shutdown();
void moe_shutdown();
void prefill_shutdown();
void layer_shutdown();
void container_shutdown();
void scratch_free(void **p, size_t *cap);
void host_scratch_free(void **p, size_t *cap);

// device residual stream (layer.hip): the residual row of a live stream of width D, and
// the last non-fused route's normed row (the expert input); NULL when not available
float *stream_resid(int D);
const float *stream_nrm_dev(int D);

}  // namespace coli
