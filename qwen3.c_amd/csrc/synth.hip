// synth.hip - device generator for the synthetic benchmark inputs.  It follows the
// same counter-based splitmix64 / Box-Muller spec as the host generator used by the
// tests, so a tensor generated here equals the host-generated buffers uploaded through
// coli_vk_tensor_ensure (checked by the GPU tests):
//   h(seed, i)      = mix64(seed + (i+1) * 0x9E3779B97F4A7C15)
//   stream(b, tag)  = mix64(b ^ mix64(tag + 1))
//   normal(seed, i) = sqrt(-2 ln u(2i)) cos(2 pi u(2i+1)),  u(j) = ((h(seed,j)>>11)+0.5) 2^-53
//   byte j          = bits [8(j&7), 8(j&7)+8) of h(seed, j>>3)
//   scale_g         = binary16-rounded |sigma * normal(seed, g)|, zero_g = h(seed^0x5A..5A, g) >> 60
#include "internal.h"

namespace coli {

__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t hash64(uint64_t seed, uint64_t i) {
    return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL);
}
static uint64_t stream_seed(uint64_t base, uint64_t tag) { return mix64(base ^ mix64(tag + 1)); }

__device__ inline double normal01(uint64_t seed, uint64_t i) {
    const double u1 = ((double)(hash64(seed, 2 * i) >> 11) + 0.5) * 0x1p-53;
    const double u2 = ((double)(hash64(seed, 2 * i + 1) >> 11) + 0.5) * 0x1p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

__device__ inline float f16_round(double v) {
    if (v == 0.0 || v != v) return (float)v;
    const double a = fabs(v);
    int e;
    (void)frexp(a, &e);
    int ulp = e - 11;
    if (ulp < -24) ulp = -24;
    double r = ldexp(rint(ldexp(a, -ulp)), ulp);
    if (r > 65504.0) r = INFINITY;
    return (float)(v < 0 ? -r : r);
}

// host-layout bytes [first, first + n) of the stream, written to dst[0, n)
__global__ void synth_bytes(uint8_t *dst, size_t first, size_t n, uint64_t seed) {
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (size_t)gridDim.x * blockDim.x) {
        const size_t j = first + k;
        dst[k] = (uint8_t)(hash64(seed, j >> 3) >> (8 * (j & 7)));
    }
}

__global__ void synth_sz(float *sz, size_t ngroups, uint64_t seed, double sigma) {
    const uint64_t zseed = seed ^ 0x5A5A5A5A5A5A5A5AULL;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < ngroups; g += (size_t)gridDim.x * blockDim.x) {
        sz[2 * g] = f16_round(fabs(sigma * normal01(seed, g)));
        sz[2 * g + 1] = (float)(hash64(zseed, g) >> 60);
    }
}

// f32 rows [rows, cols] with row stride dev_stride floats
__global__ void synth_normal_rows(float *dst, size_t rows, size_t cols, size_t dev_stride, uint64_t seed,
                                  double sigma) {
    const size_t n = rows * cols;
    for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (size_t)gridDim.x * blockDim.x) {
        const size_t r = j / cols, c = j - r * cols;
        dst[r * dev_stride + c] = (float)(sigma * normal01(seed, j));
    }
}

static int grid_1d(size_t n) {
    size_t b = (n + 255) / 256;
    const size_t cap = (size_t)n_cu() * 8;
    return (int)(b < 1 ? 1 : b > cap ? cap : b);
}

}  // namespace coli

using namespace coli;

COLI_API int coli_hip_tensor_synth(ColiVkTensor **tp, int fmt, int I, int O, int gs, uint64_t seed, double sigma) {
    if (!tp || *tp || !ok() || (fmt != 6 && fmt != 0)) return 0;
    ColiVkTensor *t = tensor_alloc(fmt, I, O, gs);
    if (!t) return 0;
    hipStream_t st = stream();
    if (fmt == 6) {
        const size_t hrb = tensor_host_row_bytes(t);
        void *stg = nullptr;
        size_t cap_rows = 0;
        if (!stage_buffer(&stg, &cap_rows, hrb)) {
            free(t);
            return 0;
        }
        for (int r0 = 0; r0 < O; r0 += (int)cap_rows) {
            const int rows = (int)((size_t)(O - r0) < cap_rows ? (size_t)(O - r0) : cap_rows);
            const size_t n = (size_t)rows * hrb;
            hipLaunchKernelGGL(synth_bytes, dim3(grid_1d(n)), dim3(256), 0, st, (uint8_t *)stg, (size_t)r0 * hrb, n,
                               stream_seed(seed, 1));
            if (!tensor_fill_rows(t, (const uint8_t *)stg, r0, rows, st)) {
                free(t);
                return 0;
            }
        }
        hipLaunchKernelGGL(synth_sz, dim3(grid_1d((size_t)O * t->ng)), dim3(256), 0, st, t->sz,
                           (size_t)O * t->ng, stream_seed(seed, 2), sigma);
    } else {
        (void)hipMemsetAsync(t->w, 0, (size_t)t->row_bytes * O, st);
        hipLaunchKernelGGL(synth_normal_rows, dim3(grid_1d((size_t)O * I)), dim3(256), 0, st, (float *)t->w,
                           (size_t)O, (size_t)I, (size_t)t->row_bytes / 4, stream_seed(seed, 3), sigma);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        free(t);
        return fail("tensor synth", e) ? 1 : 0;
    }
    tensor_register(t);
    *tp = t;
    return 1;
}

COLI_API int coli_hip_synth_normal(float *d_dst, size_t n, uint64_t seed, double sigma, void *stream_) {
    if (!ok() || !d_dst) return 0;
    hipStream_t st = stream_ ? (hipStream_t)stream_ : stream();
    hipLaunchKernelGGL(synth_normal_rows, dim3(grid_1d(n)), dim3(256), 0, st, d_dst, (size_t)1, n, n, seed, sigma);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("synth normal", e) ? 1 : 0;
    return 1;
}
