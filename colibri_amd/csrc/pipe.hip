// pipe.hip -- small elementwise / reduction kernels of the expert path and the
// routing kernels (router GEMV, top-k selection, expert union).
//
// Every reduction here runs in a fixed order (no float atomics), so repeated
// calls are bitwise reproducible, as the reference's device path is
// (c/backend_cuda.cu:2070-2078, 2216-2245).
#include "coli_hip_internal.h"

#include <math.h>

__global__ void coli_zero_i32(int *p, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// h = silu(g) * u, the expression of c/backend_cuda.cu:417-423.
__global__ void coli_silu_mul(float *gate, const float *up, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = gate[i];
        gate[i] = (v / (1.0f + expf(-v))) * up[i];
    }
}

__global__ void coli_silu_mul_to(float *h, const float *gate, const float *up, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = gate[i];
        h[i] = (v / (1.0f + expf(-v))) * up[i];
    }
}

__global__ void coli_add_n(float *x, const float *t, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += t[i];
}

// x[rows[b]] += partial[b] (rows unique by contract, c/backend_cuda.cu:2070-2078).
__global__ void coli_rows_add(float *x, const float *partial, const int *rows, int D) {
    float *xr = x + (size_t)rows[blockIdx.x] * D;
    const float *pr = partial + (size_t)blockIdx.x * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) xr[i] += pr[i];
}

// out[d] = sum_c w[c] * y[c, d], experts in fixed order (c/backend_cuda.cu:2231-2238).
__global__ void coli_weighted_sum_rows(float *out, const float *y, const float *w, int count, int D) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < D; i += gridDim.x * blockDim.x) {
        float acc = 0.0f;
        for (int c = 0; c < count; c++) acc += w[c] * y[(size_t)c * D + i];
        out[i] = acc;
    }
}

// dst[d] = sum_s slots[s, d] in issue order (c/backend_cuda.cu:2239-2245).
__global__ void coli_sum_slots(float *dst, const float *slots, int n, int D) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < D; i += gridDim.x * blockDim.x) {
        float acc = 0.0f;
        for (int s = 0; s < n; s++) acc += slots[(size_t)s * D + i];
        dst[i] = acc;
    }
}

#include "coli_route.h"

template <int SMAX>
__global__ __launch_bounds__(256) void coli_router_partial(const float *__restrict__ x, int S,
                                                           const float *__restrict__ W, int D, int E,
                                                           float *__restrict__ part, size_t chstride) {
    // readfirstlane: the wave index is wave-uniform, so everything derived from it
    // (tile indices, validity, base pointers) stays in scalar registers.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if constexpr (SMAX > 1) {
        if ((D & 3) == 0) {
            __shared__ floatx4 xs[SMAX][COLI_ROUTER_CHUNK / 4];
            router_partial_block<SMAX, false>(x, S, W, D, E, part, chstride, blockIdx.x * 4 + wave, blockIdx.y, lane,
                                              xs);
            return;
        }
    }
    router_partial_wave<SMAX, false>(x, S, W, D, E, part, chstride, blockIdx.x * 4 + wave, blockIdx.y, lane);
}

extern "C" int coli_router_chunks(int D) { return (D + COLI_ROUTER_CHUNK - 1) / COLI_ROUTER_CHUNK; }

// part: [coli_router_chunks(D)][S][E] f32 partial logits.
extern "C" hipError_t coli_launch_router_logits(const float *x, int S, const float *W, int D, int E,
                                                float *part, hipStream_t st) {
    const int nch = coli_router_chunks(D);
    const size_t chstride = (size_t)S * E;
    const dim3 grid((E + 3) / 4, nch);
    for (int s0 = 0; s0 < S; s0 += 16) {   // 16 rows of accumulators per pass
        const int n = S - s0 < 16 ? S - s0 : 16;
        const float *xs = x + (size_t)s0 * D;
        float *ps = part + (size_t)s0 * E;
        if (n == 1)
            hipLaunchKernelGGL((coli_router_partial<1>), grid, dim3(256), 0, st, xs, n, W, D, E, ps, chstride);
        else if (n <= 4)
            hipLaunchKernelGGL((coli_router_partial<4>), grid, dim3(256), 0, st, xs, n, W, D, E, ps, chstride);
        else
            hipLaunchKernelGGL((coli_router_partial<16>), grid, dim3(256), 0, st, xs, n, W, D, E, ps, chstride);
    }
    return hipGetLastError();
}

template <int JM>
__global__ __launch_bounds__(256) void coli_router_select(const float *__restrict__ part, int nch,
                                                          const float *__restrict__ bias, int S, int E, int K,
                                                          int mode, float topp, int norm_topk,
                                                          float routed_scale, int *__restrict__ idx,
                                                          float *__restrict__ wout, int *__restrict__ keff) {
    extern __shared__ float sh[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    select_row<JM, false>(part, nch, bias, S, E, K, mode, topp, norm_topk, routed_scale, idx, wout, keff,
                          sh + (size_t)wave * E, blockIdx.x * 4 + wave, lane, nullptr, nullptr);
}

extern "C" hipError_t coli_launch_router_select(const float *part, int nch, const float *bias, int S, int E,
                                                int K, int mode, float topp, int norm_topk,
                                                float routed_scale, int *idx, float *w, int *keff,
                                                hipStream_t st) {
    size_t shm = (size_t)4 * E * sizeof(float);
    // experts per lane, rounded up to a power of two (E <= 1024)
    const int jm = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
#define COLI_SEL_LAUNCH(JM)                                                                                       \
    hipLaunchKernelGGL(coli_router_select<JM>, dim3((S + 3) / 4), dim3(256), shm, st, part, nch, bias, S, E, K, mode, \
                       topp, norm_topk, routed_scale, idx, w, keff)
    switch (jm) {
    case 1: COLI_SEL_LAUNCH(1); break;
    case 2: COLI_SEL_LAUNCH(2); break;
    case 4: COLI_SEL_LAUNCH(4); break;
    case 8: COLI_SEL_LAUNCH(8); break;
    default: COLI_SEL_LAUNCH(16); break;
    }
#undef COLI_SEL_LAUNCH
    return hipGetLastError();
}

extern "C" hipError_t coli_launch_zero_i32(int *p, int n, hipStream_t st) {
    hipLaunchKernelGGL(coli_zero_i32, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
    return hipGetLastError();
}
extern "C" hipError_t coli_launch_silu_mul(float *gate, const float *up, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(coli_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gate, up, n);
    return hipGetLastError();
}
extern "C" hipError_t coli_launch_silu_mul_to(float *h, const float *gate, const float *up, size_t n,
                                              hipStream_t st) {
    hipLaunchKernelGGL(coli_silu_mul_to, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, h, gate, up, n);
    return hipGetLastError();
}
// Copy n floats between buffers either side of PCIe (pinned host memory seen
// through its device pointer): one launch instead of a DMA-engine copy.
__global__ __launch_bounds__(256) void coli_copy_f32(float *__restrict__ dst, const float *__restrict__ src,
                                                     size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (4 * i + 3 < n) {
        *(floatx4 *)(dst + 4 * i) = *(const floatx4 *)(src + 4 * i);
    } else {
        for (size_t k = 4 * i; k < n; k++) dst[k] = src[k];
    }
}
extern "C" hipError_t coli_launch_copy_f32(float *dst, const float *src, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    if ((uintptr_t)dst % 16 || (uintptr_t)src % 16) return hipErrorInvalidValue;
    const size_t n4 = (n + 3) / 4;
    hipLaunchKernelGGL(coli_copy_f32, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, dst, src, n);
    return hipGetLastError();
}
extern "C" hipError_t coli_launch_add_n(float *x, const float *t, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(coli_add_n, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, t, n);
    return hipGetLastError();
}
extern "C" hipError_t coli_launch_rows_add(float *x, const float *partial, const int *rows, int nrows,
                                           int D, hipStream_t st) {
    hipLaunchKernelGGL(coli_rows_add, dim3(nrows), dim3(256), 0, st, x, partial, rows, D);
    return hipGetLastError();
}
extern "C" hipError_t coli_launch_weighted_sum_rows(float *out, const float *y, const float *w, int count,
                                                    int D, hipStream_t st) {
    hipLaunchKernelGGL(coli_weighted_sum_rows, dim3(48), dim3(256), 0, st, out, y, w, count, D);
    return hipGetLastError();
}
extern "C" hipError_t coli_launch_sum_slots(float *dst, const float *slots, int n, int D, hipStream_t st) {
    hipLaunchKernelGGL(coli_sum_slots, dim3(48), dim3(256), 0, st, dst, slots, n, D);
    return hipGetLastError();
}

// Uniform pseudo-random bytes: splitmix64 of (seed, 8-byte word index).
__global__ void coli_fill_random(uint8_t *dst, size_t n, unsigned long long seed) {
    size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; w * 8 < n; w += stride) {
        unsigned long long z = seed + 0x9E3779B97F4A7C15ull * (w + 1);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        size_t base = w * 8;
        if (base + 8 <= n) {
            *(unsigned long long *)(dst + base) = z;   // n-aligned callers: 8-byte stores
        } else {
            for (int b = 0; base + b < n; b++) dst[base + b] = (uint8_t)(z >> (8 * b));
        }
    }
}

extern "C" hipError_t coli_launch_fill_random(void *dev, size_t n, unsigned long long seed, hipStream_t st) {
    if (((uintptr_t)dev & 7) != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(coli_fill_random, dim3(4096), dim3(256), 0, st, (uint8_t *)dev, n, seed);
    return hipGetLastError();
}
