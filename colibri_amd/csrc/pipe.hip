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

// Experts per wave of the staged router partials at 5-16 rows: two, so each
// activation read from LDS feeds two products and a workgroup stages the rows'
// chunk for eight experts (DSV3 B16 layer 416.8 -> 413.7 us, 21-row step
// 535.5 -> 528.1 us; four: 415.2 / 530.8 us). COLI_ROUTER_EPW16 overrides it
// at build time (tuning).
#ifndef COLI_ROUTER_EPW16
#define COLI_ROUTER_EPW16 2
#endif
#define COLI_ROUTER_EPW(SMAX) ((SMAX) >= 16 ? COLI_ROUTER_EPW16 : 1)

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
            constexpr int EPW = COLI_ROUTER_EPW(SMAX);
            router_partial_block<SMAX, false, EPW>(x, S, W, D, E, part, chstride, (blockIdx.x * 4 + wave) * EPW,
                                                   blockIdx.y, lane, xs);
            return;
        }
    }
    router_partial_wave<SMAX, false>(x, S, W, D, E, part, chstride, blockIdx.x * 4 + wave, blockIdx.y, lane);
}

extern "C" int coli_router_chunks(int D) { return (D + COLI_ROUTER_CHUNK - 1) / COLI_ROUTER_CHUNK; }

// Router logits of many rows (prefill): part[ch][s][e] = sum over the chunk's
// columns of x[s, d] * W[e, d], an f32 GEMM on v_mfma_f32_16x16x4_f32. A
// 256-thread workgroup computes a 64-row x 64-expert tile over one 512-column
// chunk (the same chunk partials the selection adds in chunk order); each wave
// owns a 32 x 32 quarter (2 x 2 MFMA blocks). Steps of 32 columns are staged
// in LDS with a row pitch of 33 floats, so the sixteen rows one MFMA operand
// read touches sit in sixteen different banks.
#define COLI_RG_BM 64
#define COLI_RG_BK 32
__global__ __launch_bounds__(256) void coli_router_gemm(const float *__restrict__ x, int S,
                                                        const float *__restrict__ W, int D, int E,
                                                        float *__restrict__ part) {
    __shared__ float xs[COLI_RG_BM][COLI_RG_BK + 1], ws[COLI_RG_BM][COLI_RG_BK + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s0 = blockIdx.x * COLI_RG_BM, e0 = blockIdx.y * COLI_RG_BM, ch = blockIdx.z;
    const int d_begin = ch * COLI_ROUTER_CHUNK, d_end = min(D, d_begin + COLI_ROUTER_CHUNK);
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;   // the wave's quarter
    floatx4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) acc[a][b] = (floatx4){0.f, 0.f, 0.f, 0.f};
    const bool vec = (D & 3) == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)W & 15) == 0;
    // 64 rows x COLI_RG_BK columns of x and of W per step: thread t loads
    // float4 t, t + 256, ... of each, one step ahead of the MFMAs (the loads
    // of the next step are in flight while this one is computed)
    constexpr int NH = COLI_RG_BK / 16, CPR = COLI_RG_BK / 4;   // float4 per thread; per row
    float4 xr[NH], wr4[NH];
    auto load = [&](int d0) {
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const int f = threadIdx.x + 256 * h, r = f / CPR, c = (f % CPR) * 4;
            const int d = d0 + c;
            float4 xv = make_float4(0.f, 0.f, 0.f, 0.f), wv = xv;
            if (vec && d + 4 <= d_end) {
                if (s0 + r < S) xv = *(const float4 *)(x + (size_t)(s0 + r) * D + d);
                if (e0 + r < E) wv = *(const float4 *)(W + (size_t)(e0 + r) * D + d);
            } else {
                float xa[4] = {0.f, 0.f, 0.f, 0.f}, wa[4] = {0.f, 0.f, 0.f, 0.f};
                for (int u = 0; u < 4; u++) {
                    if (d + u < d_end) {
                        if (s0 + r < S) xa[u] = x[(size_t)(s0 + r) * D + d + u];
                        if (e0 + r < E) wa[u] = W[(size_t)(e0 + r) * D + d + u];
                    }
                }
                xv = make_float4(xa[0], xa[1], xa[2], xa[3]);
                wv = make_float4(wa[0], wa[1], wa[2], wa[3]);
            }
            xr[h] = xv;
            wr4[h] = wv;
        }
    };
    load(d_begin);
    for (int d0 = d_begin; d0 < d_end; d0 += COLI_RG_BK) {
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const int f = threadIdx.x + 256 * h, r = f / CPR, c = (f % CPR) * 4;
            xs[r][c] = xr[h].x; xs[r][c + 1] = xr[h].y; xs[r][c + 2] = xr[h].z; xs[r][c + 3] = xr[h].w;
            ws[r][c] = wr4[h].x; ws[r][c + 1] = wr4[h].y; ws[r][c + 2] = wr4[h].z; ws[r][c + 3] = wr4[h].w;
        }
        __syncthreads();
        if (d0 + COLI_RG_BK < d_end) load(d0 + COLI_RG_BK);
        // A lane (m = lane % 16, k = lane / 16) of each 16 x 16 x 4 step; B likewise
#pragma unroll
        for (int k0 = 0; k0 < COLI_RG_BK; k0 += 4) {
            const int k = k0 + (lane >> 4);
            float av[2], bv[2];
#pragma unroll
            for (int a = 0; a < 2; a++) av[a] = xs[wr + 16 * a + (lane & 15)][k];
#pragma unroll
            for (int b = 0; b < 2; b++) bv[b] = ws[wc + 16 * b + (lane & 15)][k];
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    // lane holds C[4 (lane / 16) + i][lane % 16] of each 16 x 16 block
    float *dst = part + (size_t)ch * S * E;
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int s = s0 + wr + 16 * a + 4 * (lane >> 4) + i, e = e0 + wc + 16 * b + (lane & 15);
                if (s < S && e < E) dst[(size_t)s * E + e] = acc[a][b][i];
            }
}

extern "C" hipError_t coli_launch_router_gemm(const float *x, int S, const float *W, int D, int E, float *part,
                                              hipStream_t st) {
    const dim3 grid((S + COLI_RG_BM - 1) / COLI_RG_BM, (E + COLI_RG_BM - 1) / COLI_RG_BM,
                    (D + COLI_ROUTER_CHUNK - 1) / COLI_ROUTER_CHUNK);
    hipLaunchKernelGGL(coli_router_gemm, grid, dim3(256), 0, st, x, S, W, D, E, part);
    return hipGetLastError();
}



// part: [coli_router_chunks(D)][S][E] f32 partial logits.
extern "C" hipError_t coli_launch_router_logits(const float *x, int S, const float *W, int D, int E,
                                                float *part, hipStream_t st) {
    const int nch = coli_router_chunks(D);
    const size_t chstride = (size_t)S * E;
    const bool vec = (D & 3) == 0;   // the staged form (several experts a wave) needs aligned rows
    for (int s0 = 0; s0 < S; s0 += 16) {   // 16 rows of accumulators per pass
        const int n = S - s0 < 16 ? S - s0 : 16;
        const float *xs = x + (size_t)s0 * D;
        float *ps = part + (size_t)s0 * E;
        const int epw = n == 1 || !vec ? 1 : (n <= 4 ? COLI_ROUTER_EPW(4) : COLI_ROUTER_EPW(16));
        const dim3 grid((E + 4 * epw - 1) / (4 * epw), nch);
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

// Plain streaming read of n16 16-byte words (benchmark reference: what one
// launch of a given size can read, with no arithmetic and no dependency):
// consecutive lanes read consecutive words, four independent loads per
// thread in flight; the values only feed an opaque use, so nothing is written.
__global__ __launch_bounds__(256) void coli_stream_read(const uint8_t *__restrict__ p, size_t n16) {
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nt = (size_t)gridDim.x * blockDim.x;
    u32x4 acc = (u32x4){0u, 0u, 0u, 0u};
    for (size_t i = tid; i < n16; i += 4 * nt) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t w = i + u * nt;
            v[u] = w < n16 ? __builtin_nontemporal_load(GPTR(u32x4, p) + w) : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u];
    }
    asm volatile("" ::"v"(acc[0]), "v"(acc[1]), "v"(acc[2]), "v"(acc[3]));
}

extern "C" hipError_t coli_launch_stream_read(const void *dev, size_t bytes, hipStream_t st) {
    if (((uintptr_t)dev & 15) != 0 || bytes % 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(coli_stream_read, dim3(2048), dim3(256), 0, st, (const uint8_t *)dev, bytes / 16);
    return hipGetLastError();
}
