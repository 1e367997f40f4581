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

// ---------------------------------------------------------------------------
// Router logits: logits[s, e] = sum_d x[s, d] * W[e, d], f32 (the router GEMV
// of c/colibri.c:3978 / c/olmoe.c:648). One block per expert row; each thread
// walks D with float4 loads and keeps S <= 16 accumulators; a fixed-order tree
// reduction finishes each row.
// ---------------------------------------------------------------------------
template <int SMAX>
__global__ __launch_bounds__(256) void coli_router_logits(const float *__restrict__ x, int S,
                                                          const float *__restrict__ W, int D, int E,
                                                          float *__restrict__ logits) {
    int e = blockIdx.x;
    const float *w = W + (size_t)e * D;
    float acc[SMAX];
#pragma unroll
    for (int s = 0; s < SMAX; s++) acc[s] = 0.0f;
    if ((D & 3) == 0) {
        for (int d = threadIdx.x * 4; d < D; d += 1024) {
            float4 wv = *(const float4 *)(w + d);
#pragma unroll
            for (int s = 0; s < SMAX; s++) {
                if (s < S) {
                    float4 xv = *(const float4 *)(x + (size_t)s * D + d);
                    acc[s] = fmaf(xv.x, wv.x, acc[s]);
                    acc[s] = fmaf(xv.y, wv.y, acc[s]);
                    acc[s] = fmaf(xv.z, wv.z, acc[s]);
                    acc[s] = fmaf(xv.w, wv.w, acc[s]);
                }
            }
        }
    } else {
        for (int d = threadIdx.x; d < D; d += 256) {
            float wv = w[d];
#pragma unroll
            for (int s = 0; s < SMAX; s++)
                if (s < S) acc[s] = fmaf(x[(size_t)s * D + d], wv, acc[s]);
        }
    }
    __shared__ float red[SMAX][256];
#pragma unroll
    for (int s = 0; s < SMAX; s++) red[s][threadIdx.x] = acc[s];
    __syncthreads();
    for (int st = 128; st; st >>= 1) {
        if (threadIdx.x < st)
#pragma unroll
            for (int s = 0; s < SMAX; s++) red[s][threadIdx.x] += red[s][threadIdx.x + st];
        __syncthreads();
    }
    if (threadIdx.x < S && threadIdx.x < SMAX) logits[(size_t)threadIdx.x * E + e] = red[threadIdx.x][0];
}

extern "C" hipError_t coli_launch_router_logits(const float *x, int S, const float *W, int D, int E,
                                                float *logits, hipStream_t st) {
    for (int s0 = 0; s0 < S; s0 += 16) {   // 16 rows of accumulators per pass
        int n = S - s0 < 16 ? S - s0 : 16;
        const float *xs = x + (size_t)s0 * D;
        float *ls = logits + (size_t)s0 * E;
        if (n <= 4) hipLaunchKernelGGL(coli_router_logits<4>, dim3(E), dim3(256), 0, st, xs, n, W, D, E, ls);
        else hipLaunchKernelGGL(coli_router_logits<16>, dim3(E), dim3(256), 0, st, xs, n, W, D, E, ls);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Top-K selection, one block per token row (E <= 4096, K <= 64).
//   mode 0: p = softmax(z) (max-subtracted, c/olmoe.c:246-250), select on p,
//           weight p, optional norm over K without epsilon (c/olmoe.c:681).
//   mode 1: p = sigmoid(z), choice = p + bias, select on choice, weight p,
//           TOPP (sort by weight, tot = 1e-20 + sum, keep until cum >=
//           topp * tot), norm_topk (sum + 1e-20), x routed_scale
//           (c/backend_cuda.cu:2169-2194, c/colibri.c:3982-4126).
//   mode 2: as mode 1 for the selection; weights renormalized over the K
//           with +1e-20; TOPP keeps until cum >= topp and renormalizes the
//           kept set (c/kimi_k3.c:1337-1370); routed_scale applied after.
// Selection is K rounds of an argmax with strict '>' semantics (highest
// value, lowest index on ties, NaN never selected); an all-NaN round falls
// back to index kk (c/route_trace.h:383-393).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    // v is better than (bv, bi): larger value, or equal value and lower index.
    if (bi < 0) return !(v != v) && v > -1e30f;
    if (v != v) return false;
    return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(256) void coli_router_select(const float *__restrict__ logits,
                                                          const float *__restrict__ bias, int E, int K,
                                                          int mode, float topp, int norm_topk,
                                                          float routed_scale, int *__restrict__ idx,
                                                          float *__restrict__ wout, int *__restrict__ keff) {
    extern __shared__ float sh[];
    float *p = sh;          // [E] weight source
    float *c = sh + E;      // [E] selection score
    __shared__ float rv[256];
    __shared__ int ri[256];
    __shared__ int sel[64];
    __shared__ float selw[64];
    __shared__ float smax, ssum;
    const int s = blockIdx.x;
    const float *z = logits + (size_t)s * E;
    const int tid = threadIdx.x;

    if (mode == 0) {
        float m = -1e30f;
        for (int e = tid; e < E; e += 256) m = fmaxf(m, z[e] > m ? z[e] : m);
        rv[tid] = m;
        __syncthreads();
        for (int st = 128; st; st >>= 1) {
            if (tid < st) rv[tid] = fmaxf(rv[tid], rv[tid + st]);
            __syncthreads();
        }
        if (tid == 0) smax = rv[0];
        __syncthreads();
        float part = 0.0f;
        for (int e = tid; e < E; e += 256) {
            float v = expf(z[e] - smax);
            p[e] = v;
            part += v;
        }
        rv[tid] = part;
        __syncthreads();
        for (int st = 128; st; st >>= 1) {
            if (tid < st) rv[tid] += rv[tid + st];
            __syncthreads();
        }
        if (tid == 0) ssum = rv[0];
        __syncthreads();
        for (int e = tid; e < E; e += 256) {
            p[e] = p[e] / ssum;
            c[e] = p[e];
        }
    } else {
        for (int e = tid; e < E; e += 256) {
            float v = 1.0f / (1.0f + expf(-z[e]));
            p[e] = v;
            c[e] = v + (bias ? bias[e] : 0.0f);
        }
    }
    __syncthreads();

    for (int kk = 0; kk < K; kk++) {
        float bv = 0.0f;
        int bi = -1;
        for (int e = tid; e < E; e += 256) {
            bool taken = false;
            for (int j = 0; j < kk; j++) taken |= (sel[j] == e);
            if (!taken && better(c[e], e, bv, bi)) { bv = c[e]; bi = e; }
        }
        rv[tid] = bv;
        ri[tid] = bi;
        __syncthreads();
        for (int st = 128; st; st >>= 1) {
            if (tid < st) {
                int oi = ri[tid + st];
                if (oi >= 0 && better(rv[tid + st], oi, rv[tid], ri[tid])) {
                    rv[tid] = rv[tid + st];
                    ri[tid] = oi;
                }
            }
            __syncthreads();
        }
        if (tid == 0) {
            int best = ri[0];
            if (best < 0) best = kk < E ? kk : 0;
            sel[kk] = best;
            selw[kk] = p[best];
        }
        __syncthreads();
    }

    if (tid == 0) {
        int ke = K;
        if (mode == 0) {
            if (norm_topk) {
                float sm = 0.0f;
                for (int kk = 0; kk < K; kk++) sm += selw[kk];
                for (int kk = 0; kk < K; kk++) selw[kk] /= sm;
            }
        } else if (mode == 1) {
            if (topp > 0.0f && topp < 1.0f) {
                for (int a = 1; a < K; a++) {
                    int ii = sel[a]; float ww = selw[a]; int b = a - 1;
                    while (b >= 0 && selw[b] < ww) { selw[b + 1] = selw[b]; sel[b + 1] = sel[b]; b--; }
                    selw[b + 1] = ww; sel[b + 1] = ii;
                }
                float tot = 1e-20f, cum = 0.0f;
                for (int kk = 0; kk < K; kk++) tot += selw[kk];
                for (int kk = 0; kk < K; kk++) {
                    cum += selw[kk];
                    if (cum >= topp * tot) { ke = kk + 1; break; }
                }
            }
            if (norm_topk) {
                float sm = 0.0f;
                for (int kk = 0; kk < ke; kk++) sm += selw[kk];
                sm += 1e-20f;
                for (int kk = 0; kk < ke; kk++) selw[kk] /= sm;
            }
            for (int kk = 0; kk < ke; kk++) selw[kk] *= routed_scale;
        } else {
            float sm = 0.0f;
            for (int kk = 0; kk < K; kk++) sm += selw[kk];
            for (int kk = 0; kk < K; kk++) selw[kk] /= (sm + 1e-20f);
            if (topp > 0.0f && topp < 1.0f) {
                for (int a = 1; a < K; a++) {
                    int e2 = sel[a]; float w2 = selw[a]; int b = a - 1;
                    while (b >= 0 && selw[b] < w2) { sel[b + 1] = sel[b]; selw[b + 1] = selw[b]; b--; }
                    sel[b + 1] = e2; selw[b + 1] = w2;
                }
                float cum = 0.0f; int keep = K;
                for (int kk = 0; kk < K; kk++) { cum += selw[kk]; if (cum >= topp) { keep = kk + 1; break; } }
                if (keep < K) {
                    float s2 = 0.0f;
                    for (int kk = 0; kk < keep; kk++) s2 += selw[kk];
                    for (int kk = 0; kk < keep; kk++) selw[kk] /= (s2 + 1e-20f);
                    ke = keep;
                }
            }
            if (routed_scale != 1.0f)
                for (int kk = 0; kk < ke; kk++) selw[kk] *= routed_scale;
        }
        for (int kk = 0; kk < K; kk++) {
            idx[(size_t)s * K + kk] = sel[kk];
            wout[(size_t)s * K + kk] = kk < ke ? selw[kk] : 0.0f;
        }
        keff[s] = ke;
    }
}

extern "C" hipError_t coli_launch_router_select(const float *logits, const float *bias, int S, int E,
                                                int K, int mode, float topp, int norm_topk,
                                                float routed_scale, int *idx, float *w, int *keff,
                                                hipStream_t st) {
    size_t shm = (size_t)2 * E * sizeof(float);
    hipLaunchKernelGGL(coli_router_select, dim3(S), dim3(256), shm, st, logits, bias, E, K, mode, topp,
                       norm_topk, routed_scale, idx, w, keff);
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
