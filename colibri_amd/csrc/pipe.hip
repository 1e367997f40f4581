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
// of c/colibri.c:3978 / c/olmoe.c:648). EB experts per 256-thread block: each
// thread walks D with float4 loads, keeps EB x SMAX accumulators and reuses
// each activation load for the EB experts; fixed-order reductions (wave
// butterfly, then the 4 waves in order) finish each dot product.
// ---------------------------------------------------------------------------
template <int SMAX, int EB>
__global__ __launch_bounds__(256) void coli_router_logits(const float *__restrict__ x, int S,
                                                          const float *__restrict__ W, int D, int E,
                                                          float *__restrict__ logits) {
    const int e0 = blockIdx.x * EB;
    float acc[EB][SMAX];
#pragma unroll
    for (int k = 0; k < EB; k++)
#pragma unroll
        for (int s = 0; s < SMAX; s++) acc[k][s] = 0.0f;
    if ((D & 3) == 0) {
        for (int d = threadIdx.x * 4; d < D; d += 1024) {
            float4 wv[EB];
#pragma unroll
            for (int k = 0; k < EB; k++)
                wv[k] = e0 + k < E ? *(const float4 *)(W + (size_t)(e0 + k) * D + d) : make_float4(0, 0, 0, 0);
#pragma unroll
            for (int s = 0; s < SMAX; s++) {
                if (s < S) {
                    float4 xv = *(const float4 *)(x + (size_t)s * D + d);
#pragma unroll
                    for (int k = 0; k < EB; k++) {
                        acc[k][s] = fmaf(xv.x, wv[k].x, acc[k][s]);
                        acc[k][s] = fmaf(xv.y, wv[k].y, acc[k][s]);
                        acc[k][s] = fmaf(xv.z, wv[k].z, acc[k][s]);
                        acc[k][s] = fmaf(xv.w, wv[k].w, acc[k][s]);
                    }
                }
            }
        }
    } else {
        for (int d = threadIdx.x; d < D; d += 256) {
#pragma unroll
            for (int k = 0; k < EB; k++) {
                float wv = e0 + k < E ? W[(size_t)(e0 + k) * D + d] : 0.0f;
#pragma unroll
                for (int s = 0; s < SMAX; s++)
                    if (s < S) acc[k][s] = fmaf(x[(size_t)s * D + d], wv, acc[k][s]);
            }
        }
    }
    __shared__ float red[4][EB * SMAX];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < EB; k++)
#pragma unroll
        for (int s = 0; s < SMAX; s++) {
            float v = acc[k][s];
#pragma unroll
            for (int off = 32; off; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0) red[wave][k * SMAX + s] = v;
        }
    __syncthreads();
    for (int o = threadIdx.x; o < EB * SMAX; o += 256) {
        int k = o / SMAX, s = o - k * SMAX;
        if (s < S && e0 + k < E)
            logits[(size_t)s * E + e0 + k] = ((red[0][o] + red[1][o]) + red[2][o]) + red[3][o];
    }
}

extern "C" hipError_t coli_launch_router_logits(const float *x, int S, const float *W, int D, int E,
                                                float *logits, hipStream_t st) {
    for (int s0 = 0; s0 < S; s0 += 16) {   // 16 rows of accumulators per pass
        int n = S - s0 < 16 ? S - s0 : 16;
        const float *xs = x + (size_t)s0 * D;
        float *ls = logits + (size_t)s0 * E;
        if (n <= 4)
            hipLaunchKernelGGL((coli_router_logits<4, 1>), dim3(E), dim3(256), 0, st, xs, n, W, D, E, ls);
        else
            hipLaunchKernelGGL((coli_router_logits<16, 4>), dim3((E + 3) / 4), dim3(256), 0, st, xs, n, W, D, E, ls);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Top-K selection, one 64-lane wave per token row (E <= 4096, K <= 64).
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
// value, lowest index on ties, NaN never selected, values <= -1e30 never
// selected); an all-NaN round falls back to index kk (c/route_trace.h:383-393).
// Lane l owns experts e = l (mod 64); a selected expert is retired by its
// owner lane, so the rounds need no barrier.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    // (v, i) beats (bv, bi): larger value, or equal value and lower index.
    if (v != v || !(v > -1e30f)) return false;
    if (bi < 0) return true;
    return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(256) void coli_router_select(const float *__restrict__ logits,
                                                          const float *__restrict__ bias, int S, int E, int K,
                                                          int mode, float topp, int norm_topk,
                                                          float routed_scale, int *__restrict__ idx,
                                                          float *__restrict__ wout, int *__restrict__ keff) {
    extern __shared__ float sh[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s = blockIdx.x * 4 + wave;
    float *p = sh + (size_t)wave * (2 * E + 128);     // [E] weight source
    float *c = p + E;                                 // [E] selection score
    int *sel = (int *)(c + E);                        // [64]
    float *selw = c + E + 64;                         // [64]
    const bool live = s < S;
    const float *z = logits + (size_t)(live ? s : 0) * E;
    if (mode == 0) {
        float m = -1e30f;
        for (int e = lane; e < E; e += 64) m = fmaxf(m, z[e]);
#pragma unroll
        for (int off = 32; off; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float part = 0.0f;
        for (int e = lane; e < E; e += 64) {
            float v = expf(z[e] - m);
            p[e] = v;
            part += v;
        }
#pragma unroll
        for (int off = 32; off; off >>= 1) part += __shfl_xor(part, off);
        for (int e = lane; e < E; e += 64) {
            p[e] = p[e] / part;
            c[e] = p[e];
        }
    } else {
        for (int e = lane; e < E; e += 64) {
            float v = 1.0f / (1.0f + expf(-z[e]));
            p[e] = v;
            c[e] = v + (bias ? bias[e] : 0.0f);
        }
    }
    __syncthreads();
    if (!live) return;
    for (int kk = 0; kk < K; kk++) {
        float bv = 0.0f;
        int bi = -1;
        for (int e = lane; e < E; e += 64)
            if (better(c[e], e, bv, bi)) { bv = c[e]; bi = e; }
#pragma unroll
        for (int off = 32; off; off >>= 1) {
            float ov = __shfl_xor(bv, off);
            int oi = __shfl_xor(bi, off);
            if (oi >= 0 && better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        int best = bi >= 0 ? bi : (kk < E ? kk : 0);
        if (bi >= 0 && (best & 63) == lane) c[best] = __builtin_nanf("");   // retire
        if (lane == 0) {
            sel[kk] = best;
            selw[kk] = p[best];
        }
    }
    if (lane != 0) return;
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

extern "C" hipError_t coli_launch_router_select(const float *logits, const float *bias, int S, int E,
                                                int K, int mode, float topp, int norm_topk,
                                                float routed_scale, int *idx, float *w, int *keff,
                                                hipStream_t st) {
    size_t shm = (size_t)4 * (2 * E + 128) * sizeof(float);
    hipLaunchKernelGGL(coli_router_select, dim3((S + 3) / 4), dim3(256), shm, st, logits, bias, S, E, K, mode, topp,
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
