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
// of c/colibri.c:3978 / c/olmoe.c:648), in two fixed-order halves so the
// 4-byte router weights stream from every CU at once:
//  * coli_router_partial: one wave per (expert, 512-column chunk); lane l
//    covers columns 4l..4l+3 of each 256-column step, then a fixed butterfly
//    gives part[chunk][s][e];
//  * the selection kernel adds the chunks in chunk order while it reads them.
// ---------------------------------------------------------------------------
#define COLI_ROUTER_CHUNK 512
template <int SMAX>
__global__ __launch_bounds__(256) void coli_router_partial(const float *__restrict__ x, int S,
                                                           const float *__restrict__ W, int D, int E,
                                                           float *__restrict__ part, size_t chstride) {
    // readfirstlane: the wave index is wave-uniform, so everything derived from it
    // (tile indices, validity, base pointers) stays in scalar registers.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = blockIdx.x * 4 + wave, ch = blockIdx.y;
    if (e >= E) return;
    const float *wr = W + (size_t)e * D;
    float acc[SMAX];
#pragma unroll
    for (int s = 0; s < SMAX; s++) acc[s] = 0.0f;
#pragma unroll
    for (int step = 0; step < COLI_ROUTER_CHUNK / 256; step++) {
        const int d = ch * COLI_ROUTER_CHUNK + step * 256 + lane * 4;
        if (d >= D) break;
        if ((D & 3) == 0) {
            const float4 wv = *(const float4 *)(wr + d);
#pragma unroll
            for (int s = 0; s < SMAX; s++) {
                if (s >= S) break;
                const float4 xv = *(const float4 *)(x + (size_t)s * D + d);
                float a = xv.x * wv.x;
                a = fmaf(xv.y, wv.y, a);
                a = fmaf(xv.z, wv.z, a);
                acc[s] += fmaf(xv.w, wv.w, a);
            }
        } else {
            for (int t = 0; t < 4 && d + t < D; t++) {
                const float wv = wr[d + t];
#pragma unroll
                for (int s = 0; s < SMAX; s++)
                    if (s < S) acc[s] = fmaf(x[(size_t)s * D + d + t], wv, acc[s]);
            }
        }
    }
#pragma unroll
    for (int s = 0; s < SMAX; s++) {
        if (s >= S) break;
        float v = acc[s];
#pragma unroll
        for (int off = 32; off; off >>= 1) v += __shfl_xor(v, off);
        if (lane == 0) part[(size_t)ch * chstride + (size_t)s * E + e] = v;
    }
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

// ---------------------------------------------------------------------------
// Top-K selection, one 64-lane wave per token row (E <= 1024, K <= 64). The
// logits are the sum of the router's column-chunk partials, added in chunk
// order.
//   mode 0: p = softmax(z) (max-subtracted, c/olmoe.c:246-250), select on p,
//           weight p, optional norm over K without epsilon (c/olmoe.c:681).
//   mode 1: p = sigmoid(z), choice = p + bias, select on choice, weight p,
//           TOPP (sort by weight, tot = 1e-20 + sum, keep until cum >=
//           topp * tot), norm_topk (sum + 1e-20), x routed_scale
//           (c/backend_cuda.cu:2169-2194, c/colibri.c:3982-4126).
//   mode 2: as mode 1 for the selection; weights renormalized over the K
//           with +1e-20; TOPP keeps until cum >= topp and renormalizes the
//           kept set (c/kimi_k3.c:1337-1370); routed_scale applied after.
// The reference selects by K rounds of an argmax with strict '>' (highest
// value, lowest index on ties; NaN and values <= -1e30 never chosen; a round
// with nothing left picks index kk, c/route_trace.h:383-393). The same order
// is computed here in one pass: a valid expert's rank is the number of valid
// experts that beat it, and rank r < K lands in slot r. Ranks are distinct
// because the order is total (ties go to the lower index).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool valid_score(float v) { return v == v && v > -1e30f; }

__global__ __launch_bounds__(256) void coli_router_select(const float *__restrict__ part, int nch,
                                                          const float *__restrict__ bias, int S, int E, int K,
                                                          int mode, float topp, int norm_topk,
                                                          float routed_scale, int *__restrict__ idx,
                                                          float *__restrict__ wout, int *__restrict__ keff) {
    extern __shared__ float sh[];
    // readfirstlane: the wave index is wave-uniform, so everything derived from it
    // (tile indices, validity, base pointers) stays in scalar registers.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = blockIdx.x * 4 + wave;
    float *p = sh + (size_t)wave * (2 * E + 128);     // [E] weight source
    float *c = p + E;                                 // [E] selection score
    int *sel = (int *)(c + E);                        // [64]
    float *selw = c + E + 64;                         // [64]
    const bool live = s < S;
    const size_t chstride = (size_t)S * E;
    const float *z0 = part + (size_t)(live ? s : 0) * E;
    auto logit = [&](int e) {
        float v = z0[e];
        for (int ch = 1; ch < nch; ch++) v += z0[(size_t)ch * chstride + e];
        return v;
    };
    if (mode == 0) {
        float m = -1e30f;
        for (int e = lane; e < E; e += 64) {
            const float v = logit(e);
            p[e] = v;
            m = fmaxf(m, v);
        }
#pragma unroll
        for (int off = 32; off; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float sum = 0.0f;
        for (int e = lane; e < E; e += 64) {
            const float v = expf(p[e] - m);
            p[e] = v;
            sum += v;
        }
#pragma unroll
        for (int off = 32; off; off >>= 1) sum += __shfl_xor(sum, off);
        for (int e = lane; e < E; e += 64) {
            p[e] = p[e] / sum;
            c[e] = p[e];
        }
    } else {
        for (int e = lane; e < E; e += 64) {
            const float v = 1.0f / (1.0f + expf(-logit(e)));
            p[e] = v;
            c[e] = v + (bias ? bias[e] : 0.0f);
        }
    }
    if (lane < 64) sel[lane] = -1;
    __syncthreads();
    if (!live) return;
    // ranks of this lane's experts among the valid ones
    // Radix select on order-preserving keys (a valid score maps to a key > 0,
    // an invalid one to 0; +0 and -0 share a key, as they compare equal):
    // T = the K-th largest key, then everything above T plus the lowest-index
    // experts equal to T; the chosen ones are ranked among themselves.
    // Lane l holds experts l, l + 64, ... (E <= 1024: at most 16).
    int nvalid = 0;
    unsigned key[16];
    const int nmine = (E - lane + 63) / 64;   // this lane's experts
    const int jmax = (E + 63) / 64;           // wave-uniform bound (keys past nmine are 0)
#pragma unroll
    for (int j = 0; j < 16; j++) {
        unsigned k = 0;
        if (j < nmine) {
            float v = c[lane + 64 * j];
            if (valid_score(v)) {
                if (v == 0.0f) v = 0.0f;
                const unsigned b = __float_as_uint(v);
                k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
            }
        }
        key[j] = k;
        nvalid += k != 0;
    }
#pragma unroll
    for (int off = 32; off; off >>= 1) nvalid += __shfl_xor(nvalid, off);
    const int want = nvalid < K ? nvalid : K;
    unsigned T = 0;
    if (want > 0) {
        for (int bit = 31; bit >= 0; bit--) {
            const unsigned cand = T | (1u << bit);
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (j >= jmax) break;
                cnt += __popcll(__ballot(key[j] >= cand));
            }
            if (cnt >= want) T = cand;
        }
    }
    // chosen: key > T, or key == T among the first (want - above) in index order
    int above = 0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        if (j >= jmax) break;
        above += __popcll(__ballot(key[j] > T));
    }
    const unsigned long long lt = (1ull << lane) - 1ull;
    int eq_before = 0;          // experts equal to T with a lower index, running over j
    int nchosen = 0;
    __shared__ unsigned ckey[4][64];
    __shared__ int cexp[4][64];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        if (j >= jmax) break;
        const bool gt = want > 0 && key[j] > T;
        const bool eq = want > 0 && key[j] == T && key[j] != 0;
        const unsigned long long meq = __ballot(eq);
        const bool take_eq = eq && eq_before + __popcll(meq & lt) < want - above;
        const bool take = gt || take_eq;
        const unsigned long long mt = __ballot(take);
        if (take) {
            const int slot = nchosen + __popcll(mt & lt);
            ckey[wave][slot] = key[j];
            cexp[wave][slot] = lane + 64 * j;
        }
        nchosen += __popcll(mt);
        eq_before += __popcll(meq);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane < nchosen) {   // rank among the chosen: larger key first, lower index on ties
        const unsigned k0 = ckey[wave][lane];
        const int e0 = cexp[wave][lane];
        int rank = 0;
        for (int q = 0; q < nchosen; q++) {
            const unsigned k1 = ckey[wave][q];
            const int e1 = cexp[wave][q];
            rank += (k1 > k0 || (k1 == k0 && e1 < e0)) ? 1 : 0;
        }
        sel[rank] = e0;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // sel[] written by its owner lanes
    if (lane != 0) return;
    for (int kk = 0; kk < K; kk++) {
        if (kk >= nvalid) sel[kk] = kk < E ? kk : 0;
        selw[kk] = p[sel[kk]];
    }
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

extern "C" hipError_t coli_launch_router_select(const float *part, int nch, const float *bias, int S, int E,
                                                int K, int mode, float topp, int norm_topk,
                                                float routed_scale, int *idx, float *w, int *keff,
                                                hipStream_t st) {
    size_t shm = (size_t)4 * (2 * E + 128) * sizeof(float);
    hipLaunchKernelGGL(coli_router_select, dim3((S + 3) / 4), dim3(256), shm, st, part, nch, bias, S, E, K, mode,
                       topp, norm_topk, routed_scale, idx, w, keff);
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
