// coli_route.h -- device code of the router: the partial logits of one wave
// and the top-K selection of one token row by one wave, shared by the
// separate router kernels (pipe.hip) and the fused decode routing of the MoE
// layer (moe.hip).
#pragma once
#include "coli_hip_internal.h"

#include <math.h>

#include "coli_device.h"

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
// Sum of each of the SMAX per-row values over the 64 lanes, in the order of
// the butterfly v += shfl_xor(v, 32), then 16, 8, 4, 2, 1 (so bitwise that
// butterfly's result), as a reduce-scatter: at each of the first log2(SMAX)
// steps a lane keeps half of its rows and adds its partner's copy of them, so
// the steps exchange SMAX/2 + SMAX/4 + ... + 1 values instead of SMAX each.
// Row (lane >> (6 - log2 SMAX)) ends in the lanes of its group; store(row, v)
// runs on the group's first lane.
template <int SMAX, typename F>
__device__ __forceinline__ void reduce_rows64(float (&v)[SMAX], int lane, F &&store) {
    constexpr int LG = SMAX >= 32 ? 5 : SMAX >= 16 ? 4 : SMAX >= 8 ? 3 : SMAX >= 4 ? 2 : SMAX >= 2 ? 1 : 0;
    static_assert((1 << LG) == SMAX && SMAX <= 32, "a power of two up to 32 rows");
#pragma unroll
    for (int k = 0; k < LG; k++) {
        const int o = 32 >> k, n = SMAX >> k, h = n / 2;
        const bool up = (lane & o) != 0;
#pragma unroll
        for (int i = 0; i < h; i++) {
            const float send = up ? v[i] : v[i + h];
            const float keep = up ? v[i + h] : v[i];
            v[i] = keep + __shfl_xor(send, o);
        }
    }
    float t = v[0];
#pragma unroll
    for (int o = 32 >> LG; o; o >>= 1) t += __shfl_xor(t, o);
    if ((lane & ((64 >> LG) - 1)) == 0) store(lane >> (6 - LG), t);
}

// One wave's partial logits of expert e over column chunk ch, rows 0..S-1
// (S <= SMAX). ATOMIC: stored as agent-scope atomics, for a reader on
// another XCD inside the same launch.
template <int SMAX, bool ATOMIC>
__device__ __forceinline__ void router_partial_wave(const float *__restrict__ x, int S, const float *__restrict__ W,
                                                    int D, int E, float *__restrict__ part, size_t chstride, int e,
                                                    int ch, int lane) {
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
                if (s < S) {
                    const float4 xv = *(const float4 *)(x + (size_t)s * D + d);
                    float a = xv.x * wv.x;
                    a = fmaf(xv.y, wv.y, a);
                    a = fmaf(xv.z, wv.z, a);
                    acc[s] += fmaf(xv.w, wv.w, a);
                }
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
    reduce_rows64<SMAX>(acc, lane, [&](int s, float v) {
        if (s < S) {
            float *dst = part + (size_t)ch * chstride + (size_t)s * E + e;
            if constexpr (ATOMIC) __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else *dst = v;
        }
    });
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
//   mode 3: DeepSeek-V4 (c/deepseek_v4.c:1368-1432): p = sqrt(softplus(z))
//           (stable form), choice = p + bias, weights p / sum over the K x
//           routed_scale; a non-positive sum selects nothing (keff 0).
// The reference selects by K rounds of an argmax with strict '>' (highest
// value, lowest index on ties; NaN and values <= -1e30 never chosen; a round
// with nothing left picks index kk, c/route_trace.h:383-393). The same rounds
// run here across the wave: each is a 64-lane argmax over order-preserving
// keys, which leaves the chosen expert and its weight in lane kk; the
// post-processing (normalization, TOPP ranks and cumulative sums) then runs
// with one slot per lane.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool valid_score(float v) { return v == v && v > -1e30f; }

// Wave-wide reductions without LDS round trips: a butterfly inside each
// 16-lane row through DPP lane moves (quad_perm xor 1, xor 2, then row
// rotations by 4 and 8), then the four row results read into scalar registers
// and combined in row order. Every lane returns the same value; the
// combination order is fixed, so results are reproducible.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
#define COLI_DPP_XOR1 0xB1    // quad_perm [1, 0, 3, 2]
#define COLI_DPP_XOR2 0x4E    // quad_perm [2, 3, 0, 1]
#define COLI_DPP_ROR4 0x124   // row_ror:4
#define COLI_DPP_ROR8 0x128   // row_ror:8

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = op(v, __int_as_float(dpp_mov<COLI_DPP_XOR1>(__float_as_int(v))));
    v = op(v, __int_as_float(dpp_mov<COLI_DPP_XOR2>(__float_as_int(v))));
    v = op(v, __int_as_float(dpp_mov<COLI_DPP_ROR4>(__float_as_int(v))));
    v = op(v, __int_as_float(dpp_mov<COLI_DPP_ROR8>(__float_as_int(v))));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return op(op(op(r0, r1), r2), r3);
}
__device__ __forceinline__ float wave_sum(float v) {
    return wave_reduce(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ int wave_sum_i(int v) {
    v += dpp_mov<COLI_DPP_XOR1>(v);
    v += dpp_mov<COLI_DPP_XOR2>(v);
    v += dpp_mov<COLI_DPP_ROR4>(v);
    v += dpp_mov<COLI_DPP_ROR8>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, dpp_mov<COLI_DPP_XOR1>(v));
    v = min(v, dpp_mov<COLI_DPP_XOR2>(v));
    v = min(v, dpp_mov<COLI_DPP_ROR4>(v));
    v = min(v, dpp_mov<COLI_DPP_ROR8>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
// Maximum of a 64-bit value over the wave (DPP steps on both halves inside
// each 16-lane row, then the four rows); uniform result.
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    auto step = [&](unsigned long long o) { v = o > v ? o : v; };
#define COLI_MAX64_STEP(CTRL)                                                                  \
    step(((unsigned long long)(unsigned)dpp_mov<CTRL>((int)(v >> 32)) << 32) |                 \
         (unsigned)dpp_mov<CTRL>((int)(unsigned)v))
    COLI_MAX64_STEP(COLI_DPP_XOR1);
    COLI_MAX64_STEP(COLI_DPP_XOR2);
    COLI_MAX64_STEP(COLI_DPP_ROR4);
    COLI_MAX64_STEP(COLI_DPP_ROR8);
#undef COLI_MAX64_STEP
    unsigned long long r = 0ull;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const unsigned long long o = ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)(v >> 32), 16 * q) << 32) |
                                     (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, 16 * q);
        r = o > r ? o : r;
    }
    return r;
}

#define COLI_SEL_BATCH 4   // experts per lane whose chunk partials are loaded together (JM >= 4)
#define COLI_SEL_MAXCH 16  // chunk partials held in registers (more are added from memory)
// Partial logits of four experts (one per wave) over one 512-column chunk for
// up to SMAX rows, with the rows' chunk staged once in LDS by the workgroup
// (every wave reading them from L2 cost four times the traffic). The router
// weights are requested before the staging. D % 4 == 0. All 256 threads of
// the workgroup call it (it synchronizes).
template <int SMAX, bool ATOMIC, int EPW = 1>
__device__ __forceinline__ void router_partial_block(const float *__restrict__ x, int S, const float *__restrict__ W,
                                                     int D, int E, float *__restrict__ part, size_t chstride,
                                                     int e0, int ch, int lane, floatx4 (*xs)[COLI_ROUTER_CHUNK / 4]) {
    // EPW experts per wave (e0, e0 + 1, ...): each activation read from LDS
    // feeds EPW products; the arithmetic of each expert is unchanged
    constexpr int NV = COLI_ROUTER_CHUNK / 4;   // float4 per row chunk
    const int d0 = ch * COLI_ROUTER_CHUNK;
    floatx4 wv[EPW][COLI_ROUTER_CHUNK / 256];
#pragma unroll
    for (int x_ = 0; x_ < EPW; x_++)
#pragma unroll
        for (int step = 0; step < COLI_ROUTER_CHUNK / 256; step++) {
            const int d = d0 + step * 256 + lane * 4, e = e0 + x_;
            wv[x_][step] = (e < E && d < D) ? *(const floatx4 *)(W + (size_t)e * D + d)
                                             : (floatx4){0.f, 0.f, 0.f, 0.f};
        }
    // the rows' chunk (SMAX x NV float4) staged by the 256 threads: every load
    // issued before any is waited for (one memory round trip)
    constexpr int PER = (SMAX * NV + 255) / 256;
    floatx4 xv[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int v = threadIdx.x + 256 * u;
        const int s = v / NV, c = v - s * NV, d = d0 + c * 4;
        xv[u] = (v < SMAX * NV && s < S && d < D) ? *(const floatx4 *)(x + (size_t)s * D + d)
                                                  : (floatx4){0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int v = threadIdx.x + 256 * u;
        if (v < SMAX * NV) xs[v / NV][v % NV] = xv[u];
    }
    __syncthreads();
    if (e0 >= E) return;
    float acc[EPW][SMAX];
#pragma unroll
    for (int x_ = 0; x_ < EPW; x_++)
#pragma unroll
        for (int s = 0; s < SMAX; s++) acc[x_][s] = 0.0f;
#pragma unroll
    for (int step = 0; step < COLI_ROUTER_CHUNK / 256; step++) {
#pragma unroll
        for (int s = 0; s < SMAX; s++) {
            const floatx4 xv = xs[s][step * 64 + lane];
#pragma unroll
            for (int x_ = 0; x_ < EPW; x_++) {
                float a = xv[0] * wv[x_][step][0];
                a = fmaf(xv[1], wv[x_][step][1], a);
                a = fmaf(xv[2], wv[x_][step][2], a);
                acc[x_][s] += fmaf(xv[3], wv[x_][step][3], a);
            }
        }
    }
#pragma unroll
    for (int x_ = 0; x_ < EPW; x_++) {
        const int e = e0 + x_;
        if (e >= E) break;
        reduce_rows64<SMAX>(acc[x_], lane, [&](int s, float v) {
            if (s < S) {
                float *dst = part + (size_t)ch * chstride + (size_t)s * E + e;
                if constexpr (ATOMIC) __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else *dst = v;
            }
        });
    }
}

// The end of one row's selection, once lane kk < want holds the expert of
// rank kk (my_e) and its weight source (my_w, = p[my_e]): the slots past
// want (fewer valid scores than K) take experts 0, 1, ...; the mode's
// normalization, TOPP cut and scale; then the row's slots, weights and keff
// are written (see select_row).
template <bool ATOMIC>
__device__ __forceinline__ void select_finish(int my_e, float my_w, int want, int E, int K, int mode, float topp,
                                              int norm_topk, float routed_scale, const float *p,
                                              int *__restrict__ idx, float *__restrict__ wout,
                                              int *__restrict__ keff, int s, int lane, int *sidx, int *skeff,
                                              bool gwrite) {
    const bool act = lane < K;
    if (act && lane >= want) {   // fewer valid scores than K: experts 0, 1, ... fill the rest
        my_e = lane < E ? lane : 0;
        my_w = p[my_e];
    }
    if (!act) my_w = 0.0f;
    auto wsum = [](float v) { return wave_sum(v); };
    // rank of this slot when sorted by weight, descending and stable (ties
    // keep slot order), and the inclusive cumulative weight in that order
    auto sort_rank = [&](int &rank, float &cum) {
        rank = 0;
        cum = 0.0f;
        for (int j = 0; j < K; j++) {
            const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), j));
            const bool before = wj > my_w || (wj == my_w && j < lane);
            rank += before ? 1 : 0;
            cum += (before || j == lane) ? wj : 0.0f;
        }
    };
    int slot = lane, ke = K;
    const bool cut = topp > 0.0f && topp < 1.0f;
    if (mode == 0) {
        if (norm_topk) my_w /= wsum(my_w);
    } else if (mode == 1) {
        if (cut) {
            float cum;
            sort_rank(slot, cum);
            const float tot = 1e-20f + wsum(my_w);
            const int first = wave_min_i(act && cum >= topp * tot ? slot : K - 1);
            ke = first + 1;
        }
        if (norm_topk) my_w /= wsum(act && slot < ke ? my_w : 0.0f) + 1e-20f;
        if (slot < ke) my_w *= routed_scale;
    } else if (mode == 3) {
        // score / sum of the selected scores * route scale; a non-positive sum
        // (an error in coli_v4_route) selects nothing
        const float total = wsum(my_w);
        if (!(total > 0.0f)) ke = 0;
        else my_w = my_w / total * routed_scale;
    } else {
        my_w /= wsum(my_w) + 1e-20f;
        if (cut) {
            float cum;
            sort_rank(slot, cum);
            const int keep = wave_min_i(act && cum >= topp ? slot + 1 : K);
            if (keep < K) {
                my_w /= wsum(act && slot < keep ? my_w : 0.0f) + 1e-20f;
                ke = keep;
            }
        }
        if (routed_scale != 1.0f && slot < ke) my_w *= routed_scale;
    }
    if (act && gwrite) {
        if constexpr (ATOMIC) {   // read back by another workgroup of the same launch
            __hip_atomic_store(idx + (size_t)s * K + slot, my_e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(wout + (size_t)s * K + slot, slot < ke ? my_w : 0.0f, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        } else {
            idx[(size_t)s * K + slot] = my_e;
            wout[(size_t)s * K + slot] = slot < ke ? my_w : 0.0f;
        }
    }
    if (act && sidx) sidx[s * K + slot] = my_e;
    if (lane == 0) {
        if (gwrite) {
            if constexpr (ATOMIC) __hip_atomic_store(keff + s, ke, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else keff[s] = ke;
        }
        if (skeff) skeff[s] = ke;
    }
}

// Selection of token row s by one wave; p: [E] floats of LDS for this wave.
// ATOMIC: idx / wout / keff are written as agent-scope atomics (read back by
// another workgroup of the same launch); LD_ATOMIC: the partials are read as
// agent-scope atomics (written by other workgroups of the same launch). sidx / skeff (optional): copies of the
// row's slots and keff for a reader in the same workgroup. gwrite false: idx / wout / keff are not written
// (workgroups that select only for themselves).
template <int JM, bool ATOMIC, bool LD_ATOMIC = ATOMIC>
__device__ __forceinline__ void select_row(const float *__restrict__ part, int nch, const float *__restrict__ bias,
                                           int S, int E, int K, int mode, float topp, int norm_topk,
                                           float routed_scale, int *__restrict__ idx, float *__restrict__ wout,
                                           int *__restrict__ keff, float *p, int s, int lane, int *sidx,
                                           int *skeff, bool gwrite = true) {
    auto ld = [](const float *q) {
        if constexpr (LD_ATOMIC) return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else return *q;
    };
    const bool live = s < S;
    const size_t chstride = (size_t)S * E;
    const float *z0 = part + (size_t)(live ? s : 0) * E;
    // Lane l owns experts e = l + 64 j (E <= 1024: j < 16). Their chunk
    // partials (and bias) are all requested before the first add: every load
    // is unconditional (indices clamped into range, the extra values masked
    // in the sum), so none waits for another. Logits are summed in chunk order.
    constexpr int CB = COLI_SEL_BATCH < JM ? COLI_SEL_BATCH : JM, CH = COLI_SEL_MAXCH;
    const int nmine = (E - lane + 63) / 64;   // this lane's experts
    const int jmax = (E + 63) / 64;           // wave-uniform bound
    float lg[JM] = {}, bs[JM] = {};
#pragma unroll
    for (int j0 = 0; j0 < JM; j0 += CB) {
        if (j0 >= jmax) continue;
        float t[CB][CH];
        int ee[CB];
#pragma unroll
        for (int jj = 0; jj < CB; jj++) {
            ee[jj] = min(lane + 64 * (j0 + jj), E - 1);
#pragma unroll
            for (int ch = 0; ch < CH; ch++) t[jj][ch] = ld(z0 + (size_t)min(ch, nch - 1) * chstride + ee[jj]);
            bs[j0 + jj] = bias ? bias[ee[jj]] : 0.0f;
        }
#pragma unroll
        for (int jj = 0; jj < CB; jj++) {
            float v = t[jj][0];
#pragma unroll
            for (int ch = 1; ch < CH; ch++) v += ch < nch ? t[jj][ch] : 0.0f;
            for (int ch = CH; ch < nch; ch++) v += ld(z0 + (size_t)ch * chstride + ee[jj]);
            lg[j0 + jj] = v;
        }
    }
    // the weight source of each expert goes to LDS (p, read back for the
    // selected slots), its selection score to cv
    float cv[JM];
    if (mode == 0) {
        float m = -1e30f;
#pragma unroll
        for (int j = 0; j < JM; j++)
            if (j < nmine) m = fmaxf(m, lg[j]);
        m = wave_max(m);
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < JM; j++) {
            lg[j] = j < nmine ? expf(lg[j] - m) : 0.0f;
            sum += lg[j];
        }
        sum = wave_sum(sum);
#pragma unroll
        for (int j = 0; j < JM; j++) {
            const float v = lg[j] / sum;
            if (j < nmine) p[lane + 64 * j] = v;
            cv[j] = v;
        }
    } else if (mode == 3) {
        // DeepSeek-V4: sqrt of the stable softplus (c/deepseek_v4.c:1368-1392)
#pragma unroll
        for (int j = 0; j < JM; j++) {
            const float z = lg[j];
            const float v = sqrtf(fmaxf(z, 0.0f) + log1pf(expf(-fabsf(z))));
            if (j < nmine) p[lane + 64 * j] = v;
            cv[j] = v + bs[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < JM; j++) {
            const float v = 1.0f / (1.0f + expf(-lg[j]));
            if (j < nmine) p[lane + 64 * j] = v;
            cv[j] = v + bs[j];
        }
    }
    if (!live) return;
    // Order-preserving keys: a valid score maps to a key > 0, an invalid one
    // (NaN, or <= -1e30) to 0; +0 and -0 share a key, as they compare equal.
    int nvalid = 0;
    unsigned key[JM];
#pragma unroll
    for (int j = 0; j < JM; j++) {
        unsigned k = 0;
        if (j < nmine) {
            float v = cv[j];
            if (valid_score(v)) {
                if (v == 0.0f) v = 0.0f;
                const unsigned b = __float_as_uint(v);
                k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
            }
        }
        key[j] = k;
        nvalid += k != 0;
    }
    nvalid = wave_sum_i(nvalid);
    const int want = nvalid < K ? nvalid : K;
    // The selection is the order of (key desc, expert index asc): round kk
    // of the reference's argmax picks the entry of rank kk. my_e / my_w end
    // in lane kk for slot kk.
    int my_e = 0;
    float my_w = 0.0f;
    if (JM == 1 && K <= 64) {
        // One entry per lane: ranks by comparison instead of K serial rounds.
        // Entries are ordered by c = key << 32 | ~index (a larger c ranks
        // first; keys are unique per index, so c is a strict total order);
        // the entry of rank r < K goes to slot r.
        __shared__ __attribute__((aligned(16))) unsigned long long rk_c[4][64], rk_sel[4][64];
        const int wv = (threadIdx.x >> 6) & 3;
        unsigned long long *cb = rk_c[wv], *sel = rk_sel[wv];
        unsigned long long c = key[0] ? ((unsigned long long)key[0] << 32) | (0xFFFFFFFFu - (unsigned)lane) : 0ull;
        cb[lane] = c;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // all 64 entries read before the first comparison (32 reads of two
        // entries in flight together)
        unsigned long long v[64];
#pragma unroll
        for (int i = 0; i < 64; i += 2) {
            const ulonglong2 t2 = *(const ulonglong2 *)(cb + i);
            v[i] = t2.x;
            v[i + 1] = t2.y;
        }
        int r = 0;
#pragma unroll
        for (int i = 0; i < 64; i++) r += v[i] > c;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (c != 0ull && r < K) sel[r] = c;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        c = lane < want ? sel[lane] : 0ull;
        if (lane < want) {
            my_e = (int)(0xFFFFFFFFu - (unsigned)(c & 0xFFFFFFFFull));
            my_w = p[my_e];
        }
    } else {
        // K rounds over the lanes' sorted lists: every lane sorts its JM
        // entries once (c descending), then round kk takes the wave maximum
        // of the lanes' heads (the entry of rank kk) and its owner pops it.
        // c = key << 32 | ~index as above; 0 marks no entry.
        unsigned long long c[JM];
#pragma unroll
        for (int j = 0; j < JM; j++)
            c[j] = (j < jmax && key[j]) ? ((unsigned long long)key[j] << 32) | (0xFFFFFFFFu - (unsigned)(lane + 64 * j))
                                        : 0ull;
#pragma unroll
        for (int i = 1; i < JM; i++)
#pragma unroll
            for (int j = i; j > 0; j--)
                if (c[j] > c[j - 1]) {
                    const unsigned long long t = c[j];
                    c[j] = c[j - 1];
                    c[j - 1] = t;
                }
        unsigned long long mine = 0ull;
        for (int kk = 0; kk < want; kk++) {
            const unsigned long long m = wave_max_u64(c[0]);
            if (c[0] == m) {   // one lane: the entries are distinct
#pragma unroll
                for (int j = 0; j + 1 < JM; j++) c[j] = c[j + 1];
                c[JM - 1] = 0ull;
            }
            if (lane == kk) mine = m;
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // p[] written by all lanes
        if (lane < want) {
            my_e = (int)(0xFFFFFFFFu - (unsigned)(mine & 0xFFFFFFFFull));
            my_w = p[my_e];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // p[] written by all lanes
    select_finish<ATOMIC>(my_e, my_w, want, E, K, mode, topp, norm_topk, routed_scale, p, idx, wout, keff, s, lane,
                          sidx, skeff, gwrite);
}

// Selection of token row s (of S) by the first NW waves of a workgroup,
// for the sigmoid-family modes 1-3 and E <= 64 NW: wave w scores experts
// 64 w + lane (chunk partials summed in chunk order, as select_row) and ranks
// them among its 64 by comparison; each wave's top K meet in LDS, and wave 0
// ranks those to the row's top K. The order is select_row's (score key
// descending, then expert index ascending), and so are the results: an expert
// among the row's top K is among its own wave's top K. Every wave of the
// workgroup calls it (one barrier); wave 0 returns with the row's slots and
// keff in sidx / skeff and, with gwrite, idx / wout / keff written (ATOMIC:
// as agent-scope atomics).
// LDS: p [E] floats (scores), stage [NW][64] and cand [NW][64] keys, nval
// [NW], selb [64] keys.
template <int NW, bool ATOMIC>
__device__ __forceinline__ void select_row_waves(const float *__restrict__ part, int nch,
                                                 const float *__restrict__ bias, int S, int s, int E, int K, int mode,
                                                 float topp,
                                                 int norm_topk, float routed_scale, int *__restrict__ idx,
                                                 float *__restrict__ wout, int *__restrict__ keff, float *p,
                                                 unsigned long long (*stage)[64], unsigned long long (*cand)[64],
                                                 int *nval, unsigned long long *selb, int *sidx, int *skeff,
                                                 bool gwrite, int wave, int lane) {
    if (wave < NW) {
        constexpr int CH = COLI_SEL_MAXCH;
        const int e = 64 * wave + lane;
        const bool live = e < E;
        const int ee = live ? e : E - 1;
        const size_t chstride = (size_t)S * E;
        const float *z0 = part + (size_t)s * E + ee;
        float t[CH];
#pragma unroll
        for (int ch = 0; ch < CH; ch++) t[ch] = z0[(size_t)min(ch, nch - 1) * chstride];
        const float bs = bias ? bias[ee] : 0.0f;
        float z = t[0];
#pragma unroll
        for (int ch = 1; ch < CH; ch++) z += ch < nch ? t[ch] : 0.0f;
        for (int ch = CH; ch < nch; ch++) z += z0[(size_t)ch * chstride];
        const float v = mode == 3 ? sqrtf(fmaxf(z, 0.0f) + log1pf(expf(-fabsf(z)))) : 1.0f / (1.0f + expf(-z));
        if (live) p[e] = v;
        unsigned k = 0;
        if (live) {
            float c = v + bs;
            if (valid_score(c)) {
                if (c == 0.0f) c = 0.0f;
                const unsigned b = __float_as_uint(c);
                k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
            }
        }
        const int nv = wave_sum_i(k != 0);
        const unsigned long long c = k ? ((unsigned long long)k << 32) | (0xFFFFFFFFu - (unsigned)e) : 0ull;
        stage[wave][lane] = c;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        unsigned long long vv[64];
#pragma unroll
        for (int i = 0; i < 64; i += 2) {
            const ulonglong2 t2 = *(const ulonglong2 *)(stage[wave] + i);
            vv[i] = t2.x;
            vv[i + 1] = t2.y;
        }
        int r = 0;
#pragma unroll
        for (int i = 0; i < 64; i++) r += vv[i] > c;
        if (c != 0ull && r < K) cand[wave][r] = c;
        if (lane == 0) nval[wave] = nv;
    }
    __syncthreads();
    if (wave != 0) return;
    int total = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) total += nval[w];
    const int want = total < K ? total : K;
    // candidate lane l: rank l % K of wave l / K (NW K <= 64)
    const int w = lane / K, r0 = lane - w * K;
    const unsigned long long c = (w < NW && r0 < min(K, nval[w < NW ? w : 0])) ? cand[w][r0] : 0ull;
    stage[0][lane] = c;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    unsigned long long vv[64];
#pragma unroll
    for (int i = 0; i < 64; i += 2) {
        const ulonglong2 t2 = *(const ulonglong2 *)(stage[0] + i);
        vv[i] = t2.x;
        vv[i + 1] = t2.y;
    }
    int r = 0;
#pragma unroll
    for (int i = 0; i < 64; i++) r += vv[i] > c;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (c != 0ull && r < K) selb[r] = c;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    int my_e = 0;
    float my_w = 0.0f;
    if (lane < want) {
        my_e = (int)(0xFFFFFFFFu - (unsigned)(selb[lane] & 0xFFFFFFFFull));
        my_w = p[my_e];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    select_finish<ATOMIC>(my_e, my_w, want, E, K, mode, topp, norm_topk, routed_scale, p, idx, wout, keff, s, lane,
                          sidx, skeff, gwrite);
}

