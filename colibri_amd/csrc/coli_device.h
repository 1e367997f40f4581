// coli_device.h -- device-side helpers shared by the GEMV and GEMM kernels:
// vector types, global-address-space loads, the B-operand unpack of the
// tiled int4 / e2m1 storage, and the per-group scale registers.
#pragma once

#include "coli_hip_internal.h"

#include <math.h>

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Loads through address-space-1 pointers: pointers read from descriptors are
// generic to the compiler, and generic (FLAT) loads may complete out of order,
// which forces a full vmcnt(0) drain before every use. Global loads keep the
// in-order counter the software pipeline relies on.
#define GPTR(T, p) ((const __attribute__((address_space(1))) T *)(const void *)(p))

typedef __attribute__((address_space(3))) void lds_void;
// LDS written by the DMA is invisible to the compiler's memory model: read it
// through volatile pointers so no read is folded or reordered across a wait.
#define LDS_RD(T, p) (*(const volatile __attribute__((address_space(3))) T *)(lds_void *)(p))
#define LDS_WR(T, p, v) (*(volatile __attribute__((address_space(3))) T *)(lds_void *)(p) = (v))

// A pointer every lane of the wave holds, moved to scalar registers (values
// read from memory by a vector load otherwise stay in VGPRs, and so would all
// address arithmetic derived from them).
__device__ __forceinline__ const uint8_t *uniform_ptr(const void *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t *)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ ColiProb uniform_prob(const ColiProb &p) {
    ColiProb u;
    u.w0 = uniform_ptr(p.w0);
    u.s0 = uniform_ptr(p.s0);
    u.w1 = uniform_ptr(p.w1);
    u.s1 = uniform_ptr(p.s1);
    u.nrows = __builtin_amdgcn_readfirstlane(p.nrows);
    u.xrow_off = __builtin_amdgcn_readfirstlane(p.xrow_off);
    u.out_row0 = __builtin_amdgcn_readfirstlane(p.out_row0);
    u.pad = 0;
    return u;
}


// Maximum over each 16-lane row, on the VALU (DPP: swap neighbours, swap
// pairs, mirror halves of 8, mirror halves of 16).
__device__ __forceinline__ float dpp_max16(float v) {
    auto step = [](float x, int ctrl) {
        const int o = ctrl == 0xB1   ? __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false)
                      : ctrl == 0x4E ? __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false)
                      : ctrl == 0x141 ? __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false)
                                      : __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false);
        return fmaxf(x, __int_as_float(o));
    };
    v = step(v, 0xB1);    // quad_perm [1, 0, 3, 2]
    v = step(v, 0x4E);    // quad_perm [2, 3, 0, 1]
    v = step(v, 0x141);   // row_half_mirror
    return step(v, 0x140);  // row_mirror
}

// Maximum over the wave: rows by DPP, then across rows with the two lane-swap
// permutes (lane l meets l ^ 16, then l ^ 32).
__device__ __forceinline__ float wave_max64(float v) {
    v = dpp_max16(v);
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

template <int KIND>
__device__ __forceinline__ half8v unpack_b(uint32_t w) {
    if constexpr (KIND == COLI_KIND_FP4) {
        half2v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0);
        half2v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1);
        half2v c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2);
        half2v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3);
        return (half8v){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    } else {
        uint32_t lo = w & 0x0F0F0F0Fu, hi = w & 0xF0F0F0F0u;
        uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);
        uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);
        uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);
        uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);
        const half2v blo = {(_Float16)1032.0f, (_Float16)1032.0f};
        const half2v bhi = {(_Float16)1152.0f, (_Float16)1152.0f};
        half2v a = __builtin_bit_cast(half2v, p0) - blo;
        half2v b = __builtin_bit_cast(half2v, p1) - blo;
        half2v c = __builtin_bit_cast(half2v, p2) - bhi;
        half2v d = __builtin_bit_cast(half2v, p3) - bhi;
        return (half8v){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    }
}

// e2m1 nibbles times a power-of-two scale, converted exactly to fp16 when the
// products are normal fp16 values (scales 2^-13 .. 2^13).
__device__ __forceinline__ half8v unpack_fp4_scaled(uint32_t w, float s) {
    half2v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 0);
    half2v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 1);
    half2v c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 2);
    half2v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 3);
    return (half8v){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Scale of group j (0..3) of the lane's row, from the per-tile-quad scale word(s).
template <int KIND> struct ScaleRegs;
template <> struct ScaleRegs<COLI_KIND_I4_H> {
    static constexpr int kTileBytes = 16 * 8;
    u32x2 v;
    __device__ void load(const void *base, size_t tq, int r16) {
        v = *GPTR(u32x2, (const uint8_t *)base + (tq * 16 + r16) * 8);
    }
    __device__ float get(int j) const {
        uint32_t wd = v[j >> 1];
        _Float16 h = __builtin_bit_cast(half2v, wd)[j & 1];
        return (float)h;
    }
    __device__ void zero() { v = (u32x2){0u, 0u}; }
};
template <> struct ScaleRegs<COLI_KIND_I4_F> {
    static constexpr int kTileBytes = 16 * 16;
    floatx4 v;
    __device__ void load(const void *base, size_t tq, int r16) {
        v = *GPTR(floatx4, (const uint8_t *)base + (tq * 16 + r16) * 16);
    }
    __device__ float get(int j) const { return v[j]; }
    __device__ void zero() { v = (floatx4){0.f, 0.f, 0.f, 0.f}; }
};
template <> struct ScaleRegs<COLI_KIND_FP4> {
    static constexpr int kTileBytes = 16 * 4;
    uint32_t v;
    __device__ void load(const void *base, size_t tq, int r16) {
        v = *GPTR(uint32_t, (const uint8_t *)base + (tq * 16 + r16) * 4);
    }
    __device__ float get(int j) const {
        return __builtin_bit_cast(float, ((v >> (8 * j)) & 0xFFu) << 23);
    }
    __device__ void zero() { v = 0u; }
};

__device__ __forceinline__ float silu_mul(float g, float u) {
    return (g / (1.0f + expf(-g))) * u;
}

// SwiGLU of the DUAL epilogues: silu(g) * u (c/backend_cuda.cu:618-624), or
// with limit > 0 the DeepSeek-V4 form (c/deepseek_v4.c:1434-1448): gate
// clamped from above and up to +-limit, g * sigmoid(g) * u with the
// two-branch stable sigmoid (c/deepseek_v4.c:1102-1109).
__device__ __forceinline__ float swiglu_out(float g, float u, float limit) {
    if (!(limit > 0.0f)) return silu_mul(g, u);
    g = fminf(g, limit);
    u = fmaxf(-limit, fminf(u, limit));
    float sg;
    if (g >= 0.0f) {
        sg = 1.0f / (1.0f + expf(-g));
    } else {
        const float e = expf(g);
        sg = e / (1.0f + e);
    }
    return g * sg * u;
}

// Output of one lane for batch row `brow` of the problem: output row
// rt*16 + (lane & 15) of every live tile, scaled back by the row's 2^E; for
// DUAL, silu(gate) * up of the paired tiles. With a.ehi (plain matrix, R
// even), the outputs are also written as the consuming GEMV's activation
// fragments: tiles r, r + 1 (rt[r] even) are one 32-column group of its
// input, whose exponent E' (max|y| * 2^-E' in [2^14, 2^15) over the group,
// as coli_prep_frag takes it over a row) the sixteen lanes of the row agree
// on by a DPP maximum; hi / lo are split and placed as coli_prep_frag does.
template <int R, bool DUAL>
__device__ __forceinline__ void gemv_epilogue(const ColiGemvArgs &a, const ColiProb &pr, int bt, const int (&rt)[R],
                                              const bool (&live)[R], const float (&v)[R], int brow, int lane,
                                              int E) {
    constexpr int RT = DUAL ? R / 2 : R;
    const int nb = min(16, pr.nrows - 16 * bt);
    if (brow >= nb) return;
    const int orow_i = pr.out_row0 + 16 * bt + brow;
    float *orow = a.out + (size_t)orow_i * a.ldo;
    float y[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const int o = rt[r] * 16 + (lane & 15);
        y[r] = 0.0f;
        if (!live[r] || o >= a.O) continue;
        if constexpr (DUAL) {
            float gv = ldexpf(v[r], E), uv = ldexpf(v[r + RT], E);
            y[r] = swiglu_out(gv, uv, a.swiglu_limit);
        } else {
            y[r] = ldexpf(v[r], E);
        }
        orow[o] = y[r];
    }
    if constexpr (!DUAL && R % 2 == 0) {
        if (!a.ehi) return;
#pragma unroll
        for (int r = 0; r < R; r += 2) {
            if (!live[r]) continue;   // wave-uniform
            float m = dpp_max16(fmaxf(fabsf(y[r]), fabsf(y[r + 1])));
            int Eg = 0;
            if (m > 0.0f && isfinite(m)) {
                frexpf(m, &Eg);
                Eg -= 15;
            }
            Eg = min(113, max(-126, Eg));
            const int g = rt[r] >> 1;
            const size_t rbase = (size_t)orow_i * a.estride + (size_t)g * 32;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int c = 16 * h + (lane & 15), off = c & 7;
                float yy = ldexpf(y[r + h], -Eg);
                int t = off;
                if (a.eint4) {
                    t = (off & 1) ? 4 + (off >> 1) : (off >> 1);
                    if (off & 1) yy *= 0.0625f;
                }
                const _Float16 hi = (_Float16)yy;
                const size_t idx = rbase + (c >> 3) * 8 + t;
                a.ehi[idx] = hi;
                a.elo[idx] = (_Float16)(yy - (float)hi);
            }
            if ((lane & 15) == 0) a.eexp[((size_t)(g >> 2) * a.erows + orow_i) * 4 + (g & 3)] = (uint8_t)(int8_t)Eg;
        }
    }
}

// Group exponent j (signed byte j of the row's word) and its 2^E.
__device__ __forceinline__ int gexp_of(uint32_t word, int j) { return (int)(int8_t)(word >> (8 * j)); }
__device__ __forceinline__ float gexp_pow2(uint32_t word, int j) {
    return __uint_as_float((uint32_t)(gexp_of(word, j) + 127) << 23);
}

// ---- LDS DMA rings (gemv_dma.hip, gemm.hip) ----
// Scale bytes of one tile quad: 16 rows x 4 groups of fp16 / f32 / e8m0.
template <int KIND> struct ScaleGeom {
    static constexpr int kBytes = ScaleRegs<KIND>::kTileBytes;   // 128 / 256 / 64
    static constexpr int kLanes = kBytes / 4;                      // dword lanes per tile
    static constexpr int kPerInst = 64 / kLanes;                   // tiles per dword DMA
};

template <int KIND>
__device__ __forceinline__ void scale_from_lds(ScaleRegs<KIND> &s, const uint8_t *p, int r16) {
    if constexpr (KIND == COLI_KIND_I4_H) s.v = LDS_RD(u32x2, p + r16 * 8);
    else if constexpr (KIND == COLI_KIND_I4_F) s.v = LDS_RD(floatx4, p + r16 * 16);
    else s.v = LDS_RD(uint32_t, p + r16 * 4);
}

// Wait until at most `pend` (0 .. PD-2) stages of L loads are still in flight.
template <int L, int PD>
__device__ __forceinline__ void dma_wait_tail(int pend) {
#define COLI_WT(k)                                                         \
    if (pend == k) {                                                       \
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(k * L) : "memory");       \
        return;                                                            \
    }
    if constexpr (PD > 5) { COLI_WT(4) }
    if constexpr (PD > 4) { COLI_WT(3) }
    if constexpr (PD > 3) { COLI_WT(2) }
    if constexpr (PD > 2) { COLI_WT(1) }
#undef COLI_WT
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------
// Activation-fragment build (the format and its reasons are described with
// coli_prep_frag in gemv.hip), shared by that kernel and launches that run
// the build beside other work.
// ---------------------------------------------------------------------------
#define COLI_PREP_SLOTS 8
// Block `blk` of the build (every thread of a 256-thread block calls it).
__device__ __forceinline__ void prep_frag_block(const ColiPrepArgs &a, int blk) {
    const float *__restrict__ x = a.x;
    const int *__restrict__ src_row = a.src_row, *__restrict__ nrows_dev = a.nrows_dev;
    _Float16 *__restrict__ hi = a.hi, *__restrict__ lo = a.lo;
    int *__restrict__ exp2out = a.exp2out, *__restrict__ haslo = a.haslo;
    const float *__restrict__ zero = a.zero;
    const int ldx = a.ldx, K = a.K, ngp = a.ngp, int4_order = a.int4_order, gen = a.gen, vec = a.vec,
              nchunk = a.nchunk;
    const int r = blk / nchunk, chunk = blk - r * nchunk;
    if (nrows_dev && r >= *nrows_dev) return;
    const int srow = src_row ? src_row[r] : r;
    if (srow < 0) return;
    const float *xr = x + (size_t)srow * ldx;
    const int nslot = ngp * 4;
    auto load_slot = [&](int slot, float (&v)[8]) {
        const int k0 = slot * 8;
        if (vec) {   // aligned rows, K % 8 == 0: slots past K read zeros
            const float *p = slot < nslot && k0 < K ? xr + k0 : zero;
            const floatx4 a = *GPTR(floatx4, p), b = *GPTR(floatx4, p + 4);
#pragma unroll
            for (int t = 0; t < 4; t++) { v[t] = a[t]; v[t + 4] = b[t]; }
        } else {
#pragma unroll
            for (int t = 0; t < 8; t++) v[t] = slot < nslot && k0 + t < K ? xr[k0 + t] : 0.0f;
        }
    };
    float v[COLI_PREP_SLOTS][8];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < COLI_PREP_SLOTS; i++) load_slot(threadIdx.x + 256 * i, v[i]);
#pragma unroll
    for (int i = 0; i < COLI_PREP_SLOTS; i++)
#pragma unroll
        for (int t = 0; t < 8; t++) m = fmaxf(m, fabsf(v[i][t]));
    for (int slot = threadIdx.x + 256 * COLI_PREP_SLOTS; slot < nslot; slot += 256) {
        float u[8];
        load_slot(slot, u);
#pragma unroll
        for (int t = 0; t < 8; t++) m = fmaxf(m, fabsf(u[t]));
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float wmax[4];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int E = 0;
    if (m > 0.0f && isfinite(m)) {
        frexpf(m, &E);
        E -= 15;
    }
    if (threadIdx.x == 0 && chunk == 0) exp2out[r] = E;
    bool any = false;
    auto convert = [&](int slot, const float (&u)[8]) {
        if (slot >= nslot) return;
        _Float16 h[8], l[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            int off = int4_order ? ((t < 4) ? 2 * t : 2 * (t - 4) + 1) : t;
            float y = ldexpf(u[off], -E);
            if (int4_order && (off & 1)) y *= 0.0625f;
            h[t] = (_Float16)y;
            l[t] = (_Float16)(y - (float)h[t]);
            any |= (l[t] != (_Float16)0.0f);
        }
        const size_t base = (size_t)r * ngp * 32 + (size_t)slot * 8;
        *(half8v *)(hi + base) = (half8v){h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
        *(half8v *)(lo + base) = (half8v){l[0], l[1], l[2], l[3], l[4], l[5], l[6], l[7]};
    };
#pragma unroll
    for (int i = 0; i < COLI_PREP_SLOTS; i++)
        if (i % nchunk == chunk) convert(threadIdx.x + 256 * i, v[i]);
    for (int i = COLI_PREP_SLOTS; 256 * i < nslot; i++) {
        if (i % nchunk != chunk) continue;
        const int slot = threadIdx.x + 256 * i;
        float u[8];
        load_slot(slot, u);
        convert(slot, u);
    }
    // every block with a lo part raises the flag; once one has, the others
    // see it and skip their atomic (thousands of blocks on one address
    // serialize: 4096 rows took 53 us instead of 6)
    if (__syncthreads_or(any) && threadIdx.x == 0 &&
        __hip_atomic_load(haslo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gen)
        atomicMax(haslo, gen);
}
