// gemv.hip -- dequant-fused quantized expert GEMV/GEMM for gfx950 (CDNA4).
//
// y[b, o] = sum_g scale[o, g] * sum_{k in g} x[b, k] * w[o, k]
//
// int4-g32 (fmt=4/2; w = nibble - 8, c/quant.h:168-202) and MXFP4 (fmt=7;
// w = e2m1, scale = e8m0 via (u32)s << 23, c/quant.h:1391-1440) share one
// kernel skeleton, built for the HBM roofline of batch 1..16 decode:
//
//  * Weights stream once from HBM as 1 KiB tiles (16 rows x 128 columns), one
//    global_load_dwordx4 per lane per tile (see coli_hip_internal.h).
//  * Each 32-column group is one v_mfma_f32_16x16x32_f16: A = activations
//    (batch rows in M, zero-padded to 16), B = the weight group unpacked in
//    registers to exact fp16 values, so the per-group scale is applied once
//    per (row, batch) output instead of once per weight.
//      int4: v_perm_b32 drops each nibble into the mantissa of 1024.0 (low
//            nibbles) or at 16x (high nibbles), one v_pk_add_f16 removes the
//            1032 / 1152 bias -> exact (u-8) and 16(u-8); the activation of the
//            high-nibble columns is pre-scaled by 1/16 (exact).
//      fp4:  v_cvt_scalef32_pk_f16_fp4 (scale 1.0) decodes two codes per op.
//  * Activations arrive as fp16 hi + lo fragments of x * 2^-E (E = per-row
//    exponent, exact), i.e. ~22 significant bits; the lo MFMA is skipped when
//    every lo part is zero (bf16-exact inputs).
//  * K is split across the waves of a workgroup (LDS reduction in fixed wave
//    order) and, for shapes whose rows cannot fill the chip, across
//    workgroups (the last group to arrive sums the partials in split order;
//    one launch, no atomics on the data), then fused epilogues:
//    plain store, or SwiGLU (silu(g)*u, the expression of
//    c/backend_cuda.cu:618-624) for gate/up pairs. Results are bitwise
//    reproducible run to run.
#include "coli_hip_internal.h"

#include <math.h>

#include <algorithm>
#include <cstdlib>

#include "coli_device.h"

// ---------------------------------------------------------------------------
// Upload-time repack kernels
// ---------------------------------------------------------------------------

// One thread per destination dword. Source: row-major [O][ceil(I/2)] nibbles.
__global__ void coli_repack_nibbles(const uint8_t *__restrict__ src, int O, int I,
                                   uint32_t *__restrict__ dst, int nrt, int nq,
                                   uint32_t pad_nib) {
    size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)nrt * nq * 256;
    if (d >= total) return;
    int j = (int)(d & 3), lane = (int)((d >> 2) & 63);
    size_t tile = d >> 8;
    int q = (int)(tile % nq), rt = (int)(tile / nq);
    int row = rt * 16 + (lane & 15);
    int k0 = (4 * q + j) * 32 + 8 * (lane >> 4);
    size_t rb = (size_t)(I + 1) / 2;
    uint32_t v = 0;
    if (row < O && k0 + 8 <= I) {
        const uint8_t *p = src + (size_t)row * rb + (k0 >> 1);
        v = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    } else {
        for (int t = 0; t < 8; t++) {
            int k = k0 + t;
            uint32_t n = pad_nib;
            if (row < O && k < I) {
                uint8_t b = src[(size_t)row * rb + (k >> 1)];
                n = (k & 1) ? (b >> 4) : (b & 15);
            }
            v |= n << (4 * t);
        }
    }
    dst[d] = v;
}

// int4 scales: source f32 [O][ng_src] with group size gs (0 = one per row);
// gs is a multiple of 32 here, so every 32-column group lies in one source group.
// Destination tile-ordered [rt][q][16][4] as fp16 (as_half) or f32.
__global__ void coli_repack_scales_i4(const float *__restrict__ src, int O, int I, int gs,
                                     void *__restrict__ dst, int nrt, int nq, int as_half) {
    size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)nrt * nq * 64;
    if (d >= total) return;
    int j = (int)(d & 3), r = (int)((d >> 2) & 15);
    size_t tile = d >> 6;
    int q = (int)(tile % nq), rt = (int)(tile / nq);
    int row = rt * 16 + r, g = 4 * q + j;
    float v = 0.0f;
    if (row < O && g * 32 < I) {
        if (gs <= 0) v = src[row];
        else {
            int ng = (I + gs - 1) / gs;
            v = src[(size_t)row * ng + (g * 32) / gs];
        }
    }
    if (as_half) ((_Float16 *)dst)[d] = (_Float16)v;
    else ((float *)dst)[d] = v;
}

// MXFP4 scales: source e8m0 [O][ceil(I/32)], destination [rt][q][16][4] bytes.
__global__ void coli_repack_scales_e8(const uint8_t *__restrict__ src, int O, int I,
                                     uint8_t *__restrict__ dst, int nrt, int nq) {
    size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)nrt * nq * 64;
    if (d >= total) return;
    int j = (int)(d & 3), r = (int)((d >> 2) & 15);
    size_t tile = d >> 6;
    int q = (int)(tile % nq), rt = (int)(tile / nq);
    int row = rt * 16 + r, g = 4 * q + j, ng = (I + 31) / 32;
    dst[d] = (row < O && g < ng) ? src[(size_t)row * ng + g] : (uint8_t)0;
}

// ---------------------------------------------------------------------------
// Activation fragments
// ---------------------------------------------------------------------------
// For fragment row r (source row src_row[r] of x, f32 [.., ldx]; src_row[r]
// < 0 marks an unused slot):
//   E = exponent with max|x| * 2^-E in [2^14, 2^15) (0 for an all-zero row):
//   the top of the fp16 range, so hi and lo stay normal for every value
//   within 2^-18 of the row maximum (scaled to [0.5, 1) instead, every value
//   below 2^-14 of the maximum turned subnormal and most of its contribution
//   was lost in measurement),
//   hi = fp16(x * 2^-E * m), lo = fp16(x * 2^-E * m - hi), m = 1/16 on the
//   high-nibble columns of the int4 order, else 1.
// Layout per row: [ngp groups][4 kslices][8 halves]; slot t of kslice s of
// group g holds column 32g + 8s + perm[t], perm = {0,2,4,6,1,3,5,7} (int4)
// or identity (fp4), matching the B-operand order built in the GEMV.
// nchunk 256-thread blocks per row (block = row * nchunk + chunk). Every block of a row reads the
// whole row and reduces it to its maximum (the chunks re-read it from cache),
// then converts only its own share: thread t's slots are t + 256 i, and block
// c converts those with i % chunks == c. Up to 8 slots of 8 columns per
// thread stay in registers between the maximum and the conversion; longer
// rows re-read the rest. Splitting a row over blocks shortens the serial
// conversion and store tail that one block per row would carry. Whether any lo part is non-zero is published as `gen` into
// *haslo with an atomic max: the GEMV treats any flag >= its generation as
// "lo present", so the flag never needs clearing and stays correct when a
// captured graph replays an old generation.
__global__ __launch_bounds__(256) void coli_prep_frag(ColiPrepArgs a) { prep_frag_block(a, blockIdx.x); }

// ---------------------------------------------------------------------------
// GEMV problems
// ---------------------------------------------------------------------------
enum { EPI_STORE = 0, EPI_SWIGLU = 1 };

// One pipeline stage: everything one quad (4 groups x R tiles) of one wave
// reads from memory.
template <int KIND, int R, bool LO>
struct Stage {
    u32x4 w[R];
    ScaleRegs<KIND> sc[R];
    half8v xh[4];
    half8v xl[LO ? 4 : 1];   // unused (and dead) unless the lo pass runs
    u32x4 gx;                // group exponents of the lane's four result rows (GX only)
};

#ifndef COLI_PD
#define COLI_PD 2
#endif

// Scalar-register addressing of the R row tiles one wave accumulates: every
// load below is a wave-uniform base (SGPRs) plus the lane's fixed byte offset
// (VGPR), so the per-iteration address work is scalar.
template <int KIND, int R>
struct TileRows {
    const uint8_t *w[R];   // quad 0 of the row tile, or the zero tile (dead row tile)
    const uint8_t *s[R];   // its scale block, or zeros
    int qstep[R];          // 1 for a live row tile, 0 for a dead one
};

// Main loop of one wave over its quads q = q_first + it*W, it < nit.
// A ring of PD stages: the loads of iteration it+PD-1 are issued (as one
// branch-free batch) before the math of iteration it, so up to PD-1 stages
// stay in flight while the wave computes. Iterations past the end (their
// math is skipped) read the zero tile instead of weights, and the wave's last
// activation quad again (an L2 hit): every load stays unconditional, which
// keeps the in-order vmcnt accounting exact, and no tile is fetched twice.
template <int KIND, int R>
__device__ __forceinline__ void load_weights(Stage<KIND, R, true> &sg, bool valid, int q,
                                             const TileRows<KIND, R> &rows, const void *zero, int lane) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int qq = valid ? q * rows.qstep[r] : 0;
        const uint8_t *w = valid ? rows.w[r] : (const uint8_t *)zero;
        const uint8_t *sp = valid ? rows.s[r] : (const uint8_t *)zero;
        sg.w[r] = __builtin_nontemporal_load(GPTR(u32x4, w + (size_t)qq * COLI_TILE_BYTES) + lane);
        sg.sc[r].load(sp, (size_t)qq, lane & 15);
    }
}

// The caller has already issued the weight/scale loads and the hi fragments
// of iteration 0 into st[0] (before it knew whether lo fragments exist), so
// the first requests leave the CU as early as possible. xoff = the lane's
// byte offset of its fragment row and k-slice inside xh / xl.
// GX: the fragments carry one exponent per (row, group) (emitted by the GEMV
// that produced x): gx + q * gxq holds the four group exponents of the
// lane's result rows 4 (lane / 16) + i, and each group's MFMA result is
// scaled by 2^E of its row along with the group scale.
template <int KIND, int R, int NB4, int W, bool LO, bool PEEL, bool GX = false>
__device__ __forceinline__ void gemv_quads(floatx4 (&acc)[R], Stage<KIND, R, true> (&st)[COLI_PD], int q_first, int Q1,
                                           const TileRows<KIND, R> &rows, const uint8_t *xh, const uint8_t *xl,
                                           uint32_t xoff, const void *zero, int lane, const uint8_t *gx = nullptr,
                                           size_t gxq = 0) {
    constexpr int PD = COLI_PD;
    if (q_first >= Q1) return;
    const int nit = (Q1 - q_first + W - 1) / W;
    const int q_last = q_first + (nit - 1) * W;
    auto load_x = [&](Stage<KIND, R, true> &sg, int q) {
        const uint8_t *qh = xh + (size_t)q * 256, *ql = xl + (size_t)q * 256;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sg.xh[j] = *GPTR(half8v, qh + xoff + j * 64);
            if constexpr (LO) sg.xl[j] = *GPTR(half8v, ql + xoff + j * 64);
        }
        if constexpr (GX) sg.gx = *GPTR(u32x4, gx + (size_t)q * gxq);
    };
    auto load = [&](Stage<KIND, R, true> &sg, int it) {
        const bool valid = it < nit;
        const int q = q_first + it * W;
        load_weights<KIND, R>(sg, valid, q, rows, zero, lane);
        load_x(sg, valid ? q : q_last);
    };
    auto compute = [&](const Stage<KIND, R, true> &sg) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float f[NB4];
            if constexpr (GX) {
#pragma unroll
                for (int i = 0; i < NB4; i++) f[i] = gexp_pow2(sg.gx[i], j);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                half8v bw = unpack_b<KIND>(sg.w[r][j]);
                floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(sg.xh[j], bw, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                if constexpr (LO) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(sg.xl[j], bw, d, 0, 0, 0);
                float scl = sg.sc[r].get(j);
#pragma unroll
                for (int i = 0; i < NB4; i++) acc[r][i] = fmaf(d[i], GX ? scl * f[i] : scl, acc[r][i]);
            }
        }
    };
    if constexpr (LO) {
        const uint8_t *ql = xl + (size_t)q_first * 256;
#pragma unroll
        for (int j = 0; j < 4; j++) st[0].xl[j] = *GPTR(half8v, ql + xoff + j * 64);
    }
    if constexpr (GX) st[0].gx = *GPTR(u32x4, gx + (size_t)q_first * gxq);
    if constexpr (PEEL) {
        // Two-stage ring unrolled by two, with a tail that issues no load past
        // the wave's last quad. Every path leaves the loop with the same loads
        // outstanding, so the compiler's vmcnt waits stay exact. (Used where
        // its larger code keeps the register budget of two waves per SIMD.)
        static_assert(PD == 2, "the peeled loop is written for a two-stage ring");
        int it = 0;
        for (; it + 2 < nit; it += 2) {
            load(st[1], it + 1);
            compute(st[0]);
            load(st[0], it + 2);
            compute(st[1]);
        }
        if (it + 1 < nit) {
            load(st[1], it + 1);
            compute(st[0]);
            compute(st[1]);
        } else {
            compute(st[0]);
        }
    } else {
#pragma unroll
        for (int p = 1; p < PD - 1; p++) load(st[p], p);
        for (int it0 = 0; it0 < nit; it0 += PD) {
#pragma unroll
            for (int u = 0; u < PD; u++) {
                load(st[(u + PD - 1) % PD], it0 + u + PD - 1);
                if (it0 + u < nit) compute(st[u]);
            }
        }
    }
}

// CH consecutive row blocks of one problem in one wave's loop (CH = 2, 4):
// iterations b nit .. (b + 1) nit - 1 stream block b's quads through the same
// ring, so each block's first weights are requested while the previous
// block's last quads are computed (one descriptor read, one ring fill and one
// pipeline drain for all of them). Block b's row tiles are (rb + b) R + r,
// their addresses formed per load (dead past the matrix: the zero tile). The
// activations of the blocks are the same quads. One accumulator set runs in
// the loop; each finished block's is shifted into `done` (blocks 0 .. CH-2 in
// order), the last block's stays in acc.
template <int KIND, int R, int NB4, int W, bool LO, int CH>
__device__ __forceinline__ void gemv_quads_ch(floatx4 (&acc)[R], floatx4 (&done)[CH - 1][R],
                                             Stage<KIND, R, true> (&st)[COLI_PD], int q_first, int Q1,
                                             const ColiProb &pr, int rb, int nrt, int nq, const uint8_t *xh,
                                             const uint8_t *xl, uint32_t xoff, const void *zero, int lane) {
    constexpr int PD = COLI_PD;
    if (q_first >= Q1) return;
    const int nit = (Q1 - q_first + W - 1) / W, NIT = CH * nit;
    const int q_last = q_first + (nit - 1) * W;
    auto load_x = [&](Stage<KIND, R, true> &sg, int q) {
        const uint8_t *qh = xh + (size_t)q * 256, *ql = xl + (size_t)q * 256;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sg.xh[j] = *GPTR(half8v, qh + xoff + j * 64);
            if constexpr (LO) sg.xl[j] = *GPTR(half8v, ql + xoff + j * 64);
        }
    };
    auto load = [&](Stage<KIND, R, true> &sg, int it) {
        int blk = 0;
#pragma unroll
        for (int k = 1; k < CH; k++) blk += it >= k * nit ? 1 : 0;
        const bool valid = it < NIT;
        const int q = q_first + (it - blk * nit) * W;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int rt = (rb + blk) * R + r;
            const bool live = valid && rt < nrt;
            const size_t tq = live ? (size_t)(uint32_t)rt * (uint32_t)nq + q : 0;
            const uint8_t *w = live ? pr.w0 : (const uint8_t *)zero;
            const uint8_t *sp = live ? (const uint8_t *)pr.s0 : (const uint8_t *)zero;
            sg.w[r] = __builtin_nontemporal_load(GPTR(u32x4, w + tq * COLI_TILE_BYTES) + lane);
            sg.sc[r].load(sp, tq, lane & 15);
        }
        load_x(sg, valid ? q : q_last);
    };
    auto compute = [&](const Stage<KIND, R, true> &sg) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                half8v bw = unpack_b<KIND>(sg.w[r][j]);
                floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(sg.xh[j], bw, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                if constexpr (LO) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(sg.xl[j], bw, d, 0, 0, 0);
                const float scl = sg.sc[r].get(j);
#pragma unroll
                for (int i = 0; i < NB4; i++) acc[r][i] = fmaf(d[i], scl, acc[r][i]);
            }
        }
    };
    if constexpr (LO) {
        const uint8_t *ql = xl + (size_t)q_first * 256;
#pragma unroll
        for (int j = 0; j < 4; j++) st[0].xl[j] = *GPTR(half8v, ql + xoff + j * 64);
    }
#pragma unroll
    for (int p = 1; p < PD - 1; p++) load(st[p], p);
    for (int it0 = 0; it0 < NIT; it0 += PD) {
#pragma unroll
        for (int u = 0; u < PD; u++) {
            load(st[(u + PD - 1) % PD], it0 + u + PD - 1);
            const int it = it0 + u;
            if (it < NIT) compute(st[u]);
            if (it + 1 < NIT && (it + 1) % nit == 0) {
#pragma unroll
                for (int b = 0; b + 1 < CH - 1; b++)
#pragma unroll
                    for (int r = 0; r < R; r++) done[b][r] = done[b + 1][r];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    done[CH - 2][r] = acc[r];
                    acc[r] = (floatx4){0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    }
}

// One workgroup (W waves) = one work item: (problem, batch tile, row block,
// K split). The W waves interleave over the item's quads (wave w takes quads
// Q0+w, Q0+w+W, ...) so the group streams contiguous tile memory together,
// then reduce through LDS in fixed wave order: K is split inside the group,
// which needs no device-scope synchronization. A cross-group split (splits
// > 1) exists only for shapes too small to fill the chip otherwise; it uses a
// fixed-order reduction by the last-arriving group.
// R = row tiles accumulated per wave; DUAL: tiles [0, R/2) come from w0
// (gate) and [R/2, R) from w1 (up) over the same rows. NB4 = accumulator rows
// per lane that can hold real batch rows (1, 2 or 4): the MFMA result row of
// lane l, register i is batch row 4*(l/16)+i, its column is output row
// 16*tile + (l%16).
// INL: the single problem a.prob0 (a.prob null, a.nprob 1, a.nprob_dev null):
// no check precedes the first weight loads, so the kernel arguments arrive
// as one batch of scalar loads and the HBM requests follow at once (early
// exits split the scalar loads into dependent round trips).
// The MXFP4 gate/up pairs on device descriptors with two or four waves (the
// MoE layers of 2-21 rows) are held to 168 VGPRs, three waves a SIMD instead
// of two at 176: a few registers spill, and the layers still ran faster (DSV3
// B16 460 -> 444 us, 21-row verification 603 -> 564 us, four waves). The
// plain (down) matrices keep two waves without spills (DSV3 B8 282 -> 274 us,
// B16 454 -> 440 us against three); int4 spills more and keeps two.
// CH > 1 (device descriptors, plain matrices, no K split): each workgroup
// runs CH consecutive row blocks of its problem back to back in one loop.
template <int KIND, int R, bool DUAL, int NB4, int W, bool INL, int CH = 1>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(KIND == COLI_KIND_FP4 && W <= 4 && !INL && DUAL ? 3 : (CH > 1 ? 2 : 1), 8))) void coli_gemv_tiles(ColiGemvArgs a) {
    static_assert(CH == 1 || (!INL && !DUAL), "chained row blocks: device descriptors, plain matrices");
    constexpr int RT = DUAL ? R / 2 : R;
    __shared__ float red[W][R * NB4][64];
    __shared__ int split_last;
    // readfirstlane: the wave index is wave-uniform, so everything derived from it
    // (tile indices, validity, base pointers) stays in scalar registers.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // INL launches a 3-D grid (row block, split, batch tile): no index
    // arithmetic on kernel arguments precedes the first loads.
    int p = 0, bt, rb, s;
    ColiProb pdesc;
    if constexpr (INL) {
        rb = blockIdx.x;
        s = blockIdx.y;
        bt = blockIdx.z;
    } else {
        const int item = blockIdx.x;
        const int items_per_bt = CH > 1 ? (a.rb_per_prob + CH - 1) / CH : a.rb_per_prob * a.splits;
        const int items_per_p = a.n_bt * items_per_bt;
        p = item / items_per_p;
        if (p >= a.nprob) return;
        // the descriptor (inside the array: p < nprob) and the live count are
        // read together, one memory round trip before the weight loads
        pdesc = a.prob[p];
        if (a.nprob_dev && p >= *a.nprob_dev) return;
        int rem = item - p * items_per_p;
        bt = rem / items_per_bt;
        rem -= bt * items_per_bt;
        if constexpr (CH > 1) {
            rb = CH * rem;
            s = 0;
        } else {
            rb = rem / a.splits;
            s = rem - rb * a.splits;
        }
    }
    const ColiProb pr = uniform_prob(INL ? a.prob0 : pdesc);
    const int nb = min(16, pr.nrows - 16 * bt);
    if constexpr (!INL) {
        if (nb <= 0) return;
    }

    const int b = lane & 15, ks = lane >> 4;
    const int Q0 = s * a.qps, Q1 = min(a.nq, Q0 + a.qps);

    // Row tiles past the matrix read the zero tile (zero scale: no contribution).
    int rt[R];
    bool live[R];
    TileRows<KIND, R> rows;
#pragma unroll
    for (int r = 0; r < R; r++) {
        int rr = DUAL ? (r % RT) : r;
        rt[r] = rb * RT + rr;
        live[r] = rt[r] < a.nrt;
        const bool second = DUAL && r >= RT;
        // (branch-free: the clamped row tile is computed either way)
        const size_t t0 = (size_t)(uint32_t)min(rt[r], a.nrt - 1) * (uint32_t)a.nq;
        const uint8_t *wl = (second ? pr.w1 : pr.w0) + t0 * COLI_TILE_BYTES;
        const uint8_t *sl = (const uint8_t *)(second ? pr.s1 : pr.s0) + t0 * ScaleRegs<KIND>::kTileBytes;
        rows.w[r] = live[r] ? wl : (const uint8_t *)a.zero;
        rows.s[r] = live[r] ? sl : (const uint8_t *)a.zero;
        rows.qstep[r] = live[r] ? 1 : 0;
    }
    // the first weight stage goes out before anything else is resolved
    Stage<KIND, R, true> st[COLI_PD];
    const int q_first = Q0 + wave;
    load_weights<KIND, R>(st[0], q_first < Q1, q_first, rows, a.zero, lane);
    // Lanes past the problem's rows read the last real row: MFMA output rows
    // are independent, and those rows are never stored.
    const int br_lane = pr.xrow_off + 16 * bt + min(b, nb - 1);
    const int fr = a.xrows ? a.xrows[br_lane] : br_lane;
    const uint32_t xoff = ((uint32_t)fr * (uint32_t)a.xstride + ks * 8) * 2;
    const uint8_t *xh = (const uint8_t *)a.xhi, *xl = (const uint8_t *)a.xlo;
    if (q_first < Q1) {
        const uint8_t *qh = xh + (size_t)q_first * 256;
#pragma unroll
        for (int j = 0; j < 4; j++) st[0].xh[j] = *GPTR(half8v, qh + xoff + j * 64);
    }

    const bool use_lo = *a.haslo >= a.lo_gen;  // >=: stays correct under graph replay
    // emitted fragments: exponents per (row, group), read with the fragments
    const bool gx = INL && !DUAL && a.gexp;
    const uint8_t *gxp = gx ? a.gexp + ((size_t)pr.xrow_off + 16 * bt + 4 * ks) * 4 : nullptr;
    const size_t gxq = (size_t)a.gexp_rows * 4;
    // exponents of the batch rows this wave finishes (used after the loop):
    // result registers wave, wave + W, ... (one unless W < NB4)
    constexpr int NI = (NB4 + W - 1) / W;
    int E_out[NI];
#pragma unroll
    for (int k = 0; k < NI; k++) {
        E_out[k] = 0;
        const int ii = wave + k * W;
        if (!gx && ii < NB4) {   // (with a K split only the last arriver uses it)
            const int brow = ks * 4 + ii;
            if (brow < nb) {
                const int br = pr.xrow_off + 16 * bt + brow;
                E_out[k] = a.xexp[a.xrows ? a.xrows[br] : br];
            }
        }
    }

    floatx4 acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = (floatx4){0.f, 0.f, 0.f, 0.f};
    // the peeled loop fits two waves per SIMD only in these variants
    constexpr bool PEEL = INL && W == 8 && KIND == COLI_KIND_I4_H && R >= 2;
    // reduction in fixed wave order and the epilogue of one row block (the
    // chained form, CH > 1: no K split)
    auto finish_block = [&](const floatx4 (&ac)[R], const int (&rtb)[R], const bool (&liveb)[R]) {
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int i = 0; i < NB4; i++) red[wave][r * NB4 + i][lane] = ac[r][i];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int ii = wave + k * W;
            if (ii >= NB4) break;
            float vv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                float t = red[0][r * NB4 + ii][lane];
#pragma unroll
                for (int w = 1; w < W; w++) t += red[w][r * NB4 + ii][lane];
                vv[r] = t;
            }
            gemv_epilogue<R, DUAL>(a, pr, bt, rtb, liveb, vv, ks * 4 + ii, lane, E_out[k]);
        }
    };
    if constexpr (INL && !DUAL) {
        if (gx) {
            // emitted fragments are f32 rows: their lo parts are always taken
            gemv_quads<KIND, R, NB4, W, true, PEEL, true>(acc, st, q_first, Q1, rows, xh, xl, xoff, a.zero, lane, gxp,
                                                          gxq);
        } else if (use_lo) {
            gemv_quads<KIND, R, NB4, W, true, PEEL>(acc, st, q_first, Q1, rows, xh, xl, xoff, a.zero, lane);
        } else {
            gemv_quads<KIND, R, NB4, W, false, PEEL>(acc, st, q_first, Q1, rows, xh, xl, xoff, a.zero, lane);
        }
    } else if constexpr (CH > 1) {
        floatx4 done[CH - 1][R];
#pragma unroll
        for (int b = 0; b < CH - 1; b++)
#pragma unroll
            for (int r = 0; r < R; r++) done[b][r] = (floatx4){0.f, 0.f, 0.f, 0.f};
        if (use_lo)
            gemv_quads_ch<KIND, R, NB4, W, true, CH>(acc, done, st, q_first, Q1, pr, rb, a.nrt, a.nq, xh, xl, xoff,
                                                     a.zero, lane);
        else
            gemv_quads_ch<KIND, R, NB4, W, false, CH>(acc, done, st, q_first, Q1, pr, rb, a.nrt, a.nq, xh, xl, xoff,
                                                      a.zero, lane);
#pragma unroll
        for (int b = 0; b < CH; b++) {
            int rtb[R];
            bool liveb[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                rtb[r] = (rb + b) * R + r;
                liveb[r] = rtb[r] < a.nrt;
            }
            if (b > 0) __syncthreads();   // the reduction buffer is reused
            if (b < CH - 1) finish_block(done[b], rtb, liveb);
            else finish_block(acc, rtb, liveb);
        }
        return;
    } else {
        if (use_lo) gemv_quads<KIND, R, NB4, W, true, PEEL>(acc, st, q_first, Q1, rows, xh, xl, xoff, a.zero, lane);
        else gemv_quads<KIND, R, NB4, W, false, PEEL>(acc, st, q_first, Q1, rows, xh, xl, xoff, a.zero, lane);
    }

    // ---- intra-group reduction in fixed wave order; wave i finishes register i ----
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int i = 0; i < NB4; i++) red[wave][r * NB4 + i][lane] = acc[r][i];
    __syncthreads();
    if constexpr (W < NB4) {
        // fewer waves than result registers (never with a K split across
        // groups): each wave finishes registers wave, wave + W, ...
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int ii = wave + k * W;
            if (ii >= NB4) break;
            float vv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                float t = red[0][r * NB4 + ii][lane];
#pragma unroll
                for (int w = 1; w < W; w++) t += red[w][r * NB4 + ii][lane];
                vv[r] = t;
            }
            gemv_epilogue<R, DUAL>(a, pr, bt, rt, live, vv, ks * 4 + ii, lane, E_out[k]);
        }
        return;
    }
    const int i = wave;
    float v[R];
    if (i < NB4) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            float t = red[0][r * NB4 + i][lane];
#pragma unroll
            for (int w = 1; w < W; w++) t += red[w][r * NB4 + i][lane];
            v[r] = t;
        }
    }

    // ---- split K across groups: publish the partial; the last group of the
    // instance to arrive sums all partials in split order (deterministic) and
    // runs the epilogue. The groups of one instance may sit on different XCDs,
    // whose L2s are not coherent with each other: partials are written and
    // read as agent-scope atomics (coherent by themselves, no whole-cache
    // writeback or invalidate), and every group waits for its stores to
    // complete before it counts its arrival. The counter is reset by the last
    // group, so it is zero again for the next launch.
    if (a.splits > 1) {
        const size_t inst = ((size_t)p * a.n_bt + bt) * a.rb_per_prob + rb;
        const size_t pbase = (inst * a.splits * R * NB4 + i) * 64 + lane;
        if (i < NB4) {
#pragma unroll
            for (int r = 0; r < R; r++)
                __hip_atomic_store(a.partial + pbase + ((size_t)s * R + r) * NB4 * 64, v[r], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            const int old = __hip_atomic_fetch_add(a.split_cnt + inst, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            split_last = old == a.splits - 1;
            if (split_last) __hip_atomic_store(a.split_cnt + inst, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!split_last || i >= NB4) return;
#pragma unroll
        for (int r = 0; r < R; r++) v[r] = 0.0f;
        // the partials of up to eight splits requested together (one memory
        // round trip), then summed in split order
        constexpr int SB = 8;
        for (int s0 = 0; s0 < a.splits; s0 += SB) {
            float pv[SB][R];
#pragma unroll
            for (int ss = 0; ss < SB; ss++)
#pragma unroll
                for (int r = 0; r < R; r++)
                    pv[ss][r] = s0 + ss < a.splits
                                    ? __hip_atomic_load(a.partial + pbase + ((size_t)(s0 + ss) * R + r) * NB4 * 64,
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                    : 0.0f;
#pragma unroll
            for (int ss = 0; ss < SB; ss++)
#pragma unroll
                for (int r = 0; r < R; r++)
                    if (s0 + ss < a.splits) v[r] += pv[ss][r];
        }
    }
    if (i >= NB4) return;
    gemv_epilogue<R, DUAL>(a, pr, bt, rt, live, v, ks * 4 + i, lane, E_out[0]);
}

// ---------------------------------------------------------------------------
// Generic int4 kernel: any group size (incl. ones that are not a multiple of
// 32), source layout, reference group semantics (c/quant.h:168-202). One
// 256-thread block per (output row, batch row).
// ---------------------------------------------------------------------------
__global__ void coli_gemv_generic_i4(const uint8_t *__restrict__ w, const float *__restrict__ sc,
                                     int I, int O, int gs, const float *__restrict__ x, int ldx,
                                     float *__restrict__ y, int ldy) {
    int o = blockIdx.x, s = blockIdx.y;
    int rb = (I + 1) / 2, egs = gs > 0 ? gs : I, ng = (I + egs - 1) / egs;
    const uint8_t *row = w + (size_t)o * rb;
    const float *scl = sc + (size_t)o * ng;
    const float *xs = x + (size_t)s * ldx;
    float sum = 0.0f;
    for (int g = threadIdx.x; g < ng; g += blockDim.x) {
        int base = g * egs, end = min(I, base + egs);
        float part = 0.0f;
        for (int k = base; k < end; k++) {
            uint8_t v = row[k >> 1];
            int n = (k & 1) ? (v >> 4) : (v & 15);
            part = fmaf(xs[k], (float)(n - 8), part);
        }
        sum = fmaf(part, scl[g], sum);
    }
    __shared__ float red[256];
    red[threadIdx.x] = sum;
    __syncthreads();
    for (int st = 128; st; st >>= 1) {
        if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
        __syncthreads();
    }
    if (!threadIdx.x) y[(size_t)s * ldy + o] = red[0];
}


// ---------------------------------------------------------------------------
// e4m3 activation quantize-dequantize, one e8m0 scale per 128-column block
// (the native_quant contract, c/deepseek_v4.c:10495-10520), bit-exact: the
// block max, the power-of-two scale, the division by it and the
// round-to-nearest-even e4m3 encode are all exact operations.
// ---------------------------------------------------------------------------
__device__ float e4m3_qdq_value(float v) {
    // v already clamped to [-448, 448]; returns decode(encode(v)).
    if (v != v) return v;
    float mag = fabsf(v);
    float out;
    if (mag == 0.0f) {
        out = 0.0f;
    } else if (mag < 0.015625f) {
        float scaled = mag * 512.0f;
        uint32_t whole = (uint32_t)scaled;
        float frac = scaled - (float)whole;
        if (frac > 0.5f || (frac == 0.5f && (whole & 1u))) whole++;
        out = (float)whole * (1.0f / 512.0f);
    } else {
        uint32_t bits = __builtin_bit_cast(uint32_t, mag);
        int e = (int)((bits >> 23) & 0xff) - 127;
        uint32_t sig = 0x800000u | (bits & 0x7fffffu);
        uint32_t keep = sig >> 20, rest = sig & 0xfffffu;
        if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) keep++;
        out = ldexpf((float)keep, e - 3);
        if (out > 448.0f) out = 448.0f;   // 0x7e saturation
    }
    return signbit(v) ? -out : out;
}

__global__ __launch_bounds__(128) void coli_qdq_e4m3(const float *__restrict__ x, float *__restrict__ y, int K) {
    int blk = blockIdx.x, s = blockIdx.y, k = blk * 128 + threadIdx.x;
    const float *xr = x + (size_t)s * K;
    float v = k < K ? xr[k] : 0.0f;
    __shared__ float red[128];
    red[threadIdx.x] = k < K ? fabsf(v) : 0.0f;
    __syncthreads();
    for (int st = 64; st; st >>= 1) {
        if (threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
        __syncthreads();
    }
    float mx = fmaxf(red[0], 1e-4f);
    int e;
    float f = frexpf(mx / 448.0f, &e);
    int se = f == 0.5f ? e - 1 : e;
    se = se < -127 ? -127 : (se > 127 ? 127 : se);
    float sc = ldexpf(1.0f, se);
    if (k < K) {
        float q = fmaxf(-448.0f, fminf(448.0f, v / sc));
        y[(size_t)s * K + k] = e4m3_qdq_value(q) * sc;
    }
}

// ---------------------------------------------------------------------------
// int8 activation quantize-dequantize per 32-column group (the activation
// side of c/quant.h:1441-1515, matmul_mxfp4_i8): sc = max|x| / 127 floored
// at 1e-20, q = nearest-even integer of x * (1 / sc) clamped to +-127, and
// the GEMV then reads q * sc. Division, reciprocal and rounding are the
// correctly rounded IEEE operations the reference uses, so q is bit-exact;
// q * sc differs from the reference's post-dot scaling by one rounding per
// element (2^-24 relative).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void coli_qdq_i8(const float *__restrict__ x, float *__restrict__ y, int S, int K) {
    const int ng = K / 32;
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)S * ng) return;
    const float *xg = x + t * 32;
    float v[32];
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        const floatx4 a = *GPTR(floatx4, xg + i);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[i + j] = a[j];
            am = fmaxf(am, fabsf(a[j]));
        }
    }
    float sc = __fdiv_rn(am, 127.0f);
    if (sc < 1e-20f) sc = 1e-20f;
    const float inv = __fdiv_rn(1.0f, sc);
    float *yg = y + t * 32;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        floatx4 o;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float q = fminf(127.0f, fmaxf(-127.0f, __builtin_rintf(__fmul_rn(v[i + j], inv))));
            o[j] = __fmul_rn(q, sc);
        }
        *(floatx4 *)(yg + i) = o;
    }
}

// ---------------------------------------------------------------------------
// Host-side launchers (called from backend_hip.hip)
// ---------------------------------------------------------------------------
struct ColiGemvPlan {
    int R, dual, nb4;
};

// Plain matrices on device descriptors with two-wave groups (the MoE down
// projections) run two row blocks per workgroup (DSV3 B16 layer 430.7 ->
// 424.8 us, 21-row step 550.6 -> 538.4 us MXFP4, 655.7 -> 635.9 us int4;
// four blocks spilled registers and were slower: B16 464 us);
// COLI_HIP_CHAIN=0: one.
static int chain_blocks() {
    const char *e = std::getenv("COLI_HIP_CHAIN");
    return e && e[0] == '0' ? 1 : 2;
}

// 16-wave groups only for R <= 2: at R = 4 the 128-VGPR budget of a
// 1024-thread group would spill.
template <int KIND, int R, bool DUAL, int NB4>
static hipError_t launch_w(const ColiGemvArgs &a, int W, int blocks, hipStream_t st) {
    const bool inl = a.prob == nullptr;
    const dim3 grid = inl ? dim3(a.rb_per_prob, a.splits, a.n_bt) : dim3(blocks);
    if constexpr (R <= 2) {
        if (W == 16) {
            if (inl) hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 16, true>), grid, dim3(1024), 0, st, a);
            else hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 16, false>), grid, dim3(1024), 0, st, a);
            return hipGetLastError();
        }
    }
    // two waves: on device descriptors and without a K split only (the
    // split protocol has each wave finish one result register)
    if (W == 2 && !inl && a.splits == 1) {
        if constexpr (!DUAL && R == 4) {
            const int ch = chain_blocks();
            if (ch > 1) {
                const long groups = (long)a.nprob * a.n_bt * ((a.rb_per_prob + ch - 1) / ch);
                hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 2, false, 2>), dim3((unsigned)groups),
                                   dim3(128), 0, st, a);
                return hipGetLastError();
            }
        }
        hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 2, false>), grid, dim3(128), 0, st, a);
        return hipGetLastError();
    }
    if (W >= 8) {
        if (inl) hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 8, true>), grid, dim3(512), 0, st, a);
        else hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 8, false>), grid, dim3(512), 0, st, a);
    } else {
        if (inl) hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 4, true>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((coli_gemv_tiles<KIND, R, DUAL, NB4, 4, false>), grid, dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <int KIND, int R, bool DUAL>
static hipError_t launch_nb(const ColiGemvArgs &a, int nb4, int W, int blocks, hipStream_t st) {
    if (nb4 == 1) return launch_w<KIND, R, DUAL, 1>(a, W, blocks, st);
    if (nb4 == 2) return launch_w<KIND, R, DUAL, 2>(a, W, blocks, st);
    return launch_w<KIND, R, DUAL, 4>(a, W, blocks, st);
}

template <int KIND>
static hipError_t launch_kind(const ColiGemvArgs &a, int R, bool dual, int nb4, int W, int blocks, hipStream_t st) {
    if (dual) {
        if (R == 4) return launch_nb<KIND, 4, true>(a, nb4, W, blocks, st);
        return launch_nb<KIND, 2, true>(a, nb4, W, blocks, st);
    }
    if (R == 4) return launch_nb<KIND, 4, false>(a, nb4, W, blocks, st);
    if (R == 2) return launch_nb<KIND, 2, false>(a, nb4, W, blocks, st);
    return launch_nb<KIND, 1, false>(a, nb4, W, blocks, st);
}

extern "C" hipError_t coli_launch_gemv(int kind, const ColiGemvArgs *a, int R, int dual, int W, int max_rows,
                                       hipStream_t st) {
    int nb4 = max_rows <= 1 ? 1 : (max_rows <= 2 ? 2 : 4);
    if (!a->prob && (a->nprob != 1 || a->nprob_dev)) return hipErrorInvalidValue;   // inline problem: exactly one
    if (a->xf) return hipErrorInvalidValue;   // this kernel reads prepared fragments only
    long items = (long)a->nprob * a->n_bt * a->rb_per_prob * a->splits;
    int blocks = (int)items;
    if (blocks <= 0) return hipSuccess;
    switch (kind) {
    case COLI_KIND_I4_H: return launch_kind<COLI_KIND_I4_H>(*a, R, dual, nb4, W, blocks, st);
    case COLI_KIND_I4_F: return launch_kind<COLI_KIND_I4_F>(*a, R, dual, nb4, W, blocks, st);
    case COLI_KIND_FP4: return launch_kind<COLI_KIND_FP4>(*a, R, dual, nb4, W, blocks, st);
    default: return hipErrorInvalidValue;
    }
}

// args_only: the launch's arguments are returned instead (the build then runs
// inside another launch, prep_frag_block); nblocks 0 when there is nothing.
extern "C" hipError_t coli_launch_prep_frag(const float *x, int ldx, const int *src_row,
                                            const int *nrows_dev, int nrows, int K, int ngp,
                                            int int4_order, _Float16 *hi, _Float16 *lo,
                                            int *exp2out, int *haslo, int gen, const void *zero,
                                            hipStream_t st, ColiPrepArgs *args_only) {
    if (args_only) args_only->nblocks = 0;
    if (nrows <= 0) return hipSuccess;
    const int vec = ((uintptr_t)x % 16 == 0) && (ldx % 4 == 0) && (K % 8 == 0);
    // chunks per row: one per 256 slots (2048 columns), fewer when many rows
    // already fill the chip
    int nchunk = (ngp * 4 + 255) / 256;
    const char *e = std::getenv("COLI_HIP_PREP_CHUNKS");
    if (e) nchunk = std::max(1, std::min(nchunk, std::atoi(e)));
    else if (nrows >= 64) nchunk = 1;
    ColiPrepArgs a;
    a.x = x;
    a.src_row = src_row;
    a.nrows_dev = nrows_dev;
    a.hi = hi;
    a.lo = lo;
    a.exp2out = exp2out;
    a.haslo = haslo;
    a.zero = (const float *)zero;
    a.ldx = ldx;
    a.K = K;
    a.ngp = ngp;
    a.int4_order = int4_order;
    a.gen = gen;
    a.vec = vec;
    a.nchunk = nchunk;
    a.nblocks = nrows * nchunk;
    if (args_only) {
        *args_only = a;
        return hipSuccess;
    }
    hipLaunchKernelGGL(coli_prep_frag, dim3((unsigned)a.nblocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

extern "C" hipError_t coli_launch_repack(const ColiCudaTensor *t, const uint8_t *src_w,
                                         const void *src_s, hipStream_t st) {
    size_t nd = (size_t)t->nrt * t->nq * 256;
    hipLaunchKernelGGL(coli_repack_nibbles, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, st,
                       src_w, t->O, t->I, (uint32_t *)t->w, t->nrt, t->nq,
                       t->kind == COLI_KIND_FP4 ? 0u : 8u);
    size_t ns = (size_t)t->nrt * t->nq * 64;
    if (t->kind == COLI_KIND_FP4)
        hipLaunchKernelGGL(coli_repack_scales_e8, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, st,
                           (const uint8_t *)src_s, t->O, t->I, (uint8_t *)t->sc, t->nrt, t->nq);
    else
        hipLaunchKernelGGL(coli_repack_scales_i4, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, st,
                           (const float *)src_s, t->O, t->I, t->gs, t->sc, t->nrt, t->nq,
                           t->kind == COLI_KIND_I4_H ? 1 : 0);
    return hipGetLastError();
}

extern "C" hipError_t coli_launch_generic_i4(const ColiCudaTensor *t, const float *x, int ldx,
                                             float *y, int ldy, int S, hipStream_t st) {
    hipLaunchKernelGGL(coli_gemv_generic_i4, dim3(t->O, S), dim3(256), 0, st, t->w,
                       (const float *)t->sc, t->I, t->O, t->gs, x, ldx, y, ldy);
    return hipGetLastError();
}

extern "C" hipError_t coli_launch_qdq_e4m3(const float *x, float *y, int S, int K, hipStream_t st) {
    hipLaunchKernelGGL(coli_qdq_e4m3, dim3((K + 127) / 128, S), dim3(128), 0, st, x, y, K);
    return hipGetLastError();
}

extern "C" hipError_t coli_launch_qdq_i8(const float *x, float *y, int S, int K, hipStream_t st) {
    if (K % 32 || S <= 0) return K % 32 ? hipErrorInvalidValue : hipSuccess;
    const long n = (long)S * (K / 32);
    hipLaunchKernelGGL(coli_qdq_i8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, S, K);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fmt=2 with int8 activations (the IDOT path, c/colibri.c:937-945): qrow_i8
// per row (c/quant.h:581-586), then y = (float)(integer dot) * scale[o] *
// sx[s] (matmul_i4_idot, c/quant.h:924-933). On the device the integer dot
// runs on the regular GEMV: the int8 values enter as exact fp16 activation
// fragments (exponent 0, no lo part), the tensor's group scales are replaced
// by ones, and every MFMA result and partial sum is an integer below 2^24
// (|sum| <= 8 * 127 * I, I <= 16512), so the f32 accumulation is exact in any
// order; the two scale products follow in the reference's order.
// ---------------------------------------------------------------------------
// One 256-thread block per row: the row's maximum, s = max / 127 (at least
// 1e-12), inv = 1 / s, q = rint(x * inv) as fp16 fragments in the GEMV's
// A-operand order (columns past K are zero), exponent 0; sx[row] = s.
__global__ __launch_bounds__(256) void coli_qrow_i8_frag(const float *__restrict__ x, int ldx, int K, int ngp,
                                                         int int4_order, _Float16 *__restrict__ hi,
                                                         int *__restrict__ exp2out, float *__restrict__ sx) {
    const int r = blockIdx.x;
    const float *xr = x + (size_t)r * ldx;
    float m = 0.0f;
    for (int k = threadIdx.x; k < K; k += 256) m = fmaxf(m, fabsf(xr[k]));
#pragma unroll
    for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float wmax[4];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    float s = m / 127.f;
    if (s < 1e-12f) s = 1e-12f;
    const float inv = 1.f / s;
    if (threadIdx.x == 0) {
        exp2out[r] = 0;
        sx[r] = s;
    }
    const int nslot = ngp * 4;
    for (int slot = threadIdx.x; slot < nslot; slot += 256) {
        half8v h;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int off = int4_order ? ((t < 4) ? 2 * t : 2 * (t - 4) + 1) : t;
            const int k = slot * 8 + off;
            float q = k < K ? rintf(xr[k] * inv) : 0.0f;
            if (int4_order && (off & 1)) q *= 0.0625f;   // exact: |q| <= 128
            h[t] = (_Float16)q;
        }
        *(half8v *)(hi + (size_t)r * ngp * 32 + (size_t)slot * 8) = h;
    }
}

__global__ void coli_fill_u16(uint16_t *p, size_t n, uint16_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}
__global__ void coli_fill_f32(float *p, size_t n, float v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// y[s, o] = (yi[s, o] * scale[o]) * sx[s], scale[o] read from the tensor's
// tile-ordered group scales (group 0 of row o: fmt=2 scales are per row).
__global__ void coli_idot_scale(float *__restrict__ y, const float *__restrict__ yi, const float *__restrict__ sx,
                                const void *__restrict__ sc, int half_scales, int nq, int O) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x, s = blockIdx.y;
    if (o >= O) return;
    const size_t e = ((size_t)(o >> 4) * nq * 16 + (o & 15)) * 4;   // tile (o / 16, quad 0), row o % 16, group 0
    const float so = half_scales ? (float)((const _Float16 *)sc)[e] : ((const float *)sc)[e];
    y[(size_t)s * O + o] = (yi[(size_t)s * O + o] * so) * sx[s];
}

extern "C" hipError_t coli_launch_qrow_i8_frag(const float *x, int ldx, int nrows, int K, int ngp, int int4_order,
                                               _Float16 *hi, int *exp2out, float *sx, hipStream_t st) {
    if (nrows <= 0) return hipSuccess;
    hipLaunchKernelGGL(coli_qrow_i8_frag, dim3(nrows), dim3(256), 0, st, x, ldx, K, ngp, int4_order, hi, exp2out,
                       sx);
    return hipGetLastError();
}

// Ones in the tensor's scale format (fp16 or f32), n scale entries.
extern "C" hipError_t coli_launch_unit_scales(void *sc, size_t n, int half_scales, hipStream_t st) {
    if (half_scales)
        hipLaunchKernelGGL(coli_fill_u16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (uint16_t *)sc, n,
                           (uint16_t)0x3C00u);
    else
        hipLaunchKernelGGL(coli_fill_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (float *)sc, n, 1.0f);
    return hipGetLastError();
}

extern "C" hipError_t coli_launch_idot_scale(float *y, const float *yi, const float *sx, const void *sc,
                                             int half_scales, int nq, int O, int S, hipStream_t st) {
    hipLaunchKernelGGL(coli_idot_scale, dim3((O + 255) / 256, S), dim3(256), 0, st, y, yi, sx, sc, half_scales, nq,
                       O);
    return hipGetLastError();
}

// 16-row interleave of coli_fp4_pack_rows16_v10 (c/deepseek_v4.c:10975-10993)
// back to row-major bytes: row r, byte c <- packed[((r / 16) * nb + c) * 16 + r % 16]
// (nb bytes per row), one thread per destination byte.
__global__ void coli_rows16_to_rows(const uint8_t *__restrict__ packed, uint8_t *__restrict__ rows, int O, int nb) {
    const size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= (size_t)O * nb) return;
    const size_t r = d / nb, c = d - r * nb;
    rows[d] = packed[((r >> 4) * nb + c) * 16 + (r & 15)];
}

extern "C" hipError_t coli_launch_rows16_to_rows(const uint8_t *packed, uint8_t *rows, int O, int nb,
                                                 hipStream_t st) {
    const size_t n = (size_t)O * nb;
    hipLaunchKernelGGL(coli_rows16_to_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, packed, rows, O,
                       nb);
    return hipGetLastError();
}
