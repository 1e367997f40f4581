// gemv_dma.hip -- the decode GEMV with weights streamed through an LDS ring.
//
// Same problem, data layout and arithmetic as coli_gemv_tiles (gemv.hip):
// y[b, o] = sum_g scale[o, g] * sum_{k in g} x[b, k] * w[o, k], one
// v_mfma_f32_16x16x32_f16 per 32-column group with the weights unpacked to
// exact fp16 in registers, the group scale applied to the MFMA result, K split
// across the W waves of a workgroup and summed in fixed wave order. Results
// are bitwise identical to coli_gemv_tiles for the same decomposition.
//
// What differs is how the bytes arrive. Every load of the main loop is an
// LDS DMA (global_load_lds_dword / _dwordx4): the weight tiles (one 1 KiB
// dwordx4 per tile), the tile scales and the activation fragments of the
// stage go straight into a per-wave ring of PD slots, so
//  * the depth of the prefetch costs LDS, not VGPRs;
//  * the loop waits with exact s_waitcnt vmcnt(N) of its own (the compiler
//    neither tracks nor reorders these loads), and past a wave's last quad it
//    issues nothing: no tile is fetched twice and no wave re-reads a shared
//    zero tile at its tail (thousands of such reads of one address serialize
//    on one L2 channel);
//  * a group needs no split of K across workgroups: long-K narrow-O shapes
//    use one row tile per group and eight waves over K (no partials, no
//    arrival counter, no tail of dependent round trips).
// Activation fragments of one batch row (every problem of the launch has one
// row) arrive as one 256 B dword DMA per stage and are read as a broadcast.
// For more rows, each dwordx4 DMA stages four rows of the quad (1 KiB); lane
// l of the DMA fetches 16 B chunk (l % 16) ^ row of row l / 16, so the
// sixteen lanes of one k-slice read sixteen different bank groups (the
// A-operand reads are free of bank conflicts). The ring always reserves room
// for the lo fragments; they are fetched only when the fragment set has any.
//
// F32 (one to four batch rows, K a multiple of 128): no fragment prep at
// all. The stage's activations arrive as f32 (the same NXR x 512 bytes the
// hi + lo fragments would take) and each wave converts them in place before
// its MFMAs: the exponent is taken per 128-column quad and batch row (E with
// max|x| * 2^-E in [2^14, 2^15) over the quad, 0 for an all-zero quad), hi and lo
// are split as in coli_prep_frag, and the quad's partial sum, over its four
// groups, is scaled by 2^E into the accumulator. The lo MFMAs of a quad run
// only when one of its lo parts is non-zero (a wave-uniform branch). Per-quad
// exponents keep at least the precision of one exponent per row; the sums
// differ from the fragment path in rounding only.
#include "coli_hip_internal.h"

#include <math.h>

#include <type_traits>

#include "coli_device.h"


// NXR: batch rows staged per problem and stage (1, 4, 8 or 16).
template <int KIND, int R, int NXR>
struct DmaGeom {
    static constexpr int kScaleOff = R * COLI_TILE_BYTES;
    static constexpr int kScaleInst = (R + ScaleGeom<KIND>::kPerInst - 1) / ScaleGeom<KIND>::kPerInst;
    static constexpr int kXOff = kScaleOff + kScaleInst * 256;
    static constexpr int kXInst = NXR == 1 ? 1 : NXR / 4;   // DMA instructions per fragment half
    static constexpr int kXBytes = NXR * 256;
    static constexpr int kSlot = kXOff + 2 * kXBytes;     // room for hi + lo (= NXR rows of 128 f32)
    static constexpr int kF32Inst = NXR == 1 ? 2 : NXR / 2;  // f32 DMA: 256 B (one row) / 1 KiB (two rows)
    static constexpr int loads(bool lo) { return R + kScaleInst + kXInst * (lo ? 2 : 1); }
    static constexpr int loads_f32() { return R + kScaleInst + kF32Inst; }
};

// In-place conversion of one stage's f32 activations (NXR rows x 128, row
// major at x) into hi / lo fragments at x / x + NXR * 256, laid out as the
// fragment DMA would have left them. Returns 2^E of the lane's quad row in
// *scale (NXR == 1: the one row; NXR == 4: row lane / 16) and whether any lo
// part of the wave is non-zero. Every lane reads all its values before any
// lane writes (one wave, LDS in order).
template <int NXR, bool INT4>
__device__ __forceinline__ bool f32_to_frags(uint8_t *x, int lane, int *E_out) {
    if constexpr (NXR == 1) {
        // lane: chunk c = lane / 4, fragment slots 2u, 2u + 1 (u = lane % 4)
        const int c = lane >> 2, u = lane & 3;
        const int col = 8 * c + (INT4 ? (u < 2 ? 4 * u : 4 * (u - 2) + 1) : 2 * u);
        const int step = INT4 ? 2 : 1;
        const float v0 = LDS_RD(float, x + col * 4), v1 = LDS_RD(float, x + (col + step) * 4);
        const float m = wave_max64(fmaxf(fabsf(v0), fabsf(v1)));
        int E = 0;
        if (m > 0.0f && isfinite(m)) {
            frexpf(m, &E);
            E -= 15;
        }
        const float mul = (INT4 && u >= 2) ? 0.0625f : 1.0f;
        const float y0 = ldexpf(v0, -E) * mul, y1 = ldexpf(v1, -E) * mul;
        const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1;
        const _Float16 l0 = (_Float16)(y0 - (float)h0), l1 = (_Float16)(y1 - (float)h1);
        LDS_WR(half2v, x + c * 16 + u * 4, ((half2v){h0, h1}));
        LDS_WR(half2v, x + 256 + c * 16 + u * 4, ((half2v){l0, l1}));
        *E_out = E;
        return __builtin_amdgcn_ballot_w64(l0 != (_Float16)0.0f || l1 != (_Float16)0.0f) != 0;
    } else if constexpr (NXR == 4) {
        // lane: row rr = lane / 16, chunk c = lane % 16 (columns 8c .. 8c + 7)
        const int rr = lane >> 4, c = lane & 15;
        const floatx4 a = LDS_RD(floatx4, x + rr * 512 + c * 32), b = LDS_RD(floatx4, x + rr * 512 + c * 32 + 16);
        const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        float m = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) m = fmaxf(m, fabsf(v[t]));
        m = dpp_max16(m);
        int E = 0;
        if (m > 0.0f && isfinite(m)) {
            frexpf(m, &E);
            E -= 15;
        }
        half8v h, l;
        bool any = false;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int off = INT4 ? (t < 4 ? 2 * t : 2 * (t - 4) + 1) : t;
            float y = ldexpf(v[off], -E);
            if (INT4 && (off & 1)) y *= 0.0625f;
            h[t] = (_Float16)y;
            l[t] = (_Float16)(y - (float)h[t]);
            any |= l[t] != (_Float16)0.0f;
        }
        const int dst = (rr * 16 + (c ^ rr)) * 16;
        LDS_WR(half8v, x + dst, h);
        LDS_WR(half8v, x + NXR * 256 + dst, l);
        *E_out = E;
        return __builtin_amdgcn_ballot_w64(any) != 0;
    } else {
        *E_out = 0;   // not instantiated by a launch (F32 requires NXR 1 or 4)
        return false;
    }
}

// INL: the single problem a.prob0 (3-D grid: row block, 1, batch tile).
// XS (with F32, one row): the workgroup converts its row once into LDS
// (dynamic shared memory: hi [nq][256 B], lo [nq][256 B], exponents [nq]) while
// its first weight stages are in flight; the stages then carry weights and
// scales only.
template <int KIND, int R, bool DUAL, int NB4, int W, int PD, int NXR, bool INL, bool F32, bool XS = false,
          bool GX = false>
__global__ __launch_bounds__(64 * W) void coli_gemv_dma(ColiGemvArgs a) {
    static_assert(!GX || (INL && !F32 && !DUAL), "emitted fragments: one plain matrix, prepared fragments");
    using G = DmaGeom<KIND, R, NXR>;
    static_assert(!XS || (F32 && NXR == 1), "staged activations: f32, one row");
    static_assert(!F32 || NXR == 1 || NXR == 4, "f32 activations: one or four rows per stage");
    constexpr bool XF = NXR > 1;
    constexpr int RT = DUAL ? R / 2 : R;
    constexpr int RING = W * PD * G::kSlot;
    constexpr int RED = W * R * NB4 * 64 * 4;
    static_assert(RING <= 160 * 1024 && RED <= 160 * 1024, "LDS budget");
    static_assert((PD - 1) * (F32 ? G::loads_f32() : G::loads(true)) <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[RING > RED ? RING : RED];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int p = 0, bt, rb;
    ColiProb pdesc;
    if constexpr (INL) {
        rb = blockIdx.x;
        bt = blockIdx.z;
    } else {
        const int item = blockIdx.x;
        const int items_per_p = a.n_bt * a.rb_per_prob;
        p = item / items_per_p;
        if (p >= a.nprob) return;
        // the descriptor (inside the array: p < nprob) and the live count are
        // read together, one memory round trip before the weight loads
        pdesc = a.prob[p];
        if (a.nprob_dev && p >= *a.nprob_dev) return;
        const int rem = item - p * items_per_p;
        bt = rem / a.rb_per_prob;
        rb = rem - bt * a.rb_per_prob;
    }
    const ColiProb pr = uniform_prob(INL ? a.prob0 : pdesc);
    const int nb = min(16, pr.nrows - 16 * bt);
    if constexpr (!INL) {
        if (nb <= 0) return;
    }
    const int b = lane & 15, ks = lane >> 4;
    const int nq = a.nq;
    const int q_first = wave;
    const int nit = q_first < nq ? (nq - q_first + W - 1) / W : 0;

    // row tiles of this group (dead ones read the zero tile, whose scales are zero)
    int rt[R];
    bool live[R];
    const uint8_t *wr[R], *sr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int rr = DUAL ? (r % RT) : r;
        rt[r] = rb * RT + rr;
        live[r] = rt[r] < a.nrt;
        const bool second = DUAL && r >= RT;
        const size_t t0 = (size_t)(uint32_t)min(rt[r], a.nrt - 1) * (uint32_t)nq;
        wr[r] = live[r] ? (second ? pr.w1 : pr.w0) + t0 * COLI_TILE_BYTES : (const uint8_t *)a.zero;
        sr[r] = live[r] ? (const uint8_t *)(second ? pr.s1 : pr.s0) + t0 * ScaleGeom<KIND>::kBytes
                        : (const uint8_t *)a.zero;
    }
    // per-lane activation source of the DMA: NXR > 1: row 4k + lane/16 of
    // the batch tile (clamped to the last real row) for instruction k, chunk
    // (lane % 16) ^ row; else the problem's one row, 4 bytes per lane
    const uint8_t *xsrc_hi[G::kXInst], *xsrc_lo[G::kXInst];
#pragma unroll
    for (int k = 0; k < G::kXInst; k++) {
        const int brow = XF ? min(4 * k + (lane >> 4), nb - 1) : 0;
        const int br = pr.xrow_off + 16 * bt + brow;
        const int fr = a.xrows ? a.xrows[br] : br;
        const size_t off = (size_t)fr * a.xstride * 2 + (XF ? (((lane & 15) ^ (4 * k + (lane >> 4))) * 16) : lane * 4);
        xsrc_hi[k] = (const uint8_t *)a.xhi + off;
        xsrc_lo[k] = (const uint8_t *)a.xlo + off;
    }
    // f32 activations: instruction k fetches row 0, columns 64k + lane
    // (NXR 1), or rows 2k + lane / 32, columns 4 (lane % 32) .. + 3 (NXR 4)
    const uint8_t *xsrc_f[G::kF32Inst];
    if constexpr (F32) {
#pragma unroll
        for (int k = 0; k < G::kF32Inst; k++) {
            const int brow = NXR == 1 ? 0 : min(2 * k + (lane >> 5), nb - 1);
            const int br = pr.xrow_off + 16 * bt + brow;
            const int fr = a.xrows ? a.xrows[br] : br;
            const int col = NXR == 1 ? 64 * k + lane : 4 * (lane & 31);
            xsrc_f[k] = (const uint8_t *)(a.xf + (size_t)fr * a.ldx + col);
        }
    }
    uint8_t *ring = lds + wave * PD * G::kSlot;
    // the ring is written behind the compiler's back: let it escape, so the
    // "memory" clobbers of the waits below force fresh reads
    asm volatile("" ::"v"(lds) : "memory");

    auto issue = [&](int it, int slot, bool lo) {
        const int q = q_first + it * W;
        uint8_t *dst = ring + slot * G::kSlot;
#pragma unroll
        for (int r = 0; r < R; r++)
            __builtin_amdgcn_global_load_lds((const void *)(wr[r] + (size_t)(live[r] ? q : 0) * COLI_TILE_BYTES + lane * 16),
                                             (lds_void *)(dst + r * COLI_TILE_BYTES), 16, 0, 0);
#pragma unroll
        for (int k = 0; k < G::kScaleInst; k++) {
            constexpr int LPT = ScaleGeom<KIND>::kLanes;
            const int r = min(R - 1, k * ScaleGeom<KIND>::kPerInst + lane / LPT);
            // (branch-free: a per-lane select between R scalar bases)
            const uint8_t *base = sr[0];
            size_t qo = live[0] ? (size_t)q * ScaleGeom<KIND>::kBytes : 0;
#pragma unroll
            for (int rr = 1; rr < R; rr++) {
                if (r == rr) {
                    base = sr[rr];
                    qo = live[rr] ? (size_t)q * ScaleGeom<KIND>::kBytes : 0;
                }
            }
            __builtin_amdgcn_global_load_lds((const void *)(base + qo + (lane % LPT) * 4),
                                             (lds_void *)(dst + G::kScaleOff + k * 256), 4, 0, 0);
        }
        if constexpr (XS) {
            return;
        } else if constexpr (F32) {
#pragma unroll
            for (int k = 0; k < G::kF32Inst; k++) {
                if constexpr (NXR == 1)
                    __builtin_amdgcn_global_load_lds((const void *)(xsrc_f[k] + (size_t)q * 512),
                                                     (lds_void *)(dst + G::kXOff + k * 256), 4, 0, 0);
                else
                    __builtin_amdgcn_global_load_lds((const void *)(xsrc_f[k] + (size_t)q * 512),
                                                     (lds_void *)(dst + G::kXOff + k * 1024), 16, 0, 0);
            }
            return;
        }
        const size_t xo = (size_t)q * 256;
        auto xdma = [&](const uint8_t *src, int off) {
            if constexpr (NXR > 1) __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(dst + off), 16, 0, 0);
            else __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(dst + off), 4, 0, 0);
        };
        constexpr int xb = NXR > 1 ? 1024 : 256;   // bytes per DMA instruction
#pragma unroll
        for (int k = 0; k < G::kXInst; k++) xdma(xsrc_hi[k] + xo, G::kXOff + k * xb);
        if (lo) {
#pragma unroll
            for (int k = 0; k < G::kXInst; k++) xdma(xsrc_lo[k] + xo, G::kXOff + G::kXBytes + k * xb);
        }
    };

    floatx4 acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = (floatx4){0.f, 0.f, 0.f, 0.f};
    // A operand of lane (b, ks), group j: chunk 4j + ks of row min(b, nb-1)
    // (swizzled by the row when NXR > 1; one row read as a broadcast else)
    const int xrow = XF ? min(b, nb - 1) : 0;
    auto xaddr = [&](int j) -> uint32_t {
        return XF ? (uint32_t)(xrow * 16 + ((4 * j + ks) ^ xrow)) * 16 : (uint32_t)(j * 64 + ks * 16);
    };

    // GX: prepared fragments emitted by the GEMV that produced x carry one
    // exponent per (row, group); the exponents of the problem's rows of every
    // quad are staged in LDS ([quad][gxs rows] words, gxs = the rows rounded
    // up to a multiple of 4: little enough to keep two workgroups a CU) before
    // the loop, and each group's MFMA result is scaled by 2^E of its row along
    // with the group scale.
    extern __shared__ __attribute__((aligned(16))) uint8_t xs_lds[];
    constexpr bool gx = GX;
    const bool fold = KIND == COLI_KIND_FP4 && !gx && a.fold;
    const int gxs = 4 * ((nb + 3) >> 2);
    auto compute = [&](int slot, auto lo_tag, int q) {
        constexpr bool LO = decltype(lo_tag)::value;
        const uint8_t *src = ring + slot * G::kSlot;
        u32x4 ge = (u32x4){0u, 0u, 0u, 0u};
        // (lanes of rows past the problem read the last group of four)
        if constexpr (gx) ge = *(const u32x4 *)(xs_lds + ((size_t)q * gxs + 4 * min(ks, (gxs >> 2) - 1)) * 4);
        u32x4 w[R];
        ScaleRegs<KIND> sc[R];
        half8v xh[4], xl[LO ? 4 : 1];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            xh[j] = LDS_RD(half8v, src + G::kXOff + xaddr(j));
            if constexpr (LO) xl[j] = LDS_RD(half8v, src + G::kXOff + G::kXBytes + xaddr(j));
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = LDS_RD(u32x4, src + r * COLI_TILE_BYTES + lane * 16);
            scale_from_lds<KIND>(sc[r], src + G::kScaleOff + r * ScaleGeom<KIND>::kBytes, lane & 15);
        }
        if constexpr (KIND == COLI_KIND_FP4 && !gx) {
            if (fold) {   // exact fp16 e2m1 x scale: the MFMAs accumulate
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const half8v bw = unpack_fp4_scaled(w[r][j], sc[r].get(j));
                        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[j], bw, acc[r], 0, 0, 0);
                        if constexpr (LO) acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[j], bw, acc[r], 0, 0, 0);
                    }
                return;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const half8v bw = unpack_b<KIND>(w[r][j]);
                floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[j], bw, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                if constexpr (LO) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[j], bw, d, 0, 0, 0);
                const float scl = sc[r].get(j);
                if constexpr (gx) {
#pragma unroll
                    for (int i = 0; i < NB4; i++) acc[r][i] = fmaf(ldexpf(d[i], gexp_of(ge[i], j)), scl, acc[r][i]);
                } else {
#pragma unroll
                    for (int i = 0; i < NB4; i++) acc[r][i] = fmaf(d[i], scl, acc[r][i]);
                }
            }
        }
    };

    // F32: convert the stage, then the quad's partial sum over its four groups
    // is scaled by 2^E of its batch row into the accumulator
    auto compute_f32 = [&](int slot) {
        uint8_t *src = ring + slot * G::kSlot;
        int Eq;
        const bool lo = f32_to_frags<NXR, KIND != COLI_KIND_FP4>(src + G::kXOff, lane, &Eq);
        int Ei[NB4];
#pragma unroll
        for (int i = 0; i < NB4; i++)
            Ei[i] = NXR == 1 ? __builtin_amdgcn_readfirstlane(Eq) : __builtin_amdgcn_readlane(Eq, 16 * i);
        u32x4 w[R];
        ScaleRegs<KIND> sc[R];
        half8v xh[4], xl[4];
#pragma unroll
        for (int j = 0; j < 4; j++) xh[j] = LDS_RD(half8v, src + G::kXOff + xaddr(j));
        if (lo) {
#pragma unroll
            for (int j = 0; j < 4; j++) xl[j] = LDS_RD(half8v, src + G::kXOff + G::kXBytes + xaddr(j));
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = LDS_RD(u32x4, src + r * COLI_TILE_BYTES + lane * 16);
            scale_from_lds<KIND>(sc[r], src + G::kScaleOff + r * ScaleGeom<KIND>::kBytes, lane & 15);
        }
        floatx4 t[R];
#pragma unroll
        for (int r = 0; r < R; r++) t[r] = (floatx4){0.f, 0.f, 0.f, 0.f};
        if (KIND == COLI_KIND_FP4 && fold) {   // exact fp16 e2m1 x scale: the MFMAs accumulate
#pragma unroll
            for (int j = 0; j < 4; j++) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const half8v bw = unpack_fp4_scaled(w[r][j], sc[r].get(j));
                    t[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[j], bw, t[r], 0, 0, 0);
                    if (lo) t[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[j], bw, t[r], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const half8v bw = unpack_b<KIND>(w[r][j]);
                    floatx4 d =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[j], bw, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    if (lo) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[j], bw, d, 0, 0, 0);
                    const float scl = sc[r].get(j);
#pragma unroll
                    for (int i = 0; i < NB4; i++) t[r][i] = fmaf(d[i], scl, t[r][i]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int i = 0; i < NB4; i++) acc[r][i] += ldexpf(t[r][i], Ei[i]);
    };

    // XS: the staged row (set up below, before the loop, in xs_lds)
    auto compute_xs = [&](int slot, int q, bool lo) {
        const uint8_t *src = ring + slot * G::kSlot;
        const uint8_t *xq = xs_lds + q * 256 + ks * 16;
        u32x4 w[R];
        ScaleRegs<KIND> sc[R];
        half8v xh[4], xl[4];
#pragma unroll
        for (int j = 0; j < 4; j++) xh[j] = *(const half8v *)(xq + j * 64);
        if (lo) {
#pragma unroll
            for (int j = 0; j < 4; j++) xl[j] = *(const half8v *)(xq + a.nq * 256 + j * 64);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = LDS_RD(u32x4, src + r * COLI_TILE_BYTES + lane * 16);
            scale_from_lds<KIND>(sc[r], src + G::kScaleOff + r * ScaleGeom<KIND>::kBytes, lane & 15);
        }
        floatx4 t[R];
#pragma unroll
        for (int r = 0; r < R; r++) t[r] = (floatx4){0.f, 0.f, 0.f, 0.f};
        if (KIND == COLI_KIND_FP4 && fold) {   // exact fp16 e2m1 x scale: the MFMAs accumulate
#pragma unroll
            for (int j = 0; j < 4; j++) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const half8v bw = unpack_fp4_scaled(w[r][j], sc[r].get(j));
                    t[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[j], bw, t[r], 0, 0, 0);
                    if (lo) t[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[j], bw, t[r], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const half8v bw = unpack_b<KIND>(w[r][j]);
                    floatx4 d =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[j], bw, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    if (lo) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[j], bw, d, 0, 0, 0);
                    const float scl = sc[r].get(j);
#pragma unroll
                    for (int i = 0; i < NB4; i++) t[r][i] = fmaf(d[i], scl, t[r][i]);
                }
            }
        }
        const int Eq = ((const int *)(xs_lds + a.nq * 512))[q];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int i = 0; i < NB4; i++) acc[r][i] += ldexpf(t[r][i], Eq);
    };

    auto run_xs = [&]() {
        constexpr int L = G::loads(false) - G::kXInst;   // weights and scales only
#pragma unroll
        for (int s = 0; s < PD - 1; s++)
            if (s < nit) issue(s, s, false);
        // stage the row: thread t converts 8 columns (chunk) c = t + 64 W i
        // of the row; a quad's sixteen chunks sit on sixteen consecutive lanes
        const int ncc = a.nq * 16;
        const float *xrow = (const float *)xsrc_f[0] - lane;   // row start (xsrc_f[0] = row + lane)
        bool any = false;
        for (int c0 = 0; c0 < ncc; c0 += 64 * W) {
            const int c = c0 + threadIdx.x;
            floatx4 v0 = (floatx4){0.f, 0.f, 0.f, 0.f}, v1 = v0;
            if (c < ncc) {
                v0 = *GPTR(floatx4, xrow + c * 8);
                v1 = *GPTR(floatx4, xrow + c * 8 + 4);
            }
            float m = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) m = fmaxf(m, fmaxf(fabsf(v0[t]), fabsf(v1[t])));
            m = dpp_max16(m);
            int E = 0;
            if (m > 0.0f && isfinite(m)) {
                frexpf(m, &E);
                E -= 15;
            }
            if (c < ncc) {
                const float u[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                half8v h, l;
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const int off = KIND != COLI_KIND_FP4 ? (t < 4 ? 2 * t : 2 * (t - 4) + 1) : t;
                    float y = ldexpf(u[off], -E);
                    if (KIND != COLI_KIND_FP4 && (off & 1)) y *= 0.0625f;
                    h[t] = (_Float16)y;
                    l[t] = (_Float16)(y - (float)h[t]);
                    any |= l[t] != (_Float16)0.0f;
                }
                *(half8v *)(xs_lds + c * 16) = h;
                *(half8v *)(xs_lds + a.nq * 256 + c * 16) = l;
                if ((c & 15) == 0) ((int *)(xs_lds + a.nq * 512))[c >> 4] = E;
            }
        }
        const bool lo = __syncthreads_or(any);
        for (int it0 = 0; it0 < nit; it0 += PD) {
#pragma unroll
            for (int u = 0; u < PD; u++) {
                const int it = it0 + u;
                if (it >= nit) break;
                if (it + PD - 1 < nit) {
                    issue(it + PD - 1, (u + PD - 1) % PD, false);
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PD - 1) * L) : "memory");
                } else {
                    dma_wait_tail<L, PD>(nit - 1 - it);
                }
                compute_xs(u, q_first + it * W, lo);
            }
        }
    };

    auto run_f32 = [&]() {
        constexpr int L = G::loads_f32();
#pragma unroll
        for (int s = 0; s < PD - 1; s++)
            if (s < nit) issue(s, s, false);
        for (int it0 = 0; it0 < nit; it0 += PD) {
#pragma unroll
            for (int u = 0; u < PD; u++) {
                const int it = it0 + u;
                if (it >= nit) break;
                if (it + PD - 1 < nit) {
                    issue(it + PD - 1, (u + PD - 1) % PD, false);
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PD - 1) * L) : "memory");
                } else {
                    dma_wait_tail<L, PD>(nit - 1 - it);
                }
                compute_f32(u);
            }
        }
    };

    auto run = [&](auto lo_tag) {
        constexpr bool LO = decltype(lo_tag)::value;
        constexpr int L = G::loads(LO);
        // GX: the group exponents of the problem's rows, staged by LDS DMA
        // (64 words per instruction, dealt over the waves) ahead of the first
        // stages; one wait and barrier before the loop (every wave reaches it)
        if constexpr (gx) {
            const int words = nq * gxs;
            for (int k = wave; k * 64 < words; k += W) {
                const int e = k * 64 + lane, qe = min(e / gxs, nq - 1), row = min(e - (e / gxs) * gxs, nb - 1);
                __builtin_amdgcn_global_load_lds(
                    (const void *)(a.gexp + ((size_t)qe * a.gexp_rows + pr.xrow_off + 16 * bt + row) * 4),
                    (lds_void *)(xs_lds + k * 256), 4, 0, 0);
            }
        }
#pragma unroll
        for (int s = 0; s < PD - 1; s++)
            if (s < nit) issue(s, s, LO);
        if constexpr (gx) {
            // the exponents went out first: at most the stages may remain
            if (nit >= PD - 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PD - 1) * L) : "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        for (int it0 = 0; it0 < nit; it0 += PD) {
#pragma unroll
            for (int u = 0; u < PD; u++) {
                const int it = it0 + u;
                if (it >= nit) break;
                if (it + PD - 1 < nit) {
                    issue(it + PD - 1, (u + PD - 1) % PD, LO);
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((PD - 1) * L) : "memory");
                } else {
                    dma_wait_tail<L, PD>(nit - 1 - it);
                }
                compute(u, lo_tag, q_first + it * W);
            }
        }
    };
    if constexpr (XS) run_xs();
    else if constexpr (F32) run_f32();
    else if (gx || *a.haslo >= a.lo_gen) run(std::true_type{});   // >=: stays correct under graph replay
    else run(std::false_type{});

    // exponent of the batch row this wave finishes
    int E_out = 0;
    if (!F32 && !gx && wave < NB4) {
        const int brow = ks * 4 + wave;
        if (brow < nb) {
            const int br = pr.xrow_off + 16 * bt + brow;
            E_out = a.xexp[a.xrows ? a.xrows[br] : br];
        }
    }
    // ---- reduction in fixed wave order through the (drained) ring ----
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    float *red = (float *)lds;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int i = 0; i < NB4; i++) red[((wave * R + r) * NB4 + i) * 64 + lane] = acc[r][i];
    __syncthreads();
    const int i = wave;
    if (i >= NB4) return;
    float v[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float t = red[(r * NB4 + i) * 64 + lane];
#pragma unroll
        for (int w = 1; w < W; w++) t += red[((w * R + r) * NB4 + i) * 64 + lane];
        v[r] = t;
    }
    gemv_epilogue<R, DUAL>(a, pr, bt, rt, live, v, ks * 4 + i, lane, E_out);
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
template <int KIND, int R, bool DUAL, int NB4, int PD, int NXR, bool F32, int W>
static hipError_t launch_dma6(const ColiGemvArgs &a, int blocks, hipStream_t st) {
    using G = DmaGeom<KIND, R, NXR>;
    if constexpr (W * PD * G::kSlot > 160 * 1024 || (PD - 1) * (F32 ? G::loads_f32() : G::loads(true)) > 63) {
        return hipErrorInvalidConfiguration;
    } else {
        if constexpr (F32 && NXR == 1) {
            if (a.xstage) {   // the row staged once per workgroup
                const size_t shm = (size_t)a.nq * 516;
                if ((size_t)W * PD * G::kSlot + shm > 160 * 1024) return hipErrorInvalidConfiguration;
                if (!a.prob)
                    hipLaunchKernelGGL((coli_gemv_dma<KIND, R, DUAL, NB4, W, PD, NXR, true, F32, true>),
                                       dim3(a.rb_per_prob, 1, a.n_bt), dim3(64 * W), shm, st, a);
                else
                    hipLaunchKernelGGL((coli_gemv_dma<KIND, R, DUAL, NB4, W, PD, NXR, false, F32, true>),
                                       dim3(blocks), dim3(64 * W), shm, st, a);
                return hipGetLastError();
            }
        }
        // emitted fragments: their group exponents staged in LDS
        if constexpr (!F32 && !DUAL) {
            if (a.gexp && !a.prob) {   // emitted fragments: their exponents staged beside the ring
                const int gxs = 4 * ((min(16, a.prob0.nrows) + 3) / 4);
                const size_t gshm = ((size_t)a.nq * gxs + 63) / 64 * 256;
                if ((size_t)W * PD * G::kSlot + gshm > 160 * 1024) return hipErrorInvalidConfiguration;
                hipLaunchKernelGGL((coli_gemv_dma<KIND, R, DUAL, NB4, W, PD, NXR, true, F32, false, true>),
                                   dim3(a.rb_per_prob, 1, a.n_bt), dim3(64 * W), gshm, st, a);
                return hipGetLastError();
            }
        }
        if (!a.prob)
            hipLaunchKernelGGL((coli_gemv_dma<KIND, R, DUAL, NB4, W, PD, NXR, true, F32>),
                               dim3(a.rb_per_prob, 1, a.n_bt), dim3(64 * W), 0, st, a);
        else
            hipLaunchKernelGGL((coli_gemv_dma<KIND, R, DUAL, NB4, W, PD, NXR, false, F32>), dim3(blocks),
                               dim3(64 * W), 0, st, a);
        return hipGetLastError();
    }
}

// W = 16 (one row tile, long K): twice the waves per CU to cover the
// latency of each wave's serial per-quad chain.
template <int KIND, int R, bool DUAL, int NB4, int PD, int NXR, bool F32>
static hipError_t launch_dma5(const ColiGemvArgs &a, int W, int blocks, hipStream_t st) {
    if constexpr (R == 1 && !DUAL) {
        if (W == 16) return launch_dma6<KIND, R, DUAL, NB4, PD, NXR, F32, 16>(a, blocks, st);
    }
    if constexpr (DUAL && NXR == 1) {
        if (W == 4) return launch_dma6<KIND, R, DUAL, NB4, PD, NXR, F32, 4>(a, blocks, st);
    }
    return launch_dma6<KIND, R, DUAL, NB4, PD, NXR, F32, 8>(a, blocks, st);
}

template <int KIND, int R, bool DUAL, int NB4, int PD, int NXR>
static hipError_t launch_dma4(const ColiGemvArgs &a, int W, int blocks, hipStream_t st) {
    if constexpr (NXR == 1 || NXR == 4) {
        if (a.xf) return launch_dma5<KIND, R, DUAL, NB4, PD, NXR, true>(a, W, blocks, st);
    }
    return launch_dma5<KIND, R, DUAL, NB4, PD, NXR, false>(a, W, blocks, st);
}

template <int KIND, int R, bool DUAL, int NB4, int NXR>
static hipError_t launch_dma3(const ColiGemvArgs &a, int W, int PD, int blocks, hipStream_t st) {
    if (PD == 2) return launch_dma4<KIND, R, DUAL, NB4, 2, NXR>(a, W, blocks, st);
    return launch_dma4<KIND, R, DUAL, NB4, 3, NXR>(a, W, blocks, st);
}

template <int KIND, int R, bool DUAL>
static hipError_t launch_dma2(const ColiGemvArgs &a, int W, int max_rows, int PD, int blocks, hipStream_t st) {
    if (max_rows <= 1) return launch_dma3<KIND, R, DUAL, 1, 1>(a, W, PD, blocks, st);
    if (max_rows <= 2) return launch_dma3<KIND, R, DUAL, 2, 4>(a, W, PD, blocks, st);
    if (max_rows <= 4) return launch_dma3<KIND, R, DUAL, 4, 4>(a, W, PD, blocks, st);
    if (max_rows <= 8) return launch_dma3<KIND, R, DUAL, 4, 8>(a, W, PD, blocks, st);
    return launch_dma3<KIND, R, DUAL, 4, 16>(a, W, PD, blocks, st);
}

template <int KIND>
static hipError_t launch_dma1(const ColiGemvArgs &a, int R, bool dual, int W, int max_rows, int PD, int blocks,
                              hipStream_t st) {
    if (dual) {
        if (R == 4) return launch_dma2<KIND, 4, true>(a, W, max_rows, PD, blocks, st);
        return launch_dma2<KIND, 2, true>(a, W, max_rows, PD, blocks, st);
    }
    if (R == 4) return launch_dma2<KIND, 4, false>(a, W, max_rows, PD, blocks, st);
    if (R == 2) return launch_dma2<KIND, 2, false>(a, W, max_rows, PD, blocks, st);
    return launch_dma2<KIND, 1, false>(a, W, max_rows, PD, blocks, st);
}

// Returns hipErrorInvalidConfiguration for a decomposition the ring cannot
// hold (the caller then uses coli_gemv_tiles).
extern "C" hipError_t coli_launch_gemv_dma(int kind, const ColiGemvArgs *a, int R, int dual, int W, int PD, int max_rows,
                                           hipStream_t st) {
    if (a->splits != 1 || max_rows < 1 || max_rows > 16 || (W != 4 && W != 8 && W != 16)) return hipErrorInvalidValue;
    // f32 activations: up to four rows, rows of whole quads, 16-byte aligned
    if (a->xf && (max_rows > 4 || a->ldx < a->nq * 128 || a->ldx % 4 || (uintptr_t)a->xf % 16))
        return hipErrorInvalidValue;
    if (!a->prob && (a->nprob != 1 || a->nprob_dev)) return hipErrorInvalidValue;
    const long items = (long)a->nprob * a->n_bt * a->rb_per_prob;
    if (items <= 0) return hipSuccess;
    const int blocks = (int)items;
    switch (kind) {
    case COLI_KIND_I4_H: return launch_dma1<COLI_KIND_I4_H>(*a, R, dual, W, max_rows, PD, blocks, st);
    case COLI_KIND_I4_F: return launch_dma1<COLI_KIND_I4_F>(*a, R, dual, W, max_rows, PD, blocks, st);
    case COLI_KIND_FP4: return launch_dma1<COLI_KIND_FP4>(*a, R, dual, W, max_rows, PD, blocks, st);
    default: return hipErrorInvalidValue;
    }
}
