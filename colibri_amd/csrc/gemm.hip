// gemm.hip -- grouped dequant-fused GEMM for gfx950: many-row problems
// (prefill chunks, verification batches), y[b, o] = sum_g scale[o, g] *
// sum_{k in g} x[b, k] w[o, k], the same arithmetic as the GEMV (c/quant.h
// fmt=4 and fmt=7) with the weights read once per 64 rows instead of once per
// 16.
//
// Work item = (problem, 64-row tile, output block). A workgroup of
// COLI_GM_WAVES waves owns 2 row tiles per wave (DUAL: the gate tile and the up
// tile of the same 16 rows, SwiGLU in the epilogue) over the full K, one
// 128-column quad per step:
//  * every load of the main loop is an LDS DMA into a ring of PD stages: each
//    wave's two weight tiles and their scales (private to the wave), and the
//    quad's activation fragments of the 64 rows (fp16 hi + lo of x * 2^-E,
//    built by coli_prep_frag; shared by the workgroup, each wave fetching two
//    (hi) or four (hi + lo) of the 16 chunks). No load of the loop writes a
//    register, so the compiler inserts no wait of its own: the loop waits with
//    exact s_waitcnt vmcnt(N) for its oldest stage and synchronizes with a
//    bare s_barrier (the fence of __syncthreads() would drain the ring). The
//    activations ride in the same ring as the weights, as deep: loads retire
//    in order, so a shallower activation ring would retire the weights with it;
//  * the chunks are laid out in the MFMA A-operand order (lane l of a DMA
//    fetches the 16 B lane l of the MFMA reads), so the reads are free of bank
//    conflicts; chunks of dead 16-row subtiles re-read the tile's last row (one
//    cache line), which keeps the count of loads per stage fixed;
//  * each 32-column group is one v_mfma_f32_16x16x32_f16 per (weight tile,
//    live 16-row subtile) -- two with the lo fragments -- its result scaled by
//    the group scale and accumulated in f32. The unpacked B operand of a group
//    is reused by the 4 row subtiles. MXFP4 matrices whose e8m0 scales keep
//    every e2m1 value times its scale a normal fp16 (fold) take the scale into
//    the unpack instead (exact) and accumulate inside the MFMA: no per-group
//    VALU work beyond the conversion.
// The ring is 4 stages deep when no lo part is set (the common case of
// activations exact in fp16 after the row exponent), 3 with lo parts.
#include <type_traits>

#include "coli_device.h"

// per-wave weight slot: 2 tiles + their scales (one or two dword DMAs)
template <int KIND>
struct GmGeom {
    static constexpr int kScaleInst = (2 + ScaleGeom<KIND>::kPerInst - 1) / ScaleGeom<KIND>::kPerInst;
    static constexpr int kWSlot = 2 * COLI_TILE_BYTES + kScaleInst * 256;
    static constexpr int kActHi = 16384;   // 64 rows x 128 columns x fp16
    static constexpr int kPdHi = 4, kPdLo = 3;
    static constexpr int bytes(bool lo) {
        return (lo ? kPdLo : kPdHi) * ((lo ? 2 : 1) * kActHi + COLI_GM_WAVES * kWSlot);
    }
    static constexpr int kLds = bytes(true) > bytes(false) ? bytes(true) : bytes(false);
};
static_assert(GmGeom<COLI_KIND_I4_F>::kLds <= 160 * 1024, "ring exceeds the LDS of a CU");

template <int KIND, bool DUAL>
__global__ __launch_bounds__(64 * COLI_GM_WAVES) void coli_gemm_tiles(ColiGemmArgs a) {
    using G = GmGeom<KIND>;
    using SG = ScaleGeom<KIND>;
    constexpr int W = COLI_GM_WAVES;
    constexpr int R = 2;                 // weight tiles per wave
    constexpr int RT = DUAL ? 1 : 2;     // distinct output row tiles per wave
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // readfirstlane: the wave index is wave-uniform, so everything derived from it
    // (tile indices, validity, base pointers) stays in scalar registers.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    const int item = blockIdx.x / a.rb_per_prob, rb = blockIdx.x - item * a.rb_per_prob;
    if (a.n_mt_dev && item >= *a.n_mt_dev) return;
    if (item >= a.n_mt) return;
    const int tag = a.mt_list[item];
    const int p = tag >> 16, mt = tag & 0xffff;
    if (p >= a.nprob || (a.nprob_dev && p >= *a.nprob_dev)) return;
    const ColiProb pr = uniform_prob(a.prob[p]);
    const int m0 = mt * COLI_GM_ROWS;
    const int nrows = min(COLI_GM_ROWS, pr.nrows - m0);
    if (nrows <= 0) return;

    int rt[R];
    bool live[R];
    const uint8_t *wr[R], *sr[R];   // tile (rt, 0) of the wave's weights and scales
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int rr = DUAL ? 0 : r;
        rt[r] = (rb * W + wave) * RT + rr;
        live[r] = rt[r] < a.nrt;
        const bool second = DUAL && r == 1;
        const uint8_t *w = (const uint8_t *)(second ? pr.w1 : pr.w0);
        const uint8_t *sc = (const uint8_t *)(second ? pr.s1 : pr.s0);
        // a dead tile re-reads tile (0, q) of the problem: the count of loads
        // stays fixed and no address is hammered by every quad
        const size_t t0 = live[r] ? (size_t)rt[r] * a.nq : 0;
        wr[r] = w + t0 * COLI_TILE_BYTES;
        sr[r] = sc + t0 * SG::kBytes;
    }
    const bool use_lo = *a.haslo >= a.lo_gen;   // >=: stays correct under graph replay
    const int nm = (nrows + 15) >> 4;           // live 16-row subtiles

    // Activation chunks of this wave: c = wave + W k (m = c / 4, j = c % 4);
    // lane l fetches row 16 m + (l & 15) (clamped to the tile's last row),
    // columns 32 j + 8 (l >> 4) .. + 7.
    static_assert(W == 8, "the chunk assignment is written for 8 waves");
    int xoff[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int r = min(16 * ((wave >> 2) + 2 * k) + (lane & 15), nrows - 1);
        const int br = pr.xrow_off + m0 + r;
        const int fr = a.xrows ? a.xrows[br] : br;
        xoff[k] = fr * a.xstride + 32 * (wave & 3) + 8 * (lane >> 4);
    }
    // the ring is written behind the compiler's back: let it escape, so the
    // "memory" clobbers of the waits below force fresh reads (plain loads: no
    // read moves across a wait or barrier, and the compiler may batch the
    // reads of one step)
    asm volatile("" ::"v"(lds) : "memory");

    floatx4 acc[R][4];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < 4; m++) acc[r][m] = (floatx4){0.f, 0.f, 0.f, 0.f};

    auto run = [&](auto lo_tag, auto fold_tag) {
        constexpr bool LO = decltype(lo_tag)::value;
        constexpr bool FOLD = decltype(fold_tag)::value;
        constexpr int PD = LO ? G::kPdLo : G::kPdHi;
        constexpr int ACT = (LO ? 2 : 1) * G::kActHi;   // activation bytes of one stage
        constexpr int L = R + G::kScaleInst + (LO ? 4 : 2);   // DMA instructions per wave and stage
        uint8_t *const wring = lds + PD * ACT + wave * PD * G::kWSlot;
        auto issue = [&](int q, int slot) {
            uint8_t *ws = wring + slot * G::kWSlot;
#pragma unroll
            for (int r = 0; r < R; r++)
                __builtin_amdgcn_global_load_lds((const void *)(wr[r] + (size_t)q * COLI_TILE_BYTES + lane * 16),
                                                 (lds_void *)(ws + r * COLI_TILE_BYTES), 16, 0, 0);
#pragma unroll
            for (int k = 0; k < G::kScaleInst; k++) {
                const int r = min(R - 1, k * SG::kPerInst + lane / SG::kLanes);
                const uint8_t *base = r == 0 ? sr[0] : sr[1];
                __builtin_amdgcn_global_load_lds((const void *)(base + (size_t)q * SG::kBytes + (lane % SG::kLanes) * 4),
                                                 (lds_void *)(ws + 2 * COLI_TILE_BYTES + k * 256), 4, 0, 0);
            }
            uint8_t *xs = lds + slot * ACT;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const size_t o = (size_t)xoff[k] + (size_t)q * 128;
                uint8_t *dst = xs + (wave + W * k) * 1024;
                __builtin_amdgcn_global_load_lds((const void *)(a.xhi + o), (lds_void *)dst, 16, 0, 0);
                if constexpr (LO)
                    __builtin_amdgcn_global_load_lds((const void *)(a.xlo + o), (lds_void *)(dst + G::kActHi), 16,
                                                     0, 0);
            }
        };
        auto compute = [&](int slot) {
            const uint8_t *ws = wring + slot * G::kWSlot;
            const uint8_t *xs = lds + slot * ACT;
            u32x4 w[R];
            ScaleRegs<KIND> sc[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                w[r] = *(const u32x4 *)(ws + r * COLI_TILE_BYTES + lane * 16);
                sc[r].v = *(const decltype(sc[r].v) *)(ws + 2 * COLI_TILE_BYTES + r * SG::kBytes +
                                                       (lane & 15) * sizeof(sc[r].v));
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                half8v bw[R];
                float scl[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    scl[r] = sc[r].get(j);
                    if constexpr (FOLD) bw[r] = unpack_fp4_scaled(w[r][j], scl[r]);
                    else bw[r] = unpack_b<KIND>(w[r][j]);
                }
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    if (m >= nm) break;
                    const uint8_t *fo = xs + (m * 4 + j) * 1024 + lane * 16;
                    const half8v xh = *(const half8v *)fo;
                    half8v xl = xh;
                    if constexpr (LO) xl = *(const half8v *)(fo + G::kActHi);
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        if constexpr (FOLD) {
                            // the operand carries the group scale: accumulate in the MFMA
                            acc[r][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bw[r], acc[r][m], 0, 0, 0);
                            if constexpr (LO)
                                acc[r][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bw[r], acc[r][m], 0, 0, 0);
                        } else {
                            floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bw[r],
                                                                              (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                            if constexpr (LO) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bw[r], d, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 4; i++) acc[r][m][i] = fmaf(d[i], scl[r], acc[r][m][i]);
                        }
                    }
                }
            }
        };
        // Step q: wait for this wave's stage q (at most min(PD - 2, nq - 1 - q)
        // younger stages may stay in flight), barrier (every wave's chunks of
        // stage q have landed, and every wave is done with quad q - 1, whose
        // slot the next issue reuses), issue stage q + PD - 1, compute quad q.
        const int nq = a.nq;
#pragma unroll
        for (int i = 0; i < PD - 1; i++)
            if (i < nq) issue(i, i);
        int slot = 0;
        for (int q = 0; q < nq; q++) {
            dma_wait_tail<L, PD>(min(PD - 2, nq - 1 - q));
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (q + PD - 1 < nq) issue(q + PD - 1, slot == 0 ? PD - 1 : slot - 1);
            compute(slot);
            slot = slot == PD - 1 ? 0 : slot + 1;
        }
    };
    if constexpr (KIND == COLI_KIND_FP4) {
        if (a.fold) {
            if (use_lo) run(std::true_type{}, std::true_type{});
            else run(std::false_type{}, std::true_type{});
        } else if (use_lo) {
            run(std::true_type{}, std::false_type{});
        } else {
            run(std::false_type{}, std::false_type{});
        }
    } else if (use_lo) {
        run(std::true_type{}, std::false_type{});
    } else {
        run(std::false_type{}, std::false_type{});
    }

    // epilogue: batch row m0 + 16 m + 4 (lane / 16) + i, output row rt * 16 + lane % 16
#pragma unroll
    for (int m = 0; m < 4; m++) {
        if (m >= nm) break;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int bl = m * 16 + 4 * (lane >> 4) + i;
            if (bl >= nrows) continue;
            const int br = pr.xrow_off + m0 + bl;
            const int E = a.xexp[a.xrows ? a.xrows[br] : br];
            float *orow = a.out + (size_t)(pr.out_row0 + m0 + bl) * a.ldo;
#pragma unroll
            for (int r = 0; r < RT; r++) {
                if (!live[r]) continue;
                const int o = rt[r] * 16 + (lane & 15);
                if (o >= a.O) continue;
                if constexpr (DUAL)
                    orow[o] = swiglu_out(ldexpf(acc[0][m][i], E), ldexpf(acc[1][m][i], E), a.swiglu_limit);
                else orow[o] = ldexpf(acc[r][m][i], E);
            }
        }
    }
}

template <int KIND>
static hipError_t launch_gemm_kind(const ColiGemmArgs &a, bool dual, hipStream_t st) {
    const dim3 grid((unsigned)a.n_mt * a.rb_per_prob), block(64 * COLI_GM_WAVES);
    const size_t shm = GmGeom<KIND>::kLds;
    if (dual) hipLaunchKernelGGL((coli_gemm_tiles<KIND, true>), grid, block, shm, st, a);
    else hipLaunchKernelGGL((coli_gemm_tiles<KIND, false>), grid, block, shm, st, a);
    return hipGetLastError();
}

// rb_per_prob must cover the output rows: COLI_GM_WAVES x (dual ? 1 : 2) row tiles per block.
extern "C" hipError_t coli_launch_gemm(int kind, int dual, const ColiGemmArgs *a, hipStream_t st) {
    if (a->n_mt <= 0 || a->rb_per_prob <= 0) return hipSuccess;
    if ((long)a->n_mt * a->rb_per_prob > 0x7fffffffL || !a->mt_list) return hipErrorInvalidValue;
    switch (kind) {
    case COLI_KIND_I4_H: return launch_gemm_kind<COLI_KIND_I4_H>(*a, dual != 0, st);
    case COLI_KIND_I4_F: return launch_gemm_kind<COLI_KIND_I4_F>(*a, dual != 0, st);
    case COLI_KIND_FP4: return launch_gemm_kind<COLI_KIND_FP4>(*a, dual != 0, st);
    default: return hipErrorInvalidValue;
    }
}
