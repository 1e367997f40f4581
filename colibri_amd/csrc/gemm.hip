// gemm.hip -- grouped dequant-fused GEMM for gfx950: many-row problems
// (prefill chunks, verification batches), y[b, o] = sum_g scale[o, g] *
// sum_{k in g} x[b, k] w[o, k], the same arithmetic as the GEMV (c/quant.h
// fmt=4 and fmt=7) with the weights read once per 64 rows instead of once per
// 16.
//
// Work item = (problem, 64-row tile, output block of COLI_GM_BLOCK_TILES row
// tiles). A workgroup of COLI_GM_W waves gives each wave R = COLI_GM_BLOCK_TILES
// / COLI_GM_W weight tiles (DUAL: gate/up pairs of the same 16 output rows,
// SwiGLU in the epilogue) over the full K, one 128-column quad per step:
//  * every load of the main loop is an LDS DMA into a ring of PD stages: each
//    wave's weight tiles and their scales (private to the wave), and the
//    quad's activation fragments of the tile's rows (fp16 hi + lo of x * 2^-E,
//    built by coli_prep_frag; shared by the workgroup, each wave fetching a
//    fixed number of the 1 KiB chunks). No load of the loop writes a
//    register, so the compiler inserts no wait of its own: the loop waits with
//    exact s_waitcnt vmcnt(N) for its oldest stage and synchronizes with a
//    bare s_barrier (the fence of __syncthreads() would drain the ring). The
//    activations ride in the same ring as the weights, as deep: loads retire
//    in order, so a shallower activation ring would retire the weights with it;
//  * the chunks are laid out in the MFMA A-operand order (lane l of a DMA
//    fetches the 16 B lane l of the MFMA reads), so the reads are free of bank
//    conflicts; chunks of dead 16-row subtiles read the tile's last row (one
//    cache line) into a trash slot, which keeps the count of loads per stage
//    fixed;
//  * the loop is specialized per (lo parts present, folded scales, live
//    16-row subtiles NM): the stage holds only NM subtiles' activations, so
//    short tiles (the common prefill case of a few rows per expert) stream
//    through a deeper ring, and the MFMA schedule is straight-line code;
//  * each 32-column group is one v_mfma_f32_16x16x32_f16 per (weight tile,
//    live 16-row subtile) -- two with the lo fragments -- its result scaled by
//    the group scale and accumulated in f32. The unpacked B operand of a group
//    is reused by the row subtiles. MXFP4 matrices whose e8m0 scales keep
//    every e2m1 value times its scale a normal fp16 (fold) take the scale into
//    the unpack instead (exact) and accumulate inside the MFMA: no per-group
//    VALU work beyond the conversion.
// Measured limits: the LDS carries the DMA writes and every wave's operand
// reads, and its capacity bounds the ring depth; more tiles per wave (fewer
// activation reads) costs ring depth and occupancy and was slower.
#include <type_traits>

// waves per workgroup; each owns COLI_GM_BLOCK_TILES / COLI_GM_W weight tiles
#ifndef COLI_GM_W
#define COLI_GM_W 8
#endif

#include "coli_device.h"

// deepest ring a short tile gets
#ifndef COLI_GM_PDMAX
#define COLI_GM_PDMAX 6
#endif

// Ring geometry. A stage holds the activation chunks of the tile's live
// 16-row subtiles (NM of them, 4 KiB each for the hi half, as much again for
// lo) and each wave's weight tiles + scales; the ring takes as many stages as
// the LDS of a CU holds (at most 6), so short tiles stream deeper. One 1 KiB
// trash slot takes the DMAs of dead chunks (their count per wave stays fixed).
template <int KIND>
struct GmGeom {
    static constexpr int kMt = COLI_GM_ROWS / 16;                 // 16-row subtiles per tile
    static constexpr int kChunks = 4 * kMt;                        // 1 KiB activation chunks per stage half
    static constexpr int kW = COLI_GM_W, kR = COLI_GM_BLOCK_TILES / COLI_GM_W;   // waves, tiles per wave
    static constexpr int scale_inst(int rn) { return (rn + ScaleGeom<KIND>::kPerInst - 1) / ScaleGeom<KIND>::kPerInst; }
    static constexpr int wslot(int rn) { return rn * COLI_TILE_BYTES + scale_inst(rn) * 256; }
    static constexpr int kTrash = 0;                               // the trash slot, then the ring
    static constexpr int kRing = 1024;
    static constexpr int kLds = 159 * 1024;
    static constexpr int act(int nm, bool lo) { return nm * 4096 * (lo ? 2 : 1); }
    static constexpr int stage(int nm, bool lo, int rn) { return act(nm, lo) + kW * wslot(rn); }
    static constexpr int pd(int nm, bool lo, int rn) {
        return (kLds - kRing) / stage(nm, lo, rn) > COLI_GM_PDMAX ? COLI_GM_PDMAX : (kLds - kRing) / stage(nm, lo, rn);
    }
    // tiles per pass: all of the wave's tiles when three stages fit, else two
    // passes over K of half as many (the activations are staged twice)
    static constexpr int passes(int nm, bool lo) { return pd(nm, lo, kR) >= 3 ? 1 : 2; }
};
static_assert(GmGeom<COLI_KIND_I4_F>::pd(COLI_GM_ROWS / 16, true, GmGeom<COLI_KIND_I4_F>::kR / 2) >= 3,
              "the ring needs three stages");

template <int KIND, bool DUAL>
__global__ __launch_bounds__(64 * COLI_GM_W) void coli_gemm_tiles(ColiGemmArgs a) {
    using G = GmGeom<KIND>;
    using SG = ScaleGeom<KIND>;
    constexpr int W = G::kW;
    constexpr int R = G::kR;                  // weight tiles per wave
    constexpr int RT = DUAL ? R / 2 : R;      // distinct output row tiles per wave
    static_assert(W * R == COLI_GM_BLOCK_TILES && R % 2 == 0, "a block covers COLI_GM_BLOCK_TILES weight tiles");
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
        const int rr = DUAL ? r >> 1 : r;   // DUAL: tiles 2i, 2i + 1 = gate, up of row tile i
        rt[r] = (rb * W + wave) * RT + rr;
        live[r] = rt[r] < a.nrt;
        const bool second = DUAL && (r & 1);
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
    constexpr int CPW = G::kChunks / W;   // chunks per wave and stage half
    static_assert(G::kChunks % W == 0 && W % 4 == 0, "chunks must spread evenly over the waves");
    int xoff[CPW];
#pragma unroll
    for (int k = 0; k < CPW; k++) {
        const int r = min(16 * ((wave + W * k) >> 2) + (lane & 15), nrows - 1);
        const int br = pr.xrow_off + m0 + r;
        const int fr = a.xrows ? a.xrows[br] : br;
        xoff[k] = fr * a.xstride + 32 * (wave & 3) + 8 * (lane >> 4);
    }
    // the ring is written behind the compiler's back: let it escape, so the
    // "memory" clobbers of the waits below force fresh reads (plain loads: no
    // read moves across a wait or barrier, and the compiler may batch the
    // reads of one step)
    asm volatile("" ::"v"(lds) : "memory");

    floatx4 acc[R][G::kMt];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < G::kMt; m++) acc[r][m] = (floatx4){0.f, 0.f, 0.f, 0.f};

    // One pass over K for the wave's tiles RB .. RB + RN - 1.
    auto run = [&](auto lo_tag, auto fold_tag, auto nm_tag, auto rb_tag, auto rn_tag) {
        constexpr bool LO = decltype(lo_tag)::value;
        constexpr bool FOLD = decltype(fold_tag)::value;
        constexpr int NM = decltype(nm_tag)::value;     // live 16-row subtiles
        constexpr int RB = decltype(rb_tag)::value, RN = decltype(rn_tag)::value;
        constexpr int PD = G::pd(NM, LO, RN);
        constexpr int ACT = G::act(NM, LO);             // activation bytes of one stage
        constexpr int LOFF = G::act(NM, false);         // lo half of the stage
        constexpr int SI = G::scale_inst(RN);
        constexpr int WS = G::wslot(RN);
        static_assert(PD >= 3, "the ring needs three stages");
        constexpr int L = RN + SI + (LO ? 2 : 1) * CPW;   // DMA instructions per wave and stage
        uint8_t *const ring = lds + G::kRing;
        uint8_t *const wring = ring + PD * ACT + wave * PD * WS;
        auto issue = [&](int q, int slot) {
            uint8_t *ws = wring + slot * WS;
#pragma unroll
            for (int t = 0; t < RN; t++)
                __builtin_amdgcn_global_load_lds((const void *)(wr[RB + t] + (size_t)q * COLI_TILE_BYTES + lane * 16),
                                                 (lds_void *)(ws + t * COLI_TILE_BYTES), 16, 0, 0);
#pragma unroll
            for (int k = 0; k < SI; k++) {
                const int t = min(RN - 1, k * SG::kPerInst + lane / SG::kLanes);
                const uint8_t *base = sr[RB];   // (branch-free: a per-lane select between RN bases)
#pragma unroll
                for (int tt = 1; tt < RN; tt++)
                    if (t == tt) base = sr[RB + tt];
                __builtin_amdgcn_global_load_lds((const void *)(base + (size_t)q * SG::kBytes + (lane % SG::kLanes) * 4),
                                                 (lds_void *)(ws + RN * COLI_TILE_BYTES + k * 256), 4, 0, 0);
            }
            uint8_t *xs = ring + slot * ACT;
#pragma unroll
            for (int k = 0; k < CPW; k++) {
                const size_t o = (size_t)xoff[k] + (size_t)q * 128;
                const int c = wave + W * k;
                // chunks of dead subtiles read the clamped last row into the trash slot
                uint8_t *dst = c < 4 * NM ? xs + c * 1024 : lds + G::kTrash;
                __builtin_amdgcn_global_load_lds((const void *)(a.xhi + o), (lds_void *)dst, 16, 0, 0);
                if constexpr (LO)
                    __builtin_amdgcn_global_load_lds((const void *)(a.xlo + o),
                                                     (lds_void *)(c < 4 * NM ? dst + LOFF : dst), 16, 0, 0);
            }
        };
        auto compute = [&](int slot) {
            const uint8_t *ws = wring + slot * WS;
            const uint8_t *xs = ring + slot * ACT;
            u32x4 w[RN];
            ScaleRegs<KIND> sc[RN];
#pragma unroll
            for (int t = 0; t < RN; t++) {
                w[t] = *(const u32x4 *)(ws + t * COLI_TILE_BYTES + lane * 16);
                sc[t].v = *(const decltype(sc[t].v) *)(ws + RN * COLI_TILE_BYTES + t * SG::kBytes +
                                                       (lane & 15) * sizeof(sc[t].v));
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                half8v bw[RN];
                float scl[RN];
#pragma unroll
                for (int t = 0; t < RN; t++) {
                    scl[t] = sc[t].get(j);
                    if constexpr (FOLD) bw[t] = unpack_fp4_scaled(w[t][j], scl[t]);
                    else bw[t] = unpack_b<KIND>(w[t][j]);
                }
                half8v xh[NM], xl[NM];
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    const uint8_t *fo = xs + (m * 4 + j) * 1024 + lane * 16;
                    xh[m] = *(const half8v *)fo;
                    if constexpr (LO) xl[m] = *(const half8v *)(fo + LOFF);
                }
                if constexpr (FOLD) {
                    // the operand carries the group scale: accumulate in the MFMA
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int t = 0; t < RN; t++)
                            acc[RB + t][m] =
                                __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[m], bw[t], acc[RB + t][m], 0, 0, 0);
                    if constexpr (LO) {
#pragma unroll
                        for (int m = 0; m < NM; m++)
#pragma unroll
                            for (int t = 0; t < RN; t++)
                                acc[RB + t][m] =
                                    __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[m], bw[t], acc[RB + t][m], 0, 0, 0);
                    }
                } else {
                    floatx4 d[RN][NM];
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int t = 0; t < RN; t++)
                            d[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[m], bw[t],
                                                                             (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    if constexpr (LO) {
#pragma unroll
                        for (int m = 0; m < NM; m++)
#pragma unroll
                            for (int t = 0; t < RN; t++)
                                d[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[m], bw[t], d[t][m], 0, 0, 0);
                    }
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int t = 0; t < RN; t++)
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                acc[RB + t][m][i] = fmaf(d[t][m][i], scl[t], acc[RB + t][m][i]);
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
    // one specialization per (lo parts, folded scales, live subtiles); one
    // pass over K when the ring fits three stages of all the wave's tiles,
    // else one pass per half of them (the next pass refills the ring only
    // after every wave is done with the last one)
    auto by_nm = [&](auto lo_tag, auto fold_tag) {
        auto go = [&](auto nm_tag) {
            constexpr bool LO = decltype(lo_tag)::value;
            constexpr int NM = decltype(nm_tag)::value;
            using C0 = std::integral_constant<int, 0>;
            if constexpr (G::passes(NM, LO) == 1) {
                run(lo_tag, fold_tag, nm_tag, C0{}, std::integral_constant<int, R>{});
            } else {
                using H = std::integral_constant<int, R / 2>;
                run(lo_tag, fold_tag, nm_tag, C0{}, H{});
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                run(lo_tag, fold_tag, nm_tag, H{}, H{});
            }
        };
        static_assert(G::kMt == 4, "the subtile dispatch is written for 64-row tiles");
        if (nm == 1) go(std::integral_constant<int, 1>{});
        else if (nm == 2) go(std::integral_constant<int, 2>{});
        else if (nm == 3) go(std::integral_constant<int, 3>{});
        else go(std::integral_constant<int, 4>{});
    };
    auto by_lo = [&](auto fold_tag) {
        if (use_lo) by_nm(std::true_type{}, fold_tag);
        else by_nm(std::false_type{}, fold_tag);
    };
    if constexpr (KIND == COLI_KIND_FP4) {
        if (a.fold) by_lo(std::true_type{});
        else by_lo(std::false_type{});
    } else {
        by_lo(std::false_type{});
    }

    // epilogue: batch row m0 + 16 m + 4 (lane / 16) + i, output row rt * 16 + lane % 16
#pragma unroll
    for (int m = 0; m < G::kMt; m++) {
        if (m >= nm) break;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int bl = m * 16 + 4 * (lane >> 4) + i;
            if (bl >= nrows) continue;
            const int br = pr.xrow_off + m0 + bl;
            const int E = a.xexp[a.xrows ? a.xrows[br] : br];
            float *orow = a.out + (size_t)(pr.out_row0 + m0 + bl) * a.ldo;
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const int r = DUAL ? 2 * t : t;   // the gate (DUAL) or the plain tile of row tile t
                if (!live[r]) continue;
                const int o = rt[r] * 16 + (lane & 15);
                if (o >= a.O) continue;
                if constexpr (DUAL)
                    orow[o] = swiglu_out(ldexpf(acc[r][m][i], E), ldexpf(acc[r + 1][m][i], E), a.swiglu_limit);
                else orow[o] = ldexpf(acc[r][m][i], E);
            }
        }
    }
}

template <int KIND>
static hipError_t launch_gemm_kind(const ColiGemmArgs &a, bool dual, hipStream_t st) {
    const dim3 grid((unsigned)a.n_mt * a.rb_per_prob), block(64 * COLI_GM_W);
    const size_t shm = GmGeom<KIND>::kLds;
    if (dual) hipLaunchKernelGGL((coli_gemm_tiles<KIND, true>), grid, block, shm, st, a);
    else hipLaunchKernelGGL((coli_gemm_tiles<KIND, false>), grid, block, shm, st, a);
    return hipGetLastError();
}

// rb_per_prob must cover the output rows: 8 (dual) or 16 row tiles per block.
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
