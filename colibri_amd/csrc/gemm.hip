// gemm.hip -- grouped dequant-fused GEMM for gfx950: many-row problems
// (prefill chunks, verification batches), y[b, o] = sum_g scale[o, g] *
// sum_{k in g} x[b, k] w[o, k], the same arithmetic as the GEMV (c/quant.h
// fmt=4 and fmt=7) with the weights read once per 64 rows instead of once per
// 16.
//
// Work item = (problem, 64-row tile, output block). A workgroup of
// COLI_GM_WAVES waves owns 2 row tiles per wave (DUAL: the gate tile and the up
// tile of the same 16 rows, SwiGLU in the epilogue) over the full K:
//  * each wave streams its own weight tiles through a 3-stage register ring;
//  * the 64 rows' activation fragments (fp16 hi + lo of x * 2^-E, built by
//    coli_prep_frag) are staged per 128-column quad into LDS, double-buffered,
//    and read back in the MFMA A-operand order (conflict-free 16-byte lanes);
//  * each 32-column group is one v_mfma_f32_16x16x32_f16 per (row tile,
//    16-row subtile), its result scaled by the group scale and accumulated.
// The unpacked B operand of a group is reused by the 4 row subtiles.
#include "coli_device.h"

template <int KIND>
struct GmStage {
    u32x4 w[2];
    ScaleRegs<KIND> sc[2];
};

template <int KIND, bool DUAL>
__global__ __launch_bounds__(64 * COLI_GM_WAVES) void coli_gemm_tiles(ColiGemmArgs a) {
    constexpr int W = COLI_GM_WAVES;
    constexpr int R = 2;                 // weight tiles per wave
    constexpr int RT = DUAL ? 1 : 2;     // distinct output row tiles per wave
    constexpr int PD = 3;
    constexpr int BUF = 32768;           // one staging buffer: hi 16 KiB + lo 16 KiB
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
    const uint8_t *wb[R];
    const void *sb[R];
    size_t tbase[R];
    int tstep[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int rr = DUAL ? 0 : r;
        rt[r] = (rb * W + wave) * RT + rr;
        live[r] = rt[r] < a.nrt;
        const bool second = DUAL && r == 1;
        wb[r] = live[r] ? (second ? pr.w1 : pr.w0) : a.zero;
        sb[r] = live[r] ? (second ? pr.s1 : pr.s0) : (const void *)a.zero;
        tbase[r] = live[r] ? (size_t)rt[r] * a.nq : 0;
        tstep[r] = live[r] ? 1 : 0;
    }
    auto load_w = [&](GmStage<KIND> &sg, int q) {
        const bool valid = q < a.nq;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const size_t tq = valid ? tbase[r] + (size_t)q * tstep[r] : 0;
            const uint8_t *w = valid ? wb[r] : a.zero;
            const void *sp = valid ? sb[r] : (const void *)a.zero;
            sg.w[r] = __builtin_nontemporal_load(GPTR(u32x4, w + tq * COLI_TILE_BYTES) + lane);
            sg.sc[r].load(sp, tq, lane & 15);
        }
    };
    GmStage<KIND> st[PD];
    load_w(st[0], 0);
    load_w(st[1], 1);

    const bool use_lo = *a.haslo >= a.lo_gen;   // >=: stays correct under graph replay
    // Staging assignment: 2048 chunks of 16 B per quad (64 rows x 16 hi + 16
    // lo fragments); thread t takes chunks t + 512 k, all of one half (hi or
    // lo, t & 16), so the lo threads idle when no lo part is non-zero.
    const _Float16 *src[4];
    int sstep[4];
    unsigned dst[4];
    const int hl = (threadIdx.x >> 4) & 1;
    const bool stager = !hl || use_lo;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int c = threadIdx.x + 64 * W * k;
        const int r = c >> 5, f = c & 15, j = f >> 2, ks = f & 3, m = r >> 4, b = r & 15;
        if (r < nrows) {
            const int br = pr.xrow_off + m0 + r;
            const int fr = a.xrows ? a.xrows[br] : br;
            src[k] = (hl ? a.xlo : a.xhi) + (size_t)fr * a.xstride + f * 8;
            sstep[k] = 128;
        } else {
            src[k] = (const _Float16 *)a.zero;
            sstep[k] = 0;
        }
        // the 16 chunks of one row sit on 16 consecutive lanes: their slots are
        // XOR-swizzled by the chunk (f = 4 j + ks) so those lanes write 16
        // different bank groups, and the MFMA read below (16 rows of one
        // chunk) stays conflict-free
        dst[k] = hl * 16384 + (((m * 4 + j) * 4 + ks) * 16 + (b ^ f)) * 16;
    }
    // Activation staging ring: quad q's fragments are read into registers two
    // iterations ahead (slot q % 3) and written to LDS one iteration ahead, so
    // their L2 latency is covered by a full iteration of math.
    u32x4 creg[PD][4];
    auto gload = [&](u32x4 (&cr)[4], int q) {
        if (!stager) return;
#pragma unroll
        for (int k = 0; k < 4; k++) cr[k] = *GPTR(u32x4, src[k] + (size_t)q * sstep[k]);
    };
    auto swrite = [&](const u32x4 (&cr)[4], int buf) {
        if (!stager) return;
#pragma unroll
        for (int k = 0; k < 4; k++) *(u32x4 *)(lds + buf * BUF + dst[k]) = cr[k];
    };

    floatx4 acc[R][4];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < 4; m++) acc[r][m] = (floatx4){0.f, 0.f, 0.f, 0.f};
    const int nm = (nrows + 15) >> 4;   // live 16-row subtiles
    auto compute = [&](const GmStage<KIND> &sg, int buf) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            half8v bw[R];
            float scl[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                bw[r] = unpack_b<KIND>(sg.w[r][j]);
                scl[r] = sg.sc[r].get(j);
            }
#pragma unroll
            for (int m = 0; m < 4; m++) {
                if (m >= nm) break;
                const unsigned fo =
                    buf * BUF + ((((m * 4 + j) * 4 + (lane >> 4)) * 16 + ((lane & 15) ^ (4 * j + (lane >> 4)))) * 16);
                const half8v xh = *(const half8v *)(lds + fo);
                half8v xl = xh;
                if (use_lo) xl = *(const half8v *)(lds + 16384 + fo);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bw[r], (floatx4){0.f, 0.f, 0.f, 0.f},
                                                                      0, 0, 0);
                    if (use_lo) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bw[r], d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[r][m][i] = fmaf(d[i], scl[r], acc[r][m][i]);
                }
            }
        }
    };

    static_assert(PD == 3, "the staging ring below is written for three slots");
    gload(creg[0], 0);
    if (a.nq > 1) gload(creg[1], 1);
    swrite(creg[0], 0);
    __syncthreads();
    for (int q0 = 0; q0 < a.nq; q0 += PD) {
#pragma unroll
        for (int u = 0; u < PD; u++) {
            const int q = q0 + u;
            if (q >= a.nq) break;
            if (q + 2 < a.nq) gload(creg[(u + 2) % PD], q + 2);
            load_w(st[(u + PD - 1) % PD], q + PD - 1);
            compute(st[u], q & 1);
            if (q + 1 < a.nq) swrite(creg[(u + 1) % PD], (q + 1) & 1);
            __syncthreads();
        }
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
    const size_t shm = 2 * 32768;
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
