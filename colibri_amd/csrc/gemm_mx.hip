// gemm_mx.hip -- grouped MXFP4 GEMM on the CDNA4 block-scaled MFMA.
//
// y[b, o] = sum_g 2^(e[o,g]-127) * sum_{k in g} x[b, k] * e2m1[o, k]
// (c/quant.h:1391-1440, fmt=7) for problems of many rows (prefill chunks,
// verification batches), on v_mfma_scale_f32_16x16x128_f8f6f4: the hardware
// reads the e2m1 codes as they are stored and applies both e8m0 block scales
// itself, so the loop issues no unpack and no scale arithmetic at all.
//
// Operands of one 16x16x128 MFMA (measured on gfx950):
//  * B (weights, fp4): lane (c, g) holds row c's 32 codes of K-block g
//    (16 B, low nibble first) and that block's e8m0 scale. The stored tile
//    gives lane (c, ks) 8 codes of each of the 4 groups (the GEMV's
//    16x16x32 order), so each tile is transposed in registers first: a 4x4
//    dword transpose across the four 16-lane rows, two v_permlane32_swap
//    and two v_permlane16_swap.
//  * A (activations, fp8 e4m3): lane (m, g) holds row m's K in [16g, 16g+16)
//    in bytes 0-15 and [64+16g, 64+16g+16) in bytes 16-31; the scale of
//    K-block b comes from lane (m, b).
//  * D: lane l, register i = row 4(l/16)+i, column l%16.
// The activations arrive as e4m3 pieces (coli_prep_fp8): x = sum_k p_k *
// 2^(s_k), each piece with its own e8m0 scale per 32 elements, piece k
// holding the rounding residual of the pieces before it; each piece adds 4
// significant bits. bf16 activations are exact in two pieces (up to 2^-21 of
// the block maximum for elements far below it), and the GEMM then runs two;
// otherwise it runs four (16 bits per element). The pieces chain into the
// same accumulator, the quads too: the MFMA accumulator is the result.
//
// Work item = (problem, 64-row tile, output block), as coli_gemm_tiles: a
// workgroup of 8 waves, 2 weight tiles per wave (DUAL: the gate and the up
// tile of the same 16 rows, SwiGLU in the epilogue) over the full K, weights
// through a 3-stage register ring, the 64 rows' pieces staged per quad into
// LDS (double-buffered, rows padded to 144 B so the 16 lanes of one k-slice
// hit distinct banks).
#include "coli_device.h"

typedef int i32x8 __attribute__((ext_vector_type(8)));

#define COLI_MX_ROW 144   // LDS bytes per staged row of one piece (128 + pad)
#define COLI_MX_NP 4      // pieces produced; the GEMM uses 2 when the activations allow


// e4m3 (fn) encode with round-to-nearest-even; |v| <= 256 here (the block
// scale keeps it there), so no saturation case arises.
__device__ __forceinline__ uint32_t e4m3_rne(float v, float &dec) {
    const uint32_t sgn = v < 0.0f ? 0x80u : 0u;
    const float a = fabsf(v);
    uint32_t code;
    if (a < 0.015625f) {   // subnormal: multiples of 2^-9
        const float sc = a * 512.0f;
        uint32_t q = (uint32_t)sc;
        const float fr = sc - (float)q;
        if (fr > 0.5f || (fr == 0.5f && (q & 1u))) q++;
        code = q;          // q == 8 is the smallest normal (exponent field 1)
        dec = (float)q * (1.0f / 512.0f);
    } else {
        const uint32_t bits = __builtin_bit_cast(uint32_t, a);
        const int e = (int)((bits >> 23) & 0xff) - 127;
        uint32_t sig = (0x800000u | (bits & 0x7fffffu));
        uint32_t keep = sig >> 20, rest = sig & 0xfffffu;
        if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) keep++;
        dec = ldexpf((float)keep, e - 3);
        int ee = e;
        if (keep == 16u) {   // rounded up to the next binade
            keep = 8u;
            ee++;
        }
        code = (uint32_t)((ee + 7) << 3) | (keep & 7u);
    }
    if (sgn) dec = -dec;
    return sgn | code;
}

// One thread per (row, 32-column block): NP pieces of the block, each written
// as two 16 B chunks at their A-operand positions, and its scale byte. After
// the second piece the residual is compared with the block maximum: above
// 2^-20 of it (more than bf16 precision in the activations) the block needs
// all NP pieces, and the launch's flag is raised to `gen` (compared with >=
// by the GEMM, so it needs no clearing and stays correct under graph replay).
template <int NP>
__global__ __launch_bounds__(256) void coli_prep_fp8(const float *__restrict__ x, int ldx, const int *__restrict__ src_row,
                                                     const int *__restrict__ nrows_dev, int nrows, int K, int nq,
                                                     int prow, uint8_t *__restrict__ p8, uint8_t *__restrict__ s8,
                                                     int *__restrict__ more, int gen) {
    const int nb = nq * 4;
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    bool need = false;
    if (t < (long)nrows * nb) {
        const int r = (int)(t / nb), blk = (int)(t - (long)r * nb);
        const int srow = src_row ? src_row[r] : r;
        if ((!nrows_dev || r < *nrows_dev) && srow >= 0) {
            const float *xr = x + (size_t)srow * ldx;
            float v[32];
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const int k = blk * 32 + i;
                v[i] = k < K ? xr[k] : 0.0f;
            }
            const int q = blk >> 2, b = blk & 3;
            // positions of this block's two 16-element halves inside the quad's 128 B
            const int k0 = 32 * b, k1 = 32 * b + 16;
            const int pos0 = 32 * ((k0 & 63) >> 4) + 16 * (k0 >> 6), pos1 = 32 * ((k1 & 63) >> 4) + 16 * (k1 >> 6);
            float m0 = 0.0f;
#pragma unroll
            for (int p = 0; p < NP; p++) {
                float m = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; i++) m = fmaxf(m, fabsf(v[i]));
                if (p == 0) m0 = m;
                if (p == 2) need = m > ldexpf(m0, -20);
                int se = 0;
                if (m > 0.0f && isfinite(m)) {
                    int e;
                    frexpf(m, &e);          // m in [2^(e-1), 2^e)
                    se = e - 1 - 7;         // m * 2^-se in [128, 256)
                    se = max(-127, min(127, se));
                }
                uint32_t c[32];
#pragma unroll
                for (int i = 0; i < 32; i++) {
                    float d;
                    c[i] = e4m3_rne(ldexpf(v[i], -se), d);
                    v[i] -= ldexpf(d, se);
                }
                uint8_t *dst = p8 + (((size_t)p * prow + r) * nq + q) * 128;
                u32x4 w0, w1;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    w0[j] = c[4 * j] | (c[4 * j + 1] << 8) | (c[4 * j + 2] << 16) | (c[4 * j + 3] << 24);
                    w1[j] = c[16 + 4 * j] | (c[16 + 4 * j + 1] << 8) | (c[16 + 4 * j + 2] << 16) |
                            (c[16 + 4 * j + 3] << 24);
                }
                *(u32x4 *)(dst + pos0) = w0;
                *(u32x4 *)(dst + pos1) = w1;
                s8[(((size_t)p * prow + r) * nq + q) * 4 + b] = (uint8_t)(se + 127);
            }
        }
    }
    if (__builtin_amdgcn_ballot_w64(need) && (threadIdx.x & 63) == 0 &&
        __hip_atomic_load(more, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gen)   // skip once raised
        atomicMax(more, gen);
}

// 4x4 dword transpose across the four 16-lane rows: lane (c, g) ends with
// dword g of lanes (c, 0..3).
__device__ __forceinline__ u32x4 tile_to_mx(u32x4 x) {
    const auto a = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    return (u32x4){c[0], c[1], d[0], d[1]};
}

template <bool DUAL, int NP, int NPMAX>
__device__ __forceinline__ void gemm_mx_body(const ColiGemmMxArgs &a, uint8_t *lds, int p, int mt, int rb) {
    constexpr int W = COLI_GM_WAVES;
    constexpr int R = 2;                 // weight tiles per wave
    constexpr int RT = DUAL ? 1 : 2;     // distinct output row tiles per wave
    constexpr int PD = 3;
    constexpr int PIECE = 64 * COLI_MX_ROW;
    constexpr int BUF = NPMAX * PIECE + NPMAX * 64 * 4;   // pieces + their scale words
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
    struct Stage {
        u32x4 w[R];
        uint32_t sc[R];
    };
    auto load_w = [&](Stage &sg, int q) {
        const bool valid = q < a.nq;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const size_t tq = valid ? tbase[r] + (size_t)q * tstep[r] : 0;
            const uint8_t *w = valid ? wb[r] : a.zero;
            const uint8_t *sp = valid ? (const uint8_t *)sb[r] : a.zero;
            sg.w[r] = __builtin_nontemporal_load(GPTR(u32x4, w + tq * COLI_TILE_BYTES) + lane);
            sg.sc[r] = *GPTR(uint32_t, sp + (tq * 16 + (lane & 15)) * 4);
        }
    };
    Stage st[PD];
    load_w(st[0], 0);
    load_w(st[1], 1);

    // Staging assignment: NP*64 rows of 8 chunks of 16 B per quad; thread t
    // takes chunks t + 512 k; threads 0 .. NP*64-1 also move one scale word.
    // Only the live 16-row subtiles are staged.
    const int nm = (nrows + 15) >> 4;   // live 16-row subtiles
    constexpr int NCH = NP * 64 * 8, CPT = (NCH + 64 * W - 1) / (64 * W);
    const uint8_t *csrc[CPT];
    int cstep[CPT];
    unsigned cdst[CPT];
    bool cact[CPT];
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int c = threadIdx.x + 64 * W * k;
        const int pc = c / 512, r = (c >> 3) & 63, ch = c & 7;
        cact[k] = c < NCH && r < nm * 16;
        cdst[k] = pc * PIECE + r * COLI_MX_ROW + ch * 16;
        if (cact[k] && r < nrows) {
            const int br = pr.xrow_off + m0 + r;
            const int fr = a.xrows ? a.xrows[br] : br;
            csrc[k] = a.p8 + (((size_t)pc * a.prow + fr) * a.nq) * 128 + ch * 16;
            cstep[k] = 128;
        } else {
            csrc[k] = a.zero;
            cstep[k] = 0;
        }
    }
    const bool sact = threadIdx.x < NP * 64 && (int)(threadIdx.x & 63) < nm * 16;
    const uint8_t *ssrc;
    int sstep;
    {
        const int pc = threadIdx.x / 64, r = threadIdx.x & 63;
        if (sact && r < nrows) {
            const int br = pr.xrow_off + m0 + r;
            const int fr = a.xrows ? a.xrows[br] : br;
            ssrc = (const uint8_t *)(a.s8 + ((size_t)pc * a.prow + fr) * a.nq);
            sstep = 4;
        } else {
            ssrc = a.zero;
            sstep = 0;
        }
    }
    const unsigned sdst = NPMAX * PIECE + threadIdx.x * 4;
    u32x4 creg[PD][CPT];
    uint32_t sreg[PD];
    auto gload = [&](int slot, int q) {
#pragma unroll
        for (int k = 0; k < CPT; k++)
            if (cact[k]) creg[slot][k] = *GPTR(u32x4, csrc[k] + (size_t)q * cstep[k]);
        if (sact) sreg[slot] = *GPTR(uint32_t, ssrc + (size_t)q * sstep);
    };
    auto swrite = [&](int slot, int buf) {
#pragma unroll
        for (int k = 0; k < CPT; k++)
            if (cact[k]) *(u32x4 *)(lds + buf * BUF + cdst[k]) = creg[slot][k];
        if (sact) *(uint32_t *)(lds + buf * BUF + sdst) = sreg[slot];
    };

    floatx4 acc[R][4];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < 4; m++) acc[r][m] = (floatx4){0.f, 0.f, 0.f, 0.f};
    const int g = lane >> 4;
    auto compute = [&](const Stage &sg, int buf) {
        i32x8 bw[R];
        int bs[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const u32x4 t = tile_to_mx(sg.w[r]);
            bw[r] = (i32x8){(int)t[0], (int)t[1], (int)t[2], (int)t[3], 0, 0, 0, 0};
            bs[r] = (int)(sg.sc[r] >> (8 * g));
        }
        const uint8_t *base = lds + buf * BUF;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            if (m >= nm) break;
#pragma unroll
            for (int pc = 0; pc < NP; pc++) {
                const uint8_t *arow = base + pc * PIECE + (m * 16 + (lane & 15)) * COLI_MX_ROW + 32 * g;
                const u32x4 a0 = *(const u32x4 *)arow, a1 = *(const u32x4 *)(arow + 16);
                const i32x8 av = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                                  (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
                const int as = (int)(*(const uint32_t *)(base + NPMAX * PIECE + (pc * 64 + m * 16 + (lane & 15)) * 4) >>
                                     (8 * g));
#pragma unroll
                for (int r = 0; r < R; r++)
                    acc[r][m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bw[r], acc[r][m], 0, 4, 0, as,
                                                                                0, bs[r]);
            }
        }
    };

    gload(0, 0);
    if (a.nq > 1) gload(1, 1);
    swrite(0, 0);
    __syncthreads();
    for (int q0 = 0; q0 < a.nq; q0 += PD) {
#pragma unroll
        for (int u = 0; u < PD; u++) {
            const int q = q0 + u;
            if (q >= a.nq) break;
            if (q + 2 < a.nq) gload((u + 2) % PD, q + 2);
            load_w(st[(u + PD - 1) % PD], q + PD - 1);
            compute(st[u], q & 1);
            if (q + 1 < a.nq) swrite((u + 1) % PD, (q + 1) & 1);
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
            float *orow = a.out + (size_t)(pr.out_row0 + m0 + bl) * a.ldo;
#pragma unroll
            for (int r = 0; r < RT; r++) {
                if (!live[r]) continue;
                const int o = rt[r] * 16 + (lane & 15);
                if (o >= a.O) continue;
                if constexpr (DUAL) orow[o] = swiglu_out(acc[0][m][i], acc[1][m][i], a.swiglu_limit);
                else orow[o] = acc[r][m][i];
            }
        }
    }
}

template <bool DUAL>
__global__ __launch_bounds__(64 * COLI_GM_WAVES) void coli_gemm_mx(ColiGemmMxArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int item = blockIdx.x / a.rb_per_prob, rb = blockIdx.x - item * a.rb_per_prob;
    if (a.n_mt_dev && item >= *a.n_mt_dev) return;
    if (item >= a.n_mt) return;
    const int tag = a.mt_list[item];
    const int p = tag >> 16, mt = tag & 0xffff;
    if (p >= a.nprob || (a.nprob_dev && p >= *a.nprob_dev)) return;
    if (*a.more >= a.more_gen) gemm_mx_body<DUAL, COLI_MX_NP, COLI_MX_NP>(a, lds, p, mt, rb);
    else gemm_mx_body<DUAL, 2, COLI_MX_NP>(a, lds, p, mt, rb);
}


extern "C" hipError_t coli_launch_prep_fp8(const float *x, int ldx, const int *src_row, const int *nrows_dev,
                                           int nrows, int K, int nq, int prow, uint8_t *p8, uint8_t *s8, int *more,
                                           int gen, hipStream_t st) {
    if (nrows <= 0) return hipSuccess;
    const long n = (long)nrows * nq * 4;
    hipLaunchKernelGGL(coli_prep_fp8<COLI_MX_NP>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, ldx,
                       src_row, nrows_dev, nrows, K, nq, prow, p8, s8, more, gen);
    return hipGetLastError();
}

extern "C" int coli_mx_pieces(void) { return COLI_MX_NP; }

// rb_per_prob must cover the output rows: COLI_GM_WAVES x (dual ? 1 : 2) row tiles per block.
extern "C" hipError_t coli_launch_gemm_mx(int dual, const ColiGemmMxArgs *a, hipStream_t st) {
    if (a->n_mt <= 0 || a->rb_per_prob <= 0) return hipSuccess;
    if ((long)a->n_mt * a->rb_per_prob > 0x7fffffffL || !a->mt_list) return hipErrorInvalidValue;
    const dim3 grid((unsigned)a->n_mt * a->rb_per_prob), block(64 * COLI_GM_WAVES);
    constexpr size_t shm = 2 * (COLI_MX_NP * 64 * COLI_MX_ROW + COLI_MX_NP * 64 * 4);
    if (dual) hipLaunchKernelGGL((coli_gemm_mx<true>), grid, block, shm, st, *a);
    else hipLaunchKernelGGL((coli_gemm_mx<false>), grid, block, shm, st, *a);
    return hipGetLastError();
}
