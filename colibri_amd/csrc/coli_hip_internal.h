// coli_hip_internal.h -- shared types of the gfx950 backend (libcoli_hip.so).
//
// Device data layout ("MI355X tiles"), chosen at upload time:
//   A quantized matrix W[O, I] (int4 offset-binary or e2m1 nibbles) is padded
//   to Op = ceil16(O) rows and Ip = ceil128(I) columns and cut into tiles of
//   16 rows x 128 columns (4 groups of 32). A tile is 1 KiB; within it, lane l
//   of a wave owns the 16 bytes at l*16: dword j holds the 8 nibbles of row
//   (l % 16), columns [32*(4q+j) + 8*(l/16), +8) in the source byte order.
//   One global_load_dwordx4 per lane therefore streams a whole tile with
//   perfect coalescing, and every nibble lands in the lane that feeds it to
//   the MFMA B operand. Tiles are ordered [row_tile][quad] so a wave walking K
//   for one row tile reads contiguous memory.
//   Group scales are stored tile-ordered as well: [row_tile][quad][16][4] of
//   fp16 (int4 whose f32 scales are exactly fp16), f32 (other int4), or e8m0
//   bytes (MXFP4). Padding carries value 0 (nibble 8 / code 0, scale 0).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define COLI_TILE_ROWS 16
#define COLI_TILE_COLS 128
#define COLI_TILE_BYTES 1024
#define COLI_GROUP 32
#define COLI_DESC_ROWS 64
#define COLI_ZERO_BYTES (1u << 20)   // covers one fragment row of I <= 512K and a tile + its scales

// Tensor storage kinds.
enum ColiKind {
    COLI_KIND_I4_H = 0,     // int4, fp16 group scales (tiled)
    COLI_KIND_I4_F = 1,     // int4, f32 group scales (tiled)
    COLI_KIND_FP4 = 2,      // MXFP4 e2m1 + e8m0 (tiled)
    COLI_KIND_GENERIC = 3,  // int4 with a group size that is not a multiple of 32:
                            // source layout kept, scalar kernel
};

struct ColiCudaTensor {
    int fmt, I, O, device, gs;   // ABI view (fmt as passed, gs 0 = per-row)
    int kind;
    int Op, Ip, nrt, nq;         // tiled geometry
    uint8_t *w;                  // tiles (or raw rows for GENERIC)
    void *sc;                    // scale tiles (or raw f32 [O, ng] for GENERIC)
    size_t w_bytes, sc_bytes;
    int ng_src;                  // scale groups per source row (GENERIC)
    size_t accounted;            // bytes charged to the device statistics
    struct ColiProb *desc;       // device: 64 descriptors, entry s-1 = this matrix on s rows
    void *sc_unit;               // fmt=2 int8-activation path: unit group scales (made on first use)
    int e8_fold;                 // MXFP4: every e8m0 byte in [114, 140], so each e2m1 value times its
                                 // scale is a normal fp16 (the GEMM folds the scale into the operand)
};

// One GEMV problem: a matrix (or a gate/up pair) applied to a set of batch rows.
struct ColiProb {
    const uint8_t *w0;  const void *s0;   // matrix (plain) or gate (dual)
    const uint8_t *w1;  const void *s1;   // up (dual)
    int nrows;                            // batch rows of this problem
    int xrow_off;                         // -> xrows[]: fragment row per batch row
    int out_row0;                         // first output row (rows are consecutive)
    int pad;
};

// One activation-fragment build (coli_prep_frag): nblocks 256-thread blocks,
// nchunk per row.
struct ColiPrepArgs {
    const float *x;
    const int *src_row;
    const int *nrows_dev;
    _Float16 *hi;
    _Float16 *lo;
    int *exp2out;
    int *haslo;
    const float *zero;
    int ldx, K, ngp, int4_order, gen, vec, nchunk, nblocks;
};

struct ColiGemvArgs {
    const ColiProb *prob;     // device descriptors; null: the single problem prob0
    ColiProb prob0;
    const int *nprob_dev;     // if non-null, number of live problems (device)
    int nprob;                // upper bound (grid sizing)
    int nrt, nq, O;           // tiles, real output rows
    int n_bt;                 // 16-row batch tiles per problem
    int rb_per_prob;          // row blocks per problem
    int splits, qps;          // K split
    const int *xrows;         // fragment row of batch row r = xrows[xrow_off + r] (null: xrow_off + r)
    const _Float16 *xhi, *xlo;
    int xstride;              // halves per fragment row (= ngp * 32)
    const int *xexp;          // per fragment row
    const int *haslo;         // == lo_gen when some lo part of this fragment set is non-zero
    int lo_gen;
    const float *xf;          // non-null (coli_gemv_dma only): f32 activations, row r = xf + xrows-mapped r * ldx
    int ldx;
    int xstage;               // with xf and one row per problem: convert the row once per group into LDS
    const _Float16 *zero;     // >= COLI_ZERO_BYTES of zeros: inactive batch lanes, dead tiles
    float *out;
    int ldo;
    float swiglu_limit;       // > 0: DeepSeek-V4 clamped SwiGLU in the DUAL epilogue
    // MXFP4 whose every e8m0 byte lies in [114, 140] (ColiCudaTensor::e8_fold):
    // each e2m1 value times its block scale is an exact normal fp16, produced
    // by the conversion itself, so the MFMAs accumulate across groups with no
    // per-group scale arithmetic. Taken by coli_gemv_dma (not with per-group
    // activation exponents, gexp); coli_gemv_tiles keeps the per-group form
    // (its folded variant spilled more registers and measured slower).
    int fold;
    float *partial;           // split-K partials: [instance][split][R][NB4][64]
    int *split_cnt;           // split-K arrival counters, one per instance; zero between launches
    // Fragments emitted by the GEMV that produced x (coli_hip_gemm_run_dev_emit):
    // one exponent per (fragment row, 32-column group) instead of xexp, as
    // signed bytes E (-126 .. 113), laid out [quad][gexp_rows][4 groups].
    // Null: per-row xexp.
    const uint8_t *gexp;
    int gexp_rows;
    // Emission of this GEMV's output (single plain matrix, R even, no K
    // split) as the fragments of the GEMV that consumes it: hi / lo halves
    // [row][estride] in that GEMV's A-operand order (eint4: int4 order with
    // the high-nibble columns scaled by 1/16), exponents as gexp above.
    _Float16 *ehi, *elo;
    uint8_t *eexp;
    int estride, erows, eint4;
};


// Grouped GEMM (prefill): problems of many rows, tiled 64 rows x
// COLI_GM_BLOCK_TILES row tiles (half as many gate/up pairs when dual) with
// the activation fragments staged in LDS. COLI_GM_WAVES: the block-scaled
// variant (gemm_mx.hip), 8 waves x 2 row tiles.
#define COLI_GM_WAVES 8
#define COLI_GM_BLOCK_TILES 16
#ifndef COLI_GM_ROWS
#define COLI_GM_ROWS 64
#endif

struct ColiGemmArgs {
    const ColiProb *prob;
    const int *nprob_dev;     // live problems (device); null: nprob
    int nprob;
    const int *mt_list;       // work list of (problem << 16 | row tile); null: tile i of problem 0..
    const int *n_mt_dev;      // live entries of mt_list (device)
    int n_mt;                 // upper bound of the list (grid sizing)
    int nrt, nq, O;
    int rb_per_prob;          // output blocks of COLI_GM_WAVES x 2 row tiles (dual: x 1 gate + 1 up)
    const int *xrows;         // fragment row of batch row r = xrows[xrow_off + r] (null: xrow_off + r)
    const _Float16 *xhi, *xlo;
    int xstride;              // halves per fragment row
    const int *xexp;
    const int *haslo;
    int lo_gen;
    const uint8_t *zero;
    float *out;
    int ldo;
    float swiglu_limit;       // > 0: DeepSeek-V4 clamped SwiGLU in the DUAL epilogue
    int fold;                 // MXFP4, every matrix e8_fold: scales folded into the unpacked operand
};

// Grouped MXFP4 GEMM on the block-scaled MFMA (gemm_mx.hip): activations as
// e4m3 pieces with e8m0 scales per 32 columns (coli_prep_fp8).
struct ColiGemmMxArgs {
    const ColiProb *prob;
    const int *nprob_dev;
    int nprob;
    const int *mt_list;
    const int *n_mt_dev;
    int n_mt;
    int nrt, nq, O;
    int rb_per_prob;
    const int *xrows;          // piece row of batch row r = xrows[xrow_off + r] (null: xrow_off + r)
    const uint8_t *p8;         // [NP][prow][nq][128] permuted e4m3 codes
    const uint32_t *s8;        // [NP][prow][nq] e8m0 bytes of the quad's 4 blocks
    int prow;                  // rows per piece plane
    const int *more;           // >= more_gen: some block needs all pieces (else two)
    int more_gen;
    const uint8_t *zero;
    float *out;
    int ldo;
    float swiglu_limit;       // > 0: DeepSeek-V4 clamped SwiGLU in the DUAL epilogue
};

// Numeric helpers shared by host and device.
static inline int coli_ceil_div(int a, int b) { return (a + b - 1) / b; }
