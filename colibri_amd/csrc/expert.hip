// expert.hip -- compute entry points of the coli_cuda_* ABI on gfx950.
//
// All expert-path entry points share one runner: fragments of the input rows
// -> one dual (gate+up, SwiGLU epilogue) launch per storage kind -> fragments
// of the hidden rows -> one down launch per storage kind. Everything runs on
// the device context's stream; host entry points stage through pinned
// buffers (c/backend_cuda.cu:1550-1676 for the reference's sync group call,
// 1677-1812 for issue/take).
#include "coli_hip_host.h"


#include "coli_backend_abi.h"
#include "coli_hip_ext.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

// ---------------------------------------------------------------------------
// planning and launch helpers
// ---------------------------------------------------------------------------
// Work decomposition of one GEMV launch.
//  * R = 4 row tiles per wave: four 1 KiB weight loads per stage keep ~8 KiB
//    in flight per wave with the two-stage pipeline, and one activation
//    fragment load feeds four tiles. Narrow matrices fall back to 2 or 1.
//  * K is split across the W waves of a group (LDS reduction) and, when the
//    rows alone cannot fill the chip with ~12 waves per CU, across groups
//    (partials summed in split order by the last group to arrive).
//  * Every wave keeps at least 2 quads.
GemvLaunchPlan plan_gemv(const DevCtx *ctx, int nprob, int n_bt, int nrt, int nq, bool dual, int max_rows) {
    (void)max_rows;
    GemvLaunchPlan p;
    const long cus = ctx && ctx->cu_count ? ctx->cu_count : 256;
    const long target_waves = 12 * cus;
    p.R = 4;
    int RT = dual ? 2 : 4;
    if (!dual && nrt < 4) {
        p.R = nrt >= 2 ? 2 : 1;
        RT = p.R;
    }
    p.rbpp = (nrt + RT - 1) / RT;
    long groups = (long)nprob * n_bt * p.rbpp;
    // Many groups (the MoE layers of 16-21 rows: one per expert and row
    // block): two waves each, whose longer share of K pipelines better
    // (21-row verification 564 -> 552 us MXFP4, 709 -> 663 us int4 against
    // four waves; DSV3 B16 unchanged at 445); few: four, or eight to split a
    // long K.
    p.W = 4;
    if (groups * 4 < target_waves && nq >= 16) p.W = 8;
    if (groups >= target_waves) p.W = 2;
    // K splits cost a partial round trip and a serial tail: only worth it
    // when the row tiles alone leave the chip under 4 waves per CU (long-K,
    // narrow-O shapes such as a dense down projection).
    p.splits = 1;
    if (groups * p.W < 4 * cus) {
        long want = (8 * cus + groups * p.W - 1) / (groups * p.W);
        long cap = std::max(1, nq / (2 * p.W));
        p.splits = (int)std::min(want, cap);
    }
    // COLI_HIP_PLAN="R,W,splits" overrides the decomposition (tuning only).
    if (const char *ov = std::getenv("COLI_HIP_PLAN")) {
        int r = 0, w = 0, sp = 0;
        if (std::sscanf(ov, "%d,%d,%d", &r, &w, &sp) == 3 && (r == 1 || r == 2 || r == 4) &&
            (w == 2 || w == 4 || w == 8 || w == 16) && sp >= 1 && !(dual && r == 1) && !(r == 4 && w == 16)) {
            p.R = r;
            RT = dual ? r / 2 : r;
            p.rbpp = (nrt + RT - 1) / RT;
            p.W = w;
            p.splits = sp;
        }
    }
    // COLI_HIP_PLAN_PLAIN="R,W": the same for plain matrices on device
    // descriptors only (tuning the MoE down projections apart from gate/up).
    if (const char *ov = std::getenv("COLI_HIP_PLAN_PLAIN"); ov && !dual && nprob > 1) {
        int r = 0, w = 0;
        if (std::sscanf(ov, "%d,%d", &r, &w) == 2 && (r == 1 || r == 2 || r == 4) && (w == 2 || w == 4 || w == 8)) {
            p.R = r;
            p.W = w;
            p.rbpp = (nrt + r - 1) / r;
            p.splits = 1;
        }
    }
    p.qps = (nq + p.splits - 1) / p.splits;
    p.splits = (nq + p.qps - 1) / p.qps;
    p.dma = 0;
    p.PD = 0;
    return p;
}

// LDS bytes of one ring slot of coli_gemv_dma (mirrors DmaGeom in gemv_dma.hip).
static int dma_slot_bytes(int kind, int R, int max_rows) {
    const int sb = kind == COLI_KIND_I4_F ? 256 : (kind == COLI_KIND_FP4 ? 64 : 128);
    const int per = 256 / sb;
    const int scale_inst = (R + per - 1) / per;
    const int nxr = max_rows <= 1 ? 1 : (max_rows <= 4 ? 4 : (max_rows <= 8 ? 8 : 16));
    return R * COLI_TILE_BYTES + scale_inst * 256 + 2 * nxr * 256;
}

// Decomposition of the LDS-ring GEMV (gemv_dma.hip): one group of 8 waves per
// row block over the full K (no split). R row tiles per wave: one while the
// row tiles alone give about one group per CU (long-K, narrow-O shapes), two
// beyond that, four when there are many more and the batch tile is full; the
// ring is 3 stages deep for one tile, 2 for more. Returns false when the GEMV
// should stay on coli_gemv_tiles: rows too few to put one group on every CU
// (its K split fills the chip instead), or no decomposition fits the LDS.
static bool plan_dma(const DevCtx *ctx, GemvLaunchPlan &p, int kind, int nprob, int n_bt, int nrt, int nq, bool dual,
                     int max_rows) {
    const long cus = ctx && ctx->cu_count ? ctx->cu_count : 256;
    const long tiles = (long)nprob * n_bt * nrt;   // (gate, up) pairs for dual
    int force = 0;   // COLI_HIP_GEMV=dma|tiles pins the kernel (tuning and tests)
    if (const char *f = std::getenv("COLI_HIP_GEMV"))
        force = std::strcmp(f, "dma") == 0 ? 1 : (std::strcmp(f, "tiles") == 0 ? -1 : 0);
    if (force < 0 || max_rows > 16 || nq < 1) return false;
    // above four rows the staged activation block outweighs the tiles it feeds
    if (force == 0 && max_rows > 4) return false;
    // many problems of two to four rows (MoE unions): each problem's K is
    // short against the eight waves of a group; the register-ring kernel's
    // two-wave groups win (DSV3 MXFP4 layer B2 114.8 -> 100.8 us, B4 191.4 ->
    // 162.5 us; int4 B4 215.3 -> 189.1 us)
    if (force == 0 && nprob > 1 && max_rows > 1) return false;
    if (force == 0 && tiles < cus) return false;
    int RT = 1;
    if (tiles >= 2 * cus) RT = 2;
    if (!dual && tiles >= 2 * cus && max_rows > 8) RT = 4;
    // dual (gate + up): one row-tile pair per wave (measured: DSV3 B1 layer
    // 77.2 -> 71.5 us, OLMoE 32.4 -> 31.5 us against two pairs)
    if (dual) RT = 1;
    int W = 8;
    // tuning overrides: row tiles per wave, waves per group (dual only)
    if (const char *e = std::getenv("COLI_HIP_DMA_RT")) RT = std::max(1, std::min(dual ? 2 : 4, std::atoi(e)));
    if (const char *e = std::getenv("COLI_HIP_DMA_W"))
        if (dual && max_rows <= 1) W = std::atoi(e) == 4 ? 4 : 8;
    for (; RT >= 1; RT /= 2) {
        const int R = dual ? 2 * RT : RT;
        for (int PD = (R == 1 ? 3 : 2); PD >= 2; PD--) {
            if ((long)W * PD * dma_slot_bytes(kind, R, max_rows) <= 160 * 1024) {
                p.R = R;
                p.W = W;
                p.PD = PD;
                p.dma = 1;
                p.rbpp = (nrt + RT - 1) / RT;
                p.splits = 1;
                p.qps = nq;
                return true;
            }
        }
    }
    return false;
}

static int ngp_of(int K) { return (K + 127) / 128 * 4; }

// Fragments of rows x[0..nrows) (or src_rows[r]) of width K into set `set`.
static int record_frags(FragSet &f, const float *x, int ld, int nrows, int K, int int4_order, const int *src_rows,
                        const int *nrows_dev) {
    if (!x || nrows < 0 || K < 1 || ld < K) return 0;
    f.emitted = false;
    f.nolo = false;
    f.pending = true;
    f.px = x;
    f.pld = ld;
    f.pnrows = nrows;
    f.pK = K;
    f.pint4 = int4_order;
    f.psrc = src_rows;
    f.pnrows_dev = nrows_dev;
    return 1;
}

int make_frags(DevCtx *ctx, int set, const float *x, int ld, int nrows, int K, int int4_order,
               const int *src_rows, const int *nrows_dev) {
    return record_frags(ctx->frag[set], x, ld, nrows, K, int4_order, src_rows, nrows_dev);
}

// Build the pending fragments of f. ws == null: grow-only context buffers;
// else the caller's fixed buffers (capacity checked, nothing allocated).
// args_only: the build's launch arguments are returned instead of launched.
static int flush_frags_into(DevCtx *ctx, FragSet &f, int *flag, const void *zero, const GemvScratch *ws,
                            ColiPrepArgs *args_only = nullptr) {
    if (args_only) args_only->nblocks = 0;
    if (!f.pending) return 1;
    f.pending = false;
    const float *x = f.px;
    const int ld = f.pld, nrows = f.pnrows, K = f.pK, int4_order = f.pint4;
    const int *src_rows = f.psrc, *nrows_dev = f.pnrows_dev;
    int ngp = ngp_of(K);
    size_t halves = (size_t)nrows * ngp * 32;
    if (ws) {
        if (halves * 2 > f.hi.cap || halves * 2 > f.lo.cap || (size_t)nrows * sizeof(int) > f.exp.cap) return 0;
    } else if (!reserve(ctx, &f.hi, halves * 2, 0) || !reserve(ctx, &f.lo, halves * 2, 0) ||
               !reserve(ctx, &f.exp, (size_t)nrows * sizeof(int), 0)) {
        return 0;
    }
    f.gen = f.gen == 0x7fffffff ? 1 : f.gen + 1;
    if (f.gen == 1 && !hip_check(coli_launch_zero_i32(flag, 1, ctx->stream), "fragment flag")) return 0;
    return hip_check(coli_launch_prep_frag(x, ld, src_rows, nrows_dev, nrows, K, ngp, int4_order,
                                        (_Float16 *)f.hi.p, (_Float16 *)f.lo.p, (int *)f.exp.p, flag, f.gen,
                                        zero, ctx->stream, args_only),
                  "fragment prep");
}

int flush_frags(DevCtx *ctx, int set) {
    return flush_frags_into(ctx, ctx->frag[set], (int *)ctx->flags.p + set, ctx->zeros.p, nullptr);
}

int flush_frags_args(DevCtx *ctx, int set, ColiPrepArgs *a) {
    return flush_frags_into(ctx, ctx->frag[set], (int *)ctx->flags.p + set, ctx->zeros.p, nullptr, a);
}

// Many-row MXFP4 problems run the exact fp16-MFMA grouped GEMM by default.
// COLI_HIP_MX=1 selects the block-scaled MFMA GEMM (gemm_mx.hip): faster,
// but the hardware sums each 128-column block of e4m3 x e2m1 products with
// about 2^-15 of the block's magnitude sum as error (measured), so results
// carry ~3e-5 relative error (median) instead of fp32 accuracy.
bool mx_gemm_enabled() {
    const char *e = std::getenv("COLI_HIP_MX");
    return e && e[0] == '1';
}

int make_frags8(DevCtx *ctx, int set, const float *x, int ld, int nrows, int K, const int *src_rows,
                const int *nrows_dev) {
    FragSet &f = ctx->frag[set];
    const int nq = (K + 127) / 128, np = coli_mx_pieces();
    if (!reserve(ctx, &f.p8, (size_t)np * nrows * nq * 128, 0) || !reserve(ctx, &f.s8, (size_t)np * nrows * nq * 4, 0))
        return 0;
    f.prow = nrows;
    int *flag = (int *)ctx->flags.p + 8 + set;
    f.gen8 = f.gen8 == 0x7fffffff ? 1 : f.gen8 + 1;
    if (f.gen8 == 1 && !hip_check(coli_launch_zero_i32(flag, 1, ctx->stream), "piece flag")) return 0;
    return hip_check(coli_launch_prep_fp8(x, ld, src_rows, nrows_dev, nrows, K, nq, nrows, (uint8_t *)f.p8.p,
                                       (uint8_t *)f.s8.p, flag, f.gen8, ctx->stream),
                  "fp8 activation pieces");
}

// COLI_HIP_XF32=0 keeps the fragment prep for every GEMV (the LDS-ring
// kernel then reads prepared fragments, as the tiled one always does).
static bool xf32_enabled() {
    const char *e = std::getenv("COLI_HIP_XF32");
    return !(e && e[0] == '0');
}

// COLI_HIP_XSTAGE=0: one-row f32 GEMVs convert per stage and wave instead.
static bool xstage_enabled() {
    const char *e = std::getenv("COLI_HIP_XSTAGE");
    return !(e && e[0] == '0');
}

// Launch one tiled GEMV over `nprob` problems whose descriptors are on the device.
int run_gemv(DevCtx *ctx, int kind, bool dual, const ColiProb *probs_dev, int nprob, const int *nprob_dev, int nrt,
             int nq, int O, int max_rows, int set, const int *xrows_dev, float *out, int ldo,
             const ColiProb *inline_prob, float swiglu_limit, const GemvScratch *ws, GemvEmit *emit, bool fold) {
    if (emit) emit->done = false;
    if (nprob <= 0) return 1;
    int n_bt = (max_rows + 15) / 16;
    const GemvLaunchPlan tiles_plan = plan_gemv(ctx, nprob, n_bt, nrt, nq, dual, max_rows);
    GemvLaunchPlan pl = tiles_plan;
    plan_dma(ctx, pl, kind, nprob, n_bt, nrt, nq, dual, max_rows);
    // emitted fragments on the LDS-ring kernel: their exponents are staged
    // beside the ring, which must still fit
    if (pl.dma && !ws && ctx->frag[set].emitted &&
        (long)pl.W * pl.PD * dma_slot_bytes(kind, pl.R, max_rows) +
                ((long)nq * 4 * ((std::min(16, max_rows) + 3) / 4) + 63) / 64 * 256 >
            160 * 1024)
        pl = tiles_plan;
    size_t inst = (size_t)nprob * n_bt * pl.rbpp;
    const size_t part_bytes = inst * pl.splits * pl.R * 4 * 64 * sizeof(float);
    if (pl.splits > 1) {
        if (ws) {
            if (part_bytes > ws->partial_bytes || inst > ws->split_cnt_n) {
                std::fprintf(stderr, "[HIP] gemv: split-K scratch of %zu B / %zu counters exceeds the fixed buffer\n",
                             part_bytes, inst);
                return 0;
            }
        } else if (!reserve(ctx, &ctx->partial, part_bytes, 0) ||
                   !reserve(ctx, &ctx->split_cnt, inst * sizeof(int), 1)) {
            return 0;
        }
    }
    FragSet &f = ws ? *ws->frag : ctx->frag[set];
    int *flag = ws ? ws->flag : (int *)ctx->flags.p + set;
    const void *zero = ws ? ws->zero : ctx->zeros.p;
    ColiGemvArgs a;
    std::memset(&a, 0, sizeof(a));
    // Up to 32768 activations (rows x K) on the LDS-ring kernel are read as
    // f32 and converted in the kernel, which saves the prep launch; beyond,
    // every workgroup staging the f32 rows costs more than the prep (the
    // activations are re-read by every workgroup, at twice the bytes of the
    // hi fragments).
    if (pl.dma && max_rows <= 4 && (long)max_rows * nq * 128 <= 32768 && f.px && !f.psrc && f.pK == nq * 128 &&
        f.pld % 4 == 0 && (uintptr_t)f.px % 16 == 0 && xf32_enabled()) {
        a.xf = f.px;
        a.ldx = f.pld;
        // one row tile over a long K: sixteen waves, twice the per-quad
        // conversion chains in flight per CU
        if (pl.R == 1 && !dual && nq >= 64 && 16L * pl.PD * dma_slot_bytes(kind, 1, max_rows) <= 160 * 1024)
            pl.W = 16;
        // one row of one matrix: convert it once per group into LDS when the
        // ring leaves room (for the MoE's many small problems the per-stage
        // conversion measured faster)
        if (max_rows <= 1 && inline_prob && xstage_enabled() &&
            (long)pl.W * pl.PD * dma_slot_bytes(kind, pl.R, max_rows) + (long)nq * 516 <= 160 * 1024)
            a.xstage = 1;
    } else if (!flush_frags_into(ctx, f, flag, zero, ws)) {
        return 0;
    }
    // ring depth override (tuning; deeper rings measured slower: fewer
    // workgroups fit a CU): the deeper of 2, 3 that fits
    if (const char *e = std::getenv("COLI_HIP_DMA_PD"); e && pl.dma) {
        const int want = std::atoi(e);
        for (int PD : {3, 2})
            if (PD <= want && (long)pl.W * PD * dma_slot_bytes(kind, pl.R, max_rows) <= 160 * 1024) {
                pl.PD = PD;
                break;
            }
    }
    a.prob = probs_dev;
    if (inline_prob) {
        a.prob = nullptr;
        a.prob0 = *inline_prob;
    }
    a.nprob_dev = nprob_dev;
    a.nprob = nprob;
    a.nrt = nrt;
    a.nq = nq;
    a.O = O;
    a.n_bt = n_bt;
    a.rb_per_prob = pl.rbpp;
    a.splits = pl.splits;
    a.qps = pl.qps;
    a.xrows = xrows_dev;
    a.xhi = (const _Float16 *)f.hi.p;
    a.xlo = (const _Float16 *)f.lo.p;
    a.xstride = nq * 4 * 32;
    a.xexp = (const int *)f.exp.p;
    a.haslo = flag;
    a.lo_gen = f.gen;
    if (f.nolo) {   // a zero word never reaches generation 1
        a.haslo = (const int *)zero;
        a.lo_gen = 1;
    }
    a.zero = (const _Float16 *)zero;
    a.out = out;
    a.ldo = ldo;
    a.swiglu_limit = swiglu_limit;
    a.fold = fold && kind == COLI_KIND_FP4;
    a.partial = ws ? ws->partial : (float *)ctx->partial.p;
    a.split_cnt = ws ? ws->split_cnt : (int *)ctx->split_cnt.p;
    if (f.emitted && !ws) {
        // fragments emitted by the producing GEMV: per-group exponents, lo
        // parts always taken (a lo_gen of 0 passes every flag)
        a.gexp = (const uint8_t *)f.gexp.p;
        a.gexp_rows = f.erows_pad;
        a.lo_gen = 0;
    }
    if (emit && !ws && inline_prob && !dual && pl.splits == 1 && pl.R % 2 == 0 && O % 128 == 0 && max_rows <= 16) {
        FragSet &e = ctx->frag[emit->set];
        const int rows_pad = (max_rows + 15) / 16 * 16;
        const size_t halves = (size_t)max_rows * O;
        if (!reserve(ctx, &e.hi, halves * 2, 0) || !reserve(ctx, &e.lo, halves * 2, 0) ||
            !reserve(ctx, &e.gexp, (size_t)(O / 128) * rows_pad * 4, 0))
            return 0;
        e.pending = false;
        e.px = nullptr;
        e.psrc = nullptr;
        e.emitted = false;   // set by the caller once the launch is queued
        e.erows = max_rows;
        e.erows_pad = rows_pad;
        e.eK = O;
        e.esrc = out;
        a.ehi = (_Float16 *)e.hi.p;
        a.elo = (_Float16 *)e.lo.p;
        a.eexp = (uint8_t *)e.gexp.p;
        a.estride = O;
        a.erows = rows_pad;
        a.eint4 = emit->int4_order;
        emit->done = true;
    }
    if (pl.dma) return hip_check(coli_launch_gemv_dma(kind, &a, pl.R, dual ? 1 : 0, pl.W, pl.PD, max_rows, ctx->stream),
                              "gemv launch");
    return hip_check(coli_launch_gemv(kind, &a, pl.R, dual ? 1 : 0, pl.W, max_rows, ctx->stream), "gemv launch");
}

// Grouped GEMM over problems of many rows (see gemm.hip); mt_list_dev holds
// n_mt entries (problem << 16 | 64-row tile), problem indices relative to
// probs_dev.
int run_gemm(DevCtx *ctx, int kind, bool dual, const ColiProb *probs_dev, int nprob, const int *nprob_dev,
             const int *mt_list_dev, const int *n_mt_dev, int n_mt, int nrt, int nq, int O, int set,
             const int *xrows_dev, float *out, int ldo, float swiglu_limit, bool fold) {
    if (n_mt <= 0) return 1;
    FragSet &f = ctx->frag[set];
    if (!(kind == COLI_KIND_FP4 && mx_gemm_enabled()) && !flush_frags(ctx, set)) return 0;
    if (kind == COLI_KIND_FP4 && mx_gemm_enabled()) {
        ColiGemmMxArgs m;
        std::memset(&m, 0, sizeof(m));
        m.prob = probs_dev;
        m.nprob_dev = nprob_dev;
        m.nprob = nprob;
        m.mt_list = mt_list_dev;
        m.n_mt_dev = n_mt_dev;
        m.n_mt = n_mt;
        m.nrt = nrt;
        m.nq = nq;
        m.O = O;
        m.rb_per_prob = (nrt + COLI_GM_WAVES * (dual ? 1 : 2) - 1) / (COLI_GM_WAVES * (dual ? 1 : 2));
        m.xrows = xrows_dev;
        m.p8 = (const uint8_t *)f.p8.p;
        m.s8 = (const uint32_t *)f.s8.p;
        m.prow = f.prow;
        m.more = (const int *)ctx->flags.p + 8 + set;
        m.more_gen = f.gen8;
        m.zero = (const uint8_t *)ctx->zeros.p;
        m.out = out;
        m.ldo = ldo;
        m.swiglu_limit = swiglu_limit;
        return hip_check(coli_launch_gemm_mx(dual ? 1 : 0, &m, ctx->stream), "gemm launch");
    }
    ColiGemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.prob = probs_dev;
    a.nprob_dev = nprob_dev;
    a.nprob = nprob;
    a.mt_list = mt_list_dev;
    a.n_mt_dev = n_mt_dev;
    a.n_mt = n_mt;
    a.nrt = nrt;
    a.nq = nq;
    a.O = O;
    const int tiles_per_block = COLI_GM_BLOCK_TILES / (dual ? 2 : 1);
    a.rb_per_prob = (nrt + tiles_per_block - 1) / tiles_per_block;
    a.xrows = xrows_dev;
    a.xhi = (const _Float16 *)f.hi.p;
    a.xlo = (const _Float16 *)f.lo.p;
    a.xstride = nq * 4 * 32;
    a.xexp = (const int *)f.exp.p;
    a.haslo = (const int *)ctx->flags.p + set;
    a.lo_gen = f.gen;
    a.zero = (const uint8_t *)ctx->zeros.p;
    a.out = out;
    a.ldo = ldo;
    a.swiglu_limit = swiglu_limit;
    a.fold = fold && kind == COLI_KIND_FP4;
    return hip_check(coli_launch_gemm(kind, dual ? 1 : 0, &a, ctx->stream), "gemm launch");
}

int frag_set_of(int kind, bool hidden) {
    return (hidden ? 2 : 0) + (kind == COLI_KIND_FP4 ? 1 : 0);
}

static int tensor_computable(const ColiCudaTensor *t) {
    if (!t) return 0;
    if (t->fmt == 4 && t->gs <= 0) return 0;   // c/backend_cuda.cu:1355-1359
    return t->fmt == 2 || t->fmt == 4 || t->fmt == 7;
}

// ---------------------------------------------------------------------------
// the expert runner
// ---------------------------------------------------------------------------
struct Member {
    ColiCudaTensor *g, *u, *d;
    int rows, off;
};

// x_dev: [total, D] rows in member order; result y_dev: [total, D].
// drained: the stream was synchronized since the last copy out of the
// pinned descriptor staging was queued (it is not waited for again).
static int run_expert_group(DevCtx *ctx, const Member *m, int count, int total, int D, int I, float *y_dev,
                            const float *x_dev, bool drained) {
    if (!reserve(ctx, &ctx->h, (size_t)total * I * sizeof(float), 0)) return 0;
    float *h = (float *)ctx->h.p;

    // classify members
    std::vector<int> dual_kind(count, -1);
    bool need_x[2] = {false, false}, need_h[2] = {false, false}, need_gu = false;
    int max_rows = 0;
    bool fold = true;   // every MXFP4 matrix of the call allows the folded scales
    for (int c = 0; c < count; c++) {
        const Member &mm = m[c];
        max_rows = std::max(max_rows, mm.rows);
        for (const ColiCudaTensor *t : {mm.g, mm.u, mm.d})
            if (t->kind == COLI_KIND_FP4 && !t->e8_fold) fold = false;
        bool tiled_g = mm.g->kind != COLI_KIND_GENERIC, tiled_u = mm.u->kind != COLI_KIND_GENERIC;
        if (tiled_g && tiled_u && mm.g->kind == mm.u->kind) dual_kind[c] = mm.g->kind;
        else need_gu = true;
        if (tiled_g) need_x[mm.g->kind == COLI_KIND_FP4] = true;
        if (tiled_u) need_x[mm.u->kind == COLI_KIND_FP4] = true;
        if (mm.d->kind != COLI_KIND_GENERIC) need_h[mm.d->kind == COLI_KIND_FP4] = true;
    }
    if (need_gu && (!reserve(ctx, &ctx->g, (size_t)total * I * sizeof(float), 0) ||
                    !reserve(ctx, &ctx->u, (size_t)total * I * sizeof(float), 0)))
        return 0;
    // many-row MXFP4 members run the block-scaled MFMA GEMM on e4m3 pieces
    const bool mx_gemm = max_rows > COLI_GEMM_MIN_ROWS && mx_gemm_enabled();
    for (int o = 0; o < 2; o++) {
        const int set = frag_set_of(o ? COLI_KIND_FP4 : 0, false);
        if (need_x[o] && !((o && mx_gemm) ? make_frags8(ctx, set, x_dev, D, total, D)
                                          : make_frags(ctx, set, x_dev, D, total, D, !o)))
            return 0;
    }

    // descriptors: [dual by kind][split gate/up][down by kind]
    std::vector<ColiProb> probs;
    struct Launch { int kind; bool dual; int first, n, set; float *out; int ldo, O, nrt, nq; };
    std::vector<Launch> launches;
    const ColiCudaTensor *t0g = m[0].g, *t0d = m[0].d;
    for (int kind = 0; kind < 3; kind++) {
        int first = (int)probs.size();
        for (int c = 0; c < count; c++)
            if (dual_kind[c] == kind)
                probs.push_back({m[c].g->w, m[c].g->sc, m[c].u->w, m[c].u->sc, m[c].rows, m[c].off, m[c].off, 0});
        if ((int)probs.size() > first)
            launches.push_back({kind, true, first, (int)probs.size() - first, frag_set_of(kind, false), h, I, I,
                                (I + 15) / 16, (D + 127) / 128});
    }
    int split_first = (int)probs.size();
    for (int c = 0; c < count; c++) {
        if (dual_kind[c] >= 0) continue;
        ColiCudaTensor *pair[2] = {m[c].g, m[c].u};
        float *dst[2] = {(float *)ctx->g.p, (float *)ctx->u.p};
        for (int w = 0; w < 2; w++) {
            if (pair[w]->kind == COLI_KIND_GENERIC) continue;
            probs.push_back({pair[w]->w, pair[w]->sc, nullptr, nullptr, m[c].rows, m[c].off, m[c].off, 0});
            launches.push_back({pair[w]->kind, false, (int)probs.size() - 1, 1, frag_set_of(pair[w]->kind, false),
                                dst[w], I, I, (I + 15) / 16, (D + 127) / 128});
        }
    }
    int down_first = (int)probs.size();
    for (int kind = 0; kind < 3; kind++) {
        int first = (int)probs.size();
        for (int c = 0; c < count; c++)
            if (m[c].d->kind == kind)
                probs.push_back({m[c].d->w, m[c].d->sc, nullptr, nullptr, m[c].rows, m[c].off, m[c].off, 0});
        if ((int)probs.size() > first)
            launches.push_back({kind, false, first, (int)probs.size() - first, frag_set_of(kind, true),
                                y_dev, D, D, (D + 15) / 16, (I + 127) / 128});
    }
    (void)t0g; (void)t0d; (void)split_first;
    // Members of many rows go through the grouped GEMM: one work list of
    // (problem, 64-row tile) per launch, uploaded after the descriptors.
    const bool use_gemm = max_rows > COLI_GEMM_MIN_ROWS;
    std::vector<int> mt;
    std::vector<int> mt_first(launches.size(), 0), mt_count(launches.size(), 0);
    if (use_gemm)
        for (size_t l = 0; l < launches.size(); l++) {
            mt_first[l] = (int)mt.size();
            for (int q = 0; q < launches[l].n; q++) {
                const int rows = probs[launches[l].first + q].nrows;
                for (int t = 0; t * COLI_GM_ROWS < rows; t++) mt.push_back(q << 16 | t);
            }
            mt_count[l] = (int)mt.size() - mt_first[l];
        }
    if (!probs.empty()) {
        size_t pb = probs.size() * sizeof(ColiProb), mb = mt.size() * sizeof(int);
        if (!reserve_pinned(ctx, &ctx->host_prob, pb + mb) ||
            !reserve(ctx, &ctx->prob, pb + mb, 0))
            return 0;
        // the pinned staging may still feed a queued copy of the previous call
        if (!drained && !hip_check(hipStreamSynchronize(ctx->stream), "descriptor staging")) return 0;
        std::memcpy(ctx->host_prob.h, probs.data(), pb);
        if (mb) std::memcpy((char *)ctx->host_prob.h + pb, mt.data(), mb);
        if (!hip_check(hipMemcpyAsync(ctx->prob.p, ctx->host_prob.h, pb + mb, hipMemcpyHostToDevice, ctx->stream),
                    "descriptor upload"))
            return 0;
    }
    const ColiProb *pdev = (const ColiProb *)ctx->prob.p;
    const int *mtdev = (const int *)((const char *)ctx->prob.p + probs.size() * sizeof(ColiProb));
    auto launch = [&](size_t l, bool dual) {
        const Launch &L = launches[l];
        if (use_gemm)
            return run_gemm(ctx, L.kind, dual, pdev + L.first, L.n, nullptr, mtdev + mt_first[l], nullptr,
                            mt_count[l], L.nrt, L.nq, L.O, L.set, nullptr, L.out, L.ldo, 0.0f, fold);
        return run_gemv(ctx, L.kind, dual, pdev + L.first, L.n, nullptr, L.nrt, L.nq, L.O, max_rows, L.set,
                        nullptr, L.out, L.ldo, nullptr, 0.0f, nullptr, nullptr, fold);
    };

    // gate/up: dual launches and split members
    for (size_t l = 0; l < launches.size(); l++) {
        if (launches[l].first >= down_first) break;
        if (!launch(l, launches[l].dual)) return 0;
    }
    for (int c = 0; c < count; c++) {
        if (dual_kind[c] >= 0) continue;
        ColiCudaTensor *pair[2] = {m[c].g, m[c].u};
        float *dst[2] = {(float *)ctx->g.p, (float *)ctx->u.p};
        for (int w = 0; w < 2; w++)
            if (pair[w]->kind == COLI_KIND_GENERIC &&
                !hip_check(coli_launch_generic_i4(pair[w], x_dev + (size_t)m[c].off * D, D,
                                               dst[w] + (size_t)m[c].off * I, I, m[c].rows, ctx->stream),
                        "generic gemv"))
                return 0;
        size_t o = (size_t)m[c].off * I, n = (size_t)m[c].rows * I;
        if (!hip_check(coli_launch_silu_mul_to(h + o, (float *)ctx->g.p + o, (float *)ctx->u.p + o, n, ctx->stream),
                    "silu"))
            return 0;
    }
    // down
    for (int o = 0; o < 2; o++) {
        const int set = frag_set_of(o ? COLI_KIND_FP4 : 0, true);
        if (need_h[o] &&
            !((o && mx_gemm) ? make_frags8(ctx, set, h, I, total, I) : make_frags(ctx, set, h, I, total, I, !o)))
            return 0;
    }
    for (size_t l = 0; l < launches.size(); l++) {
        if (launches[l].first < down_first) continue;
        if (!launch(l, false)) return 0;
    }
    for (int c = 0; c < count; c++)
        if (m[c].d->kind == COLI_KIND_GENERIC &&
            !hip_check(coli_launch_generic_i4(m[c].d, h + (size_t)m[c].off * I, I, y_dev + (size_t)m[c].off * D, D,
                                           m[c].rows, ctx->stream),
                    "generic down"))
            return 0;
    return 1;
}

// Validate a group call's members; fills Member[] and returns the device context.
static DevCtx *collect_members(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups,
                               ColiCudaTensor *const *downs, const int *rows, int count,
                               std::vector<Member> &mem, int *total, int *D, int *I) {
    if (!gates || !ups || !downs || !rows || count < 1 || count > 64 || !gates[0]) return nullptr;
    int device = gates[0]->device;
    *D = gates[0]->I;
    *I = gates[0]->O;
    *total = 0;
    mem.resize(count);
    for (int c = 0; c < count; c++) {
        ColiCudaTensor *g = gates[c], *u = ups[c], *d = downs[c];
        if (!g || !u || !d || rows[c] < 1 || g->device != device || u->device != device || d->device != device ||
            g->I != *D || u->I != *D || g->O != *I || u->O != *I || d->I != *I || d->O != *D)
            return nullptr;
        if (!tensor_computable(g) || !tensor_computable(u) || !tensor_computable(d)) return nullptr;
        mem[c] = {g, u, d, rows[c], *total};
        *total += rows[c];
    }
    DevCtx *ctx = ctx_of(device);
    return bind_ctx(ctx) ? ctx : nullptr;
}

static double now_ms() {
    using clk = std::chrono::steady_clock;
    return std::chrono::duration<double, std::milli>(clk::now().time_since_epoch()).count();
}

// Stage host x -> device, run, device y -> pinned host_y (not yet synchronized).
static int group_stage_and_run(DevCtx *ctx, std::vector<Member> &mem, int count, int total, int D, int I,
                               const float *x, hipEvent_t *ev) {
    size_t xb = (size_t)total * D * sizeof(float);
    if (!reserve(ctx, &ctx->x, xb, 0) || !reserve(ctx, &ctx->y, xb, 0) ||
        !reserve_pinned(ctx, &ctx->host_x, xb) ||
        !reserve_pinned(ctx, &ctx->host_y, xb))
        return 0;
    if (!hip_check(hipStreamSynchronize(ctx->stream), "group staging")) return 0;
    std::memcpy(ctx->host_x.h, x, xb);
    if (ev) (void)hipEventRecord(ev[0], ctx->stream);
    // Decode-sized groups cross PCIe in copy kernels that read / write the
    // pinned buffers through their device addresses (measured: the sync group
    // call at decode 47 -> 39 us against DMA-engine copies). Above 1 MiB each
    // way (prefill-sized groups) the DMA engines' hipMemcpyAsync is used, as
    // always with COLI_HIP_KCOPY=0.
    const char *kc = std::getenv("COLI_HIP_KCOPY");
    const bool kcopy = !(kc && kc[0] == '0') && xb <= ((size_t)1 << 20);
    void *hx_dev = ctx->host_x.d, *hy_dev = ctx->host_y.d;
    if (kcopy ? !hip_check(coli_launch_copy_f32((float *)ctx->x.p, (const float *)hx_dev, xb / 4, ctx->stream),
                        "group input upload")
              : !hip_check(hipMemcpyAsync(ctx->x.p, ctx->host_x.h, xb, hipMemcpyHostToDevice, ctx->stream),
                        "group input upload"))
        return 0;
    if (ev) (void)hipEventRecord(ev[1], ctx->stream);
    // the stream was drained above; what it holds since reads host_x only
    if (!run_expert_group(ctx, mem.data(), count, total, D, I, (float *)ctx->y.p, (const float *)ctx->x.p, true))
        return 0;
    if (ev) (void)hipEventRecord(ev[2], ctx->stream);
    if (kcopy ? !hip_check(coli_launch_copy_f32((float *)hy_dev, (const float *)ctx->y.p, xb / 4, ctx->stream),
                        "group output download")
              : !hip_check(hipMemcpyAsync(ctx->host_y.h, ctx->y.p, xb, hipMemcpyDeviceToHost, ctx->stream),
                        "group output download"))
        return 0;
    if (ev) (void)hipEventRecord(ev[3], ctx->stream);
    return 1;
}

extern "C" int coli_cuda_expert_group(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups,
                                      ColiCudaTensor *const *downs, const int *rows, int count, float *y,
                                      const float *x) {
    if (fault_injected()) return 0;
    if (!x || !y) return 0;
    std::vector<Member> mem;
    int total, D, I;
    DevCtx *ctx = collect_members(gates, ups, downs, rows, count, mem, &total, &D, &I);
    if (!ctx || ctx->group_pending) return 0;
    int profile = std::getenv("COLI_CUDA_PROFILE") && std::atoi(std::getenv("COLI_CUDA_PROFILE"));
    hipEvent_t ev[4] = {};
    if (profile)
        for (int i = 0; i < 4; i++)
            if (!hip_check(hipEventCreate(&ev[i]), "profile event")) {
                for (int j = 0; j < i; j++) (void)hipEventDestroy(ev[j]);
                profile = 0;
                break;
            }
    int ok = group_stage_and_run(ctx, mem, count, total, D, I, x, profile ? ev : nullptr) &&
             hip_check(hipStreamSynchronize(ctx->stream), "expert group synchronize");
    double a = 0, b = 0, c = 0;
    if (profile) {
        float fa = 0, fb = 0, fc = 0;
        if (ok) {
            (void)hipEventElapsedTime(&fa, ev[0], ev[1]);
            (void)hipEventElapsedTime(&fb, ev[1], ev[2]);
            (void)hipEventElapsedTime(&fc, ev[2], ev[3]);
        }
        a = fa; b = fb; c = fc;
        for (int i = 0; i < 4; i++) (void)hipEventDestroy(ev[i]);
    }
    if (!ok) return 0;
    std::memcpy(y, ctx->host_y.h, (size_t)total * D * sizeof(float));
    note_group(ctx, count, total, a, b, c);
    return 1;
}

extern "C" int coli_cuda_expert_group_issue(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups,
                                            ColiCudaTensor *const *downs, const int *rows, int count,
                                            const float *x) {
    if (fault_injected()) return 0;
    if (!x) return 0;
    std::vector<Member> mem;
    int total, D, I;
    DevCtx *ctx = collect_members(gates, ups, downs, rows, count, mem, &total, &D, &I);
    // decode-scale only, as c/backend_cuda.cu:1716: larger packs take the sync call
    if (!ctx || ctx->group_pending || total > 8) return 0;
    if (!group_stage_and_run(ctx, mem, count, total, D, I, x, nullptr)) return 0;
    ctx->group_pending = 1;
    note_group(ctx, count, total, 0, 0, 0);
    return 1;
}

extern "C" const float *coli_cuda_expert_group_take(int device) {
    DevCtx *ctx = ctx_of(device);
    if (!ctx || !ctx->group_pending) return nullptr;
    ctx->group_pending = 0;
    if (!bind_ctx(ctx)) return nullptr;
    if (!hip_check(hipStreamSynchronize(ctx->stream), "expert group take")) return nullptr;
    return (const float *)ctx->host_y.h;
}

extern "C" int coli_cuda_expert_mlp(ColiCudaTensor *gate, ColiCudaTensor *up, ColiCudaTensor *down, float *y,
                                    const float *x, int S) {
    if (fault_injected()) return 0;
    if (!gate || !up || !down || !x || !y || S < 1) return 0;
    ColiCudaTensor *g[1] = {gate}, *u[1] = {up}, *d[1] = {down};
    int rows[1] = {S};
    std::vector<Member> mem;
    int total, D, I;
    DevCtx *ctx = collect_members(g, u, d, rows, 1, mem, &total, &D, &I);
    if (!ctx || ctx->group_pending) return 0;
    if (!group_stage_and_run(ctx, mem, 1, total, D, I, x, nullptr) ||
        !hip_check(hipStreamSynchronize(ctx->stream), "expert mlp synchronize"))
        return 0;
    std::memcpy(y, ctx->host_y.h, (size_t)total * D * sizeof(float));
    return 1;
}

// The prefill shared expert of c/backend_cuda.cu:1457-1484: the same contract
// as expert_mlp, restricted as there to per-row int4 (fmt=2) tensors; any
// other format is refused (return 0) so the engine keeps its CPU path.
extern "C" int coli_cuda_shared_mlp_w4a16(ColiCudaTensor *gate, ColiCudaTensor *up, ColiCudaTensor *down,
                                          float *y, const float *x, int S) {
    if (!gate || !up || !down || gate->fmt != 2 || up->fmt != 2 || down->fmt != 2) return 0;
    return coli_cuda_expert_mlp(gate, up, down, y, x, S);
}

// ---------------------------------------------------------------------------
// single-matrix GEMV / GEMM
// ---------------------------------------------------------------------------
// Records x_dev's S rows as t's input (fragment set of t's kind). When the GEMV that wrote x_dev
// emitted them as fragments of t's order (coli_hip_gemm_run_dev_emit), the
// next gemm_run reads those instead and no prep runs.
static int gemm_prep(DevCtx *ctx, ColiCudaTensor *t, const float *x_dev, int S) {
    const int order = t->kind == COLI_KIND_FP4 ? 1 : 0;
    const int hidden = frag_set_of(t->kind, true);
    const FragSet &h = ctx->frag[hidden];
    if (h.emitted && h.esrc == x_dev && h.erows == S && h.eK == t->I) {
        ctx->dense_set[order] = hidden;
        return 1;
    }
    ctx->dense_set[order] = frag_set_of(t->kind, false);
    return make_frags(ctx, frag_set_of(t->kind, false), x_dev, t->I, S, t->I, t->kind != COLI_KIND_FP4);
}

// Fragments emitted from a device buffer describe what it held when they
// were written: every entry point that writes device memory calls this for
// the bytes it writes, and an emitted set overlapping them is dropped (its
// next prep builds fragments from the buffer again). bytes == SIZE_MAX: the
// extent is not known on the host, every emitted set of the device goes.
void forget_emitted(DevCtx *ctx, const void *dst, size_t bytes) {
    const uintptr_t a = (uintptr_t)dst;
    const uintptr_t b = bytes == SIZE_MAX ? UINTPTR_MAX : a + bytes;
    for (int s = 2; s < 4; s++) {
        FragSet &f = ctx->frag[s];
        if (!f.emitted) continue;
        const uintptr_t ea = (uintptr_t)f.esrc, eb = ea + (size_t)f.erows * f.eK * sizeof(float);
        if (bytes == SIZE_MAX || (a < eb && ea < b)) f.emitted = false;
    }
}

// GEMV of t over the prepared fragments of S rows -> y_dev[S, O]; the
// problem travels in the kernel arguments (no descriptor, no host sync).
// With next: y_dev is also emitted as next's input fragments (set 2 / 3).
static int gemm_run(DevCtx *ctx, ColiCudaTensor *t, float *y_dev, int S, const ColiCudaTensor *next = nullptr) {
    const ColiProb p = {t->w, t->sc, nullptr, nullptr, S, 0, 0, 0};
    const int set = ctx->dense_set[t->kind == COLI_KIND_FP4 ? 1 : 0];
    const bool fold = t->kind == COLI_KIND_FP4 && t->e8_fold;
    forget_emitted(ctx, y_dev, (size_t)S * t->O * sizeof(float));
    if (!next) {
        return run_gemv(ctx, t->kind, false, nullptr, 1, nullptr, t->nrt, t->nq, t->O, S, set, nullptr, y_dev, t->O,
                        &p, 0.0f, nullptr, nullptr, fold);
    }
    GemvEmit em = {frag_set_of(next->kind, true), next->kind != COLI_KIND_FP4, false};
    // the set this launch reads (itself emitted) cannot be written by it: run
    // without emitting, next's prep builds its fragments as usual
    if (em.set == set)
        return run_gemv(ctx, t->kind, false, nullptr, 1, nullptr, t->nrt, t->nq, t->O, S, set, nullptr, y_dev, t->O,
                        &p, 0.0f, nullptr, nullptr, fold);
    if (!run_gemv(ctx, t->kind, false, nullptr, 1, nullptr, t->nrt, t->nq, t->O, S, set, nullptr, y_dev, t->O, &p,
                  0.0f, nullptr, &em, fold))
        return 0;
    ctx->frag[em.set].emitted = em.done;
    ctx->frag[em.set].nolo = false;
    return em.done ? 2 : 1;
}

// y_dev[S, O] = x_dev[S, I] W^T on the stream (tensor already resident).
static int gemm_dev(DevCtx *ctx, ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    if (t->kind == COLI_KIND_GENERIC) {
        forget_emitted(ctx, y_dev, (size_t)S * t->O * sizeof(float));
        return hip_check(coli_launch_generic_i4(t, x_dev, t->I, y_dev, t->O, S, ctx->stream), "generic gemv");
    }
    return gemm_prep(ctx, t, x_dev, S) && gemm_run(ctx, t, y_dev, S);
}

extern "C" int coli_hip_gemm_prep_dev(ColiCudaTensor *t, const float *x_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || !x_dev || S < 1 || t->kind == COLI_KIND_GENERIC || !tensor_computable(t)) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return gemm_prep(ctx, t, x_dev, S);
}

extern "C" int coli_hip_gemm_run_dev(ColiCudaTensor *t, float *y_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || !y_dev || S < 1 || t->kind == COLI_KIND_GENERIC || !tensor_computable(t)) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return gemm_run(ctx, t, y_dev, S);
}

// As coli_hip_gemm_run_dev, and the output rows are also written as the
// activation fragments of `next` (next->I == t->O), which a following
// coli_hip_gemm_prep_dev(next, y_dev, S) then uses without a prep launch.
// Emitted only where it pays and the launch allows (2..16 rows whose f32
// form the consumer would not convert itself, t->O a multiple of 128, a
// plain launch with an even number of row tiles per wave and no K split);
// otherwise the prep runs as usual. The caller must not modify y_dev before
// that prep's GEMV has run. Returns 2 when the fragments were emitted, 1 when
// only the GEMV ran, 0 on failure.
extern "C" int coli_hip_gemm_run_dev_emit(ColiCudaTensor *t, float *y_dev, int S, const ColiCudaTensor *next) {
    if (fault_injected()) return 0;
    if (!t || !y_dev || S < 1 || t->kind == COLI_KIND_GENERIC || !tensor_computable(t)) return 0;
    if (!next || next->kind == COLI_KIND_GENERIC || next->I != t->O || next->device != t->device) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    // the consumer converts up to 32768 f32 activations of 1..4 rows itself;
    // one long row it reads faster as emitted fragments (dense down at B1,
    // K = 14336: 10.7 -> 10.1 us, the up launch 0.2 us slower for emitting).
    // COLI_HIP_EMIT=0 never emits, =force emits wherever the launch allows
    // (tests and measurements).
    const char *e = std::getenv("COLI_HIP_EMIT");
    bool worth = S <= 16 && ((S > 1 && (long)S * next->I > 32768) || (S == 1 && next->I >= 8192));
    if (e && e[0] == '0') worth = false;
    if (e && std::strcmp(e, "force") == 0) worth = S <= 16;
    return gemm_run(ctx, t, y_dev, S, worth ? next : nullptr);
}

// fmt=2 with int8 activations (c/colibri.c:937-945, matmul_i4_idot): the
// rows quantized by qrow_i8 into exact fp16 fragments, the integer dot on the
// tiled GEMV over unit group scales (every partial sum an exact integer), then
// y = (dot * scale[o]) * sx[s]. Results are bitwise the reference's.
#define COLI_IDOT_MAX_I 16512   // 8 * 127 * I < 2^24: every f32 partial sum is exact
static int idot_dev(DevCtx *ctx, ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    if (t->fmt != 2 || (t->kind != COLI_KIND_I4_H && t->kind != COLI_KIND_I4_F) || t->I > COLI_IDOT_MAX_I)
        return 0;
    const int half = t->kind == COLI_KIND_I4_H;
    if (!t->sc_unit) {
        void *p = nullptr;
        if (!hip_check(hipMalloc(&p, t->sc_bytes), "unit scales") ||
            !hip_check(coli_launch_unit_scales(p, t->sc_bytes / (half ? 2 : 4), half, ctx->stream), "unit scales")) {
            if (p) (void)hipFree(p);
            return 0;
        }
        t->sc_unit = p;
    }
    const int set = frag_set_of(t->kind, false), ngp = ngp_of(t->I);
    FragSet &f = ctx->frag[set];
    const size_t halves = (size_t)S * ngp * 32;
    if (!reserve(ctx, &f.hi, halves * 2, 0) || !reserve(ctx, &f.lo, halves * 2, 0) ||
        !reserve(ctx, &f.exp, (size_t)S * sizeof(int), 0) || !reserve(ctx, &ctx->idot_y, (size_t)S * t->O * 4, 0) ||
        !reserve(ctx, &ctx->idot_sx, (size_t)S * 4, 0))
        return 0;
    // hi parts only: the GEMVs over this set never read its lo buffer
    f.pending = false;
    f.nolo = true;
    f.emitted = false;
    f.px = nullptr;
    f.psrc = nullptr;
    f.gen = f.gen == 0x7fffffff ? 1 : f.gen + 1;
    if (f.gen == 1 && !hip_check(coli_launch_zero_i32((int *)ctx->flags.p + set, 1, ctx->stream), "fragment flag"))
        return 0;
    if (!hip_check(coli_launch_qrow_i8_frag(x_dev, t->I, S, t->I, ngp, 1, (_Float16 *)f.hi.p, (int *)f.exp.p,
                                            (float *)ctx->idot_sx.p, ctx->stream),
                   "int8 activation rows"))
        return 0;
    const ColiProb p = {t->w, t->sc_unit, nullptr, nullptr, S, 0, 0, 0};
    if (!run_gemv(ctx, t->kind, false, nullptr, 1, nullptr, t->nrt, t->nq, t->O, S, set, nullptr,
                  (float *)ctx->idot_y.p, t->O, &p))
        return 0;
    forget_emitted(ctx, y_dev, (size_t)S * t->O * sizeof(float));
    return hip_check(coli_launch_idot_scale(y_dev, (const float *)ctx->idot_y.p, (const float *)ctx->idot_sx.p, t->sc,
                                            half, t->nq, t->O, S, ctx->stream),
                     "int8 activation scales");
}

static int gemm_host(DevCtx *ctx, ColiCudaTensor *t, float *y, const float *x, int S, int qdq) {
    size_t xb = (size_t)S * t->I * sizeof(float), yb = (size_t)S * t->O * sizeof(float);
    if (!reserve(ctx, &ctx->x, xb, 0) || !reserve(ctx, &ctx->y, yb, 0) ||
        !reserve_pinned(ctx, &ctx->host_x, xb) ||
        !reserve_pinned(ctx, &ctx->host_y, yb) ||
        !hip_check(hipStreamSynchronize(ctx->stream), "gemm staging"))
        return 0;
    std::memcpy(ctx->host_x.h, x, xb);
    if (!hip_check(hipMemcpyAsync(ctx->x.p, ctx->host_x.h, xb, hipMemcpyHostToDevice, ctx->stream), "input upload"))
        return 0;
    const float *xin = (const float *)ctx->x.p;
    // qdq 1: e4m3 per 128 (native_quant contract); 2: int8 per 32 (matmul_mxfp4_i8)
    if (qdq == 1 || (qdq == 2 && t->I % 32 == 0)) {
        if (!reserve(ctx, &ctx->qdq, xb, 0) ||
            !hip_check(qdq == 1 ? coli_launch_qdq_e4m3(xin, (float *)ctx->qdq.p, S, t->I, ctx->stream)
                             : coli_launch_qdq_i8(xin, (float *)ctx->qdq.p, S, t->I, ctx->stream),
                    "activation qdq"))
            return 0;
        xin = (const float *)ctx->qdq.p;
    }
    if (!(qdq == 3 ? idot_dev(ctx, t, (float *)ctx->y.p, xin, S) : gemm_dev(ctx, t, (float *)ctx->y.p, xin, S)) ||
        !hip_check(hipMemcpyAsync(ctx->host_y.h, ctx->y.p, yb, hipMemcpyDeviceToHost, ctx->stream), "output download") ||
        !hip_check(hipStreamSynchronize(ctx->stream), "gemm synchronize"))
        return 0;
    std::memcpy(y, ctx->host_y.h, yb);
    return 1;
}

extern "C" int coli_hip_matmul_i4_idot(ColiCudaTensor *t, float *y, const float *x, int S) {
    if (fault_injected()) return 0;
    if (!t || !y || !x || S < 1 || t->fmt != 2) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return gemm_host(ctx, t, y, x, S, 3);
}

extern "C" int coli_hip_matmul_i4_idot_dev(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || !y_dev || !x_dev || S < 1 || t->fmt != 2) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return idot_dev(ctx, t, y_dev, x_dev, S);
}

extern "C" int coli_cuda_matmul(ColiCudaTensor **tensor, float *y, const float *x, const void *weights,
                                const float *scales, int fmt, int S, int I, int O, int device, int gs) {
    if (fault_injected()) return 0;
    if (fmt == 4 && gs <= 0) return 0;
    if (S < 1 || !y || !x || !tensor) return 0;
    if (!upload_impl(tensor, weights, scales, nullptr, fmt, I, O, device, gs > 0 ? gs : (fmt == 7 ? 32 : 0), 0))
        return 0;
    ColiCudaTensor *t = *tensor;
    if (!tensor_computable(t)) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return gemm_host(ctx, t, y, x, S, 0);
}

static int matmul_mxfp4_stateless(float *y, const float *x, const unsigned char *q4, const unsigned char *e8s, int S,
                                  int I, int O, int qdq) {
    if (S < 1 || I < 1 || O < 1 || !y || !x || !q4 || !e8s) return 0;
    DevCtx *ctx = ctx_of(0);
    if (!bind_ctx(ctx)) return 0;
    // Stateless (c/backend_cuda.cu:1377-1416): the weights go up with the call,
    // into reusable scratch instead of a fresh allocation.
    ColiCudaTensor t;
    std::memset(&t, 0, sizeof(t));
    t.fmt = 7; t.I = I; t.O = O; t.device = ctx->device; t.gs = 32; t.kind = COLI_KIND_FP4;
    t.Op = (O + 15) / 16 * 16; t.Ip = (I + 127) / 128 * 128; t.nrt = t.Op / 16; t.nq = t.Ip / 128;
    t.w_bytes = (size_t)t.nrt * t.nq * COLI_TILE_BYTES;
    t.sc_bytes = (size_t)t.nrt * t.nq * 64;
    size_t wsrc = (size_t)(I + 1) / 2 * O, ssrc = (size_t)O * ((I + 31) / 32);
    if (!reserve(ctx, &ctx->tmp_tiles, t.w_bytes, 0) || !reserve(ctx, &ctx->tmp_scales, t.sc_bytes, 0) ||
        !reserve(ctx, &ctx->stage_w, wsrc, 0) || !reserve(ctx, &ctx->stage_s, ssrc, 0) ||
        !hip_check(hipStreamSynchronize(ctx->stream), "mxfp4 staging"))
        return 0;
    t.w = (uint8_t *)ctx->tmp_tiles.p;
    t.sc = ctx->tmp_scales.p;
    if (!hip_check(hipMemcpyAsync(ctx->stage_w.p, q4, wsrc, hipMemcpyHostToDevice, ctx->stream), "mxfp4 weight upload") ||
        !hip_check(hipMemcpyAsync(ctx->stage_s.p, e8s, ssrc, hipMemcpyHostToDevice, ctx->stream), "mxfp4 scale upload") ||
        !hip_check(coli_launch_repack(&t, (const uint8_t *)ctx->stage_w.p, ctx->stage_s.p, ctx->stream), "mxfp4 repack"))
        return 0;
    return gemm_host(ctx, &t, y, x, S, qdq);
}

extern "C" int coli_cuda_matmul_mxfp4(float *y, const float *x, const unsigned char *q4, const unsigned char *e8s,
                                      int S, int I, int O) {
    if (fault_injected()) return 0;
    return matmul_mxfp4_stateless(y, x, q4, e8s, S, I, O, 0);
}

// matmul_mxfp4_i8 (c/quant.h:1441-1515): the same stateless call with the
// activations quantized to int8 per 32 columns first (I % 32 != 0: the float
// path, as the reference falls back).
extern "C" int coli_hip_matmul_mxfp4_i8(float *y, const float *x, const unsigned char *q4, const unsigned char *e8s,
                                        int S, int I, int O) {
    if (fault_injected()) return 0;
    return matmul_mxfp4_stateless(y, x, q4, e8s, S, I, O, 2);
}

// Resident-tensor variants of matmul_mxfp4_i8 (host and device buffers).
extern "C" int coli_hip_fp4_matmul_i8(ColiCudaTensor *t, float *y, const float *x, int S) {
    if (fault_injected()) return 0;
    if (!t || t->kind != COLI_KIND_FP4 || !y || !x || S < 1) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return gemm_host(ctx, t, y, x, S, 2);
}

extern "C" int coli_hip_fp4_matmul_i8_dev(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || t->kind != COLI_KIND_FP4 || !y_dev || !x_dev || S < 1) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    if (t->I % 32) return gemm_dev(ctx, t, y_dev, x_dev, S);
    size_t xb = (size_t)S * t->I * sizeof(float);
    if (!reserve(ctx, &ctx->qdq, xb, 0) ||
        !hip_check(coli_launch_qdq_i8(x_dev, (float *)ctx->qdq.p, S, t->I, ctx->stream), "activation qdq"))
        return 0;
    return gemm_dev(ctx, t, y_dev, (const float *)ctx->qdq.p, S);
}

extern "C" int coli_hip_fp4_matmul_qdq(ColiCudaTensor *t, float *y, const float *x, int S) {
    if (fault_injected()) return 0;
    if (!t || t->kind != COLI_KIND_FP4 || !y || !x || S < 1 || t->I % 128) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return gemm_host(ctx, t, y, x, S, 1);
}

extern "C" int coli_hip_fp4_matmul_qdq_dev(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || t->kind != COLI_KIND_FP4 || !y_dev || !x_dev || S < 1 || t->I % 128) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    size_t xb = (size_t)S * t->I * sizeof(float);
    if (!reserve(ctx, &ctx->qdq, xb, 0) ||
        !hip_check(coli_launch_qdq_e4m3(x_dev, (float *)ctx->qdq.p, S, t->I, ctx->stream), "activation qdq"))
        return 0;
    return gemm_dev(ctx, t, y_dev, (const float *)ctx->qdq.p, S);
}

extern "C" int coli_cuda_pipe_gemm(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || S < 1 || !y_dev || !x_dev || !tensor_computable(t)) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    return gemm_dev(ctx, t, y_dev, x_dev, S);
}

// coli_cuda_pipe_gemm without any allocation: every buffer the launch needs
// beyond x and y (activation fragments, their lo flag, the zero block,
// split-K partials and arrival counters) lives in the library's static
// scratch array, whose per-device address the init call looked up. The
// decomposition is pipe_gemm's, so the results are bitwise equal.
extern "C" int coli_hip_pipe_gemm_noalloc(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S) {
    if (fault_injected()) return 0;
    if (!t || S < 1 || !y_dev || !x_dev || !tensor_computable(t)) return 0;
    if (S > COLI_NA_MAX_ROWS || t->I > COLI_NA_MAX_K) {
        std::fprintf(stderr, "[HIP] pipe_gemm_noalloc: %d rows x I = %d exceed the fixed scratch (rows <= %d, I <= %d)\n",
                     S, t->I, COLI_NA_MAX_ROWS, COLI_NA_MAX_K);
        return 0;
    }
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx) || !ctx->scratch) return 0;
    forget_emitted(ctx, y_dev, (size_t)S * t->O * sizeof(float));
    if (t->kind == COLI_KIND_GENERIC)
        return hip_check(coli_launch_generic_i4(t, x_dev, t->I, y_dev, t->O, S, ctx->stream), "generic gemv");
    uint8_t *sc = ctx->scratch;
    FragSet &f = ctx->na_frag;
    f.hi.p = sc + COLI_NA_OFF_HI;
    f.hi.cap = COLI_NA_FRAG_BYTES;
    f.lo.p = sc + COLI_NA_OFF_LO;
    f.lo.cap = COLI_NA_FRAG_BYTES;
    f.exp.p = sc + COLI_NA_OFF_EXP;
    f.exp.cap = COLI_NA_EXP_BYTES;
    if (!record_frags(f, x_dev, t->I, S, t->I, t->kind != COLI_KIND_FP4, nullptr, nullptr)) return 0;
    const GemvScratch ws = {&f,
                            (int *)(sc + COLI_NA_OFF_FLAG),
                            sc + COLI_NA_OFF_ZERO,
                            (float *)(sc + COLI_NA_OFF_PART),
                            COLI_NA_PART_BYTES,
                            (int *)(sc + COLI_NA_OFF_CNT),
                            COLI_NA_CNT_BYTES / sizeof(int)};
    const ColiProb p = {t->w, t->sc, nullptr, nullptr, S, 0, 0, 0};
    return run_gemv(ctx, t->kind, false, nullptr, 1, nullptr, t->nrt, t->nq, t->O, S, frag_set_of(t->kind, false),
                    nullptr, y_dev, t->O, &p, 0.0f, &ws, nullptr, t->kind == COLI_KIND_FP4 && t->e8_fold);
}

// ---------------------------------------------------------------------------
// resident expert group (c/backend_cuda.cu:2246-2316)
// ---------------------------------------------------------------------------
extern "C" int coli_cuda_expert_group_resident_issue(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups,
                                                     ColiCudaTensor *const *downs, const float *weights,
                                                     int count, int home_device, const float *x_src_dev,
                                                     float *partial_slot_dev) {
    if (fault_injected()) return 0;
    if (!weights || count < 1 || count > 64 || !x_src_dev || !partial_slot_dev) return 0;
    std::vector<int> rows(count, 1);
    std::vector<Member> mem;
    int total, D, I;
    DevCtx *ctx = collect_members(gates, ups, downs, rows.data(), count, mem, &total, &D, &I);
    if (!ctx) return 0;
    if (!ctx->ev_ok) {
        if (!hip_check(hipEventCreateWithFlags(&ctx->ev_done, hipEventDisableTiming), "resident group event")) return 0;
        ctx->ev_ok = 1;
    }
    // Fixed 64-expert capacity: a growth here could free a buffer queued work reads.
    size_t xb = (size_t)64 * D * sizeof(float);
    if (!reserve(ctx, &ctx->x, xb, 0) || !reserve(ctx, &ctx->y, xb, 0) ||
        !reserve(ctx, &ctx->rw, 64 * sizeof(float), 0) || !reserve(ctx, &ctx->rslot, (size_t)D * sizeof(float), 0) ||
        !reserve_pinned(ctx, &ctx->host_small, 64 * sizeof(float)))
        return 0;
    if (!hip_check(hipStreamSynchronize(ctx->stream), "resident staging")) return 0;
    std::memcpy(ctx->host_small.h, weights, (size_t)count * sizeof(float));
    if (!hip_check(hipMemcpyAsync(ctx->rw.p, ctx->host_small.h, (size_t)count * sizeof(float), hipMemcpyHostToDevice,
                               ctx->stream),
                "resident weights"))
        return 0;
    // every member reads the same input row: replicate it (count rows)
    float *xr = (float *)ctx->x.p;
    for (int c = 0; c < count; c++) {
        hipError_t e = home_device == ctx->device
                           ? hipMemcpyAsync(xr + (size_t)c * D, x_src_dev, (size_t)D * sizeof(float),
                                            hipMemcpyDeviceToDevice, ctx->stream)
                           : hipMemcpyPeerAsync(xr + (size_t)c * D, ctx->device, x_src_dev, home_device,
                                                (size_t)D * sizeof(float), ctx->stream);
        if (!hip_check(e, "resident input")) return 0;
    }
    if (!run_expert_group(ctx, mem.data(), count, total, D, I, (float *)ctx->y.p, xr, false)) return 0;
    if (DevCtx *home = ctx_of(home_device)) forget_emitted(home, partial_slot_dev, (size_t)D * sizeof(float));
    float *local = home_device == ctx->device ? partial_slot_dev : (float *)ctx->rslot.p;
    if (!hip_check(coli_launch_weighted_sum_rows(local, (const float *)ctx->y.p, (const float *)ctx->rw.p, count, D,
                                              ctx->stream),
                "resident reduce"))
        return 0;
    if (home_device != ctx->device &&
        !hip_check(hipMemcpyPeerAsync(partial_slot_dev, home_device, local, ctx->device, (size_t)D * sizeof(float),
                                   ctx->stream),
                "resident partial push"))
        return 0;
    return hip_check(hipEventRecord(ctx->ev_done, ctx->stream), "resident event record");
}

extern "C" int coli_cuda_expert_group_resident_take(int home_device, const int *devices, int n_issued,
                                                    float *slots_dev, float *acc_dev, int D) {
    if (n_issued < 1 || !slots_dev || !acc_dev || D < 1 || !devices) return 0;
    DevCtx *home = ctx_of(home_device);
    if (!bind_ctx(home)) return 0;
    for (int i = 0; i < n_issued; i++) {
        DevCtx *src = ctx_of(devices[i]);
        if (!src || !src->ev_ok) return 0;
        if (!hip_check(hipStreamWaitEvent(home->stream, src->ev_done, 0), "resident take wait")) return 0;
    }
    forget_emitted(home, acc_dev, (size_t)D * sizeof(float));
    return hip_check(coli_launch_sum_slots(acc_dev, slots_dev, n_issued, D, home->stream), "resident take reduce");
}

// ---------------------------------------------------------------------------
// Router logits as per-chunk partials (one partial per 512-column chunk of
// D, summed in chunk order by the selection). Up to 64 rows: the GEMV-shaped
// partial kernel coli_router_partial (pipe.hip, passes of 16 rows). Beyond:
// coli_router_gemm (pipe.hip), 64 x 64 output tiles per 512-column chunk on
// the f32 MFMA, writing the same chunk partials. No vendor library is used.
// ---------------------------------------------------------------------------
int router_logits(DevCtx *ctx, const float *x, int S, const float *W, int D, int E, float *part) {
    // up to 64 rows: the GEMV-shaped partial kernel (passes of 16 rows);
    // beyond: the MFMA f32 GEMM (pipe.hip). Both leave the same chunk partials.
    const hipError_t err = S <= 64 ? coli_launch_router_logits(x, S, W, D, E, part, ctx->stream)
                                   : coli_launch_router_gemm(x, S, W, D, E, part, ctx->stream);
    return hip_check(err, "router logits") ? coli_router_chunks(D) : 0;
}

// ---------------------------------------------------------------------------
// device router (c/backend_cuda.cu:2139-2215)
// ---------------------------------------------------------------------------
extern "C" int coli_cuda_pipe_router(int device, const float *x_dev, const void *rw_dev, const void *rb_dev, int D,
                                     int E, int Ksel, float topp, int norm_topk, float routed_scale, int *idx_host,
                                     float *w_host, int *keff_host) {
    if (fault_injected()) return 0;
    DevCtx *ctx = ctx_of(device);
    if (!x_dev || !rw_dev || !rb_dev || D < 1 || E < 1 || E > 1024 || Ksel < 1 || Ksel > 64 || !idx_host ||
        !w_host || !keff_host || !bind_ctx(ctx))
        return 0;
    const int nch = coli_router_chunks(D);
    size_t pack = (size_t)nch * E * sizeof(float) + (size_t)Ksel * 8 + 16;
    if (!reserve(ctx, &ctx->pipe[22], pack, 0) ||
        !reserve_pinned(ctx, &ctx->host_small, (size_t)Ksel * 8 + 16))
        return 0;
    float *logit = (float *)ctx->pipe[22].p;
    int *idx = (int *)(logit + (size_t)nch * E);
    float *w = (float *)(idx + Ksel);
    int *keff = (int *)(w + Ksel);
    if (!hip_check(coli_launch_router_logits(x_dev, 1, (const float *)rw_dev, D, E, logit, ctx->stream), "router logits") ||
        !hip_check(coli_launch_router_select(logit, nch, (const float *)rb_dev, 1, E, Ksel, 1, topp, norm_topk, routed_scale,
                                          idx, w, keff, ctx->stream),
                "router select") ||
        !hip_check(hipMemcpyAsync(ctx->host_small.h, idx, (size_t)Ksel * 8 + sizeof(int), hipMemcpyDeviceToHost,
                               ctx->stream),
                "router readback") ||
        !hip_check(hipStreamSynchronize(ctx->stream), "router sync"))
        return 0;
    const char *hb = (const char *)ctx->host_small.h;
    std::memcpy(idx_host, hb, (size_t)Ksel * sizeof(int));
    std::memcpy(w_host, hb + (size_t)Ksel * sizeof(int), (size_t)Ksel * sizeof(float));
    std::memcpy(keff_host, hb + (size_t)Ksel * 8, sizeof(int));
    return 1;
}

// ---------------------------------------------------------------------------
// resident-pipeline primitives (c/backend_cuda.cu:2036-2135, 2317-2448)
// ---------------------------------------------------------------------------
extern "C" float *coli_cuda_pipe_scratch(int device, int slot, size_t bytes) {
    DevCtx *ctx = ctx_of(device);
    if (slot < 0 || slot >= COLI_PIPE_SLOTS || !bind_ctx(ctx)) return nullptr;
    if (!reserve(ctx, &ctx->pipe[slot], bytes, 0)) return nullptr;
    return (float *)ctx->pipe[slot].p;
}

extern "C" void *coli_cuda_pipe_alloc(int device, size_t bytes) {
    DevCtx *ctx = ctx_of(device);
    if (!bind_ctx(ctx)) return nullptr;
    void *p = nullptr;
    if (!hip_check(hipMalloc(&p, bytes), "pipe alloc")) return nullptr;
    return p;
}

extern "C" void coli_cuda_pipe_free(int device, void *p) {
    DevCtx *ctx = ctx_of(device);
    if (!p || !bind_ctx(ctx)) return;
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(p);
}

extern "C" int coli_cuda_pipe_upload(int device, void *dst, const void *src, size_t bytes) {
    DevCtx *ctx = ctx_of(device);
    if (!bind_ctx(ctx)) return 0;
    forget_emitted(ctx, dst, bytes);
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "pipe upload") &&
           hip_check(hipStreamSynchronize(ctx->stream), "pipe upload sync");
}

extern "C" int coli_cuda_pipe_download(int device, const void *src, void *dst, size_t bytes) {
    DevCtx *ctx = ctx_of(device);
    if (!bind_ctx(ctx)) return 0;
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "pipe download") &&
           hip_check(hipStreamSynchronize(ctx->stream), "pipe download sync");
}

extern "C" int coli_cuda_pipe_silu_mul(int device, float *gate_dev, const float *up_dev, size_t n) {
    if (fault_injected()) return 0;
    DevCtx *ctx = ctx_of(device);
    if (!n || !gate_dev || !up_dev || !bind_ctx(ctx)) return 0;
    forget_emitted(ctx, gate_dev, n * sizeof(float));
    return hip_check(coli_launch_silu_mul(gate_dev, up_dev, n, ctx->stream), "pipe silu mul");
}

extern "C" int coli_cuda_pipe_add(int device, float *x_dev, const float *t_dev, size_t n) {
    if (fault_injected()) return 0;
    DevCtx *ctx = ctx_of(device);
    if (!n || !x_dev || !t_dev || !bind_ctx(ctx)) return 0;
    forget_emitted(ctx, x_dev, n * sizeof(float));
    return hip_check(coli_launch_add_n(x_dev, t_dev, n, ctx->stream), "pipe add");
}

extern "C" int coli_cuda_pipe_rows_add(int device, float *x_dev, const float *partial_dev, const int *rows_dev,
                                       int nrows, int D) {
    if (fault_injected()) return 0;
    DevCtx *ctx = ctx_of(device);
    if (nrows < 1 || D < 1 || !x_dev || !partial_dev || !rows_dev || !bind_ctx(ctx)) return 0;
    forget_emitted(ctx, x_dev, SIZE_MAX);   // the rows written are known on the device only
    return hip_check(coli_launch_rows_add(x_dev, partial_dev, rows_dev, nrows, D, ctx->stream), "pipe rows add");
}

extern "C" int coli_cuda_pipe_copy2d(int device, float *dst, int dpitch, const float *src, int spitch, int width,
                                     int height) {
    DevCtx *ctx = ctx_of(device);
    if (!bind_ctx(ctx)) return 0;
    if (height > 0) forget_emitted(ctx, dst, ((size_t)(height - 1) * dpitch + width) * sizeof(float));
    return hip_check(hipMemcpy2DAsync(dst, (size_t)dpitch * 4, src, (size_t)spitch * 4, (size_t)width * 4, height,
                                   hipMemcpyDeviceToDevice, ctx->stream),
                  "pipe copy2d") &&
           hip_check(hipStreamSynchronize(ctx->stream), "pipe copy2d sync");
}

extern "C" int coli_cuda_pipe_peer_copy(int dst_dev, float *dst, int src_dev, const float *src, size_t bytes) {
    if (!dst || !src) return 0;
    if (DevCtx *d = ctx_of(dst_dev)) forget_emitted(d, dst, bytes);
    if (dst_dev == src_dev) {
        DevCtx *c = ctx_of(dst_dev);
        if (!bind_ctx(c)) return 0;
        return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream), "pipe intra copy") &&
               hip_check(hipStreamSynchronize(c->stream), "pipe intra copy sync");
    }
    return hip_check(hipMemcpyPeer(dst, dst_dev, src, src_dev, bytes), "pipe peer copy");
}

extern "C" int coli_cuda_pipe_sync(int device) {
    DevCtx *ctx = ctx_of(device);
    if (!bind_ctx(ctx)) return 0;
    return hip_check(hipStreamSynchronize(ctx->stream), "pipe sync") && hip_check(hipDeviceSynchronize(), "pipe sync");
}

// ---------------------------------------------------------------------------
// Outside this backend's scope (attention-side layers): refused with 0, the
// reference's "compute on the CPU" answer, so the engine keeps its own path.
// ---------------------------------------------------------------------------
extern "C" int coli_cuda_pipe_rmsnorm(int, float *, const float *, const float *, int, int, float) { return 0; }
extern "C" int coli_cuda_pipe_rmsnorm_s(int, float *, const float *, const float *, int, int, float, int, int) {
    return 0;
}
extern "C" int coli_cuda_pipe_rope(int, float *, const int *, int, int, int, int, int, float) { return 0; }
extern "C" int coli_cuda_pipe_rope_base(int, float *, int, int, int, int, int, int, float) { return 0; }
extern "C" int coli_cuda_attention_absorb(ColiCudaTensor *, float *, const float *, const float *, const float *,
                                          int, int, int, int, int, int, float) {
    return 0;
}
extern "C" int coli_cuda_attention_absorb_batch(ColiCudaTensor *, float *, const float *, const float *,
                                                const float *, int, int, int, int, int, int, int, float) {
    return 0;
}
extern "C" int coli_cuda_attention_project_batch(ColiCudaTensor *, ColiCudaTensor *, float *, const float *,
                                                 const float *, const float *, int, int, int, int, int, int, int,
                                                 float) {
    return 0;
}
extern "C" int coli_cuda_attention_project_ragged(ColiCudaTensor *, ColiCudaTensor *, float *, const float *,
                                                  const void *const *, const float *const *, const float *const *,
                                                  const int *, int, int, int, int, int, int, int, float) {
    return 0;
}
extern "C" int coli_cuda_attention_project_batch_dev(ColiCudaTensor *, ColiCudaTensor *, float *, const float *,
                                                     const float *, const float *, int, int, int, int, int, int, int,
                                                     float) {
    return 0;
}
extern "C" int coli_cuda_attention_absorb_batch_dev(ColiCudaTensor *, float *, const float *, const float *,
                                                    const float *, int, int, int, int, int, int, int, float) {
    return 0;
}
extern "C" int coli_cuda_attention_absorb_kvdev(ColiCudaTensor *, float *, const float *, const float *,
                                                const float *, int, int, int, int, int, int, float) {
    return 0;
}
extern "C" int coli_cuda_attention_project_batch_dev_out(ColiCudaTensor *, ColiCudaTensor *, float *,
                                                         const float *, const float *, const float *, int, int, int,
                                                         int, int, int, int, float) {
    return 0;
}
