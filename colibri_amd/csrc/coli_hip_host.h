// coli_hip_host.h -- host-side state of the gfx950 backend (not part of the ABI).
#pragma once

#include "coli_hip_internal.h"

#include <stdint.h>

#define COLI_PIPE_SLOTS 27
// Batches larger than this run the grouped GEMM instead of the GEMV.
#define COLI_GEMM_MIN_ROWS 32

// The static scratch array behind coli_hip_pipe_gemm_noalloc (one copy per
// device, held until the process ends): regions and the limits they imply.
#define COLI_NA_MAX_ROWS 16
#define COLI_NA_MAX_K 16384
#define COLI_NA_FRAG_BYTES ((size_t)COLI_NA_MAX_ROWS * (COLI_NA_MAX_K / 128) * 4 * 32 * 2)   // 512 KiB
#define COLI_NA_EXP_BYTES ((size_t)4096)
#define COLI_NA_CNT_BYTES ((size_t)64 << 10)
#define COLI_NA_OFF_ZERO ((size_t)0)                                           // COLI_ZERO_BYTES of zeros
#define COLI_NA_OFF_HI (COLI_NA_OFF_ZERO + COLI_ZERO_BYTES)
#define COLI_NA_OFF_LO (COLI_NA_OFF_HI + COLI_NA_FRAG_BYTES)
#define COLI_NA_OFF_EXP (COLI_NA_OFF_LO + COLI_NA_FRAG_BYTES)
#define COLI_NA_OFF_FLAG (COLI_NA_OFF_EXP + COLI_NA_EXP_BYTES)                 // the lo flag (256 B slot)
#define COLI_NA_OFF_CNT (COLI_NA_OFF_FLAG + 256)
#define COLI_NA_OFF_PART (COLI_NA_OFF_CNT + COLI_NA_CNT_BYTES)
#define COLI_NA_BYTES ((size_t)8 << 20)
#define COLI_NA_PART_BYTES (COLI_NA_BYTES - COLI_NA_OFF_PART)

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

// Pinned host staging: the host address and the device address kernels use
// to read or write it across PCIe, both set when the buffer is (re)allocated.
struct PinBuf {
    void *h = nullptr;
    void *d = nullptr;
    size_t cap = 0;
};

// Activation fragments of one kind of input (see coli_prep_frag in gemv.hip).
struct FragSet {
    DevBuf hi, lo, exp;
    int gen = 0;      // generation of the last prep (see coli_prep_frag)
    DevBuf p8, s8;    // e4m3 pieces + e8m0 scales for the MXFP4 GEMM (coli_prep_fp8)
    int prow = 0;     // rows per piece plane
    int gen8 = 0;     // generation of the last piece prep (flag slot 8 + set)
    // The set holds hi parts only and its lo buffer is stale (the fmt=2 int8
    // rows of idot_dev): GEMVs over it read a flag that is always zero, so
    // they never take lo parts, also when a captured launch is replayed
    // after a later prep raised the set's own flag.
    bool nolo = false;
    // The rows the set was last asked for (make_frags): the prep is deferred
    // until a kernel needs fragments (flush_frags); a GEMV that converts f32
    // activations itself reads px directly and never needs it.
    bool pending = false;
    const float *px = nullptr;
    int pld = 0, pnrows = 0, pK = 0, pint4 = 0;
    const int *psrc = nullptr, *pnrows_dev = nullptr;
    // Fragments emitted by a GEMV's epilogue (coli_hip_gemm_run_dev_emit):
    // rows [0, erows) of the output esrc, K = eK, one exponent per (row,
    // group) in gexp ([quad][erows_pad][4] signed bytes). Any other use of
    // the set clears `emitted`.
    DevBuf gexp;
    bool emitted = false;
    const float *esrc = nullptr;
    int erows = 0, erows_pad = 0, eK = 0;
};

struct DevCtx {
    int device = -1;
    int cu_count = 0;
    hipStream_t stream = nullptr;
    size_t tensor_count = 0, tensor_bytes = 0;
    // grow-only scratch
    DevBuf x, h, y, g, u, partial, prob, zeros, stage_w, stage_s, qdq, flags;
    DevBuf rslot, rw, tmp_tiles, tmp_scales, split_cnt, idot_y, idot_sx;
    FragSet frag[4];                   // 0/1: inputs (int4 / fp4 order), 2/3: hidden rows
    int dense_set[2] = {0, 1};         // set the next coli_hip_gemm_run_dev reads, per order (gemm_prep)
    DevBuf pipe[COLI_PIPE_SLOTS];
    // pinned staging
    PinBuf host_x, host_y, host_prob, host_small;
    // this device's copy of the library's static scratch array (see
    // coli_hip_pipe_gemm_noalloc), looked up at init; null if unavailable
    uint8_t *scratch = nullptr;
    FragSet na_frag;                   // views into scratch (no allocations)
    int group_pending = 0;
    hipEvent_t ev_done = nullptr;
    int ev_ok = 0;
    // statistics
    uint64_t st_calls = 0, st_experts = 0, st_rows = 0;
    double st_h2d = 0, st_kernel = 0, st_d2h = 0;
};

extern DevCtx g_ctx[];
extern int g_nctx;

int hip_check(hipError_t err, const char *what);
DevCtx *ctx_of(int device);
int bind_ctx(DevCtx *ctx);
int fault_injected(void);
int reserve(DevCtx *ctx, DevBuf *b, size_t bytes, int zero);
int reserve_pinned(DevCtx *ctx, PinBuf *b, size_t bytes);
void forget_emitted(DevCtx *ctx, const void *dst, size_t bytes);
void note_group(DevCtx *ctx, int count, int total, double h2d, double ker, double d2h);
int upload_impl(ColiCudaTensor **tensor, const void *weights, const float *scales, const uint8_t *e8,
                int fmt, int I, int O, int device, int gs, int w_on_device);

// kernels (gemv.hip / pipe.hip)
extern "C" {
hipError_t coli_launch_gemv(int kind, const ColiGemvArgs *a, int R, int dual, int W, int max_rows,
                            hipStream_t st);
hipError_t coli_launch_gemv_dma(int kind, const ColiGemvArgs *a, int R, int dual, int W, int PD, int max_rows,
                                hipStream_t st);
hipError_t coli_launch_prep_frag(const float *x, int ldx, const int *src_row, const int *nrows_dev,
                                 int nrows, int K, int ngp, int int4_order, _Float16 *hi, _Float16 *lo,
                                 int *exp2out, int *haslo, int gen, const void *zero, hipStream_t st,
                                 ColiPrepArgs *args_only = nullptr);
hipError_t coli_launch_gemm(int kind, int dual, const ColiGemmArgs *a, hipStream_t st);
hipError_t coli_launch_gemm_mx(int dual, const ColiGemmMxArgs *a, hipStream_t st);
hipError_t coli_launch_prep_fp8(const float *x, int ldx, const int *src_row, const int *nrows_dev, int nrows, int K,
                                int nq, int prow, uint8_t *p8, uint8_t *s8, int *more, int gen, hipStream_t st);
int coli_mx_pieces(void);
hipError_t coli_launch_repack(const ColiCudaTensor *t, const uint8_t *src_w, const void *src_s,
                              hipStream_t st);
hipError_t coli_launch_generic_i4(const ColiCudaTensor *t, const float *x, int ldx, float *y, int ldy,
                                  int S, hipStream_t st);
hipError_t coli_launch_qdq_e4m3(const float *x, float *y, int S, int K, hipStream_t st);
hipError_t coli_launch_qdq_i8(const float *x, float *y, int S, int K, hipStream_t st);
hipError_t coli_launch_qrow_i8_frag(const float *x, int ldx, int nrows, int K, int ngp, int int4_order,
                                    _Float16 *hi, int *exp2out, float *sx, hipStream_t st);
hipError_t coli_launch_rows16_to_rows(const uint8_t *packed, uint8_t *rows, int O, int nb, hipStream_t st);
hipError_t coli_launch_unit_scales(void *sc, size_t n, int half_scales, hipStream_t st);
hipError_t coli_launch_idot_scale(float *y, const float *yi, const float *sx, const void *sc, int half_scales,
                                  int nq, int O, int S, hipStream_t st);
int coli_router_chunks(int D);   // column chunks of the router partials
hipError_t coli_launch_router_logits(const float *x, int S, const float *W, int D, int E, float *part,
                                     hipStream_t st);
hipError_t coli_launch_router_gemm(const float *x, int S, const float *W, int D, int E, float *part, hipStream_t st);
hipError_t coli_launch_router_select(const float *part, int nch, const float *bias, int S, int E, int K, int mode,
                                     float topp, int norm_topk, float routed_scale, int *idx, float *w,
                                     int *keff, hipStream_t st);
hipError_t coli_launch_zero_i32(int *p, int n, hipStream_t st);
hipError_t coli_launch_fill_random(void *dev, size_t n, unsigned long long seed, hipStream_t st);
hipError_t coli_launch_stream_read(const void *dev, size_t bytes, hipStream_t st);
hipError_t coli_launch_silu_mul(float *gate, const float *up, size_t n, hipStream_t st);
hipError_t coli_launch_silu_mul_to(float *h, const float *gate, const float *up, size_t n, hipStream_t st);
hipError_t coli_launch_copy_f32(float *dst, const float *src, size_t n, hipStream_t st);
hipError_t coli_launch_add_n(float *x, const float *t, size_t n, hipStream_t st);
hipError_t coli_launch_rows_add(float *x, const float *partial, const int *rows, int nrows, int D,
                                hipStream_t st);
hipError_t coli_launch_weighted_sum_rows(float *out, const float *y, const float *w, int count, int D,
                                         hipStream_t st);
hipError_t coli_launch_sum_slots(float *dst, const float *slots, int n, int D, hipStream_t st);
}

// Expert path runner (expert.hip): one shared routine behind expert_group,
// issue, expert_mlp, resident_issue and the MoE layer.
struct GemvLaunchPlan {
    int R, W, rbpp, splits, qps;
    int dma, PD;   // LDS-ring kernel (gemv_dma.hip) and its ring depth
};
GemvLaunchPlan plan_gemv(const DevCtx *ctx, int nprob, int n_bt, int nrt, int nq, bool dual, int max_rows);

// Activation fragments of rows x[0..nrows) (or src_rows[r]; nrows_dev: live
// count on the device) of width K into fragment set `set` (0/1: inputs of the
// int4 / fp4 order, 2/3: hidden rows). Records the request; the prep runs
// when a kernel first needs the fragments (flush_frags). x must hold its
// values until then.
int make_frags(DevCtx *ctx, int set, const float *x, int ld, int nrows, int K, int int4_order,
               const int *src_rows = nullptr, const int *nrows_dev = nullptr);
int flush_frags(DevCtx *ctx, int set);
// the pending build of `set` made ready (buffers, generation) but returned as
// launch arguments for a launch that runs it beside other work (nblocks 0:
// nothing pending)
int flush_frags_args(DevCtx *ctx, int set, ColiPrepArgs *a);
int frag_set_of(int kind, bool hidden);
// Activation pieces of the MXFP4 grouped GEMM (e4m3 + e8m0 per 32 columns)
// of the same rows, into fragment set `set`.
bool mx_gemm_enabled();
int make_frags8(DevCtx *ctx, int set, const float *x, int ld, int nrows, int K, const int *src_rows = nullptr,
                const int *nrows_dev = nullptr);
// Fixed buffers a GEMV launch may use in place of the context's grow-only
// scratch (the allocation-free entry point): the fragment set (hi / lo / exp
// with their capacities), its lo flag, the zero block, and the split-K
// partials and arrival counters.
struct GemvScratch {
    FragSet *frag;
    int *flag;
    const void *zero;
    float *partial;
    size_t partial_bytes;
    int *split_cnt;
    size_t split_cnt_n;
};
// One tiled GEMV over `nprob` problems (descriptors on the device, or one
// inline problem) reading fragment set `set` (or ws's buffers, allocating
// nothing, when ws is given).
// Emission request of run_gemv: write the output also as fragment set
// `set` for a consumer of the given order (see ColiGemvArgs::ehi); `done`
// reports whether the launch could (plain inline matrix, R even, no K split).
struct GemvEmit {
    int set;
    int int4_order;
    bool done;
};
int run_gemv(DevCtx *ctx, int kind, bool dual, const ColiProb *probs_dev, int nprob, const int *nprob_dev, int nrt,
             int nq, int O, int max_rows, int set, const int *xrows_dev, float *out, int ldo,
             const ColiProb *inline_prob = nullptr, float swiglu_limit = 0.0f, const GemvScratch *ws = nullptr,
             GemvEmit *emit = nullptr, bool fold = false);
// One grouped GEMM over a device work list of (problem << 16 | 64-row tile).
int run_gemm(DevCtx *ctx, int kind, bool dual, const ColiProb *probs_dev, int nprob, const int *nprob_dev,
             const int *mt_list_dev, const int *n_mt_dev, int n_mt, int nrt, int nq, int O, int set,
             const int *xrows_dev, float *out, int ldo, float swiglu_limit = 0.0f, bool fold = false);

// Router logits of S rows into `part`; returns the number of column-chunk
// partials the selection must add, or 0 on failure.
int router_logits(DevCtx *ctx, const float *x, int S, const float *W, int D, int E, float *part);
