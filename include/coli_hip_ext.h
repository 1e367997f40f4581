/* coli_hip_ext.h -- entry points libcoli_hip.so adds beyond the reference ABI.
 *
 * None of these has a counterpart in c/backend_cuda.h; each states the
 * reference code whose behaviour it provides on the device.
 */
#ifndef COLI_HIP_EXT_H
#define COLI_HIP_EXT_H

#include "coli_backend_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Resident MXFP4 (fmt=7) tensor from its native bytes: q4 [O, ceil(I/2)]
 * e2m1 nibbles, e8 [O, ceil(I/32)] ue8m0 exponents (the layout of
 * c/quant.h:1375-1390). The CUDA backend has no resident fmt=7 group path
 * (c/backend_cuda.cu:1636-1643); this is new capability. */
int coli_hip_tensor_upload_mxfp4(ColiCudaTensor **tensor, const unsigned char *q4,
                                 const unsigned char *e8, int I, int O, int device);

/* Resident MXFP4 tensor from the 16-row interleaved layout of
 * coli_fp4_pack_rows16_v10 (c/deepseek_v4.c:10975-10993): O % 16 == 0,
 * I % 128 == 0. */
int coli_hip_tensor_upload_fp4_rows16(ColiCudaTensor **tensor, const unsigned char *packed_data,
                                      const unsigned char *packed_scales, int I, int O,
                                      int device);

/* Upload whose weight source is already in device memory (row-major source
 * layout, e.g. landed there by a GPU-side loader); scales come from the host:
 * f32 (fmt 2/4) or ue8m0 bytes (fmt 7, e8 != NULL). Same semantics otherwise
 * as coli_cuda_tensor_upload_g. */
int coli_hip_tensor_upload_from_device(ColiCudaTensor **tensor, const void *weights_dev,
                                       const float *scales, const unsigned char *e8, int fmt,
                                       int I, int O, int device, int gs);

/* native_quant contract on the device: every activation row is first
 * quantize-dequantized to e4m3 in blocks of 128 with an e8m0 scale
 * (c/deepseek_v4.c:10495-10520), then multiplied with the resident MXFP4
 * tensor (coli_fp4_matmul_batch_ref, c/deepseek_v4.c:10906-10933; batch 1 is
 * coli_fp4_matvec_ref, 10571-10605). Host pointers; returns 1 / 0. */
int coli_hip_fp4_matmul_qdq(ColiCudaTensor *tensor, float *y, const float *x, int S);

/* Same, device pointers, asynchronous on the backend stream. */
int coli_hip_fp4_matmul_qdq_dev(ColiCudaTensor *tensor, float *y_dev, const float *x_dev, int S);

/* MXFP4 with int8 activations: replaces matmul_mxfp4_i8 (c/quant.h:1441-1515,
 * the K3 IDOT path selected by K3_IDOT=1, c/kimi_k3.c). Each activation row
 * is quantized per 32 columns to int8 (sc = max|x| / 127, q = rint(x / sc)
 * clamped to +-127, bit-exact with the reference) and multiplied with the
 * MXFP4 weights; I % 32 != 0 falls back to the float path as the reference
 * does. Stateless like coli_cuda_matmul_mxfp4 (host q4 [O][I/2], e8
 * [O][I/32]). Returns 1 / 0 (y untouched on failure). */
int coli_hip_matmul_mxfp4_i8(float *y, const float *x, const unsigned char *q4,
                             const unsigned char *e8s, int S, int I, int O);

/* Same on a resident MXFP4 tensor: host pointers (synchronous) / device
 * pointers (asynchronous on the backend stream). */
int coli_hip_fp4_matmul_i8(ColiCudaTensor *tensor, float *y, const float *x, int S);
int coli_hip_fp4_matmul_i8_dev(ColiCudaTensor *tensor, float *y_dev, const float *x_dev, int S);

/* fmt=2 (int4, one f32 scale per row) with int8 activations: replaces the
 * reference's IDOT path for fmt=2 experts (c/colibri.c:937-945: qrow_i8
 * c/quant.h:581-586 per row, then matmul_i4_idot c/quant.h:924-933 with
 * dot_i4i8 674-801). Each row is quantized to int8 (s = max|x| / 127, at least
 * 1e-12; q = rint(x * (1 / s))), the integer dot is exact, and y[s, o] =
 * (float)dot * scale[o] * s: bitwise the reference's result. I <= 16512.
 * Resident fmt=2 tensor; host pointers (synchronous) / device pointers
 * (asynchronous on the backend stream). Returns 1 / 0 (y untouched on
 * failure). */
int coli_hip_matmul_i4_idot(ColiCudaTensor *tensor, float *y, const float *x, int S);
int coli_hip_matmul_i4_idot_dev(ColiCudaTensor *tensor, float *y_dev, const float *x_dev, int S);

/* ---- fused MoE layer (router -> union -> experts -> SwiGLU -> scatter) ---- */
typedef struct ColiHipMoe ColiHipMoe;

typedef struct {
    int D, I, E, K;        /* hidden, expert intermediate, routed experts, top-k */
    int route_mode;        /* 0 softmax then top-k (c/olmoe.c:666-681)
                              1 sigmoid, choice = sigmoid + bias (c/colibri.c:3978-4126)
                              2 sigmoid + bias select, weights renormalized over the
                                selection (c/kimi_k3.c:1337-1356)
                              3 DeepSeek-V4: sqrt(softplus) + bias select, weights
                                score / sum x routed_scale (c/deepseek_v4.c:1368-1432) */
    int norm_topk;
    float topp;            /* 0 disables */
    float routed_scale;    /* 1.0 for none */
    int has_shared;        /* one always-on expert, added after the routed sum */
    float swiglu_limit;    /* > 0: DeepSeek-V4 clamped SwiGLU (c/deepseek_v4.c:1434-1448) */
} ColiHipMoeConfig;

/* Router weights f32 [E, D] (+ bias [E] or NULL) are copied to the device;
 * expert tensors are resident handles of one device (gate/up [I, D], down
 * [D, I]). All experts must share one storage kind. */
int coli_hip_moe_create(ColiHipMoe **moe, int device, const ColiHipMoeConfig *cfg,
                        const float *router_w, const float *router_bias,
                        ColiCudaTensor *const *gates, ColiCudaTensor *const *ups,
                        ColiCudaTensor *const *downs, ColiCudaTensor *shared_gate,
                        ColiCudaTensor *shared_up, ColiCudaTensor *shared_down);
void coli_hip_moe_free(ColiHipMoe *moe);

/* Device-resident forward of S <= 2048 rows (decode, verification or
 * prefill; S * K <= 16384): x_dev [S, D] f32 -> out_dev [S, D] f32,
 * asynchronous on the backend stream (no host sync, no allocation after the
 * first call at a given S). Up to 32 rows the experts run the tiled GEMV,
 * beyond it the grouped GEMM. */
int coli_hip_moe_forward_dev(ColiHipMoe *moe, const float *x_dev, float *out_dev, int S);

/* Host forward with routing read back: idx/w [S, K], keff [S] (may be NULL). */
int coli_hip_moe_forward(ColiHipMoe *moe, const float *x, float *out, int S, int *idx,
                         float *w, int *keff);

/* Union of the last forward: nu and the unique expert ids in first-seen order
 * (c/colibri.c:4146-4152). Synchronizes. */
int coli_hip_moe_last_union(ColiHipMoe *moe, int *nu, int *uniq);

/* coli_cuda_pipe_gemm (device pointers, asynchronous on the backend stream)
 * that allocates nothing. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Every buffer beyond x and
 * y lives in one static 8 MiB device array per GPU, held until the process
 * ends. Limits: S <= 16 rows and I <= 16384 (larger calls return 0 with a
 * diagnostic); results are bitwise those of coli_cuda_pipe_gemm. All calls on
 * one GPU share that array: calls that overlap on one GPU (other host
 * threads, other streams) race. Returns 1 / 0. */
int coli_hip_pipe_gemm_noalloc(ColiCudaTensor *tensor, float *y_dev, const float *x_dev, int S);

/* ---- plumbing for benchmarks and tests ----------------------------------- */
/* coli_cuda_pipe_gemm in two halves, so a timer can bracket the GEMV kernel
 * alone: prep names the activations x_dev[S, I] for the tensor's storage
 * kind (no launch); run launches the GEMV y_dev[S, O]. The first run after a
 * prep also launches the fragment build when its kernel needs fragments (the
 * LDS-ring kernel of up to 32768 activations reads x_dev itself), so x_dev
 * must hold its values until the runs are issued. A run must follow the prep
 * of the same kind of tensor and the same S. */
int coli_hip_gemm_prep_dev(ColiCudaTensor *tensor, const float *x_dev, int S);
int coli_hip_gemm_run_dev(ColiCudaTensor *tensor, float *y_dev, int S);
/* As coli_hip_gemm_run_dev, and the output rows are also written, from the
 * GEMV's epilogue, as the activation fragments of `next` (next->I ==
 * tensor->O, fp16 hi + lo with one exponent per row and 32-column group), so
 * that a following coli_hip_gemm_prep_dev(next, y_dev, S) + run needs no
 * fragment build (an FFN's up projection feeding its down projection).
 * Emitted only where it pays and the launch allows it (2..16 rows whose f32
 * form next's GEMV would not convert itself, tensor->O a multiple of 128, a
 * plain launch with an even number of row tiles per wave and no K split);
 * otherwise the later prep builds the fragments as usual. The caller must not
 * modify y_dev between this call and that prep's run; another run writing
 * y_dev drops the emitted fragments. Returns 2 when the fragments were
 * emitted, 1 when only the GEMV ran, 0 on failure. */
int coli_hip_gemm_run_dev_emit(ColiCudaTensor *tensor, float *y_dev, int S, const ColiCudaTensor *next);
/* Fill n bytes of device memory with uniform pseudo-random bytes (seeded,
 * deterministic): synthetic weights for benchmarks without a host round trip. */
int coli_hip_fill_random_u8(int device, void *dev, size_t n, unsigned long long seed);
/* Queue a plain streaming read of `bytes` (a multiple of 16, 16-byte aligned)
 * of device memory on the device's stream: no arithmetic, nothing written.
 * The benchmark's reference for what one launch of a given size can read. */
int coli_hip_stream_read(int device, const void *dev, size_t bytes);
/* The hipStream_t every asynchronous entry point of `device` runs on. */
void *coli_hip_stream(int device);
/* Bytes the tensor streams per full GEMV (weights + scales, tiled storage). */
size_t coli_hip_tensor_stream_bytes(const ColiCudaTensor *tensor);
/* Storage kind: 0 int4+fp16 scales, 1 int4+f32 scales, 2 MXFP4, 3 generic int4. */
int coli_hip_tensor_kind(const ColiCudaTensor *tensor);

#ifdef __cplusplus
}
#endif

#endif
