/* coli_backend_abi.h -- the GPU backend C ABI that libcoli_hip.so exports.
 *
 * This is the drop-in boundary: colibri's engine binds exactly these
 * `coli_cuda_*` symbols (statically on Linux, through GetProcAddress on
 * Windows: c/backend_loader.c:1355-1435), whichever vendor backend provides
 * them; the prefix stays `coli_cuda_` for every vendor
 * (c/backend_loader.c:38-41). Each declaration below cites the reference
 * declaration it replaces in c/backend_cuda.h. Names, argument order and
 * meaning, and return conventions are the reference's; the implementation
 * behind them is this repository's gfx950 backend.
 *
 * Conventions (c/backend_cuda.h, c/backend_cuda.cu:127-133, 1340-1348):
 *   - success returns 1 (or a non-NULL pointer); any failure returns 0 / NULL
 *     and leaves outputs untouched so the caller recomputes on the CPU;
 *   - failures never abort; a diagnostic line tagged "[HIP]" goes to stderr
 *     and the sticky device error is consumed;
 *   - COLI_GPU_FAIL_AFTER=N makes every compute entry point fail after N
 *     successful calls (host-forced fault injection for CPU-fallback tests);
 *   - fmt codes: 0 f32, 1 int8, 2 int4 per-row scale, 3 int2, 4 int4 with
 *     per-group f32 scales (gs), 6 E8, 7 MXFP4, 8 fp8. This backend computes
 *     fmt 2, 4 and 7 (the quantized MoE expert path); other formats are
 *     refused with 0 so the engine keeps its CPU path for them;
 *   - int4 nibbles arrive offset-binary (stored u means u-8), low nibble =
 *     even column (c/quant.h:161-163); scales arrive as f32.
 *   - x / y of the group calls hold sum(rows) consecutive rows in call order.
 */
#ifndef COLI_BACKEND_ABI_H
#define COLI_BACKEND_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define COLI_CUDA_MAX_DEVICES 16

/* Opaque resident quantized tensor (c/backend_cuda.h:25). */
typedef struct ColiCudaTensor ColiCudaTensor;

/* ---- lifecycle and queries ---------------------------------------------- */
int coli_cuda_init(const int *devices, int count);                           /* backend_cuda.h:28 */
void coli_cuda_shutdown(void);                                               /* backend_cuda.h:29 */
int coli_cuda_device_count(void);                                            /* backend_cuda.h:30 */
int coli_cuda_device_at(int index);                                          /* backend_cuda.h:31 */
int coli_cuda_mem_info(int device, size_t *free_bytes, size_t *total_bytes); /* backend_cuda.h:32 */
int coli_cuda_device_integrated(int device);                                 /* backend_cuda.h:33 */
void coli_cuda_stats(int device, size_t *tensor_count, size_t *tensor_bytes);/* backend_cuda.h:35 */
void coli_cuda_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows,
                           double *h2d_ms, double *kernel_ms, double *d2h_ms);  /* backend_cuda.h:36 */
void coli_cuda_group_stats_device(int device, uint64_t *calls, uint64_t *experts,
                                  uint64_t *rows, double *h2d_ms, double *kernel_ms,
                                  double *d2h_ms);                              /* backend_cuda.h:39 */
/* fmt 6 / fmt 8 tables: not computed by this backend, always 0 (optional
 * symbols in the loader, c/backend_loader.c:1399-1400). */
int coli_cuda_e8_set_grid(const void *grid);                                 /* backend_cuda.h:46 */
int coli_cuda_fp8_set_lut(const float *lut);                                 /* backend_cuda.h:51 */

/* ---- resident tensors ---------------------------------------------------- */
/* fmt 2/4: int4 + f32 scales ([O] per row, or [O, ceil(I/gs)] for fmt 4);
 * fmt 7: MXFP4 nibbles + scales passed as f32 exact powers of two with
 * gs = 32 (the Vulkan resident convention, docs/FORMATS.md:68), stored as
 * e8m0 bytes. A non-NULL *tensor is reused only if fmt, I, O, device and gs
 * all match (c/backend_cuda.cu:1101-1110). */
int coli_cuda_tensor_upload_g(ColiCudaTensor **tensor, const void *weights,
                              const float *scales, int fmt, int I, int O,
                              int device, int gs);                           /* backend_cuda.h:54 */
int coli_cuda_tensor_upload(ColiCudaTensor **tensor, const void *weights,
                            const float *scales, int fmt, int I, int O,
                            int device);                                     /* backend_cuda.h:57 */
void coli_cuda_tensor_free(ColiCudaTensor *tensor);                          /* backend_cuda.h:148 */
size_t coli_cuda_tensor_bytes(const ColiCudaTensor *tensor);                 /* backend_cuda.h:149 */
int coli_cuda_tensor_device(const ColiCudaTensor *tensor);                   /* backend_cuda.h:150 */
int coli_cuda_tensor_update(ColiCudaTensor *tensor, const void *weights,
                            const float *scales);                            /* backend_cuda.h:153 */

/* ---- compute (host pointers) ---------------------------------------------- */
/* y[S,O] = x[S,I] @ dequant_mxfp4(W)^T, stateless (c/backend_cuda.h:76-84). */
int coli_cuda_matmul_mxfp4(float *y, const float *x, const unsigned char *q4,
                           const unsigned char *e8s, int S, int I, int O);   /* backend_cuda.h:81 */
/* y[S,O] = x[S,I] @ W^T; the first call uploads and caches (backend_cuda.h:86). */
int coli_cuda_matmul(ColiCudaTensor **tensor, float *y, const float *x,
                     const void *weights, const float *scales, int fmt, int S,
                     int I, int O, int device, int gs);                      /* backend_cuda.h:86 */
/* y = down(silu(gate(x)) * up(x)) for S rows of one expert (backend_cuda.h:94). */
int coli_cuda_expert_mlp(ColiCudaTensor *gate, ColiCudaTensor *up,
                         ColiCudaTensor *down, float *y, const float *x, int S);  /* backend_cuda.h:94 */
/* Prefill shared expert (fmt=2 in the reference): same math as expert_mlp. */
int coli_cuda_shared_mlp_w4a16(ColiCudaTensor *gate, ColiCudaTensor *up,
                               ColiCudaTensor *down, float *y, const float *x,
                               int S);                                       /* backend_cuda.h:101 */
/* Packed group of same-shaped experts; rows[c] consecutive rows per expert. */
int coli_cuda_expert_group_issue(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups,
                                 ColiCudaTensor *const *downs, const int *rows,
                                 int count, const float *x);                 /* backend_cuda.h:111 */
const float *coli_cuda_expert_group_take(int device);                        /* backend_cuda.h:115 */
int coli_cuda_expert_group(ColiCudaTensor *const *gates, ColiCudaTensor *const *ups,
                           ColiCudaTensor *const *downs, const int *rows, int count,
                           float *y, const float *x);                        /* backend_cuda.h:117 */

/* ---- MLA attention: outside this backend's scope, always 0 --------------- */
int coli_cuda_attention_absorb(ColiCudaTensor *kv_b, float *ctx, const float *q,
                               const float *latent, const float *rope, int H, int Q,
                               int R, int V, int K, int T, float attention_scale);  /* backend_cuda.h:124 */
int coli_cuda_attention_absorb_batch(ColiCudaTensor *kv_b, float *ctx, const float *q,
                                     const float *latent, const float *rope, int S,
                                     int H, int Q, int R, int V, int K, int T,
                                     float attention_scale);                 /* backend_cuda.h:131 */
int coli_cuda_attention_project_batch(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj,
                                      float *out, const float *q, const float *latent,
                                      const float *rope, int S, int H, int Q, int R,
                                      int V, int K, int T, float attention_scale);  /* backend_cuda.h:138 */
int coli_cuda_attention_project_ragged(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj,
                                       float *out, const float *q, const void *const *keys,
                                       const float *const *latent, const float *const *rope,
                                       const int *lengths, int S, int H, int Q, int R,
                                       int V, int K, int max_t, float attention_scale);  /* backend_cuda.h:143 */
int coli_cuda_attention_project_batch_dev(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj,
                                          float *out, const float *q_dev, const float *latent_dev,
                                          const float *rope_dev, int S, int H, int Q, int R,
                                          int V, int K, int T, float scale);  /* backend_cuda.h:188 */
int coli_cuda_attention_absorb_batch_dev(ColiCudaTensor *kv_b_shard, float *ctx_dev,
                                         const float *q_dev, const float *latent_dev,
                                         const float *rope_dev, int S, int H, int Q, int R,
                                         int V, int K, int T, float scale);   /* backend_cuda.h:191 */
int coli_cuda_attention_absorb_kvdev(ColiCudaTensor *kv_b, float *ctx, const float *q,
                                     const float *latent_dev, const float *rope_dev, int H,
                                     int Q, int R, int V, int K, int T, float scale);  /* backend_cuda.h:194 */
int coli_cuda_attention_project_batch_dev_out(ColiCudaTensor *kv_b, ColiCudaTensor *o_proj,
                                              float *out_dev, const float *q_dev,
                                              const float *latent_dev, const float *rope_dev,
                                              int S, int H, int Q, int R, int V, int K, int T,
                                              float scale);                  /* backend_cuda.h:199 */

/* ---- resident pipeline (device pointers) --------------------------------- */
float *coli_cuda_pipe_scratch(int device, int slot, size_t bytes);          /* backend_cuda.h:157 */
void *coli_cuda_pipe_alloc(int device, size_t bytes);                        /* backend_cuda.h:158 */
void coli_cuda_pipe_free(int device, void *p);                               /* backend_cuda.h:159 */
int coli_cuda_pipe_upload(int device, void *dst, const void *src, size_t bytes);    /* backend_cuda.h:160 */
int coli_cuda_pipe_download(int device, const void *src, void *dst, size_t bytes);  /* backend_cuda.h:161 */
/* rmsnorm / rope belong to attention-side layers outside this backend: 0. */
int coli_cuda_pipe_rmsnorm(int device, float *y_dev, const float *x_dev,
                           const float *w_dev, int S, int D, float eps);     /* backend_cuda.h:162 */
int coli_cuda_pipe_rope(int device, float *v_dev, const int *pos_dev, int rows,
                        int stride, int offset, int R, int heads, float theta);  /* backend_cuda.h:164 */
int coli_cuda_pipe_silu_mul(int device, float *gate_dev, const float *up_dev, size_t n);  /* backend_cuda.h:166 */
int coli_cuda_pipe_add(int device, float *x_dev, const float *t_dev, size_t n);  /* backend_cuda.h:167 */
int coli_cuda_pipe_rows_add(int device, float *x_dev, const float *partial_dev,
                            const int *rows_dev, int nrows, int D);          /* backend_cuda.h:168 */
int coli_cuda_pipe_gemm(ColiCudaTensor *t, float *y_dev, const float *x_dev, int S);  /* backend_cuda.h:170 */
int coli_cuda_pipe_rmsnorm_s(int device, float *y_dev, const float *x_dev,
                             const float *w_dev, int S, int D, float eps,
                             int xstride, int ystride);                      /* backend_cuda.h:171 */
int coli_cuda_pipe_rope_base(int device, float *v_dev, int pos_base, int rows,
                             int stride, int offset, int R, int heads, float theta);  /* backend_cuda.h:174 */
/* Decode group with on-device weighted reduction into a slot of the home
 * device (c/backend_cuda.cu:2246-2301). */
int coli_cuda_expert_group_resident_issue(ColiCudaTensor *const *gates,
                                          ColiCudaTensor *const *ups,
                                          ColiCudaTensor *const *downs,
                                          const float *weights, int count,
                                          int home_device, const float *x_src_dev,
                                          float *partial_slot_dev);          /* backend_cuda.h:176 */
int coli_cuda_expert_group_resident_take(int home_device, const int *devices,
                                         int n_issued, float *slots_dev,
                                         float *acc_dev, int D);             /* backend_cuda.h:180 */
/* One decode row: logits = Wr x, sigmoid, choice = sigmoid + bias, top-K
 * (strict >, lowest index wins), route TOPP, norm_topk, routed_scale
 * (c/backend_cuda.cu:2139-2215). */
int coli_cuda_pipe_router(int device, const float *x_dev, const void *rw_dev,
                          const void *rb_dev, int D, int E, int Ksel, float topp,
                          int norm_topk, float routed_scale, int *idx_host,
                          float *w_host, int *keff_host);                    /* backend_cuda.h:182 */
int coli_cuda_pipe_copy2d(int device, float *dst, int dpitch, const float *src,
                          int spitch, int width, int height);                /* backend_cuda.h:186 */
int coli_cuda_pipe_peer_copy(int dst_dev, float *dst, int src_dev, const float *src,
                             size_t bytes);                                  /* backend_cuda.h:197 */
int coli_cuda_pipe_sync(int device);                                         /* backend_cuda.h:202 */

#ifdef __cplusplus
}
#endif

#endif
