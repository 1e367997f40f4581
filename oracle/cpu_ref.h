/* cpu_ref.h -- CPU restatement of colibri's quantized MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity oracle and the timed
 * CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker. The product path
 * (libcoli_hip.so) never links, loads or falls back to it.
 *
 * Every function restates the reference algorithm from the mathematics and
 * the reference's documented loop structure; each cites the reference
 * file:line it follows (paths relative to the colibri source tree).
 *
 * Pinning status (how each function is checked before it is trusted):
 *   cref_e2m1_decode / cref_e8m0_decode / cref_e4m3fn_* / cref_bf16_round:
 *       known-answer tests of c/tests/test_native_quant.c:13-52 + exhaustive
 *       256-code comparison with the compiled reference (oracle/_ref).
 *   cref_fp8_activation_qdq: test_native_quant.c:40-45 KAT (scale 119) +
 *       bitwise vs oracle/_ref on random vectors.
 *   cref_matmul_i4_grouped: bitwise vs oracle/_ref matmul_i4_grouped on
 *       aligned shapes; double-precision brute force with the
 *       magnitude-relative 1e-6 metric of c/tests/test_i4_grouped.c:28-54
 *       on ragged shapes; closed form (unit scales, x = e_i gives nibble-8).
 *   cref_matmul_i4: fmt=2 == fmt=4 with gs = I (c/tests/test_grouped_g4_cuda.cu:29-46)
 *   cref_qrow_i8 / cref_matmul_i4_idot (fmt=2 int8 activations): bitwise vs
 *       oracle/_ref qrow_i8 + matmul_i4_idot and tests/golden/golden_idot.npz;
 *       the exact-integer closed form (int64 dot, then the two f32 products).
 *       + brute force.
 *   cref_matmul_mxfp4: bitwise vs oracle/_ref matmul_mxfp4; all-16-codes
 *       exactness (c/tests/test_mxfp4_cuda.cu:106-132); e8 edges 0/127/255.
 *   cref_matmul_mxfp4_i8: bitwise vs tests/golden/golden_mxfp4_i8.npz and
 *       oracle/_ref matmul_mxfp4_i8; the int8 quantization checked against
 *       its definition (|q| <= 127, q = nearest integer of x / sc, the
 *       group maximum maps to +-127); float64 dequantized product within
 *       the quantization bound; I % 32 != 0 equals matmul_mxfp4.
 *   cref_fp4_matvec / cref_fp4_matmul_batch: fp4 matvec KAT = 128.0
 *       (test_native_quant.c:76-88) + bitwise vs oracle/_ref.
 *   cref_fp4_pack_rows16 / cref_fp4_matvec_rows16: bitwise vs oracle/_ref
 *       + permutation invariant rows16(W) == row-major(W) up to the
 *       no-FMA order (c/deepseek_v4.c:11059-11062).
 *   cref_route mode 3 (DeepSeek-V4 sqrt-softplus) and cref_swiglu_v4:
 *       bitwise vs oracle/_ref coli_v4_route / coli_v4_swiglu and
 *       tests/golden/golden_v4.npz; score and clamp closed forms.
 *   cref_route_*: brute force (full stable sort of all E) + NaN fallback
 *       (c/tests/test_router_nan.c:37-75 semantics).
 *   cref_expert_union: set invariant + first-seen order.
 *   cref_swiglu: closed form.
 *   cref_moe_layer: against the layer evaluated in float64 from dequantized
 *       weights (full-sort router, silu * up, slot-order weighted sum, shared
 *       expert weight 1) in fmt 4 / 7 / 17, route modes 0-3, with and
 *       without the shared expert: indices exact, outputs within 2e-5 of
 *       the magnitude sum (tests/test_oracle_cpu.py
 *       test_moe_layer_vs_f64_composition).
 */
#ifndef COLI_CPU_REF_H
#define COLI_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- codecs ---------------------------------------------------------- */
float cref_e2m1_decode(uint8_t nibble);
float cref_e8m0_decode(uint8_t value);          /* native_quant semantics: 0xff NaN */
float cref_mx4_scale(uint8_t value);            /* quant.h bit trick: 0 -> +0, 255 -> +inf */
float cref_e4m3fn_decode(uint8_t value);
uint8_t cref_e4m3fn_encode(float value);
float cref_bf16_round(float value);
int cref_fp8_activation_qdq(float *out, uint8_t *scales, const float *in,
                            size_t length, size_t block);

/* ---- GEMV / GEMM (y[S,O] = x[S,I] W^T) --------------------------------- */
void cref_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O);
void cref_matmul_i4_grouped(float *y, const float *x, const uint8_t *q4,
                            const float *scale, int S, int I, int O, int gs);
float cref_qrow_i8(const float *x, int8_t *q, int I);
void cref_matmul_i4_idot(float *y, const float *x, const uint8_t *q4,
                         const float *scale, int S, int I, int O);
void cref_matmul_i4(float *y, const float *x, const uint8_t *q4,
                    const float *scale, int S, int I, int O);
void cref_matmul_mxfp4(float *y, const float *x, const uint8_t *q4,
                       const uint8_t *e8, int S, int I, int O);
void cref_matmul_mxfp4_i8(float *y, const float *x, const uint8_t *q4,
                          const uint8_t *e8, int S, int I, int O);
/* native_quant contract: e4m3 QDQ of each activation row (block 128), then
 * the fmt=7 GEMV. Returns 0 on success, -1 on invalid shape (cols%128). */
int cref_fp4_matmul_batch(float *y, const uint8_t *q4, const uint8_t *e8,
                          int rows, int cols, const float *x, int batch);
int cref_fp4_pack_rows16(uint8_t *pdata, uint8_t *pscales, const uint8_t *q4,
                         const uint8_t *e8, int rows, int cols);
int cref_fp4_matvec_rows16(float *y, const uint8_t *pdata, const uint8_t *pscales,
                           int rows, int cols, const float *x);

/* ---- routing ----------------------------------------------------------- */
/* mode 0: softmax over E then top-K of probabilities (olmoe.c:246-250, 666-681)
 * mode 1: sigmoid, choice = sigmoid + bias, weight = sigmoid (colibri.c:3978-4126)
 * mode 2: sigmoid-normalized: like mode 1 but weights renormalized over the
 *         selected K with +1e-20 (kimi_k3.c:1337-1356)
 * topp in (0,1) applies the route-level TOPP truncation of
 * backend_cuda.cu:2183-2188 (modes 1/2). norm_topk renormalizes the kept
 * weights; routed_scale multiplies them (modes 1/2).
 * logits[S,E] in, idx[S,K], w[S,K], keff[S] out. */
void cref_route(const float *logits, const float *bias, int S, int E, int K,
                int mode, float topp, int norm_topk, float routed_scale,
                int *idx, float *w, int *keff);
/* Unique experts in first-seen (s, kk) order (colibri.c:4146-4152) and, for
 * each, its position list in ascending s (kimi_k3.c:1386-1410 counting sort).
 * Returns nu. rows_of[j*S .. +cnt[j]] are token indices; slot_of[j*S+..]
 * the kk slot; wsel the weights. */
int cref_expert_union(const int *idx, const float *w, const int *keff, int S, int K,
                      int E, int *uniq, int *cnt, int *rows_of, int *slot_of,
                      float *wsel);

/* h = silu(g) * u, the exact expression of backend_cuda.cu:417-423 / 618-624 */
void cref_swiglu(float *h, const float *g, const float *u, size_t n);
void cref_swiglu_v4(float *h, const float *g, const float *u, size_t n, float limit);

/* One MoE layer, decode rows x[S,D] -> out[S,D].
 * fmt 4: int4 group-scaled (scales f32 [O, I/gs]); fmt 7: MXFP4 (e8 bytes);
 * fmt 17: MXFP4 with the native_quant e4m3-QDQ activation contract.
 * Expert e's tensors are gq[e]/gs[e] (gate [I,D]), uq/us (up [I,D]),
 * dq/ds (down [D,I]). has_shared adds one always-on expert (weight 1) after
 * the routed sum (colibri.c:4940-5002 FASE E order). */
typedef struct {
    int fmt, D, I, E, K, gs, route_mode, norm_topk, has_shared;
    float topp, routed_scale;
    const float *router_w;      /* [E, D] f32 */
    const float *router_bias;   /* [E] or NULL */
    const uint8_t *const *gq; const void *const *gsc;
    const uint8_t *const *uq; const void *const *usc;
    const uint8_t *const *dq; const void *const *dsc;
    const uint8_t *sh_gq, *sh_uq, *sh_dq;
    const void *sh_gsc, *sh_usc, *sh_dsc;
} CrefMoe;
int cref_moe_layer(const CrefMoe *m, const float *x, int S, float *out,
                   int *idx, float *w, int *keff);

#ifdef __cplusplus
}
#endif
#endif
