/* ref_shim.c -- exposes the reference's own static CPU kernels as symbols.
 *
 * TEST INFRASTRUCTURE ONLY (oracle/_ref). Compiled in the build container
 * from the reference sources where they lie (COLI_REF_DIR, default
 * /root/reference/c): quant.h is #included from there, nothing is copied.
 * The same arrangement the reference itself uses for its GPU differential
 * tests (c/tests/mxfp4_ref.c:1-12). Built with -march=x86-64-v3, i.e. the
 * reference's AVX2+FMA code paths.
 */
#include "quant.h"

void ref_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O) {
    matmul(y, x, W, S, I, O);
}
void ref_matmul_i4_grouped(float *y, const float *x, const uint8_t *q4,
                           const float *scale, int S, int I, int O, int gs) {
    matmul_i4_grouped(y, x, q4, scale, S, I, O, gs);
}
void ref_matmul_i4(float *y, const float *x, const uint8_t *q4,
                   const float *scale, int S, int I, int O) {
    matmul_i4(y, x, q4, scale, S, I, O);
}
void ref_matmul_i4_pair(float *yg, float *yu, const float *x,
                        const uint8_t *qg, const float *sg,
                        const uint8_t *qu, const float *su, int I, int O) {
    matmul_i4_pair(yg, yu, x, qg, sg, qu, su, I, O);
}
void ref_matmul_mxfp4(float *y, const float *x, const uint8_t *q4,
                      const uint8_t *e8, int S, int I, int O) {
    matmul_mxfp4(y, x, q4, e8, S, I, O);
}
void ref_matmul_mxfp4_i8(float *y, const float *x, const uint8_t *q4,
                         const uint8_t *e8, int S, int I, int O) {
    matmul_mxfp4_i8(y, x, q4, e8, S, I, O);
}
float ref_qrow_i8(const float *x, int8_t *q, int I) { return qrow_i8(x, q, I); }
/* the fmt=2 IDOT path as c/colibri.c:937-945 runs it: qrow_i8 per row, then
 * matmul_i4_idot */
void ref_matmul_i4_idot(float *y, const float *x, const uint8_t *q4,
                        const float *scale, int S, int I, int O) {
    int8_t *xq = (int8_t *)malloc((size_t)S * (I > 0 ? I : 1));
    float *sx = (float *)malloc((size_t)(S > 0 ? S : 1) * sizeof(float));
    if (!xq || !sx) { free(xq); free(sx); return; }
    for (int s = 0; s < S; s++) sx[s] = qrow_i8(x + (int64_t)s * I, xq + (int64_t)s * I, I);
    matmul_i4_idot(y, xq, sx, q4, scale, S, I, O);
    free(xq);
    free(sx);
}
