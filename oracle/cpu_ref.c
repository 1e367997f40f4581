/* cpu_ref.c -- CPU restatement of colibri's quantized MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity oracle and the timed CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, as the checker. The product library never links or calls it.
 *
 * Build: see oracle/Makefile (-O3 -fopenmp -ffp-contract=off; every fused
 * multiply-add that the reference's AVX2 path performs is written here as an
 * explicit fmaf, every separate multiply/add as separate operations, so the
 * association matches the reference's vector code on every host).
 */
#include "cpu_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------
 * Codecs -- c/deepseek_v4.c:10390-10487 (native_quant) and c/quant.h:1375-1390
 * ------------------------------------------------------------------------ */

/* OCP e2m1: bit3 sign, bits0..2 index {0,.5,1,1.5,2,3,4,6}
 * (c/deepseek_v4.c:10395-10401). Code 8 decodes to -0. */
float cref_e2m1_decode(uint8_t nibble) {
    int n = nibble & 15, e = (n >> 1) & 3, m = n & 1;
    float mag = e ? ldexpf(1.0f + 0.5f * (float)m, e - 1) : 0.5f * (float)m;
    return (n & 8) && mag != 0.0f ? -mag : mag;  /* code 8 decodes to +0 */
}

/* native_quant e8m0: 2^(v-127), 0xff -> NaN (c/deepseek_v4.c:10390-10393). */
float cref_e8m0_decode(uint8_t value) {
    if (value == 0xff) return NAN;
    return ldexpf(1.0f, (int)value - 127);
}

/* quant.h's fmt=7 scale: (u32)v << 23 reinterpreted, so 0 -> +0 and
 * 255 -> +inf (c/quant.h:1386-1390). */
float cref_mx4_scale(uint8_t value) {
    union { uint32_t u; float f; } b;
    b.u = (uint32_t)value << 23;
    return b.f;
}

/* e4m3fn (no inf; 0x7f/0xff NaN), c/deepseek_v4.c:10403-10415. */
float cref_e4m3fn_decode(uint8_t value) {
    int sign = value >> 7, exponent = (value >> 3) & 15, mantissa = value & 7;
    if (exponent == 15 && mantissa == 7) return NAN;
    float number = exponent ? ldexpf(1.0f + (float)mantissa / 8.0f, exponent - 7)
                            : ldexpf((float)mantissa, -9);
    return sign ? -number : number;
}

/* Round-to-nearest-even encode with saturation to 448
 * (c/deepseek_v4.c:10417-10462). Restated on the binary32 fields: below the
 * normal range the value is an integer multiple of 2^-9; above, the 24-bit
 * significand is rounded to 4 bits. */
uint8_t cref_e4m3fn_encode(float value) {
    if (isnan(value)) return 0x7f;
    int negative = signbit(value) != 0;
    float magnitude = fabsf(value);
    uint8_t sign = negative ? 0x80 : 0;
    if (magnitude == 0.0f) return sign;
    if (magnitude >= 448.0f) return (uint8_t)(sign | 0x7e);
    uint8_t code;
    if (magnitude < 0.015625f) {                      /* < 2^-6: subnormal grid */
        float scaled = magnitude * 512.0f;            /* exact: power of two */
        uint32_t whole = (uint32_t)scaled;
        float frac = scaled - (float)whole;
        if (frac > 0.5f || (frac == 0.5f && (whole & 1u))) whole++;
        code = (uint8_t)whole;                        /* 8 -> smallest normal */
    } else {
        uint32_t bits;
        memcpy(&bits, &magnitude, 4);
        int e = (int)((bits >> 23) & 0xff) - 127;
        uint32_t sig = 0x800000u | (bits & 0x7fffffu);
        uint32_t keep = sig >> 20, rest = sig & 0xfffffu;
        if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) keep++;
        if (keep == 16u) { keep = 8u; e++; }
        code = (uint8_t)((e + 7) * 8 + (int)keep - 8);
    }
    return (uint8_t)(code | sign);
}

/* bf16 round-to-nearest-even on the bit pattern, non-finite values kept
 * (c/deepseek_v4.c:10464-10475). */
float cref_bf16_round(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if ((bits & 0x7f800000u) != 0x7f800000u) bits += 0x7fffu + ((bits >> 16) & 1u);
    bits &= 0xffff0000u;
    memcpy(&value, &bits, 4);
    return value;
}

/* ceil(log2(v)) for v > 0 (c/deepseek_v4.c:10489-10493). */
static int ceil_log2_pos(float v) {
    int e;
    float f = frexpf(v, &e);
    return f == 0.5f ? e - 1 : e;
}

/* Dynamic e4m3 activation quantize-dequantize, one e8m0 power-of-two scale
 * per block (c/deepseek_v4.c:10495-10520). */
int cref_fp8_activation_qdq(float *out, uint8_t *scales, const float *in,
                            size_t length, size_t block) {
    if (!out || !scales || !in || !length || !block) return -1;
    for (size_t base = 0; base < length; base += block) {
        size_t n = length - base < block ? length - base : block;
        float mx = 0.0f;
        for (size_t i = 0; i < n; i++) mx = fmaxf(mx, fabsf(in[base + i]));
        mx = fmaxf(mx, 1e-4f);
        int se = ceil_log2_pos(mx / 448.0f);
        if (se < -127) se = -127;
        if (se > 127) se = 127;
        uint8_t code = (uint8_t)(se + 127);
        float sc = cref_e8m0_decode(code);
        scales[base / block] = code;
        for (size_t i = 0; i < n; i++) {
            float v = fmaxf(-448.0f, fminf(448.0f, in[base + i] / sc));
            out[base + i] = cref_e4m3fn_decode(cref_e4m3fn_encode(v)) * sc;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------
 * GEMV kernels
 * ------------------------------------------------------------------------ */

/* Horizontal sum of an 8-lane accumulator in the reference's order
 * (c/quant.h:20-24): ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). */
static inline float hsum8(const float a[8]) {
    float l0 = a[0] + a[4], l1 = a[1] + a[5], l2 = a[2] + a[6], l3 = a[3] + a[7];
    return (l0 + l2) + (l1 + l3);
}

/* y = x W^T, W f32 [O,I]; the loop of c/quant.h:97-102 as gcc -O3
 * -march=x86-64-v3 builds it: ascending i, each product rounded then added
 * (the vectorised body) for i < (I & ~3), and the last I mod 4 columns
 * contracted to one fma each (the scalar epilogue). */
void cref_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O) {
    const int body = I & ~3;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const float *w = W + (int64_t)o * I;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float a = 0.0f;
            for (int i = 0; i < body; i++) {
                float p = xs[i] * w[i];
                a = a + p;
            }
            for (int i = body; i < I; i++) a = fmaf(xs[i], w[i], a);
            y[(int64_t)s * O + o] = a;
        }
    }
}

static inline int nib_at(const uint8_t *w, int i) {
    uint8_t b = w[i >> 1];
    return (i & 1) ? (b >> 4) : (b & 15);
}

/* fmt=4 grouped int4, c/quant.h:168-202. Per group: an 8-lane accumulator
 * takes the 16-column chunks (columns i..i+7 then i+8..i+15, one fma each),
 * is reduced with hsum8, multiplied by the group scale and added to the row
 * accumulator (fused: a = fma(hsum, sc, a)). The group's ragged tail
 * (glen % 16) runs the scalar pair loop of c/quant.h:193-197. */
void cref_matmul_i4_grouped(float *y, const float *x, const uint8_t *q4,
                            const float *scale, int S, int I, int O, int gs) {
    int rb = (I + 1) / 2, ng = (I + gs - 1) / gs;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        const float *scl = scale + (int64_t)o * ng;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float a = 0.0f;
            for (int g = 0; g * gs < I; g++) {
                int base = g * gs, glen = gs;
                if (base + glen > I) glen = I - base;
                float sc = scl[g];
                int i = base;
                float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (; i + 16 <= base + glen; i += 16) {
                    for (int j = 0; j < 8; j++)
                        acc[j] = fmaf(xs[i + j], (float)(nib_at(w, i + j) - 8), acc[j]);
                    for (int j = 0; j < 8; j++)
                        acc[j] = fmaf(xs[i + 8 + j], (float)(nib_at(w, i + 8 + j) - 8), acc[j]);
                }
                a = fmaf(hsum8(acc), sc, a);
                for (; i < base + glen; i += 2) {
                    if (i + 1 < base + glen) {
                        float t = fmaf(xs[i + 1], (float)(nib_at(w, i + 1) - 8),
                                       xs[i] * (float)(nib_at(w, i) - 8));
                        a = fmaf(t, sc, a);
                    } else {
                        a = fmaf(xs[i] * (float)(nib_at(w, i) - 8), sc, a);
                    }
                }
            }
            y[(int64_t)s * O + o] = a;
        }
    }
}

/* fmt=2 per-row int4, c/quant.h:125-165 (the 16-column AVX2 body: one
 * 8-lane accumulator over the whole row, hsum8, pair tail, then x scale). */
/* Row quantization of the int8-activation (IDOT) path, qrow_i8
 * (c/quant.h:581-586): s = max|x| / 127 (at least 1e-12), q = rint(x * (1 / s))
 * in f32, no clamp. Returns s. */
float cref_qrow_i8(const float *x, int8_t *q, int I) {
    float amax = 0.0f;
    for (int i = 0; i < I; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float s = amax / 127.f;
    if (s < 1e-12f) s = 1e-12f;
    float inv = 1.f / s;
    for (int i = 0; i < I; i++) q[i] = (int8_t)lrintf(x[i] * inv);
    return s;
}

/* fmt=2 with int8 activations (the IDOT path, c/colibri.c:937-945 and
 * matmul_i4_idot c/quant.h:924-933 with dot_i4i8 674-801): each row is
 * quantized by qrow_i8; y[s, o] = (float)(sum_i (nib - 8) * q[s, i]) *
 * scale[o] * sx[s], the integer sum exact. */
void cref_matmul_i4_idot(float *y, const float *x, const uint8_t *q4,
                         const float *scale, int S, int I, int O) {
    int rb = (I + 1) / 2;
    int8_t *xq = (int8_t *)malloc((size_t)S * (I > 0 ? I : 1));
    float *sx = (float *)malloc((size_t)(S > 0 ? S : 1) * sizeof(float));
    if (!xq || !sx) { free(xq); free(sx); return; }
    for (int s = 0; s < S; s++) sx[s] = cref_qrow_i8(x + (int64_t)s * I, xq + (int64_t)s * I, I);
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        for (int s = 0; s < S; s++) {
            const int8_t *xs = xq + (int64_t)s * I;
            int32_t d = 0;
            for (int i = 0; i < I; i++) d += (nib_at(w, i) - 8) * (int32_t)xs[i];
            y[(int64_t)s * O + o] = (float)d * scale[o] * sx[s];
        }
    }
    free(xq);
    free(sx);
}

void cref_matmul_i4(float *y, const float *x, const uint8_t *q4,
                    const float *scale, int S, int I, int O) {
    int rb = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int i = 0;
            for (; i + 16 <= I; i += 16) {
                for (int j = 0; j < 8; j++)
                    acc[j] = fmaf(xs[i + j], (float)(nib_at(w, i + j) - 8), acc[j]);
                for (int j = 0; j < 8; j++)
                    acc[j] = fmaf(xs[i + 8 + j], (float)(nib_at(w, i + 8 + j) - 8), acc[j]);
            }
            float a = hsum8(acc);
            for (; i + 1 < I; i += 2)
                a = a + fmaf(xs[i], (float)(nib_at(w, i) - 8),
                             xs[i + 1] * (float)(nib_at(w, i + 1) - 8));
            if (i < I) a = fmaf(xs[i], (float)(nib_at(w, i) - 8), a);
            y[(int64_t)s * O + o] = a * scale[o];
        }
    }
}

/* fmt=7 MXFP4, c/quant.h:1391-1440. When I % 32 == 0 (the AVX2 body): per
 * group the four 8-column slices of doubled e2m1 integers are folded into an
 * 8-lane group partial (first a multiply, then three fma), and the partial is
 * fma'd into the 8-lane row accumulator with (scale * 0.5); hsum8 at the end.
 * Otherwise the scalar per-group loop. */
void cref_matmul_mxfp4(float *y, const float *x, const uint8_t *q4,
                       const uint8_t *e8, int S, int I, int O) {
    static const float lut2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    int rb = (I + 1) / 2, ng = (I + 31) / 32;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        const uint8_t *scl = e8 + (int64_t)o * ng;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            if (I % 32 == 0) {
                float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int g = 0; g < ng; g++) {
                    const float *xg = xs + g * 32;
                    int c0 = g * 32;
                    float ga[8];
                    for (int j = 0; j < 8; j++) ga[j] = xg[j] * lut2[nib_at(w, c0 + j)];
                    for (int j = 0; j < 8; j++) ga[j] = fmaf(xg[8 + j], lut2[nib_at(w, c0 + 8 + j)], ga[j]);
                    for (int j = 0; j < 8; j++) ga[j] = fmaf(xg[16 + j], lut2[nib_at(w, c0 + 16 + j)], ga[j]);
                    for (int j = 0; j < 8; j++) ga[j] = fmaf(xg[24 + j], lut2[nib_at(w, c0 + 24 + j)], ga[j]);
                    float sc = cref_mx4_scale(scl[g]) * 0.5f;
                    for (int j = 0; j < 8; j++) acc[j] = fmaf(ga[j], sc, acc[j]);
                }
                y[(int64_t)s * O + o] = hsum8(acc);
                continue;
            }
            float a = 0.0f;
            for (int g = 0; g < ng; g++) {
                int base = g * 32, glen = 32;
                if (base + glen > I) glen = I - base;
                float sc = cref_mx4_scale(scl[g]), ga = 0.0f;
                for (int i = base; i < base + glen; i += 2) {
                    ga = fmaf(xs[i], cref_e2m1_decode((uint8_t)nib_at(w, i)), ga);
                    if (i + 1 < base + glen)
                        ga = fmaf(xs[i + 1], cref_e2m1_decode((uint8_t)nib_at(w, i + 1)), ga);
                }
                a = fmaf(ga, sc, a);
            }
            y[(int64_t)s * O + o] = a;
        }
    }
}

/* native_quant batch contract (c/deepseek_v4.c:10906-10933): each row is
 * e4m3-QDQ'd in blocks of 128, then the fmt=7 GEMV runs on the batch. */
int cref_fp4_matmul_batch(float *y, const uint8_t *q4, const uint8_t *e8,
                          int rows, int cols, const float *x, int batch) {
    if (!y || !q4 || !e8 || !x || rows < 1 || cols < 1 || cols % 128 || batch < 1)
        return -1;
    float *a = (float *)malloc((size_t)batch * cols * sizeof(float));
    uint8_t *sc = (uint8_t *)malloc((size_t)batch * cols / 128);
    if (!a || !sc) { free(a); free(sc); return -1; }
    for (int b = 0; b < batch; b++)
        cref_fp8_activation_qdq(a + (size_t)b * cols, sc + (size_t)b * cols / 128,
                                x + (size_t)b * cols, (size_t)cols, 128);
    cref_matmul_mxfp4(y, a, q4, e8, batch, cols, rows);
    free(a); free(sc);
    return 0;
}

/* MXFP4 with int8 activations (c/quant.h:1441-1515, the K3 IDOT path), AVX2
 * association: each row's 32-column groups are quantized to int8 with
 * sc = max|x| / 127 (floored at 1e-20), q = lrint(x * (1 / sc)) clamped to
 * +-127; the group's integer dot with the doubled e2m1 codes is kept as 8
 * int32 partials of 4 adjacent columns (maddubs + madd), each converted and
 * fused into its lane accumulator with the group scale
 * (mx4_scale(e8) * 0.5f) * sc, and the 8 lanes are summed as hsum256.
 * I % 32 != 0 falls back to matmul_mxfp4, as the reference does. */
void cref_matmul_mxfp4_i8(float *y, const float *x, const uint8_t *q4,
                          const uint8_t *e8, int S, int I, int O) {
    static const int lut2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    if (I % 32) {
        cref_matmul_mxfp4(y, x, q4, e8, S, I, O);
        return;
    }
    int rb = I / 2, ng = I / 32;
    int8_t *xq = (int8_t *)malloc((size_t)S * I);
    float *xsc = (float *)malloc((size_t)S * ng * sizeof(float));
    if (!xq || !xsc) {
        free(xq);
        free(xsc);
        return;
    }
    for (int s = 0; s < S; s++)
        for (int g = 0; g < ng; g++) {
            const float *xg = x + (int64_t)s * I + g * 32;
            float am = 0.0f;
            for (int i = 0; i < 32; i++) {
                float a = fabsf(xg[i]);
                if (a > am) am = a;
            }
            float sc = am / 127.f;
            if (sc < 1e-20f) sc = 1e-20f;
            xsc[(int64_t)s * ng + g] = sc;
            float inv = 1.f / sc;
            for (int i = 0; i < 32; i++) {
                int v = (int)lrintf(xg[i] * inv);
                if (v > 127) v = 127;
                if (v < -127) v = -127;
                xq[(int64_t)s * I + g * 32 + i] = (int8_t)v;
            }
        }
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        const uint8_t *scl = e8 + (int64_t)o * ng;
        for (int s = 0; s < S; s++) {
            const int8_t *xr = xq + (int64_t)s * I;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int g = 0; g < ng; g++) {
                float sc = cref_mx4_scale(scl[g]) * 0.5f * xsc[(int64_t)s * ng + g];
                for (int j = 0; j < 8; j++) {
                    int32_t lane = 0;
                    for (int i = 4 * j; i < 4 * j + 4; i++) lane += lut2[nib_at(w, g * 32 + i)] * xr[g * 32 + i];
                    acc[j] = fmaf((float)lane, sc, acc[j]);
                }
            }
            y[(int64_t)s * O + o] = hsum8(acc);
        }
    }
    free(xq);
    free(xsc);
}

/* 16-row interleave: packed[(tile*cols/2 + col)*16 + lane]
 * (c/deepseek_v4.c:10975-10993). */
int cref_fp4_pack_rows16(uint8_t *pdata, uint8_t *pscales, const uint8_t *q4,
                         const uint8_t *e8, int rows, int cols) {
    if (rows < 1 || rows % 16 || cols < 1 || cols % 128) return -1;
    size_t ds = (size_t)cols / 2, ss = (size_t)cols / 32;
    for (size_t r = 0; r < (size_t)rows; r++) {
        size_t tile = r / 16, lane = r % 16;
        for (size_t c = 0; c < ds; c++) pdata[(tile * ds + c) * 16 + lane] = q4[r * ds + c];
        for (size_t c = 0; c < ss; c++) pscales[(tile * ss + c) * 16 + lane] = e8[r * ss + c];
    }
    return 0;
}

/* rows16 matvec: e4m3 QDQ of x, then per row sum += (x * v) * scale in
 * ascending column order with no fused multiply-add
 * (c/deepseek_v4.c:11120-11170, 11059-11062); scale via native e8m0 decode. */
int cref_fp4_matvec_rows16(float *y, const uint8_t *pdata, const uint8_t *pscales,
                           int rows, int cols, const float *x) {
    if (rows < 1 || rows % 16 || cols < 1 || cols % 128) return -1;
    float *a = (float *)malloc((size_t)cols * sizeof(float));
    uint8_t *as = (uint8_t *)malloc((size_t)cols / 128);
    if (!a || !as) { free(a); free(as); return -1; }
    cref_fp8_activation_qdq(a, as, x, (size_t)cols, 128);
    size_t ds = (size_t)cols / 2, ss = (size_t)cols / 32;
    #pragma omp parallel for schedule(static)
    for (int tile = 0; tile < rows / 16; tile++) {
        for (int lane = 0; lane < 16; lane++) {
            float sum = 0.0f;
            for (size_t c = 0; c < (size_t)cols; c++) {
                uint8_t byte = pdata[((size_t)tile * ds + c / 2) * 16 + lane];
                float v = cref_e2m1_decode((c & 1) ? (byte >> 4) : (byte & 15));
                float sc = cref_e8m0_decode(pscales[((size_t)tile * ss + c / 32) * 16 + lane]);
                float p = a[c] * v;
                p = p * sc;
                sum = sum + p;
            }
            y[(size_t)tile * 16 + lane] = sum;
        }
    }
    free(a); free(as);
    return 0;
}

/* ------------------------------------------------------------------------
 * Routing
 * ------------------------------------------------------------------------ */

/* K-fold argmax with strict '>' (lowest index wins ties, NaN never wins);
 * an all-NaN row falls back to index kk < E ? kk : 0
 * (c/olmoe.c:668-680, c/route_trace.h:383-393, c/colibri.c:3858-3864). */
static void topk_scan(const float *score, int E, int K, int *idx) {
    for (int kk = 0; kk < K; kk++) {
        int best = -1;
        float bv = -1e30f;
        for (int e = 0; e < E; e++) {
            int taken = 0;
            for (int j = 0; j < kk; j++) if (idx[j] == e) { taken = 1; break; }
            if (!taken && score[e] > bv) { bv = score[e]; best = e; }
        }
        if (best < 0) best = kk < E ? kk : 0;
        idx[kk] = best;
    }
}

static float sigmoid_ref(float z) { return 1.0f / (1.0f + expf(-z)); }

void cref_route(const float *logits, const float *bias, int S, int E, int K,
                int mode, float topp, int norm_topk, float routed_scale,
                int *idx, float *w, int *keff) {
    float *p = (float *)malloc((size_t)E * sizeof(float));
    float *c = (float *)malloc((size_t)E * sizeof(float));
    for (int s = 0; s < S; s++) {
        const float *z = logits + (int64_t)s * E;
        int *ix = idx + (int64_t)s * K;
        float *wx = w + (int64_t)s * K;
        int ke = K;
        if (mode == 3) {
            /* DeepSeek-V4 (coli_v4_route, c/deepseek_v4.c:1368-1432): score =
             * sqrt(softplus(z)) (stable form), selection = score + bias,
             * top-K by strict > (the first unselected expert seeds each
             * round, so the lowest index wins ties), weight = score /
             * sum of the selected scores * route_scale. A non-positive sum
             * is an error there; here the row selects nothing (keff 0). */
            unsigned char *taken = (unsigned char *)calloc((size_t)E, 1);
            for (int e = 0; e < E; e++) {
                float v = z[e];
                p[e] = sqrtf(fmaxf(v, 0.0f) + log1pf(expf(-fabsf(v))));
                c[e] = p[e] + (bias ? bias[e] : 0.0f);
            }
            for (int kk = 0; kk < K; kk++) {
                int best = -1;
                for (int e = 0; e < E; e++)
                    if (!taken[e] && (best < 0 || c[e] > c[best])) best = e;
                ix[kk] = best;
                taken[best] = 1;
            }
            free(taken);
            float total = 0.0f;
            for (int kk = 0; kk < K; kk++) total += p[ix[kk]];
            if (!(total > 0.0f)) {
                ke = 0;
                for (int kk = 0; kk < K; kk++) wx[kk] = 0.0f;
            } else {
                for (int kk = 0; kk < K; kk++) wx[kk] = p[ix[kk]] / total * routed_scale;
            }
        } else if (mode == 0) {
            /* softmax_row, c/olmoe.c:246-250 */
            float m = -1e30f, sum = 0.0f;
            for (int e = 0; e < E; e++) if (z[e] > m) m = z[e];
            for (int e = 0; e < E; e++) { p[e] = expf(z[e] - m); sum += p[e]; }
            for (int e = 0; e < E; e++) p[e] /= sum;
            topk_scan(p, E, K, ix);
            for (int kk = 0; kk < K; kk++) wx[kk] = p[ix[kk]];
            if (norm_topk) {                       /* c/olmoe.c:681, no epsilon */
                float sm = 0.0f;
                for (int kk = 0; kk < K; kk++) sm += wx[kk];
                for (int kk = 0; kk < K; kk++) wx[kk] /= sm;
            }
        } else {
            for (int e = 0; e < E; e++) {
                p[e] = sigmoid_ref(z[e]);
                c[e] = p[e] + (bias ? bias[e] : 0.0f);
            }
            topk_scan(c, E, K, ix);
            for (int kk = 0; kk < K; kk++) wx[kk] = p[ix[kk]];
            if (mode == 1) {
                /* TOPP + norm_topk + routed_scale, backend_cuda.cu:2180-2193 */
                if (topp > 0.0f && topp < 1.0f) {
                    for (int a = 1; a < K; a++) {
                        int ii = ix[a]; float ww = wx[a]; int b = a - 1;
                        while (b >= 0 && wx[b] < ww) { wx[b + 1] = wx[b]; ix[b + 1] = ix[b]; b--; }
                        wx[b + 1] = ww; ix[b + 1] = ii;
                    }
                    float tot = 1e-20f, cum = 0.0f;
                    for (int kk = 0; kk < K; kk++) tot += wx[kk];
                    for (int kk = 0; kk < K; kk++) {
                        cum += wx[kk];
                        if (cum >= topp * tot) { ke = kk + 1; break; }
                    }
                }
                if (norm_topk) {
                    float sm = 0.0f;
                    for (int kk = 0; kk < ke; kk++) sm += wx[kk];
                    sm += 1e-20f;
                    for (int kk = 0; kk < ke; kk++) wx[kk] /= sm;
                }
                for (int kk = 0; kk < ke; kk++) wx[kk] *= routed_scale;
            } else {
                /* sigmoid-normalized, c/kimi_k3.c:1355-1370 */
                float sm = 0.0f;
                for (int kk = 0; kk < K; kk++) sm += wx[kk];
                for (int kk = 0; kk < K; kk++) wx[kk] /= (sm + 1e-20f);
                if (topp > 0.0f && topp < 1.0f) {
                    for (int a = 1; a < K; a++) {
                        int e2 = ix[a]; float w2 = wx[a]; int b = a - 1;
                        while (b >= 0 && wx[b] < w2) { ix[b + 1] = ix[b]; wx[b + 1] = wx[b]; b--; }
                        ix[b + 1] = e2; wx[b + 1] = w2;
                    }
                    float cum = 0.0f; int keep = K;
                    for (int kk = 0; kk < K; kk++) { cum += wx[kk]; if (cum >= topp) { keep = kk + 1; break; } }
                    if (keep < K) {
                        float s2 = 0.0f;
                        for (int kk = 0; kk < keep; kk++) s2 += wx[kk];
                        for (int kk = 0; kk < keep; kk++) wx[kk] /= (s2 + 1e-20f);
                        ke = keep;
                    }
                }
                if (routed_scale != 1.0f)
                    for (int kk = 0; kk < ke; kk++) wx[kk] *= routed_scale;
            }
        }
        keff[s] = ke;
    }
    free(p); free(c);
}

int cref_expert_union(const int *idx, const float *w, const int *keff, int S, int K,
                      int E, int *uniq, int *cnt, int *rows_of, int *slot_of,
                      float *wsel) {
    int *map = (int *)malloc((size_t)E * sizeof(int));
    for (int e = 0; e < E; e++) map[e] = -1;
    int nu = 0;
    for (int s = 0; s < S; s++)
        for (int kk = 0; kk < keff[s]; kk++) {
            int e = idx[(int64_t)s * K + kk];
            if (map[e] < 0) { map[e] = nu; uniq[nu] = e; cnt[nu] = 0; nu++; }
            int j = map[e], p = cnt[j]++;
            rows_of[(int64_t)j * S * K + p] = s;
            slot_of[(int64_t)j * S * K + p] = kk;
            wsel[(int64_t)j * S * K + p] = w[(int64_t)s * K + kk];
        }
    free(map);
    return nu;
}

void cref_swiglu(float *h, const float *g, const float *u, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float v = g[i];
        h[i] = (v / (1.0f + expf(-v))) * u[i];
    }
}

/* DeepSeek-V4 SwiGLU (coli_v4_swiglu, c/deepseek_v4.c:1434-1448): with
 * limit > 0 the gate is clamped from above and the up value to +-limit;
 * h = g * sigmoid(g) * u with the two-branch stable sigmoid of
 * c/deepseek_v4.c:1102-1109. */
static float sigmoid_stable_ref(float v) {
    if (v >= 0.0f) {
        float decay = expf(-v);
        return 1.0f / (1.0f + decay);
    }
    float growth = expf(v);
    return growth / (1.0f + growth);
}

void cref_swiglu_v4(float *h, const float *g, const float *u, size_t n, float limit) {
    for (size_t i = 0; i < n; i++) {
        float gv = g[i], uv = u[i];
        if (limit > 0.0f) {
            gv = fminf(gv, limit);
            uv = fmaxf(-limit, fminf(uv, limit));
        }
        h[i] = gv * sigmoid_stable_ref(gv) * uv;
    }
}

/* ------------------------------------------------------------------------
 * One MoE layer (composition; decode rows)
 * router GEMV (c/colibri.c:3978) -> route (above) -> per (token, slot):
 * gate, up (fmt kernel) -> silu*up -> down -> out[s] += w * y in slot order
 * (c/olmoe.c:687-698) -> shared expert added last (FASE E).
 * ------------------------------------------------------------------------ */
static void expert_gemv(int fmt, float *y, const float *x, const uint8_t *q,
                        const void *sc, int S, int I, int O, int gs) {
    if (fmt == 4) cref_matmul_i4_grouped(y, x, q, (const float *)sc, S, I, O, gs);
    else if (fmt == 7) cref_matmul_mxfp4(y, x, q, (const uint8_t *)sc, S, I, O);
    else cref_fp4_matmul_batch(y, q, (const uint8_t *)sc, O, I, x, S);
}

static void expert_forward(const CrefMoe *m, float *y, const float *xs,
                           const uint8_t *gq, const void *gsc,
                           const uint8_t *uq, const void *usc,
                           const uint8_t *dq, const void *dsc, float *g, float *u) {
    expert_gemv(m->fmt, g, xs, gq, gsc, 1, m->D, m->I, m->gs);
    expert_gemv(m->fmt, u, xs, uq, usc, 1, m->D, m->I, m->gs);
    cref_swiglu(g, g, u, (size_t)m->I);
    expert_gemv(m->fmt, y, g, dq, dsc, 1, m->I, m->D, m->gs);
}

int cref_moe_layer(const CrefMoe *m, const float *x, int S, float *out,
                   int *idx, float *w, int *keff) {
    int D = m->D, E = m->E, K = m->K;
    float *logits = (float *)malloc((size_t)S * E * sizeof(float));
    float *g = (float *)malloc((size_t)m->I * sizeof(float));
    float *u = (float *)malloc((size_t)m->I * sizeof(float));
    float *y = (float *)malloc((size_t)D * sizeof(float));
    if (!logits || !g || !u || !y) { free(logits); free(g); free(u); free(y); return -1; }
    cref_matmul_f32(logits, x, m->router_w, S, D, E);
    cref_route(logits, m->router_bias, S, E, K, m->route_mode, m->topp, m->norm_topk,
               m->routed_scale, idx, w, keff);
    for (int s = 0; s < S; s++) {
        const float *xs = x + (int64_t)s * D;
        float *os = out + (int64_t)s * D;
        for (int d = 0; d < D; d++) os[d] = 0.0f;
        for (int kk = 0; kk < keff[s]; kk++) {
            int e = idx[(int64_t)s * K + kk];
            expert_forward(m, y, xs, m->gq[e], m->gsc[e], m->uq[e], m->usc[e],
                           m->dq[e], m->dsc[e], g, u);
            float wk = w[(int64_t)s * K + kk];
            for (int d = 0; d < D; d++) os[d] = fmaf(wk, y[d], os[d]);
        }
        if (m->has_shared) {
            expert_forward(m, y, xs, m->sh_gq, m->sh_gsc, m->sh_uq, m->sh_usc,
                           m->sh_dq, m->sh_dsc, g, u);
            for (int d = 0; d < D; d++) os[d] += y[d];
        }
    }
    free(logits); free(g); free(u); free(y);
    return 0;
}
