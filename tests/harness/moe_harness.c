/* moe_harness.c -- the engine's MoE call sequence, in C, against libcoli_hip.so.
 *
 * Test infrastructure. This program binds the backend the way colibri's engine
 * does (the coli_cuda_* symbols of include/coli_backend_abi.h, linked
 * directly) and replays one decode MoE layer the way moe() drives it
 * (c/colibri.c:4467-4531 issue, 4782-4810 take; router c/colibri.c:5520-5541):
 *
 *   per token: x -> device (pipe_alloc / pipe_upload), pipe_router on the
 *              device -> idx / w / keff on the host
 *   host:      expert union in first-seen order (c/colibri.c:4146-4152);
 *              per expert the rows that selected it (<= 4, as prow[64][4])
 *   resident experts (even ids): rows packed contiguously in call order,
 *              expert_group_issue
 *   CPU share (odd ids, "not resident"): computed on the host while the GPU
 *              works, with the oracle's restatement of the reference kernels
 *   take:      expert_group_take, then the weighted scatter out[row] += w * y
 *              in slot order
 *
 * The layer output is compared with the oracle's cref_moe_layer on the same
 * inputs (route mode 1: sigmoid + bias, norm_topk, routed_scale, as
 * pipe_router computes it): indices must be bit-exact (inputs are redrawn
 * until the rank-TOPK / rank-TOPK+1 gap of the selection score is >= 1e-4), outputs
 * within 1e-3 of max(|ref|, 1e-2 * sum|terms|). Also checked: a second
 * take without an issue returns NULL; the sync expert_group call gives the
 * same bytes as issue/take.
 *
 * Usage: moe_harness FMT(4|7) S(1..4) SEED. Exit status 0 = pass.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "coli_backend_abi.h"
#include "cpu_ref.h"

#define HID 1024
#define INTER 512
#define NEXP 32
#define TOPK 4

static uint64_t g_rng;
static uint32_t rnd_u32(void) {
    g_rng = g_rng * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(g_rng >> 33);
}
static float rnd_unit(void) { return (rnd_u32() + 0.5f) / 2147483648.0f; }   /* (0, 1) */
static float rnd_normal(void) {
    float u = rnd_unit(), v = rnd_unit();
    return sqrtf(-2.0f * logf(u)) * cosf(6.2831853f * v);
}
static float bf16_round(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    memcpy(&f, &u, 4);
    return f;
}

typedef struct {
    uint8_t *q[3];     /* gate [INTER, HID/2], up [INTER, HID/2], down [HID, INTER/2] */
    float *sc[3];      /* f32 scales per 32 (fmt 4) or f32 powers of two (fmt 7) */
    uint8_t *e8[3];    /* fmt 7: e8m0 bytes (for the oracle) */
    ColiCudaTensor *t[3];
} Expert;

static void make_matrix(int fmt, int O, int In, uint8_t **q, float **sc, uint8_t **e8) {
    size_t nq = (size_t)O * In / 2, ns = (size_t)O * In / 32;
    *q = malloc(nq);
    *sc = malloc(ns * sizeof(float));
    *e8 = malloc(ns);
    for (size_t i = 0; i < nq; i++) (*q)[i] = (uint8_t)rnd_u32();
    for (size_t i = 0; i < ns; i++) {
        if (fmt == 4) {
            /* |N(0, 0.01)| on the grid m * 2^-16, m in 1..2047: exact in fp16 */
            float m = rintf(fabsf(rnd_normal()) * 0.01f * 65536.0f);
            (*sc)[i] = fminf(fmaxf(m, 1.0f), 2047.0f) / 65536.0f;
            (*e8)[i] = 0;
        } else {
            uint8_t e = (uint8_t)(119 + rnd_u32() % 5);
            uint32_t bits = (uint32_t)e << 23;
            (*e8)[i] = e;
            memcpy(&(*sc)[i], &bits, 4);
        }
    }
}

static void gemv_cpu(int fmt, float *y, const float *x, const Expert *e, int m, int S, int In, int O) {
    if (fmt == 4) cref_matmul_i4_grouped(y, x, e->q[m], e->sc[m], S, In, O, 32);
    else cref_matmul_mxfp4(y, x, e->q[m], e->e8[m], S, In, O);
}

/* sigmoid + bias selection scores of one row, sorted: gap between rank TOPK-1 and TOPK */
static double selection_gap(const float *logits, const float *bias) {
    double s[NEXP];
    for (int e = 0; e < NEXP; e++) s[e] = 1.0 / (1.0 + exp(-(double)logits[e])) + bias[e];
    for (int a = 0; a < NEXP; a++)
        for (int b = a + 1; b < NEXP; b++)
            if (s[b] > s[a]) { double t = s[a]; s[a] = s[b]; s[b] = t; }
    return s[TOPK - 1] - s[TOPK];
}

int main(int argc, char **argv) {
    if (argc < 4) {
        fprintf(stderr, "usage: %s FMT S SEED\n", argv[0]);
        return 2;
    }
    const int fmt = atoi(argv[1]), S = atoi(argv[2]);
    g_rng = strtoull(argv[3], NULL, 10) * 0x9E3779B97F4A7C15ull + 1;
    if ((fmt != 4 && fmt != 7) || S < 1 || S > 4) return 2;
    const float routed_scale = 2.5f;
    const int norm_topk = 1;
    printf("moe_harness fmt=%d S=%d HID=%d INTER=%d NEXP=%d TOPK=%d\n", fmt, S, HID, INTER, NEXP, TOPK);
    fflush(stdout);

    int dev = 0;
    if (!coli_cuda_init(&dev, 1)) { fprintf(stderr, "init failed\n"); return 1; }

    /* ---- synthetic layer: experts resident on the device ---- */
    Expert ex[NEXP];
    for (int e = 0; e < NEXP; e++) {
        const int shp[3][2] = {{INTER, HID}, {INTER, HID}, {HID, INTER}};
        for (int m = 0; m < 3; m++) {
            make_matrix(fmt, shp[m][0], shp[m][1], &ex[e].q[m], &ex[e].sc[m], &ex[e].e8[m]);
            ex[e].t[m] = NULL;
            if (!coli_cuda_tensor_upload_g(&ex[e].t[m], ex[e].q[m], ex[e].sc[m], fmt, shp[m][1], shp[m][0], dev,
                                           32)) {
                fprintf(stderr, "upload failed (expert %d, matrix %d)\n", e, m);
                return 1;
            }
        }
    }
    float *rw = malloc((size_t)NEXP * HID * sizeof(float)), rb[NEXP];
    for (int i = 0; i < NEXP * HID; i++) rw[i] = rnd_normal() * 0.02f;
    for (int e = 0; e < NEXP; e++) rb[e] = rnd_normal() * 0.01f;
    void *rw_dev = coli_cuda_pipe_alloc(dev, (size_t)NEXP * HID * 4), *rb_dev = coli_cuda_pipe_alloc(dev, NEXP * 4);
    void *x_dev = coli_cuda_pipe_alloc(dev, (size_t)HID * 4);
    if (!rw_dev || !rb_dev || !x_dev || !coli_cuda_pipe_upload(dev, rw_dev, rw, (size_t)NEXP * HID * 4) ||
        !coli_cuda_pipe_upload(dev, rb_dev, rb, NEXP * 4)) {
        fprintf(stderr, "router upload failed\n");
        return 1;
    }

    /* ---- tokens, redrawn until the selection gap is >= 1e-4 ---- */
    float *x = malloc((size_t)S * HID * sizeof(float)), logits[NEXP];
    for (int s = 0; s < S; s++) {
        for (int tries = 0;; tries++) {
            for (int d = 0; d < HID; d++) x[(size_t)s * HID + d] = bf16_round(rnd_normal());
            cref_matmul_f32(logits, x + (size_t)s * HID, rw, 1, HID, NEXP);
            if (selection_gap(logits, rb) >= 1e-4) break;
            if (tries > 1000) return 1;
        }
    }

    /* ---- route each token on the device (c/colibri.c:5520-5541) ---- */
    int idx[4 * TOPK], keff[4];
    float w[4 * TOPK];
    for (int s = 0; s < S; s++) {
        if (!coli_cuda_pipe_upload(dev, x_dev, x + (size_t)s * HID, (size_t)HID * 4) ||
            !coli_cuda_pipe_router(dev, x_dev, rw_dev, rb_dev, HID, NEXP, TOPK, 0.0f, norm_topk, routed_scale, idx + s * TOPK,
                                   w + s * TOPK, keff + s)) {
            fprintf(stderr, "pipe_router failed\n");
            return 1;
        }
    }

    /* ---- union in first-seen order, rows per expert ---- */
    int uniq[NEXP], nu = 0, nrow[NEXP] = {0}, prow[NEXP][4];
    for (int s = 0; s < S; s++)
        for (int kk = 0; kk < keff[s]; kk++) {
            int e = idx[s * TOPK + kk], u = 0;
            while (u < nu && uniq[u] != e) u++;
            if (u == nu) uniq[nu++] = e;
            prow[u][nrow[u]] = s;
            nrow[u]++;
        }

    /* ---- pack the resident (even) experts and issue ---- */
    ColiCudaTensor *gg[NEXP], *uu[NEXP], *dd[NEXP];
    int grows[NEXP], which[NEXP], nc = 0, total = 0;
    float *gx = malloc((size_t)S * TOPK * HID * sizeof(float));
    for (int u = 0; u < nu; u++) {
        if (uniq[u] % 2) continue;
        const Expert *e = &ex[uniq[u]];
        gg[nc] = e->t[0];
        uu[nc] = e->t[1];
        dd[nc] = e->t[2];
        grows[nc] = nrow[u];
        which[nc] = u;
        for (int r = 0; r < nrow[u]; r++) memcpy(gx + (size_t)(total + r) * HID, x + (size_t)prow[u][r] * HID, HID * 4);
        total += nrow[u];
        nc++;
    }
    float *out = calloc((size_t)S * HID, sizeof(float));
    float *hg = malloc(INTER * 4), *hu = malloc(INTER * 4);
    /* issue is decode-only (<= 8 rows per device, c/backend_cuda.cu:1692): a
     * larger pack takes the engine's other route, one sync group call after
     * the CPU share */
    const int use_issue = nc > 0 && total <= 8;
    int issued = use_issue && coli_cuda_expert_group_issue(gg, uu, dd, grows, nc, gx);
    if (use_issue && !issued) {
        fprintf(stderr, "expert_group_issue failed (nc=%d rows=%d)\n", nc, total);
        return 1;
    }
    if (nc > 0 && !use_issue && coli_cuda_expert_group_issue(gg, uu, dd, grows, nc, gx)) {
        fprintf(stderr, "expert_group_issue accepted %d rows (decode-only: <= 8)\n", total);
        return 1;
    }
    /* ---- CPU share: the odd experts, while the GPU works ---- */
    float *ycpu[NEXP] = {0};
    for (int u = 0; u < nu; u++) {
        if (!(uniq[u] % 2)) continue;
        const Expert *e = &ex[uniq[u]];
        ycpu[u] = malloc((size_t)nrow[u] * HID * sizeof(float));
        for (int r = 0; r < nrow[u]; r++) {
            const float *xs = x + (size_t)prow[u][r] * HID;
            gemv_cpu(fmt, hg, xs, e, 0, 1, HID, INTER);
            gemv_cpu(fmt, hu, xs, e, 1, 1, HID, INTER);
            cref_swiglu(hg, hg, hu, INTER);
            gemv_cpu(fmt, ycpu[u] + (size_t)r * HID, hg, e, 2, 1, INTER, HID);
        }
    }
    /* ---- take, then the weighted scatter in slot (union) order ---- */
    float *ygpu = NULL;
    if (nc > 0 && !use_issue) {
        ygpu = malloc((size_t)total * HID * sizeof(float));
        if (!coli_cuda_expert_group(gg, uu, dd, grows, nc, ygpu, gx)) {
            fprintf(stderr, "expert_group failed (nc=%d rows=%d)\n", nc, total);
            return 1;
        }
    }
    if (issued) {
        const float *hyp = coli_cuda_expert_group_take(dev);
        if (!hyp) {
            fprintf(stderr, "expert_group_take returned NULL\n");
            return 1;
        }
        ygpu = malloc((size_t)total * HID * sizeof(float));
        memcpy(ygpu, hyp, (size_t)total * HID * sizeof(float));
        if (coli_cuda_expert_group_take(dev) != NULL) {
            fprintf(stderr, "second take without an issue did not return NULL\n");
            return 1;
        }
        float *ysync = malloc((size_t)total * HID * sizeof(float));
        if (!coli_cuda_expert_group(gg, uu, dd, grows, nc, ysync, gx) ||
            memcmp(ysync, ygpu, (size_t)total * HID * sizeof(float)) != 0) {
            fprintf(stderr, "sync expert_group differs from issue/take\n");
            return 1;
        }
        free(ysync);
    }
    int gpu_slot[NEXP];
    for (int u = 0; u < nu; u++) gpu_slot[u] = -1;
    for (int c = 0, off = 0; c < nc; c++) {
        gpu_slot[which[c]] = off;
        off += grows[c];
    }
    /* per token, experts in its slot order (as the oracle adds them) */
    for (int s = 0; s < S; s++)
        for (int kk = 0; kk < keff[s]; kk++) {
            int e = idx[s * TOPK + kk], u = 0;
            while (uniq[u] != e) u++;
            int r = 0;
            while (prow[u][r] != s) r++;
            const float *yr = gpu_slot[u] >= 0 ? ygpu + (size_t)(gpu_slot[u] + r) * HID : ycpu[u] + (size_t)r * HID;
            const float wk = w[s * TOPK + kk];
            for (int d = 0; d < HID; d++) out[(size_t)s * HID + d] = fmaf(wk, yr[d], out[(size_t)s * HID + d]);
        }

    /* ---- oracle ---- */
    const uint8_t *oq[3][NEXP];
    const void *os[3][NEXP];
    for (int e = 0; e < NEXP; e++)
        for (int m = 0; m < 3; m++) {
            oq[m][e] = ex[e].q[m];
            os[m][e] = fmt == 4 ? (const void *)ex[e].sc[m] : (const void *)ex[e].e8[m];
        }
    CrefMoe cm;
    memset(&cm, 0, sizeof(cm));
    cm.fmt = fmt; cm.D = HID; cm.I = INTER; cm.E = NEXP; cm.K = TOPK; cm.gs = 32;
    cm.route_mode = 1; cm.norm_topk = norm_topk; cm.topp = 0.0f; cm.routed_scale = routed_scale;
    cm.router_w = rw; cm.router_bias = rb;
    cm.gq = oq[0]; cm.gsc = os[0]; cm.uq = oq[1]; cm.usc = os[1]; cm.dq = oq[2]; cm.dsc = os[2];
    float *ref = malloc((size_t)S * HID * sizeof(float));
    int ridx[4 * TOPK], rkeff[4];
    float rwt[4 * TOPK];
    if (cref_moe_layer(&cm, x, S, ref, ridx, rwt, rkeff) != 0) return 1;
    int bad_idx = 0;
    for (int s = 0; s < S; s++) {
        bad_idx |= keff[s] != rkeff[s];
        for (int kk = 0; kk < TOPK; kk++) bad_idx |= idx[s * TOPK + kk] != ridx[s * TOPK + kk];
        for (int kk = 0; kk < keff[s]; kk++)
            if (fabsf(w[s * TOPK + kk] - rwt[s * TOPK + kk]) > 1e-5f * fabsf(rwt[s * TOPK + kk])) bad_idx |= 2;
    }
    /* magnitude: sum over the token's experts of |w| * |h| . |W_down| bounds the terms */
    double worst = 0.0;
    for (int s = 0; s < S; s++) {
        double *mag = calloc(HID, sizeof(double));
        for (int kk = 0; kk < rkeff[s]; kk++) {
            const Expert *e = &ex[ridx[s * TOPK + kk]];
            gemv_cpu(fmt, hg, x + (size_t)s * HID, e, 0, 1, HID, INTER);
            gemv_cpu(fmt, hu, x + (size_t)s * HID, e, 1, 1, HID, INTER);
            cref_swiglu(hg, hg, hu, INTER);
            for (int o = 0; o < HID; o++) {
                double acc = 0;
                for (int i = 0; i < INTER; i++) {
                    uint8_t b = e->q[2][(size_t)o * (INTER / 2) + i / 2];
                    int nib = (i & 1) ? b >> 4 : b & 15;
                    double wv;
                    if (fmt == 4) wv = (nib - 8) * (double)e->sc[2][(size_t)o * (INTER / 32) + i / 32];
                    else wv = cref_e2m1_decode((uint8_t)nib) * (double)e->sc[2][(size_t)o * (INTER / 32) + i / 32];
                    acc += fabs(wv * hg[i]);
                }
                mag[o] += fabs(rwt[s * TOPK + kk]) * acc;
            }
        }
        for (int d = 0; d < HID; d++) {
            double r = ref[(size_t)s * HID + d], g = out[(size_t)s * HID + d];
            double den = fmax(fabs(r), 1e-2 * mag[d]);
            double err = den > 0 ? fabs(g - r) / den : fabs(g - r);
            if (err > worst) worst = err;
        }
        free(mag);
    }
    printf("union %d experts (%d on the GPU, %d rows, %s), routing %s, max rel err %.3e\n", nu, nc, total,
           use_issue ? "issue/take" : "sync group", bad_idx ? "DIFFERS" : "bit-exact", worst);
    coli_cuda_shutdown();
    if (bad_idx || !(worst <= 1e-3)) {
        printf("FAIL\n");
        return 1;
    }
    printf("PASS\n");
    return 0;
}
