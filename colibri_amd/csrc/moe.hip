// moe.hip -- one device-resident MoE layer for decode / verification rows.
//
//   x [S, D] --router GEMV--> logits [S, E] (column-chunk partials) --top-K--> idx, w, keff
//            --union (first-seen order)--> per-expert row lists + descriptors
//            --dual GEMV (gate/up + SwiGLU)--> h [P, RS, I]
//            --down GEMV--> y [P, RS, D]
//            --combine (slot order, + shared)--> out [S, D]
//
// The composition follows the reference layer: router and selection of
// c/colibri.c:3978-4126 / c/olmoe.c:645-681 / c/kimi_k3.c:1331-1370, the union
// of c/colibri.c:4146-4152 with per-expert position lists as in
// c/kimi_k3.c:1386-1410, the expert MLP with the fused silu*up epilogue of
// c/backend_cuda.cu:618-624, the weighted scatter out[s] += w * y in slot
// order (c/olmoe.c:694-697), and the shared expert added after the routed sum
// (FASE E, c/colibri.c:4940-5002). Every stage is stream-ordered on the
// device; nothing returns to the host between stages, and no stage allocates
// once the layer has run at a given S.
#include "coli_hip_host.h"

#include "coli_backend_abi.h"
#include "coli_hip_ext.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

struct ColiHipMoe {
    int device;
    ColiHipMoeConfig cfg;
    int kind;                 // storage kind shared by every expert matrix
    int RS;                   // row slots per problem (ceil16(S) of the largest S seen)
    int S_cap;
    float *rw = nullptr, *rb = nullptr;
    ColiProb *tab = nullptr;  // [E (+1 shared)][2]: dual template, down template
    // per-forward state (device)
    float *logits = nullptr, *wsel = nullptr, *h = nullptr, *y = nullptr;
    int *idx = nullptr, *keff = nullptr, *state = nullptr;   // state: nprob, nhrows, nu
    int *uniq = nullptr, *xrows = nullptr, *hrows = nullptr, *slotrow = nullptr;
    ColiProb *pdual = nullptr, *pdown = nullptr;
    size_t h_cap = 0, y_cap = 0;
};

// ---------------------------------------------------------------------------
// union + descriptor build, one 256-thread block, all threads in parallel.
// Selection i = (t, kk) in row-major order is live when kk < keff[t] and its
// expert is in range. The union lists the experts in first-seen order: a
// live selection opens a new slot when no earlier live selection names the
// same expert, and its slot number is the count of such openings before it.
// Within an expert, rows keep their selection order (pos = earlier live
// selections of the same expert), so every list is the reference's.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void coli_moe_union(const int *__restrict__ idx, const int *__restrict__ keff,
                                                      int S, int K, int E, int has_shared, int RS,
                                                      const ColiProb *__restrict__ tab, ColiProb *__restrict__ pdual,
                                                      ColiProb *__restrict__ pdown, int *__restrict__ uniq,
                                                      int *__restrict__ xrows, int *__restrict__ hrows,
                                                      int *__restrict__ slotrow, int *__restrict__ state) {
    // sel [n4] | open [n4 + 1] | uq [n4 + 1] | cnt [n4 + 1] | map [E]; n4 = n rounded up to 4
    // (int4 scans); open[] later holds the per-slot counts, shared expert included
    extern __shared__ int sm[];
    const int n = S * K, n4 = (n + 3) & ~3;
    int *sel = sm, *open = sel + n4, *uq = open + n4 + 1, *cnt = uq + n4 + 1, *map = cnt + n4 + 1;
    __shared__ int s_nu;
    for (int i = threadIdx.x; i < n4; i += blockDim.x) {
        int e = -1;
        if (i < n) {
            const int t = i / K, kk = i - t * K;
            const int v = idx[i];
            if (kk < keff[t] && v >= 0 && v < E) e = v;
        }
        sel[i] = e;
    }
    __syncthreads();
    // pass 1: earlier and total occurrences of this selection's expert
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int e = sel[i];
        int before = 0, total = 0;
        if (e >= 0) {
            for (int j = 0; j < n4; j += 4) {
                const int4 v = *(const int4 *)(sel + j);
                const int m0 = v.x == e, m1 = v.y == e, m2 = v.z == e, m3 = v.w == e;
                total += m0 + m1 + m2 + m3;
                before += (j < i ? m0 : 0) + (j + 1 < i ? m1 : 0) + (j + 2 < i ? m2 : 0) + (j + 3 < i ? m3 : 0);
            }
        }
        open[i] = e >= 0 && before == 0;
        cnt[i] = total;       // kept at the opening index until the slot is known
        slotrow[i] = before;  // position inside the expert's list, finished below
    }
    for (int i = n + threadIdx.x; i < n4; i += blockDim.x) open[i] = 0;
    __syncthreads();
    // pass 2: slot = openings before this one
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        if (!open[i]) continue;
        int slot = 0;
        for (int j = 0; j < n4; j += 4) {
            const int4 v = *(const int4 *)(open + j);
            slot += (j < i ? v.x : 0) + (j + 1 < i ? v.y : 0) + (j + 2 < i ? v.z : 0) + (j + 3 < i ? v.w : 0);
        }
        map[sel[i]] = slot;
    }
    if (threadIdx.x < 64) {   // number of openings, one wave
        int c = 0;
        for (int j = threadIdx.x; j < n; j += 64) c += open[j];
#pragma unroll
        for (int off = 32; off; off >>= 1) c += __shfl_xor(c, off);
        if (threadIdx.x == 0) s_nu = c;
    }
    __syncthreads();
    const int nu = s_nu;
    int *cslot = open;   // open[] is not read past the barrier above: reuse it for per-slot counts
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int e = sel[i];
        if (e < 0) continue;
        const int slot = map[e], before = slotrow[i];
        if (before == 0) {
            uq[slot] = e;
            cslot[slot] = cnt[i];
        }
        const int row = slot * RS + before;
        xrows[row] = i / K;
        slotrow[i] = row;
    }
    int np = nu;
    if (has_shared) {
        if (threadIdx.x == 0) {
            uq[nu] = E;            // the shared expert sits at table row E
            cslot[nu] = S;
        }
        np++;
        for (int t = threadIdx.x; t < S; t += blockDim.x) xrows[nu * RS + t] = t;
    }
    if (threadIdx.x == 0) {
        state[0] = np;
        state[1] = np * RS;
        state[2] = nu;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < np; j += blockDim.x) {
        const int e = uq[j];
        if (j < nu) uniq[j] = e;
        ColiProb d = tab[2 * e], dn = tab[2 * e + 1];
        d.nrows = dn.nrows = cslot[j];
        d.xrow_off = dn.xrow_off = j * RS;
        d.out_row0 = dn.out_row0 = j * RS;
        pdual[j] = d;
        pdown[j] = dn;
    }
    for (int r = threadIdx.x; r < np * RS; r += blockDim.x) {
        const int j = r / RS, p = r - j * RS;
        hrows[r] = p < cslot[j] ? r : -1;
    }
}

// out[t, d] = sum_{kk < keff[t]} w[t, kk] * y[slotrow[t, kk], d]  (+ y[shared row])
__global__ void coli_moe_combine(const float *__restrict__ y, int D, const float *__restrict__ w,
                                 const int *__restrict__ keff, const int *__restrict__ slotrow, int K,
                                 const int *__restrict__ state, int has_shared, int RS, float *__restrict__ out) {
    int t = blockIdx.y, d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    float acc = 0.0f;
    int ke = keff[t];
    for (int kk = 0; kk < ke; kk++) acc = fmaf(w[t * K + kk], y[(size_t)slotrow[t * K + kk] * D + d], acc);
    if (has_shared) acc += y[((size_t)(state[0] - 1) * RS + t) * D + d];
    out[(size_t)t * D + d] = acc;
}

extern "C" void coli_hip_moe_free(ColiHipMoe *m) {
    if (!m) return;
    DevCtx *ctx = find_ctx(m->device);
    if (ctx) {
        select_ctx(ctx);
        (void)hipStreamSynchronize(ctx->stream);
    }
    void *bufs[] = {m->rw, m->rb, m->tab, m->logits, m->wsel, m->h, m->y, m->idx, m->keff, m->state,
                    m->uniq, m->xrows, m->hrows, m->slotrow, m->pdual, m->pdown};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    delete m;
}

extern "C" int coli_hip_moe_create(ColiHipMoe **out, int device, const ColiHipMoeConfig *cfg, const float *router_w,
                                   const float *router_bias, ColiCudaTensor *const *gates,
                                   ColiCudaTensor *const *ups, ColiCudaTensor *const *downs,
                                   ColiCudaTensor *sg, ColiCudaTensor *su, ColiCudaTensor *sd) {
    if (!out || !cfg || !router_w || !gates || !ups || !downs) return 0;
    const ColiHipMoeConfig c = *cfg;
    if (c.D < 1 || c.I < 1 || c.E < 1 || c.E > 1024 || c.K < 1 || c.K > 64 || c.K > c.E || c.route_mode < 0 ||
        c.route_mode > 2)
        return 0;
    if (c.has_shared && (!sg || !su || !sd)) return 0;
    DevCtx *ctx = find_ctx(device);
    if (!select_ctx(ctx)) return 0;
    int kind = gates[0] ? gates[0]->kind : -1;
    if (kind < 0 || kind == COLI_KIND_GENERIC) return 0;
    int n = c.E + (c.has_shared ? 1 : 0);
    std::vector<ColiProb> tab(2 * (c.E + 1));
    for (int e = 0; e < n; e++) {
        ColiCudaTensor *g = e < c.E ? gates[e] : sg, *u = e < c.E ? ups[e] : su, *d = e < c.E ? downs[e] : sd;
        if (!g || !u || !d || g->device != device || u->device != device || d->device != device ||
            g->kind != kind || u->kind != kind || d->kind != kind || g->I != c.D || u->I != c.D || g->O != c.I ||
            u->O != c.I || d->I != c.I || d->O != c.D)
            return 0;
        tab[2 * e] = {g->w, g->sc, u->w, u->sc, 0, 0, 0, 0};
        tab[2 * e + 1] = {d->w, d->sc, nullptr, nullptr, 0, 0, 0, 0};
    }
    ColiHipMoe *m = new ColiHipMoe();
    m->device = device;
    m->cfg = c;
    m->kind = kind;
    m->RS = 0;
    m->S_cap = 0;
    size_t rwb = (size_t)c.E * c.D * sizeof(float);
    int ok = hip_ok(hipMalloc((void **)&m->rw, rwb), "router weights") &&
             hip_ok(hipMemcpy(m->rw, router_w, rwb, hipMemcpyHostToDevice), "router weights upload") &&
             hip_ok(hipMalloc((void **)&m->tab, tab.size() * sizeof(ColiProb)), "expert table") &&
             hip_ok(hipMemcpy(m->tab, tab.data(), tab.size() * sizeof(ColiProb), hipMemcpyHostToDevice),
                    "expert table upload");
    if (ok && router_bias)
        ok = hip_ok(hipMalloc((void **)&m->rb, (size_t)c.E * sizeof(float)), "router bias") &&
             hip_ok(hipMemcpy(m->rb, router_bias, (size_t)c.E * sizeof(float), hipMemcpyHostToDevice),
                    "router bias upload");
    if (!ok) {
        coli_hip_moe_free(m);
        return 0;
    }
    *out = m;
    return 1;
}

// Per-forward buffers for up to S rows (allocated once per growth of S).
static int moe_reserve(DevCtx *ctx, ColiHipMoe *m, int S) {
    if (S <= m->S_cap) return 1;
    if (!hip_ok(hipStreamSynchronize(ctx->stream), "moe reserve sync")) return 0;
    const ColiHipMoeConfig &c = m->cfg;
    int RS = (S + 15) / 16 * 16;
    int P = std::min(c.E, S * c.K) + (c.has_shared ? 1 : 0);
    void **bufs[] = {(void **)&m->logits, (void **)&m->wsel, (void **)&m->h, (void **)&m->y, (void **)&m->idx,
                     (void **)&m->keff, (void **)&m->state, (void **)&m->uniq, (void **)&m->xrows,
                     (void **)&m->hrows, (void **)&m->slotrow, (void **)&m->pdual, (void **)&m->pdown};
    for (void **b : bufs)
        if (*b) {
            (void)hipFree(*b);
            *b = nullptr;
        }
    size_t sizes[] = {(size_t)coli_router_chunks(c.D) * S * c.E * 4, (size_t)S * c.K * 4, (size_t)P * RS * c.I * 4, (size_t)P * RS * c.D * 4,
                      (size_t)S * c.K * 4, (size_t)S * 4, 16, (size_t)c.E * 4, (size_t)P * RS * 4,
                      (size_t)P * RS * 4, (size_t)S * c.K * 4, (size_t)P * sizeof(ColiProb),
                      (size_t)P * sizeof(ColiProb)};
    for (int i = 0; i < 13; i++)
        if (!hip_ok(hipMalloc(bufs[i], sizes[i]), "moe buffers")) return 0;
    m->RS = RS;
    m->S_cap = S;
    return 1;
}

extern "C" int coli_hip_moe_forward_dev(ColiHipMoe *m, const float *x_dev, float *out_dev, int S) {
    if (fault_injected()) return 0;
    if (!m || !x_dev || !out_dev || S < 1 || S > 64) return 0;
    DevCtx *ctx = find_ctx(m->device);
    if (!select_ctx(ctx) || !moe_reserve(ctx, m, S)) return 0;
    const ColiHipMoeConfig &c = m->cfg;
    const int RS = m->RS;
    const int P = std::min(c.E, S * c.K) + (c.has_shared ? 1 : 0);
    const int ord = m->kind == COLI_KIND_FP4 ? 1 : 0;
    hipStream_t st = ctx->stream;
    const int nq_d = (c.D + 127) / 128, nq_i = (c.I + 127) / 128;
    // make sure every scratch the kernels touch exists before the first launch
    {
        GemvLaunchPlan a = plan_gemv(ctx, P, (S + 15) / 16, (c.I + 15) / 16, nq_d, true, S);
        GemvLaunchPlan b = plan_gemv(ctx, P, (S + 15) / 16, (c.D + 15) / 16, nq_i, false, S);
        size_t ia = (size_t)P * ((S + 15) / 16) * a.rbpp, ib = (size_t)P * ((S + 15) / 16) * b.rbpp;
        size_t pa = a.splits > 1 ? ia * a.splits * a.R * 4 * 64 * 4 : 0;
        size_t pb = b.splits > 1 ? ib * b.splits * b.R * 4 * 64 * 4 : 0;
        size_t ngp_d = (size_t)nq_d * 4, ngp_i = (size_t)nq_i * 4;
        FragSet &fx = ctx->frag[ord], &fh = ctx->frag[2 + ord];
        if (!reserve(ctx, &ctx->partial, std::max<size_t>(std::max(pa, pb), 256), 0) ||
            !reserve(ctx, &fx.hi, (size_t)S * ngp_d * 64, 0) || !reserve(ctx, &fx.lo, (size_t)S * ngp_d * 64, 0) ||
            !reserve(ctx, &fx.exp, (size_t)S * 4, 0) || !reserve(ctx, &fh.hi, (size_t)P * RS * ngp_i * 64, 0) ||
            !reserve(ctx, &fh.lo, (size_t)P * RS * ngp_i * 64, 0) || !reserve(ctx, &fh.exp, (size_t)P * RS * 4, 0))
            return 0;
    }
    int *flags = (int *)ctx->flags.p;
    FragSet &fx = ctx->frag[ord], &fh = ctx->frag[2 + ord];
    // 1. activation fragments, 2-3. router
    fx.gen = fx.gen == 0x7fffffff ? 1 : fx.gen + 1;
    if (fx.gen == 1 && !hip_ok(coli_launch_zero_i32(flags + ord, 1, st), "moe flag")) return 0;
    if (!hip_ok(coli_launch_prep_frag(x_dev, c.D, nullptr, nullptr, S, c.D, nq_d * 4, !ord, (_Float16 *)fx.hi.p,
                                      (_Float16 *)fx.lo.p, (int *)fx.exp.p, flags + ord, fx.gen, ctx->zeros.p, st),
                "moe x fragments") ||
        !hip_ok(coli_launch_router_logits(x_dev, S, m->rw, c.D, c.E, m->logits, st), "moe router logits") ||
        !hip_ok(coli_launch_router_select(m->logits, coli_router_chunks(c.D), m->rb, S, c.E, c.K, c.route_mode, c.topp,
                                          c.norm_topk,
                                          c.routed_scale, m->idx, m->wsel, m->keff, st),
                "moe router select"))
        return 0;
    // 4. union
    hipLaunchKernelGGL(coli_moe_union, dim3(1), dim3(256), (size_t)(c.E + 4 * ((S * c.K + 3) & ~3) + 3) * sizeof(int), st, m->idx, m->keff, S, c.K,
                       c.E, c.has_shared, RS, m->tab, m->pdual, m->pdown, m->uniq, m->xrows, m->hrows, m->slotrow,
                       m->state);
    if (!hip_ok(hipGetLastError(), "moe union")) return 0;
    // 5. gate/up + SwiGLU over the union
    ColiGemvArgs a;
    GemvLaunchPlan pl = plan_gemv(ctx, P, (S + 15) / 16, (c.I + 15) / 16, nq_d, true, S);
    a.prob = m->pdual;
    a.nprob_dev = m->state;
    a.nprob = P;
    a.nrt = (c.I + 15) / 16;
    a.nq = nq_d;
    a.O = c.I;
    a.n_bt = (S + 15) / 16;
    a.rb_per_prob = pl.rbpp;
    a.splits = pl.splits;
    a.qps = pl.qps;
    a.xrows = m->xrows;
    a.xhi = (const _Float16 *)fx.hi.p;
    a.xlo = (const _Float16 *)fx.lo.p;
    a.xstride = nq_d * 128;
    a.xexp = (const int *)fx.exp.p;
    a.haslo = flags + ord;
    a.lo_gen = fx.gen;
    a.zero = (const _Float16 *)ctx->zeros.p;
    a.out = m->h;
    a.ldo = c.I;
    a.partial = (float *)ctx->partial.p;
    if (!hip_ok(coli_launch_gemv(m->kind, &a, pl.R, 1, pl.W, S, st), "moe dual")) return 0;
    // 6. hidden fragments (valid slots only)
    fh.gen = fh.gen == 0x7fffffff ? 1 : fh.gen + 1;
    if (fh.gen == 1 && !hip_ok(coli_launch_zero_i32(flags + 2 + ord, 1, st), "moe flag")) return 0;
    if (!hip_ok(coli_launch_prep_frag(m->h, c.I, m->hrows, m->state + 1, P * RS, c.I, nq_i * 4, !ord,
                                      (_Float16 *)fh.hi.p, (_Float16 *)fh.lo.p, (int *)fh.exp.p, flags + 2 + ord,
                                      fh.gen, ctx->zeros.p, st),
                "moe hidden fragments"))
        return 0;
    // 7. down
    pl = plan_gemv(ctx, P, (S + 15) / 16, (c.D + 15) / 16, nq_i, false, S);
    a.prob = m->pdown;
    a.nrt = (c.D + 15) / 16;
    a.nq = nq_i;
    a.O = c.D;
    a.rb_per_prob = pl.rbpp;
    a.splits = pl.splits;
    a.qps = pl.qps;
    a.xrows = nullptr;   // hidden rows are fragment rows
    a.xhi = (const _Float16 *)fh.hi.p;
    a.xlo = (const _Float16 *)fh.lo.p;
    a.xstride = nq_i * 128;
    a.xexp = (const int *)fh.exp.p;
    a.haslo = flags + 2 + ord;
    a.lo_gen = fh.gen;
    a.out = m->y;
    a.ldo = c.D;
    if (!hip_ok(coli_launch_gemv(m->kind, &a, pl.R, 0, pl.W, S, st), "moe down")) return 0;
    // 8. combine
    hipLaunchKernelGGL(coli_moe_combine, dim3((c.D + 255) / 256, S), dim3(256), 0, st, m->y, c.D, m->wsel, m->keff,
                       m->slotrow, c.K, m->state, c.has_shared, RS, out_dev);
    return hip_ok(hipGetLastError(), "moe combine");
}

extern "C" int coli_hip_moe_forward(ColiHipMoe *m, const float *x, float *out, int S, int *idx, float *w,
                                    int *keff) {
    if (!m || !x || !out || S < 1 || S > 64) return 0;
    DevCtx *ctx = find_ctx(m->device);
    if (!select_ctx(ctx)) return 0;
    const ColiHipMoeConfig &c = m->cfg;
    size_t xb = (size_t)S * c.D * sizeof(float);
    if (!reserve(ctx, &ctx->x, xb, 0) || !reserve(ctx, &ctx->y, xb, 0) ||
        !hip_ok(hipStreamSynchronize(ctx->stream), "moe staging") ||
        !hip_ok(hipMemcpyAsync(ctx->x.p, x, xb, hipMemcpyHostToDevice, ctx->stream), "moe input upload") ||
        !coli_hip_moe_forward_dev(m, (const float *)ctx->x.p, (float *)ctx->y.p, S) ||
        !hip_ok(hipMemcpyAsync(out, ctx->y.p, xb, hipMemcpyDeviceToHost, ctx->stream), "moe output download"))
        return 0;
    if (idx && !hip_ok(hipMemcpyAsync(idx, m->idx, (size_t)S * c.K * 4, hipMemcpyDeviceToHost, ctx->stream), "idx"))
        return 0;
    if (w && !hip_ok(hipMemcpyAsync(w, m->wsel, (size_t)S * c.K * 4, hipMemcpyDeviceToHost, ctx->stream), "w"))
        return 0;
    if (keff && !hip_ok(hipMemcpyAsync(keff, m->keff, (size_t)S * 4, hipMemcpyDeviceToHost, ctx->stream), "keff"))
        return 0;
    return hip_ok(hipStreamSynchronize(ctx->stream), "moe synchronize");
}

extern "C" int coli_hip_moe_last_union(ColiHipMoe *m, int *nu, int *uniq) {
    if (!m || !nu || !m->state) return 0;
    DevCtx *ctx = find_ctx(m->device);
    if (!select_ctx(ctx) || !hip_ok(hipStreamSynchronize(ctx->stream), "union sync")) return 0;
    int st[3];
    if (!hip_ok(hipMemcpy(st, m->state, sizeof(st), hipMemcpyDeviceToHost), "union state")) return 0;
    *nu = st[2];
    if (uniq && st[2] > 0 &&
        !hip_ok(hipMemcpy(uniq, m->uniq, (size_t)st[2] * sizeof(int), hipMemcpyDeviceToHost), "union ids"))
        return 0;
    return 1;
}
