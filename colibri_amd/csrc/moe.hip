// moe.hip -- one device-resident MoE layer for decode, verification and
// prefill rows.
//
//   x [S, D] --router GEMV--> logits (column-chunk partials) --top-K--> idx, w, keff
//            --union (first-seen order)--> per-expert row lists, packed
//            --gate/up + SwiGLU--> h [S*K (+S), I]
//            --down--> y [S*K (+S), D]
//            --combine (slot order, + shared)--> out [S, D]
//
// The composition follows the reference layer: router and selection of
// c/colibri.c:3978-4126 / c/olmoe.c:645-681 / c/kimi_k3.c:1331-1370, the union
// of c/colibri.c:4146-4152 with per-expert position lists as in
// c/kimi_k3.c:1386-1410, the expert MLP with the fused silu*up epilogue of
// c/backend_cuda.cu:618-624, the weighted scatter out[s] += w * y in slot
// order (c/olmoe.c:694-697), and the shared expert added after the routed sum
// (FASE E, c/colibri.c:4940-5002). Expert row lists are packed back to back
// (an expert's rows start at the sum of the earlier experts' counts), so h
// and y hold S*K (+S) rows whatever the batch. Up to COLI_GEMM_MIN_ROWS rows
// the experts run the tiled GEMV; beyond, the grouped GEMM over a device-built
// list of 64-row tiles. Every stage is stream-ordered on the device; nothing
// returns to the host between stages, and no stage allocates once the layer
// has run at a given S.
#include "coli_hip_host.h"
#include "coli_route.h"

#include "coli_backend_abi.h"
#include "coli_hip_ext.h"

#include <algorithm>
#include <type_traits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define COLI_MOE_MAX_ROWS 2048
#define COLI_MOE_MAX_SEL 16384

struct ColiHipMoe {
    int device;
    ColiHipMoeConfig cfg;
    int kind;                 // storage kind shared by every expert matrix
    std::vector<const ColiCudaTensor *> mats;   // every expert matrix (e8_fold is read per forward)
    int S_cap;
    float *rw = nullptr, *rb = nullptr;
    ColiProb *tab = nullptr;  // [E (+1 shared)][2]: dual template, down template
    // per-forward state (device)
    float *logits = nullptr, *wsel = nullptr, *h = nullptr, *y = nullptr;
    int *idx = nullptr, *keff = nullptr;
    int *state = nullptr;     // [0] problems, [1] packed rows, [2] union size, [3] GEMM row tiles
    int *uniq = nullptr, *xrows = nullptr, *slotrow = nullptr, *mt = nullptr;
    ColiProb *pdual = nullptr, *pdown = nullptr;
    int *route_cnt = nullptr;   // arrival counter of coli_moe_route (zero between launches)
    bool route_cnt_dirty = false;   // a forward failed part-way: clear the counter before the next
};

// ---------------------------------------------------------------------------
// union + descriptor build, one 1024-thread block.
// Selection i = (t, kk) in row-major order is live when kk < keff[t] and its
// expert is in range. The union lists the experts in first-seen order: an
// expert's rank is the number of experts whose first live selection comes
// earlier. Row lists are packed in that order; inside an expert's list rows
// are placed by an LDS counter (the placement of a row inside its list does
// not change any result: every row is computed on its own, and the combine
// addresses rows through slotrow).
// Also emits the GEMM work list (expert << 16 | 64-row tile) in union order.
// ---------------------------------------------------------------------------
// The body runs on any block size; sm: (7 E + 5) ints of LDS. idx / keff may
// point to LDS.
__device__ __forceinline__ void moe_union_body(const int *idx, const int *keff, int S, int K, int E, int has_shared,
                                               const ColiProb *__restrict__ tab, ColiProb *__restrict__ pdual,
                                               ColiProb *__restrict__ pdown, int *__restrict__ uniq,
                                               int *__restrict__ xrows, int *__restrict__ slotrow,
                                               int *__restrict__ mt, int *__restrict__ state, int *sm) {
    // first [E] | cnt [E] | cur [E] | rank [E] | order [E + 1] | off [E + 2] | toff [E + 2]
    int *first = sm, *cnt = first + E, *cur = cnt + E, *rank = cur + E, *order = rank + E, *off = order + E + 1,
        *toff = off + E + 2;
    __shared__ int s_nu;
    const int n = S * K;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        first[e] = 0x7fffffff;
        cnt[e] = 0;
        cur[e] = 0;
        rank[e] = -1;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int t = i / K, kk = i - t * K, e = idx[i];
        if (kk < keff[t] && e >= 0 && e < E) {
            atomicMin(first + e, i);
            atomicAdd(cnt + e, 1);
        }
    }
    __syncthreads();
    // Ranks straight from the selection positions, in chunks of one position
    // per thread: position i is its expert's first when first[e] == i, and
    // the expert's rank is the number of such positions before i (a ballot
    // per wave and a prefix over the waves' counts; no scan over E).
    {
        __shared__ int s_wc[32];
        const int w = threadIdx.x >> 6, ln = threadIdx.x & 63, nw = (blockDim.x + 63) >> 6;
        int base = 0;
        for (int c0 = 0; c0 < n; c0 += blockDim.x) {
            const int i = c0 + threadIdx.x;
            int e = -1;
            bool f = false;
            if (i < n) {
                const int t = i / K, kk = i - t * K;
                e = idx[i];
                f = kk < keff[t] && e >= 0 && e < E && first[e] == i;
            }
            const unsigned long long m = __builtin_amdgcn_ballot_w64(f);
            if (ln == 0) s_wc[w] = __popcll(m);
            __syncthreads();
            int pre = base, tot = 0;
            for (int v = 0; v < nw; v++) {
                pre += v < w ? s_wc[v] : 0;
                tot += s_wc[v];
            }
            if (f) {
                const int r = pre + __popcll(m & ((1ull << ln) - 1ull));
                rank[e] = r;
                order[r] = e;
            }
            base += tot;
            __syncthreads();   // s_wc is rewritten by the next chunk
        }
        if (threadIdx.x == 0) s_nu = base;
    }
    __syncthreads();
    const int nu = s_nu, np = nu + (has_shared ? 1 : 0);
    if (has_shared && threadIdx.x == 0) order[nu] = E;
    __syncthreads();
    // packed offsets and GEMM tile offsets in union order: exclusive prefix
    // sums over the problems, a wave scan per chunk of one problem per thread
    // plus a prefix over the waves' totals
    {
        __shared__ int s_ws[32], s_wt[32];
        const int w = threadIdx.x >> 6, ln = threadIdx.x & 63, nw = (blockDim.x + 63) >> 6;
        int base_o = 0, base_t = 0;
        for (int c0 = 0; c0 <= np; c0 += blockDim.x) {
            const int j = c0 + threadIdx.x;
            int c = 0, tl = 0;
            if (j < np) {
                c = order[j] == E ? S : cnt[order[j]];
                tl = (c + COLI_GM_ROWS - 1) / COLI_GM_ROWS;
            }
            int xc = c, xt = tl;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int yc = __shfl_up(xc, o), yt = __shfl_up(xt, o);
                if (ln >= o) {
                    xc += yc;
                    xt += yt;
                }
            }
            if (ln == 63) {
                s_ws[w] = xc;
                s_wt[w] = xt;
            }
            __syncthreads();
            int pc = base_o, pt = base_t, tc = 0, tt = 0;
            for (int v = 0; v < nw; v++) {
                if (v < w) {
                    pc += s_ws[v];
                    pt += s_wt[v];
                }
                tc += s_ws[v];
                tt += s_wt[v];
            }
            if (j <= np) {
                off[j] = pc + xc - c;
                toff[j] = pt + xt - tl;
            }
            base_o += tc;
            base_t += tt;
            __syncthreads();   // s_ws / s_wt are rewritten by the next chunk
        }
    }
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int t = i / K, kk = i - t * K, e = idx[i];
        if (kk < keff[t] && e >= 0 && e < E) {
            const int row = off[rank[e]] + atomicAdd(cur + e, 1);
            xrows[row] = t;
            slotrow[i] = row;
        }
    }
    if (has_shared)
        for (int t = threadIdx.x; t < S; t += blockDim.x) xrows[off[nu] + t] = t;
    for (int j = threadIdx.x; j < np; j += blockDim.x) {
        const int e = order[j];
        const int c = e == E ? S : cnt[e];
        if (j < nu) uniq[j] = e;
        ColiProb d = tab[2 * e], dn = tab[2 * e + 1];
        d.nrows = dn.nrows = c;
        d.xrow_off = dn.xrow_off = off[j];
        d.out_row0 = dn.out_row0 = off[j];
        pdual[j] = d;
        pdown[j] = dn;
        for (int q = 0; q * COLI_GM_ROWS < c; q++) mt[toff[j] + q] = j << 16 | q;
    }
    if (threadIdx.x == 0) {
        state[0] = np;
        state[1] = off[np];
        state[2] = nu;
        state[3] = toff[np];
    }
}

// ints of the selection / union work area (LDS) of E experts; the decode
// kernels keep the descriptor templates [2 (E + 1)] after it
__host__ __device__ inline int moe_work_ints(int E) { return 4 * E > 7 * E + 5 ? 4 * E : 7 * E + 5; }

// The union of at most 64 selections (S * K <= 64, decode) by one wave, no
// LDS and no barrier: lane i holds selection i = (t, kk). Same results as
// moe_union_body: first-seen order of the experts, each expert's rows packed
// in selection order, the shared expert's rows last, the GEMM tile list.
__device__ __forceinline__ void moe_union_wave(const int *idx, const int *keff, int S, int K, int E, int has_shared,
                                               const ColiProb *__restrict__ tab, ColiProb *__restrict__ pdual,
                                               ColiProb *__restrict__ pdown, int *__restrict__ uniq,
                                               int *__restrict__ xrows, int *__restrict__ slotrow,
                                               int *__restrict__ mt, int *__restrict__ state, int lane,
                                               int shared_row = -1) {
    const int n = S * K;
    const int t = lane / K, kk = lane - t * K;
    int e = -1;
    if (lane < n) {
        const int ei = idx[lane];
        if (kk < keff[t] && ei >= 0 && ei < E) e = ei;
    }
    // the descriptor templates are requested first: their latency overlaps
    // the scans below
    const int et = e >= 0 ? e : 0;
    ColiProb d = tab[2 * et], dn = tab[2 * et + 1];
    ColiProb sd = tab[2 * E], sdn = tab[2 * E + 1];   // the shared expert's row (E + 1 templates exist)
    // per lane: same-expert selections before it, in total, and the first one
    int before = 0, total = 0, firstl = lane;
    for (int j = 0; j < n; j++) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        const bool same = ej == e && e >= 0;
        before += same && j < lane ? 1 : 0;
        total += same ? 1 : 0;
        if (same && j < firstl) firstl = j;
    }
    const bool first = e >= 0 && before == 0;
    const unsigned long long fm = __builtin_amdgcn_ballot_w64(first);
    const int rank = __popcll(fm & ((1ull << lane) - 1ull));   // valid on first lanes
    const int nu = __popcll(fm);
    // packed offset of each expert's list: exclusive prefix of the counts in
    // first-seen (lane) order
    int c = first ? total : 0, inc = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(inc, o);
        if (lane >= o) inc += y;
    }
    const int off = inc - c;                                    // valid on first lanes
    const int rows_routed = __shfl(inc, 63);
    const int my_off = __shfl(off, firstl);
    if (e >= 0) {
        const int row = my_off + before;
        xrows[row] = t;
        slotrow[lane] = row;
    }
    if (first) {
        uniq[rank] = e;
        d.nrows = dn.nrows = total;
        d.xrow_off = dn.xrow_off = off;
        d.out_row0 = dn.out_row0 = off;
        pdual[rank] = d;
        pdown[rank] = dn;
        mt[rank] = rank << 16;   // one 64-row tile per expert (total <= S <= 64)
    }
    const int np = nu + (has_shared ? 1 : 0);
    if (has_shared) {
        if (lane < S) xrows[rows_routed + lane] = lane;
        if (lane == 0) {
            sd.nrows = sdn.nrows = S;
            sd.xrow_off = sdn.xrow_off = rows_routed;
            sd.out_row0 = sdn.out_row0 = rows_routed;
            // (its h row written elsewhere, at a row the selection does not move)
            if (shared_row >= 0) sdn.xrow_off = shared_row;
            pdual[nu] = sd;
            pdown[nu] = sdn;
            mt[nu] = nu << 16;
        }
    }
    if (lane == 0) {
        state[0] = np;
        state[1] = rows_routed + (has_shared ? S : 0);
        state[2] = nu;
        state[3] = np;
    }
}

__global__ __launch_bounds__(1024) void coli_moe_union(const int *__restrict__ idx, const int *__restrict__ keff,
                                                       int S, int K, int E, int has_shared,
                                                       const ColiProb *__restrict__ tab, ColiProb *__restrict__ pdual,
                                                       ColiProb *__restrict__ pdown, int *__restrict__ uniq,
                                                       int *__restrict__ xrows, int *__restrict__ slotrow,
                                                       int *__restrict__ mt, int *__restrict__ state) {
    extern __shared__ int sm[];
    moe_union_body(idx, keff, S, K, E, has_shared, tab, pdual, pdown, uniq, xrows, slotrow, mt, state, sm);
}

// ---------------------------------------------------------------------------
// Selection and union in one launch (partials from coli_router_partial): one
// wave per row; each workgroup publishes its rows' slots as agent-scope
// atomics, waits for its stores and counts its arrival; the last one to
// arrive reads every row's slots back and builds the union. Same arithmetic
// and results as coli_router_select followed by coli_moe_union.
// ---------------------------------------------------------------------------
template <int JM, bool MW = false>
__global__ __launch_bounds__(256) void coli_moe_select_union(const float *__restrict__ part, int nch,
                                                             const float *__restrict__ bias, int S, int E, int K,
                                                             int mode, float topp, int norm_topk, float routed_scale,
                                                             int *__restrict__ idx, float *__restrict__ wsel,
                                                             int *__restrict__ keff, int *__restrict__ counter,
                                                             int has_shared, const ColiProb *__restrict__ tab,
                                                             ColiProb *__restrict__ pdual, ColiProb *__restrict__ pdown,
                                                             int *__restrict__ uniq, int *__restrict__ xrows,
                                                             int *__restrict__ slotrow, int *__restrict__ mt,
                                                             int *__restrict__ state, ColiPrepArgs prep) {
    extern __shared__ int sm[];
    __shared__ int s_last;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // MW: workgroups past the S selecting ones build the rows' activation
    // fragments for the gate/up GEMV (independent of the selection)
    if constexpr (MW) {
        if ((int)blockIdx.x >= S) {
            prep_frag_block(prep, (int)blockIdx.x - S);
            return;
        }
    }
    const int nsel = MW ? S : (int)gridDim.x;   // selecting workgroups
    // LDS: slots [S K] | keff [S] | selection weights [4 E] floats, then the union's (7 E + 5) ints
    int *sidx = sm, *skeff = sm + S * K, *work = skeff + S;
    // decode: the descriptor templates go to LDS while the selection runs
    const bool small = S * K <= 64 && nsel == 1;
    ColiProb *stab = (ColiProb *)(((uintptr_t)(work + moe_work_ints(E)) + 15) & ~(uintptr_t)15);
    if (small)
        for (int i = threadIdx.x; i < 2 * (E + 1); i += blockDim.x) stab[i] = tab[i];
    if constexpr (MW) {
        // one row per workgroup (65-256 experts, sigmoid-family router, K <=
        // 16): the four waves score and rank 64 experts each and wave 0
        // merges their top K (same order and results as one wave's K rounds
        // over all of them)
        __shared__ __attribute__((aligned(16))) unsigned long long stage[4][64], cand[4][64], selb[64];
        __shared__ int nval[4];
        select_row_waves<4, true>(part, nch, bias, S, blockIdx.x, E, K, mode, topp, norm_topk, routed_scale, idx,
                                  wsel, keff, (float *)work, stage, cand, nval, selb, sidx, skeff, true, wave, lane);
    } else {
        select_row<JM, true, false>(part, nch, bias, S, E, K, mode, topp, norm_topk, routed_scale, idx, wsel, keff,
                                    (float *)work + (size_t)wave * E, blockIdx.x * 4 + wave, lane, sidx, skeff);
    }
    if (nsel > 1) {
        // publish, count; only the last workgroup goes on
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = old == nsel - 1;
            if (s_last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!s_last) return;
        // the other workgroups' rows (this one's are in LDS already)
        const int own0 = MW ? blockIdx.x : blockIdx.x * 4, own1 = MW ? own0 + 1 : min(S, own0 + 4);
        for (int i = threadIdx.x; i < S * K; i += blockDim.x)
            if (i / K < own0 || i / K >= own1)
                sidx[i] = __hip_atomic_load(idx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int t = threadIdx.x; t < S; t += blockDim.x)
            if (t < own0 || t >= own1)
                skeff[t] = __hip_atomic_load(keff + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (S * K <= 64) {   // decode: the one-wave union
        if (wave == 0) moe_union_wave(sidx, skeff, S, K, E, has_shared, small ? stab : tab, pdual, pdown, uniq, xrows,
                                      slotrow, mt, state, lane);
        return;
    }
    moe_union_body(sidx, skeff, S, K, E, has_shared, tab, pdual, pdown, uniq, xrows, slotrow, mt, state, work);
}

// ---------------------------------------------------------------------------
// Decode routing in one launch (S <= 16, up to 128 workgroups): router partial logits, top-K
// selection and union. Every workgroup computes the partials of 4 experts x
// one 512-column chunk and publishes them as agent-scope atomics (coherent
// across the XCDs' L2s), waits for its stores, then counts its arrival; the
// last workgroup to arrive runs the selection of every row (one wave per row,
// the partials read back as agent-scope atomics) and the union, and resets
// the counter for the next launch. No workgroup waits for another. Same
// arithmetic, order and results as the three separate kernels.
// ---------------------------------------------------------------------------
template <int SMAX, int JM>
__global__ __launch_bounds__(256) void coli_moe_route(const float *__restrict__ x, int S, const float *__restrict__ W,
                                                      int D, int E, float *__restrict__ part, int nch,
                                                      const float *__restrict__ bias, int K, int mode, float topp,
                                                      int norm_topk, float routed_scale, int *__restrict__ idx,
                                                      float *__restrict__ wsel, int *__restrict__ keff,
                                                      int *__restrict__ counter, int has_shared,
                                                      const ColiProb *__restrict__ tab, ColiProb *__restrict__ pdual,
                                                      ColiProb *__restrict__ pdown, int *__restrict__ uniq,
                                                      int *__restrict__ xrows, int *__restrict__ slotrow,
                                                      int *__restrict__ mt, int *__restrict__ state) {
    extern __shared__ int sm[];
    __shared__ int s_last;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int neb = (E + 3) / 4;
    const int eb = blockIdx.x % neb, ch = blockIdx.x / neb;
    router_partial_wave<SMAX, true>(x, S, W, D, E, part, (size_t)S * E, eb * 4 + wave, ch, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == (int)gridDim.x - 1;
        if (s_last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    // LDS: slots [S K] | keff [S] | selection weights [4 E] floats, then the union's (7 E + 5) ints
    int *sidx = sm, *skeff = sm + S * K, *work = skeff + S;
    // decode: the descriptor templates go to LDS while the selection runs
    ColiProb *stab = (ColiProb *)(((uintptr_t)(work + moe_work_ints(E)) + 15) & ~(uintptr_t)15);
    if (S * K <= 64)
        for (int i = threadIdx.x; i < 2 * (E + 1); i += blockDim.x) stab[i] = tab[i];
    for (int s = wave; s < S; s += 4)
        select_row<JM, true>(part, nch, bias, S, E, K, mode, topp, norm_topk, routed_scale, idx, wsel, keff,
                             (float *)work + (size_t)wave * E, s, lane, sidx, skeff);
    __syncthreads();
    if (S * K <= 64) {
        if (wave == 0) moe_union_wave(sidx, skeff, S, K, E, has_shared, stab, pdual, pdown, uniq, xrows, slotrow, mt,
                                      state, lane);
        return;
    }
    moe_union_body(sidx, skeff, S, K, E, has_shared, tab, pdual, pdown, uniq, xrows, slotrow, mt, state, work);
}

// ---------------------------------------------------------------------------
// Decode (one token): the down projection of every problem and the weighted
// combine in one launch. Workgroup = one 16-row output tile; wave j = problem
// j (the routed experts in union order, then the shared expert), whose one
// row of SwiGLU output h (f32, row j) it multiplies with its expert's tile on
// the VALU in f32: at one row an MFMA would compute 16 rows for one, and the
// f32 dot needs no hi / lo fragments. Lane l owns the tile's 16 B of row
// l % 16 and k-slice l / 16 (8 columns of each 32-column group); the four
// k-slices are summed with lane swaps. The products are summed per group
// and scaled by the group scale (folded into the e2m1 conversion for MXFP4;
// for int4, sum n x - 8 sum x). The waves' outputs meet in LDS and one wave
// forms out = sum over slots in slot order of w * y (+ the shared expert's y)
// with the same arithmetic as coli_moe_combine.
// ---------------------------------------------------------------------------

template <int KIND>
__device__ __forceinline__ float dc_group(uint32_t wd, const ScaleRegs<KIND> &sc, int j, const floatx4 &a,
                                          const floatx4 &b) {
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        x[i] = a[i];
        x[i + 4] = b[i];
    }
    if constexpr (KIND == COLI_KIND_FP4) {
        typedef float float2v __attribute__((ext_vector_type(2)));
        const float s = sc.get(j);
        const float2v w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 0);
        const float2v w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 1);
        const float2v w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 2);
        const float2v w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 3);
        const float wv[8] = {w0[0], w0[1], w1[0], w1[1], w2[0], w2[1], w3[0], w3[1]};
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) p = fmaf(wv[i], x[i], p);
        return p;
    } else {
        // nibble i = column i (offset binary, value n - 8)
        float p = 0.0f, sx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            p = fmaf((float)((wd >> (4 * i)) & 15u), x[i], p);
            sx += x[i];
        }
        return (p - 8.0f * sx) * sc.get(j);
    }
}

template <int KIND>
__device__ __forceinline__ float dc_group(uint32_t wd, const ScaleRegs<KIND> &sc, int j, const float *xp) {
    return dc_group<KIND>(wd, sc, j, *(const floatx4 *)xp, *(const floatx4 *)(xp + 4));
}

// One-token down projection of every problem + the combine, one workgroup
// per 16-row tile of the output: wave p holds problem p's whole tile (NQ
// 128-column quads: the expert's intermediate size is exactly NQ x 128, all
// in registers, all requested at once) and reduces it against its row of h;
// wave 0 then adds the problems' rows in slot order (c/colibri.c:4781-4782),
// the shared expert last. At most COLI_DC_WAVES problems (routed + shared).
// The row of h stays in registers: lane (ks, r) loads h[32 (4q + r/4) + 8 ks +
// 2 (r%4) + {0, 1}] of each quad q (the 32 activations its 16-lane row ks
// needs, two a lane), and every product takes its activation from lane
// 4j + i/2 of the row by a DPP row broadcast, with no LDS traffic (staging the
// row in LDS, 64 B read per lane and group, was slower: DSV3 B1 layer 60.1 ->
// 57.5 us, the 21 per-token passes 1236 -> 1172 us).
#define COLI_DC_WAVES 10
template <int ROWLANE>
__device__ __forceinline__ float row_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + ROWLANE, 0xF, 0xF,
                                                              true));
}
template <int KIND, int J>
__device__ __forceinline__ float dc_group_dpp(uint32_t wd, const ScaleRegs<KIND> &sc, const float (&xr)[2]) {
    if constexpr (KIND == COLI_KIND_FP4) {
        // the broadcast folded into the products: one v_fmac_f32 with a DPP
        // source per product, in the order of dc_group (p = x_i * w_i + p,
        // bitwise fmaf(w_i, x_i, p)); the leading s_nop keeps the DPP read
        // of xr two wait states after any VALU write to it
        typedef float float2v __attribute__((ext_vector_type(2)));
        const float s = sc.get(J);
        const float2v w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 0);
        const float2v w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 1);
        const float2v w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 2);
        const float2v w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd, s, 3);
        float p = 0.0f;
        asm("s_nop 1\n\t"
            "v_fmac_f32_dpp %0, %1, %3 row_newbcast:%11 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
            "v_fmac_f32_dpp %0, %2, %4 row_newbcast:%11 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
            "v_fmac_f32_dpp %0, %1, %5 row_newbcast:%12 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
            "v_fmac_f32_dpp %0, %2, %6 row_newbcast:%12 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
            "v_fmac_f32_dpp %0, %1, %7 row_newbcast:%13 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
            "v_fmac_f32_dpp %0, %2, %8 row_newbcast:%13 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
            "v_fmac_f32_dpp %0, %1, %9 row_newbcast:%14 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
            "v_fmac_f32_dpp %0, %2, %10 row_newbcast:%14 row_mask:0xf bank_mask:0xf bound_ctrl:1"
            : "+v"(p)
            : "v"(xr[0]), "v"(xr[1]), "v"(w0[0]), "v"(w0[1]), "v"(w1[0]), "v"(w1[1]), "v"(w2[0]), "v"(w2[1]),
              "v"(w3[0]), "v"(w3[1]), "n"(4 * J), "n"(4 * J + 1), "n"(4 * J + 2), "n"(4 * J + 3));
        return p;
    }
    float x[8];
    x[0] = row_bcast<4 * J + 0>(xr[0]);
    x[1] = row_bcast<4 * J + 0>(xr[1]);
    x[2] = row_bcast<4 * J + 1>(xr[0]);
    x[3] = row_bcast<4 * J + 1>(xr[1]);
    x[4] = row_bcast<4 * J + 2>(xr[0]);
    x[5] = row_bcast<4 * J + 2>(xr[1]);
    x[6] = row_bcast<4 * J + 3>(xr[0]);
    x[7] = row_bcast<4 * J + 3>(xr[1]);
    return dc_group<KIND>(wd, sc, J, (floatx4){x[0], x[1], x[2], x[3]}, (floatx4){x[4], x[5], x[6], x[7]});
}

template <int KIND, int NQ>
__global__ __launch_bounds__(64 * COLI_DC_WAVES) void coli_moe_down_combine1(const ColiProb *__restrict__ pdown,
                                                                const int *__restrict__ state,
                                                                const float *__restrict__ h, int D,
                                                                const float *__restrict__ w,
                                                                const int *__restrict__ keff,
                                                                const int *__restrict__ slotrow, int K,
                                                                int has_shared, float *__restrict__ out) {
    __shared__ float ys[COLI_DC_WAVES][16];   // [problem][tile row]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rb = blockIdx.x;
    // the live count, this wave's descriptor (the array holds one per wave
    // of the block) and the combine's inputs are loaded together: one round
    // trip before the weights, none before the combine
    const int P = state[0];
    const ColiProb pd = pdown[wave];
    float wk[COLI_DC_WAVES];
    int sk[COLI_DC_WAVES];
    int ke = 0;
    if (wave == 0) {
        ke = keff[0];
#pragma unroll
        for (int kk = 0; kk < COLI_DC_WAVES; kk++) {
            wk[kk] = kk < K ? w[kk] : 0.0f;
            sk[kk] = kk < K ? slotrow[kk] : 0;
        }
    }
    if (wave < P) {
        const ColiProb pr = uniform_prob(pd);
        const int ks = lane >> 4, r16 = lane & 15;
        const float *hr = h + (size_t)pr.xrow_off * (NQ * 128) + 8 * ks + 2 * (r16 & 3) + 32 * (r16 >> 2);
        const size_t t0 = (size_t)rb * NQ;
        const uint8_t *wt = pr.w0 + t0 * COLI_TILE_BYTES;
        // h first, then the weight quads of the tile (the compiler spreads
        // the later quads' requests over the first quads' products, which
        // keeps the wave at ~66 VGPRs: every workgroup of the launch is
        // resident at once; a barrier forcing all requests first measured
        // the same). (Two scalar loads for h, which the compiler pairs: the
        // elements of one vector load broadcast by DPP were folded into one
        // broadcast by this toolchain, a wrong result.)
        float xq[NQ][2];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            xq[q][0] = hr[q * 128];
            xq[q][1] = hr[q * 128 + 1];
        }
        u32x4 wq[NQ];
        ScaleRegs<KIND> sq[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            wq[q] = __builtin_nontemporal_load(GPTR(u32x4, wt + (size_t)q * COLI_TILE_BYTES) + lane);
            sq[q].load(pr.s0, t0 + q, r16);
        }
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            acc += dc_group_dpp<KIND, 0>(wq[q][0], sq[q], xq[q]);
            acc += dc_group_dpp<KIND, 1>(wq[q][1], sq[q], xq[q]);
            acc += dc_group_dpp<KIND, 2>(wq[q][2], sq[q], xq[q]);
            acc += dc_group_dpp<KIND, 3>(wq[q][3], sq[q], xq[q]);
        }
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        if (lane < 16) ys[wave][lane] = acc;
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
        const int d = rb * 16 + lane;
        if (d < D) {
            float acc = 0.0f;
#pragma unroll
            for (int kk = 0; kk < COLI_DC_WAVES; kk++)
                if (kk < ke) acc = fmaf(wk[kk], ys[sk[kk]][lane], acc);
            if (has_shared) acc += ys[P - 1][lane];
            out[d] = acc;
        }
    }
}

// The same launch on the matrix cores (used at an intermediate size of 1024,
// OLMoE's: 7.1 -> 6.6 us a layer; at 2048 the f32 form above measured
// faster): each wave converts its row of h once into fp16 hi / lo fragments in
// LDS (one exponent for the row, the column order and factors of
// coli_prep_frag), then runs two v_mfma_f32_16x16x32_f16 per 32-column group
// (hi, and lo when the row has any), the token's row in every row of the A
// operand: lane l ends with output row l % 16 of the tile, no lane sums
// needed. MXFP4 tensors whose scales fold exactly into the fp16 operand (FOLD)
// accumulate inside the MFMA; otherwise the group's result is scaled and
// accumulated on the VALU, one sum per group position.
template <bool INT4, int NCL>
__device__ __forceinline__ bool row_to_frags(const floatx4 (&v)[2 * NCL], _Float16 *dst, int ncol, int lane,
                                             int *E_out) {
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < 2 * NCL; k++)
#pragma unroll
        for (int i = 0; i < 4; i++) m = fmaxf(m, fabsf(v[k][i]));
    m = wave_max64(m);
    int E = 0;
    if (m > 0.0f && isfinite(m)) {
        frexpf(m, &E);
        E -= 15;
    }
    bool any = false;
#pragma unroll
    for (int c = 0; c < NCL; c++) {
        const float u[8] = {v[2 * c][0], v[2 * c][1], v[2 * c][2], v[2 * c][3],
                            v[2 * c + 1][0], v[2 * c + 1][1], v[2 * c + 1][2], v[2 * c + 1][3]};
        half8v hh, ll;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int off = INT4 ? (t < 4 ? 2 * t : 2 * (t - 4) + 1) : t;
            float y = ldexpf(u[off], -E);
            if (INT4 && (off & 1)) y *= 0.0625f;
            hh[t] = (_Float16)y;
            ll[t] = (_Float16)(y - (float)hh[t]);
            any |= ll[t] != (_Float16)0.0f;
        }
        const int ch = c * 64 + lane;   // 8-column chunk
        *(half8v *)(dst + ch * 8) = hh;
        *(half8v *)(dst + ncol + ch * 8) = ll;
    }
    *E_out = E;
    return __builtin_amdgcn_ballot_w64(any) != 0;
}

template <int KIND, int NQ, bool FOLD>
__global__ __launch_bounds__(64 * COLI_DC_WAVES) void coli_moe_down_combine1m(const ColiProb *__restrict__ pdown,
                                                                const int *__restrict__ state,
                                                                const float *__restrict__ h, int D,
                                                                const float *__restrict__ w,
                                                                const int *__restrict__ keff,
                                                                const int *__restrict__ slotrow, int K,
                                                                int has_shared, float *__restrict__ out) {
    static_assert(!FOLD || KIND == COLI_KIND_FP4, "folded scales: MXFP4 only");
    constexpr int NC = NQ * 128;   // columns of the row of h
    constexpr int NCL = NQ / 4;    // 8-column chunks per lane
    __shared__ float ys[COLI_DC_WAVES][16];   // [problem][tile row]
    extern __shared__ __attribute__((aligned(16))) _Float16 hfr[];   // [wave][hi NC | lo NC]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rb = blockIdx.x;
    const int P = state[0];
    const ColiProb pd = pdown[wave];
    float wk[COLI_DC_WAVES];
    int sk[COLI_DC_WAVES];
    int ke = 0;
    if (wave == 0) {
        ke = keff[0];
#pragma unroll
        for (int kk = 0; kk < COLI_DC_WAVES; kk++) {
            wk[kk] = kk < K ? w[kk] : 0.0f;
            sk[kk] = kk < K ? slotrow[kk] : 0;
        }
    }
    if (wave < P) {
        const ColiProb pr = uniform_prob(pd);
        const float *hr = h + (size_t)pr.xrow_off * NC;
        _Float16 *hs = hfr + wave * (2 * NC);
        const size_t t0 = (size_t)rb * NQ;
        const uint8_t *wt = pr.w0 + t0 * COLI_TILE_BYTES;
        const int ks = lane >> 4, r16 = lane & 15;
        // the row of h (8-column chunks c * 64 + lane), then every weight quad
        floatx4 hv[2 * NCL];
#pragma unroll
        for (int c = 0; c < NCL; c++) {
            hv[2 * c] = *GPTR(floatx4, hr + (size_t)(c * 64 + lane) * 8);
            hv[2 * c + 1] = *GPTR(floatx4, hr + (size_t)(c * 64 + lane) * 8 + 4);
        }
        u32x4 wq[NQ];
        ScaleRegs<KIND> sq[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            wq[q] = __builtin_nontemporal_load(GPTR(u32x4, wt + (size_t)q * COLI_TILE_BYTES) + lane);
            sq[q].load(pr.s0, t0 + q, r16);
        }
        int E;
        // the wave reads back only its own LDS writes: in order, no barrier
        const bool lo = row_to_frags<KIND != COLI_KIND_FP4, NCL>(hv, hs, NC, lane, &E);
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        float acc0[4] = {0.f, 0.f, 0.f, 0.f};   // unfolded: one VALU sum per group position
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int col = 32 * (4 * q + j) + 8 * ks;
                const half8v xh = *(const half8v *)(hs + col);
                const float scl = sq[q].get(j);
                half8v bw;
                if constexpr (FOLD) bw = unpack_fp4_scaled(wq[q][j], scl);
                else bw = unpack_b<KIND>(wq[q][j]);
                if constexpr (FOLD) {
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bw, acc, 0, 0, 0);
                    if (lo) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8v *)(hs + NC + col), bw, acc, 0, 0, 0);
                } else {
                    floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bw, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    if (lo) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8v *)(hs + NC + col), bw, d, 0, 0, 0);
                    acc0[j] = fmaf(d[0], scl, acc0[j]);
                }
            }
        }
        const float y = FOLD ? acc[0] : (acc0[0] + acc0[1]) + (acc0[2] + acc0[3]);
        if (lane < 16) ys[wave][lane] = ldexpf(y, E);
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
        const int d = rb * 16 + lane;
        if (d < D) {
            float acc = 0.0f;
#pragma unroll
            for (int kk = 0; kk < COLI_DC_WAVES; kk++)
                if (kk < ke) acc = fmaf(wk[kk], ys[sk[kk]][lane], acc);
            if (has_shared) acc += ys[P - 1][lane];
            out[d] = acc;
        }
    }
}

// ---------------------------------------------------------------------------
// Decode (one token): gate/up of every problem with the SwiGLU epilogue.
// Workgroup = (problem, 16-row tile of the intermediate); its W waves split K
// (wave w takes quads w, w + W, ...), each holding every weight quad of its
// share (gate and up tiles) in registers at once; the token's row of x is
// staged in LDS once per workgroup. f32 VALU dots as in
// coli_moe_down_combine1, then the waves' sums meet in LDS in fixed wave order
// and wave 0 applies SwiGLU and writes the tile's 16 values of h.
// ---------------------------------------------------------------------------
// The token's row of x: each wave loads its share (quads w, w + W, ...) into
// registers first, before anything else is requested. MXFP4 keeps them there
// (two activations a lane and quad, taken by the products through DPP row
// broadcasts: f32 VALU dots); int4 converts them into fp16 hi / lo fragments
// for the matrix cores.
// 8-column chunks of a wave's share per lane (int4 matrix-core form)
#define COLI_D1_NCL(NQW) (((NQW) * 16 + 63) / 64)
template <int KIND, int NQW>
struct Dual1X {
    float q[NQW][2];                       // MXFP4: lane (ks, r)'s two activations of each quad
    floatx4 m[2 * COLI_D1_NCL(NQW)];       // int4: chunks lane + 64 c of the wave's quads
};
template <int KIND, int W, int NQW>
__device__ __forceinline__ void dual1_load_x(const float *__restrict__ x, Dual1X<KIND, NQW> &xv, int wave, int lane) {
    if constexpr (KIND == COLI_KIND_FP4) {
#pragma unroll
        for (int i = 0; i < NQW; i++) {
            const float *p = x + (size_t)(wave + W * i) * 128 + 32 * ((lane & 15) >> 2) + 8 * (lane >> 4) +
                             2 * (lane & 3);
            xv.q[i][0] = p[0];
            xv.q[i][1] = p[1];
        }
    } else {
#pragma unroll
        for (int c = 0; c < COLI_D1_NCL(NQW); c++) {
            const int ch = c * 64 + lane, i = ch >> 4;
            const float *p = x + (size_t)(wave + W * i) * 128 + (ch & 15) * 8;
            xv.m[2 * c] = ch < NQW * 16 ? *GPTR(floatx4, p) : (floatx4){0.f, 0.f, 0.f, 0.f};
            xv.m[2 * c + 1] = ch < NQW * 16 ? *GPTR(floatx4, p + 4) : (floatx4){0.f, 0.f, 0.f, 0.f};
        }
    }
}
// LDS floats of the row staging of a dual1 workgroup
#define COLI_D1_XS(W, NQW) ((W) * COLI_D1_NCL(NQW) * 512)

// Gate/up of row tile rt of problem pr for the row whose share each wave
// holds in xv: every weight quad of the wave's share requested at once, the
// dots (MXFP4: f32 VALU with DPP sources; int4: on the matrix cores),
// the waves' sums in fixed order, SwiGLU by wave 0.
template <int KIND, int W, int NQW>
__device__ __forceinline__ void dual1_tile(const ColiProb &pr, int rt, const Dual1X<KIND, NQW> &xv,
                                           float *__restrict__ xs, float (&red)[W][2][16], float *__restrict__ h,
                                           int I, float swiglu_limit, int wave, int lane) {
    constexpr int NQ = W * NQW;   // the row's 128-column quads (D = NQ x 128)
    const int ks = lane >> 4, r16 = lane & 15;
    const size_t t0 = (size_t)rt * NQ;
    u32x4 wg[NQW], wu[NQW];
    ScaleRegs<KIND> sg[NQW], su[NQW];
#pragma unroll
    for (int i = 0; i < NQW; i++) {
        const int q = wave + W * i;
        wg[i] = __builtin_nontemporal_load(GPTR(u32x4, pr.w0 + (t0 + q) * COLI_TILE_BYTES) + lane);
        wu[i] = __builtin_nontemporal_load(GPTR(u32x4, pr.w1 + (t0 + q) * COLI_TILE_BYTES) + lane);
        sg[i].load(pr.s0, t0 + q, r16);
        su[i].load(pr.s1, t0 + q, r16);
    }
    float ag = 0.0f, au = 0.0f;
    if constexpr (KIND == COLI_KIND_FP4) {
        auto group = [&](auto jt, int i) {
            constexpr int J = decltype(jt)::value;
            ag += dc_group_dpp<KIND, J>(wg[i][J], sg[i], xv.q[i]);
            au += dc_group_dpp<KIND, J>(wu[i][J], su[i], xv.q[i]);
        };
#pragma unroll
        for (int i = 0; i < NQW; i++) {
            group(std::integral_constant<int, 0>{}, i);
            group(std::integral_constant<int, 1>{}, i);
            group(std::integral_constant<int, 2>{}, i);
            group(std::integral_constant<int, 3>{}, i);
        }
    } else {
        // int4 on the matrix cores: the wave's quads of x as fp16 hi / lo
        // fragments with one exponent for the wave (its LDS region, read back
        // by the wave only), the token's row in every row of the A operand;
        // lane l ends with output row l % 16 of each group's product, scaled
        // by the group scale and summed per group position
        constexpr int NCL = COLI_D1_NCL(NQW), NC = NCL * 512;
        _Float16 *hs = (_Float16 *)xs + (size_t)wave * (2 * NC);
        int E;
        const bool lo = row_to_frags<true, NCL>(xv.m, hs, NC, lane, &E);
        float g4[4] = {0.f, 0.f, 0.f, 0.f}, u4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NQW; i++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int col = 128 * i + 32 * j + 8 * ks;
                const half8v xh = *(const half8v *)(hs + col);
                const half8v bg = unpack_b<KIND>(wg[i][j]), bu = unpack_b<KIND>(wu[i][j]);
                floatx4 dg = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bg, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                floatx4 du = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bu, (floatx4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                if (lo) {
                    const half8v xl = *(const half8v *)(hs + NC + col);
                    dg = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bg, dg, 0, 0, 0);
                    du = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bu, du, 0, 0, 0);
                }
                g4[j] = fmaf(dg[0], sg[i].get(j), g4[j]);
                u4[j] = fmaf(du[0], su[i].get(j), u4[j]);
            }
        }
        if (lane < 16) {
            red[wave][0][lane] = ldexpf((g4[0] + g4[1]) + (g4[2] + g4[3]), E);
            red[wave][1][lane] = ldexpf((u4[0] + u4[1]) + (u4[2] + u4[3]), E);
        }
    }
    if constexpr (KIND == COLI_KIND_FP4) {
        ag += __shfl_xor(ag, 16);
        ag += __shfl_xor(ag, 32);
        au += __shfl_xor(au, 16);
        au += __shfl_xor(au, 32);
        if (lane < 16) {
            red[wave][0][lane] = ag;
            red[wave][1][lane] = au;
        }
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
        float g = red[0][0][lane], u = red[0][1][lane];
#pragma unroll
        for (int w = 1; w < W; w++) {
            g += red[w][0][lane];
            u += red[w][1][lane];
        }
        const int o = rt * 16 + lane;
        if (o < I) h[(size_t)pr.out_row0 * I + o] = swiglu_out(g, u, swiglu_limit);
    }
}

template <int KIND, int W, int NQW>
__global__ __launch_bounds__(64 * W) void coli_moe_dual1(const ColiProb *__restrict__ pdual,
                                                         const int *__restrict__ state, const float *__restrict__ x,
                                                         int D, int nrt, float *__restrict__ h, int I,
                                                         float swiglu_limit, int routed_only) {
    __shared__ __attribute__((aligned(16))) float xs[COLI_D1_XS(W, NQW)];
    __shared__ float red[W][2][16];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p = blockIdx.x / nrt, rt = blockIdx.x - p * nrt;
    // the live count and the descriptor (in the array: p < the launch's
    // problem count) in one round trip; routed_only: the shared expert's
    // gate/up ran in the selection launch
    const int np = state[routed_only ? 2 : 0];
    const ColiProb pd = pdual[p];
    if (p >= np) return;
    const ColiProb pr = uniform_prob(pd);
    Dual1X<KIND, NQW> xv;
    dual1_load_x<KIND, W, NQW>(x, xv, wave, lane);
    dual1_tile<KIND, W, NQW>(pr, rt, xv, xs, red, h, I, swiglu_limit, wave, lane);
}

// ---------------------------------------------------------------------------
// One token, 65-256 experts with a shared expert: the selection + union of
// coli_moe_select_union (workgroup 0, its first four waves) and the shared
// expert's gate/up + SwiGLU (workgroups 1..nrt, one 16-row tile each, the code
// and decomposition of coli_moe_dual1) in one launch: the shared expert needs
// no selection, so its weights stream while one workgroup selects. Its row of
// h goes to row K (the routed experts take rows 0..keff-1); the union points
// the down projection there, and the gate/up launch that follows runs the
// routed problems only.
// ---------------------------------------------------------------------------
template <int KIND, int W, int NQW>
__global__ __launch_bounds__(64 * W) void coli_moe_select_union_sh(
    const float *__restrict__ part, int nch, const float *__restrict__ bias, int E, int K, int mode, float topp,
    int norm_topk, float routed_scale, int *__restrict__ idx, float *__restrict__ wsel, int *__restrict__ keff,
    const ColiProb *__restrict__ tab, ColiProb *__restrict__ pdual, ColiProb *__restrict__ pdown,
    int *__restrict__ uniq, int *__restrict__ xrows, int *__restrict__ slotrow, int *__restrict__ mt,
    int *__restrict__ state, const float *__restrict__ x, float *__restrict__ h, int I, float swiglu_limit) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blockIdx.x > 0) {
        __shared__ __attribute__((aligned(16))) float xs[COLI_D1_XS(W, NQW)];
        __shared__ float red[W][2][16];
        Dual1X<KIND, NQW> xv;
        dual1_load_x<KIND, W, NQW>(x, xv, wave, lane);
        ColiProb pr = uniform_prob(tab[2 * E]);
        pr.nrows = 1;
        pr.xrow_off = 0;
        pr.out_row0 = K;
        dual1_tile<KIND, W, NQW>(pr, (int)blockIdx.x - 1, xv, xs, red, h, I, swiglu_limit, wave, lane);
        return;
    }
    extern __shared__ int sm[];
    // LDS: slots [K] | keff [1] | selection weights, then the descriptor templates
    int *sidx = sm, *skeff = sm + K, *work = skeff + 1;
    ColiProb *stab = (ColiProb *)(((uintptr_t)(work + moe_work_ints(E)) + 15) & ~(uintptr_t)15);
    for (int i = threadIdx.x; i < 2 * (E + 1); i += blockDim.x) stab[i] = tab[i];
    __shared__ __attribute__((aligned(16))) unsigned long long stage[4][64], cand[4][64], selb[64];
    __shared__ int nval[4];
    select_row_waves<4, true>(part, nch, bias, 1, 0, E, K, mode, topp, norm_topk, routed_scale, idx, wsel, keff,
                              (float *)work, stage, cand, nval, selb, sidx, skeff, true, wave, lane);
    __syncthreads();
    if (wave == 0)
        moe_union_wave(sidx, skeff, 1, K, E, 1, stab, pdual, pdown, uniq, xrows, slotrow, mt, state, lane, K);
}

// ---------------------------------------------------------------------------
// Decode (one token), routing and gate/up in one launch after the router
// partials (coli_router_partial): every workgroup of the gate/up grid selects
// the token's experts itself (one wave, select_row on the partials: the same
// code, inputs and order in every workgroup, so every workgroup finds the
// same experts) and takes its problem's descriptor from the templates staged
// in LDS meanwhile; problem p < keff is the expert of slot p (the union order
// of one row), p == keff the shared expert. Workgroup 0 also writes the
// selection and builds the union's descriptors and lists, as the separate
// selection + union launch would, for the down projection + combine that
// follows. No workgroup waits for another. Results are bitwise those of the
// separate launches.
// ---------------------------------------------------------------------------
template <int KIND, int W, int NQW>
__global__ __launch_bounds__(64 * W) void coli_moe_route_dual1(
    const float *__restrict__ part, int nch, const float *__restrict__ bias, int E, int K, int mode, float topp,
    int norm_topk, float routed_scale, int *__restrict__ idx, float *__restrict__ wsel, int *__restrict__ keff,
    int has_shared, const ColiProb *__restrict__ tab, ColiProb *__restrict__ pdual, ColiProb *__restrict__ pdown,
    int *__restrict__ uniq, int *__restrict__ xrows, int *__restrict__ slotrow, int *__restrict__ mt,
    int *__restrict__ state, const float *__restrict__ x, int nrt, float *__restrict__ h, int I, float swiglu_limit) {
    extern __shared__ __attribute__((aligned(16))) uint8_t dsm[];
    __shared__ __attribute__((aligned(16))) float xs[COLI_D1_XS(W, NQW)];
    __shared__ float red[W][2][16];
    __shared__ int sidx[64], skeff[1];
    // dynamic LDS: the selection's E floats, then the 2 (E + 1) descriptor templates
    float *psel = (float *)dsm;
    ColiProb *stab = (ColiProb *)(dsm + (((size_t)E * sizeof(float) + 15) & ~(size_t)15));
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p = blockIdx.x / nrt, rt = blockIdx.x - p * nrt;
    Dual1X<KIND, NQW> xv;
    dual1_load_x<KIND, W, NQW>(x, xv, wave, lane);
    for (int i = threadIdx.x; i < 2 * (E + 1); i += 64 * W) stab[i] = tab[i];
    const bool first = blockIdx.x == 0;
    if (wave == 0)
        select_row<1, false, false>(part, nch, bias, 1, E, K, mode, topp, norm_topk, routed_scale, idx, wsel, keff,
                                    psel, 0, lane, sidx, skeff, first);
    __syncthreads();
    if (first && wave == 0)
        moe_union_wave(sidx, skeff, 1, K, E, has_shared, stab, pdual, pdown, uniq, xrows, slotrow, mt, state, lane);
    const int ke = skeff[0];
    int e;
    if (p < ke) e = sidx[p];
    else if (p == ke && has_shared) e = E;
    else return;
    if (e < 0 || e >= E + 1) return;
    ColiProb pr = uniform_prob(stab[2 * e]);
    pr.nrows = 1;
    pr.xrow_off = p;
    pr.out_row0 = p;
    dual1_tile<KIND, W, NQW>(pr, rt, xv, xs, red, h, I, swiglu_limit, wave, lane);
}

// out[t, d] = sum_{kk < keff[t]} w[t, kk] * y[slotrow[t, kk], d]  (+ y[shared row of t])
__global__ void coli_moe_combine(const float *__restrict__ y, int D, const float *__restrict__ w,
                                 const int *__restrict__ keff, const int *__restrict__ slotrow, int K,
                                 const int *__restrict__ state, int has_shared, int S, float *__restrict__ out) {
    int t = blockIdx.y, d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    // keff, the weights, the slot rows and the shared row's position are
    // loaded together, then the expert outputs: two memory round trips
    const int ke = keff[t];
    const int shared_row = has_shared ? state[1] - S + t : 0;
    float acc = 0.0f;
    for (int kk0 = 0; kk0 < K; kk0 += 8) {
        float wv[8], yv[8];
        int sr[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int kk = kk0 + u;
            wv[u] = kk < K ? w[t * K + kk] : 0.0f;
            sr[u] = kk < K ? slotrow[t * K + kk] : 0;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) yv[u] = kk0 + u < ke ? y[(size_t)sr[u] * D + d] : 0.0f;
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (kk0 + u < ke) acc = fmaf(wv[u], yv[u], acc);
    }
    if (has_shared) acc += y[(size_t)shared_row * D + d];
    out[(size_t)t * D + d] = acc;
}

extern "C" void coli_hip_moe_free(ColiHipMoe *m) {
    if (!m) return;
    DevCtx *ctx = ctx_of(m->device);
    if (ctx) {
        bind_ctx(ctx);
        (void)hipStreamSynchronize(ctx->stream);
    }
    void *bufs[] = {m->rw, m->rb, m->tab, m->logits, m->wsel, m->h, m->y, m->idx, m->keff, m->state,
                    m->uniq, m->xrows, m->slotrow, m->mt, m->pdual, m->pdown, m->route_cnt};
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
        c.route_mode > 3 || !(c.swiglu_limit >= 0.0f))
        return 0;
    if (c.has_shared && (!sg || !su || !sd)) return 0;
    DevCtx *ctx = ctx_of(device);
    if (!bind_ctx(ctx)) return 0;
    int kind = gates[0] ? gates[0]->kind : -1;
    if (kind < 0 || kind == COLI_KIND_GENERIC) return 0;
    int n = c.E + (c.has_shared ? 1 : 0);
    std::vector<const ColiCudaTensor *> mats;
    std::vector<ColiProb> tab(2 * (c.E + 1));
    for (int e = 0; e < n; e++) {
        ColiCudaTensor *g = e < c.E ? gates[e] : sg, *u = e < c.E ? ups[e] : su, *d = e < c.E ? downs[e] : sd;
        if (!g || !u || !d || g->device != device || u->device != device || d->device != device ||
            g->kind != kind || u->kind != kind || d->kind != kind || g->I != c.D || u->I != c.D || g->O != c.I ||
            u->O != c.I || d->I != c.I || d->O != c.D)
            return 0;
        mats.push_back(g);
        mats.push_back(u);
        mats.push_back(d);
        tab[2 * e] = {g->w, g->sc, u->w, u->sc, 0, 0, 0, 0};
        tab[2 * e + 1] = {d->w, d->sc, nullptr, nullptr, 0, 0, 0, 0};
    }
    ColiHipMoe *m = new ColiHipMoe();
    m->device = device;
    m->cfg = c;
    m->kind = kind;
    m->mats = std::move(mats);
    m->S_cap = 0;
    size_t rwb = (size_t)c.E * c.D * sizeof(float);
    int ok = hip_check(hipMalloc((void **)&m->rw, rwb), "router weights") &&
             hip_check(hipMemcpy(m->rw, router_w, rwb, hipMemcpyHostToDevice), "router weights upload") &&
             hip_check(hipMalloc((void **)&m->tab, tab.size() * sizeof(ColiProb)), "expert table") &&
             hip_check(hipMemcpy(m->tab, tab.data(), tab.size() * sizeof(ColiProb), hipMemcpyHostToDevice),
                    "expert table upload") &&
             hip_check(hipMalloc((void **)&m->route_cnt, sizeof(int)), "routing counter") &&
             hip_check(hipMemset(m->route_cnt, 0, sizeof(int)), "routing counter clear");
    if (ok && router_bias)
        ok = hip_check(hipMalloc((void **)&m->rb, (size_t)c.E * sizeof(float)), "router bias") &&
             hip_check(hipMemcpy(m->rb, router_bias, (size_t)c.E * sizeof(float), hipMemcpyHostToDevice),
                    "router bias upload");
    if (!ok) {
        coli_hip_moe_free(m);
        return 0;
    }
    *out = m;
    return 1;
}

// Upper bounds of one forward of S rows.
static int moe_problems(const ColiHipMoeConfig &c, int S) { return std::min(c.E, S * c.K) + (c.has_shared ? 1 : 0); }
static int moe_rows(const ColiHipMoeConfig &c, int S) { return S * c.K + (c.has_shared ? S : 0); }
static int moe_tiles(const ColiHipMoeConfig &c, int S) {
    return (moe_rows(c, S) + COLI_GM_ROWS - 1) / COLI_GM_ROWS + moe_problems(c, S);
}

// Per-forward buffers for up to S rows (allocated once per growth of S).
static int moe_reserve(DevCtx *ctx, ColiHipMoe *m, int S) {
    if (S <= m->S_cap) return 1;
    if (!hip_check(hipStreamSynchronize(ctx->stream), "moe reserve sync")) return 0;
    const ColiHipMoeConfig &c = m->cfg;
    const int P = moe_problems(c, S), rows = moe_rows(c, S);
    void **bufs[] = {(void **)&m->logits, (void **)&m->wsel, (void **)&m->h, (void **)&m->y, (void **)&m->idx,
                     (void **)&m->keff, (void **)&m->state, (void **)&m->uniq, (void **)&m->xrows,
                     (void **)&m->slotrow, (void **)&m->mt, (void **)&m->pdual, (void **)&m->pdown};
    for (void **b : bufs)
        if (*b) {
            (void)hipFree(*b);
            *b = nullptr;
        }
    const size_t sizes[] = {(size_t)coli_router_chunks(c.D) * S * c.E * 4, (size_t)S * c.K * 4,
                            (size_t)rows * c.I * 4, (size_t)rows * c.D * 4, (size_t)S * c.K * 4, (size_t)S * 4, 16,
                            (size_t)c.E * 4, (size_t)rows * 4, (size_t)S * c.K * 4, (size_t)moe_tiles(c, S) * 4,
                            (size_t)P * sizeof(ColiProb), (size_t)P * sizeof(ColiProb)};
    for (int i = 0; i < 13; i++)
        if (!hip_check(hipMalloc(bufs[i], sizes[i]), "moe buffers")) return 0;
    m->S_cap = S;
    return 1;
}

// COLI_HIP_FUSED_ROUTE=0 runs the router, selection and union as three
// launches at every S.
static bool fused_route_disabled() {
    const char *e = std::getenv("COLI_HIP_FUSED_ROUTE");
    return e && e[0] == '0';
}

static int launch_route(ColiHipMoe *m, const float *x_dev, int S, hipStream_t st) {
    const ColiHipMoeConfig &c = m->cfg;
    const int nch = coli_router_chunks(c.D), neb = (c.E + 3) / 4;
    const size_t work = (size_t)moe_work_ints(c.E) * sizeof(int) + 16 + (size_t)2 * (c.E + 1) * sizeof(ColiProb);
    const size_t shm = (size_t)(S * c.K + S) * sizeof(int) + work;
    const int jm = c.E <= 64 ? 1 : c.E <= 128 ? 2 : c.E <= 256 ? 4 : c.E <= 512 ? 8 : 16;
    const dim3 grid((unsigned)(neb * nch)), block(256);
#define COLI_ROUTE_ARGS                                                                                         \
    x_dev, S, m->rw, c.D, c.E, m->logits, nch, m->rb, c.K, c.route_mode, c.topp, c.norm_topk, c.routed_scale, \
        m->idx, m->wsel, m->keff, m->route_cnt, c.has_shared, m->tab, m->pdual, m->pdown, m->uniq, m->xrows,  \
        m->slotrow, m->mt, m->state
#define COLI_ROUTE_JM(SM)                                                                                    \
    switch (jm) {                                                                                            \
    case 1: hipLaunchKernelGGL((coli_moe_route<SM, 1>), grid, block, shm, st, COLI_ROUTE_ARGS); break;       \
    case 2: hipLaunchKernelGGL((coli_moe_route<SM, 2>), grid, block, shm, st, COLI_ROUTE_ARGS); break;       \
    case 4: hipLaunchKernelGGL((coli_moe_route<SM, 4>), grid, block, shm, st, COLI_ROUTE_ARGS); break;       \
    case 8: hipLaunchKernelGGL((coli_moe_route<SM, 8>), grid, block, shm, st, COLI_ROUTE_ARGS); break;       \
    default: hipLaunchKernelGGL((coli_moe_route<SM, 16>), grid, block, shm, st, COLI_ROUTE_ARGS); break;     \
    }
    if (S == 1) {
        COLI_ROUTE_JM(1)
    } else if (S <= 4) {
        COLI_ROUTE_JM(4)
    } else {
        COLI_ROUTE_JM(16)
    }
#undef COLI_ROUTE_JM
#undef COLI_ROUTE_ARGS
    return hip_check(hipGetLastError(), "moe routing");
}

// prep: a fragment build run by extra workgroups of the four-wave selection
// launch (nblocks 0: none; only passed when that launch is taken)
static bool select_union_mw(const ColiHipMoeConfig &c) {
    return c.route_mode != 0 && c.E > 64 && c.E <= 256 && c.K <= 16;
}

static int launch_select_union(ColiHipMoe *m, int nch, int S, hipStream_t st, const ColiPrepArgs &prep) {
    const ColiHipMoeConfig &c = m->cfg;
    const size_t work = (size_t)moe_work_ints(c.E) * sizeof(int) + 16 + (size_t)2 * (c.E + 1) * sizeof(ColiProb);
    const size_t shm = (size_t)(S * c.K + S) * sizeof(int) + work;
    const int jm = c.E <= 64 ? 1 : c.E <= 128 ? 2 : c.E <= 256 ? 4 : c.E <= 512 ? 8 : 16;
    const dim3 grid((unsigned)((S + 3) / 4)), block(256);
#define COLI_SU(JM)                                                                                             \
    hipLaunchKernelGGL((coli_moe_select_union<JM>), grid, block, shm, st, m->logits, nch, m->rb, S, c.E, c.K,     \
                       c.route_mode, c.topp, c.norm_topk, c.routed_scale, m->idx, m->wsel, m->keff, m->route_cnt, \
                       c.has_shared, m->tab, m->pdual, m->pdown, m->uniq, m->xrows, m->slotrow, m->mt, m->state,  \
                       prep)
    if (select_union_mw(c)) {
        // one row per workgroup, selected by its four waves (DSV3's 256
        // experts: S = 1 selection 8.0 -> 6.5 us), and the fragment build
        hipLaunchKernelGGL((coli_moe_select_union<4, true>), dim3((unsigned)(S + prep.nblocks)), block, shm, st,
                           m->logits, nch, m->rb, S, c.E, c.K, c.route_mode, c.topp, c.norm_topk, c.routed_scale,
                           m->idx, m->wsel, m->keff, m->route_cnt, c.has_shared, m->tab, m->pdual, m->pdown, m->uniq,
                           m->xrows, m->slotrow, m->mt, m->state, prep);
        return hip_check(hipGetLastError(), "moe selection + union");
    }
    switch (jm) {
    case 1: COLI_SU(1); break;
    case 2: COLI_SU(2); break;
    case 4: COLI_SU(4); break;
    case 8: COLI_SU(8); break;
    default: COLI_SU(16); break;
    }
#undef COLI_SU
    return hip_check(hipGetLastError(), "moe selection + union");
}

static int moe_forward_impl(ColiHipMoe *m, DevCtx *ctx, const float *x_dev, float *out_dev, int S);

// COLI_HIP_DUAL1=0: at one token, gate/up run on the decode GEMV instead.
static bool dual1_enabled() {
    const char *e = std::getenv("COLI_HIP_DUAL1");
    return !(e && e[0] == '0');
}

// One token's gate/up + SwiGLU for the hidden sizes it is built for (2048:
// 4 waves x 4 quads, 7168: 8 waves x 7 quads); false: not launched.
static bool launch_dual1(ColiHipMoe *m, hipStream_t st, const float *x, int nrt, int nq, int P,
                         bool routed_only = false) {
    const ColiHipMoeConfig &c = m->cfg;
    const dim3 grid((unsigned)((routed_only ? P - 1 : P) * nrt));
#define COLI_D1(KD, W, NQW)                                                                                   \
    hipLaunchKernelGGL((coli_moe_dual1<KD, W, NQW>), grid, dim3(64 * W), 0, st, m->pdual, m->state, x, c.D, nrt, \
                       m->h, c.I, c.swiglu_limit, routed_only ? 1 : 0)
#define COLI_D1_KIND(W, NQW)                                                  \
    if (m->kind == COLI_KIND_I4_H) COLI_D1(COLI_KIND_I4_H, W, NQW);          \
    else if (m->kind == COLI_KIND_I4_F) COLI_D1(COLI_KIND_I4_F, W, NQW);     \
    else COLI_D1(COLI_KIND_FP4, W, NQW);                                     \
    return true
    if (c.D == 2048 && nq == 16) { COLI_D1_KIND(4, 4); }
    if (c.D == 7168 && nq == 56) { COLI_D1_KIND(8, 7); }
#undef COLI_D1_KIND
#undef COLI_D1
    return false;
}

// COLI_HIP_PREP_BESIDE=0: the rows' activation fragments keep their own
// launch instead of running beside the four-wave selection.
static bool prep_beside_enabled() {
    const char *e = std::getenv("COLI_HIP_PREP_BESIDE");
    return !(e && e[0] == '0');
}

// COLI_HIP_SHARED_OVERLAP=0: the shared expert's gate/up stays in the gate/up
// launch instead of running beside the selection.
static bool shared_overlap_enabled() {
    const char *e = std::getenv("COLI_HIP_SHARED_OVERLAP");
    return !(e && e[0] == '0');
}

// The selection + union with the shared expert's gate/up beside it (one
// token, four-wave selection of 65-256 experts, the hidden sizes the one-token
// gate/up is built for); false: not built for the shape.
static bool launch_select_union_sh(ColiHipMoe *m, hipStream_t st, int nch, const float *x, int nrt, int nq) {
    const ColiHipMoeConfig &c = m->cfg;
    if (!c.has_shared || c.route_mode == 0 || c.E <= 64 || c.E > 256 || c.K > 16 ||
        !((c.D == 2048 && nq == 16) || (c.D == 7168 && nq == 56)))
        return false;
    const size_t shm = (size_t)(c.K + 1) * sizeof(int) + (size_t)moe_work_ints(c.E) * sizeof(int) + 16 +
                       (size_t)2 * (c.E + 1) * sizeof(ColiProb);
    const dim3 grid((unsigned)(1 + nrt));
#define COLI_SUS(KD, W, NQW)                                                                                    \
    hipLaunchKernelGGL((coli_moe_select_union_sh<KD, W, NQW>), grid, dim3(64 * W), shm, st, m->logits, nch, m->rb, \
                       c.E, c.K, c.route_mode, c.topp, c.norm_topk, c.routed_scale, m->idx, m->wsel, m->keff,      \
                       m->tab, m->pdual, m->pdown, m->uniq, m->xrows, m->slotrow, m->mt, m->state, x, m->h, c.I,   \
                       c.swiglu_limit)
#define COLI_SUS_KIND(W, NQW)                                                 \
    if (m->kind == COLI_KIND_I4_H) COLI_SUS(COLI_KIND_I4_H, W, NQW);          \
    else if (m->kind == COLI_KIND_I4_F) COLI_SUS(COLI_KIND_I4_F, W, NQW);     \
    else COLI_SUS(COLI_KIND_FP4, W, NQW);                                     \
    return true
    if (c.D == 2048) { COLI_SUS_KIND(4, 4); }
    COLI_SUS_KIND(8, 7);
#undef COLI_SUS_KIND
#undef COLI_SUS
}

// COLI_HIP_ROUTE_DUAL1=0: at one token, the selection + union keep their own
// launch before the gate/up (instead of running inside it).
static bool route_dual1_enabled() {
    const char *e = std::getenv("COLI_HIP_ROUTE_DUAL1");
    return !(e && e[0] == '0');
}

// One token's selection, union and gate/up + SwiGLU in one launch after the
// router partials (nch chunks in m->logits), for at most 64 experts (one per
// lane of the selecting wave); false: not built for the shape. With more
// experts every workgroup's selection costs more than the separate launch
// (DSV3, 256 experts: layer 60.6-62.9 -> 65.1-65.8 us; OLMoE, 64: 22.0 ->
// 18.9 us).
static bool launch_route_dual1(ColiHipMoe *m, hipStream_t st, int nch, const float *x, int nrt, int nq, int P) {
    const ColiHipMoeConfig &c = m->cfg;
    if (c.K > 64 || c.E > 64 || !((c.D == 2048 && nq == 16) || (c.D == 7168 && nq == 56))) return false;
    const size_t shm = (((size_t)c.E * sizeof(float) + 15) & ~(size_t)15) + (size_t)2 * (c.E + 1) * sizeof(ColiProb);
    const dim3 grid((unsigned)(P * nrt));
#define COLI_RD1(KD, W, NQW)                                                                                   \
    hipLaunchKernelGGL((coli_moe_route_dual1<KD, W, NQW>), grid, dim3(64 * W), shm, st, m->logits, nch, m->rb, c.E, \
                       c.K, c.route_mode, c.topp, c.norm_topk, c.routed_scale, m->idx, m->wsel, m->keff,          \
                       c.has_shared, m->tab, m->pdual, m->pdown, m->uniq, m->xrows, m->slotrow, m->mt, m->state, x, \
                       nrt, m->h, c.I, c.swiglu_limit)
#define COLI_RD1_KIND(W, NQW)                                      \
    if (m->kind == COLI_KIND_I4_H) COLI_RD1(COLI_KIND_I4_H, W, NQW);      \
    else if (m->kind == COLI_KIND_I4_F) COLI_RD1(COLI_KIND_I4_F, W, NQW); \
    else COLI_RD1(COLI_KIND_FP4, W, NQW);                                 \
    return true
    if (c.D == 2048) { COLI_RD1_KIND(4, 4); }
    COLI_RD1_KIND(8, 7);
#undef COLI_RD1_KIND
#undef COLI_RD1
}

// COLI_HIP_DOWNCOMBINE=0: at one token, the down projection and the combine
// run as separate launches (the GEMV of any batch size, then the combine).
static bool down_combine_enabled() {
    const char *e = std::getenv("COLI_HIP_DOWNCOMBINE");
    return !(e && e[0] == '0');
}

// COLI_HIP_DC_MFMA=0: the one-token down + combine takes its f32 VALU form.
static bool dc_mfma_enabled() {
    const char *e = std::getenv("COLI_HIP_DC_MFMA");
    return !(e && e[0] == '0');
}

extern "C" int coli_hip_moe_forward_dev(ColiHipMoe *m, const float *x_dev, float *out_dev, int S) {
    if (fault_injected()) return 0;
    if (!m || !x_dev || !out_dev || S < 1 || S > COLI_MOE_MAX_ROWS || S * m->cfg.K > COLI_MOE_MAX_SEL) return 0;
    DevCtx *ctx = ctx_of(m->device);
    if (!bind_ctx(ctx)) return 0;
    // The routing kernels count arrivals on route_cnt and the last workgroup
    // resets it; a forward that failed after its routing launch was queued
    // may leave it non-zero, so it is cleared (fill kernel) before the next.
    if (m->route_cnt_dirty) {
        if (!hip_check(coli_launch_zero_i32(m->route_cnt, 1, ctx->stream), "routing counter reset")) return 0;
        m->route_cnt_dirty = false;
    }
    forget_emitted(ctx, out_dev, (size_t)S * m->cfg.D * sizeof(float));
    const int ok = moe_forward_impl(m, ctx, x_dev, out_dev, S);
    if (!ok) m->route_cnt_dirty = true;
    return ok;
}

static int moe_forward_impl(ColiHipMoe *m, DevCtx *ctx, const float *x_dev, float *out_dev, int S) {
    if (!moe_reserve(ctx, m, S)) return 0;
    const ColiHipMoeConfig &c = m->cfg;
    const int P = moe_problems(c, S), rows = moe_rows(c, S);
    const int nq_d = (c.D + 127) / 128, nq_i = (c.I + 127) / 128;
    const int fx = frag_set_of(m->kind, false), fh = frag_set_of(m->kind, true);
    const int int4 = m->kind != COLI_KIND_FP4;
    hipStream_t st = ctx->stream;
    // many-row MXFP4 layers run the block-scaled MFMA GEMM on e4m3 pieces
    const bool gemm = S > COLI_GEMM_MIN_ROWS, mx = gemm && m->kind == COLI_KIND_FP4 && mx_gemm_enabled();
    // 1. activation fragments, 2-3. router
    if (!(mx ? make_frags8(ctx, fx, x_dev, c.D, S, c.D) : make_frags(ctx, fx, x_dev, c.D, S, c.D, int4))) return 0;
    const int nrt_i = (c.I + 15) / 16, nrt_d = (c.D + 15) / 16;
    // One token, up to 64 experts: the router partials, then the selection and
    // the union inside the gate/up launch (every workgroup selects for itself).
    bool gateup_done = false;
    // One token, 65-256 experts and a shared expert, the one-token gate/up and
    // down + combine: the shared expert's gate/up runs in the selection launch
    // (the down + combine reads its h from row K).
    const int pmax1 = c.K + (c.has_shared ? 1 : 0);
    const bool shared_overlap = S == 1 && !gemm && c.has_shared && shared_overlap_enabled() && dual1_enabled() &&
                                c.route_mode != 0 && c.E > 64 && c.E <= 256 && c.K <= 16 &&
                                ((c.D == 2048 && nq_d == 16) || (c.D == 7168 && nq_d == 56)) &&
                                pmax1 <= COLI_DC_WAVES && (c.I == 1024 || c.I == 2048) && down_combine_enabled() && !fused_route_disabled() &&
                                !(S <= 16 && (long)((c.E + 3) / 4) * coli_router_chunks(c.D) <= 128);
    if (S == 1 && !gemm && dual1_enabled() && route_dual1_enabled() && !fused_route_disabled() &&
        c.K <= 64 && c.E <= 64 && ((c.D == 2048 && nq_d == 16) || (c.D == 7168 && nq_d == 56))) {
        const int nch = router_logits(ctx, x_dev, S, m->rw, c.D, c.E, m->logits);
        if (!nch || !launch_route_dual1(m, st, nch, x_dev, nrt_i, nq_d, P) ||
            !hip_check(hipGetLastError(), "moe routing + gate/up"))
            return 0;
        gateup_done = true;
    } else if (S <= 16 && (long)((c.E + 3) / 4) * coli_router_chunks(c.D) <= 128 && !fused_route_disabled()) {
        // 2-4. router, selection and union in one launch, when few workgroups
        // arrive: every arrival is an atomic on one counter, and hundreds of
        // them serialize (measured: 896 arrivals cost more than the two
        // launches they save)
        if (!launch_route(m, x_dev, S, st)) return 0;
    } else if (S == 1 && !gemm && shared_overlap && !fused_route_disabled()) {
        // 2. router partials, 3-4. selection and union with the shared
        // expert's gate/up beside them
        const int nch = router_logits(ctx, x_dev, S, m->rw, c.D, c.E, m->logits);
        if (!nch || !launch_select_union_sh(m, st, nch, x_dev, nrt_i, nq_d) ||
            !hip_check(hipGetLastError(), "moe selection + union + shared gate/up"))
            return 0;
    } else if (S <= 64 && !fused_route_disabled()) {
        // 2. router partials, 3-4. selection and union in one launch (with
        // the four-wave selection, the rows' fragments built beside it)
        const int nch = router_logits(ctx, x_dev, S, m->rw, c.D, c.E, m->logits);
        ColiPrepArgs prep;
        prep.nblocks = 0;
        if (S > 1 && !mx && select_union_mw(c) && prep_beside_enabled() && !flush_frags_args(ctx, fx, &prep))
            return 0;
        if (!nch || !launch_select_union(m, nch, S, st, prep)) return 0;
    } else {
        const int nch = router_logits(ctx, x_dev, S, m->rw, c.D, c.E, m->logits);
        if (!nch || !hip_check(coli_launch_router_select(m->logits, nch, m->rb, S, c.E, c.K, c.route_mode, c.topp,
                                                      c.norm_topk, c.routed_scale, m->idx, m->wsel, m->keff, st),
                            "moe router select"))
            return 0;
        // 4. union
        const size_t ush = (size_t)(7 * c.E + 5) * sizeof(int);
        hipLaunchKernelGGL(coli_moe_union, dim3(1), dim3(1024), ush, st, m->idx, m->keff, S, c.K, c.E, c.has_shared,
                           m->tab, m->pdual, m->pdown, m->uniq, m->xrows, m->slotrow, m->mt, m->state);
        if (!hip_check(hipGetLastError(), "moe union")) return 0;
    }
    // 5. gate/up + SwiGLU over the union, 6. hidden fragments, 7. down
    // (MXFP4 scales folded into the operand when every matrix allows it;
    // re-checked per call, since tensor_update may change the scales)
    bool fold = m->kind == COLI_KIND_FP4;
    for (size_t i = 0; fold && i < m->mats.size(); i++) fold = m->mats[i]->e8_fold != 0;
    if (gateup_done) {
    } else if (gemm) {
        if (!run_gemm(ctx, m->kind, true, m->pdual, P, m->state, m->mt, m->state + 3, moe_tiles(c, S), nrt_i, nq_d,
                      c.I, fx, m->xrows, m->h, c.I, c.swiglu_limit, fold))
            return 0;
    } else if (S == 1 && dual1_enabled() && launch_dual1(m, st, x_dev, nrt_i, nq_d, P, shared_overlap)) {
        if (!hip_check(hipGetLastError(), "moe gate/up")) return 0;
    } else if (!run_gemv(ctx, m->kind, true, m->pdual, P, m->state, nrt_i, nq_d, c.I, S, fx, m->xrows, m->h, c.I,
                         nullptr, c.swiglu_limit, nullptr, nullptr, fold)) {
        return 0;
    }
    // decode, one token: down projection and combine in one launch
    const int pmax = c.K + (c.has_shared ? 1 : 0);
    // (the matrix-core form at an intermediate size of 1024; at 2048 its
    // registers left no more occupancy and the f32 form measured faster)
    const bool fold_all = fold;
    if (!gemm && S == 1 && pmax <= COLI_DC_WAVES && c.I == 1024 && down_combine_enabled() && dc_mfma_enabled()) {
        const dim3 grid((unsigned)nrt_d), block(64 * pmax);
        const size_t shm = (size_t)pmax * c.I * 4;
#define COLI_DCM_LAUNCH(KD, NQ, FD)                                                                         \
    hipLaunchKernelGGL((coli_moe_down_combine1m<KD, NQ, FD>), grid, block, shm, st, m->pdown, m->state, m->h, \
                       c.D, m->wsel, m->keff, m->slotrow, c.K, c.has_shared, out_dev)
        if (fold_all) {
            COLI_DCM_LAUNCH(COLI_KIND_FP4, 8, true);
        } else if (m->kind == COLI_KIND_I4_H) {
            COLI_DCM_LAUNCH(COLI_KIND_I4_H, 8, false);
        } else if (m->kind == COLI_KIND_I4_F) {
            COLI_DCM_LAUNCH(COLI_KIND_I4_F, 8, false);
        } else {
            COLI_DCM_LAUNCH(COLI_KIND_FP4, 8, false);
        }
#undef COLI_DCM_LAUNCH
        return hip_check(hipGetLastError(), "moe down + combine");
    }
    if (!gemm && S == 1 && pmax <= COLI_DC_WAVES && (c.I == 1024 || c.I == 2048) && down_combine_enabled()) {
        const dim3 grid((unsigned)nrt_d), block(64 * pmax);
#define COLI_DC_LAUNCH(KD, NQ)                                                                                  \
    hipLaunchKernelGGL((coli_moe_down_combine1<KD, NQ>), grid, block, 0, st, m->pdown, m->state, m->h, c.D,     \
                       m->wsel, m->keff, m->slotrow, c.K, c.has_shared, out_dev)
#define COLI_DC_KIND(KD)                \
    if (nq_i == 8) COLI_DC_LAUNCH(KD, 8); \
    else COLI_DC_LAUNCH(KD, 16)
        if (m->kind == COLI_KIND_I4_H) { COLI_DC_KIND(COLI_KIND_I4_H); }
        else if (m->kind == COLI_KIND_I4_F) { COLI_DC_KIND(COLI_KIND_I4_F); }
        else { COLI_DC_KIND(COLI_KIND_FP4); }
#undef COLI_DC_KIND
#undef COLI_DC_LAUNCH
        return hip_check(hipGetLastError(), "moe down + combine");
    }
    if (!(mx ? make_frags8(ctx, fh, m->h, c.I, rows, c.I, nullptr, m->state + 1)
             : make_frags(ctx, fh, m->h, c.I, rows, c.I, int4, nullptr, m->state + 1)))
        return 0;
    if (gemm) {
        if (!run_gemm(ctx, m->kind, false, m->pdown, P, m->state, m->mt, m->state + 3, moe_tiles(c, S), nrt_d, nq_i,
                      c.D, fh, nullptr, m->y, c.D, 0.0f, fold))
            return 0;
    } else if (!run_gemv(ctx, m->kind, false, m->pdown, P, m->state, nrt_d, nq_i, c.D, S, fh, nullptr, m->y, c.D,
                         nullptr, 0.0f, nullptr, nullptr, fold)) {
        return 0;
    }
    // 8. combine
    hipLaunchKernelGGL(coli_moe_combine, dim3((c.D + 255) / 256, S), dim3(256), 0, st, m->y, c.D, m->wsel, m->keff,
                       m->slotrow, c.K, m->state, c.has_shared, S, out_dev);
    return hip_check(hipGetLastError(), "moe combine");
}

extern "C" int coli_hip_moe_forward(ColiHipMoe *m, const float *x, float *out, int S, int *idx, float *w,
                                    int *keff) {
    if (fault_injected()) return 0;
    if (!m || !x || !out || S < 1 || S > COLI_MOE_MAX_ROWS) return 0;
    DevCtx *ctx = ctx_of(m->device);
    if (!bind_ctx(ctx)) return 0;
    const ColiHipMoeConfig &c = m->cfg;
    size_t xb = (size_t)S * c.D * sizeof(float);
    if (!reserve(ctx, &ctx->x, xb, 0) || !reserve(ctx, &ctx->y, xb, 0) ||
        !hip_check(hipStreamSynchronize(ctx->stream), "moe staging") ||
        !hip_check(hipMemcpyAsync(ctx->x.p, x, xb, hipMemcpyHostToDevice, ctx->stream), "moe input upload") ||
        !coli_hip_moe_forward_dev(m, (const float *)ctx->x.p, (float *)ctx->y.p, S) ||
        !hip_check(hipMemcpyAsync(out, ctx->y.p, xb, hipMemcpyDeviceToHost, ctx->stream), "moe output download"))
        return 0;
    if (idx && !hip_check(hipMemcpyAsync(idx, m->idx, (size_t)S * c.K * 4, hipMemcpyDeviceToHost, ctx->stream), "idx"))
        return 0;
    if (w && !hip_check(hipMemcpyAsync(w, m->wsel, (size_t)S * c.K * 4, hipMemcpyDeviceToHost, ctx->stream), "w"))
        return 0;
    if (keff && !hip_check(hipMemcpyAsync(keff, m->keff, (size_t)S * 4, hipMemcpyDeviceToHost, ctx->stream), "keff"))
        return 0;
    return hip_check(hipStreamSynchronize(ctx->stream), "moe synchronize");
}

extern "C" int coli_hip_moe_last_union(ColiHipMoe *m, int *nu, int *uniq) {
    if (!m || !nu || !m->state) return 0;
    DevCtx *ctx = ctx_of(m->device);
    if (!bind_ctx(ctx) || !hip_check(hipStreamSynchronize(ctx->stream), "union sync")) return 0;
    int st[3];
    if (!hip_check(hipMemcpy(st, m->state, sizeof(st), hipMemcpyDeviceToHost), "union state")) return 0;
    *nu = st[2];
    if (uniq && st[2] > 0 &&
        !hip_check(hipMemcpy(uniq, m->uniq, (size_t)st[2] * sizeof(int), hipMemcpyDeviceToHost), "union ids"))
        return 0;
    return 1;
}
