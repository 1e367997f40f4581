// backend_hip.hip -- the coli_cuda_* C ABI on gfx950 (libcoli_hip.so).
//
// Host side of the drop-in backend: device contexts, resident tensor upload
// (with the re-layout into MI355X tiles), and the entry points of
// c/backend_cuda.h. Compute is in gemv.hip (quantized GEMV/GEMM), pipe.hip
// (router, elementwise) and moe.hip (fused MoE layer).
#include "coli_hip_internal.h"

#include <atomic>

#include "coli_backend_abi.h"
#include "coli_hip_ext.h"
#include "coli_hip_host.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

DevCtx g_ctx[COLI_CUDA_MAX_DEVICES];

// Fixed device scratch of the allocation-free entry point
// (coli_hip_pipe_gemm_noalloc): each device holds its own copy from module
// load to process end. Host code never passes this name to a kernel or a
// copy: it is a host-side stand-in; the device address comes from
// hipGetSymbolAddress at init (DevCtx::scratch).
static __device__ __align__(256) uint8_t scratch[COLI_NA_BYTES];
int g_nctx;
static std::mutex g_stats_mu;
static uint64_t g_calls, g_experts, g_rows;
static double g_h2d_ms, g_kernel_ms, g_d2h_ms;

// Every HIP status passes through here: a failure is reported once with a
// "[HIP]" tag and the runtime's last-error slot is read back, so a later,
// unrelated call does not see this error again.
int hip_check(hipError_t status, const char *op) {
    if (status != hipSuccess) {
        std::fprintf(stderr, "[HIP] %s: %s\n", op, hipGetErrorString(status));
        (void)hipGetLastError();
    }
    return status == hipSuccess;
}

// Contexts are addressed by HIP device ordinal through a small direct table
// (ordinals beyond it, or not initialised, map to null).
static int8_t g_slot_of_device[64];
static void map_device_slots(void) {
    std::memset(g_slot_of_device, -1, sizeof(g_slot_of_device));
    for (int i = 0; i < g_nctx; i++)
        if (g_ctx[i].device >= 0 && g_ctx[i].device < 64) g_slot_of_device[g_ctx[i].device] = (int8_t)i;
}

DevCtx *ctx_of(int device) {
    if (device < 0 || device >= 64 || g_nctx == 0) return nullptr;
    const int slot = g_slot_of_device[device];
    return slot < 0 ? nullptr : &g_ctx[slot];
}

// Make ctx's device the calling thread's HIP device. The runtime keeps the
// current device per host thread; asking it first is cheaper than setting it
// on every entry point (the expert loop calls in once per layer and expert).
int bind_ctx(DevCtx *ctx) {
    if (!ctx) return 0;
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur == ctx->device) return 1;
    return hip_check(hipSetDevice(ctx->device), "select device");
}

// Test hook of the reference ABI (c/backend_cuda.cu:1340-1348): while
// COLI_GPU_FAIL_AFTER=N is set, every compute entry point reports failure
// once N compute calls have been made with it set (N = 0: all of them);
// uploads and queries are not gated, and unsetting it restores normal
// operation. The count of armed calls is shared by all threads.
static std::atomic<long> g_armed_compute_calls{0};
int fault_injected(void) {
    const char *budget = std::getenv("COLI_GPU_FAIL_AFTER");
    if (budget == nullptr) return 0;
    const long allowed = std::strtol(budget, nullptr, 10);
    return g_armed_compute_calls.fetch_add(1, std::memory_order_relaxed) >= allowed;
}

// Grow-only device buffer. Growing waits for the stream first, because queued
// work may still read the old allocation.
int reserve(DevCtx *ctx, DevBuf *b, size_t bytes, int zero) {
    if (bytes <= b->cap) return 1;
    if (b->p) {
        if (!hip_check(hipStreamSynchronize(ctx->stream), "reserve sync")) return 0;
        (void)hipFree(b->p);
        b->p = nullptr;
        b->cap = 0;
    }
    size_t want = bytes + bytes / 4 + 256;
    if (!hip_check(hipMalloc(&b->p, want), "scratch allocation")) return 0;
    if (zero && !hip_check(hipMemset(b->p, 0, want), "scratch clear")) return 0;
    b->cap = want;
    return 1;
}

int reserve_pinned(DevCtx *ctx, PinBuf *b, size_t bytes) {
    if (bytes <= b->cap) return 1;
    if (b->h) {
        if (!hip_check(hipStreamSynchronize(ctx->stream), "pinned reserve sync")) return 0;
        (void)hipHostFree(b->h);
        *b = PinBuf{};
    }
    const size_t want = bytes + bytes / 4 + 256;
    void *h = nullptr, *d = nullptr;
    if (!hip_check(hipHostMalloc(&h, want, hipHostMallocDefault), "pinned allocation")) return 0;
    if (!hip_check(hipHostGetDevicePointer(&d, h, 0), "pinned buffer device pointer")) {
        (void)hipHostFree(h);
        return 0;
    }
    b->h = h;
    b->d = d;
    b->cap = want;
    return 1;
}

static void free_buf(DevBuf *b) {
    if (b->p) (void)hipFree(b->p);
    b->p = nullptr;
    b->cap = 0;
}

// ---------------------------------------------------------------------------
// lifecycle (c/backend_cuda.cu:929-1040)
// ---------------------------------------------------------------------------
extern "C" int coli_cuda_init(const int *devices, int count) {
    int available = 0;
    if (!devices || count < 1 || count > COLI_CUDA_MAX_DEVICES) return 0;
    if (!hip_check(hipGetDeviceCount(&available), "device discovery")) return 0;
    if (g_nctx) coli_cuda_shutdown();
    map_device_slots();
    for (int i = 0; i < count; i++) {
        int device = devices[i];
        if (device < 0 || device >= available) {
            std::fprintf(stderr, "[HIP] invalid device %d (available: 0..%d)\n", device, available - 1);
            g_nctx = 0;
            return 0;
        }
        bool dup = false;
        for (int j = 0; j < i; j++) dup |= devices[j] == device;
        if (dup) {
            std::fprintf(stderr, "[HIP] duplicate device %d\n", device);
            g_nctx = 0;
            return 0;
        }
        DevCtx *ctx = &g_ctx[g_nctx];
        *ctx = DevCtx();
        ctx->device = device;
        if (!bind_ctx(ctx)) { g_nctx = 0; return 0; }
        hipDeviceProp_t prop{};
        if (!hip_check(hipGetDeviceProperties(&prop, device), "device properties")) { g_nctx = 0; return 0; }
        ctx->cu_count = prop.multiProcessorCount;
        if (!hip_check(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "stream creation")) {
            g_nctx = 0;
            return 0;
        }
        if (!reserve(ctx, &ctx->flags, 64 * sizeof(int), 1) || !reserve(ctx, &ctx->zeros, COLI_ZERO_BYTES, 1)) {
            g_nctx = 0;
            return 0;
        }
        // this device's copy of the static scratch, cleared (zero block, lo
        // flag, split-K counters must start at zero): with a fill kernel on
        // the stream, then waited for
        void *sp = nullptr;
        if (hip_check(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)), "scratch symbol address") &&
            hip_check(coli_launch_zero_i32((int *)sp, (int)(COLI_NA_BYTES / sizeof(int)), ctx->stream), "scratch clear") &&
            hip_check(hipStreamSynchronize(ctx->stream), "scratch clear sync"))
            ctx->scratch = (uint8_t *)sp;
        g_nctx++;
        map_device_slots();
        std::fprintf(stderr, "[HIP] device %d: %s (%s), %.1f GB HBM, %d CUs\n", device, prop.name,
                     prop.gcnArchName, prop.totalGlobalMem / 1e9, prop.multiProcessorCount);
    }
    return 1;
}

extern "C" void coli_cuda_shutdown(void) {
    for (int i = 0; i < g_nctx; i++) {
        DevCtx *ctx = &g_ctx[i];
        if (!bind_ctx(ctx)) continue;
        (void)hipStreamSynchronize(ctx->stream);
        DevBuf *bufs[] = {&ctx->x, &ctx->h, &ctx->y, &ctx->g, &ctx->u, &ctx->partial,
                          &ctx->prob, &ctx->stage_w, &ctx->stage_s, &ctx->qdq, &ctx->flags,
                          &ctx->rslot, &ctx->rw, &ctx->tmp_tiles, &ctx->tmp_scales, &ctx->zeros,
                          &ctx->split_cnt, &ctx->idot_y, &ctx->idot_sx};
        for (DevBuf *b : bufs) free_buf(b);
        for (int f = 0; f < 4; f++) {
            free_buf(&ctx->frag[f].hi);
            free_buf(&ctx->frag[f].lo);
            free_buf(&ctx->frag[f].exp);
        }
        for (int s = 0; s < COLI_PIPE_SLOTS; s++) free_buf(&ctx->pipe[s]);
        if (ctx->host_x.h) (void)hipHostFree(ctx->host_x.h);
        if (ctx->host_y.h) (void)hipHostFree(ctx->host_y.h);
        if (ctx->host_prob.h) (void)hipHostFree(ctx->host_prob.h);
        if (ctx->host_small.h) (void)hipHostFree(ctx->host_small.h);
        if (ctx->ev_ok) (void)hipEventDestroy(ctx->ev_done);
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
        *ctx = DevCtx();
    }
    g_nctx = 0;
    map_device_slots();
}

extern "C" int coli_cuda_device_count(void) { return g_nctx; }
extern "C" int coli_cuda_device_at(int index) { return index >= 0 && index < g_nctx ? g_ctx[index].device : -1; }

extern "C" int coli_cuda_mem_info(int device, size_t *free_bytes, size_t *total_bytes) {
    DevCtx *ctx = ctx_of(device);
    if (!free_bytes || !total_bytes || !bind_ctx(ctx)) return 0;
    return hip_check(hipMemGetInfo(free_bytes, total_bytes), "memory info");
}

extern "C" int coli_cuda_device_integrated(int device) {
    hipDeviceProp_t prop{};
    if (!hip_check(hipGetDeviceProperties(&prop, device), "device properties")) return 0;
    return prop.integrated ? 1 : 0;
}

extern "C" void coli_cuda_stats(int device, size_t *tensor_count, size_t *tensor_bytes) {
    size_t count = 0, bytes = 0;
    for (int i = 0; i < g_nctx; i++)
        if (device < 0 || g_ctx[i].device == device) {
            count += g_ctx[i].tensor_count;
            bytes += g_ctx[i].tensor_bytes;
        }
    if (tensor_count) *tensor_count = count;
    if (tensor_bytes) *tensor_bytes = bytes;
}

extern "C" void coli_cuda_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows, double *h2d_ms,
                                      double *kernel_ms, double *d2h_ms) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    if (calls) *calls = g_calls;
    if (experts) *experts = g_experts;
    if (rows) *rows = g_rows;
    if (h2d_ms) *h2d_ms = g_h2d_ms;
    if (kernel_ms) *kernel_ms = g_kernel_ms;
    if (d2h_ms) *d2h_ms = g_d2h_ms;
}

extern "C" void coli_cuda_group_stats_device(int device, uint64_t *calls, uint64_t *experts, uint64_t *rows,
                                             double *h2d_ms, double *kernel_ms, double *d2h_ms) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    DevCtx *ctx = ctx_of(device);
    if (calls) *calls = ctx ? ctx->st_calls : 0;
    if (experts) *experts = ctx ? ctx->st_experts : 0;
    if (rows) *rows = ctx ? ctx->st_rows : 0;
    if (h2d_ms) *h2d_ms = ctx ? ctx->st_h2d : 0;
    if (kernel_ms) *kernel_ms = ctx ? ctx->st_kernel : 0;
    if (d2h_ms) *d2h_ms = ctx ? ctx->st_d2h : 0;
}

void note_group(DevCtx *ctx, int count, int total, double h2d, double ker, double d2h) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_calls++;
    g_experts += (uint64_t)count;
    g_rows += (uint64_t)total;
    g_h2d_ms += h2d;
    g_kernel_ms += ker;
    g_d2h_ms += d2h;
    ctx->st_calls++;
    ctx->st_experts += (uint64_t)count;
    ctx->st_rows += (uint64_t)total;
    ctx->st_h2d += h2d;
    ctx->st_kernel += ker;
    ctx->st_d2h += d2h;
}

// fmt 6 (E8) and fmt 8 (fp8) are not computed here: the tables are refused
// so the engine keeps those formats on its CPU path.
extern "C" int coli_cuda_e8_set_grid(const void *) { return 0; }
extern "C" int coli_cuda_fp8_set_lut(const float *) { return 0; }

// ---------------------------------------------------------------------------
// tensors
// ---------------------------------------------------------------------------
static int scales_fp16_exact(const float *s, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float v = s[i];
        if (!std::isfinite(v)) return 0;
        _Float16 h = (_Float16)v;
        if ((float)h != v) return 0;
    }
    return 1;
}

// f32 power-of-two scales -> e8m0 bytes (s with (u32)s << 23 == bits):
// +0 -> 0, +inf -> 255, 2^(s-127) for s in 1..254; anything else refused.
static int scales_to_e8(const float *s, size_t n, uint8_t *out) {
    for (size_t i = 0; i < n; i++) {
        uint32_t bits;
        std::memcpy(&bits, &s[i], 4);
        if (bits & 0x807fffffu) return 0;
        out[i] = (uint8_t)(bits >> 23);
    }
    return 1;
}

static size_t src_scale_count(int fmt, int I, int O, int gs) {
    if (fmt == 7) return (size_t)O * ((I + 31) / 32);
    if (fmt == 4 && gs > 0) return (size_t)O * ((I + gs - 1) / gs);
    return (size_t)O;
}

// Copy source bytes to the device and build the tiled layout of t.
static int fill_tensor(DevCtx *ctx, ColiCudaTensor *t, const void *weights, const void *scales_src,
                       size_t scale_src_bytes, int w_on_device = 0) {
    size_t rb = (size_t)(t->I + 1) / 2, wsrc = rb * t->O;
    hipMemcpyKind wkind = w_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    if (t->kind == COLI_KIND_GENERIC) {
        if (!hip_check(hipMemcpy(t->w, weights, wsrc, wkind), "tensor upload") ||
            !hip_check(hipMemcpy(t->sc, scales_src, scale_src_bytes, hipMemcpyHostToDevice), "scale upload"))
            return 0;
        return 1;
    }
    if ((!w_on_device && !reserve(ctx, &ctx->stage_w, wsrc, 0)) || !reserve(ctx, &ctx->stage_s, scale_src_bytes, 0))
        return 0;
    if (!hip_check(hipStreamSynchronize(ctx->stream), "upload sync") ||
        (!w_on_device && !hip_check(hipMemcpy(ctx->stage_w.p, weights, wsrc, hipMemcpyHostToDevice), "tensor upload")) ||
        !hip_check(hipMemcpy(ctx->stage_s.p, scales_src, scale_src_bytes, hipMemcpyHostToDevice), "scale upload"))
        return 0;
    if (t->kind == COLI_KIND_FP4) {
        // 0.5 * 2^(e-127) >= 2^-14 and 6 * 2^(e-127) <= 65504
        const uint8_t *e8 = (const uint8_t *)scales_src;
        int fold = 1;
        for (size_t i = 0; i < scale_src_bytes && fold; i++) fold = e8[i] >= 114 && e8[i] <= 140;
        t->e8_fold = fold;
    }
    const uint8_t *wsrc_dev = w_on_device ? (const uint8_t *)weights : (const uint8_t *)ctx->stage_w.p;
    if (!hip_check(coli_launch_repack(t, wsrc_dev, ctx->stage_s.p, ctx->stream),
                "tile repack"))
        return 0;
    return hip_check(hipStreamSynchronize(ctx->stream), "tile repack sync");
}

static ColiCudaTensor *alloc_tensor(DevCtx *ctx, int fmt, int I, int O, int gs, int kind) {
    ColiCudaTensor *t = (ColiCudaTensor *)std::calloc(1, sizeof(ColiCudaTensor));
    if (!t) return nullptr;
    t->fmt = fmt; t->I = I; t->O = O; t->device = ctx->device; t->gs = gs; t->kind = kind;
    if (kind == COLI_KIND_GENERIC) {
        t->ng_src = (I + gs - 1) / gs;
        t->w_bytes = (size_t)(I + 1) / 2 * O;
        t->sc_bytes = (size_t)O * t->ng_src * sizeof(float);
    } else {
        t->Op = (O + 15) / 16 * 16;
        t->Ip = (I + 127) / 128 * 128;
        t->nrt = t->Op / 16;
        t->nq = t->Ip / 128;
        t->w_bytes = (size_t)t->nrt * t->nq * COLI_TILE_BYTES;
        size_t per = kind == COLI_KIND_I4_H ? 2 : (kind == COLI_KIND_I4_F ? 4 : 1);
        t->sc_bytes = (size_t)t->nrt * t->nq * 64 * per;
    }
    if (!hip_check(hipMalloc((void **)&t->w, t->w_bytes), "tensor allocation") ||
        !hip_check(hipMalloc(&t->sc, t->sc_bytes), "scale allocation")) {
        if (t->w) (void)hipFree(t->w);
        std::free(t);
        return nullptr;
    }
    if (kind != COLI_KIND_GENERIC) {
        ColiProb d[COLI_DESC_ROWS];
        for (int r = 0; r < COLI_DESC_ROWS; r++) d[r] = {t->w, t->sc, nullptr, nullptr, r + 1, 0, 0, 0};
        if (!hip_check(hipMalloc((void **)&t->desc, sizeof(d)), "descriptor allocation") ||
            !hip_check(hipMemcpy(t->desc, d, sizeof(d), hipMemcpyHostToDevice), "descriptor upload")) {
            (void)hipFree(t->w);
            (void)hipFree(t->sc);
            if (t->desc) (void)hipFree(t->desc);
            std::free(t);
            return nullptr;
        }
    }
    t->accounted = t->w_bytes + t->sc_bytes;
    ctx->tensor_count++;
    ctx->tensor_bytes += t->accounted;
    return t;
}

// Upload for fmt 2 / 4 (f32 scales) and fmt 7 (e8 bytes, or f32 powers of two).
int upload_impl(ColiCudaTensor **tensor, const void *weights, const float *scales, const uint8_t *e8,
                int fmt, int I, int O, int device, int gs, int w_on_device) {
    if (!tensor) return 0;
    int want_gs = (fmt == 4 && gs > 0) ? gs : (fmt == 7 ? 32 : 0);
    if (*tensor) {
        ColiCudaTensor *t = *tensor;
        return t->fmt == fmt && t->I == I && t->O == O && t->device == device && t->gs == want_gs;
    }
    DevCtx *ctx = ctx_of(device);
    if (!weights || I < 1 || O < 1 || !bind_ctx(ctx)) return 0;
    if (fmt != 2 && fmt != 4 && fmt != 7) return 0;
    if (fmt == 7) {
        if (!e8 && !scales) return 0;
        if (!e8 && gs != 32 && gs != 0) return 0;
    } else if (!scales) {
        return 0;
    }
    size_t ns = src_scale_count(fmt, I, O, want_gs);
    std::vector<uint8_t> e8buf;
    int kind;
    const void *ssrc;
    size_t sbytes;
    if (fmt == 7) {
        kind = COLI_KIND_FP4;
        if (!e8) {
            e8buf.resize(ns);
            if (!scales_to_e8(scales, ns, e8buf.data())) {
                std::fprintf(stderr, "[HIP] fmt=7 upload: scales are not exact powers of two\n");
                return 0;
            }
            e8 = e8buf.data();
        }
        ssrc = e8;
        sbytes = ns;
    } else {
        if (want_gs > 0 && want_gs % 32) kind = COLI_KIND_GENERIC;
        else kind = scales_fp16_exact(scales, ns) ? COLI_KIND_I4_H : COLI_KIND_I4_F;
        ssrc = scales;
        sbytes = ns * sizeof(float);
    }
    ColiCudaTensor *t = alloc_tensor(ctx, fmt, I, O, want_gs, kind);
    if (!t) return 0;
    if (!fill_tensor(ctx, t, weights, ssrc, sbytes, w_on_device)) {
        coli_cuda_tensor_free(t);
        return 0;
    }
    *tensor = t;
    return 1;
}

extern "C" int coli_cuda_tensor_upload_g(ColiCudaTensor **tensor, const void *weights, const float *scales,
                                         int fmt, int I, int O, int device, int gs) {
    return upload_impl(tensor, weights, scales, nullptr, fmt, I, O, device, gs > 0 ? gs : 0, 0);
}

extern "C" int coli_cuda_tensor_upload(ColiCudaTensor **tensor, const void *weights, const float *scales,
                                       int fmt, int I, int O, int device) {
    return upload_impl(tensor, weights, scales, nullptr, fmt, I, O, device, fmt == 7 ? 32 : 0, 0);
}

extern "C" int coli_hip_tensor_upload_mxfp4(ColiCudaTensor **tensor, const unsigned char *q4,
                                            const unsigned char *e8, int I, int O, int device) {
    if (!e8) return 0;
    return upload_impl(tensor, q4, nullptr, e8, 7, I, O, device, 32, 0);
}

extern "C" int coli_hip_tensor_upload_fp4_rows16(ColiCudaTensor **tensor, const unsigned char *pd,
                                                 const unsigned char *ps, int I, int O, int device) {
    if (!tensor || *tensor || !pd || !ps || O < 16 || O % 16 || I < 128 || I % 128) return 0;
    DevCtx *ctx = ctx_of(device);
    if (!bind_ctx(ctx)) return 0;
    // The 16-row interleave (c/deepseek_v4.c:10975-10993) is undone on the
    // device, into row-major bytes the tiled repack then reads from device
    // memory; the e8m0 scales (1/16 of the bytes) are de-interleaved here.
    const size_t ds = (size_t)I / 2, ss = (size_t)I / 32, wb = (size_t)O * ds;
    std::vector<uint8_t> e8((size_t)O * ss);
    for (size_t r = 0; r < (size_t)O; r++)
        for (size_t c = 0; c < ss; c++) e8[r * ss + c] = ps[((r / 16) * ss + c) * 16 + r % 16];
    if (!reserve(ctx, &ctx->stage_w, 2 * wb, 0) || !hip_check(hipStreamSynchronize(ctx->stream), "rows16 staging") ||
        !hip_check(hipMemcpy(ctx->stage_w.p, pd, wb, hipMemcpyHostToDevice), "rows16 upload"))
        return 0;
    uint8_t *rows = (uint8_t *)ctx->stage_w.p + wb;
    if (!hip_check(coli_launch_rows16_to_rows((const uint8_t *)ctx->stage_w.p, rows, O, (int)ds, ctx->stream),
                   "rows16 de-interleave") ||
        !hip_check(hipStreamSynchronize(ctx->stream), "rows16 de-interleave sync"))
        return 0;
    return upload_impl(tensor, rows, nullptr, e8.data(), 7, I, O, device, 32, 1);
}

extern "C" int coli_hip_tensor_upload_from_device(ColiCudaTensor **tensor, const void *weights_dev,
                                                  const float *scales, const unsigned char *e8, int fmt, int I,
                                                  int O, int device, int gs) {
    if (!tensor || *tensor) return 0;   // a fresh tensor only: no cached-handle reuse here
    if (fmt == 7 && !e8) return 0;
    return upload_impl(tensor, weights_dev, fmt == 7 ? nullptr : scales, fmt == 7 ? e8 : nullptr, fmt, I, O, device,
                       fmt == 7 ? 32 : (gs > 0 ? gs : 0), 1);
}

extern "C" void coli_cuda_tensor_free(ColiCudaTensor *t) {
    if (!t) return;
    DevCtx *ctx = ctx_of(t->device);
    if (ctx) {
        bind_ctx(ctx);
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->tensor_count) ctx->tensor_count--;
        if (ctx->tensor_bytes >= t->accounted) ctx->tensor_bytes -= t->accounted;
    }
    if (t->w) (void)hipFree(t->w);
    if (t->sc) (void)hipFree(t->sc);
    if (t->desc) (void)hipFree(t->desc);
    if (t->sc_unit) (void)hipFree(t->sc_unit);
    std::free(t);
}

extern "C" size_t coli_cuda_tensor_bytes(const ColiCudaTensor *t) { return t ? t->w_bytes + t->sc_bytes : 0; }
extern "C" int coli_cuda_tensor_device(const ColiCudaTensor *t) { return t ? t->device : -1; }
extern "C" size_t coli_hip_tensor_stream_bytes(const ColiCudaTensor *t) { return t ? t->w_bytes + t->sc_bytes : 0; }
extern "C" int coli_hip_tensor_kind(const ColiCudaTensor *t) { return t ? t->kind : -1; }

extern "C" int coli_cuda_tensor_update(ColiCudaTensor *t, const void *weights, const float *scales) {
    if (!t || !weights || !scales) return 0;
    DevCtx *ctx = ctx_of(t->device);
    if (!bind_ctx(ctx)) return 0;
    size_t ns = src_scale_count(t->fmt, t->I, t->O, t->gs);
    if (t->kind == COLI_KIND_FP4) {
        std::vector<uint8_t> e8(ns);
        if (!scales_to_e8(scales, ns, e8.data())) return 0;
        return fill_tensor(ctx, t, weights, e8.data(), ns);
    }
    // The storage kind was fixed at upload: fp16 storage needs fp16-exact scales.
    if (t->kind == COLI_KIND_I4_H && !scales_fp16_exact(scales, ns)) {
        std::fprintf(stderr, "[HIP] tensor_update: scales no longer fp16-exact for an fp16-scale tensor\n");
        return 0;
    }
    return fill_tensor(ctx, t, weights, scales, ns * sizeof(float));
}

extern "C" int coli_hip_fill_random_u8(int device, void *dev, size_t n, unsigned long long seed) {
    DevCtx *ctx = ctx_of(device);
    if (!dev || !bind_ctx(ctx)) return 0;
    return hip_check(coli_launch_fill_random(dev, n, seed, ctx->stream), "random fill") &&
           hip_check(hipStreamSynchronize(ctx->stream), "random fill sync");
}

extern "C" int coli_hip_stream_read(int device, const void *dev, size_t bytes) {
    DevCtx *ctx = ctx_of(device);
    if (!dev || !bind_ctx(ctx)) return 0;
    return hip_check(coli_launch_stream_read(dev, bytes, ctx->stream), "stream read");
}

extern "C" void *coli_hip_stream(int device) {
    DevCtx *ctx = ctx_of(device);
    return ctx ? (void *)ctx->stream : nullptr;
}
