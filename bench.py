#!/usr/bin/env python3
"""Benchmark of the quantized MoE expert hot path on one MI355X.

Headline (BASELINE.json metric "expert GEMV HBM GB/s (% of 8 TB/s peak) +
MoE-layer tokens/s, 1 GPU"):

  value      = algorithmic GB/s of the dense int4-g32 GEMV workload of
               W_up 14336x4096 then W_down 4096x14336 (Llama-8B
               FFN shape), at batch 1, 4, 8 and 16. One step = the up and
               down GEMV at each of the four batch sizes (8 GEMVs), inputs
               resident in HBM. Weight copies rotate through >= 2 GB of
               distinct memory so the 256 MB MALL cannot serve them.
  roofline   = the GEMV kernel alone (coli_gemv_tiles), bracketed by HIP
               events on the backend stream, against 8 TB/s.
  moe_layer  = tokens/s of one fused MoE layer (router -> union -> experts
               -> SwiGLU -> scatter) for configs[0] (OLMoE-shaped, int4) and
               configs[2] (DeepSeek-V3-shaped, MXFP4, + shared expert).
  cpu_baseline = the reference's own OpenMP CPU kernel (c/quant.h
               matmul_i4_grouped, compiled from its sources into
               oracle/_ref) on this host's cores, bounded sample.

Algorithmic bytes per GEMV = O*I/2 nibble bytes + O*I/32 scales (2 bytes
fp16 for int4, 1 byte e8m0 for MXFP4) + bf16 activations in and out; each
weight byte counted once per call. Synthetic data, seeded.
"""
import argparse
import ctypes as C
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0
BATCHES = (1, 4, 8, 16)
UP = (14336, 4096)      # (O, I)
DOWN = (4096, 14336)
METRIC = "expert GEMV HBM GB/s (% of 8 TB/s peak) + MoE-layer tokens/s, 1 GPU"


def bytes_i4(O, I, B):
    return O * I // 2 + O * (I // 32) * 2 + B * I * 2 + B * O * 2


def bytes_fp4(O, I, B):
    return O * I // 2 + O * (I // 32) + B * I * 2 + B * O * 2


def bf16_exact(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def fp16_scales(rng, O, ng):
    return np.abs(rng.standard_normal((O, ng)) * 0.01).astype(np.float16).astype(np.float32)


def cpu_baseline(secs):
    """The reference's CPU path on this host (as the reference publishes its
    CPU numbers: OpenMP over the physical cores, OMP_PROC_BIND=close, set in
    main() before any OpenMP library loads): the dense int4 step of configs[1] (`value`), plus an
    MXFP4 expert GEMV leg (configs[2] shapes) and an OLMoE-shaped MoE layer
    leg (configs[0], the reference's kernels composed in the order of
    c/olmoe.c:645-697). It runs in a child process of its own that never
    loads the HIP runtime (main()), so the OpenMP runtime and the GPU runtime
    (and a profiler's preloaded tool library) never share a process. Inputs are
    the workload's shapes and distributions from numpy's generator: the CPU
    time does not depend on the values."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_lib import REF_PATH, Ref, Cref
    kind = "reference" if os.path.exists(REF_PATH) else "port"
    lib = Ref() if kind == "reference" else Cref()
    cref = Cref()
    rng = np.random.default_rng(4242)
    (qu, su), (qd, sd) = [(rng.integers(0, 256, (O, I // 2), dtype=np.uint8), fp16_scales(rng, O, I // 32))
                          for O, I in (UP, DOWN)]
    cpu_x = bf16_exact(rng.standard_normal((16, UP[1])).astype(np.float32))
    h = np.empty((16, UP[0]), np.float32)

    def timed(fn):
        fn()                          # warm the page cache / thread pool
        t0 = time.perf_counter()
        work, reps = 0, 0
        while time.perf_counter() - t0 < secs:
            work += fn()
            reps += 1
        return work, reps, time.perf_counter() - t0

    def dense_pass():
        nbytes = 0
        for B in BATCHES:
            xb = np.ascontiguousarray(cpu_x[:B])
            h[:B] = lib.matmul_i4_grouped(xb, qu, su, UP[0], UP[1], 32)
            lib.matmul_i4_grouped(np.ascontiguousarray(h[:B]), qd, sd, DOWN[0], DOWN[1], 32)
            nbytes += bytes_i4(*UP, B) + bytes_i4(*DOWN, B)
        return nbytes

    nbytes, reps, dt = timed(dense_pass)
    out = {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": CPU_INFO["threads"], "kind": kind,
           "sample": f"{reps} passes of the bench step (up+down GEMV at batch 1/4/8/16) over one "
                     f"weight copy, {dt:.1f} s, c/quant.h matmul_i4_grouped (OpenMP)",
           "ms_per_step": round(dt / reps * 1e3, 2), "cpu": CPU_INFO}
    # MXFP4 expert GEMV, DeepSeek-V3 expert shapes (gate/up 2048x7168, down 7168x2048), batch 1
    mats = [(rng.integers(0, 256, (O, I // 2), dtype=np.uint8), rng.integers(119, 124, (O, I // 32), dtype=np.uint8),
             O, I) for O, I in ((2048, 7168), (7168, 2048))]
    x1 = {I: bf16_exact(rng.standard_normal((1, I)).astype(np.float32)) for I in (7168, 2048)}

    def mx_pass():
        nb = 0
        for q4, e8, O, I in mats:
            lib.matmul_mxfp4(x1[I], q4, e8, O, I)
            nb += bytes_fp4(O, I, 1)
        return nb

    nb, reps, dt = timed(mx_pass)
    out["mxfp4_gemv"] = {"value": round(nb / dt / 1e9, 3), "unit": "GB/s", "kind": kind,
                         "sample": f"{reps} x (2048x7168 + 7168x2048) matmul_mxfp4 at batch 1, {dt:.1f} s"}
    # OLMoE-shaped MoE layer: 64 int4 experts, top-8 softmax, batch 1
    D, I, E, K = 2048, 1024, 64, 8
    experts = []
    for _ in range(E):
        trip = []
        for O, II in ((I, D), (I, D), (D, I)):
            trip.append((rng.integers(0, 256, (O, II // 2), dtype=np.uint8), fp16_scales(rng, O, II // 32)))
        experts.append(tuple(trip))
    W = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)
    xs = bf16_exact(rng.standard_normal((64, D)).astype(np.float32))
    state = {"i": 0}

    def moe_pass():
        # the reference's kernels for the router GEMV and the experts
        # (c/olmoe.c:645-697 order): softmax top-8, silu(gate) * up, down,
        # weighted sum in slot order
        r = state["i"] % 64
        state["i"] += 1
        x = xs[r:r + 1]
        logits = lib.matmul_f32(x, W)
        idx, w, keff = cref.route(logits, K, 0)
        acc = np.zeros(D, np.float32)
        for kk in range(keff[0]):
            (gq, gs), (uq, us), (dq, dsc) = experts[idx[0, kk]]
            g = lib.matmul_i4_grouped(x, gq, gs, I, D, 32)
            u = lib.matmul_i4_grouped(x, uq, us, I, D, 32)
            hid = cref.swiglu(g, u)
            acc += w[0, kk] * lib.matmul_i4_grouped(hid, dq, dsc, D, I, 32)[0]
        return 1

    toks, reps, dt = timed(moe_pass)
    out["moe_layer_olmoe_int4"] = {"value": round(toks / dt, 1), "unit": "tokens/s", "kind": kind,
                                   "sample": f"{reps} single-token layers (router GEMV + top-8 + 8 experts on "
                                             f"the reference's c/quant.h kernels), {dt:.1f} s"}
    return out


def cpu_baseline_child(secs):
    """Runs cpu_baseline() in a child process started before this process
    touches the GPU, and returns its JSON result."""
    import subprocess
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", "--cpu-seconds", str(secs)],
                       capture_output=True, text=True, env=dict(os.environ), timeout=secs * 6 + 120)
    if r.returncode != 0:
        raise RuntimeError(f"CPU baseline child failed ({r.returncode}): {r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


class Bench:
    def __init__(self, args):
        from colibri_amd.backend import Session
        from colibri_amd import hiprt
        self.args = args
        self.hiprt = hiprt
        self.s = Session(0)
        self.b = self.s.b
        self.stream = self.b.hip_stream(0)
        self.rng = np.random.default_rng(1234)
        self.allocs = []

    def alloc(self, nbytes):
        p = self.b.cuda_pipe_alloc(0, nbytes)
        if not p:
            raise RuntimeError("device allocation failed")
        self.allocs.append(p)
        return p

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes)
        if not self.b.cuda_pipe_upload(0, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes):
            raise RuntimeError("upload failed")
        return p

    # -- tensors with device-generated weights ------------------------------
    def tensor_i4(self, stage, O, I, scales, seed):
        nb = O * ((I + 1) // 2)
        assert self.b.hip_fill_random_u8(0, stage, nb, seed)
        h = C.c_void_p()
        from colibri_amd.backend import f32p
        sc = np.ascontiguousarray(scales, np.float32)
        if not self.b.hip_tensor_upload_from_device(C.byref(h), stage, f32p(sc), None, 4, I, O, 0, 32):
            raise RuntimeError("upload_from_device (int4) failed")
        return h

    def tensor_fp4(self, stage, O, I, e8, seed):
        nb = O * ((I + 1) // 2)
        assert self.b.hip_fill_random_u8(0, stage, nb, seed)
        h = C.c_void_p()
        from colibri_amd.backend import u8p
        e8 = np.ascontiguousarray(e8, np.uint8)
        if not self.b.hip_tensor_upload_from_device(C.byref(h), stage, None, u8p(e8), 7, I, O, 0, 32):
            raise RuntimeError("upload_from_device (mxfp4) failed")
        return h

    # -- dense GEMV ---------------------------------------------
    def dense(self):
        b, hrt = self.b, self.hiprt
        pair = bytes_i4(*UP, 0) + bytes_i4(*DOWN, 0)
        copies = max(2, math.ceil(self.args.anticache_gb * 1e9 / pair))
        stage = self.alloc(UP[0] * UP[1] // 2)
        sc_up = fp16_scales(self.rng, UP[0], UP[1] // 32)
        sc_dn = fp16_scales(self.rng, DOWN[0], DOWN[1] // 32)
        ups, downs = [], []
        for c in range(copies):
            ups.append(self.tensor_i4(stage, *UP, np.roll(sc_up, 7 * c, axis=0), 2 * c + 1))
            downs.append(self.tensor_i4(stage, *DOWN, np.roll(sc_dn, 7 * c, axis=0), 2 * c + 2))
        x = bf16_exact(self.rng.standard_normal((16, UP[1])).astype(np.float32))
        xd = self.put(x)
        hd = self.alloc(16 * UP[0] * 4)
        yd = self.alloc(16 * DOWN[0] * 4)
        K, W = self.args.steps, self.args.warmup
        state = {"c": 0}

        def step():
            for B in BATCHES:
                c = state["c"] % copies
                state["c"] += 1
                ok = b.hip_gemm_prep_dev(ups[c], xd, B)
                # the up GEMV also writes h as the down GEMV's fragments
                # (from its epilogue) where that replaces a fragment build
                # (returns 2 then, 1 when it ran alone)
                ok = ok and b.hip_gemm_run_dev_emit(ups[c], hd, B, downs[c])
                ok = ok and b.hip_gemm_prep_dev(downs[c], hd, B)
                ok = ok and b.hip_gemm_run_dev(downs[c], yd, B)
                if not ok:
                    raise RuntimeError("GEMV launch failed")

        for _ in range(W):
            step()
        hrt.device_sync()
        # The K timed steps are captured once into a HIP graph and replayed:
        # the host enqueues one graph instead of 16 calls per step, so the GPU
        # is never starved by the Python driver. The first replay warms up;
        # the second is timed (wall clock and HIP events on the backend
        # stream around it).
        state["c"] = 0
        with hrt.Graph(self.stream) as graph:
            for _ in range(K):
                step()
        graph.launch()
        hrt.device_sync()
        e0, e1 = hrt.Event(), hrt.Event()
        t0 = time.perf_counter()
        e0.record(self.stream)
        graph.launch()
        e1.record(self.stream)
        hrt.device_sync()
        wall = time.perf_counter() - t0
        gpu_ms = e0.elapsed_ms(e1)
        step_bytes = sum(bytes_i4(*UP, B) + bytes_i4(*DOWN, B) for B in BATCHES)

        # GEMV kernel alone (the roofline figure): per batch size and shape, a
        # graph of back-to-back GEMV launches over all weight copies, timed
        # with events around the replay; the activation fragments they read
        # were built once beforehand.
        by_batch = {}
        kern_bytes, kern_ms, kern_n = 0.0, 0.0, 0
        for B in BATCHES:
            rec = {}
            for name, mats, (O, I), xin, yout in (("up", ups, UP, xd, hd), ("down", downs, DOWN, hd, yd)):
                # each kernel as the step runs it: up with its epilogue
                # emitting h, down on the emitted fragments (where the step
                # emits them)
                if name == "down":
                    assert b.hip_gemm_prep_dev(ups[0], xd, B)
                    assert b.hip_gemm_run_dev_emit(ups[0], hd, B, downs[0])
                assert b.hip_gemm_prep_dev(mats[0], xin, B)
                run = ((lambda m: b.hip_gemm_run_dev_emit(m, yout, B, downs[0])) if name == "up"
                       else (lambda m: b.hip_gemm_run_dev(m, yout, B)))
                # the first run launches any deferred fragment prep, outside the graph
                assert run(mats[0])
                with hrt.Graph(self.stream) as g2:
                    for c in range(copies):
                        assert run(mats[c])
                g2.launch()
                hrt.device_sync()
                a0, a1 = hrt.Event(), hrt.Event()
                a0.record(self.stream)
                g2.launch()
                a1.record(self.stream)
                ms = a0.elapsed_ms(a1) / copies
                byts = bytes_i4(O, I, B)
                rec[name] = (ms, byts)
                kern_bytes += byts * copies
                kern_ms += ms * copies
                kern_n += copies
            (mu, bu), (md, bd) = rec["up"], rec["down"]
            by_batch[str(B)] = {
                "up_us": round(mu * 1e3, 2), "down_us": round(md * 1e3, 2),
                "up_GBs": round(bu / mu / 1e6, 1), "down_GBs": round(bd / md / 1e6, 1),
                "frac_of_peak": round((bu + bd) / (mu + md) / 1e6 / PEAK_GBS, 3),
            }
        kern_gbs = kern_bytes / kern_ms / 1e6
        # The same bytes as one plain streaming read per launch (no
        # arithmetic, no dependency), over as many fresh buffers: what one
        # launch of this size can read at all on this part.
        nb = bytes_i4(*UP, 0)
        nb -= nb % 16
        bufs = [self.alloc(nb) for _ in range(copies)]
        for p in bufs:
            assert b.hip_stream_read(0, p, nb)
        with hrt.Graph(self.stream) as g3:
            for p in bufs:
                assert b.hip_stream_read(0, p, nb)
        g3.launch()
        hrt.device_sync()
        a0, a1 = hrt.Event(), hrt.Event()
        a0.record(self.stream)
        g3.launch()
        a1.record(self.stream)
        read_floor_us = a0.elapsed_ms(a1) / copies * 1e3
        value = K * step_bytes / wall / 1e9
        self.dense_result = dict(value=value, wall=wall, gpu_ms=gpu_ms, K=K, W=W, by_batch=by_batch, copies=copies,
                                 read_floor_us=read_floor_us, read_floor_bytes=nb,
                                 kern_gbs=kern_gbs, kern_avg_us=kern_ms / kern_n * 1e3,
                                 kern_avg_bytes=kern_bytes / kern_n, pair=pair)
        for t in ups + downs:
            b.cuda_tensor_free(t)

    # -- fused MoE layer ------------------------------
    def moe(self, name, fmt, D, I, E, K, mode, shared, batches, layers_for_anticache, bias, zipf=None,
            per_token=False, steps=None, w_std=0.02):
        """One fused MoE layer (router -> union -> experts -> SwiGLU -> combine)
        timed over `steps` calls per batch size, replayed from a captured graph.
        per_token: each step runs the B rows as B separate 1-row layers (the
        per-token GEMV alternative to the union GEMM). zipf: selection bias
        -(zipf / 11) * ln(1 + e) on top of sigmoid scores of logits ~N(0, 1):
        for zipf = 1.1 and 512 tokens about 150 of 384 experts are touched and
        the head expert takes ~300 rows (skewed, Zipf-like loads)."""
        from colibri_amd.backend import ColiHipMoeConfig, f32p, tensor_array
        b, hrt = self.b, self.hiprt
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        from oracle_lib import Cref
        cref = Cref()
        per_expert = 2 * (bytes_i4(I, D, 0) if fmt == 4 else bytes_fp4(I, D, 0)) + \
            (bytes_i4(D, I, 0) if fmt == 4 else bytes_fp4(D, I, 0))
        n_layers = layers_for_anticache
        stage = self.alloc(max(I * D // 2, D * I // 2))
        layers = []
        seed = 1000
        for L in range(n_layers):
            hs = []
            for e in range(E + (1 if shared else 0)):
                trip = []
                for (O, II) in ((I, D), (I, D), (D, I)):
                    seed += 1
                    if fmt == 4:
                        trip.append(self.tensor_i4(stage, O, II, fp16_scales(self.rng, O, II // 32), seed))
                    else:
                        e8 = self.rng.integers(119, 124, (O, II // 32), dtype=np.uint8)
                        trip.append(self.tensor_fp4(stage, O, II, e8, seed))
                hs.append(trip)
            W = (self.rng.standard_normal((E, D)) * w_std).astype(np.float32)
            if zipf is not None:
                bvec = (-zipf / 11.0 * np.log1p(np.arange(E))).astype(np.float32)
            else:
                bvec = (self.rng.standard_normal(E) * 0.01).astype(np.float32) if bias else None
            routed = hs[:E]
            sh = hs[E] if shared else [None, None, None]
            g, ga = tensor_array([t[0] for t in routed])
            u, ua = tensor_array([t[1] for t in routed])
            d, da = tensor_array([t[2] for t in routed])
            cfg = ColiHipMoeConfig(D, I, E, K, mode, 0, 0.0, 1.0, 1 if shared else 0)
            m = C.c_void_p()
            if not b.hip_moe_create(C.byref(m), 0, C.byref(cfg), f32p(W), f32p(bvec) if bvec is not None else None,
                                    g, u, d, sh[0], sh[1], sh[2]):
                raise RuntimeError("moe_create failed")
            layers.append((m, hs, W, bvec))
        npool = max(64, max(batches))
        xpool = bf16_exact(self.rng.standard_normal((npool, D)).astype(np.float32))
        xd = self.put(xpool)
        od = self.alloc(npool * D * 4)
        result = {}
        for B in batches:
            n_steps = steps or self.args.moe_steps
            # unique experts (and rows per expert) per call, from the reference
            # router on the same inputs
            nus, loads = [], []
            for k in range(n_steps):
                L = k % n_layers
                r0 = (k * B) % npool
                if r0 + B > npool:
                    r0 = 0
                xb = np.ascontiguousarray(xpool[r0:r0 + B])
                W, bvec = layers[L][2], layers[L][3]
                idx, _, keff = cref.route(cref.matmul_f32(xb, W), K, mode, bias=bvec)
                sel = [int(e) for s_ in range(B) for e in idx[s_, :keff[s_]]]
                if per_token:
                    nus.append(B * (K + (1 if shared else 0)))
                else:
                    nus.append(len(set(sel)) + (1 if shared else 0))
                loads.append(np.bincount(np.array(sel), minlength=E))

            def call(k):
                L = k % n_layers
                r0 = (k * B) % npool
                if r0 + B > npool:
                    r0 = 0
                if per_token:
                    for r in range(B):
                        if not b.hip_moe_forward_dev(layers[L][0], C.c_void_p(xd + (r0 + r) * D * 4),
                                                     C.c_void_p(od + r * D * 4), 1):
                            raise RuntimeError("moe forward failed")
                elif not b.hip_moe_forward_dev(layers[L][0], C.c_void_p(xd + r0 * D * 4), od, B):
                    raise RuntimeError("moe forward failed")

            for k in range(max(self.args.warmup, n_layers)):   # every layer sized before capture
                call(k)
            hrt.device_sync()
            # timed layers replayed from one captured graph (see dense())
            with hrt.Graph(self.stream) as graph:
                for k in range(n_steps):
                    call(k)
            graph.launch()
            hrt.device_sync()
            e0, e1 = hrt.Event(), hrt.Event()
            t0 = time.perf_counter()
            e0.record(self.stream)
            graph.launch()
            e1.record(self.stream)
            hrt.device_sync()
            wall = time.perf_counter() - t0
            gpu_ms = e0.elapsed_ms(e1)
            router = E * D * 4
            byts = np.array([nu * per_expert + router + 2 * B * D * 2 for nu in nus], np.float64)
            rec = {"tokens_per_s": round(B * n_steps / wall, 1),
                   "layer_us": round(gpu_ms / n_steps * 1e3, 2),
                   "layer_us_wall": round(wall / n_steps * 1e6, 2),
                   "avg_unique_experts": round(float(np.mean(nus)), 2),
                   "GBs": round(byts.sum() / gpu_ms / 1e6, 1),
                   "frac_of_peak": round(byts.sum() / gpu_ms / 1e6 / PEAK_GBS, 3)}
            if B >= 64:
                flops = 2.0 * 3 * D * I * (B * K + (B if shared else 0))
                rec["max_rows_per_expert"] = int(max(int(l.max()) for l in loads))
                rec["row_tiles_64"] = round(float(np.mean([int(np.sum((l + 63) // 64)) for l in loads])), 1)
                rec["mfma_TFLOPs"] = round(flops * n_steps / gpu_ms / 1e9, 1)
                rec["mfma_frac_of_fp16_peak"] = round(flops * n_steps / gpu_ms / 1e9 / 2500.0, 4)
            result[f"B{B}" + ("_per_token" if per_token else "")] = rec
        for (m, hs, W, bvec) in layers:
            b.hip_moe_free(m)
            for trip in hs:
                for t in trip:
                    b.cuda_tensor_free(t)
        result["layers_cycled"] = n_layers
        result["weights_GB"] = round(n_layers * (E + (1 if shared else 0)) * per_expert / 1e9, 2)
        return result

    def close(self):
        for p in self.allocs:
            self.b.cuda_pipe_free(0, p)
        self.s.close()


def measured_traffic():
    """HBM bytes per GEMV launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs (scaled by a calibration copy of known size); None when
    that profile is absent."""
    path = os.path.join(ROOT, "profiles", "coli_gemv_dense_int4_traffic.json")
    try:
        with open(path) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def issue_take(bench, name, fmt, D, I, count=8, reps=200):
    """Decode-time expert group (one row for each of `count` experts), the
    reference's async split (c/backend_cuda.cu:1677-1812; the CPU share of a
    layer runs between issue and take, c/colibri.c:4467-4531 and 4795):
    host wall time of the sync call, of issue() and of take(), and of
    issue -> host work of the sync call's length -> take, against the two
    run back to back. Host buffers in and out, as the ABI has them."""
    from colibri_amd.backend import f32p, i32p, tensor_array
    b = bench.b
    stage = bench.alloc(I * D // 2)
    hs = []
    seed = 7000
    for e in range(count):
        trip = []
        for (O, II) in ((I, D), (I, D), (D, I)):
            seed += 1
            if fmt == 4:
                trip.append(bench.tensor_i4(stage, O, II, fp16_scales(bench.rng, O, II // 32), seed))
            else:
                trip.append(bench.tensor_fp4(stage, O, II, bench.rng.integers(119, 124, (O, II // 32),
                                                                               dtype=np.uint8), seed))
        hs.append(trip)
    g, ga = tensor_array([t[0] for t in hs])
    u, ua = tensor_array([t[1] for t in hs])
    d, da = tensor_array([t[2] for t in hs])
    rows = np.ones(count, np.int32)
    x = bf16_exact(bench.rng.standard_normal((count, D)).astype(np.float32))
    y = np.zeros((count, D), np.float32)
    pc = time.perf_counter

    def sync():
        if not b.cuda_expert_group(g, u, d, i32p(rows), count, f32p(y), f32p(x)):
            raise RuntimeError("coli_cuda_expert_group failed")

    def issue():
        if not b.cuda_expert_group_issue(g, u, d, i32p(rows), count, f32p(x)):
            raise RuntimeError("coli_cuda_expert_group_issue failed")

    def take():
        if not b.cuda_expert_group_take(0):
            raise RuntimeError("coli_cuda_expert_group_take returned NULL")

    def spin(sec):
        t = pc() + sec
        while pc() < t:
            pass

    for _ in range(10):
        sync()
        issue()
        take()
    t_sync, t_issue, t_take, t_ovl = [], [], [], []
    for _ in range(reps):
        t0 = pc()
        sync()
        t_sync.append(pc() - t0)
    cpu = float(np.median(t_sync))
    for _ in range(reps):
        t0 = pc()
        issue()
        t1 = pc()
        take()
        t2 = pc()
        t_issue.append(t1 - t0)
        t_take.append(t2 - t1)
    for _ in range(reps):
        t0 = pc()
        issue()
        spin(cpu)
        take()
        t_ovl.append(pc() - t0)
    for trip in hs:
        for t in trip:
            b.cuda_tensor_free(t)
    med = lambda v: round(float(np.median(v)) * 1e6, 1)
    return {"shape": f"{name}: {count} experts x 1 row, D={D}, I={I}, fmt={fmt}",
            "sync_call_us": med(t_sync), "issue_us": med(t_issue), "take_after_issue_us": med(t_take),
            "issue_hostwork_take_us": med(t_ovl), "hostwork_us": round(cpu * 1e6, 1),
            "serial_us": round(2 * cpu * 1e6, 1)}


MOE_PARTS = ("olmoe", "dsv3", "verify", "issue_take", "kimi", "kimi_mx")


def moe_layers(bench, only=None):
    """The MoE-layer measurements of configs[0], [2], [3] and [4] (only: the
    subset of MOE_PARTS to run, a profiling aid)."""
    want = lambda part: only is None or part in only
    res = {}
    if want("olmoe"):
        res["configs[0]_olmoe_int4"] = bench.moe("olmoe", 4, 2048, 1024, 64, 8, 0, False, (1,), 10, False)
    if want("dsv3"):
        # two layers cycled (each with its own router and shared expert): every
        # call streams weights the previous call did not touch
        res["configs[2]_dsv3_mxfp4"] = bench.moe("dsv3", 7, 7168, 2048, 256, 8, 2, True, (1, 4, 8, 16), 2, True)
    # one verification step of 21 rows (16-node tree + 5-token
    # draft) on the configs[2] layer shape, union GEMM vs 21 per-token passes
    if want("verify"):
        ver = {}
        for fmt, tag in ((7, "mxfp4"), (4, "int4")):
            r = bench.moe("dsv3", fmt, 7168, 2048, 256, 8, 2, True, (21,), 2, True, steps=20)
            r.update({k + "": v for k, v in bench.moe("dsv3", fmt, 7168, 2048, 256, 8, 2, True, (21,), 2, True,
                                                          steps=6, per_token=True).items() if k.startswith("B")})
            ver[tag] = r
        res["configs[3]_verification_21rows"] = ver
    # the async issue/take split at decode, overlapped with host work
    if want("issue_take"):
        res["issue_take"] = {"olmoe_int4": issue_take(bench, "olmoe", 4, 2048, 1024),
                             "dsv3_mxfp4": issue_take(bench, "dsv3", 7, 7168, 2048)}
    # Kimi-shaped prefill chunk, 512 tokens, 384 experts top-8,
    # router logits ~N(0,1) with a Zipf(1.1) selection bias
    if want("kimi"):
        res["configs[4]_kimi_prefill_512"] = {
            tag: bench.moe("kimi", fmt, 7168, 2048, 384, 8, 2, False, (512,), 2, True, zipf=1.1, steps=6,
                           w_std=1.0 / math.sqrt(7168))
            for fmt, tag in ((7, "mxfp4"), (4, "int4"))}
    # the opt-in MXFP4 GEMM on the block-scaled MFMA (COLI_HIP_MX=1; not
    # fp32-exact: the hardware's per-block summation error is ~2^-15 of the
    # block's magnitude sum)
    if want("kimi_mx"):
        os.environ["COLI_HIP_MX"] = "1"
        try:
            res.setdefault("configs[4]_kimi_prefill_512", {})["mxfp4_block_scaled_mfma_optin"] = bench.moe(
                "kimi", 7, 7168, 2048, 384, 8, 2, False, (512,), 2, True, zipf=1.1, steps=6,
                w_std=1.0 / math.sqrt(7168))
        finally:
            del os.environ["COLI_HIP_MX"]
    return res


def cpu_topology():
    """CPU model, physical cores and logical CPUs this process may run on."""
    cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    model, cores, cur = "unknown", set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f.read().split("\n\n"):
                kv = dict(l.split(":", 1) for l in line.splitlines() if ":" in l)
                kv = {k.strip(): v.strip() for k, v in kv.items()}
                if "processor" not in kv:
                    continue
                model = kv.get("model name", model)
                if int(kv["processor"]) in cpus:
                    cores.add((kv.get("physical id", "0"), kv.get("core id", kv["processor"])))
    except (OSError, ValueError, KeyError):
        pass
    return model, max(1, len(cores)), len(cpus)


CPU_INFO = {}


def main():
    # The CPU baseline's OpenMP runs on the physical cores, bound close (the
    # reference's published CPU setup): set before any OpenMP library is loaded. An
    # OMP_NUM_THREADS already in the environment (the host's CPU share) caps it.
    model, phys, logical = cpu_topology()
    threads = min(phys, int(os.environ.get("OMP_NUM_THREADS", phys)))
    os.environ["OMP_NUM_THREADS"] = str(threads)
    os.environ["OMP_PROC_BIND"] = "close"
    CPU_INFO.update({"model": model, "physical_cores": phys, "logical_cpus": logical, "threads": threads,
                     "OMP_NUM_THREADS": threads, "OMP_PROC_BIND": "close"})
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--anticache-gb", type=float, default=2.0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-moe", action="store_true")
    ap.add_argument("--skip-dense", action="store_true",
                    help="run only the MoE-layer measurements (profiling aid; prints the moe_layer object)")
    ap.add_argument("--moe-steps", type=int, default=50)
    ap.add_argument("--moe-only", default=None,
                    help="with --skip-dense: comma-separated subset of " + ",".join(MOE_PARTS))
    ap.add_argument("--copy-calib", action="store_true",
                    help="only copy 256 MiB device-to-device 4 times (the known-size reference that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    ap.add_argument("--cpu-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_child:   # the CPU baseline alone, no GPU runtime in this process
        print(json.dumps(cpu_baseline(args.cpu_seconds)))
        sys.stdout.flush()
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the expert path has no collectives; "
                                   "run with --gpus 1 (expert parallelism across GPUs is not built here)"}))
        sys.exit(2)
    # the CPU baseline first, in a child process, before this process loads
    # the GPU runtime (and so before any GPU work that host load could disturb)
    cpu = None
    if not args.skip_cpu and not args.skip_dense and not args.copy_calib:
        cpu = cpu_baseline_child(args.cpu_seconds)
    bench = Bench(args)
    if args.copy_calib:
        nb = 256 << 20
        src, dst = bench.alloc(nb), bench.alloc(nb)
        assert bench.b.hip_fill_random_u8(0, src, nb, 7)
        for _ in range(4):
            bench.hiprt.copy_d2d_async(dst, src, nb, bench.stream)
        bench.hiprt.device_sync()
        bench.close()
        print(json.dumps({"copy_calib_bytes": nb, "copies": 4}))
        return
    if args.skip_dense:
        only = None
        if args.moe_only:
            only = set(args.moe_only.split(","))
            if not only <= set(MOE_PARTS):
                ap.error(f"--moe-only: parts are {','.join(MOE_PARTS)}")
        print(json.dumps({"moe_layer": moe_layers(bench, only)}), flush=True)
        bench.close()
        return
    bench.dense()
    r = bench.dense_result
    out = {
        "metric": METRIC, "value": round(r["value"], 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(r["wall"] / r["K"] * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4", "data": "synthetic",
        "config": {"workload": "configs[1]: dense int4-g32 GEMV, W_up 14336x4096 then W_down 4096x14336, "
                               "batch 1/4/8/16 per step, fp16 group scales, bf16 activations, f32 accumulate",
                   "weight_copies": r["copies"], "distinct_weight_GB": round(r["copies"] * r["pair"] / 1e9, 2)},
        "frac_of_peak": round(r["value"] / PEAK_GBS, 3),
        "roofline": {"bound": "hbm", "achieved": round(r["kern_gbs"], 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["kern_gbs"] / PEAK_GBS, 3), "traffic": measured_traffic(),
                     "kernel": "coli_gemv_dma (B1, B4) + coli_gemv_tiles (B8, B16); up launches emit h as the down GEMV fragments", "avg_launch_us": round(r["kern_avg_us"], 2),
                     "avg_launch_bytes": int(r["kern_avg_bytes"]),
                     # a plain streaming read of the same bytes, one launch each
                     "read_floor_us": round(r["read_floor_us"], 2),
                     "read_floor_frac": round(r["read_floor_bytes"] / r["read_floor_us"] / 1e3 / PEAK_GBS, 3)},
        "gemv_by_batch": r["by_batch"],
    }
    if not args.skip_moe:
        out["moe_layer"] = moe_layers(bench)
    if cpu is not None:
        out["cpu_baseline"] = cpu
    # the result line goes out (flushed) before the backend is torn down
    print(json.dumps(out), flush=True)
    bench.close()


if __name__ == "__main__":
    main()
