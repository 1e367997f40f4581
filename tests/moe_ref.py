"""Synthetic MoE layers and their CPU reference (test infrastructure).

The reference composition uses the oracle's bit-exact restatements of the
reference kernels (router f32 GEMV, top-K, int4/MXFP4 GEMV, silu*up) and
accumulates the weighted scatter in float64, so parity checks compare the GPU
against the reference arithmetic without depending on one particular f32
summation order.
"""
import numpy as np

from oracle_lib import Cref
from quant_util import bf16_exact, deq_i4, deq_mxfp4, rand_i4, rand_mxfp4

cref = Cref()


def make_router_inputs(rng, S, D, E, K, mode, gap=1e-4, bias=False, zipf=None):
    """x [S, D] (bf16-exact), router W [E, D] ~ N(0, 0.02), optional bias; rows
    are redrawn until the rank-K / rank-(K+1) gap of the selection score is
    >= gap in every row (computed with the oracle's f32 router arithmetic)."""
    W = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(E) * 0.01).astype(np.float32) if bias else None
    if zipf is not None:
        ranks = np.arange(1, E + 1, dtype=np.float64)
        zb = np.log(1.0 / ranks ** zipf)
        b = (zb - zb.mean()).astype(np.float32) * 0.2 if b is None else b + zb.astype(np.float32)
    x = np.empty((S, D), np.float32)
    for s in range(S):
        for _ in range(1000):
            xs = bf16_exact(rng.standard_normal((1, D)).astype(np.float32))
            z = cref.matmul_f32(xs, W)[0].astype(np.float64)
            if mode == 0:
                sc = np.exp(z - z.max())
                sc = sc / sc.sum()
                # selection is monotone in z; require the gap in logit space
                srt = np.sort(z)[::-1]
            elif mode == 3:
                sc = np.sqrt(np.logaddexp(0.0, z)) + (b if b is not None else 0)
                srt = np.sort(sc)[::-1]
            else:
                sc = 1.0 / (1.0 + np.exp(-z)) + (b if b is not None else 0)
                srt = np.sort(sc)[::-1]
            if srt[K - 1] - srt[K] >= gap:
                x[s] = xs[0]
                break
        else:
            raise RuntimeError("could not draw a router input with the required gap")
    return x, W, b


class Layer:
    """Expert weights of one synthetic MoE layer in source layout.
    distinct: number of distinct weight sets, expert e using set e % distinct
    (full-size layers without full-size host and device memory)."""

    def __init__(self, rng, fmt, D, I, E, shared=False, swiglu_limit=0.0, distinct=None, e8_range=(119, 123)):
        self.fmt, self.D, self.I, self.E = fmt, D, I, E
        self.e8_range = e8_range   # MXFP4 scale exponents drawn from [lo, hi]
        self.swiglu_limit = swiglu_limit   # > 0: DeepSeek-V4 clamped SwiGLU
        n = E if distinct is None else min(E, distinct)
        sets = [self._expert(rng) for _ in range(n)]
        self.experts = [sets[e % n] for e in range(E)]
        self.shared = self._expert(rng) if shared else None
        self._deq = {}

    def _expert(self, rng):
        D, I = self.D, self.I
        if self.fmt == 4:
            g = rand_i4(rng, I, D, 32)
            u = rand_i4(rng, I, D, 32)
            d = rand_i4(rng, D, I, 32)
        else:
            g = rand_mxfp4(rng, I, D, *self.e8_range)
            u = rand_mxfp4(rng, I, D, *self.e8_range)
            d = rand_mxfp4(rng, D, I, *self.e8_range)
        return g, u, d

    def gemv(self, mat, x, O, I):
        q, s = mat
        if self.fmt == 4:
            return cref.matmul_i4_grouped(x, q, s, O, I, 32)
        return cref.matmul_mxfp4(x, q, s, O, I)

    def deq(self, mat, I):
        key = id(mat[0])
        if key not in self._deq:
            q, s = mat
            self._deq[key] = np.abs(deq_i4(q, s, I, 32) if self.fmt == 4 else deq_mxfp4(q, s, I)).T.copy()
        return self._deq[key]

    def expert_forward(self, e, x):
        g, u, d = self.experts[e] if e >= 0 else self.shared
        gv = self.gemv(g, x, self.I, self.D)
        uv = self.gemv(u, x, self.I, self.D)
        h = cref.swiglu_v4(gv, uv, self.swiglu_limit) if self.swiglu_limit > 0 else cref.swiglu(gv, uv)
        return h, self.gemv(d, h, self.D, self.I)

    def upload(self, session):
        """Device handles per expert (+ shared); experts sharing a weight set
        share its handles (free them with free_handles)."""
        hs, done = [], {}
        for trip in self.experts + ([self.shared] if self.shared else []):
            key = id(trip)
            if key not in done:
                g, u, d = trip
                done[key] = tuple(self._up(session, m, O, I) for m, O, I in
                                  ((g, self.I, self.D), (u, self.I, self.D), (d, self.D, self.I)))
            hs.append(done[key])
        return hs

    def _up(self, session, m, O, I):
        q, s = m
        if self.fmt == 4:
            return session.upload(q, s, 4, I, O, 32)
        return session.upload_mxfp4(q, s, I, O)


def moe_reference(layer, x, W, b, K, mode, norm_topk=0, topp=0.0, routed_scale=1.0):
    """Routing (bit-exact oracle) and the layer output (float64 scatter).
    Returns idx, w, keff, out, mag where mag bounds sum|terms| per output."""
    S, D = x.shape
    logits = cref.matmul_f32(x, W)
    idx, w, keff = cref.route(logits, K, mode, bias=b, topp=topp, norm_topk=norm_topk,
                              routed_scale=routed_scale)
    out = np.zeros((S, D), np.float64)
    mag = np.zeros((S, D), np.float64)
    for s in range(S):
        xs = x[s:s + 1]
        experts = [(int(idx[s, kk]), float(w[s, kk])) for kk in range(keff[s])]
        if layer.shared is not None:
            experts.append((-1, 1.0))
        for e, wk in experts:
            h, y = layer.expert_forward(e, xs)
            dm = layer.experts[e][2] if e >= 0 else layer.shared[2]
            out[s] += wk * y[0].astype(np.float64)
            mag[s] += abs(wk) * (np.abs(h[0].astype(np.float64)) @ layer.deq(dm, layer.I))
    return idx, w, keff, out, mag


def free_handles(session, hs):
    """Free every distinct device handle of Layer.upload once."""
    seen = set()
    for trip in hs:
        for t in trip:
            if t is not None and id(t) not in seen:
                seen.add(id(t))
                session.free(t)
