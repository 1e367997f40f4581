"""Synthetic inputs and tolerance helpers shared by the tests and the bench.

Distributions follow the benchmark configurations: int4 nibbles uniform over
0..15 (value u-8), group scales |N(0, 0.01)| rounded to fp16 and handed over
as their exact f32 widening, MXFP4 codes uniform over the 16 e2m1 codes with
e8m0 bytes in 119..123 (2^-8..2^-4), activations bf16-exact ~N(0, 1).
"""
import numpy as np

E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def bf16_exact(a):
    """Round f32 values to bf16 (RNE) and return them as f32."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rand_x(rng, S, I):
    return bf16_exact(rng.standard_normal((S, I)).astype(np.float32))


def rand_i4(rng, O, I, gs, fp16_scales=True):
    q4 = rng.integers(0, 256, (O, (I + 1) // 2), dtype=np.uint8)
    ng = 1 if gs <= 0 else (I + gs - 1) // gs
    sc = np.abs(rng.standard_normal((O, ng)) * 0.01)
    sc = sc.astype(np.float16).astype(np.float32) if fp16_scales else sc.astype(np.float32)
    if gs <= 0:
        sc = sc[:, 0].copy()
    return q4, sc


def rand_mxfp4(rng, O, I, lo=119, hi=123):
    q4 = rng.integers(0, 256, (O, (I + 1) // 2), dtype=np.uint8)
    e8 = rng.integers(lo, hi + 1, (O, (I + 31) // 32), dtype=np.uint8)
    return q4, e8


def nibbles(q4, I):
    lo = (q4 & 15).astype(np.int64)
    hi = (q4 >> 4).astype(np.int64)
    n = np.empty((q4.shape[0], q4.shape[1] * 2), np.int64)
    n[:, 0::2] = lo
    n[:, 1::2] = hi
    return n[:, :I]


def deq_i4(q4, sc, I, gs):
    """Dense f64 dequant of an int4 matrix (value u-8 times its group scale)."""
    w = (nibbles(q4, I) - 8).astype(np.float64)
    if gs <= 0:
        return w * sc.astype(np.float64)[:, None]
    g = np.arange(I) // gs
    return w * sc.astype(np.float64)[:, g]


def mx4_scale(e8):
    return (e8.astype(np.uint32) << 23).view(np.float32).astype(np.float64)


def deq_mxfp4(q4, e8, I):
    w = E2M1[nibbles(q4, I)]
    return w * mx4_scale(e8)[:, np.arange(I) // 32]


def magnitude(x, wdeq):
    """sum_k |x_k w_k| per output: the scale rounding error lives on."""
    return np.abs(x.astype(np.float64)) @ np.abs(wdeq).T


def rel_err(got, ref, mag, floor=1e-2):
    """|got - ref| / max(|ref|, floor * sum|terms|): the north-star metric with a
    floor for outputs that cancel to near zero."""
    den = np.maximum(np.abs(ref.astype(np.float64)), floor * mag)
    den = np.where(den == 0, 1.0, den)
    return np.abs(got.astype(np.float64) - ref.astype(np.float64)) / den
