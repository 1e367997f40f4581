"""Pins the CPU oracle (oracle/cpu_ref.c) before any GPU result is compared
with it:

* bitwise against the committed vectors of the reference's own compiled
  kernels (tests/golden/golden.npz, written by tests/golden/make_golden.py);
* bitwise against oracle/_ref (the reference compiled from its sources) on
  random ragged shapes, where that library is present;
* against the known-answer tests of c/tests/test_native_quant.c:13-85;
* against what the mathematics fixes: float64 brute-force dequantisation
  (c/tests/test_i4_grouped.c:28-54 metric), unit-vector probes that isolate
  one code, the fmt=2 == fmt=4(gs=I) identity
  (c/tests/test_grouped_g4_cuda.cu:29-46), a sort-based router, the set and
  first-seen-order invariants of the expert union, the closed form of SwiGLU.
"""
import os

import numpy as np
import pytest

from oracle_lib import Cref, Ref, have_ref
from quant_util import E2M1, deq_i4, deq_mxfp4, magnitude, rand_i4, rand_mxfp4, rand_x, rel_err

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
cref = Cref()


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


def cases(gold, prefix):
    n = 0
    while f"{prefix}{n}_shape" in gold.files:
        yield n
        n += 1


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# -- golden vectors of the compiled reference ---------------------------------

def test_golden_i4_grouped(gold):
    seen = 0
    for n in cases(gold, "i4g"):
        S, I, O, gs = gold[f"i4g{n}_shape"]
        y = cref.matmul_i4_grouped(gold[f"i4g{n}_x"], gold[f"i4g{n}_q4"], gold[f"i4g{n}_sc"], O, I, gs)
        assert np.array_equal(bits(y), bits(gold[f"i4g{n}_y"])), (S, I, O, gs)
        seen += 1
    assert seen >= 5


def test_golden_i4_per_row(gold):
    for n in cases(gold, "i4r"):
        S, I, O = gold[f"i4r{n}_shape"]
        y = cref.matmul_i4(gold[f"i4r{n}_x"], gold[f"i4r{n}_q4"], gold[f"i4r{n}_sc"], O, I)
        assert np.array_equal(bits(y), bits(gold[f"i4r{n}_y"])), (S, I, O)


def test_golden_mxfp4(gold):
    for n in cases(gold, "mx"):
        S, I, O = gold[f"mx{n}_shape"]
        y = cref.matmul_mxfp4(gold[f"mx{n}_x"], gold[f"mx{n}_q4"], gold[f"mx{n}_e8"], O, I)
        assert np.array_equal(bits(y), bits(gold[f"mx{n}_y"])), (S, I, O)


def test_golden_f32(gold):
    y = cref.matmul_f32(gold["f32_x"], gold["f32_W"])
    assert np.array_equal(bits(y), bits(gold["f32_y"]))


@pytest.mark.parametrize("blk", [128, 64, 32])
def test_golden_qdq(gold, blk):
    y, sc = cref.qdq(gold["qdq_x"], blk)
    assert np.array_equal(sc, gold[f"qdq_b{blk}_sc"])
    assert np.array_equal(bits(y), bits(gold[f"qdq_b{blk}_y"]))


def test_golden_fp4_batch_and_rows16(gold):
    for n in cases(gold, "fb"):
        S, I, O = gold[f"fb{n}_shape"]
        q4, e8, x = gold[f"fb{n}_q4"], gold[f"fb{n}_e8"], gold[f"fb{n}_x"]
        y = cref.fp4_matmul_batch(x, q4, e8, O, I)
        assert np.array_equal(bits(y), bits(gold[f"fb{n}_y"]))
        pd, ps = cref.pack_rows16(q4, e8, O, I)
        assert np.array_equal(pd, gold[f"fb{n}_pd"]) and np.array_equal(ps, gold[f"fb{n}_ps"])
        y16 = cref.matvec_rows16(np.ascontiguousarray(x[0]), pd, ps, O, I)
        assert np.array_equal(bits(y16), bits(gold[f"fb{n}_y16"]))


def test_golden_codecs(gold):
    assert np.array_equal(bits([cref.e2m1(i) for i in range(16)]), bits(gold["e2m1"]))
    assert np.array_equal(bits([cref.e8m0(i) for i in range(256)]), gold["e8m0_bits"])
    assert np.array_equal(bits([cref.e4m3_dec(i) for i in range(256)]), gold["e4m3_dec_bits"])
    enc = np.array([cref.e4m3_enc(float(v)) for v in gold["e4m3_enc_in"]], np.uint8)
    assert np.array_equal(enc, gold["e4m3_enc_out"])
    bf = np.array([cref.bf16_round(float(v)) for v in gold["bf16_in"]], np.float32)
    assert np.array_equal(bits(bf), bits(gold["bf16_out"]))


# -- the compiled reference, on random ragged shapes --------------------------

@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (needs the reference tree)")
def test_random_shapes_vs_compiled_reference():
    ref = Ref()
    rng = np.random.default_rng(11)
    for t in range(60):
        S = int(rng.integers(1, 6))
        I = int(rng.integers(8, 300))
        O = int(rng.integers(1, 24))
        gs = int(rng.choice([16, 32, 64, 128]))
        x = rand_x(rng, S, I)
        q4, sc = rand_i4(rng, O, I, gs, fp16_scales=bool(t % 2))
        assert np.array_equal(bits(cref.matmul_i4_grouped(x, q4, sc, O, I, gs)),
                              bits(ref.matmul_i4_grouped(x, q4, sc, O, I, gs))), (S, I, O, gs)
        q4, sc = rand_i4(rng, O, I, 0)
        assert np.array_equal(bits(cref.matmul_i4(x, q4, sc, O, I)), bits(ref.matmul_i4(x, q4, sc, O, I)))
        q4, e8 = rand_mxfp4(rng, O, I, 100, 140)
        assert np.array_equal(bits(cref.matmul_mxfp4(x, q4, e8, O, I)),
                              bits(ref.matmul_mxfp4(x, q4, e8, O, I))), (S, I, O)
        W = rng.standard_normal((O, I)).astype(np.float32)
        assert np.array_equal(bits(cref.matmul_f32(x, W)), bits(ref.matmul_f32(x, W))), (S, I, O)


# -- known-answer tests, c/tests/test_native_quant.c:13-85 --------------------

def test_kat_codecs():
    assert cref.bf16_round(1.00390625) == 1.0
    assert cref.bf16_round(1.01171875) == 1.015625
    assert [cref.e2m1(i) for i in range(16)] == list(E2M1)
    assert cref.e8m0(0x7E) == 0.5 and cref.e8m0(0x7F) == 1.0 and cref.e8m0(0x80) == 2.0
    assert np.isnan(cref.e8m0(0xFF))
    for v in (0.0, 0.001953125, 0.5, 1.0, 1.5, 6.0, 224.0, 448.0, -0.5, -6.0, -448.0):
        assert cref.e4m3_dec(cref.e4m3_enc(v)) == v


def test_kat_qdq_ones():
    y, sc = cref.qdq(np.ones(128, np.float32), 128)
    assert sc[0] == 119 and np.all(y == 1.0)
    y, sc = cref.qdq(np.ones(20, np.float32), 64)  # partial block
    assert sc[0] == 119 and np.all(y == 1.0)


def test_kat_fp4_matvec_128():
    """64 bytes of 0x44 (+2.0 twice) at e8m0 0x7e (0.5), x = 1: 128 * 2 * 0.5."""
    q4 = np.full((1, 64), 0x44, np.uint8)
    e8 = np.full((1, 4), 0x7E, np.uint8)
    x = np.ones((1, 128), np.float32)
    assert cref.fp4_matmul_batch(x, q4, e8, 1, 128)[0, 0] == 128.0
    assert cref.matmul_mxfp4(x, q4, e8, 1, 128)[0, 0] == 128.0


# -- what the mathematics fixes -----------------------------------------------

def test_e8m0_closed_form():
    for s in range(1, 255):
        assert cref.e8m0(s) == 2.0 ** (s - 127)
        assert cref.mx4_scale(s) == 2.0 ** (s - 127)
    assert cref.mx4_scale(0) == 0.0 and np.isinf(cref.mx4_scale(255))


def test_e4m3_decode_closed_form():
    for b in range(256):
        s, e, m = b >> 7, (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            assert np.isnan(cref.e4m3_dec(b))
            continue
        v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        assert cref.e4m3_dec(b) == (-v if s else v)


def test_qdq_error_bound():
    """Each QDQ value is the e4m3 code nearest to x / 2^(s-127), times 2^(s-127);
    the block maximum must not saturate."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(1024) * np.exp(rng.uniform(-6, 6, 1024))).astype(np.float32)
    y, sc = cref.qdq(x, 128)
    grid = np.array([cref.e4m3_dec(b) for b in range(127)], np.float64)  # non-negative finite codes
    for blk in range(8):
        scale = 2.0 ** (int(sc[blk]) - 127)
        xs = x[blk * 128:(blk + 1) * 128].astype(np.float64) / scale
        assert np.abs(xs).max() <= 448.0
        best = np.abs(np.abs(xs)[:, None] - grid[None, :]).min(axis=1)
        got = np.abs(y[blk * 128:(blk + 1) * 128].astype(np.float64) / scale)
        assert np.all(np.abs(got - np.abs(xs)) <= best + 1e-12)


@pytest.mark.parametrize("gs", [16, 32, 64, 128])
def test_i4_grouped_vs_f64_dequant(gs):
    rng = np.random.default_rng(gs)
    for S, I, O in [(1, 256, 33), (3, 517, 17), (5, 64, 8)]:
        q4, sc = rand_i4(rng, O, I, gs)
        x = rand_x(rng, S, I)
        wd = deq_i4(q4, sc, I, gs)
        ref = x.astype(np.float64) @ wd.T
        assert rel_err(cref.matmul_i4_grouped(x, q4, sc, O, I, gs), ref, magnitude(x, wd), 1.0).max() <= 2e-6


def test_i4_unit_vector_isolates_nibble():
    """Scales 1, x = e_i: output row o is exactly nibble(o, i) - 8."""
    rng = np.random.default_rng(4)
    O, I = 16, 96
    q4 = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    sc = np.ones((O, I // 32), np.float32)
    nib = np.empty((O, I), np.int64)
    nib[:, 0::2], nib[:, 1::2] = q4 & 15, q4 >> 4
    for i in (0, 1, 31, 32, 95):
        x = np.zeros((1, I), np.float32)
        x[0, i] = 1.0
        y = cref.matmul_i4_grouped(x, q4, sc, O, I, 32)
        assert np.array_equal(y[0], (nib[:, i] - 8).astype(np.float32))


def test_fmt2_equals_fmt4_with_whole_row_group():
    rng = np.random.default_rng(5)
    O, I, S = 9, 192, 2
    q4, sc = rand_i4(rng, O, I, 0)
    x = rand_x(rng, S, I)
    a = cref.matmul_i4(x, q4, sc, O, I)
    b = cref.matmul_i4_grouped(x, q4, sc[:, None].copy(), O, I, I)
    wd = deq_i4(q4, sc, I, 0)
    assert rel_err(a, b, magnitude(x, wd), 1.0).max() <= 2e-6


def test_mxfp4_vs_f64_and_single_codes():
    rng = np.random.default_rng(6)
    O, I, S = 21, 320, 3
    q4, e8 = rand_mxfp4(rng, O, I, 110, 140)
    x = rand_x(rng, S, I)
    wd = deq_mxfp4(q4, e8, I)
    ref = x.astype(np.float64) @ wd.T
    assert rel_err(cref.matmul_mxfp4(x, q4, e8, O, I), ref, magnitude(x, wd), 1.0).max() <= 2e-6
    # every code on its own, exact
    for code in range(16):
        q = np.full((1, 16), code | (code << 4), np.uint8)
        e = np.full((1, 1), 127, np.uint8)
        x1 = np.zeros((1, 32), np.float32)
        x1[0, 5] = 1.0
        assert cref.matmul_mxfp4(x1, q, e, 1, 32)[0, 0] == E2M1[code]


def sort_route(logits, K, mode, bias, norm_topk, routed_scale):
    """Float64 routing by a full stable sort (ties to the lower index)."""
    z = logits.astype(np.float64)
    if mode == 0:
        p = np.exp(z - z.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        sel = p
    else:
        p = 1.0 / (1.0 + np.exp(-z))
        sel = p + (bias.astype(np.float64) if bias is not None else 0.0)
    idx = np.argsort(-sel, axis=1, kind="stable")[:, :K]
    w = np.take_along_axis(p, idx, axis=1)
    if (mode == 0 and norm_topk) or (mode == 1 and norm_topk) or mode == 2:
        w = w / w.sum(axis=1, keepdims=True)
    if mode != 0:
        w = w * routed_scale
    return idx, w


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_router_vs_sort(mode):
    from moe_ref import make_router_inputs
    rng = np.random.default_rng(40 + mode)
    S, D, E, K = 12, 64, 64, 6
    x, W, b = make_router_inputs(rng, S, D, E, K, mode, bias=(mode != 0))
    logits = cref.matmul_f32(x, W)
    norm = 1 if mode != 2 else 0
    scale = 2.5 if mode == 1 else 1.0
    ri, rw, rk = cref.route(logits, K, mode, bias=b, norm_topk=norm, routed_scale=scale)
    si, sw = sort_route(logits, K, mode, b, norm, scale)
    assert np.all(rk == K)
    assert np.array_equal(ri, si)
    assert np.allclose(rw, sw, rtol=2e-6, atol=0)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_router_exact_ties_lowest_index(mode):
    """Exactly tied scores: the selection is K rounds of a strict '>' argmax,
    so among equal scores the lowest expert index wins (c/backend_cuda.cu:2176-2178,
    c/olmoe.c:667-673), i.e. the order of a stable descending sort. Logits
    come from four exactly representable values, so equal logits give equal
    f32 scores and the ties are exact; tied experts are spread over the whole
    index range (different lane groups of the GPU selection)."""
    rng = np.random.default_rng(2176 + mode)
    S, E, K = 16, 64, 8
    levels = np.array([-1.5, -0.5, 0.25, 1.0], np.float32)
    logits = levels[rng.integers(0, 4, (S, E))]
    # the top level held by a few experts spread from 0 to E-1, the next one by
    # more than the K - (their count) slots left, so the K boundary cuts a tie
    for s in range(S):
        top = rng.choice(E, 3, replace=False)
        logits[s] = np.where(logits[s] == levels[3], levels[2], logits[s])
        logits[s, top] = levels[3]
    bias = None
    if mode != 0:
        bias = np.zeros(E, np.float32)
        bias[rng.choice(E, 6, replace=False)] = 0.125   # exact; ties within each (logit, bias) class remain
    norm = 1 if mode != 2 else 0
    ri, rw, rk = cref.route(logits, K, mode, bias=bias, norm_topk=norm, routed_scale=1.0)
    si, sw = sort_route(logits, K, mode, bias, norm, 1.0)
    assert np.all(rk == K)
    assert np.array_equal(ri, si)
    assert np.allclose(rw, sw, rtol=2e-6, atol=0)
    # spelled out: every tied class inside the selection is taken in index order
    for s in range(S):
        sel = ri[s]
        z = logits[s].astype(np.float64) + (bias.astype(np.float64) if bias is not None else 0.0)
        for a in range(K - 1):
            if z[sel[a]] == z[sel[a + 1]]:
                assert sel[a] < sel[a + 1]
        # the tie at the boundary: no unselected expert with the K-th score has a lower index
        kth = z[sel[-1]]
        rest = [e for e in range(E) if e not in set(sel.tolist())]
        assert all(not (z[e] == kth and e < sel[-1]) for e in rest)


def test_router_topp_keeps_smallest_prefix():
    """TOPP (c/backend_cuda.cu:2180-2193): weights sorted descending, keep the
    shortest prefix whose mass reaches topp of the total."""
    rng = np.random.default_rng(9)
    E, K = 32, 8
    for _ in range(40):
        z = rng.standard_normal((1, E)).astype(np.float32) * 2
        ri, rw, rk = cref.route(z, K, 1, topp=0.7, norm_topk=0)
        p = 1.0 / (1.0 + np.exp(-z[0].astype(np.float64)))
        top = np.sort(p)[::-1][:K]
        cum = np.cumsum(top) / top.sum()
        if np.min(np.abs(cum - 0.7)) < 1e-5:
            continue  # too close to the threshold for a float64 comparison
        assert rk[0] == int(np.argmax(cum >= 0.7)) + 1
        assert np.all(np.diff(rw[0, :rk[0]]) <= 0)


def test_union_invariants():
    rng = np.random.default_rng(12)
    S, K, E = 21, 8, 40
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(S)]).astype(np.int32)
    w = rng.random((S, K)).astype(np.float32)
    keff = rng.integers(1, K + 1, S).astype(np.int32)
    nu, uq, cnt, rows, slots, ws = cref.expert_union(idx, w, keff, E)
    order = []
    for s in range(S):
        for k in range(keff[s]):
            if idx[s, k] not in order:
                order.append(int(idx[s, k]))
    assert nu == len(order) and list(uq) == order
    assert cnt.sum() == keff.sum()
    for j, e in enumerate(uq):
        pairs = [(s, k) for s in range(S) for k in range(keff[s]) if idx[s, k] == e]
        assert [(int(a), int(b)) for a, b in zip(rows[j, :cnt[j]], slots[j, :cnt[j]])] == pairs
        assert np.array_equal(ws[j, :cnt[j]], np.array([w[s, k] for s, k in pairs], np.float32))


def test_swiglu_closed_form():
    rng = np.random.default_rng(13)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    h = cref.swiglu(g, u)
    g64 = g.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u
    assert np.allclose(h, ref, rtol=1e-6, atol=1e-30)


# -- matmul_mxfp4_i8 (c/quant.h:1441-1515, the K3 IDOT path) --------------------

GOLDEN_I8 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_mxfp4_i8.npz")


def i8_quantize64(x):
    """The int8 quantization of matmul_mxfp4_i8, per its definition: per row
    and 32-column group, sc = max|x| / 127 (f32, floored at 1e-20), q = the
    nearest integer (ties to even) of x * f32(1 / sc), clamped to +-127."""
    S, I = x.shape
    g = x.reshape(S, I // 32, 32)
    sc = (np.abs(g).max(axis=2) / np.float32(127.0)).astype(np.float32)
    sc = np.maximum(sc, np.float32(1e-20))
    inv = (np.float32(1.0) / sc).astype(np.float32)
    q = np.clip(np.rint((g * inv[:, :, None]).astype(np.float32)), -127, 127)
    return q, sc


def test_golden_mxfp4_i8():
    gold = np.load(GOLDEN_I8, allow_pickle=False)
    n = 0
    while f"c{n}_shape" in gold.files:
        S, I, O = gold[f"c{n}_shape"]
        y = cref.matmul_mxfp4_i8(gold[f"c{n}_x"], gold[f"c{n}_q4"], gold[f"c{n}_e8"], O, I)
        assert np.array_equal(bits(y), bits(gold[f"c{n}_y"])), (S, I, O)
        n += 1
    assert n >= 5


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (needs the reference tree)")
def test_mxfp4_i8_vs_compiled_reference():
    ref = Ref()
    rng = np.random.default_rng(808)
    for t in range(30):
        S = int(rng.integers(1, 17))
        I = int(rng.choice([32, 64, 96, 256, 512, 100]))
        O = int(rng.integers(1, 20))
        x = rng.standard_normal((S, I)).astype(np.float32) * np.float32(10.0 ** rng.uniform(-3, 3))
        q4, e8 = rand_mxfp4(rng, O, I, 100, 140)
        assert np.array_equal(bits(cref.matmul_mxfp4_i8(x, q4, e8, O, I)),
                              bits(ref.matmul_mxfp4_i8(x, q4, e8, O, I))), (S, I, O)


def test_mxfp4_i8_quantized_dot_math():
    """Against float64 on the quantized operands: the result is the exact
    integer dot of each group with the doubled e2m1 codes times the group
    scale, so y64 = sum_g sc_g * sum_k q_k w_k agrees to f32 rounding; and on
    activations that are already k * s (integers with the group maximum at
    127) the quantization is the identity."""
    rng = np.random.default_rng(809)
    S, I, O = 4, 256, 24
    q4, e8 = rand_mxfp4(rng, O, I, 115, 130)
    wd = deq_mxfp4(q4, e8, I)
    x = rng.standard_normal((S, I)).astype(np.float32)
    q, sc = i8_quantize64(x)
    assert np.abs(q).max() == 127
    xq = (q * sc[:, :, None].astype(np.float64)).reshape(S, I)
    y64 = xq @ wd.T
    assert rel_err(cref.matmul_mxfp4_i8(x, q4, e8, O, I), y64, magnitude(xq, wd), 1.0).max() <= 2e-6
    # quantization error of the int8 grid itself: within half a step per element
    assert np.all(np.abs(xq.reshape(S, I // 32, 32) - x.reshape(S, I // 32, 32)) <= 0.5 * sc[:, :, None] * 1.0001)
    # identity on the grid
    k = rng.integers(-127, 128, (S, I)).astype(np.float64)
    k.reshape(S, I // 32, 32)[:, :, 0] = 127
    s = 2.0 ** rng.integers(-6, 3, (S, I // 32))
    xg = (k.reshape(S, I // 32, 32) * s[:, :, None]).reshape(S, I).astype(np.float32)
    qg, _ = i8_quantize64(xg)
    assert np.array_equal(qg.reshape(S, I), k)


def test_mxfp4_i8_ragged_falls_back():
    rng = np.random.default_rng(810)
    x = rand_x(rng, 2, 100)
    q4, e8 = rand_mxfp4(rng, 5, 100)
    assert np.array_equal(bits(cref.matmul_mxfp4_i8(x, q4, e8, 5, 100)), bits(cref.matmul_mxfp4(x, q4, e8, 5, 100)))


# -- DeepSeek-V4 router and SwiGLU (c/deepseek_v4.c:1368-1448) -------------------

GOLDEN_V4 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_v4.npz")


def test_golden_v4_route_and_swiglu():
    gold = np.load(GOLDEN_V4, allow_pickle=False)
    n = 0
    while f"r{n}_meta" in gold.files:
        E, K, has_b = (int(v) for v in gold[f"r{n}_meta"])
        b = gold[f"r{n}_b"] if has_b else None
        idx, w, keff = cref.route(gold[f"r{n}_z"][None, :], K, 3, bias=b, routed_scale=float(gold[f"r{n}_scale"][0]))
        assert np.array_equal(idx[0], gold[f"r{n}_idx"]), n
        assert np.array_equal(bits(w[0]), bits(gold[f"r{n}_w"])), n
        assert keff[0] == K
        n += 1
    assert n >= 4
    for k in range(3):
        h = cref.swiglu_v4(gold["sw_g"], gold["sw_u"], float(gold[f"sw{k}_limit"][0]))
        assert np.array_equal(bits(h), bits(gold[f"sw{k}_h"])), k


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (needs the reference tree)")
def test_v4_vs_compiled_reference():
    ref = Ref()
    rng = np.random.default_rng(811)
    for t in range(40):
        E = int(rng.integers(8, 400))
        K = int(rng.integers(1, min(E, 16) + 1))
        z = (rng.standard_normal(E) * float(rng.uniform(0.1, 20))).astype(np.float32)
        b = (rng.standard_normal(E) * 0.1).astype(np.float32) if t % 2 else None
        rc, ridx, rw = ref.v4_route(z, K, b, 2.0)
        idx, w, _ = cref.route(z[None, :], K, 3, bias=b, routed_scale=2.0)
        assert rc == 0 and np.array_equal(idx[0], ridx) and np.array_equal(bits(w[0]), bits(rw)), t
    g = (rng.standard_normal(5000) * 8).astype(np.float32)
    u = (rng.standard_normal(5000) * 8).astype(np.float32)
    for limit in (0.0, 0.5, 3.0, 10.0):
        assert np.array_equal(bits(cref.swiglu_v4(g, u, limit)), bits(ref.v4_swiglu(g, u, limit)))


def test_v4_route_math():
    """Against float64: score = sqrt(log(1 + e^z)), selection by score + bias
    (a full stable sort gives the same top-K under a clear gap), weights =
    score / sum * scale; clamps of the V4 SwiGLU."""
    rng = np.random.default_rng(812)
    E, K = 96, 8
    z = (rng.standard_normal(E) * 4).astype(np.float32)
    b = (rng.standard_normal(E) * 0.05).astype(np.float32)
    sc = np.sqrt(np.logaddexp(0.0, z.astype(np.float64)))
    sel = sc + b
    order = np.argsort(-sel, kind="stable")[:K]
    idx, w, keff = cref.route(z[None, :], K, 3, bias=b, routed_scale=1.5)
    assert list(idx[0]) == list(order)
    assert np.allclose(w[0], sc[order] / sc[order].sum() * 1.5, rtol=2e-6)
    g = np.array([-3.0, 0.5, 2.0, 9.0], np.float32)
    u = np.array([-9.0, -0.5, 3.0, 0.25], np.float32)
    h = cref.swiglu_v4(g, u, 1.0).astype(np.float64)
    gc, uc = np.minimum(g, 1.0).astype(np.float64), np.clip(u, -1.0, 1.0).astype(np.float64)
    assert np.allclose(h, gc / (1 + np.exp(-gc)) * uc, rtol=1e-6)


def _f64_layer(fmt, x, W, b, experts, shared, K, mode, norm_topk, routed_scale):
    """The MoE layer in float64 from dequantized weights: routing by a full
    stable sort, silu(g) * u, the weighted sum over the selected experts in
    slot order, the shared expert added with weight 1."""
    D = x.shape[1]
    logits = cref.matmul_f32(x, W)
    if mode == 3:
        sc = np.sqrt(np.logaddexp(0.0, logits.astype(np.float64)))
        sel = sc + (b.astype(np.float64) if b is not None else 0.0)
        idx = np.argsort(-sel, axis=1, kind="stable")[:, :K]
        w = np.take_along_axis(sc, idx, axis=1)
        w = w / w.sum(axis=1, keepdims=True) * routed_scale
    else:
        idx, w = sort_route(logits, K, mode, b, norm_topk, routed_scale)

    def deq(m, I):
        q, s = m
        return deq_i4(q, s, I, 32) if fmt == 4 else deq_mxfp4(q, s, I)

    def act(v):
        return cref.qdq(v.astype(np.float32))[0].astype(np.float64) if fmt == 17 else v.astype(np.float64)

    def expert(trip, xs):
        g, u, d = trip
        gv = deq(g, D) @ act(xs)
        uv = deq(u, D) @ act(xs)
        h = gv / (1.0 + np.exp(-gv)) * uv
        dm = deq(d, h.size)
        return dm @ act(h), np.abs(dm) @ np.abs(h)

    out = np.zeros(x.shape, np.float64)
    mag = np.zeros(x.shape, np.float64)
    for s in range(x.shape[0]):
        terms = [(experts[int(e)], float(wk)) for e, wk in zip(idx[s], w[s])]
        if shared is not None:
            terms.append((shared, 1.0))
        for trip, wk in terms:
            y, m = expert(trip, x[s])
            out[s] += wk * y
            mag[s] += abs(wk) * m
    return idx, w, out, mag


@pytest.mark.parametrize("fmt", [4, 7, 17])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("shared", [False, True])
def test_moe_layer_vs_f64_composition(fmt, mode, shared):
    """cref_moe_layer (router -> top-K -> experts -> SwiGLU -> weighted sum
    -> shared expert, c/colibri.c:4467-4531 and 4940-5002) against the same
    layer evaluated in float64 from dequantized weights: indices exact under
    a 1e-4 rank-K gap, outputs within 2e-5 of the magnitude sum."""
    from moe_ref import make_router_inputs
    from oracle_lib import cref_moe_layer
    rng = np.random.default_rng(900 + 10 * fmt + mode + (5 if shared else 0))
    S, D, I, E, K = 5, 128, 128, 12, 3

    def mat(O, II):
        if fmt == 4:
            return rand_i4(rng, O, II, 32)
        return rand_mxfp4(rng, O, II)

    experts = [(mat(I, D), mat(I, D), mat(D, I)) for _ in range(E)]
    sh = (mat(I, D), mat(I, D), mat(D, I)) if shared else None
    x, W, b = make_router_inputs(rng, S, D, E, K, mode, bias=(mode != 0))
    norm = 1 if mode in (0, 1) else 0
    scale = 2.5 if mode in (1, 3) else 1.0
    out, idx, w, keff = cref_moe_layer(cref, fmt, x, W, b, experts, sh, K, mode,
                                       norm_topk=norm, routed_scale=scale)
    ri, rw, ref, mag = _f64_layer(fmt, x, W, b, experts, sh, K, mode, norm, scale)
    assert np.all(keff == K)
    assert np.array_equal(idx, ri)
    assert np.allclose(w, rw, rtol=2e-6, atol=0)
    err = np.abs(out.astype(np.float64) - ref) / np.maximum(mag, 1e-30)
    assert err.max() <= 2e-5, err.max()


# ---- fmt=2 with int8 activations (IDOT, c/quant.h:581-586, 674-801, 924-933) ----
def _idot_closed_form(x, q4, sc, O, I):
    """qrow_i8 in float32 numpy (IEEE round-to-nearest-even, as lrintf), the
    integer dot in int64, then (float)d * scale * sx in float32."""
    from quant_util import nibbles
    S = x.shape[0]
    y = np.empty((S, O), np.float32)
    w = (nibbles(q4, I) - 8).astype(np.int64)
    for s in range(S):
        amax = np.float32(np.max(np.abs(x[s]))) if I else np.float32(0)
        sx = np.float32(amax / np.float32(127.0))
        if sx < np.float32(1e-12):
            sx = np.float32(1e-12)
        inv = np.float32(np.float32(1.0) / sx)
        q = np.rint((x[s] * inv).astype(np.float32)).astype(np.int64)
        d = w @ q
        y[s] = (d.astype(np.float32) * sc.astype(np.float32)) * sx
    return y


def test_golden_idot():
    g = np.load(os.path.join(os.path.dirname(GOLDEN), "golden_idot.npz"))
    n = 0
    while f"c{n}_x" in g:
        S, I, O = (int(v) for v in g[f"c{n}_shape"])
        got = cref.matmul_i4_idot(g[f"c{n}_x"], g[f"c{n}_q4"], g[f"c{n}_sc"], O, I)
        assert np.array_equal(bits(got), bits(g[f"c{n}_y"])), n
        n += 1
    assert n >= 5


def test_idot_closed_form():
    rng = np.random.default_rng(4242)
    for S, I, O in [(1, 64, 9), (3, 255, 17), (2, 1024, 5)]:
        q4, sc = rand_i4(rng, O, I, 0, fp16_scales=False)
        x = (rng.standard_normal((S, I)) * 5).astype(np.float32)
        x[0, :4] = [0.5, -2.5, 127.0, 0.0]
        got = cref.matmul_i4_idot(x, q4, sc, O, I)
        assert np.array_equal(bits(got), bits(_idot_closed_form(x, q4, sc, O, I)))


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (needs the reference tree)")
def test_idot_vs_compiled_reference():
    ref = Ref()
    rng = np.random.default_rng(4343)
    for _ in range(25):
        S, I, O = int(rng.integers(1, 6)), int(rng.integers(1, 700)), int(rng.integers(1, 40))
        q4, sc = rand_i4(rng, O, I, 0, fp16_scales=False)
        x = (rng.standard_normal((S, I)) * 10 ** rng.uniform(-3, 3)).astype(np.float32)
        a = cref.matmul_i4_idot(x, q4, sc, O, I)
        b = ref.matmul_i4_idot(x, q4, sc, O, I)
        assert np.array_equal(bits(a), bits(b)), (S, I, O)
        qa, sa = cref.qrow_i8(x[0])
        qb, sb = ref.qrow_i8(x[0])
        assert np.array_equal(qa, qb) and sa == sb
