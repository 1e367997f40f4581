"""GPU parity of the quantized GEMV through the C ABI (coli_cuda_matmul and
friends) against the CPU oracle (bit-exact restatement of c/quant.h)."""
import numpy as np
import pytest

from oracle_lib import Cref
from quant_util import (deq_i4, deq_mxfp4, magnitude, rand_i4, rand_mxfp4, rand_x, rel_err)

pytestmark = pytest.mark.gpu
TOL = 1e-3

cref = Cref()


def check(got, ref, mag, tol=TOL):
    e = rel_err(got, ref, mag)
    assert np.isfinite(got).all()
    assert e.max() <= tol, f"max rel err {e.max():.3e}"
    return e.max()


@pytest.mark.parametrize("O,I", [(64, 256), (1024, 2048), (48, 200), (17, 96), (2048, 1024)])
@pytest.mark.parametrize("S", [1, 2, 3, 4, 8, 16, 21])
def test_int4_g32_fp16_scales(session, O, I, S):
    rng = np.random.default_rng(O * 131 + I * 7 + S)
    q4, sc = rand_i4(rng, O, I, 32)
    x = rand_x(rng, S, I)
    h = session.upload(q4, sc, 4, I, O, 32)
    try:
        assert session.b.hip_tensor_kind(h) == 0
        y = session.matmul(h, x, 4, I, O, 32)
    finally:
        session.free(h)
    ref = cref.matmul_i4_grouped(x, q4, sc, O, I, 32)
    check(y, ref, magnitude(x, deq_i4(q4, sc, I, 32)))


def error_stats(tag, got, ref, mag):
    """Print the error distribution three ways: the test metric (|ref| with a
    floor of 1e-2 of the magnitude sum), |ref| alone, and the magnitude sum
    alone (the reference's own c/tests/test_i4_grouped.c metric)."""
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    r = np.abs(ref.astype(np.float64))
    m = rel_err(got, ref, mag)
    pure = d / np.where(r > 0, r, np.inf)
    print(f"\n[err] {tag}: metric max {m.max():.2e} p50 {np.median(m):.2e}; "
          f"|err|/|ref| max {pure.max():.2e} p99 {np.quantile(pure, 0.99):.2e} "
          f"(|ref| >= 1e-2 sum|t|: max {pure[r >= 1e-2 * mag].max():.2e}); "
          f"|err|/sum|t| max {(d / mag).max():.2e}; under the floor {(r < 1e-2 * mag).mean():.1%}")


# The dense benchmark shapes: the up projection runs one group per
# row block, the down projection splits K across workgroups. bf16-exact
# activations as the benchmark feeds them, and full f32 ones (lo parts).
@pytest.mark.parametrize("O,I", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("S", [1, 4, 8, 16])
@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_int4_dense_bench_shapes(session, O, I, S, act):
    rng = np.random.default_rng(O + I + S + (7 if act == "f32" else 0))
    q4, sc = rand_i4(rng, O, I, 32)
    x = rand_x(rng, S, I) if act == "bf16" else rng.standard_normal((S, I)).astype(np.float32)
    h = session.upload(q4, sc, 4, I, O, 32)
    try:
        y = session.matmul(h, x, 4, I, O, 32)
        y2 = session.matmul(h, x, 4, I, O, 32)
    finally:
        session.free(h)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))   # run-to-run bitwise
    ref = cref.matmul_i4_grouped(x, q4, sc, O, I, 32)
    mag = magnitude(x, deq_i4(q4, sc, I, 32))
    error_stats(f"int4 {O}x{I} S={S} {act}", y, ref, mag)
    check(y, ref, mag)


# The MXFP4 expert shapes of configs[2] (DeepSeek-V3: gate/up 2048 x 7168, down
# 7168 x 2048) at decode batches, full f32 activations.
@pytest.mark.parametrize("O,I", [(2048, 7168), (7168, 2048)])
@pytest.mark.parametrize("S", [1, 16])
def test_mxfp4_expert_shapes(session, O, I, S):
    rng = np.random.default_rng(O * 3 + I + S)
    q4, e8 = rand_mxfp4(rng, O, I)
    x = rng.standard_normal((S, I)).astype(np.float32)
    h = session.upload_mxfp4(q4, e8, I, O)
    try:
        y = session.matmul(h, x, 7, I, O)
    finally:
        session.free(h)
    ref = cref.matmul_mxfp4(x, q4, e8, O, I)
    mag = magnitude(x, deq_mxfp4(q4, e8, I))
    error_stats(f"mxfp4 {O}x{I} S={S} f32", y, ref, mag)
    check(y, ref, mag)


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("S", [1, 5])
def test_int4_f32_scales_and_group_sizes(session, gs, S):
    rng = np.random.default_rng(gs + S)
    O, I = 96, 640
    q4, sc = rand_i4(rng, O, I, gs, fp16_scales=False)
    x = rng.standard_normal((S, I)).astype(np.float32)   # not bf16-exact: exercises the lo MFMA
    h = session.upload(q4, sc, 4, I, O, gs)
    try:
        assert session.b.hip_tensor_kind(h) == 1
        y = session.matmul(h, x, 4, I, O, gs)
    finally:
        session.free(h)
    ref = cref.matmul_i4_grouped(x, q4, sc, O, I, gs)
    check(y, ref, magnitude(x, deq_i4(q4, sc, I, gs)))


def test_int4_per_row_fmt2(session):
    rng = np.random.default_rng(3)
    O, I, S = 80, 333, 3
    q4, sc = rand_i4(rng, O, I, 0)
    x = rand_x(rng, S, I)
    h = session.upload(q4, sc, 2, I, O, 0)
    try:
        y = session.matmul(h, x, 2, I, O, 0)
    finally:
        session.free(h)
    ref = cref.matmul_i4(x, q4, sc, O, I)
    check(y, ref, magnitude(x, deq_i4(q4, sc, I, 0)))


def test_int4_generic_group16(session):
    rng = np.random.default_rng(4)
    O, I, S = 40, 200, 2
    q4, sc = rand_i4(rng, O, I, 16)
    x = rand_x(rng, S, I)
    h = session.upload(q4, sc, 4, I, O, 16)
    try:
        assert session.b.hip_tensor_kind(h) == 3
        y = session.matmul(h, x, 4, I, O, 16)
    finally:
        session.free(h)
    ref = cref.matmul_i4_grouped(x, q4, sc, O, I, 16)
    check(y, ref, magnitude(x, deq_i4(q4, sc, I, 16)))


def test_int4_nibble_edges_closed_form(session):
    """Unit scales and x = e_i return the nibble value - 8 exactly (0x00 -> -8, 0xF -> +7)."""
    O, I = 16, 128
    q4 = np.zeros((O, I // 2), np.uint8)
    q4[:, 0] = 0xF0        # column 0 -> nibble 0 (-8), column 1 -> nibble 15 (+7)
    sc = np.ones((O, I // 32), np.float32)
    x = np.zeros((2, I), np.float32)
    x[0, 0] = 1.0
    x[1, 1] = 1.0
    h = session.upload(q4, sc, 4, I, O, 32)
    try:
        y = session.matmul(h, x, 4, I, O, 32)
    finally:
        session.free(h)
    assert (y[0] == -8.0).all() and (y[1] == 7.0).all()


@pytest.mark.parametrize("O,I", [(64, 256), (2048, 7168), (7168, 2048), (40, 96)])
@pytest.mark.parametrize("S", [1, 4, 16])
def test_mxfp4(session, O, I, S):
    rng = np.random.default_rng(O + I + S)
    q4, e8 = rand_mxfp4(rng, O, I)
    x = rand_x(rng, S, I)
    h = session.upload_mxfp4(q4, e8, I, O)
    try:
        assert session.b.hip_tensor_kind(h) == 2
        y = session.matmul(h, x, 7, I, O, 32)
    finally:
        session.free(h)
    ref = cref.matmul_mxfp4(x, q4, e8, O, I)
    check(y, ref, magnitude(x, deq_mxfp4(q4, e8, I)))


def test_mxfp4_all_codes_exact(session):
    """One column set to code c, x = 1: the result is the decoded value
    (c/tests/test_mxfp4_cuda.cu:106-132)."""
    want = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    I, O = 32, 16
    q4 = np.zeros((O, I // 2), np.uint8)
    q4[:, 0] = np.arange(16, dtype=np.uint8)
    e8 = np.full((O, 1), 127, np.uint8)
    x = np.zeros((1, I), np.float32)
    x[0, 0] = 1.0
    y = np.zeros((1, O), np.float32)
    from colibri_amd.backend import f32p, u8p
    assert session.b.cuda_matmul_mxfp4(f32p(y), f32p(x), u8p(q4), u8p(e8), 1, I, O)
    assert np.array_equal(y[0], want)


@pytest.mark.parametrize("e", [0, 127, 255])
def test_mxfp4_scale_edges(session, e):
    """e8m0 0 -> +0 and 255 -> +inf follow quant.h's bit trick (c/quant.h:1375-1390)."""
    rng = np.random.default_rng(e)
    O, I = 16, 64
    q4 = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    e8 = np.full((O, 2), e, np.uint8)
    x = rng.standard_normal((1, I)).astype(np.float32)
    y = np.zeros((1, O), np.float32)
    from colibri_amd.backend import f32p, u8p
    assert session.b.cuda_matmul_mxfp4(f32p(y), f32p(x), u8p(q4), u8p(e8), 1, I, O)
    ref = cref.matmul_mxfp4(x, q4, e8, O, I)
    if e == 0:
        assert np.array_equal(y, ref) and (y == 0).all()
    elif e == 255:
        # +inf scales: every output is non-finite on both sides; which ones end
        # as inf and which as NaN depends on how partial sums of opposite sign
        # meet (the reference's 8-lane accumulator mixes them into NaN), the
        # same latitude c/tests/test_mxfp4_cuda.cu:84-92 gives the CUDA kernel.
        assert not np.isfinite(y).any() and not np.isfinite(ref).any()
    else:
        check(y, ref, magnitude(x, deq_mxfp4(q4, e8, I)))


@pytest.mark.parametrize("S,I,O", [(1, 80, 8), (4, 128, 64), (1, 2048, 16), (3, 96, 8)])
def test_matmul_mxfp4_stateless(session, S, I, O):
    rng = np.random.default_rng(S * I + O)
    q4, e8 = rand_mxfp4(rng, O, I, 110, 139)
    x = rng.standard_normal((S, I)).astype(np.float32)
    y = np.zeros((S, O), np.float32)
    from colibri_amd.backend import f32p, u8p
    assert session.b.cuda_matmul_mxfp4(f32p(y), f32p(x), u8p(q4), u8p(e8), S, I, O)
    ref = cref.matmul_mxfp4(x, q4, e8, O, I)
    check(y, ref, magnitude(x, deq_mxfp4(q4, e8, I)))


@pytest.mark.parametrize("S", [1, 3])
def test_fp4_native_quant_contract(session, S):
    """coli_hip_fp4_matmul_qdq == e4m3 QDQ (block 128) + fmt=7 GEMV
    (coli_fp4_matmul_batch_ref, c/deepseek_v4.c:10906-10933)."""
    rng = np.random.default_rng(10 + S)
    O, I = 256, 1024
    q4, e8 = rand_mxfp4(rng, O, I)
    x = (rng.standard_normal((S, I)) * 3).astype(np.float32)
    h = session.upload_mxfp4(q4, e8, I, O)
    y = np.zeros((S, O), np.float32)
    from colibri_amd.backend import f32p
    try:
        assert session.b.hip_fp4_matmul_qdq(h, f32p(y), f32p(x), S)
    finally:
        session.free(h)
    ref = cref.fp4_matmul_batch(x, q4, e8, O, I)
    xq = np.stack([cref.qdq(x[s])[0] for s in range(S)])
    check(y, ref, magnitude(xq, deq_mxfp4(q4, e8, I)))


@pytest.mark.parametrize("S,I,O", [(1, 512, 64), (4, 2048, 256), (16, 256, 33), (3, 100, 9)])
def test_matmul_mxfp4_i8(session, S, I, O):
    """coli_hip_matmul_mxfp4_i8 (stateless) and coli_hip_fp4_matmul_i8
    (resident) against the oracle's matmul_mxfp4_i8 (c/quant.h:1441-1515,
    int8 activations per 32 columns; I % 32 != 0 is the float path)."""
    rng = np.random.default_rng(900 + S * I + O)
    q4, e8 = rand_mxfp4(rng, O, I, 110, 139)
    x = (rng.standard_normal((S, I)) * 2).astype(np.float32)
    x[0, :min(I, 32)] = 0.0          # one all-zero group (scale floor)
    from colibri_amd.backend import f32p, u8p
    ref = cref.matmul_mxfp4_i8(x, q4, e8, O, I)
    y = np.zeros((S, O), np.float32)
    assert session.b.hip_matmul_mxfp4_i8(f32p(y), f32p(x), u8p(q4), u8p(e8), S, I, O)
    check(y, ref, magnitude(x, deq_mxfp4(q4, e8, I)))
    h = session.upload_mxfp4(q4, e8, I, O)
    y2 = np.zeros((S, O), np.float32)
    try:
        assert session.b.hip_fp4_matmul_i8(h, f32p(y2), f32p(x), S)
    finally:
        session.free(h)
    assert np.array_equal(y, y2)


def test_fp4_matvec_kat(session):
    """weights 0x44 (+2.0, +2.0), scale 0x7e (0.5), x = 1 over 128 columns gives
    exactly 128.0 (c/tests/test_native_quant.c:76-88)."""
    q4 = np.full((1, 64), 0x44, np.uint8)
    e8 = np.full((1, 4), 0x7E, np.uint8)
    x = np.ones((1, 128), np.float32)
    h = session.upload_mxfp4(q4, e8, 128, 1)
    y = np.zeros((1, 1), np.float32)
    from colibri_amd.backend import f32p
    try:
        assert session.b.hip_fp4_matmul_qdq(h, f32p(y), f32p(x), 1)
    finally:
        session.free(h)
    assert y[0, 0] == 128.0


def wild_x(rng, S, I):
    """Activations that stress the per-quad exponent of the f32 path: full
    f32 mantissas (lo parts), quads scaled by 2^-24 .. 2^20, an all-zero
    quad, subnormals and one quad holding a single large value."""
    x = rng.standard_normal((S, I)).astype(np.float32)
    nq = (I + 127) // 128
    for s in range(S):
        for q in range(nq):
            x[s, 128 * q:128 * (q + 1)] *= np.float32(2.0 ** int(rng.integers(-24, 21)))
    if nq > 1:
        x[:, 128:256] = 0.0
    x[0, :16] = np.float32(1e-40)
    if nq > 2:
        x[-1, 256:384] = 0.0
        x[-1, 300] = 3.0e4
    return x


def outlier_x(rng, S, I):
    """Gaussian rows with a few massive activations (up to 1e6 x typical):
    with the fragments scaled to [0.5, 1) of the row maximum instead of the
    top of the fp16 range, the typical values turned subnormal and these rows
    failed the tolerance."""
    x = rng.standard_normal((S, I)).astype(np.float32)
    amp = [1e2, 3e4, 1e6, 5e3]
    for s in range(S):
        x[s, 7] = amp[s % 4]
        x[s, (131 * s + 300) % I] = -amp[(s + 1) % 4] / 3
    return x


# Both GEMV kernels and both activation paths of the LDS-ring kernel (f32
# rows converted in the kernel, per-quad exponents; or prepared fragments,
# per-row exponents) on the same inputs, including wild_x's 2^44 range across
# a row on every path and batch size: values far below the row maximum lose
# bits on the per-row-exponent paths, but their terms are as small against
# the magnitude sum, and every output stays within the bar.
@pytest.mark.parametrize("mode", [("dma", "1"), ("dma", "1", "stage0"), ("dma", "0"), ("tiles", "1")])
@pytest.mark.parametrize("fmt", ["i4h", "i4f", "mx"])
@pytest.mark.parametrize("S", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("O,I,xkind", [(256, 1024, "bf16"), (96, 768, "wild"), (128, 640, "outlier"),
                                       (40, 384, "f32"), (48, 200, "f32")])
def test_gemv_kernel_paths(session, monkeypatch, mode, fmt, S, O, I, xkind):
    monkeypatch.setenv("COLI_HIP_GEMV", mode[0])
    monkeypatch.setenv("COLI_HIP_XF32", mode[1])
    # one-row f32 GEMVs: the row staged once per workgroup (default) or per stage
    monkeypatch.setenv("COLI_HIP_XSTAGE", "0" if len(mode) > 2 else "1")
    rng = np.random.default_rng(S * 1000 + O + I)
    if xkind == "bf16":
        x = rand_x(rng, S, I)
    elif xkind == "wild":
        x = wild_x(rng, S, I)
    elif xkind == "outlier":
        x = outlier_x(rng, S, I)
    else:
        x = rng.standard_normal((S, I)).astype(np.float32)
    if fmt == "mx":
        q4, e8 = rand_mxfp4(rng, O, I)
        h = session.upload_mxfp4(q4, e8, I, O)
        ref = cref.matmul_mxfp4(x, q4, e8, O, I)
        mag = magnitude(x, deq_mxfp4(q4, e8, I))
        fmtc, gs = 7, 32
    else:
        q4, sc = rand_i4(rng, O, I, 32, fp16_scales=fmt == "i4h")
        h = session.upload(q4, sc, 4, I, O, 32)
        ref = cref.matmul_i4_grouped(x, q4, sc, O, I, 32)
        mag = magnitude(x, deq_i4(q4, sc, I, 32))
        fmtc, gs = 4, 32
    try:
        y = session.matmul(h, x, fmtc, I, O, gs)
        y2 = session.matmul(h, x, fmtc, I, O, gs)
    finally:
        session.free(h)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    check(y, ref, mag)


# fmt=2 with int8 activations (the reference's IDOT path for fmt=2 experts,
# c/colibri.c:937-945): bitwise equal to the oracle, which is pinned bitwise
# to the reference's qrow_i8 + matmul_i4_idot.
@pytest.mark.parametrize("O,I,S,fp16", [(64, 256, 1, True), (1024, 2048, 4, True), (100, 97, 3, False),
                                        (4096, 14336, 2, True), (48, 640, 16, False), (300, 512, 40, True)])
def test_int4_fmt2_int8_activations(session, O, I, S, fp16):
    import ctypes as C
    from colibri_amd.backend import f32p
    rng = np.random.default_rng(O * 3 + I + S)
    q4, sc = rand_i4(rng, O, I, 0, fp16_scales=fp16)
    x = (rng.standard_normal((S, I)) * 3).astype(np.float32)
    x[0, :3] = [0.5, -2.5, 0.0]
    h = session.upload(q4, sc, 2, I, O)
    y = np.zeros((S, O), np.float32)
    b = session.b
    try:
        assert b.hip_tensor_kind(h) == (0 if fp16 else 1)
        assert b.hip_matmul_i4_idot(h, f32p(y), f32p(x), S)
        # device-pointer form, twice (the unit scales are made on first use)
        px, py = b.cuda_pipe_alloc(0, x.nbytes), b.cuda_pipe_alloc(0, y.nbytes)
        try:
            assert b.cuda_pipe_upload(0, px, x.ctypes.data_as(C.c_void_p), x.nbytes)
            assert b.hip_matmul_i4_idot_dev(h, py, px, S)
            y2 = np.zeros_like(y)
            assert b.cuda_pipe_sync(0)
            assert b.cuda_pipe_download(0, py, y2.ctypes.data_as(C.c_void_p), y2.nbytes)
        finally:
            b.cuda_pipe_free(0, px)
            b.cuda_pipe_free(0, py)
    finally:
        session.free(h)
    ref = cref.matmul_i4_idot(x, q4, sc, O, I)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), np.abs(y - ref).max()
    assert np.array_equal(y2.view(np.uint32), ref.view(np.uint32))


def test_int4_fmt2_int8_activations_refusals(session):
    from colibri_amd.backend import f32p
    rng = np.random.default_rng(5)
    q4, sc = rand_i4(rng, 32, 256, 32)
    h = session.upload(q4, sc, 4, 256, 32, 32)          # fmt=4: not this path
    x = rand_x(rng, 1, 256)
    y = np.full((1, 32), 3.0, np.float32)
    try:
        assert not session.b.hip_matmul_i4_idot(h, f32p(y), f32p(x), 1)
    finally:
        session.free(h)
    assert np.all(y == 3.0)
    q4, sc = rand_i4(rng, 16, 16640, 0)                  # I > 16512: an f32 partial sum could round
    h = session.upload(q4, sc, 2, 16640, 16)
    x = rand_x(rng, 1, 16640)
    y = np.full((1, 16), 3.0, np.float32)
    try:
        assert not session.b.hip_matmul_i4_idot(h, f32p(y), f32p(x), 1)
    finally:
        session.free(h)
    assert np.all(y == 3.0)
