"""The allocation-free GEMV entry point (coli_hip_pipe_gemm_noalloc) against
coli_cuda_pipe_gemm through the C ABI: bitwise equal on two calls in a row,
the second with a smaller input, for every storage kind and for shapes that
take the split-K path (its partials and counters live in the static scratch
too); refusal beyond the stated limits."""
import ctypes as C

import numpy as np
import pytest

from colibri_amd.backend import f32p
from quant_util import rand_i4, rand_mxfp4, rand_x

pytestmark = pytest.mark.gpu


def run(session, fn, h, x, O):
    b = session.b
    S, I = x.shape
    px = b.cuda_pipe_alloc(0, x.nbytes)
    py = b.cuda_pipe_alloc(0, S * O * 4)
    try:
        assert b.cuda_pipe_upload(0, px, x.ctypes.data_as(C.c_void_p), x.nbytes)
        assert fn(h, py, px, S)
        assert b.cuda_pipe_sync(0)
        y = np.empty((S, O), np.float32)
        assert b.cuda_pipe_download(0, py, y.ctypes.data_as(C.c_void_p), y.nbytes)
    finally:
        b.cuda_pipe_free(0, px)
        b.cuda_pipe_free(0, py)
    return y


@pytest.mark.parametrize("kind,O,I,S1,S2", [
    ("i4h", 4096, 14336, 16, 3),     # dense down: split-K partials in the scratch
    ("i4h", 14336, 4096, 8, 1),
    ("i4f", 512, 1024, 5, 2),
    ("fp4", 2048, 7168, 4, 1),
    ("fp4", 7168, 2048, 16, 9),
    ("gen", 96, 200, 3, 1),          # group size 40: the generic kernel
])
def test_noalloc_matches_pipe_gemm(session, kind, O, I, S1, S2):
    rng = np.random.default_rng(O + I + S1)
    if kind == "fp4":
        q4, e8 = rand_mxfp4(rng, O, I)
        h = session.upload_mxfp4(q4, e8, I, O)
    elif kind == "gen":
        q4, sc = rand_i4(rng, O, I, 40, fp16_scales=False)
        h = session.upload(q4, sc, 4, I, O, 40)
    else:
        q4, sc = rand_i4(rng, O, I, 32, fp16_scales=(kind == "i4h"))
        h = session.upload(q4, sc, 4, I, O, 32)
    try:
        for S in (S1, S2):
            x = rand_x(rng, S, I) if S != 9 else rng.standard_normal((S, I)).astype(np.float32)
            ref = run(session, session.b.cuda_pipe_gemm, h, x, O)
            got = run(session, session.b.hip_pipe_gemm_noalloc, h, x, O)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (S, np.abs(got - ref).max())
    finally:
        session.free(h)


def test_noalloc_allocates_nothing(session):
    """Called first on shapes this context has not run (larger than anything
    pipe_gemm sized its buffers for here), the entry point leaves the device's
    free memory unchanged: its fragments, lo flag and split-K partials and
    counters are all in the static scratch. A small pipe_gemm first loads the
    library's code and creates the context's (small) buffers, so growing them
    would show as an allocation."""
    b = session.b
    rng = np.random.default_rng(5)
    qs, ss = rand_i4(rng, 32, 128, 32)
    hs = session.upload(qs, ss, 4, 128, 32, 32)
    run(session, b.cuda_pipe_gemm, hs, rand_x(rng, 1, 128), 32)
    session.free(hs)
    O, I, S = 2048, 16384, 16           # split-K shape at the row and K limits
    q4, sc = rand_i4(rng, O, I, 32)
    h = session.upload(q4, sc, 4, I, O, 32)
    x = rng.standard_normal((S, I)).astype(np.float32)
    px, py = b.cuda_pipe_alloc(0, x.nbytes), b.cuda_pipe_alloc(0, S * O * 4)
    try:
        assert b.cuda_pipe_upload(0, px, x.ctypes.data_as(C.c_void_p), x.nbytes)
        assert b.cuda_pipe_sync(0)
        free0, free1, total = C.c_size_t(), C.c_size_t(), C.c_size_t()
        assert b.cuda_mem_info(0, C.byref(free0), C.byref(total))
        for _ in range(2):
            assert b.hip_pipe_gemm_noalloc(h, py, px, S)
        assert b.cuda_pipe_sync(0)
        assert b.cuda_mem_info(0, C.byref(free1), C.byref(total))
        assert free1.value == free0.value, (free0.value, free1.value)
        got = np.empty((S, O), np.float32)
        assert b.cuda_pipe_download(0, py, got.ctypes.data_as(C.c_void_p), got.nbytes)
    finally:
        b.cuda_pipe_free(0, px)
        b.cuda_pipe_free(0, py)
    try:
        ref = run(session, b.cuda_pipe_gemm, h, x, O)
    finally:
        session.free(h)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_refuses_beyond_limits(session):
    rng = np.random.default_rng(3)
    O, I = 64, 256
    q4, sc = rand_i4(rng, O, I, 32)
    h = session.upload(q4, sc, 4, I, O, 32)
    b = session.b
    try:
        px = b.cuda_pipe_alloc(0, 17 * I * 4)
        py = b.cuda_pipe_alloc(0, 17 * O * 4)
        assert not b.hip_pipe_gemm_noalloc(h, py, px, 17)       # 17 rows > 16
        b.cuda_pipe_free(0, px)
        b.cuda_pipe_free(0, py)
    finally:
        session.free(h)
    big = rand_i4(rng, 16, 16512, 32)
    hb = session.upload(big[0], big[1], 4, 16512, 16, 32)
    try:
        px = b.cuda_pipe_alloc(0, 16512 * 4)
        py = b.cuda_pipe_alloc(0, 16 * 4)
        assert not b.hip_pipe_gemm_noalloc(hb, py, px, 1)        # I > 16384
        b.cuda_pipe_free(0, px)
        b.cuda_pipe_free(0, py)
    finally:
        session.free(hb)
