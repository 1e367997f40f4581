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
