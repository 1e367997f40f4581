"""Fragments emitted by a GEMV's epilogue (coli_hip_gemm_run_dev_emit): the up
projection writes its output rows also as the down projection's activation
fragments (fp16 hi + lo, one exponent per row and 32-column group), and the
down GEMV reads them instead of a fragment build.

Parity: the down projection of the GPU's own up output, against the CPU
oracle on that output (c/quant.h matmul_i4_grouped / matmul_mxfp4), within
the 1e-3 bar; the up output itself is bitwise that of the plain run. The
entry point returns 2 when it emitted the fragments."""
import ctypes as C

import numpy as np
import pytest

from colibri_amd import hiprt
from oracle_lib import Cref
from quant_util import deq_i4, deq_mxfp4, magnitude, rand_i4, rand_mxfp4, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
cref = Cref()


def _dev(b, arr):
    p = b.cuda_pipe_alloc(0, max(arr.nbytes, 4))
    assert p and b.cuda_pipe_upload(0, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes)
    return p


def _get(b, p, shape):
    out = np.zeros(shape, np.float32)
    assert b.cuda_pipe_sync(0)
    assert b.cuda_pipe_download(0, p, out.ctypes.data_as(C.c_void_p), out.nbytes)
    return out


class Mat:
    def __init__(self, session, rng, kind, O, I):
        self.kind, self.O, self.I = kind, O, I
        if kind == "mx":
            self.q, self.e8 = rand_mxfp4(rng, O, I)
            self.h = session.upload_mxfp4(self.q, self.e8, I, O)
        else:
            self.q, self.sc = rand_i4(rng, O, I, 32, fp16_scales=kind == "i4h")
            self.h = session.upload(self.q, self.sc, 4, I, O, 32)

    def ref(self, x):
        if self.kind == "mx":
            return (cref.matmul_mxfp4(x, self.q, self.e8, self.O, self.I),
                    magnitude(x, deq_mxfp4(self.q, self.e8, self.I)))
        return (cref.matmul_i4_grouped(x, self.q, self.sc, self.O, self.I, 32),
                magnitude(x, deq_i4(self.q, self.sc, self.I, 32)))


def _chain(b, up, down, xd, hd, yd, S, emit):
    assert b.hip_gemm_prep_dev(up.h, xd, S)
    if emit:
        assert b.hip_gemm_run_dev_emit(up.h, hd, S, down.h) == 2   # emitted
    else:
        assert b.hip_gemm_run_dev(up.h, hd, S)
    assert b.hip_gemm_prep_dev(down.h, hd, S)
    assert b.hip_gemm_run_dev(down.h, yd, S)


# (4096, 12288) and (4096, 14336) at 1 row and (4096, 12288) at 2 and 4 rows:
# the LDS-ring kernel produces (f32 rows, two row tiles per wave) and consumes; the others: the tiled
# kernel on both sides, the down projection with K split across workgroups at
# the benchmark's shape (configs[1]: 4, 8 and 16 rows).
@pytest.mark.parametrize("kinds", [("i4h", "i4h"), ("i4f", "mx"), ("mx", "i4h"), ("mx", "mx")])
@pytest.mark.parametrize("D,H,S", [(4096, 12288, 1), (4096, 12288, 2), (4096, 12288, 4), (1024, 2048, 5),
                                   (1024, 2048, 8), (512, 1024, 16), (4096, 14336, 1), (4096, 14336, 4),
                                   (4096, 14336, 8), (4096, 14336, 16)])
def test_emitted_fragments_chain(session, monkeypatch, kinds, D, H, S):
    monkeypatch.setenv("COLI_HIP_EMIT", "force")
    b = session.b
    rng = np.random.default_rng(D + H + S + len(kinds[0]) * 7 + len(kinds[1]))
    up, down = Mat(session, rng, kinds[0], H, D), Mat(session, rng, kinds[1], D, H)
    x = rng.standard_normal((S, D)).astype(np.float32)
    xd = _dev(b, x)
    hd, yd = b.cuda_pipe_alloc(0, S * H * 4), b.cuda_pipe_alloc(0, S * D * 4)
    try:
        _chain(b, up, down, xd, hd, yd, S, emit=False)
        h_plain, y_plain = _get(b, hd, (S, H)), _get(b, yd, (S, D))
        _chain(b, up, down, xd, hd, yd, S, emit=True)
        h, y = _get(b, hd, (S, H)), _get(b, yd, (S, D))
        y2 = np.zeros_like(y)
        _chain(b, up, down, xd, hd, yd, S, emit=True)
        y2 = _get(b, yd, (S, D))
    finally:
        for p in (xd, hd, yd):
            b.cuda_pipe_free(0, p)
        session.free(up.h)
        session.free(down.h)
    assert np.array_equal(h.view(np.uint32), h_plain.view(np.uint32))
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))   # run to run
    ref, mag = down.ref(h)
    for got in (y, y_plain):
        e = rel_err(got, ref, mag)
        assert np.isfinite(got).all() and e.max() <= TOL, f"max rel err {e.max():.3e}"


def test_emitted_fragments_dropped_by_a_new_write(session, monkeypatch):
    """A plain run that rewrites the emitting GEMV's output drops the emitted
    fragments: the next prep builds from the new values."""
    monkeypatch.setenv("COLI_HIP_EMIT", "force")
    b = session.b
    rng = np.random.default_rng(7)
    D, H, S = 1024, 2048, 8
    up, down = Mat(session, rng, "i4h", H, D), Mat(session, rng, "i4h", D, H)
    x = rng.standard_normal((S, D)).astype(np.float32)
    x2 = (rng.standard_normal((S, D)) * 5).astype(np.float32)
    xd, x2d = _dev(b, x), _dev(b, x2)
    hd, yd = b.cuda_pipe_alloc(0, S * H * 4), b.cuda_pipe_alloc(0, S * D * 4)
    try:
        assert b.hip_gemm_prep_dev(up.h, xd, S) and b.hip_gemm_run_dev_emit(up.h, hd, S, down.h) == 2
        assert b.hip_gemm_prep_dev(up.h, x2d, S) and b.hip_gemm_run_dev(up.h, hd, S)
        assert b.hip_gemm_prep_dev(down.h, hd, S) and b.hip_gemm_run_dev(down.h, yd, S)
        h, y = _get(b, hd, (S, H)), _get(b, yd, (S, D))
    finally:
        for p in (xd, x2d, hd, yd):
            b.cuda_pipe_free(0, p)
        session.free(up.h)
        session.free(down.h)
    ref, mag = down.ref(h)
    e = rel_err(y, ref, mag)
    assert e.max() <= TOL, f"max rel err {e.max():.3e}"


def test_emitted_fragments_graph_replay(session, monkeypatch):
    """The chain captured in a HIP graph: every replay, with eager work on
    other inputs in between, equals the eager result bitwise."""
    monkeypatch.setenv("COLI_HIP_EMIT", "force")
    b = session.b
    st = b.hip_stream(0)
    rng = np.random.default_rng(11)
    D, H, S = 1024, 2048, 16
    up, down = Mat(session, rng, "i4h", H, D), Mat(session, rng, "mx", D, H)
    x = rng.standard_normal((S, D)).astype(np.float32)
    x2 = rng.standard_normal((S, D)).astype(np.float32)
    xd, x2d = _dev(b, x), _dev(b, x2)
    hd, yd = b.cuda_pipe_alloc(0, S * H * 4), b.cuda_pipe_alloc(0, S * D * 4)
    h2d, y2d = b.cuda_pipe_alloc(0, S * H * 4), b.cuda_pipe_alloc(0, S * D * 4)
    try:
        _chain(b, up, down, xd, hd, yd, S, emit=True)
        hiprt.device_sync()
        eager = _get(b, yd, (S, D))
        with hiprt.Graph(st) as g:
            _chain(b, up, down, xd, hd, yd, S, emit=True)
        for rep in range(3):
            b.hip_fill_random_u8(0, yd, S * D * 4, 5 + rep)
            b.hip_fill_random_u8(0, hd, S * H * 4, 9 + rep)
            g.launch()
            hiprt.device_sync()
            got = _get(b, yd, (S, D))
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {rep}"
            _chain(b, up, down, x2d, h2d, y2d, S, emit=True)
            hiprt.device_sync()
    finally:
        for p in (xd, x2d, hd, yd, h2d, y2d):
            b.cuda_pipe_free(0, p)
        session.free(up.h)
        session.free(down.h)


def test_emitted_fragments_chain_of_three(session, monkeypatch):
    """A -> B -> C with emission at every step: B reads the fragments A
    emitted, so it cannot emit into the same set and runs without emitting
    (returns 1); C's prep then builds its fragments. Every output within the
    bar against the oracle on the GPU's own inputs."""
    monkeypatch.setenv("COLI_HIP_EMIT", "force")
    b = session.b
    rng = np.random.default_rng(23)
    D, H, S = 1024, 2048, 8
    A, B, Cm = Mat(session, rng, "i4h", H, D), Mat(session, rng, "i4h", D, H), Mat(session, rng, "i4h", H, D)
    x = rng.standard_normal((S, D)).astype(np.float32)
    xd = _dev(b, x)
    ad, bd, cd = (b.cuda_pipe_alloc(0, S * n * 4) for n in (H, D, H))
    try:
        assert b.hip_gemm_prep_dev(A.h, xd, S) and b.hip_gemm_run_dev_emit(A.h, ad, S, B.h) == 2
        assert b.hip_gemm_prep_dev(B.h, ad, S) and b.hip_gemm_run_dev_emit(B.h, bd, S, Cm.h) == 1
        assert b.hip_gemm_prep_dev(Cm.h, bd, S) and b.hip_gemm_run_dev(Cm.h, cd, S)
        a_out, b_out, c_out = _get(b, ad, (S, H)), _get(b, bd, (S, D)), _get(b, cd, (S, H))
    finally:
        for p in (xd, ad, bd, cd):
            b.cuda_pipe_free(0, p)
        for m in (A, B, Cm):
            session.free(m.h)
    for m, inp, got in ((A, x, a_out), (B, a_out, b_out), (Cm, b_out, c_out)):
        ref, mag = m.ref(inp)
        e = rel_err(got, ref, mag)
        assert e.max() <= TOL, f"max rel err {e.max():.3e}"


@pytest.mark.parametrize("H,S", [(1000, 8), (2048, 1)])
def test_emission_declined(session, monkeypatch, H, S):
    """Where the launch cannot emit (up O not a multiple of 128) or it would
    not pay (one row: the down GEMV converts its f32 row itself), the call
    only runs the GEMV (returns 1) and the down GEMV's prep builds as usual."""
    b = session.b
    rng = np.random.default_rng(H + S)
    D = 512
    up, down = Mat(session, rng, "i4h", H, D), Mat(session, rng, "mx", D, H)
    x = rng.standard_normal((S, D)).astype(np.float32)
    xd = _dev(b, x)
    hd, yd = b.cuda_pipe_alloc(0, S * H * 4), b.cuda_pipe_alloc(0, S * D * 4)
    try:
        assert b.hip_gemm_prep_dev(up.h, xd, S) and b.hip_gemm_run_dev_emit(up.h, hd, S, down.h) == 1
        assert b.hip_gemm_prep_dev(down.h, hd, S) and b.hip_gemm_run_dev(down.h, yd, S)
        h, y = _get(b, hd, (S, H)), _get(b, yd, (S, D))
    finally:
        for p in (xd, hd, yd):
            b.cuda_pipe_free(0, p)
        session.free(up.h)
        session.free(down.h)
    for m, inp, got in ((up, x, h), (down, h, y)):
        ref, mag = m.ref(inp)
        e = rel_err(got, ref, mag)
        assert e.max() <= TOL, f"max rel err {e.max():.3e}"


@pytest.mark.parametrize("writer", ["noalloc", "idot", "silu_mul", "upload", "pipe_gemm"])
def test_emitted_fragments_dropped_by_other_writers(session, monkeypatch, writer):
    """Every entry point that writes a device buffer drops fragments emitted
    from it (the allocation-free GEMV, the fmt=2 int8-activation GEMV, the
    pipe element-wise ops and uploads, pipe_gemm): after the up GEMV emitted
    from hd and `writer` rewrote hd, the down projection is that of the new
    contents of hd, against the oracle."""
    monkeypatch.setenv("COLI_HIP_EMIT", "force")
    b = session.b
    rng = np.random.default_rng(11 + len(writer))
    D, H, S = 1024, 2048, 8
    up, down = Mat(session, rng, "i4h", H, D), Mat(session, rng, "i4h", D, H)
    x = rng.standard_normal((S, D)).astype(np.float32)
    other = (rng.standard_normal((S, D)) * 3).astype(np.float32)
    xd, od = _dev(b, x), _dev(b, other)
    hd, yd = b.cuda_pipe_alloc(0, S * H * 4), b.cuda_pipe_alloc(0, S * D * 4)
    extra = []
    try:
        assert b.hip_gemm_prep_dev(up.h, xd, S) and b.hip_gemm_run_dev_emit(up.h, hd, S, down.h) == 2
        if writer == "noalloc":
            assert b.hip_pipe_gemm_noalloc(up.h, hd, od, S)
        elif writer == "pipe_gemm":
            assert b.cuda_pipe_gemm(up.h, hd, od, S)
        elif writer == "idot":
            q2, s2 = rand_i4(rng, H, D, 0)
            h2 = session.upload(q2, s2, 2, D, H)
            extra.append(h2)
            assert b.hip_matmul_i4_idot_dev(h2, hd, od, S)
        elif writer == "silu_mul":
            ud = _dev(b, (rng.standard_normal((S, H)) * 2).astype(np.float32))
            extra.append(("dev", ud))
            assert b.cuda_pipe_silu_mul(0, hd, ud, S * H)
        else:
            new = rng.standard_normal((S, H)).astype(np.float32)
            assert b.cuda_pipe_upload(0, hd, new.ctypes.data_as(C.c_void_p), new.nbytes)
        assert b.hip_gemm_prep_dev(down.h, hd, S) and b.hip_gemm_run_dev(down.h, yd, S)
        h, y = _get(b, hd, (S, H)), _get(b, yd, (S, D))
    finally:
        for p in (xd, od, hd, yd):
            b.cuda_pipe_free(0, p)
        for e in extra:
            if isinstance(e, tuple):
                b.cuda_pipe_free(0, e[1])
            else:
                session.free(e)
        session.free(up.h)
        session.free(down.h)
    ref, mag = down.ref(h)
    e = rel_err(y, ref, mag)
    assert e.max() <= TOL, f"{writer}: max rel err {e.max():.3e}"
