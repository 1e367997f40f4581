"""HIP-graph replay of the device entry points (the benchmark's timing mode).

A captured graph freezes kernel arguments, including the generation number of
the activation fragments' lo flag; the GEMV treats any flag >= its generation
as "lo present", so replays stay exact. Every replay, with other eager work and
synchronisations in between, must match the eager result bitwise.
"""
import ctypes as C

import numpy as np
import pytest

from colibri_amd import hiprt
from colibri_amd.backend import ColiHipMoeConfig, f32p, i32p, tensor_array
from moe_ref import Layer, free_handles, make_router_inputs
from quant_util import rand_i4, rand_mxfp4

pytestmark = pytest.mark.gpu


def _dev(b, arr):
    p = b.cuda_pipe_alloc(0, arr.nbytes)
    assert p and b.cuda_pipe_upload(0, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes)
    return p


def _get(b, p, shape):
    out = np.zeros(shape, np.float32)
    assert b.cuda_pipe_download(0, p, out.ctypes.data_as(C.c_void_p), out.nbytes)
    return out


# (200, 384): one group per row block; (128, 16384): long K split across
# workgroups, whose arrival counters must be back at zero after every launch;
# (4096, 4096): the LDS-ring kernel on f32 rows (one row: staged once per
# workgroup; three rows: converted per stage).
@pytest.mark.parametrize("fmt", [4, 7])
@pytest.mark.parametrize("O,I,S", [(200, 384, 3), (128, 16384, 3), (4096, 4096, 1), (4096, 4096, 3)])
def test_gemm_graph_replays_match_eager(session, fmt, O, I, S):
    b = session.b
    st = b.hip_stream(0)
    rng = np.random.default_rng(50 + fmt + I + S)
    if fmt == 4:
        q4, sc = rand_i4(rng, O, I, 32)
        h = session.upload(q4, sc, 4, I, O, 32)
    else:
        q4, e8 = rand_mxfp4(rng, O, I)
        h = session.upload_mxfp4(q4, e8, I, O)
    # full f32 inputs: the lo fragments are non-zero
    x = rng.standard_normal((S, I)).astype(np.float32)
    x2 = rng.standard_normal((S, I)).astype(np.float32) * 3
    xd, x2d = _dev(b, x), _dev(b, x2)
    yd = b.cuda_pipe_alloc(0, S * O * 4)
    y2d = b.cuda_pipe_alloc(0, S * O * 4)
    try:
        assert b.hip_gemm_prep_dev(h, xd, S) and b.hip_gemm_run_dev(h, yd, S)
        hiprt.device_sync()
        eager = _get(b, yd, (S, O))
        with hiprt.Graph(st) as g:
            assert b.hip_gemm_prep_dev(h, xd, S)
            assert b.hip_gemm_run_dev(h, yd, S)
        for rep in range(3):
            b.hip_fill_random_u8(0, yd, S * O * 4, 99 + rep)   # poison the output
            g.launch()
            hiprt.device_sync()
            got = _get(b, yd, (S, O))
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {rep}"
            # eager work on other inputs between replays (new fragments, new lo flag generation)
            assert b.hip_gemm_prep_dev(h, x2d, S) and b.hip_gemm_run_dev(h, y2d, S)
            hiprt.device_sync()
    finally:
        for p in (xd, x2d, yd, y2d):
            b.cuda_pipe_free(0, p)
        session.free(h)


# (256, 16): routing in one launch; (1536, 256): router partials, then the
# selection and union in one launch (both with arrival counters that must be
# back at zero after every replay)
# The last case is one token at OLMoE's shapes (routing in one launch, the
# one-token gate/up and down + combine kernels).
@pytest.mark.parametrize("D,E,I,K,S,olmoe", [(256, 16, 128, 4, 5, False), (1536, 256, 128, 4, 5, False),
                                             (2048, 64, 1024, 8, 1, True)])
def test_moe_graph_replays_match_eager(session, D, E, I, K, S, olmoe):
    b = session.b
    st = b.hip_stream(0)
    rng = np.random.default_rng(61 + E)
    fmt, mode = (4, 0) if olmoe else (7, 1)
    layer = Layer(rng, fmt, D, I, E, shared=not olmoe, distinct=4 if olmoe else None)
    x, W, bias = make_router_inputs(rng, S, D, E, K, mode, bias=not olmoe)
    hs = layer.upload(session)
    g_, ga = tensor_array([t[0] for t in hs[:E]])
    u_, ua = tensor_array([t[1] for t in hs[:E]])
    d_, da = tensor_array([t[2] for t in hs[:E]])
    if olmoe:
        cfg = ColiHipMoeConfig(D, I, E, K, 0, 0, 0.0, 1.0, 0)
        m = C.c_void_p()
        assert b.hip_moe_create(C.byref(m), 0, C.byref(cfg), f32p(W), None, g_, u_, d_, None, None, None)
    else:
        cfg = ColiHipMoeConfig(D, I, E, K, 1, 1, 0.0, 2.5, 1)
        m = C.c_void_p()
        assert b.hip_moe_create(C.byref(m), 0, C.byref(cfg), f32p(W), f32p(bias), g_, u_, d_, hs[E][0], hs[E][1],
                                hs[E][2])
    xd = _dev(b, np.ascontiguousarray(x))
    x2d = _dev(b, np.ascontiguousarray(x[::-1] * 2))
    od = b.cuda_pipe_alloc(0, S * D * 4)
    o2d = b.cuda_pipe_alloc(0, S * D * 4)
    try:
        assert b.hip_moe_forward_dev(m, xd, od, S)
        hiprt.device_sync()
        eager = _get(b, od, (S, D))
        with hiprt.Graph(st) as g:
            assert b.hip_moe_forward_dev(m, xd, od, S)
        for rep in range(3):
            b.hip_fill_random_u8(0, od, S * D * 4, 7 + rep)
            g.launch()
            hiprt.device_sync()
            got = _get(b, od, (S, D))
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {rep}"
            assert b.hip_moe_forward_dev(m, x2d, o2d, S)
            hiprt.device_sync()
    finally:
        b.hip_moe_free(m)
        for p in (xd, x2d, od, o2d):
            b.cuda_pipe_free(0, p)
        free_handles(session, hs)


def test_idot_graph_replay_ignores_later_lo_flag(session):
    """The fmt=2 int8-activation GEMV builds hi parts only; a captured call
    replayed after eager GEMVs on the same fragment set raised that set's lo
    flag (full f32 inputs) still takes no lo parts: every replay is bitwise
    the eager result."""
    b = session.b
    st = b.hip_stream(0)
    rng = np.random.default_rng(933)
    O, I, S = 512, 1024, 3
    q2, s2 = rand_i4(rng, O, I, 0)
    h2 = session.upload(q2, s2, 2, I, O)
    q4, s4 = rand_i4(rng, O, I, 32)
    h4 = session.upload(q4, s4, 4, I, O, 32)
    x = rng.standard_normal((S, I)).astype(np.float32)
    xf = rng.standard_normal((S, I)).astype(np.float32) * 3   # lo parts non-zero
    xd, xfd = _dev(b, x), _dev(b, xf)
    yd, y2d = b.cuda_pipe_alloc(0, S * O * 4), b.cuda_pipe_alloc(0, S * O * 4)
    try:
        assert b.hip_matmul_i4_idot_dev(h2, yd, xd, S)
        hiprt.device_sync()
        eager = _get(b, yd, (S, O))
        with hiprt.Graph(st) as g:
            assert b.hip_matmul_i4_idot_dev(h2, yd, xd, S)
        for rep in range(3):
            # eager GEMVs of the same input kind with lo parts: the set's flag moves on
            assert b.hip_gemm_prep_dev(h4, xfd, S) and b.hip_gemm_run_dev(h4, y2d, S)
            assert b.cuda_pipe_gemm(h4, y2d, xfd, S)
            hiprt.device_sync()
            b.hip_fill_random_u8(0, yd, S * O * 4, 7 + rep)
            g.launch()
            hiprt.device_sync()
            got = _get(b, yd, (S, O))
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {rep}"
    finally:
        for p in (xd, xfd, yd, y2d):
            b.cuda_pipe_free(0, p)
        session.free(h2)
        session.free(h4)
