"""GPU parity of the reference-ABI entry points the engine calls outside the
GEMV hot loop (c/backend_cuda.h), each through the C ABI against the CPU
oracle or a closed form:

* coli_cuda_tensor_upload_g with fmt=7 and f32 power-of-two scales, gs=32
  (the resident MXFP4 convention of docs/FORMATS.md:68), and its refusal of a
  scale that is not a power of two;
* coli_cuda_tensor_update (c/backend_cuda.h:153) for fmt 4 and 7: the new
  contents are what the next GEMV computes with, on the same handle;
* coli_cuda_shared_mlp_w4a16 (c/backend_cuda.cu:1457-1484): fmt=2 tensors,
  other formats refused;
* coli_cuda_pipe_silu_mul / pipe_add / pipe_rows_add / pipe_copy2d
  (c/backend_cuda.cu:2073-2078, 2317-2368);
* coli_hip_tensor_upload_fp4_rows16, fed by the oracle's rows16 packer
  (cref_fp4_pack_rows16, pinned bitwise to coli_fp4_pack_rows16_v10);
* the expert group's two staging routes (copy kernels and DMA copies).
"""
import ctypes as C

import numpy as np
import pytest

from colibri_amd.backend import f32p, i32p, tensor_array
from moe_ref import Layer
from oracle_lib import Cref
from quant_util import deq_i4, deq_mxfp4, magnitude, rand_i4, rand_mxfp4, rand_x, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
cref = Cref()


def e8_to_f32(e8):
    return (e8.astype(np.uint32) << 23).view(np.float32)


@pytest.mark.parametrize("O,I,S", [(96, 256, 1), (2048, 7168, 3), (40, 200, 5)])
def test_upload_g_fmt7_pow2_scales(session, O, I, S):
    """Resident MXFP4 through the engine's own upload route: f32 scales that
    are exact powers of two (incl. +0 for an all-zero block), gs = 32."""
    rng = np.random.default_rng(O + I + S)
    q4, e8 = rand_mxfp4(rng, O, I)
    e8[0, 0] = 0
    x = rand_x(rng, S, I)
    h = session.upload(q4, e8_to_f32(e8), 7, I, O, 32)
    try:
        assert session.b.hip_tensor_kind(h) == 2
        y = session.matmul(h, x, 7, I, O, 32)
    finally:
        session.free(h)
    ref = cref.matmul_mxfp4(x, q4, e8, O, I)
    assert rel_err(y, ref, magnitude(x, deq_mxfp4(q4, e8, I))).max() <= TOL


def test_upload_g_fmt7_refuses_non_pow2(session):
    rng = np.random.default_rng(4)
    O, I = 32, 128
    q4, e8 = rand_mxfp4(rng, O, I)
    sc = e8_to_f32(e8)
    sc[3, 1] *= 1.5
    h = C.c_void_p()
    assert not session.b.cuda_tensor_upload_g(C.byref(h), q4.ctypes.data_as(C.c_void_p), f32p(sc), 7, I, O, 0, 32)
    assert not h.value
    sc[3, 1] = -sc[3, 0]
    assert not session.b.cuda_tensor_upload_g(C.byref(h), q4.ctypes.data_as(C.c_void_p), f32p(sc), 7, I, O, 0, 32)


@pytest.mark.parametrize("fmt", [4, 7])
def test_tensor_update(session, fmt):
    """Contents replaced in place: the handle keeps its address and size and
    the next GEMV uses the new weights and scales."""
    rng = np.random.default_rng(70 + fmt)
    O, I, S = 160, 384, 2
    x = rand_x(rng, S, I)
    if fmt == 4:
        (qa, sa), (qb, sb) = rand_i4(rng, O, I, 32), rand_i4(rng, O, I, 32)
        h = session.upload(qa, sa, 4, I, O, 32)
    else:
        (qa, ea), (qb, eb) = rand_mxfp4(rng, O, I), rand_mxfp4(rng, O, I)
        sa, sb = e8_to_f32(ea), e8_to_f32(eb)
        h = session.upload(qa, sa, 7, I, O, 32)
    try:
        nbytes = session.b.cuda_tensor_bytes(h)
        ya = session.matmul(h, x, fmt, I, O, 32)
        assert session.b.cuda_tensor_update(h, qb.ctypes.data_as(C.c_void_p), f32p(np.ascontiguousarray(sb)))
        assert session.b.cuda_tensor_bytes(h) == nbytes
        yb = session.matmul(h, x, fmt, I, O, 32)
        if fmt == 7:
            bad = sb.copy()
            bad[0, 0] = 3.0
            assert not session.b.cuda_tensor_update(h, qb.ctypes.data_as(C.c_void_p), f32p(bad))
    finally:
        session.free(h)
    if fmt == 4:
        ra, rb = cref.matmul_i4_grouped(x, qa, sa, O, I, 32), cref.matmul_i4_grouped(x, qb, sb, O, I, 32)
        ma, mb = magnitude(x, deq_i4(qa, sa, I, 32)), magnitude(x, deq_i4(qb, sb, I, 32))
    else:
        ra, rb = cref.matmul_mxfp4(x, qa, ea, O, I), cref.matmul_mxfp4(x, qb, eb, O, I)
        ma, mb = magnitude(x, deq_mxfp4(qa, ea, I)), magnitude(x, deq_mxfp4(qb, eb, I))
    assert rel_err(ya, ra, ma).max() <= TOL
    assert rel_err(yb, rb, mb).max() <= TOL


@pytest.mark.parametrize("S", [1, 16, 40])
def test_shared_mlp_w4a16_fmt2(session, S):
    """silu(gate x) * (up x) -> down, per-row int4 (fmt=2) tensors, against
    cref_matmul_i4 + cref_swiglu."""
    rng = np.random.default_rng(500 + S)
    D, I = 256, 384
    (gq, gs), (uq, us), (dq, ds) = rand_i4(rng, I, D, 0), rand_i4(rng, I, D, 0), rand_i4(rng, D, I, 0)
    x = rand_x(rng, S, D)
    hg, hu, hd = session.upload(gq, gs, 2, D, I), session.upload(uq, us, 2, D, I), session.upload(dq, ds, 2, I, D)
    y = np.zeros((S, D), np.float32)
    try:
        assert session.b.cuda_shared_mlp_w4a16(hg, hu, hd, f32p(y), f32p(x), S)
    finally:
        for h in (hg, hu, hd):
            session.free(h)
    hid = cref.swiglu(cref.matmul_i4(x, gq, gs, I, D), cref.matmul_i4(x, uq, us, I, D))
    ref = cref.matmul_i4(hid, dq, ds, D, I)
    assert rel_err(y, ref, magnitude(hid, deq_i4(dq, ds, I, 0))).max() <= TOL


def test_shared_mlp_w4a16_refuses_other_formats(session):
    rng = np.random.default_rng(8)
    D, I = 128, 128
    hs = [session.upload(*rand_i4(rng, O, II, 32), 4, II, O, 32) for O, II in ((I, D), (I, D), (D, I))]
    x = rand_x(rng, 2, D)
    y = np.full((2, D), 7.0, np.float32)
    try:
        assert not session.b.cuda_shared_mlp_w4a16(hs[0], hs[1], hs[2], f32p(y), f32p(x), 2)
    finally:
        for h in hs:
            session.free(h)
    assert np.all(y == 7.0)   # untouched on refusal


class Dev:
    """Device buffers through the pipe_* allocation entry points."""

    def __init__(self, session):
        self.s, self.b, self.ptrs = session, session.b, []

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = self.b.cuda_pipe_alloc(0, max(a.nbytes, 4))
        assert p
        self.ptrs.append(p)
        assert self.b.cuda_pipe_upload(0, p, a.ctypes.data_as(C.c_void_p), a.nbytes)
        return p

    def get(self, p, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        assert self.b.cuda_pipe_sync(0)
        assert self.b.cuda_pipe_download(0, p, out.ctypes.data_as(C.c_void_p), out.nbytes)
        return out

    def close(self):
        for p in self.ptrs:
            self.b.cuda_pipe_free(0, p)


@pytest.fixture
def dev(session):
    d = Dev(session)
    yield d
    d.close()


@pytest.mark.parametrize("n", [1, 255, 70001])
def test_pipe_silu_mul_and_add(session, dev, n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    t = rng.standard_normal(n).astype(np.float32)
    pg, pu, pt = dev.put(g), dev.put(u), dev.put(t)
    assert session.b.cuda_pipe_silu_mul(0, pg, pu, n)
    h = dev.get(pg, n)
    ref = cref.swiglu(g, u)
    assert np.allclose(h, ref, rtol=1e-6, atol=1e-30)
    assert session.b.cuda_pipe_add(0, pg, pt, n)
    s = dev.get(pg, n)
    assert np.array_equal(s, (h + t).astype(np.float32))   # one f32 add: exact
    assert not session.b.cuda_pipe_add(0, pg, pt, 0)


def test_pipe_rows_add(session, dev):
    """x[rows[i]] += partial[i] (c/backend_cuda.cu:2073-2078)."""
    rng = np.random.default_rng(31)
    S, D, n = 10, 7168, 6
    x = rng.standard_normal((S, D)).astype(np.float32)
    part = rng.standard_normal((n, D)).astype(np.float32)
    rows = np.array([3, 0, 9, 5, 1, 7], np.int32)
    px, pp, pr = dev.put(x), dev.put(part), dev.put(rows)
    assert session.b.cuda_pipe_rows_add(0, px, pp, pr, n, D)
    got = dev.get(px, (S, D))
    ref = x.copy()
    ref[rows] += part
    assert np.array_equal(got, ref)
    assert not session.b.cuda_pipe_rows_add(0, px, pp, pr, 0, D)


def test_pipe_copy2d(session, dev):
    rng = np.random.default_rng(32)
    H, sp, dp, W = 9, 300, 260, 200
    src = rng.standard_normal((H, sp)).astype(np.float32)
    dst0 = np.full((H, dp), -1.0, np.float32)
    ps, pd = dev.put(src), dev.put(dst0)
    assert session.b.cuda_pipe_copy2d(0, pd, dp, ps, sp, W, H)
    got = dev.get(pd, (H, dp))
    ref = dst0.copy()
    ref[:, :W] = src[:, :W]
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("O,I,S", [(16, 128, 1), (2048, 7168, 2), (7168, 2048, 4)])
def test_upload_fp4_rows16(session, O, I, S):
    """Input in the 16-row interleave of coli_fp4_pack_rows16_v10
    (c/deepseek_v4.c:10975-10993) packed by the oracle: the GEMV equals the
    row-major upload bitwise; with the e4m3 activation QDQ of the native_quant
    contract it matches the oracle's rows16 matvec (coli_fp4_matvec_rows16_v10,
    c/deepseek_v4.c:11120-11243) within the bar."""
    rng = np.random.default_rng(O + S)
    q4, e8 = rand_mxfp4(rng, O, I)
    pd, ps = cref.pack_rows16(q4, e8, O, I)
    x = rand_x(rng, S, I)
    h = C.c_void_p()
    assert session.b.hip_tensor_upload_fp4_rows16(C.byref(h), pd.ctypes.data_as(C.POINTER(C.c_uint8)),
                                                  ps.ctypes.data_as(C.POINTER(C.c_uint8)), I, O, 0)
    h2 = session.upload_mxfp4(q4, e8, I, O)
    yq = np.zeros((S, O), np.float32)
    try:
        y = session.matmul(h, x, 7, I, O, 32)
        y2 = session.matmul(h2, x, 7, I, O, 32)
        # the native_quant contract on the rows16 tensor: e4m3-QDQ activations
        assert session.b.hip_fp4_matmul_qdq(h, f32p(yq), f32p(x), S)
    finally:
        session.free(h)
        session.free(h2)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    assert rel_err(y, cref.matmul_mxfp4(x, q4, e8, O, I), magnitude(x, deq_mxfp4(q4, e8, I))).max() <= TOL
    ref = np.stack([cref.matvec_rows16(x[s], pd, ps, O, I) for s in range(S)])
    xq = np.stack([cref.qdq(x[s])[0] for s in range(S)])
    assert rel_err(yq, ref, magnitude(xq, deq_mxfp4(q4, e8, I))).max() <= TOL
    # refusal of shapes the layout cannot hold
    bad = C.c_void_p()
    assert not session.b.hip_tensor_upload_fp4_rows16(C.byref(bad), pd.ctypes.data_as(C.POINTER(C.c_uint8)),
                                                      ps.ctypes.data_as(C.POINTER(C.c_uint8)), I, O - 1, 0)


@pytest.mark.parametrize("kcopy", ["0", "1"])
@pytest.mark.parametrize("rows", [[1, 1, 1], [60, 50, 45]])
def test_expert_group_staging_routes(session, monkeypatch, kcopy, rows):
    """Sync and issue/take group calls bitwise equal under both PCIe staging
    routes (copy kernels on the pinned buffers, DMA copies) and against the
    oracle; the 155-row group is above the copy-kernel threshold."""
    monkeypatch.setenv("COLI_HIP_KCOPY", kcopy)
    rng = np.random.default_rng(sum(rows) + int(kcopy))
    D, I = 2048, 256
    layer = Layer(rng, 4, D, I, len(rows))
    hs = layer.upload(session)
    x = rand_x(rng, sum(rows), D)
    try:
        y = session.expert_group([h[0] for h in hs], [h[1] for h in hs], [h[2] for h in hs], rows, x)
        g, _ga = tensor_array([h[0] for h in hs])
        u, _ua = tensor_array([h[1] for h in hs])
        d, _da = tensor_array([h[2] for h in hs])
        r = np.array(rows, np.int32)
        if sum(rows) <= 8:
            assert session.b.cuda_expert_group_issue(g, u, d, i32p(r), len(rows), f32p(x))
            yp = session.b.cuda_expert_group_take(0)
            assert yp
            ya = np.ctypeslib.as_array(yp, shape=(sum(rows) * D,)).reshape(sum(rows), D).copy()
            assert np.array_equal(ya.view(np.uint32), y.view(np.uint32))
        else:   # issue is decode-scale only (c/backend_cuda.cu:1716)
            assert not session.b.cuda_expert_group_issue(g, u, d, i32p(r), len(rows), f32p(x))
    finally:
        for h in hs:
            for t in h:
                session.free(t)
    off = 0
    for e, n in enumerate(rows):
        xs = x[off:off + n]
        hid, ref = layer.expert_forward(e, xs)
        mag = magnitude(hid, np.abs(deq_i4(*layer.experts[e][2], I, 32)))
        assert rel_err(y[off:off + n], ref, mag).max() <= TOL
        off += n


SENTINEL = np.uint32(0x7FC0DEAD)   # a quiet-NaN bit pattern no kernel writes


def _sentinel(shape):
    return np.full(shape, SENTINEL, np.uint32).view(np.float32)


def _untouched(a):
    return bool(np.all(a.view(np.uint32) == SENTINEL))


def test_fault_injection_contract(session, monkeypatch):
    """The ABI's failure contract on a live device (c/backend_cuda.cu:1340-1348,
    1384-1385; exercised by c/tests/test_backend_cuda.cu:313-318): with
    COLI_GPU_FAIL_AFTER=0 every compute entry point returns 0 (take: NULL)
    and leaves its output bitwise untouched; once the variable is unset the
    next call of each matches the oracle again."""
    rng = np.random.default_rng(1340)
    b = session.b
    D, I, S = 256, 128, 2
    q4, sc = rand_i4(rng, I, D, 32)
    x = rand_x(rng, S, D)
    layer = Layer(rng, 4, D, I, 2)
    hs = layer.upload(session)
    h = session.upload(q4, sc, 4, D, I, 32)
    g, _ga = tensor_array([t[0] for t in hs])
    u, _ua = tensor_array([t[1] for t in hs])
    d, _da = tensor_array([t[2] for t in hs])
    rows = np.ones(2, np.int32)
    E, K = 16, 4
    W = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)
    bias = np.zeros(E, np.float32)
    xd, wd, bd, yd = (b.cuda_pipe_alloc(0, n) for n in (S * D * 4, E * D * 4, E * 4, S * I * 4))
    try:
        for p, a in ((xd, x), (wd, W), (bd, bias)):
            assert b.cuda_pipe_upload(0, p, a.ctypes.data_as(C.c_void_p), a.nbytes)

        def calls():
            """(name, run) pairs; run() returns (ok, outputs...)."""
            def matmul():
                y = _sentinel((S, I))
                hh = C.c_void_p(h.value)
                return b.cuda_matmul(C.byref(hh), f32p(y), f32p(x), None, None, 4, S, D, I, 0, 32), y

            def group():
                y = _sentinel((2, D))
                return b.cuda_expert_group(g, u, d, i32p(rows), 2, f32p(y), f32p(x)), y

            def issue():
                ok = b.cuda_expert_group_issue(g, u, d, i32p(rows), 2, f32p(x))
                yp = b.cuda_expert_group_take(0)
                y = (np.ctypeslib.as_array(yp, shape=(2 * D,)).reshape(2, D).copy() if yp else _sentinel((2, D)))
                return bool(ok) and bool(yp), y

            def pipe_gemm():
                y = _sentinel((S, I))
                assert b.cuda_pipe_upload(0, yd, y.ctypes.data_as(C.c_void_p), y.nbytes)
                ok = b.cuda_pipe_gemm(h, yd, xd, S)
                assert b.cuda_pipe_sync(0)
                assert b.cuda_pipe_download(0, yd, y.ctypes.data_as(C.c_void_p), y.nbytes)
                return ok, y

            def router():
                idx, w, keff = (np.full(K, SENTINEL, np.uint32).view(np.int32), _sentinel(K),
                                np.full(1, SENTINEL, np.uint32).view(np.int32))
                ok = b.cuda_pipe_router(0, xd, wd, bd, D, E, K, 0.0, 1, 1.0, i32p(idx), f32p(w), i32p(keff))
                return ok, idx.view(np.float32), w, keff.view(np.float32)

            return [("matmul", matmul), ("expert_group", group), ("expert_group_issue", issue),
                    ("pipe_gemm", pipe_gemm), ("pipe_router", router)]

        monkeypatch.setenv("COLI_GPU_FAIL_AFTER", "0")
        for name, run in calls():
            ok, *outs = run()
            assert not ok, f"{name} ran with COLI_GPU_FAIL_AFTER=0"
            assert all(_untouched(o) for o in outs), f"{name} wrote its output on a refused call"
        monkeypatch.delenv("COLI_GPU_FAIL_AFTER")
        res = {name: run() for name, run in calls()}
        assert all(r[0] for r in res.values()), {n: r[0] for n, r in res.items()}
    finally:
        for p in (xd, wd, bd, yd):
            b.cuda_pipe_free(0, p)
        session.free(h)
        for t3 in hs:
            for t in t3:
                session.free(t)
    ref = cref.matmul_i4_grouped(x, q4, sc, I, D, 32)
    mag = magnitude(x, deq_i4(q4, sc, D, 32))
    assert rel_err(res["matmul"][1], ref, mag).max() <= TOL
    assert rel_err(res["pipe_gemm"][1], ref, mag).max() <= TOL
    for name in ("expert_group", "expert_group_issue"):
        y = res[name][1]
        for e in range(2):
            hid, yr = layer.expert_forward(e, x[e:e + 1])
            m = magnitude(hid, np.abs(deq_i4(*layer.experts[e][2], I, 32)))
            assert rel_err(y[e:e + 1], yr, m).max() <= TOL, name
    _, idx, w, keff = res["pipe_router"]
    ri, rw, rk = cref.route(cref.matmul_f32(x[:1], W), K, 1, bias=bias, norm_topk=1, routed_scale=1.0)
    assert keff.view(np.int32)[0] == rk[0]
    assert np.array_equal(idx.view(np.int32)[:rk[0]], ri[0, :rk[0]])
    assert np.allclose(w[:rk[0]], rw[0, :rk[0]], rtol=1e-5, atol=0)


def test_fmt4_without_group_size_refused(session):
    """fmt=4 carries [O, ceil(I/gs)] scales, so a call without a group size is
    refused on a live device with the output untouched
    (c/backend_cuda.cu:1355-1359)."""
    rng = np.random.default_rng(1355)
    O, I, S = 64, 256, 2
    q4, sc = rand_i4(rng, O, I, 32)
    x = rand_x(rng, S, I)
    y = _sentinel((S, O))
    h = C.c_void_p()
    assert not session.b.cuda_matmul(C.byref(h), f32p(y), f32p(x), q4.ctypes.data_as(C.c_void_p), f32p(sc),
                                     4, S, I, O, 0, 0)
    assert not h.value
    assert _untouched(y)
