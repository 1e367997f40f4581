"""Seeded sweep of MoE layer shapes through the decode and verification paths
of the fused layer (one-token kernels, the four-wave selection with the
fragment build and the shared expert beside it, two row blocks a down
workgroup, the grouped GEMM past 16 rows): routing bit-exact against the
oracle, outputs within 1e-3 of its composition, and bitwise equal with the
overlapped forms switched off (COLI_HIP_SHARED_OVERLAP, COLI_HIP_PREP_BESIDE,
COLI_HIP_CHAIN = 0). Weight sets are shared cyclically between experts
(Layer distinct=4) to keep the test small."""
import ctypes as C

import numpy as np
import pytest

from colibri_amd.backend import ColiHipMoeConfig, f32p, i32p, tensor_array
from moe_ref import Layer, cref, free_handles, make_router_inputs, moe_reference
from quant_util import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
SWITCHES = ("COLI_HIP_SHARED_OVERLAP", "COLI_HIP_PREP_BESIDE", "COLI_HIP_CHAIN")


def _cases(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        mode = int(rng.choice([0, 1, 2, 3]))
        out.append((i, int(rng.choice([4, 7])), int(rng.choice([1536, 2048, 2048, 7168])),
                    int(rng.choice([1024, 2048])), int(rng.choice([48, 64, 65, 128, 200, 256])),
                    int(rng.choice([1, 2, 6, 8, 16])), mode, int(rng.choice([1, 1, 2, 3, 5, 12, 16, 21, 40])),
                    bool(rng.integers(0, 2)), float(rng.choice([0.0, 0.6])) if mode in (1, 2) else 0.0))
    return out


@pytest.mark.parametrize("n,fmt,D,I,E,K,mode,S,shared,topp", _cases(2024, 14))
def test_moe_layer_sweep(session, monkeypatch, n, fmt, D, I, E, K, mode, S, shared, topp):
    rng = np.random.default_rng(8000 + n)
    layer = Layer(rng, fmt, D, I, E, shared=shared, distinct=4)
    x, W, b = make_router_inputs(rng, S, D, E, K, mode, bias=(mode != 0))
    norm = 1 if mode == 1 else 0
    hs = layer.upload(session)
    routed, sh = hs[:E], (hs[E] if shared else (None, None, None))
    g, _ga = tensor_array([h[0] for h in routed])
    u, _ua = tensor_array([h[1] for h in routed])
    d, _da = tensor_array([h[2] for h in routed])
    cfg = ColiHipMoeConfig(D, I, E, K, mode, norm, topp, 1.0, 1 if shared else 0, 0.0)
    m = C.c_void_p()
    bc = np.ascontiguousarray(b) if b is not None else None
    assert session.b.hip_moe_create(C.byref(m), 0, C.byref(cfg), f32p(np.ascontiguousarray(W)),
                                    f32p(bc) if bc is not None else None, g, u, d, sh[0], sh[1], sh[2])
    res = []
    try:
        for off in (False, True):
            for k in SWITCHES:
                if off:
                    monkeypatch.setenv(k, "0")
                else:
                    monkeypatch.delenv(k, raising=False)
            out = np.zeros((S, D), np.float32)
            idx = np.zeros((S, K), np.int32)
            w = np.zeros((S, K), np.float32)
            keff = np.zeros(S, np.int32)
            assert session.b.hip_moe_forward(m, f32p(x), f32p(out), S, i32p(idx), f32p(w), i32p(keff))
            res.append((out, idx, w, keff))
    finally:
        session.b.hip_moe_free(m)
        free_handles(session, hs)
    for ta, tb in zip(res[0], res[1]):
        assert np.array_equal(ta.view(np.uint32) if ta.dtype == np.float32 else ta,
                              tb.view(np.uint32) if tb.dtype == np.float32 else tb)
    out, idx, w, keff = res[0]
    ri, rw, rk = cref.route(cref.matmul_f32(x, W), K, mode, bias=b, norm_topk=norm, topp=topp)
    assert np.array_equal(keff, rk)
    for s in range(S):
        assert np.array_equal(idx[s, :rk[s]], ri[s, :rk[s]]), "router top-K indices must be bit-exact"
    _, _, _, ref, mag = moe_reference(layer, x, W, b, K, mode, norm_topk=norm, topp=topp)
    assert rel_err(out, ref, mag).max() <= TOL
