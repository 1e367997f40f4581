"""ctypes bindings for the parity oracle (test infrastructure only).

``cref`` is this repository's C restatement (oracle/libcpu_ref.so);
``ref`` is the reference's own CPU code compiled from its sources
(oracle/_ref/libcoli_ref.so), present when it was built in the build
container. Only tests, __graft_entry__.smoke() and bench.py's cpu_baseline
leg use this module.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CREF_PATH = os.path.join(ROOT, "oracle", "libcpu_ref.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libcoli_ref.so")

_f = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_i32 = C.POINTER(C.c_int)
_i = C.c_int


def ptr(a, t):
    return a.ctypes.data_as(t)


def f32p(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return ptr(a, _f)


def u8p(a):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return ptr(a, _u8)


def i32p(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return ptr(a, _i32)


class _Lib:
    def __init__(self, path, prefix):
        self.path = path
        self.lib = C.CDLL(path)
        self.p = prefix

    def fn(self, name, argtypes, restype=None):
        f = getattr(self.lib, self.p + name)
        f.argtypes = argtypes
        f.restype = restype
        return f


class Cref(_Lib):
    """The C restatement (cpu_ref.c)."""

    def __init__(self, path=CREF_PATH):
        super().__init__(path, "cref_")
        self.e2m1 = self.fn("e2m1_decode", [C.c_uint8], C.c_float)
        self.e8m0 = self.fn("e8m0_decode", [C.c_uint8], C.c_float)
        self.mx4_scale = self.fn("mx4_scale", [C.c_uint8], C.c_float)
        self.e4m3_dec = self.fn("e4m3fn_decode", [C.c_uint8], C.c_float)
        self.e4m3_enc = self.fn("e4m3fn_encode", [C.c_float], C.c_uint8)
        self.bf16_round = self.fn("bf16_round", [C.c_float], C.c_float)
        self._qdq = self.fn("fp8_activation_qdq", [_f, _u8, _f, C.c_size_t, C.c_size_t], _i)
        self._f32 = self.fn("matmul_f32", [_f, _f, _f, _i, _i, _i])
        self._i4g = self.fn("matmul_i4_grouped", [_f, _f, _u8, _f, _i, _i, _i, _i])
        self._i4 = self.fn("matmul_i4", [_f, _f, _u8, _f, _i, _i, _i])
        self._i4d = self.fn("matmul_i4_idot", [_f, _f, _u8, _f, _i, _i, _i])
        self._qrow = self.fn("qrow_i8", [_f, C.POINTER(C.c_int8), _i], C.c_float)
        self._mx = self.fn("matmul_mxfp4", [_f, _f, _u8, _u8, _i, _i, _i])
        self._mx8 = self.fn("matmul_mxfp4_i8", [_f, _f, _u8, _u8, _i, _i, _i])
        self._fp4b = self.fn("fp4_matmul_batch", [_f, _u8, _u8, _i, _i, _f, _i], _i)
        self._pack16 = self.fn("fp4_pack_rows16", [_u8, _u8, _u8, _u8, _i, _i], _i)
        self._mv16 = self.fn("fp4_matvec_rows16", [_f, _u8, _u8, _i, _i, _f], _i)
        self._route = self.fn("route", [_f, _f, _i, _i, _i, _i, C.c_float, _i, C.c_float,
                                         _i32, _f, _i32])
        self._union = self.fn("expert_union", [_i32, _f, _i32, _i, _i, _i, _i32, _i32,
                                               _i32, _i32, _f], _i)
        self._swiglu = self.fn("swiglu", [_f, _f, _f, C.c_size_t])
        self._moe = self.fn("moe_layer", [C.c_void_p, _f, _i, _f, _i32, _f, _i32], _i)
        self._swiglu_v4 = self.fn("swiglu_v4", [_f, _f, _f, C.c_size_t, C.c_float])

    def qdq(self, x, block=128):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        sc = np.empty((x.size + block - 1) // block, np.uint8)
        assert self._qdq(f32p(out), u8p(sc), f32p(x), x.size, block) == 0
        return out, sc

    def matmul_f32(self, x, W):
        S, I = x.shape
        O = W.shape[0]
        y = np.empty((S, O), np.float32)
        self._f32(f32p(y), f32p(x), f32p(W), S, I, O)
        return y

    def matmul_i4_grouped(self, x, q4, sc, O, I, gs):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._i4g(f32p(y), f32p(x), u8p(q4), f32p(sc), S, I, O, gs)
        return y

    def matmul_i4(self, x, q4, sc, O, I):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._i4(f32p(y), f32p(x), u8p(q4), f32p(sc), S, I, O)
        return y

    def matmul_i4_idot(self, x, q4, sc, O, I):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty((x.shape[0], O), np.float32)
        self._i4d(f32p(y), f32p(x), u8p(np.ascontiguousarray(q4)), f32p(np.ascontiguousarray(sc, np.float32)),
                  x.shape[0], I, O)
        return y

    def qrow_i8(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.empty(x.size, np.int8)
        s = self._qrow(f32p(x), q.ctypes.data_as(C.POINTER(C.c_int8)), x.size)
        return q, np.float32(s)

    def matmul_mxfp4(self, x, q4, e8, O, I):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._mx(f32p(y), f32p(x), u8p(q4), u8p(e8), S, I, O)
        return y

    def matmul_mxfp4_i8(self, x, q4, e8, O, I):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._mx8(f32p(y), f32p(x), u8p(q4), u8p(e8), S, I, O)
        return y

    def fp4_matmul_batch(self, x, q4, e8, O, I):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        assert self._fp4b(f32p(y), u8p(q4), u8p(e8), O, I, f32p(x), S) == 0
        return y

    def pack_rows16(self, q4, e8, O, I):
        pd = np.empty_like(q4)
        ps = np.empty_like(e8)
        assert self._pack16(u8p(pd), u8p(ps), u8p(q4), u8p(e8), O, I) == 0
        return pd, ps

    def matvec_rows16(self, x, pd, ps, O, I):
        y = np.empty(O, np.float32)
        assert self._mv16(f32p(y), u8p(pd), u8p(ps), O, I, f32p(x)) == 0
        return y

    def route(self, logits, K, mode, bias=None, topp=0.0, norm_topk=0, routed_scale=1.0):
        logits = np.ascontiguousarray(logits, np.float32)
        S, E = logits.shape
        idx = np.empty((S, K), np.int32)
        w = np.zeros((S, K), np.float32)
        keff = np.empty(S, np.int32)
        b = np.ascontiguousarray(bias, np.float32) if bias is not None else None
        self._route(f32p(logits), f32p(b) if b is not None else None, S, E, K, mode,
                    topp, norm_topk, routed_scale, i32p(idx), f32p(w), i32p(keff))
        return idx, w, keff

    def expert_union(self, idx, w, keff, E):
        S, K = idx.shape
        uniq = np.empty(E, np.int32)
        cnt = np.zeros(E, np.int32)
        rows = np.empty((E, S * K), np.int32)
        slots = np.empty((E, S * K), np.int32)
        ws = np.empty((E, S * K), np.float32)
        nu = self._union(i32p(idx), f32p(w), i32p(keff), S, K, E, i32p(uniq), i32p(cnt),
                         i32p(rows), i32p(slots), f32p(ws))
        return nu, uniq[:nu], cnt[:nu], rows[:nu], slots[:nu], ws[:nu]

    def swiglu(self, g, u):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        h = np.empty_like(g)
        self._swiglu(f32p(h), f32p(g), f32p(u), g.size)
        return h

    def swiglu_v4(self, g, u, limit):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        h = np.empty_like(g)
        self._swiglu_v4(f32p(h), f32p(g), f32p(u), g.size, limit)
        return h


class CrefMoe(C.Structure):
    """cpu_ref.h CrefMoe."""
    _fields_ = [(n, C.c_int) for n in ("fmt", "D", "I", "E", "K", "gs", "route_mode", "norm_topk",
                                      "has_shared")] + \
        [("topp", C.c_float), ("routed_scale", C.c_float), ("router_w", _f), ("router_bias", _f)] + \
        [(n, C.POINTER(C.c_void_p)) for n in ("gq", "gsc", "uq", "usc", "dq", "dsc")] + \
        [(n, C.c_void_p) for n in ("sh_gq", "sh_uq", "sh_dq", "sh_gsc", "sh_usc", "sh_dsc")]


def cref_moe_layer(lib, fmt, x, W, bias, experts, shared, K, mode, norm_topk=0, topp=0.0,
                   routed_scale=1.0, gs=32):
    """cref_moe_layer on source-layout experts [(gq, gsc), (uq, usc), (dq, dsc)]
    (fmt 4: f32 scales; fmt 7 / 17: e8m0 bytes). Returns out, idx, w, keff."""
    x = np.ascontiguousarray(x, np.float32)
    S, D = x.shape
    E = len(experts)
    I = experts[0][0][0].shape[0]
    keep = [x, W, bias]
    def arr(k, j):
        a = (C.c_void_p * E)(*[e[k][j].ctypes.data for e in experts])
        keep.append(a)
        return C.cast(a, C.POINTER(C.c_void_p))
    m = CrefMoe(fmt, D, I, E, K, gs, mode, norm_topk, 1 if shared is not None else 0, topp, routed_scale,
                f32p(W), f32p(bias) if bias is not None else None,
                arr(0, 0), arr(0, 1), arr(1, 0), arr(1, 1), arr(2, 0), arr(2, 1))
    if shared is not None:
        m.sh_gq, m.sh_gsc = shared[0][0].ctypes.data, shared[0][1].ctypes.data
        m.sh_uq, m.sh_usc = shared[1][0].ctypes.data, shared[1][1].ctypes.data
        m.sh_dq, m.sh_dsc = shared[2][0].ctypes.data, shared[2][1].ctypes.data
    out = np.empty((S, D), np.float32)
    idx = np.zeros((S, K), np.int32)
    w = np.zeros((S, K), np.float32)
    keff = np.zeros(S, np.int32)
    rc = lib._moe(C.byref(m), f32p(x), S, f32p(out), i32p(idx), f32p(w), i32p(keff))
    assert rc == 0
    return out, idx, w, keff


class Ref(_Lib):
    """The reference's own CPU kernels, compiled from its sources."""

    def __init__(self, path=REF_PATH):
        super().__init__(path, "")
        self._i4g = self.fn("ref_matmul_i4_grouped", [_f, _f, _u8, _f, _i, _i, _i, _i])
        self._i4 = self.fn("ref_matmul_i4", [_f, _f, _u8, _f, _i, _i, _i])
        self._i4d = self.fn("ref_matmul_i4_idot", [_f, _f, _u8, _f, _i, _i, _i])
        self._qrow = self.fn("ref_qrow_i8", [_f, C.POINTER(C.c_int8), _i], C.c_float)
        self._mx = self.fn("ref_matmul_mxfp4", [_f, _f, _u8, _u8, _i, _i, _i])
        self._mx8 = self.fn("ref_matmul_mxfp4_i8", [_f, _f, _u8, _u8, _i, _i, _i])
        self._f32 = self.fn("ref_matmul_f32", [_f, _f, _f, _i, _i, _i])
        self._qdq = self.fn("coli_fp8_activation_qdq_ref", [_f, _u8, _f, C.c_size_t, C.c_size_t], _i)
        self.e2m1 = self.fn("coli_e2m1_decode", [C.c_uint8], C.c_float)
        self.e8m0 = self.fn("coli_e8m0_decode", [C.c_uint8], C.c_float)
        self.e4m3_dec = self.fn("coli_e4m3fn_decode", [C.c_uint8], C.c_float)
        self.e4m3_enc = self.fn("coli_e4m3fn_encode", [C.c_float], C.c_uint8)
        self.bf16_round = self.fn("coli_bf16_round", [C.c_float], C.c_float)
        self._v4route = self.fn("coli_v4_route", [_f, _i32, _f, _f, _f, _i32, _i, _i, _i, C.c_float], _i)
        self._v4swiglu = self.fn("coli_v4_swiglu", [_f, _f, _f, _i, C.c_float], _i)

    def v4_route(self, logits, K, bias=None, route_scale=1.0):
        """coli_v4_route on given logits: hidden = [1.0] and a one-column gate
        make the reference's own dot product return each logit exactly."""
        logits = np.ascontiguousarray(logits, np.float32)
        E = logits.size
        one = np.ones(1, np.float32)
        w = np.zeros(K, np.float32)
        idx = np.zeros(K, np.int32)
        b = np.ascontiguousarray(bias, np.float32) if bias is not None else None
        rc = self._v4route(f32p(w), i32p(idx), f32p(one), f32p(logits), f32p(b) if b is not None else None,
                           None, E, 1, K, route_scale)
        return rc, idx, w

    def v4_swiglu(self, g, u, limit):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        h = np.empty_like(g)
        assert self._v4swiglu(f32p(h), f32p(g), f32p(u), g.size, limit) == 0
        return h

    def matmul_i4_grouped(self, x, q4, sc, O, I, gs):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._i4g(f32p(y), f32p(x), u8p(q4), f32p(sc), S, I, O, gs)
        return y

    matmul_i4_idot = Cref.matmul_i4_idot
    qrow_i8 = Cref.qrow_i8

    def matmul_i4(self, x, q4, sc, O, I):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._i4(f32p(y), f32p(x), u8p(q4), f32p(sc), S, I, O)
        return y

    def matmul_mxfp4(self, x, q4, e8, O, I):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._mx(f32p(y), f32p(x), u8p(q4), u8p(e8), S, I, O)
        return y

    def matmul_mxfp4_i8(self, x, q4, e8, O, I):
        S = x.shape[0]
        y = np.empty((S, O), np.float32)
        self._mx8(f32p(y), f32p(x), u8p(q4), u8p(e8), S, I, O)
        return y

    def matmul_f32(self, x, W):
        S, I = x.shape
        O = W.shape[0]
        y = np.empty((S, O), np.float32)
        self._f32(f32p(y), f32p(x), f32p(W), S, I, O)
        return y

    def qdq(self, x, block=128):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        sc = np.empty((x.size + block - 1) // block, np.uint8)
        assert self._qdq(f32p(out), u8p(sc), f32p(x), x.size, block) == 0
        return out, sc


def have_ref():
    return os.path.exists(REF_PATH)
