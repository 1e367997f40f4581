"""ctypes binding of libcoli_hip.so, the gfx950 backend's C ABI.

This mirrors how colibri's engine binds its GPU backend: every `coli_cuda_*`
symbol of c/backend_cuda.h is resolved by name, mandatory symbols must all be
present and optional ones may be absent (the RESOLVE / RESOLVE_OPT rules of
c/backend_loader.c:1355-1379). There is no CPU fallback here: a missing or
incomplete library raises, and a compute entry point returning 0 is reported
as a failure to the caller, exactly as the engine would see it.
"""
import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libcoli_hip.so")
INCLUDE_DIR = os.path.join(ROOT, "include")

# Optional in the reference loader (c/backend_loader.c:1388, 1399-1400).
OPTIONAL = {"coli_cuda_device_integrated", "coli_cuda_e8_set_grid", "coli_cuda_fp8_set_lut",
            "coli_cuda_matmul_mxfp4"}

_f = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_i32 = C.POINTER(C.c_int)
_vp = C.c_void_p
_i = C.c_int
_sz = C.c_size_t
_tp = C.c_void_p                # ColiCudaTensor*
_tpp = C.POINTER(C.c_void_p)    # ColiCudaTensor**


class ColiHipMoeConfig(C.Structure):
    _fields_ = [("D", C.c_int), ("I", C.c_int), ("E", C.c_int), ("K", C.c_int),
                ("route_mode", C.c_int), ("norm_topk", C.c_int), ("topp", C.c_float),
                ("routed_scale", C.c_float), ("has_shared", C.c_int), ("swiglu_limit", C.c_float)]


def declared_symbols():
    """Every function name declared in include/*.h."""
    names = []
    for fn in sorted(os.listdir(INCLUDE_DIR)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE_DIR, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(coli_(?:cuda|hip)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


_SIGS = {
    "coli_cuda_init": ([_i32, _i], _i),
    "coli_cuda_shutdown": ([], None),
    "coli_cuda_device_count": ([], _i),
    "coli_cuda_device_at": ([_i], _i),
    "coli_cuda_mem_info": ([_i, C.POINTER(_sz), C.POINTER(_sz)], _i),
    "coli_cuda_device_integrated": ([_i], _i),
    "coli_cuda_stats": ([_i, C.POINTER(_sz), C.POINTER(_sz)], None),
    "coli_cuda_group_stats": ([C.POINTER(C.c_uint64)] * 3 + [C.POINTER(C.c_double)] * 3, None),
    "coli_cuda_group_stats_device": ([_i] + [C.POINTER(C.c_uint64)] * 3 + [C.POINTER(C.c_double)] * 3, None),
    "coli_cuda_e8_set_grid": ([_vp], _i),
    "coli_cuda_fp8_set_lut": ([_f], _i),
    "coli_cuda_tensor_upload_g": ([_tpp, _vp, _f, _i, _i, _i, _i, _i], _i),
    "coli_cuda_tensor_upload": ([_tpp, _vp, _f, _i, _i, _i, _i], _i),
    "coli_cuda_tensor_free": ([_tp], None),
    "coli_cuda_tensor_bytes": ([_tp], _sz),
    "coli_cuda_tensor_device": ([_tp], _i),
    "coli_cuda_tensor_update": ([_tp, _vp, _f], _i),
    "coli_cuda_matmul_mxfp4": ([_f, _f, _u8, _u8, _i, _i, _i], _i),
    "coli_cuda_matmul": ([_tpp, _f, _f, _vp, _f, _i, _i, _i, _i, _i, _i], _i),
    "coli_cuda_expert_mlp": ([_tp, _tp, _tp, _f, _f, _i], _i),
    "coli_cuda_shared_mlp_w4a16": ([_tp, _tp, _tp, _f, _f, _i], _i),
    "coli_cuda_expert_group_issue": ([_tpp, _tpp, _tpp, _i32, _i, _f], _i),
    "coli_cuda_expert_group_take": ([_i], _f),
    "coli_cuda_expert_group": ([_tpp, _tpp, _tpp, _i32, _i, _f, _f], _i),
    "coli_cuda_pipe_scratch": ([_i, _i, _sz], _vp),
    "coli_cuda_pipe_alloc": ([_i, _sz], _vp),
    "coli_cuda_pipe_free": ([_i, _vp], None),
    "coli_cuda_pipe_upload": ([_i, _vp, _vp, _sz], _i),
    "coli_cuda_pipe_download": ([_i, _vp, _vp, _sz], _i),
    "coli_cuda_pipe_silu_mul": ([_i, _vp, _vp, _sz], _i),
    "coli_cuda_pipe_add": ([_i, _vp, _vp, _sz], _i),
    "coli_cuda_pipe_rows_add": ([_i, _vp, _vp, _vp, _i, _i], _i),
    "coli_cuda_pipe_gemm": ([_tp, _vp, _vp, _i], _i),
    "coli_cuda_expert_group_resident_issue": ([_tpp, _tpp, _tpp, _f, _i, _i, _vp, _vp], _i),
    "coli_cuda_expert_group_resident_take": ([_i, _i32, _i, _vp, _vp, _i], _i),
    "coli_cuda_pipe_router": ([_i, _vp, _vp, _vp, _i, _i, _i, C.c_float, _i, C.c_float, _i32, _f, _i32], _i),
    "coli_cuda_pipe_copy2d": ([_i, _vp, _i, _vp, _i, _i, _i], _i),
    "coli_cuda_pipe_peer_copy": ([_i, _vp, _i, _vp, _sz], _i),
    "coli_cuda_pipe_sync": ([_i], _i),
    "coli_hip_tensor_upload_mxfp4": ([_tpp, _u8, _u8, _i, _i, _i], _i),
    "coli_hip_tensor_upload_fp4_rows16": ([_tpp, _u8, _u8, _i, _i, _i], _i),
    "coli_hip_fp4_matmul_qdq": ([_tp, _f, _f, _i], _i),
    "coli_hip_fp4_matmul_qdq_dev": ([_tp, _vp, _vp, _i], _i),
    "coli_hip_matmul_mxfp4_i8": ([_f, _f, _u8, _u8, _i, _i, _i], _i),
    "coli_hip_fp4_matmul_i8": ([_tp, _f, _f, _i], _i),
    "coli_hip_fp4_matmul_i8_dev": ([_tp, _vp, _vp, _i], _i),
    "coli_hip_matmul_i4_idot": ([_tp, _f, _f, _i], _i),
    "coli_hip_matmul_i4_idot_dev": ([_tp, _vp, _vp, _i], _i),
    "coli_hip_moe_create": ([C.POINTER(_vp), _i, C.POINTER(ColiHipMoeConfig), _f, _f, _tpp, _tpp, _tpp,
                             _tp, _tp, _tp], _i),
    "coli_hip_moe_free": ([_vp], None),
    "coli_hip_moe_forward_dev": ([_vp, _vp, _vp, _i], _i),
    "coli_hip_moe_forward": ([_vp, _f, _f, _i, _i32, _f, _i32], _i),
    "coli_hip_moe_last_union": ([_vp, _i32, _i32], _i),
    "coli_hip_stream": ([_i], _vp),
    "coli_hip_tensor_upload_from_device": ([_tpp, _vp, _f, _u8, _i, _i, _i, _i, _i], _i),
    "coli_hip_fill_random_u8": ([_i, _vp, _sz, C.c_ulonglong], _i),
    "coli_hip_stream_read": ([_i, _vp, _sz], _i),
    "coli_hip_gemm_prep_dev": ([_tp, _vp, _i], _i),
    "coli_hip_pipe_gemm_noalloc": ([_tp, _vp, _vp, _i], _i),
    "coli_hip_gemm_run_dev": ([_tp, _vp, _i], _i),
    "coli_hip_gemm_run_dev_emit": ([_tp, _vp, _i, _tp], _i),
    "coli_hip_tensor_stream_bytes": ([_tp], _sz),
    "coli_hip_tensor_kind": ([_tp], _i),
}


class Backend:
    """Loaded libcoli_hip.so with typed entry points (attribute = symbol name
    without the `coli_` prefix, e.g. ``b.cuda_matmul``)."""

    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"libcoli_hip.so not built: {path} (run __graft_entry__.build())")
        self.path = path
        self.lib = C.CDLL(path, mode=C.RTLD_GLOBAL)
        missing = []
        for name in declared_symbols():
            fn = getattr(self.lib, name, None) if hasattr(self.lib, name) else None
            if fn is None:
                if name not in OPTIONAL:
                    missing.append(name)
                continue
            if name in _SIGS:
                fn.argtypes, fn.restype = _SIGS[name]
            setattr(self, name[len("coli_"):], fn)
        if missing:
            raise RuntimeError(f"libcoli_hip.so lacks mandatory symbols: {missing}")


def f32p(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f)


def u8p(a):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8)


def i32p(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_i32)


def tensor_array(handles):
    arr = (C.c_void_p * len(handles))(*[h.value if isinstance(h, C.c_void_p) else h for h in handles])
    return C.cast(arr, _tpp), arr


# ---------------------------------------------------------------------------
# numpy conveniences (used by tests and the benchmark)
# ---------------------------------------------------------------------------
class Session:
    """An initialised backend on one device."""

    def __init__(self, device=0, path=LIB_PATH):
        self.b = Backend(path)
        self.device = device
        devs = (C.c_int * 1)(device)
        if not self.b.cuda_init(devs, 1):
            raise RuntimeError("coli_cuda_init failed")

    def close(self):
        self.b.cuda_shutdown()

    def upload(self, q4, scales, fmt, I, O, gs=0):
        """fmt 2/4: scales f32; fmt 7: scales f32 powers of two (gs 32)."""
        h = C.c_void_p()
        q4 = np.ascontiguousarray(q4, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        ok = self.b.cuda_tensor_upload_g(C.byref(h), q4.ctypes.data_as(_vp), f32p(scales), fmt, I, O,
                                         self.device, gs)
        if not ok:
            raise RuntimeError(f"tensor upload refused (fmt={fmt} I={I} O={O} gs={gs})")
        return h

    def upload_mxfp4(self, q4, e8, I, O):
        h = C.c_void_p()
        q4 = np.ascontiguousarray(q4, np.uint8)
        e8 = np.ascontiguousarray(e8, np.uint8)
        if not self.b.hip_tensor_upload_mxfp4(C.byref(h), u8p(q4), u8p(e8), I, O, self.device):
            raise RuntimeError("mxfp4 upload refused")
        return h

    def free(self, h):
        self.b.cuda_tensor_free(h)

    def matmul(self, h, x, fmt, I, O, gs=0):
        x = np.ascontiguousarray(x, np.float32)
        S = x.shape[0]
        y = np.zeros((S, O), np.float32)
        hh = C.c_void_p(h.value)
        if not self.b.cuda_matmul(C.byref(hh), f32p(y), f32p(x), None, None, fmt, S, I, O, self.device, gs):
            raise RuntimeError("coli_cuda_matmul failed")
        return y

    def expert_group(self, gates, ups, downs, rows, x):
        x = np.ascontiguousarray(x, np.float32)
        total, D = x.shape
        y = np.zeros((total, D), np.float32)
        g, ga = tensor_array(gates)
        u, ua = tensor_array(ups)
        d, da = tensor_array(downs)
        r = np.ascontiguousarray(rows, np.int32)
        if not self.b.cuda_expert_group(g, u, d, i32p(r), len(gates), f32p(y), f32p(x)):
            raise RuntimeError("coli_cuda_expert_group failed")
        return y
