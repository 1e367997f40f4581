"""Writes tests/golden/golden.npz: input/output vectors of the reference's own
CPU kernels, compiled from its C sources by oracle/Makefile into
oracle/_ref/libcoli_ref.so (build container only; the reference tree does not
exist on the GPU box, so the vectors are committed).

Functions captured (reference file:line):
  matmul_i4_grouped   c/quant.h:168-202       (fmt=4, int4 + per-group scale)
  matmul_i4           c/quant.h (fmt=2, per-row scale)
  matmul_mxfp4        c/quant.h:1386-1440     (fmt=7, e2m1 + e8m0 per 32)
  matmul (f32)        c/quant.h               (router logits)
  coli_fp8_activation_qdq_ref  c/deepseek_v4.c:10390-10605
  coli_fp4_matmul_batch_ref    c/deepseek_v4.c:10906
  coli_fp4_pack_rows16_v10 / coli_fp4_matvec_rows16_v10  c/deepseek_v4.c:10975-11243
  codecs: coli_e2m1_decode, coli_e8m0_decode, coli_e4m3fn_{de,en}code,
          coli_bf16_round  c/deepseek_v4.c:10390-10487

Seeds are fixed; run `python tests/golden/make_golden.py` after
`make -C oracle` to regenerate.
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from oracle_lib import REF_PATH, Ref, f32p, u8p  # noqa: E402
from quant_util import bf16_exact, rand_i4, rand_mxfp4, rand_x  # noqa: E402

SEED = 20261201
FP4_NATIVE_BLOCK, SCALE_UE8M0 = 5, 2


class TensorView(C.Structure):
    """ColiTensorView, c/tensor.h:30-41."""
    _fields_ = [("format", C.c_int), ("scale_format", C.c_int), ("data", C.c_void_p),
                ("scales", C.c_void_p), ("data_bytes", C.c_size_t), ("scale_bytes", C.c_size_t),
                ("rows", C.c_int64), ("columns", C.c_int64), ("block_rows", C.c_uint32),
                ("block_columns", C.c_uint32)]


def view(q4, e8, O, I, block_rows=1):
    return TensorView(FP4_NATIVE_BLOCK, SCALE_UE8M0, q4.ctypes.data, e8.ctypes.data, q4.nbytes,
                      e8.nbytes, O, I, block_rows, 32)


def main():
    if not os.path.exists(REF_PATH):
        raise SystemExit("oracle/_ref/libcoli_ref.so not built (make -C oracle with the reference tree)")
    ref = Ref()
    lib = ref.lib
    rng = np.random.default_rng(SEED)
    out = {"seed": np.array(SEED)}

    # fmt=4: (S, I, O, gs) including ragged I (tails of 1..7 columns) and partial groups
    i4_cases = [(1, 64, 16, 32), (3, 96, 17, 32), (2, 100, 9, 32), (4, 257, 5, 32),
                (2, 128, 8, 64), (1, 384, 6, 128), (5, 75, 3, 16)]
    for n, (S, I, O, gs) in enumerate(i4_cases):
        q4, sc = rand_i4(rng, O, I, gs, fp16_scales=(n % 2 == 0))
        x = rand_x(rng, S, I)
        out[f"i4g{n}_shape"] = np.array([S, I, O, gs])
        out[f"i4g{n}_q4"], out[f"i4g{n}_sc"], out[f"i4g{n}_x"] = q4, sc, x
        out[f"i4g{n}_y"] = ref.matmul_i4_grouped(x, q4, sc, O, I, gs)

    # fmt=2: per-row scale
    for n, (S, I, O) in enumerate([(1, 64, 8), (3, 70, 5), (2, 33, 4)]):
        q4, sc = rand_i4(rng, O, I, 0)
        x = rand_x(rng, S, I)
        out[f"i4r{n}_shape"] = np.array([S, I, O])
        out[f"i4r{n}_q4"], out[f"i4r{n}_sc"], out[f"i4r{n}_x"] = q4, sc, x
        out[f"i4r{n}_y"] = ref.matmul_i4(x, q4, sc, O, I)

    # fmt=7, including e8 edges 0 and 254 in the last case
    mx_cases = [(1, 64, 16), (4, 96, 13), (2, 50, 7), (3, 256, 4)]
    for n, (S, I, O) in enumerate(mx_cases):
        q4, e8 = rand_mxfp4(rng, O, I)
        if n == 3:
            e8[0, 0], e8[1, 1], e8[2, 2] = 0, 254, 1
        x = rand_x(rng, S, I)
        out[f"mx{n}_shape"] = np.array([S, I, O])
        out[f"mx{n}_q4"], out[f"mx{n}_e8"], out[f"mx{n}_x"] = q4, e8, x
        out[f"mx{n}_y"] = ref.matmul_mxfp4(x, q4, e8, O, I)

    # f32 matmul (router logits)
    x = rng.standard_normal((3, 70)).astype(np.float32)
    W = (rng.standard_normal((11, 70)) * 0.02).astype(np.float32)
    out["f32_x"], out["f32_W"], out["f32_y"] = x, W, ref.matmul_f32(x, W)

    # e4m3 activation QDQ: random, magnitudes across the range, exact ties,
    # a partial block and zeros
    q = rng.standard_normal(384).astype(np.float32) * np.float32(3.0)
    q[:16] = np.array([0, -0.0, 1, 448, -448, 1e-9, 6.5, 0.001953125, 17, 18, 19, 20, 300, 320, 352, 5.5],
                      np.float32)
    q[128:256] = 0.0
    for blk in (128, 64, 32):
        y, sc = ref.qdq(q[:300], blk)
        out[f"qdq_b{blk}_y"], out[f"qdq_b{blk}_sc"] = y, sc
    out["qdq_x"] = q[:300]

    # batched fp4 matmul and rows16 (no-FMA order)
    fb = lib.coli_fp4_matmul_batch_ref
    fb.argtypes = [C.POINTER(C.c_float), C.POINTER(TensorView), C.POINTER(C.c_float), C.c_int]
    pk = lib.coli_fp4_pack_rows16_v10
    pk.argtypes = [C.POINTER(C.c_uint8), C.POINTER(C.c_uint8), C.POINTER(TensorView)]
    mv = lib.coli_fp4_matvec_rows16_v10
    mv.argtypes = [C.POINTER(C.c_float), C.POINTER(TensorView), C.POINTER(C.c_float)]
    for n, (S, I, O) in enumerate([(3, 128, 16), (5, 256, 32)]):
        q4, e8 = rand_mxfp4(rng, O, I)
        x = rand_x(rng, S, I)
        v = view(q4, e8, O, I)
        y = np.zeros((S, O), np.float32)
        assert fb(f32p(y), C.byref(v), f32p(x), S) == 0
        pd = np.zeros_like(q4)
        ps = np.zeros_like(e8)
        assert pk(u8p(pd), u8p(ps), C.byref(v)) == 0
        pv = view(pd, ps, O, I, 16)
        y16 = np.zeros(O, np.float32)
        assert mv(f32p(y16), C.byref(pv), f32p(np.ascontiguousarray(x[0]))) == 0
        out[f"fb{n}_shape"] = np.array([S, I, O])
        out[f"fb{n}_q4"], out[f"fb{n}_e8"], out[f"fb{n}_x"] = q4, e8, x
        out[f"fb{n}_y"], out[f"fb{n}_pd"], out[f"fb{n}_ps"], out[f"fb{n}_y16"] = y, pd, ps, y16

    # codecs, exhaustive where the domain is a byte
    out["e2m1"] = np.array([ref.e2m1(i) for i in range(16)], np.float32)
    out["e8m0_bits"] = np.array([ref.e8m0(i) for i in range(256)], np.float32).view(np.uint32)
    out["e4m3_dec_bits"] = np.array([ref.e4m3_dec(i) for i in range(256)], np.float32).view(np.uint32)
    enc_in = np.concatenate([rng.standard_normal(200).astype(np.float32) * 50,
                             np.array([0, 448, 464, 480, 1e6, -1e6, 2.0 ** -9, 2.0 ** -10, 0.0029296875,
                                       1.0625, 1.1875, -1.0625], np.float32)])
    out["e4m3_enc_in"] = enc_in
    out["e4m3_enc_out"] = np.array([ref.e4m3_enc(float(v)) for v in enc_in], np.uint8)
    bf_in = np.concatenate([rng.standard_normal(200).astype(np.float32),
                            np.array([1.00390625, 1.01171875, 1.0078125, 3.0e38, -0.0], np.float32)])
    out["bf16_in"] = bf_in
    out["bf16_out"] = np.array([ref.bf16_round(float(v)) for v in bf_in], np.float32)
    assert np.array_equal(bf16_exact(out["bf16_out"]), out["bf16_out"])

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
