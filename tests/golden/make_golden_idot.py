"""Writes tests/golden/golden_idot.npz: input/output vectors of the
reference's fmt=2 int8-activation (IDOT) path -- qrow_i8 per row
(c/quant.h:581-586) then matmul_i4_idot (c/quant.h:924-933, dot_i4i8
674-801), as c/colibri.c:937-945 chains them -- compiled from its C sources
by oracle/Makefile into oracle/_ref/libcoli_ref.so (build container only; the
vectors are committed). Cases: aligned and ragged I (odd: the last byte's
high nibble unused), several batch sizes, an all-zero row (scale floor
1e-12), a row whose maximum is exactly representable, rounding ties of
x * inv, and a wide row (I = 14336). Seeded; run after `make -C oracle`.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from oracle_lib import REF_PATH, Ref  # noqa: E402
from quant_util import rand_i4  # noqa: E402

SEED = 20261203


def main():
    if not os.path.exists(REF_PATH):
        raise SystemExit("oracle/_ref/libcoli_ref.so not built (make -C oracle with the reference tree)")
    ref = Ref()
    rng = np.random.default_rng(SEED)
    out = {"seed": np.array(SEED)}
    cases = [(1, 64, 16), (3, 256, 33), (16, 512, 8), (4, 97, 7), (2, 14336, 12)]
    for n, (S, I, O) in enumerate(cases):
        q4, sc = rand_i4(rng, O, I, 0, fp16_scales=False)
        x = (rng.standard_normal((S, I)) * 2).astype(np.float32)
        if n == 1:
            x[0] = 0.0                                              # all-zero row: scale floor
            x[1] = (np.arange(I, dtype=np.float32) - 128.0) * 0.5   # maximum 64: exact scale
            x[2, :8] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 127.0, -127.0, 3.5], np.float32)
        out[f"c{n}_x"], out[f"c{n}_q4"], out[f"c{n}_sc"] = x, q4, sc
        out[f"c{n}_y"] = ref.matmul_i4_idot(x, q4, sc, O, I)
        out[f"c{n}_shape"] = np.array([S, I, O])
    np.savez_compressed(os.path.join(HERE, "golden_idot.npz"), **out)
    print("wrote golden_idot.npz:", len(cases), "cases")


if __name__ == "__main__":
    main()
