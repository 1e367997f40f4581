"""Writes tests/golden/golden_mxfp4_i8.npz: input/output vectors of the
reference's matmul_mxfp4_i8 (c/quant.h:1441-1515, MXFP4 with per-32 int8
activation quantization, the K3 IDOT path), compiled from its C sources by
oracle/Makefile into oracle/_ref/libcoli_ref.so (build container only; the
vectors are committed). Cases: aligned shapes at several batch sizes, a
group whose maximum sits exactly on +-127, an all-zero group (scale floor
1e-20), rounding ties (x * inv landing on k + 0.5), and a ragged I that
falls back to matmul_mxfp4. Seeded; run after `make -C oracle`.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from oracle_lib import REF_PATH, Ref  # noqa: E402
from quant_util import rand_mxfp4  # noqa: E402

SEED = 20261202


def main():
    if not os.path.exists(REF_PATH):
        raise SystemExit("oracle/_ref/libcoli_ref.so not built (make -C oracle with the reference tree)")
    ref = Ref()
    rng = np.random.default_rng(SEED)
    out = {"seed": np.array(SEED)}
    cases = [(1, 64, 16), (3, 256, 33), (16, 512, 8), (5, 96, 7), (2, 100, 9)]
    for n, (S, I, O) in enumerate(cases):
        q4, e8 = rand_mxfp4(rng, O, I, 110, 135)
        x = rng.standard_normal((S, I)).astype(np.float32)
        if n == 1:
            x[0, :32] = 0.0                                  # all-zero group: scale floor
            x[1, 32:64] = np.linspace(-2.0, 2.0, 32, dtype=np.float32)
            x[2, 64:96] = (np.arange(32, dtype=np.float32) - 16.0) * 0.25   # ties at x * inv = k + 0.5
            x[2, 64] = 127.0 * 0.25                                       # group maximum -> q = 127
        out[f"c{n}_x"], out[f"c{n}_q4"], out[f"c{n}_e8"] = x, q4, e8
        out[f"c{n}_y"] = ref.matmul_mxfp4_i8(x, q4, e8, O, I)
        out[f"c{n}_shape"] = np.array([S, I, O])
    np.savez_compressed(os.path.join(HERE, "golden_mxfp4_i8.npz"), **out)
    print("wrote", len(cases), "cases")


if __name__ == "__main__":
    main()
