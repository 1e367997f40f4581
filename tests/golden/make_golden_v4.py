"""Writes tests/golden/golden_v4.npz: vectors of the reference's DeepSeek-V4
router and SwiGLU (c/deepseek_v4.c:1368-1448, coli_v4_route and
coli_v4_swiglu), compiled from its C sources by oracle/Makefile into
oracle/_ref/libcoli_ref.so (build container only; the vectors are
committed). The router gets its logits through a one-column gate and
hidden = [1.0], so the reference's own dot product returns each logit
exactly. Seeded; run after `make -C oracle`.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from oracle_lib import REF_PATH, Ref  # noqa: E402

SEED = 20261203


def main():
    if not os.path.exists(REF_PATH):
        raise SystemExit("oracle/_ref/libcoli_ref.so not built (make -C oracle with the reference tree)")
    ref = Ref()
    rng = np.random.default_rng(SEED)
    out = {"seed": np.array(SEED)}
    cases = [(64, 6, True, 2.5), (256, 8, True, 2.5), (384, 8, False, 1.0), (32, 4, True, 1.0)]
    for n, (E, K, bias, scale) in enumerate(cases):
        z = (rng.standard_normal(E) * 3).astype(np.float32)
        if n == 3:
            z[:8] = -40.0            # softplus underflow region
            z[8] = z[9]              # a tie in the selection
        b = (rng.standard_normal(E) * 0.1).astype(np.float32) if bias else None
        rc, idx, w = ref.v4_route(z, K, b, scale)
        assert rc == 0
        out[f"r{n}_z"], out[f"r{n}_idx"], out[f"r{n}_w"] = z, idx, w
        out[f"r{n}_b"] = b if b is not None else np.zeros(0, np.float32)
        out[f"r{n}_meta"] = np.array([E, K, int(bias)], np.int32)
        out[f"r{n}_scale"] = np.array([scale], np.float32)
    g = (rng.standard_normal(2048) * 6).astype(np.float32)
    u = (rng.standard_normal(2048) * 6).astype(np.float32)
    g[:4] = [0.0, -0.0, 100.0, -100.0]
    out["sw_g"], out["sw_u"] = g, u
    for n, limit in enumerate((0.0, 1.0, 7.0)):
        out[f"sw{n}_limit"] = np.array([limit], np.float32)
        out[f"sw{n}_h"] = ref.v4_swiglu(g, u, limit)
    np.savez_compressed(os.path.join(HERE, "golden_v4.npz"), **out)
    print("wrote", len(cases), "router cases and 3 swiglu cases")


if __name__ == "__main__":
    main()
