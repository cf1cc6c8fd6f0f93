"""Write tests/golden/glm_router.npz: the GLM engine's router GEMV (c/quant.h:98-102,
the f32 matmul c/colibri.c:2871 calls) as the reference compiles (oracle/_ref/
libref_glm_avx512.so, built by oracle/Makefile from the reference sources), on seeded
inputs whose input counts cover its vector body and scalar tail (D = 5, 13, 37, 5120,
5127).  Run from the repository root with the reference built:
    python tests/golden/make_glm_golden.py
The fixture holds inputs and outputs only."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.oracle import RefGlm  # noqa: E402


def main():
    r = RefGlm()
    rng = np.random.default_rng(20261201)
    out = {}
    for D, E in ((5, 3), (13, 4), (37, 6), (5120, 2), (5127, 1)):
        x = rng.standard_normal((2, D)).astype(np.float32)
        W = (rng.standard_normal((E, D)) * 0.05).astype(np.float32)
        out[f"x_{D}"], out[f"w_{D}"], out[f"y_{D}"] = x, W, r.matmul(x, W)
    np.savez_compressed(os.path.join(ROOT, "tests", "golden", "glm_router.npz"), **out)


if __name__ == "__main__":
    main()
