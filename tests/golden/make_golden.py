"""Writes the golden fixtures of tests/golden/ (run from the repository root: python tests/golden/make_golden.py).

- gemm_small.npz: seeded U[-1, 1] inputs for every GEMM type and their float64 closed-form product
  alpha·A·B + beta·C0 with the reference's error scale |alpha|·|A|·|B| + |beta·C0| (reference: lib/test_basic.py:53-56).
- level12_small.npz: seeded vectors, a matrix, the exactly rounded dot product (math.fsum of the exact float64
  products) and the float64 GEMV with its scale |A|·|x| (reference: lib/test_level12.py:63, 80).
- reference_error_profile.json: the error statistics the reference publishes for its own kernels at n = 4096
  (reference: README.md:73-74) and the maxima its test accepts (lib/test_basic.py:4-8).
Nothing here runs or imports reference code; the outputs are closed forms of the inputs.
"""
import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.realpath(__file__))
SEED = 2024


def main():
    out = {"seed": SEED, "alpha": 0.75, "beta": -1.5}
    for kind, dt in (("H", np.float16), ("HS", np.float16), ("S", np.float32), ("D", np.float64)):
        a = np.random.default_rng(SEED).uniform(-1, 1, (23, 77)).astype(dt)
        b = np.random.default_rng(SEED + 1).uniform(-1, 1, (77, 19)).astype(dt)
        c0 = np.random.default_rng(SEED + 2).uniform(-1, 1, (23, 19)).astype(dt)
        a64, b64, c64 = a.astype(np.float64), b.astype(np.float64), c0.astype(np.float64)
        out[f"{kind}_A"], out[f"{kind}_B"], out[f"{kind}_C0"] = a, b, c0
        out[f"{kind}_ref"] = out["alpha"] * (a64 @ b64) + out["beta"] * c64
        out[f"{kind}_scale"] = abs(out["alpha"]) * (np.abs(a64) @ np.abs(b64)) + abs(out["beta"]) * np.abs(c64)
    np.savez_compressed(os.path.join(HERE, "gemm_small.npz"), **out)

    rng = np.random.default_rng(SEED + 3)
    x = rng.uniform(-1, 1, 4099).astype(np.float32)
    y = rng.uniform(-1, 1, 4099).astype(np.float32)
    A = rng.uniform(-1, 1, (61, 513)).astype(np.float32)
    x64, y64, A64 = x.astype(np.float64), y.astype(np.float64), A.astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "level12_small.npz"), x=x, y=y, A=A,
                        dot=math.fsum((x64 * y64).tolist()), dot_scale=float(np.abs(x64) @ np.abs(y64)),
                        gemv=A64 @ x64[:513], gemv_scale=np.abs(A64) @ np.abs(x64[:513]))

    profile = {
        "source": "reference README.md:73-74 (n = 4096, mean / max of |C - ref| / sum|a*b|); max_test: the maximum the "
                  "reference's own test accepts (lib/test_basic.py:4-8: H 'max 1.7-2.4e-3', HS 1e-3 for K >= 256, S 1e-5)",
        "H": {"mean": 1.4e-4, "max": 8.5e-4, "max_test": 2.4e-3},
        "HS": {"mean": 1.5e-5, "max": 5.6e-5, "max_test": 1e-3},
        "S": {"mean": 1.6e-8, "max": 7.8e-8, "max_test": 1e-5},
    }
    with open(os.path.join(HERE, "reference_error_profile.json"), "w") as f:
        json.dump(profile, f, indent=1)


if __name__ == "__main__":
    main()
