"""Write the committed golden fixtures for tests/test_oracle.py.

    python tests/golden/make_golden.py

generators.json  sha256 of seeded generator streams (the build's own
                 UNIFORM/NORMAL generators and the reference-test mode).
gemm_small.npz   small GEMM cases: inputs, scales and expected bf16 outputs.

Expected outputs come from the oracle and, for every unscaled case, are
checked here against the reference's own gemm_cpu (test.cpp:19-30) compiled
from its sources into oracle/_ref (``make -C oracle ref``); this script
refuses to write fixtures if that library is missing or disagrees.  Scaled
cases are checked against bf16(acc * (sa*sb)) from the oracle's fp32
accumulators, which the unscaled cross-check pins.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import pyoracle as po  # noqa: E402


def main():
    o = po.get()
    ref = po.RefLib()  # raises if oracle/_ref is not built

    gens = {"cases": [], "scales": []}
    for seed, dist, p0, p1 in ((1, "uniform", -1.0, 1.0),
                               (2, "normal", 0.0, 1.0),
                               (3, "normal", 0.0, 0.5),
                               (4, "uniform", -1.0, 1.0)):
        n = 1 << 16
        d = po.UNIFORM if dist == "uniform" else po.NORMAL
        a = o.fill((n,), seed, d, p0, p1)
        gens["cases"].append({"seed": seed, "dist": dist, "p0": p0, "p1": p1,
                              "n": n,
                              "sha256": hashlib.sha256(a.tobytes()).hexdigest()})
    for seed in (0, 1):
        n = 1 << 16
        a = o.fill_reftest((n,), seed)
        assert np.array_equal(a, ref.init_random(n, seed))
        gens["cases"].append({"seed": seed, "dist": "reftest", "p0": -1.0,
                              "p1": 1.0, "n": n,
                              "sha256": hashlib.sha256(a.tobytes()).hexdigest()})
    for seed in (1, 2, 3):
        gens["scales"].append({"seed": seed, "value": o.draw_scale(seed)})
    with open(os.path.join(HERE, "generators.json"), "w") as f:
        json.dump(gens, f, indent=1)

    cases = {}
    specs = [
        ("u64x48x96", 64, 48, 96, po.UNIFORM, -1.0, 1.0, 1.0, 1.0),
        ("n33x17x160", 33, 17, 160, po.NORMAL, 0.0, 1.0, 1.0, 1.0),
        ("n40x72x256s", 40, 72, 256, po.NORMAL, 0.0, 1.0, 1.25, 0.75),
        ("h16x32x512s", 16, 32, 512, po.NORMAL, 0.0, 0.5, 0.5, 1.5),
        ("r96x80x128", 96, 80, 128, None, 0, 0, 1.0, 1.0),
    ]
    for i, (nm, M, N, K, d, p0, p1, sa, sb) in enumerate(specs):
        if d is None:
            A = o.fill_reftest((M, K), 2 * i)
            B = o.fill_reftest((N, K), 2 * i + 1)
        else:
            A = o.fill((M, K), 100 + 2 * i, d, p0, p1)
            B = o.fill((N, K), 101 + 2 * i, d, p0, p1)
        sa, sb = float(np.float32(sa)), float(np.float32(sb))
        C = o.gemm(A, B, sa, sb)
        if sa == 1.0 and sb == 1.0:
            assert np.array_equal(C, ref.gemm_cpu(A, B)), nm
        else:
            acc = o.gemm_rows_acc(A, B, np.arange(M))
            assert np.array_equal(ref.gemm_cpu(A, B), o.f32_to_bf16(acc)), nm
            want = o.f32_to_bf16(acc * np.float32(np.float32(sa) * np.float32(sb)))
            assert np.array_equal(C, want), nm
        cases[nm + "_A"], cases[nm + "_B"], cases[nm + "_C"] = A, B, C
        cases[nm + "_S"] = np.array([sa, sb], np.float32)
    np.savez_compressed(os.path.join(HERE, "gemm_small.npz"), **cases)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
