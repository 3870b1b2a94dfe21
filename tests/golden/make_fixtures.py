"""Write the golden GEMM fixtures used by the tests.

    python tests/golden/make_fixtures.py

The reference holds no stored arrays for this path; its numeric test is
tests/test_examples.py:23-33 (shapes (16,16,16), (32,32,32), (17,19,18),
inputs from make_demo_inputs(seed=7), simulator output vs a blocked fp32
reference within atol=2e-6) and the example's main (32^3, seed 0,
examples/amdgpu_gfx11_wmma_matmul.py:428-441).  Those inputs are
regenerated here with the same generator (numpy default_rng, A then B,
uniform(-1, 1) -> float16) and stored with:

* ``c_seq``: the reference simulator's result, restated as the sequential
  float32 fold (oracle.gemm_bruteforce, a scalar np.float32 triple loop);
* ``c_blocked``: the reference test's blocked check value.

Plus BASELINE config 1 (128^3, N(0,1) fp16, seed 0) with its sequential-fold
output.  Each file is a plain .npz (no pickles).
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "5_amd"))

import hc_oracle as oracle  # noqa: E402
from hc.gfx950.workloads import make_demo_inputs, make_inputs  # noqa: E402

REFERENCE_CASES = [
    # (name, m, n, k, seed) -- tests/test_examples.py:23-33 and the example main
    ("ref_16x16x16_seed7", 16, 16, 16, 7),
    ("ref_32x32x32_seed7", 32, 32, 32, 7),
    ("ref_17x19x18_seed7", 17, 19, 18, 7),
    ("ref_32x32x32_seed0", 32, 32, 32, 0),
]


def main() -> None:
    for name, m, n, k, seed in REFERENCE_CASES:
        a, b = make_demo_inputs(m=m, n=n, k=k, seed=seed)
        c_seq = oracle.gemm_bruteforce(a, b)
        c_blocked = oracle.gemm_blocked(a, b)
        np.savez(os.path.join(HERE, f"{name}.npz"), a=a, b=b, c_seq=c_seq, c_blocked=c_blocked,
                 meta=np.array([m, n, k, seed]))
        print(name, "max|seq-blocked| =", float(np.max(np.abs(c_seq - c_blocked))))
    a, b = make_inputs("c1_128_f16", seed=0)
    c_seq = oracle.gemm_sequential(a, b)
    np.savez(os.path.join(HERE, "c1_128_f16_seed0.npz"), a=a, b=b, c_seq=c_seq, meta=np.array([128, 128, 128, 0]))
    print("c1_128_f16_seed0 written")


if __name__ == "__main__":
    main()
