"""The streaming kernel's in-kernel split-K reduction (the last workgroup of a
column block to arrive sums the partials) against the separate reduce
launch, which hcg_gemm_noalloc still uses.

Both sum the splits' partials in the same order, so the two entry points
must agree bit for bit.  Every round draws new operands: a partial that a
workgroup on another XCD read stale (from an earlier call with other
inputs) would change the sums, so the small-integer rounds also check the
exact product.
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DEV = "cuda:0"

# (m, n, k): the first four take the in-kernel reduction (R = 1 with 4 and 8
# splits, R = 2 with 4 splits, N not a multiple of 128); the last two keep
# the reduce launch (more than 8 splits; four row blocks).
CASES = [(16, 8192, 8192), (16, 4096, 2048), (32, 8192, 4096), (12, 6000, 4096), (8, 1000, 4096),
         (64, 4096, 4096)]


def _run(entry, ta, tb, m, n, k):
    from hc.gfx950 import _native

    lib = _native.load()
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    rc = getattr(lib, entry)(_native.HCG_F16, ta.data_ptr(), k, tb.data_ptr(), n, out.data_ptr(), n, m, n, k,
                             torch.cuda.current_stream().cuda_stream)
    assert rc == _native.HCG_OK, _native.last_error(lib)
    return out


@pytest.mark.parametrize("kind", ["int", "uniform"])
def test_in_kernel_reduction_matches_the_reduce_launch(kind):
    for rnd in range(4):
        for m, n, k in CASES:
            print(f"case stream reduce {kind} round {rnd} m={m} n={n} k={k}", flush=True)
            rng = np.random.default_rng(1000 * rnd + m + n + k)
            if kind == "int":
                a = rng.integers(-3, 4, size=(m, k)).astype(np.float16)
                b = rng.integers(-3, 4, size=(k, n)).astype(np.float16)
            else:
                a = rng.uniform(-1, 1, size=(m, k)).astype(np.float16)
                b = rng.uniform(-1, 1, size=(k, n)).astype(np.float16)
            ta, tb = torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV)
            fused = _run("hcg_gemm", ta, tb, m, n, k)
            launched = _run("hcg_gemm_noalloc", ta, tb, m, n, k)
            torch.cuda.synchronize()
            assert torch.equal(fused, launched), (rnd, m, n, k)
            if kind == "int":
                # integers below 2^24 in every partial sum: float64 is exact
                want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
                assert np.array_equal(fused.cpu().numpy(), want), (rnd, m, n, k)
