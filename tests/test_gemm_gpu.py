"""GPU parity: the gfx950 kernels against the CPU oracle (sequential float32
fold, the reference simulator's semantics) on seeded inputs.

Bar: relative Frobenius error <= 1e-3 and
max |err| <= 2e-2 * sqrt(K / 1024); bit-exact where every summation order is
exact (small-integer inputs)."""

from __future__ import annotations

import numpy as np
import pytest

import hc_oracle as oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _gemm(a, b, algo="auto", dtype="float16"):
    import hc.gfx950 as g
    from hc.gfx950.workloads import to_torch

    dev = torch.device("cuda", 0)
    ta, tb = to_torch(a, dtype, dev), to_torch(b, dtype, dev)
    out = g.gemm(ta, tb, algo=algo)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _dt(dtype):
    return oracle.F16 if dtype == "float16" else oracle.BF16


@pytest.mark.parametrize("algo", ["tiled", "auto"])
@pytest.mark.parametrize("m,n,k", [(128, 128, 128), (256, 256, 64), (17, 19, 18), (300, 520, 200)])
def test_small_parity_f16(m, n, k, algo):
    from hc.gfx950.workloads import make_inputs

    print(f"case m={m} n={n} k={k} algo={algo}", flush=True)
    a, b = make_inputs("c1_128_f16", seed=1, m=m, n=n, k=k)
    got = _gemm(a, b, algo)
    want = oracle.gemm_sequential(a, b)
    rep = oracle.parity_check(got, want, k)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("m,n,k", [(16, 8192, 8192), (1, 1000, 333), (7, 260, 1000), (16, 128, 32)])
def test_skinny_parity(m, n, k):
    from hc.gfx950.workloads import make_inputs

    print(f"case skinny m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c4_skinny_f16", seed=2, m=m, n=n, k=k)
    got = _gemm(a, b, "skinny")
    want = oracle.gemm_c(a, b)
    rep = oracle.parity_check(got, want, k)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("algo", ["tiled", "skinny"])
def test_integer_inputs_bit_exact(algo):
    rng = np.random.default_rng(3)
    m = 16 if algo == "skinny" else 300
    n, k = 520, 1000
    a = rng.integers(-4, 5, size=(m, k)).astype(np.float16)
    b = rng.integers(-4, 5, size=(k, n)).astype(np.float16)
    print(f"case integer {algo}", flush=True)
    got = _gemm(a, b, algo)
    want = oracle.gemm_sequential(a, b)
    assert np.array_equal(got, want)
