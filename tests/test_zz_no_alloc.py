"""hcg_gemm_noalloc: the allocation-free variant of hcg_gemm, through the C
ABI, against hcg_gemm itself and the oracle.

Each case makes two calls in a row, the second with a smaller input, so the
second reads scratch that still holds the first call's bytes: it must
produce exactly what hcg_gemm produces.  Small-integer inputs make every
summation order exact, so the two entry points must agree bit for bit;
seeded uniform inputs are checked against the oracle to the north_star bar.
"""

from __future__ import annotations

import numpy as np
import pytest

import hc_oracle as oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DEV = "cuda:0"


def _lib():
    from hc.gfx950 import _native

    return _native, _native.load()


def _call(entry: str, ta, lda, tb, ldb, m, n, k, pad=(1, 4)):
    """Runs one entry point into a NaN guard band; returns (rc, C, band_ok)."""
    native, lib = _lib()
    top, left = pad
    guard = torch.full((m + 2 * top, n + 2 * left), float("nan"), dtype=torch.float32, device=DEV)
    view = guard[top : top + m, left : left + n]
    stream = torch.cuda.current_stream().cuda_stream
    fn = getattr(lib, entry)
    rc = fn(native.HCG_F16, ta.data_ptr(), lda, tb.data_ptr(), ldb, view.data_ptr(), view.stride(0), m, n, k,
            stream)
    torch.cuda.synchronize()
    out = guard.cpu().numpy()
    inner = np.zeros(out.shape, bool)
    inner[top : top + m, left : left + n] = True
    return rc, out[top : top + m, left : left + n], bool(np.isnan(out[~inner]).all())


def _operands(m, n, k, lda, ldb, kind, seed):
    """fp16 A (m x k, row stride lda) and B (k x n, row stride ldb) on the
    device as strided views; values small integers or uniform[-1, 1]."""
    rng = np.random.default_rng(seed)
    if kind == "int":
        a = rng.integers(-4, 5, size=(m, k)).astype(np.float16)
        b = rng.integers(-4, 5, size=(k, n)).astype(np.float16)
    else:
        a = rng.uniform(-1, 1, size=(m, k)).astype(np.float16)
        b = rng.uniform(-1, 1, size=(k, n)).astype(np.float16)
    ta = torch.full((m, lda), float("nan"), dtype=torch.float16, device=DEV)
    tb = torch.full((k, ldb), float("nan"), dtype=torch.float16, device=DEV)
    ta[:, :k] = torch.from_numpy(a).to(DEV)
    tb[:, :n] = torch.from_numpy(b).to(DEV)
    return a, b, ta, tb


# (first call, second smaller call): (m, n, k, lda, ldb)
PAIRS = [
    # unaligned rows read in place on the tiled kernel (no scratch), then a smaller one
    ((4095, 3001, 1027, 1027, 3001), (1000, 700, 515, 515, 700)),
    # split-K partials on the streaming kernel, then fewer rows and columns
    ((16, 8192, 8192, 8192, 8192), (16, 4096, 4096, 4096, 4096)),
    # K not a multiple of 8, A read in place: rows 65..128 on the tiled
    # kernel with split partials, then 40 rows on the streaming kernel
    ((100, 6000, 8191, 8191, 6000), (40, 3000, 4001, 4001, 3000)),
    # narrow output: split partials of the narrow kernel (B rows unaligned in the second call)
    ((6000, 40, 8192, 8192, 40), (3000, 13, 4096, 4096, 13)),
    # tiled split-K partials (few tiles, long K), then a smaller one
    ((1024, 1024, 8192, 8192, 1024), (512, 512, 4096, 4096, 512)),
    # a peeled shape (tiled bulk + streaming remainder)
    ((4100, 4096, 1024, 1024, 4096), (2052, 2048, 512, 512, 2048)),
]


@pytest.mark.parametrize("kind", ["int", "uniform"])
@pytest.mark.parametrize("first,second", PAIRS, ids=[f"{p[0][0]}x{p[0][1]}x{p[0][2]}" for p in PAIRS])
def test_noalloc_matches_hcg_gemm_on_two_calls(first, second, kind):
    for index, (m, n, k, lda, ldb) in enumerate((first, second)):
        print(f"case noalloc {kind} call {index} {m}x{n}x{k} lda={lda} ldb={ldb}", flush=True)
        a, b, ta, tb = _operands(m, n, k, lda, ldb, kind, seed=100 * index + m % 97)
        rc, got, band = _call("hcg_gemm_noalloc", ta, lda, tb, ldb, m, n, k)
        native, lib = _lib()
        native.check(lib, rc, "hcg_gemm_noalloc")
        assert band, "hcg_gemm_noalloc wrote outside C"
        rc, ref, band = _call("hcg_gemm", ta, lda, tb, ldb, m, n, k)
        native.check(lib, rc, "hcg_gemm")
        if kind == "int":
            assert np.array_equal(got, ref), "noalloc differs from hcg_gemm on exact inputs"
            # float64 products of these small integers are exact (BLAS speed)
            assert np.array_equal(got, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32))
        else:
            rep = oracle.parity_check(got, oracle.gemm_c(a, b, oracle.F16), k)
            assert rep.ok, str(rep)
            rep = oracle.parity_check(got, ref, k)
            assert rep.ok, f"against hcg_gemm: {rep}"


def test_noalloc_rejects_a_call_beyond_its_scratch_before_any_launch():
    native, lib = _lib()
    # 40 rows (the streaming kernel, four 16-row blocks) with a row stride of
    # 2^24 + 8 elements: in place its offsets would pass 2^31, so A is
    # repacked, 40 x 524296 x 2 bytes (42 MB), more than the 32 MiB array.
    m, n, k, lda = 40, 128, (1 << 19) + 1, (1 << 24) + 8
    _, _, ta, tb = _operands(m, n, k, lda, n, "int", seed=5)
    print("case noalloc over the scratch limit", flush=True)
    rc, got, band = _call("hcg_gemm_noalloc", ta, lda, tb, n, m, n, k)
    assert rc == native.HCG_EINVAL
    msg = native.last_error(lib)
    assert "bytes of scratch" in msg and str(native.NOALLOC_SCRATCH_BYTES) in msg, msg
    assert band and np.isnan(got).all(), "a rejected call must not launch"
    # the same call through hcg_gemm (which allocates) works
    rc, _, band = _call("hcg_gemm", ta, lda, tb, n, m, n, k)
    native.check(lib, rc, "hcg_gemm")
    assert band


def test_noalloc_zero_sizes():
    native, lib = _lib()
    assert lib.hcg_gemm_noalloc(native.HCG_F16, None, 0, None, 0, None, 0, 0, 5, 5, None) == native.HCG_OK
    c = torch.full((3, 5), float("nan"), dtype=torch.float32, device=DEV)
    rc = lib.hcg_gemm_noalloc(native.HCG_F16, None, 0, None, 5, c.data_ptr(), 5, 3, 5, 0, None)
    native.check(lib, rc, "hcg_gemm_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(c, torch.zeros_like(c))
