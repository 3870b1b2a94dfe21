"""GPU parity: the gfx950 kernels, called through the hc launch surface and
the C ABI, against the CPU oracle (the reference simulator's sequential
float32 fold) on seeded inputs.

Bar: relative Frobenius error <= 1e-3 and
max |err| <= 2e-2 * sqrt(K / 1024) (``oracle.parity_check``); bit-exact where
every summation order is exact (small-integer inputs); bit-identical across
repeated runs (every reduction has a fixed order).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import hc_oracle as oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda:0"


def _dt(dtype: str) -> int:
    return oracle.F16 if dtype == "float16" else oracle.BF16


def _dev(x: np.ndarray, dtype: str = "float16"):
    from hc.gfx950.workloads import to_torch

    return to_torch(x, dtype, torch.device(DEV))


def _gemm(a: np.ndarray, b: np.ndarray, algo: str = "auto", dtype: str = "float16") -> np.ndarray:
    import hc.gfx950 as g

    out = g.gemm(_dev(a, dtype), _dev(b, dtype), algo=algo)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(got, want, k):
    rep = oracle.parity_check(got, want, k)
    assert rep.ok, str(rep)


# -- the reference's own test shapes, through the unchanged launch call ---------


@pytest.mark.parametrize("name", ["ref_16x16x16_seed7", "ref_32x32x32_seed7", "ref_17x19x18_seed7",
                                  "ref_32x32x32_seed0", "c1_128_f16_seed0"])
def test_golden_fixtures_through_the_launch_surface(name):
    import hc
    import hc.gfx950 as g

    from . import _kernels

    fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    a, b = fx["a"], fx["b"]
    print(f"case {name}", flush=True)
    c = np.full((a.shape[0], b.shape[1]), np.nan, dtype=np.float32)
    hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, a, b, c, target=g.Gfx950Target())
    _check(c, fx["c_seq"], a.shape[1])
    if "c_blocked" in fx:
        # the reference test's own criterion against its blocked check value
        np.testing.assert_allclose(c, fx["c_blocked"], rtol=0, atol=2e-5)


def test_default_target_env_runs_an_unchanged_simulator_call(monkeypatch):
    import hc

    from . import _kernels

    monkeypatch.setenv("HC_DEFAULT_TARGET", "gfx950")
    fx = np.load(os.path.join(GOLDEN, "ref_32x32x32_seed0.npz"))
    c = np.zeros((32, 32), np.float32)
    hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, fx["a"], fx["b"], c)
    _check(c, fx["c_seq"], 32)


def test_unchanged_simulator_call_runs_on_the_gpu_without_configuration(monkeypatch):
    """The reference driver's call, sim.launch(kernel, a, b, c) with no target
    (examples/amdgpu_gfx11_wmma_matmul.py:338-348), on numpy inputs."""
    import hc
    import hc.gfx950 as g

    from . import _kernels

    monkeypatch.delenv("HC_DEFAULT_TARGET", raising=False)
    assert g.device_available()
    for name in ("ref_17x19x18_seed7", "c1_128_f16_seed0"):
        fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
        a, b = fx["a"], fx["b"]
        print(f"case {name}", flush=True)
        c = np.zeros((a.shape[0], b.shape[1]), np.float32)
        hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, a, b, c)
        _check(c, fx["c_seq"], a.shape[1])


@pytest.mark.parametrize("m,n,k", [(4095, 3001, 1027), (300, 4100, 513), (16, 8192, 8191), (4100, 4096, 256),
                                   (1000, 33, 4096)])
def test_plain_hcg_gemm_entry_point(m, n, k):
    """hcg_gemm itself (not hcg_gemm_algo) with data: ragged, peeled, skinny
    and narrow shapes, against the oracle, into a NaN guard band."""
    from hc.gfx950 import _native
    from hc.gfx950.workloads import make_inputs

    print(f"case hcg_gemm {m}x{n}x{k}", flush=True)
    a, b = make_inputs("c5_ragged_f16", seed=11, m=m, n=n, k=k)
    ta, tb = _dev(a), _dev(b)
    guard = torch.full((m + 2, n + 8), float("nan"), dtype=torch.float32, device=DEV)
    view = guard[1 : m + 1, 4 : n + 4]
    lib = _native.load()
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.hcg_gemm(_native.HCG_F16, ta.data_ptr(), k, tb.data_ptr(), n, view.data_ptr(), view.stride(0), m, n, k,
                      stream)
    _native.check(lib, rc, "hcg_gemm")
    torch.cuda.synchronize()
    out = guard.cpu().numpy()
    _check(out[1 : m + 1, 4 : n + 4], oracle.gemm_c(a, b, oracle.F16), k)
    inner = np.zeros(out.shape, bool)
    inner[1 : m + 1, 4 : n + 4] = True
    assert np.isnan(out[~inner]).all(), "hcg_gemm wrote outside C"


def test_tiled_split_override_past_16_sums_every_partial():
    """HCG_TILED_SPLITS (read once, at the library's first call) past the
    16 partials the vector reduce holds: 512 x 512 x 16384 in 32 K splits
    must still sum all of K (a fresh process, so the override applies)."""
    import subprocess
    import sys
    import textwrap

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{os.path.join(root, "5_amd")!r}, {os.path.join(root, "oracle")!r}]
        import numpy as np, torch
        import hc.gfx950 as g, hc_oracle as oracle
        from hc.gfx950.workloads import make_inputs, to_torch
        a, b = make_inputs("c5_ragged_f16", seed=21, m=512, n=500, k=16384)
        dev = torch.device("cuda:0")
        for n in (512, 500):  # vector reduce (N % 4 == 0) and the element reduce
            out = g.gemm(to_torch(a, "float16", dev), to_torch(b[:, :n].copy(), "float16", dev), algo="tiled")
            torch.cuda.synchronize()
            rep = oracle.parity_check(out.cpu().numpy(), oracle.gemm_c(a, b[:, :n].copy()), 16384)
            print(n, rep, flush=True)
            assert rep.ok, rep
    """)
    print("case HCG_TILED_SPLITS=32 512x512x16384", flush=True)
    env = dict(os.environ, HCG_TILED_SPLITS="32")
    proc = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_compiled_handle_launches():
    import hc
    from hc.gfx950.kernels import tiled_gfx950_mfma_matmul_bf16
    from hc.gfx950.workloads import make_inputs

    a, b = make_inputs("c3_8192_bf16", seed=4, m=300, n=260, k=96)
    ta, tb = _dev(a, "bfloat16"), _dev(b, "bfloat16")
    tc = torch.empty((300, 260), dtype=torch.float32, device=DEV)
    hc.compile(tiled_gfx950_mfma_matmul_bf16)(ta, tb, tc)
    torch.cuda.synchronize()
    _check(tc.cpu().numpy(), oracle.gemm_sequential(a, b, oracle.BF16), 96)


# -- BASELINE.json configurations ------------------------------------------------


@pytest.mark.parametrize("name", ["c1_128_f16", "c2_4096_f16", "c3_8192_bf16", "c4_skinny_f16", "c5_ragged_f16"])
def test_baseline_config_full_size_against_oracle(name):
    from hc.gfx950.workloads import CONFIGS, make_inputs

    cfg = CONFIGS[name]
    print(f"case {name}", flush=True)
    a, b = make_inputs(cfg, seed=0)
    got = _gemm(a, b, dtype=cfg.dtype)
    want = oracle.gemm_c(a, b, _dt(cfg.dtype))
    _check(got, want, cfg.k)


def test_c3_bf16_8192_row_sums():
    """A size-independent property over the whole C3 output besides the
    elementwise check above: row sums of C equal A @ (B @ 1) (float64 on the
    host)."""
    from hc.gfx950.workloads import CONFIGS, make_inputs

    cfg = CONFIGS["c3_8192_bf16"]
    print("case c3 8192^3 bf16 row sums", flush=True)
    a, b = make_inputs(cfg, seed=0)
    got = _gemm(a, b, dtype=cfg.dtype)
    a64 = oracle.bf16_bits_to_f32(a).astype(np.float64)
    b64 = oracle.bf16_bits_to_f32(b).astype(np.float64)
    want = a64 @ b64.sum(axis=1)
    np.testing.assert_allclose(got.astype(np.float64).sum(axis=1), want, rtol=1e-3, atol=1e-3)


# -- tails, layouts, algorithms ---------------------------------------------------


SHAPES = [
    (1, 1, 1), (17, 19, 18), (128, 128, 128), (255, 257, 33), (256, 256, 32), (300, 520, 200),
    (513, 7, 1000), (64, 1024, 8), (1000, 1000, 1000), (257, 384, 4100), (4095, 3001, 1027),
]


@pytest.mark.parametrize("algo", ["auto", "tiled", "generic"])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_tails_f16(m, n, k, algo):
    from hc.gfx950.workloads import make_inputs

    print(f"case f16 m={m} n={n} k={k} algo={algo}", flush=True)
    a, b = make_inputs("c2_4096_f16", seed=m + n + k, m=m, n=n, k=k)
    _check(_gemm(a, b, algo), oracle.gemm_c(a, b), k)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("m,n,k", [(4095, 4100, 1000), (4096, 4096, 520), (4352, 3840, 96)])
def test_large_tile_variant_tails(m, n, k, dtype):
    """Shapes with at least 256 tiles of 256x256 take the 256-row tile
    variant; ragged M, N and K tails on it."""
    from hc.gfx950.workloads import make_inputs

    print(f"case large-tile {dtype} m={m} n={n} k={k}", flush=True)
    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + k, m=m, n=n, k=k)
    _check(_gemm(a, b, dtype=dtype), oracle.gemm_c(a, b, _dt(dtype)), k)


def test_large_tile_variant_integer_bit_exact():
    rng = np.random.default_rng(8)
    ai = rng.integers(-4, 5, size=(4096, 512))
    bi = rng.integers(-4, 5, size=(512, 4104))
    got = _gemm(ai.astype(np.float16), bi.astype(np.float16))
    assert np.array_equal(got, (ai @ bi).astype(np.float32))


TILE_ALGOS = ["tiled_256x256", "tiled_256x192", "tiled_128x256", "tiled_128x128", "tiled_256x64"]


@pytest.mark.parametrize("algo", TILE_ALGOS)
@pytest.mark.parametrize("m,n,k", [(17, 19, 18), (255, 257, 33), (520, 400, 1027), (1000, 3001, 264),
                                   (768, 768, 4096)])
def test_tile_shapes_tails(algo, m, n, k):
    """Every output tile shape of the LDS-tiled kernel, forced, on ragged
    M/N/K (K past and within one 32-wide tile, unaligned rows) and on a
    shape where every K tile takes the unchecked load path."""
    from hc.gfx950.workloads import make_inputs

    print(f"case {algo} m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c2_4096_f16", seed=m + 3 * n + k, m=m, n=n, k=k)
    _check(_gemm(a, b, algo), oracle.gemm_c(a, b), k)


@pytest.mark.parametrize("algo", TILE_ALGOS)
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_tile_shapes_integer_bit_exact(algo, dtype):
    rng = np.random.default_rng(11)
    ai = rng.integers(-4, 5, size=(600, 1024))
    bi = rng.integers(-4, 5, size=(1024, 712))
    if dtype == "float16":
        a, b = ai.astype(np.float16), bi.astype(np.float16)
    else:
        a, b = oracle.f32_to_bf16_bits(ai.astype(np.float32)), oracle.f32_to_bf16_bits(bi.astype(np.float32))
    print(f"case integer {algo} {dtype}", flush=True)
    assert np.array_equal(_gemm(a, b, algo, dtype), (ai @ bi).astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(17, 19, 18), (300, 520, 200), (1000, 1000, 1000), (2048, 512, 3000)])
def test_tails_bf16(m, n, k):
    from hc.gfx950.workloads import make_inputs

    print(f"case bf16 m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c3_8192_bf16", seed=m + n + k, m=m, n=n, k=k)
    _check(_gemm(a, b, dtype="bfloat16"), oracle.gemm_c(a, b, oracle.BF16), k)


@pytest.mark.parametrize("m", [1, 2, 5, 8, 13, 16])
@pytest.mark.parametrize("n,k", [(8192, 8192), (1000, 333), (260, 1000), (128, 32), (3001, 1027)])
def test_skinny(m, n, k):
    from hc.gfx950.workloads import make_inputs

    print(f"case skinny m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c4_skinny_f16", seed=m * 7 + n + k, m=m, n=n, k=k)
    _check(_gemm(a, b, "skinny"), oracle.gemm_c(a, b), k)


@pytest.mark.parametrize("m,n,k", [(16, 1000, 1000), (3, 8192, 520), (16, 4104, 8192), (7, 64, 4096),
                                   (16, 65536, 4096), (16, 128, 256)])
def test_skinny_split_and_block_mapping(m, n, k):
    """The streaming kernel's split-K and workgroup-to-column-block mapping:
    column-block counts that are not multiples of 8 (padding workgroups),
    ragged last splits, one split (C written directly) and many blocks."""
    from hc.gfx950.workloads import make_inputs

    print(f"case skinny mapping m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c4_skinny_f16", seed=m + n + 5 * k, m=m, n=n, k=k)
    _check(_gemm(a, b, "skinny"), oracle.gemm_c(a, b), k)


# M up to 128 streams B once through the skinny kernel with 1, 2, 4 or 8
# 16-row blocks of A (rows past M load as zero and are never stored).
@pytest.mark.parametrize("m", [17, 24, 32, 33, 48, 64, 65, 100, 128])
@pytest.mark.parametrize("n,k", [(8192, 8192), (1000, 336), (256, 1024), (4104, 520)])
@pytest.mark.parametrize("algo", ["auto", "skinny"])
def test_skinny_row_blocks(m, n, k, algo):
    from hc.gfx950.workloads import make_inputs

    print(f"case skinny rows {algo} m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c4_skinny_f16", seed=m * 5 + n + k, m=m, n=n, k=k)
    _check(_gemm(a, b, algo), oracle.gemm_c(a, b), k)


@pytest.mark.parametrize("m", [20, 40, 72, 128])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_skinny_row_blocks_integer_bit_exact(m, dtype):
    rng = np.random.default_rng(m)
    ai = rng.integers(-4, 5, size=(m, 2048))
    bi = rng.integers(-4, 5, size=(2048, 1024))
    if dtype == "float16":
        a, b = ai.astype(np.float16), bi.astype(np.float16)
    else:
        a, b = oracle.f32_to_bf16_bits(ai.astype(np.float32)), oracle.f32_to_bf16_bits(bi.astype(np.float32))
    print(f"case skinny rows integer {dtype} m={m}", flush=True)
    assert np.array_equal(_gemm(a, b, "skinny", dtype), (ai @ bi).astype(np.float32))


def test_skinny_rows_take_any_layout_but_a_tiny_b():
    """Above 16 rows the skinny path is the streaming kernel only: A is
    repacked when its rows cannot be read in place, B's unaligned rows are
    read in place by DMA (or register-staged).  A B of fewer than 8 elements
    is read in place too."""
    from hc.gfx950.workloads import make_inputs

    for seed, (m, n, k) in enumerate([(40, 1001, 333), (40, 1000, 333), (17, 9, 7)]):
        a, b = make_inputs("c4_skinny_f16", seed=3 + seed, m=m, n=n, k=k)
        _check(_gemm(a, b, "skinny"), oracle.gemm_c(a, b), k)
    a, b = make_inputs("c4_skinny_f16", seed=9, m=40, n=5, k=1)
    _check(_gemm(a, b, "skinny"), oracle.gemm_c(a, b), 1)
    # (test_paths_for_operands_the_dma_cannot_read covers the LaunchError)


@pytest.mark.parametrize("m,n,k", [(1, 8191, 8192), (16, 8191, 8191), (17, 50257, 1024), (64, 1001, 4096),
                                   (128, 333, 2049), (5, 7, 9), (100, 8, 1), (16, 4099, 16384)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_streaming_kernel_register_staged_b(m, n, k, dtype):
    """B's rows not 16-byte aligned (tight, odd N): the streaming kernel reads
    them in place by DMA (16-byte chunks at 2-byte alignment; the chunk
    holding column N - 1 brings columns that reach no stored element), C in a
    NaN guard band.  (The page-end test below forces the register-staged
    form.)"""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    cfg = "c4_skinny_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + n + k, m=m, n=n, k=k)
    guard = torch.full((m + 2, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    out = guard[1 : m + 1, 1 : n + 1]
    print(f"case stream register-staged B {dtype} m={m} n={n} k={k}", flush=True)
    g.gemm(_dev(a, dtype), _dev(b, dtype), out=out, algo="skinny")
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 1 : n + 1], oracle.gemm_c(a, b, _dt(dtype)), k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


@pytest.mark.parametrize("m,n,k,pad_a,pad_b", [(4096, 13, 4096, 3, 0), (3000, 40, 2048, 0, 5), (777, 64, 1024, 1, 1)])
def test_narrow_kernel_unaligned_rows_in_place(m, n, k, pad_a, pad_b):
    """The narrow kernel reads A (K a multiple of 8) and B with rows that are
    not 16-byte aligned in place; row padding holds NaN."""
    import hc.gfx950 as g

    rng = np.random.default_rng(m + n + k)
    ai = rng.integers(-4, 5, size=(m, k))
    bi = rng.integers(-4, 5, size=(k, n))
    big_a = torch.full((m, k + pad_a), float("nan"), dtype=torch.float16, device=DEV)
    big_b = torch.full((k, n + pad_b), float("nan"), dtype=torch.float16, device=DEV)
    big_a[:, :k] = torch.from_numpy(ai).to(DEV, torch.float16)
    big_b[:, :n] = torch.from_numpy(bi).to(DEV, torch.float16)
    guard = torch.full((m + 2, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    out = guard[1 : m + 1, 1 : n + 1]
    print(f"case narrow unaligned in place m={m} n={n} k={k} pad_a={pad_a} pad_b={pad_b}", flush=True)
    g.gemm(big_a[:, :k], big_b[:, :n], out=out, algo="narrow")
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    assert np.array_equal(host[1 : m + 1, 1 : n + 1], (ai @ bi).astype(np.float32))
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


@pytest.mark.parametrize("m,n,k,pad", [(16, 8192, 8192, 3), (64, 2048, 4096, 1), (40, 1000, 1024, 5)])
def test_streaming_kernel_unaligned_a_in_place(m, n, k, pad):
    """A as a column-sliced view with odd row stride and K a multiple of 8:
    read in place by the DMA; the row padding holds NaN."""
    import hc.gfx950 as g

    rng = np.random.default_rng(m + n + k)
    ai = rng.integers(-4, 5, size=(m, k))
    bi = rng.integers(-4, 5, size=(k, n))
    big_a = torch.full((m, k + pad), float("nan"), dtype=torch.float16, device=DEV)
    big_a[:, :k] = torch.from_numpy(ai).to(DEV, torch.float16)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    print(f"case stream unaligned A in place m={m} n={n} k={k} pad={pad}", flush=True)
    g.gemm(big_a[:, :k], torch.from_numpy(bi).to(DEV, torch.float16), out=out, algo="skinny")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), (ai @ bi).astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(16, 8192, 8191), (64, 2048, 4095), (128, 1000, 1001), (5, 4096, 2049)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_streaming_kernel_k_not_a_multiple_of_8(m, n, k, dtype):
    """K not a multiple of 8 (A's rows unaligned): A is read in place, the
    chunk straddling K cleared past K in the fragments, while A's row
    padding holds NaN; B streams through the DMA.  (A whose last chunk
    cannot be read safely is repacked instead: the HCG_UNALIGNED_DMA=0
    test.)"""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    cfg = "c4_skinny_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + k, m=m, n=n, k=k)
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    big_a = torch.full((m, k + 3), float("nan"), dtype=tdt, device=DEV)
    big_a[:, :k] = _dev(a, dtype)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    print(f"case stream K tail {dtype} m={m} n={n} k={k}", flush=True)
    g.gemm(big_a[:, :k], _dev(b, dtype), out=out, algo="skinny")
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), oracle.gemm_c(a, b, _dt(dtype)), k)


# Few output tiles and a long K: the tiled kernel splits K over several
# workgroups per tile and sums their partials in a fixed order.  Shapes
# include ragged M/N tails, a last split shorter than the others, unaligned
# rows (read in place by every split) and bf16.
SPLITK_SHAPES = [(1024, 1024, 8192), (512, 512, 16384), (700, 900, 12000), (200, 8000, 8200), (1500, 1500, 4104),
                 (333, 444, 9999), (1024, 4096, 16384)]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("m,n,k", SPLITK_SHAPES)
def test_split_k_against_oracle(m, n, k, dtype):
    from hc.gfx950.workloads import make_inputs

    print(f"case split-k {dtype} m={m} n={n} k={k}", flush=True)
    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + 2 * n + k, m=m, n=n, k=k)
    want = oracle.gemm_c(a, b, oracle.F16 if dtype == "float16" else oracle.BF16)
    _check(_gemm(a, b, "auto", dtype), want, k)


@pytest.mark.parametrize("m,n,k", [(512, 512, 16384), (300, 1000, 8200)])
def test_split_k_integer_bit_exact_and_reproducible(m, n, k):
    rng = np.random.default_rng(k)
    ai = rng.integers(-3, 4, size=(m, k))
    bi = rng.integers(-3, 4, size=(k, n))
    a, b = ai.astype(np.float16), bi.astype(np.float16)
    print(f"case split-k integer m={m} n={n} k={k}", flush=True)
    first = _gemm(a, b)
    assert np.array_equal(first, (ai @ bi).astype(np.float32))
    assert np.array_equal(first.view(np.uint32), _gemm(a, b).view(np.uint32))


# Narrow N (few output columns, e.g. low-rank projections): 256x64 tiles
# over M with a K split, including N not a multiple of 4 (partials summed
# one element at a time) and unaligned K.
@pytest.mark.parametrize("m,n,k", [(4096, 13, 8192), (16384, 8, 16384), (5000, 7, 5000), (3000, 1, 9000),
                                   (4096, 64, 4096), (8000, 33, 2048), (2048, 3, 777)])
def test_narrow_n_against_oracle(m, n, k):
    from hc.gfx950.workloads import make_inputs

    print(f"case narrow n m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c2_4096_f16", seed=m + n + k, m=m, n=n, k=k)
    _check(_gemm(a, b), oracle.gemm_c(a, b), k)


# N <= 32 with aligned rows: the narrow streaming kernel (A in 256-byte row
# pieces, row blocks of 64, K split to fill the chip).
@pytest.mark.parametrize("m,n,k", [(17, 1, 8), (64, 16, 128), (100, 13, 1000), (1000, 32, 4096), (4096, 8, 8192),
                                   (16384, 16, 16384), (333, 17, 520), (2048, 24, 12000), (65, 3, 136)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_narrow_streaming_kernel_against_oracle(m, n, k, dtype):
    from hc.gfx950.workloads import make_inputs

    print(f"case narrow streaming {dtype} m={m} n={n} k={k}", flush=True)
    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m * 3 + n + k, m=m, n=n, k=k)
    want = oracle.gemm_c(a, b, oracle.F16 if dtype == "float16" else oracle.BF16)
    _check(_gemm(a, b, "narrow", dtype), want, k)


@pytest.mark.parametrize("m,n,k", [(4096, 13, 8192), (300, 32, 2048), (129, 1, 4096)])
def test_narrow_streaming_integer_bit_exact_and_reproducible(m, n, k):
    rng = np.random.default_rng(m + n + k)
    ai = rng.integers(-4, 5, size=(m, k))
    bi = rng.integers(-4, 5, size=(k, n))
    a, b = ai.astype(np.float16), bi.astype(np.float16)
    print(f"case narrow integer m={m} n={n} k={k}", flush=True)
    first = _gemm(a, b, "narrow")
    assert np.array_equal(first, (ai @ bi).astype(np.float32))
    assert np.array_equal(first.view(np.uint32), _gemm(a, b, "narrow").view(np.uint32))


def test_narrow_streaming_views_and_guard_band():
    """Row strides above K and N (multiples of 8), C into a NaN guard band."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    m, n, k = 777, 19, 2056
    a, b = make_inputs("c2_4096_f16", seed=77, m=m, n=n, k=k)
    big_a = torch.zeros((m, k + 8), dtype=torch.float16, device=DEV)
    big_b = torch.zeros((k, 24 + 16), dtype=torch.float16, device=DEV)
    va, vb = big_a[:, :k], big_b[:, :n]
    va.copy_(_dev(a))
    vb.copy_(_dev(b))
    guard = torch.full((m + 2, n + 3), float("nan"), dtype=torch.float32, device=DEV)
    vc = guard[1 : m + 1, 1 : n + 1]
    print("case narrow views", flush=True)
    g.gemm(va, vb, out=vc, algo="narrow")
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 1 : n + 1], oracle.gemm_c(a, b), k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


def test_narrow_kernel_rejects_what_it_cannot_run():
    from hc import LaunchError
    from hc.gfx950.workloads import make_inputs

    a, b = make_inputs("c2_4096_f16", seed=1, m=100, n=65, k=256)
    with pytest.raises(LaunchError, match="narrow kernel needs N <= 64"):
        _gemm(a, b, "narrow")


@pytest.mark.parametrize("m,n,k", [(100, 8, 257), (16384, 8, 16383), (4096, 13, 8191), (3000, 32, 4095),
                                   (777, 1, 9), (65, 17, 1), (2049, 24, 130)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_narrow_kernel_k_not_a_multiple_of_8(m, n, k, dtype):
    """K not a multiple of 8 (odd K in a tight A, plus NaN row padding
    beyond K in a view): the narrow kernel's DMA brings the chunk that
    straddles K, and the fragments clear its elements at k >= K before they
    meet B (A whose last chunk cannot be read safely goes through registers,
    with the same clearing; see the HCG_UNALIGNED_DMA=0 test)."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + n + k, m=m, n=n, k=k)
    want = oracle.gemm_c(a, b, _dt(dtype))
    print(f"case narrow K tail {dtype} m={m} n={n} k={k}", flush=True)
    _check(_gemm(a, b, "narrow", dtype), want, k)
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    big_a = torch.full((m, k + 5), float("nan"), dtype=tdt, device=DEV)
    big_a[:, :k] = _dev(a, dtype)
    guard = torch.full((m + 2, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    out = guard[1 : m + 1, 1 : n + 1]
    g.gemm(big_a[:, :k], _dev(b, dtype), out=out, algo="narrow")
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 1 : n + 1], want, k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


@pytest.mark.parametrize("m,n,k", [(1000, 48, 4096), (4096, 64, 8192), (333, 40, 520), (2049, 63, 130),
                                   (16384, 64, 16384), (129, 33, 4095), (5000, 57, 777)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_narrow_kernel_64_columns(m, n, k, dtype):
    """33..64 columns: the narrow kernel's 64-column form (5-stage ring, A
    and B of a stage in one 32 KB object), A by DMA (odd K: the chunk
    straddling K cleared past K), C in a NaN guard band."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + 3 * n + k, m=m, n=n, k=k)
    guard = torch.full((m + 2, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    out = guard[1 : m + 1, 1 : n + 1]
    print(f"case narrow 64 {dtype} m={m} n={n} k={k}", flush=True)
    g.gemm(_dev(a, dtype), _dev(b, dtype), out=out, algo="narrow")
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 1 : n + 1], oracle.gemm_c(a, b, _dt(dtype)), k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


def test_narrow_kernel_k_tail_integer_bit_exact():
    rng = np.random.default_rng(21)
    ai = rng.integers(-4, 5, size=(5000, 4095))
    bi = rng.integers(-4, 5, size=(4095, 11))
    want = (ai.astype(np.float64) @ bi.astype(np.float64)).astype(np.float32)
    got = _gemm(ai.astype(np.float16), bi.astype(np.float16), "narrow")
    assert np.array_equal(got, want)


def test_skinny_repeated_launches_alternating_shapes():
    """The per-stream workspace is reused across launches of different
    shapes: each result matches the oracle, and the same input gives the
    same bits again."""
    from hc.gfx950.workloads import make_inputs

    big = make_inputs("c4_skinny_f16", seed=21, m=16, n=8192, k=8192)
    small = make_inputs("c4_skinny_f16", seed=22, m=16, n=1024, k=2048)
    first = _gemm(*big, "skinny")
    _check(first, oracle.gemm_c(*big), 8192)
    _check(_gemm(*small, "skinny"), oracle.gemm_c(*small), 2048)
    again = _gemm(*big, "skinny")
    assert np.array_equal(first.view(np.uint32), again.view(np.uint32))


@pytest.mark.parametrize("algo,m", [("tiled", 300), ("skinny", 16), ("generic", 300)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_integer_inputs_bit_exact(algo, m, dtype):
    rng = np.random.default_rng(3)
    ai = rng.integers(-4, 5, size=(m, 1000))
    bi = rng.integers(-4, 5, size=(1000, 520))
    if dtype == "float16":
        a, b = ai.astype(np.float16), bi.astype(np.float16)
    else:
        a, b = oracle.f32_to_bf16_bits(ai.astype(np.float32)), oracle.f32_to_bf16_bits(bi.astype(np.float32))
    print(f"case integer {algo} {dtype}", flush=True)
    got = _gemm(a, b, algo, dtype)
    assert np.array_equal(got, (ai @ bi).astype(np.float32))


@pytest.mark.parametrize("algo,m", [("auto", 1024), ("skinny", 16)])
def test_runs_are_bit_identical(algo, m):
    from hc.gfx950.workloads import make_inputs

    a, b = make_inputs("c2_4096_f16", seed=9, m=m, n=2048, k=2048)
    first = _gemm(a, b, algo)
    for _ in range(2):
        assert np.array_equal(first.view(np.uint32), _gemm(a, b, algo).view(np.uint32))


# Operands whose rows are not 16-byte aligned (odd K or N, odd row strides,
# 2-byte aligned starts), forced onto 256x192 tiles and read in place: no
# element past K or N may reach C (K and N down to 1 element past a chunk).
UNALIGNED_SHAPES = [(601, 713, 1027), (513, 200, 353), (300, 8, 5), (300, 9, 1), (17, 8, 1), (40, 8, 352),
             (257, 193, 320), (600, 1001, 2049), (300, 7, 40)]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("m,n,k", UNALIGNED_SHAPES)
def test_unaligned_operands_integer_bit_exact(m, n, k, dtype):
    """Small-integer inputs make every summation order exact, so the
    unaligned operands must give A @ B bit for bit, tails included."""
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    ai = rng.integers(-4, 5, size=(m, k))
    bi = rng.integers(-4, 5, size=(k, n))
    if dtype == "float16":
        a, b = ai.astype(np.float16), bi.astype(np.float16)
    else:
        a, b = oracle.f32_to_bf16_bits(ai.astype(np.float32)), oracle.f32_to_bf16_bits(bi.astype(np.float32))
    print(f"case unaligned integer {dtype} m={m} n={n} k={k}", flush=True)
    assert np.array_equal(_gemm(a, b, "tiled_256x192", dtype), (ai @ bi).astype(np.float32))


@pytest.mark.parametrize("m,n,k,pad_a,pad_b", [(601, 713, 1027, 3, 1), (333, 270, 150, 9, 5), (300, 8, 40, 1, 7),
                                               (4095, 3001, 1027, 0, 0)])
def test_unaligned_strided_views_against_oracle(m, n, k, pad_a, pad_b):
    """Column-sliced views with odd row strides and 2-byte aligned starts,
    C into a NaN guard band, against the oracle's float32 fold."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    a, b = make_inputs("c2_4096_f16", seed=m + n + k, m=m, n=n, k=k)
    big_a = torch.zeros((m, k + pad_a + 1), dtype=torch.float16, device=DEV)
    big_b = torch.zeros((k, n + pad_b + 1), dtype=torch.float16, device=DEV)
    va, vb = big_a[:, 1 : k + 1], big_b[:, 1 : n + 1]
    va.copy_(_dev(a))
    vb.copy_(_dev(b))
    guard = torch.full((m + 2, n + 3), float("nan"), dtype=torch.float32, device=DEV)
    vc = guard[1 : m + 1, 1 : n + 1]
    print(f"case unaligned views m={m} n={n} k={k}", flush=True)
    g.gemm(va, vb, out=vc, algo="tiled_256x192")
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 1 : n + 1], oracle.gemm_c(a, b), k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


# Rows that are not 16-byte aligned are read in place by the tiled kernel's
# DMA (16-byte chunks at 2-byte alignment).  The chunk of A holding column
# K - 1 also brings up to 7 elements past K: row padding (here +Inf, so an
# uncleared element would turn a product with B's zeroed rows into NaN) or,
# for tight rows, the next row.
@pytest.mark.parametrize(
    "m,n,k,pad_a,pad_b,algo,dtype",
    [
        (4095, 3001, 1027, 0, 0, "auto", "float16"),
        (601, 713, 1027, 9, 3, "tiled_256x192", "float16"),
        (333, 270, 150, 1, 1, "tiled_128x128", "bfloat16"),
        (300, 1000, 8195, 3, 5, "auto", "float16"),
        (257, 129, 31, 7, 0, "tiled_256x256", "bfloat16"),
        (64, 200, 13, 3, 3, "tiled_128x256", "float16"),
        (700, 64, 2049, 5, 1, "tiled_256x64", "float16"),
        # 65..128 rows with B's rows unaligned: AUTO sends them to the tiled
        # kernel (split along K), which reads B in place
        (128, 3001, 1027, 0, 0, "auto", "float16"),
        (100, 5001, 1024, 3, 0, "auto", "bfloat16"),
        (72, 1229, 4096, 0, 1, "auto", "float16"),
    ],
)
def test_unaligned_rows_read_in_place(m, n, k, pad_a, pad_b, algo, dtype):
    import hc.gfx950 as g

    rng = np.random.default_rng(m + 3 * n + 7 * k)
    ai = rng.integers(-4, 5, size=(m, k))
    bi = rng.integers(-4, 5, size=(k, n))
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    big_a = torch.full((m, k + pad_a), float("inf"), dtype=tdt, device=DEV)
    big_b = torch.full((k, n + pad_b), float("inf"), dtype=tdt, device=DEV)
    va, vb = big_a[:, :k], big_b[:, :n]
    va.copy_(torch.from_numpy(ai).to(DEV, tdt))
    vb.copy_(torch.from_numpy(bi).to(DEV, tdt))
    guard = torch.full((m + 2, n + 3), float("nan"), dtype=torch.float32, device=DEV)
    vc = guard[1 : m + 1, 1 : n + 1]
    print(f"case in-place unaligned {algo} {dtype} m={m} n={n} k={k} pad_a={pad_a} pad_b={pad_b}", flush=True)
    g.gemm(va, vb, out=vc, algo=algo)
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    assert np.array_equal(host[1 : m + 1, 1 : n + 1], (ai @ bi).astype(np.float32))
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


def test_paths_for_operands_the_dma_cannot_read():
    """With HCG_UNALIGNED_DMA=0 (a fresh process: the library reads it once)
    no row that is not 16-byte aligned is read in place, as for an operand
    whose last chunk would reach past its allocation: the tiled kernel then
    repacks A and B (C5's shape, +Inf in the row padding), the streaming
    kernel register-stages B (fp16 and bf16, the chunk ending at B's last
    element included) and repacks A, the narrow kernel repacks B and stages
    A through registers, and a B of fewer than 8 elements is a LaunchError
    for an explicit skinny request while auto still runs."""
    import subprocess
    import sys
    import textwrap

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{os.path.join(root, "5_amd")!r}, {os.path.join(root, "oracle")!r}]
        import numpy as np, torch
        import hc.gfx950 as g, hc_oracle as oracle
        from hc import LaunchError
        from hc.gfx950.workloads import make_inputs, to_torch
        dev = torch.device("cuda:0")
        rng = np.random.default_rng(5)
        for m, n, k, pad_a, pad_b, algo in [(4095, 3001, 1027, 0, 0, "auto"), (601, 713, 1027, 9, 3, "tiled_256x192"),
                                            (16, 8191, 4096, 0, 0, "skinny"), (17, 50257, 1024, 0, 0, "skinny"),
                                            (16, 4096, 2049, 0, 0, "skinny"),
                                            (64, 1001, 4096, 3, 0, "skinny"), (5, 7, 9, 0, 0, "skinny"),
                                            (3000, 13, 4096, 0, 0, "narrow"), (300, 40, 1024, 3, 5, "narrow"),
                                            (4096, 13, 8191, 0, 0, "narrow"), (100, 8, 257, 5, 0, "narrow")]:
            for dt in (torch.float16, torch.bfloat16):
                ai = rng.integers(-4, 5, size=(m, k)); bi = rng.integers(-4, 5, size=(k, n))
                big_a = torch.full((m, k + pad_a), float("inf"), dtype=dt, device=dev)
                big_b = torch.full((k, n + pad_b), float("inf"), dtype=dt, device=dev)
                big_a[:, :k] = torch.from_numpy(ai).to(dev, dt); big_b[:, :n] = torch.from_numpy(bi).to(dev, dt)
                out = g.gemm(big_a[:, :k], big_b[:, :n], algo=algo)
                torch.cuda.synchronize()
                ok = np.array_equal(out.cpu().numpy(), (ai @ bi).astype(np.float32))
                print(m, n, k, algo, dt, ok, flush=True)
                assert ok
        a, b = make_inputs("c4_skinny_f16", seed=9, m=40, n=5, k=1)
        ta, tb = to_torch(a, "float16", dev), to_torch(b, "float16", dev)
        try:
            g.gemm(ta, tb, algo="skinny")
            raise SystemExit("expected a LaunchError for a B of 5 elements")
        except LaunchError as exc:
            assert "B under 8 elements" in str(exc), exc
        out = g.gemm(ta, tb, algo="auto")
        torch.cuda.synchronize()
        assert oracle.parity_check(out.cpu().numpy(), oracle.gemm_c(a, b), 1).ok
    """)
    print("case HCG_UNALIGNED_DMA=0 repack and register-staged paths", flush=True)
    env = dict(os.environ, HCG_UNALIGNED_DMA="0")
    proc = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stdout + proc.stderr


@pytest.mark.parametrize("algo", ["auto"] + TILE_ALGOS)
def test_strided_views_and_guard_band(algo):
    """A and B as column-sliced views (lda > K, ldb > N, 2-byte aligned
    starts), C as a view into a NaN-filled buffer: only C's M x N elements
    change (hc/simulator.py:1441-1458 writes only in-bounds C)."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    m, n, k = 333, 270, 150
    a, b = make_inputs("c2_4096_f16", seed=12, m=m, n=n, k=k)
    big_a = torch.zeros((m, k + 9), dtype=torch.float16, device=DEV)
    big_b = torch.zeros((k, n + 5), dtype=torch.float16, device=DEV)
    va, vb = big_a[:, 1 : k + 1], big_b[:, 3 : n + 3]
    va.copy_(_dev(a))
    vb.copy_(_dev(b))
    guard = torch.full((m + 2, n + 7), float("nan"), dtype=torch.float32, device=DEV)
    vc = guard[1 : m + 1, 2 : n + 2]
    print(f"case guard band {algo}", flush=True)
    g.gemm(va, vb, out=vc, algo=algo)
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 2 : n + 2], oracle.gemm_c(a, b), k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 2 : n + 2] = False
    assert np.all(np.isnan(host[mask]))


def test_k_zero_writes_zeros_and_empty_output_is_untouched():
    import hc.gfx950 as g

    a = torch.zeros((40, 0), dtype=torch.float16, device=DEV)
    b = torch.zeros((0, 30), dtype=torch.float16, device=DEV)
    c = torch.full((40, 30), 7.0, dtype=torch.float32, device=DEV)
    g.gemm(a, b, out=c)
    torch.cuda.synchronize()
    assert torch.count_nonzero(c).item() == 0
    e = torch.full((0, 30), 7.0, dtype=torch.float32, device=DEV)
    g.gemm(torch.zeros((0, 5), dtype=torch.float16, device=DEV), torch.zeros((5, 30), dtype=torch.float16, device=DEV), out=e)


def test_k_zero_output_over_2_to_32_elements():
    """K = 0 writes zeros over a C of more than 2^32 elements (a launch holds
    fewer work-items than that), a view in a NaN buffer whose other columns
    and row stay untouched."""
    import hc.gfx950 as g

    m, n, ld = 65537, 65536, 65540
    print(f"case K=0 C of {m * n} elements", flush=True)
    buf = torch.full((m + 1, ld), float("nan"), dtype=torch.float32, device=DEV)
    a = torch.zeros((m, 0), dtype=torch.float16, device=DEV)
    b = torch.zeros((0, n), dtype=torch.float16, device=DEV)
    g.gemm(a, b, out=buf[:m, :n])
    torch.cuda.synchronize()
    assert bool((buf[:m, :n] == 0).all())
    assert bool(torch.isnan(buf[:m, n:]).all()) and bool(torch.isnan(buf[m:]).all())
    del buf


# C over 2 GiB on each kernel family that writes C directly (the tiled
# kernel, the streaming kernel, the narrow kernel): small-integer inputs make
# every sum exact, so float32 products on the host are the exact answer.
@pytest.mark.parametrize("algo,m,n,k", [("auto", 24000, 24000, 40), ("skinny", 128, 4200000, 40),
                                        ("narrow", 8400000, 64, 40)])
def test_output_over_2gib_bit_exact(algo, m, n, k):
    import hc.gfx950 as g

    print(f"case C over 2 GiB {algo} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m + n)
    ai = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    bi = rng.integers(-3, 4, size=(k, n)).astype(np.float32)
    c = g.gemm(torch.from_numpy(ai).to(DEV).half(), torch.from_numpy(bi).to(DEV).half(), algo=algo)
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    del c
    assert np.array_equal(got, ai @ bi)  # |sums| <= 360: exact in float32


def test_two_streams_use_separate_workspaces():
    """The split-K workspace is per stream: two streams running skinny GEMMs
    concurrently must not corrupt each other."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    a1, b1 = make_inputs("c4_skinny_f16", seed=1, m=16, n=4096, k=8192)
    a2, b2 = make_inputs("c4_skinny_f16", seed=2, m=16, n=4096, k=8192)
    t = [(_dev(a1), _dev(b1)), (_dev(a2), _dev(b2))]
    outs = [torch.empty((16, 4096), dtype=torch.float32, device=DEV) for _ in range(2)]
    streams = [torch.cuda.Stream(device=DEV) for _ in range(2)]
    torch.cuda.synchronize()
    for _ in range(5):
        for s, (ta, tb), o in zip(streams, t, outs):
            with torch.cuda.stream(s):
                g.gemm(ta, tb, out=o, algo="skinny")
    torch.cuda.synchronize()
    _check(outs[0].cpu().numpy(), oracle.gemm_c(a1, b1), 8192)
    _check(outs[1].cpu().numpy(), oracle.gemm_c(a2, b2), 8192)


def test_numpy_bf16_is_not_accepted_and_launch_errors_surface():
    import hc.gfx950 as g
    from hc import LaunchError

    with pytest.raises(LaunchError):
        g.gemm(np.zeros((4, 4), np.uint16), np.zeros((4, 4), np.uint16))
    with pytest.raises(LaunchError, match="same device|torch tensors"):
        g.gemm(torch.zeros((4, 4), dtype=torch.float16), torch.zeros((4, 4), dtype=torch.float16, device=DEV))


# Seeded random shapes, layouts and kernel choices against the oracle: every
# path (tiled with and without a K split, unaligned operands read in place,
# the streaming kernel at every row-block count, the narrow kernel, the
# register-staged skinny fallback and the generic kernel) on shapes nobody
# picked by hand,
# with NaN in the operands' row padding and around C.
_RANDOM_ALGOS = ["auto", "auto", "auto", "tiled", "skinny", "generic", "tiled_128x128", "tiled_256x192"]


def _random_case(i):
    rng = np.random.default_rng(1000 + i)
    algo = _RANDOM_ALGOS[i % len(_RANDOM_ALGOS)]
    if algo == "skinny" or rng.random() < 0.3:
        m = int(rng.integers(1, 129))
    else:
        m = int(rng.integers(1, 1600))
    n = int(rng.integers(1, 1600))
    k = int(rng.choice([rng.integers(1, 64), rng.integers(64, 2048), rng.integers(2048, 9000)]))
    if algo == "skinny" and m > 16:
        # above 16 rows the skinny path needs aligned rows and K a multiple of 8
        k = max(8, k // 8 * 8)
    pad_a = int(rng.choice([0, 0, 1, 3, 8]))
    pad_b = int(rng.choice([0, 0, 1, 5, 8]))
    if algo == "skinny" and m > 16:
        # aligned rows: B's row stride padded to a multiple of 8 (N itself may not be)
        pad_a, pad_b = pad_a // 8 * 8, (-n) % 8 + pad_b // 8 * 8
    dtype = "float16" if rng.random() < 0.7 else "bfloat16"
    return algo, m, n, k, pad_a, pad_b, dtype


@pytest.mark.parametrize("i", range(48))
def test_random_shapes_and_layouts_against_oracle(i):
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    algo, m, n, k, pad_a, pad_b, dtype = _random_case(i)
    print(f"case random {i}: {algo} {dtype} m={m} n={n} k={k} pad_a={pad_a} pad_b={pad_b}", flush=True)
    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=i, m=m, n=n, k=k)
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    # row padding holds NaN: no kernel may let an element outside the views reach C
    big_a = torch.full((m, k + pad_a), float("nan"), dtype=tdt, device=DEV)
    big_b = torch.full((k, n + pad_b), float("nan"), dtype=tdt, device=DEV)
    va, vb = big_a[:, :k], big_b[:, :n]
    va.copy_(_dev(a, dtype))
    vb.copy_(_dev(b, dtype))
    guard = torch.full((m + 1, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    vc = guard[:m, 1 : n + 1]
    g.gemm(va, vb, out=vc, algo=algo)
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[:m, 1 : n + 1], oracle.gemm_c(a, b, oracle.F16 if dtype == "float16" else oracle.BF16), k)
    mask = np.ones_like(host, dtype=bool)
    mask[:m, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


# Views that start 1..7 elements into their allocation (so rows sit at any
# 2-byte alignment) with odd row pitches, for every kernel choice: the DMA
# kernels read such rows in place, and a chunk past a row's end must never
# reach C.  NaN fills everything outside the views.
_OFFSET_ALGOS = ["auto", "auto", "tiled", "tiled_256x256", "tiled_256x192", "tiled_128x256", "tiled_128x128",
                 "tiled_256x64", "skinny", "narrow", "generic"]


@pytest.mark.parametrize("i", range(44))
def test_random_base_offsets_against_oracle(i):
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    rng = np.random.default_rng(70000 + i)
    algo = _OFFSET_ALGOS[i % len(_OFFSET_ALGOS)]
    m = int(rng.integers(1, 129)) if algo == "skinny" or rng.random() < 0.2 else int(rng.integers(1, 1300))
    n = int(rng.integers(1, 65)) if algo == "narrow" else int(rng.integers(1, 1300))
    k = int(rng.choice([rng.integers(1, 64), rng.integers(64, 3000)]))
    pad_a, pad_b = int(rng.choice([0, 1, 2, 3, 7, 64])), int(rng.choice([0, 1, 2, 5, 64]))
    off_a, off_b = int(rng.integers(0, 8)), int(rng.integers(0, 8))
    dtype = "float16" if rng.random() < 0.7 else "bfloat16"
    print(f"case offsets {i}: {algo} {dtype} m={m} n={n} k={k} pads={pad_a},{pad_b} offs={off_a},{off_b}",
          flush=True)
    a, b = make_inputs("c2_4096_f16" if dtype == "float16" else "c3_8192_bf16", seed=i, m=m, n=n, k=k)
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    big_a = torch.full((m, off_a + k + pad_a), float("nan"), dtype=tdt, device=DEV)
    big_b = torch.full((k, off_b + n + pad_b), float("nan"), dtype=tdt, device=DEV)
    va, vb = big_a[:, off_a : off_a + k], big_b[:, off_b : off_b + n]
    va.copy_(_dev(a, dtype))
    vb.copy_(_dev(b, dtype))
    guard = torch.full((m + 1, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    g.gemm(va, vb, out=guard[:m, 1 : n + 1], algo=algo)
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[:m, 1 : n + 1], oracle.gemm_c(a, b, oracle.F16 if dtype == "float16" else oracle.BF16), k)
    mask = np.ones_like(host, dtype=bool)
    mask[:m, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


# Extreme aspect ratios: K in the millions for a 1 x 1 or 3 x 5 output,
# one-column and one-row outputs of 10^5, K of 1..9, through every kernel
# that takes the shape, C in a NaN guard band.
@pytest.mark.parametrize("m,n,k", [(1, 1, 4194304), (3, 5, 1000003), (100000, 1, 10), (1, 100000, 7),
                                   (70000, 3, 3), (2, 3, 1), (300000, 8, 64), (17, 100000, 9)])
def test_extreme_shapes(m, n, k):
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    a, b = make_inputs("c2_4096_f16", seed=m + n + k, m=m, n=n, k=k)
    want = oracle.gemm_c(a, b)
    guard = torch.full((m + 2, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    out = guard[1 : m + 1, 1 : n + 1]
    for algo in ["auto", "skinny" if m <= 128 else "tiled", "narrow" if n <= 64 else "generic"]:
        print(f"case extreme {algo} m={m} n={n} k={k}", flush=True)
        out.fill_(float("nan"))
        g.gemm(_dev(a), _dev(b), out=out, algo=algo)
        torch.cuda.synchronize()
        host = guard.cpu().numpy()
        _check(host[1 : m + 1, 1 : n + 1], want, k)
        mask = np.ones_like(host, dtype=bool)
        mask[1 : m + 1, 1 : n + 1] = False
        assert np.all(np.isnan(host[mask]))


# Small outputs over a long K: up to 256 K splits, summed past 16 by the
# split reduce (16 waves per 64 outputs, each a fixed residue class of
# splits, the waves' sums added in order) -- on the streaming kernel (N > 64)
# and the narrow one; integer inputs bit-exact and reproducible.
@pytest.mark.parametrize("m,n,k,algo", [(8, 128, 262144, "skinny"), (100, 200, 131072, "skinny"),
                                        (64, 32, 262144, "auto"), (200, 8, 262144, "narrow"),
                                        (16, 130, 65536, "auto")])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_long_k_many_splits(m, n, k, algo, dtype):
    from hc.gfx950.workloads import make_inputs

    cfg = "c4_skinny_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + n + k, m=m, n=n, k=k)
    print(f"case long K {algo} {dtype} m={m} n={n} k={k}", flush=True)
    _check(_gemm(a, b, algo, dtype), oracle.gemm_c(a, b, _dt(dtype)), k)


@pytest.mark.parametrize("m,n,k,algo", [(8, 128, 262144, "skinny"), (64, 32, 262144, "narrow")])
def test_long_k_many_splits_integer_bit_exact_and_reproducible(m, n, k, algo):
    rng = np.random.default_rng(m * n)
    ai = rng.integers(-2, 3, size=(m, k))
    bi = rng.integers(-2, 3, size=(k, n))
    want = (ai.astype(np.float64) @ bi.astype(np.float64)).astype(np.float32)  # |sums| <= 2^20
    first = _gemm(ai.astype(np.float16), bi.astype(np.float16), algo)
    assert np.array_equal(first, want)
    assert np.array_equal(first.view(np.uint32), _gemm(ai.astype(np.float16), bi.astype(np.float16), algo).view(np.uint32))


# Operands whose byte offsets reach 2^31 (over 2 GiB): the tiled kernel's
# WIDE form rebases its buffer resources per tile (A) and per 32-row K
# step (B).  Inputs are periodic small integers built on the device, so the
# exact product has a closed form that is cheap on the host.
def test_wide_b_operand_over_2gib_bit_exact():
    import hc.gfx950 as g

    m, n, k = 200, 16392, 65536  # B: 2.0 GiB + 1 MiB
    print(f"case wide B m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(5)
    ai = rng.integers(-3, 4, size=(m, k))
    kk = torch.arange(k, device=DEV, dtype=torch.int32).view(k, 1)
    nn = torch.arange(n, device=DEV, dtype=torch.int32).view(1, n)
    b = ((kk + nn) % 5 - 2).to(torch.float16)  # B[k, j] = ((k + j) mod 5) - 2
    a = torch.from_numpy(ai.astype(np.float16)).to(DEV)
    c = g.gemm(a, b)
    torch.cuda.synchronize()
    del b
    # C[i, j] = sum_r (r - 2) * S[i, (r - j) mod 5], S[i, q] = sum of A[i, k] over k = q mod 5
    s = np.stack([ai[:, q::5].sum(axis=1) for q in range(5)], axis=1)
    j = np.arange(n)
    want = sum((r - 2) * s[:, (r - j) % 5] for r in range(5)).astype(np.float32)
    assert np.array_equal(c.cpu().numpy(), want)


def test_wide_b_view_with_nan_padding_columns_bit_exact():
    """B over 2 GiB, N not a multiple of 8, B a view whose 3 padding
    columns hold NaN: the chunk holding column N - 1 loads them, and they
    must reach no stored element of C."""
    import hc.gfx950 as g

    m, n, ld, k = 136, 16389, 16392, 65536
    print(f"case wide B view m={m} n={n} ldb={ld} k={k}", flush=True)
    rng = np.random.default_rng(9)
    ai = rng.integers(-3, 4, size=(m, k))
    kk = torch.arange(k, device=DEV, dtype=torch.int32).view(k, 1)
    nn = torch.arange(ld, device=DEV, dtype=torch.int32).view(1, ld)
    full = ((kk + nn) % 5 - 2).to(torch.float16)
    del kk, nn
    full[:, n:] = float("nan")
    a = torch.from_numpy(ai.astype(np.float16)).to(DEV)
    c = g.gemm(a, full[:, :n])
    torch.cuda.synchronize()
    del full
    s = np.stack([ai[:, q::5].sum(axis=1) for q in range(5)], axis=1)
    j = np.arange(n)
    want = sum((r - 2) * s[:, (r - j) % 5] for r in range(5)).astype(np.float32)
    assert np.array_equal(c.cpu().numpy(), want)


@pytest.mark.parametrize("algo", ["auto", "tiled", "tiled_256x192", "tiled_128x128", "tiled_256x64"])
@pytest.mark.parametrize("m,n,k", [(1000, 3001, 1024), (300, 601, 8192), (4096, 129, 512)])
def test_b_view_with_nan_padding_columns(algo, m, n, k):
    """N not a multiple of 8 with B's rows aligned (no repack): the padding
    columns B loads with column N - 1 hold NaN and must not reach C."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    a, b = make_inputs("c2_4096_f16", seed=n + k, m=m, n=n, k=k)
    ld = (n + 7) // 8 * 8
    full = torch.full((k, ld), float("nan"), dtype=torch.float16, device=DEV)
    full[:, :n] = _dev(b)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    print(f"case B NaN padding {algo} m={m} n={n} k={k}", flush=True)
    g.gemm(_dev(a), full[:, :n], out=out, algo=algo)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), oracle.gemm_c(a, b), k)


# Remainder peeling (algo "auto"): rows or columns just past a multiple of
# 256 run the bulk on the tiled kernel and the remainder on a streaming
# kernel (rows: the M <= 128 one; columns: the N <= 64 one).  At K = 1024
# the library's cost model peels all of these (4 / 15 / 100 rows, 4 / 24 / 48
# columns); at K <= 512 it keeps them whole.
PEEL_SHAPES = [(4100, 4096, 1024, "float16"), (4111, 4096, 1024, "bfloat16"), (4196, 4096, 1024, "float16"),
               (4096, 4100, 1024, "bfloat16"), (4096, 4120, 1024, "float16"), (4096, 4144, 2048, "float16")]


@pytest.mark.parametrize("m,n,k,dtype", PEEL_SHAPES)
def test_remainder_peel_against_oracle_with_guard_band(m, n, k, dtype):
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + 7 * n + k, m=m, n=n, k=k)
    guard = torch.full((m + 2, n + 8), float("nan"), dtype=torch.float32, device=DEV)
    out = guard[1 : m + 1, 4 : n + 4]
    print(f"case peel {dtype} m={m} n={n} k={k}", flush=True)
    g.gemm(_dev(a, dtype), _dev(b, dtype), out=out)
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 4 : n + 4], oracle.gemm_c(a, b, _dt(dtype)), k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 4 : n + 4] = False
    assert np.all(np.isnan(host[mask]))


@pytest.mark.parametrize("m,n,k", [(64, 8191, 8192), (100, 4099, 2048), (17, 30, 4096), (128, 1, 1024)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_streaming_kernel_any_n_with_nan_padding(m, n, k, dtype):
    """17..128 rows, N not a multiple of 8, B's rows padded to a multiple of
    8 with NaN: the chunk holding column N - 1 loads padding that must
    reach no stored element (with and without a K split; the split's
    partials are summed one element per thread when N % 4 != 0)."""
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    cfg = "c2_4096_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=m + n, m=m, n=n, k=k)
    ld = (n + 7) // 8 * 8
    full = torch.full((k, ld), float("nan"), dtype=torch.float16 if dtype == "float16" else torch.bfloat16,
                      device=DEV)
    full[:, :n] = _dev(b, dtype)
    guard = torch.full((m + 2, n + 2), float("nan"), dtype=torch.float32, device=DEV)
    out = guard[1 : m + 1, 1 : n + 1]
    print(f"case stream any N {dtype} m={m} n={n} k={k}", flush=True)
    g.gemm(_dev(a, dtype), full[:, :n], out=out, algo="skinny")
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[1 : m + 1, 1 : n + 1], oracle.gemm_c(a, b, _dt(dtype)), k)
    mask = np.ones_like(host, dtype=bool)
    mask[1 : m + 1, 1 : n + 1] = False
    assert np.all(np.isnan(host[mask]))


@pytest.mark.parametrize("m,n,k", [(4100, 4096, 1024), (4096, 4104, 1024), (4111, 4096, 1025)])
def test_remainder_peel_integer_bit_exact(m, n, k):
    """Exact sums, so the peeled and unpeeled results must agree bit for
    bit; 4111 x 4096 x 1025 has unaligned rows of A and K not a multiple of
    8 (read in place by the bulk and by the 15 remainder rows on the
    streaming kernel)."""
    rng = np.random.default_rng(m + n + k)
    ai = rng.integers(-4, 5, size=(m, k))
    bi = rng.integers(-4, 5, size=(k, n))
    a, b = ai.astype(np.float16), bi.astype(np.float16)
    print(f"case peel integer m={m} n={n} k={k}", flush=True)
    want = (ai.astype(np.float64) @ bi.astype(np.float64)).astype(np.float32)  # exact: |sums| <= 16400
    assert np.array_equal(_gemm(a, b), want)
    assert np.array_equal(_gemm(a, b, "tiled"), want)


def test_wide_a_operand_over_2gib_bit_exact():
    import hc.gfx950 as g

    m, n, k = 65600, 264, 16384  # A: 2.0 GiB + 3 MiB
    print(f"case wide A m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(6)
    bi = rng.integers(-3, 4, size=(k, n))
    ii = torch.arange(m, device=DEV, dtype=torch.int32).view(m, 1)
    kk = torch.arange(k, device=DEV, dtype=torch.int32).view(1, k)
    a = ((ii + 2 * kk) % 7 - 3).to(torch.float16)  # A[i, k] = ((i + 2k) mod 7) - 3
    b = torch.from_numpy(bi.astype(np.float16)).to(DEV)
    c = g.gemm(a, b)
    torch.cuda.synchronize()
    del a
    # (i + 2k) mod 7 = r  <=>  k = 4 (r - i) mod 7, so C[i] depends on i mod 7 only
    t = np.stack([bi[q::7].sum(axis=0) for q in range(7)], axis=0)
    rows = np.stack([sum((r - 3) * t[(4 * (r - i)) % 7] for r in range(7)) for i in range(7)]).astype(np.float32)
    got = c.cpu().numpy()
    for i in range(7):
        assert np.array_equal(got[i::7], np.broadcast_to(rows[i], got[i::7].shape)), f"rows = {i} mod 7"


@pytest.mark.parametrize("m,n,k,dtype", [(128, 128, 128, "float16"), (4095, 3001, 1027, "float16"),
                                         (16, 8192, 8192, "bfloat16"), (3000, 13, 4096, "float16")])
def test_compiled_binding_matches_the_ctypes_path(m, n, k, dtype):
    """hc.gfx950.gemm on device tensors goes through the compiled binding
    (_hcg_torch); the ctypes call of the same entry point gives the same
    bits, and a case the binding leaves to Python (a transposed view of B)
    still runs through the general path."""
    import hc.gfx950 as g
    from hc.gfx950 import _hcg_torch, _native
    from hc.gfx950.workloads import make_inputs

    print(f"case compiled binding {dtype} m={m} n={n} k={k}", flush=True)
    a, b = make_inputs("c2_4096_f16" if dtype == "float16" else "c3_8192_bf16", seed=m + n, m=m, n=n, k=k)
    ta, tb = _dev(a, dtype), _dev(b, dtype)
    via_binding = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    assert _hcg_torch.gemm(ta, tb, via_binding, _native.HCG_ALGO_AUTO) == 0
    via_ctypes = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    lib = _native.load()
    rc = lib.hcg_gemm_algo(_native.HCG_ALGO_AUTO, _native.HCG_F16 if dtype == "float16" else _native.HCG_BF16,
                           ta.data_ptr(), k, tb.data_ptr(), n, via_ctypes.data_ptr(), n, m, n, k,
                           torch.cuda.current_stream().cuda_stream)
    _native.check(lib, rc, "hcg_gemm_algo")
    via_wrapper = g.gemm(ta, tb, out=torch.empty((m, n), dtype=torch.float32, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(via_binding, via_ctypes) and torch.equal(via_wrapper, via_ctypes)
    _check(via_binding.cpu().numpy(), oracle.gemm_c(a, b, _dt(dtype)), k)
    tbt = tb.t().contiguous().t()  # column-major B: the binding declines, the wrapper copies it
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    assert _hcg_torch.gemm(ta, tbt, out, _native.HCG_ALGO_AUTO) == -1
    g.gemm(ta, tbt, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, via_ctypes)


# Edge tiles whose C rows are 16-byte aligned (ldc a multiple of 4, N a
# multiple of 4) store whole chunks non-temporally and skip rows past M and
# chunks past N; C here is a view into a NaN-filled buffer with extra columns
# and rows, so a chunk stored past N or a row past M would show.
_ALIGNED_C_CASES = [
    ("auto", 300, 520, 200), ("auto", 4095, 3008, 96), ("auto", 1000, 1000, 300), ("tiled_256x256", 257, 260, 64),
    ("tiled_256x192", 255, 196, 40), ("tiled_128x256", 129, 260, 33), ("tiled_128x128", 130, 132, 70),
    ("tiled_256x64", 300, 68, 50), ("tiled", 520, 4, 2000), ("auto", 17, 1028, 257),
]


@pytest.mark.parametrize("algo,m,n,k", _ALIGNED_C_CASES)
def test_aligned_c_rows_edge_tiles_write_only_inside(algo, m, n, k):
    import hc.gfx950 as g
    from hc.gfx950.workloads import make_inputs

    assert n % 4 == 0
    print(f"case aligned C {algo} {m}x{n}x{k}", flush=True)
    a, b = make_inputs("c2_4096_f16", seed=m + n + k, m=m, n=n, k=k)
    ldc = n + 8  # 16-byte aligned rows with 8 guard columns
    guard = torch.full((m + 3, ldc), float("nan"), dtype=torch.float32, device=DEV)
    g.gemm(_dev(a), _dev(b), out=guard[:m, :n], algo=algo)
    torch.cuda.synchronize()
    host = guard.cpu().numpy()
    _check(host[:m, :n], oracle.gemm_c(a, b), k)
    mask = np.ones_like(host, dtype=bool)
    mask[:m, :n] = False
    assert np.all(np.isnan(host[mask]))
