"""Pins for the CPU oracle (oracle/hc_oracle.py, oracle/hc_oracle.c).

Each check is independent of the oracle's own formula: a scalar np.float32
triple loop, the reference test's own blocked-sum criterion, exact integer
arithmetic, the float64 product with the Higham error bound, library
conversions, and planted mistakes that must be caught.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest

import hc_oracle as oracle
from hc.gfx950.workloads import CONFIGS, make_demo_inputs, make_inputs

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not oracle.available():
        import importlib.util

        spec = importlib.util.spec_from_file_location(
            "oracle_build", os.path.join(os.path.dirname(oracle.__file__), "build.py")
        )
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()


def _rand(shape, dtype, rng, scale=1.0):
    x = rng.uniform(-scale, scale, size=shape)
    if dtype == oracle.F16:
        return x.astype(np.float16)
    return oracle.f32_to_bf16_bits(x.astype(np.float32))


# -- conversions ------------------------------------------------------------


def test_f16_conversion_matches_numpy_for_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.to_float_c(bits, oracle.F16)
    want = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    x = np.concatenate(
        [
            rng.normal(0, 1, 20000).astype(np.float32),
            rng.normal(0, 0.02, 20000).astype(np.float32),
            # exact ties: low 16 bits 0x8000, even and odd kept parts
            (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x00008000], dtype=np.uint32)).view(np.float32),
            # the largest finite magnitudes (the rounding add must not wrap;
            # 0x7F7F8000 and up round to infinity, as torch does), subnormals
            (np.array([0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F7FFF, 0xFF7F8000, 0x00000001, 0x807FFFFF],
                      dtype=np.uint32)).view(np.float32),
        ]
    )
    ours = oracle.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    from hc.gfx950.workloads import f32_to_bf16_bits

    assert np.array_equal(f32_to_bf16_bits(x), theirs)


def test_bf16_tie_cases_by_hand():
    # 1 + 2^-8 is halfway between bf16 1.0 and 1 + 2^-7 -> even (1.0).
    x = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8)], dtype=np.float32)
    assert list(oracle.f32_to_bf16_bits(x)) == [0x3F80, 0x3F82, 0xBF80]
    assert np.array_equal(oracle.bf16_bits_to_f32(np.array([0x3F80, 0xC000], dtype=np.uint16)),
                          np.array([1.0, -2.0], dtype=np.float32))


# -- the sequential fold ------------------------------------------------------


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.BF16])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 7), (8, 8, 16), (17, 19, 18), (4, 6, 33)])
def test_sequential_equals_scalar_triple_loop(m, n, k, dtype):
    rng = np.random.default_rng(m * 100 + n * 10 + k)
    a, b = _rand((m, k), dtype, rng), _rand((k, n), dtype, rng)
    seq = oracle.gemm_sequential(a, b, dtype)
    brute = oracle.gemm_bruteforce(a, b, dtype)
    assert np.array_equal(seq.view(np.uint32), brute.view(np.uint32))


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.BF16])
@pytest.mark.parametrize("m,n,k", [(17, 19, 18), (64, 33, 100), (5, 300, 257), (130, 70, 1)])
def test_c_oracle_bit_equal_to_numpy(m, n, k, dtype):
    rng = np.random.default_rng(7 + m + n + k)
    a, b = _rand((m, k), dtype, rng), _rand((k, n), dtype, rng, scale=3.0)
    seq = oracle.gemm_sequential(a, b, dtype)
    c = oracle.gemm_c(a, b, dtype, threads=3)
    assert np.array_equal(seq.view(np.uint32), c.view(np.uint32))
    rows = np.array([m - 1, 0, m // 2], dtype=np.int64)
    cr = oracle.gemm_c_rows(a, b, rows, dtype, threads=2)
    assert np.array_equal(cr.view(np.uint32), seq[rows].view(np.uint32))


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.BF16])
def test_integer_known_answer_is_exact(dtype):
    # |values| <= 8 and K <= 512 keep every partial sum an integer below 2^24,
    # so every summation order is exact: the result must equal int64 A@B.
    rng = np.random.default_rng(5)
    ai = rng.integers(-8, 9, size=(37, 512))
    bi = rng.integers(-8, 9, size=(512, 29))
    if dtype == oracle.F16:
        a, b = ai.astype(np.float16), bi.astype(np.float16)
    else:
        a, b = oracle.f32_to_bf16_bits(ai.astype(np.float32)), oracle.f32_to_bf16_bits(bi.astype(np.float32))
    want = (ai @ bi).astype(np.float32)
    assert np.array_equal(oracle.gemm_sequential(a, b, dtype), want)
    assert np.array_equal(oracle.gemm_c(a, b, dtype), want)


def test_identity_and_permutation_select_rows_exactly():
    rng = np.random.default_rng(3)
    b = rng.uniform(-1, 1, size=(24, 40)).astype(np.float16)
    perm = rng.permutation(24)
    p = np.zeros((24, 24), dtype=np.float16)
    p[np.arange(24), perm] = 1
    assert np.array_equal(oracle.gemm_c(p, b), b[perm].astype(np.float32))


def test_zero_k_and_empty_shapes():
    a = np.zeros((3, 0), dtype=np.float16)
    b = np.zeros((0, 4), dtype=np.float16)
    assert np.array_equal(oracle.gemm_sequential(a, b), np.zeros((3, 4), np.float32))
    assert np.array_equal(oracle.gemm_c(a, b), np.zeros((3, 4), np.float32))
    assert oracle.gemm_c(np.zeros((0, 5), np.float16), np.zeros((5, 2), np.float16)).shape == (0, 2)


@pytest.mark.parametrize("name,m,n,k,seed", [
    ("ref_16x16x16_seed7", 16, 16, 16, 7),
    ("ref_32x32x32_seed7", 32, 32, 32, 7),
    ("ref_17x19x18_seed7", 17, 19, 18, 7),
    ("ref_32x32x32_seed0", 32, 32, 32, 0),
])
def test_reference_test_shapes_within_reference_tolerance(name, m, n, k, seed):
    # The reference's own check: simulator vs blocked fp32 sum, atol 2e-6
    # (tests/test_examples.py:23-33; examples/amdgpu_gfx11_wmma_matmul.py:438-441).
    a, b = make_demo_inputs(m=m, n=n, k=k, seed=seed)
    seq = oracle.gemm_sequential(a, b)
    np.testing.assert_allclose(seq, oracle.gemm_blocked(a, b), rtol=0.0, atol=2e-6)
    # ... and the committed fixture holds exactly these inputs and this result.
    fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    assert np.array_equal(fx["a"], a) and np.array_equal(fx["b"], b)
    assert np.array_equal(fx["c_seq"].view(np.uint32), seq.view(np.uint32))


def test_c1_fixture_matches_oracle():
    fx = np.load(os.path.join(GOLDEN, "c1_128_f16_seed0.npz"))
    a, b = make_inputs("c1_128_f16", seed=0)
    assert np.array_equal(fx["a"], a) and np.array_equal(fx["b"], b)
    assert np.array_equal(fx["c_seq"].view(np.uint32), oracle.gemm_c(a, b).view(np.uint32))


def _gamma(k):
    u = 2.0**-24
    return k * u / (1 - k * u)


@pytest.mark.parametrize("dtype,m,n,k", [(oracle.F16, 40, 50, 1027), (oracle.BF16, 30, 20, 4096)])
def test_error_within_higham_bound_of_float64_product(dtype, m, n, k):
    rng = np.random.default_rng(k)
    a, b = _rand((m, k), dtype, rng), _rand((k, n), dtype, rng)
    a64 = oracle.operand_to_f32(a, dtype).astype(np.float64)
    b64 = oracle.operand_to_f32(b, dtype).astype(np.float64)
    exact = a64 @ b64  # products exact; fp64 sum error is far below the bound
    bound = _gamma(k) * (np.abs(a64) @ np.abs(b64))
    got = oracle.gemm_c(a, b, dtype).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bound)


# -- planted mistakes must be caught --------------------------------------------


def _dropped_last_term(a, b):
    return oracle.gemm_sequential(a[:, :-1], b[:-1, :])


def _sign_flipped_term(a, b):
    c = oracle.gemm_sequential(a, b)
    return c - 2 * np.outer(a[:, 3].astype(np.float32), b[3, :].astype(np.float32))


def _transposed_b(a, b):
    return oracle.gemm_sequential(a, np.ascontiguousarray(b.T))


def _started_from_one(a, b):
    return oracle.gemm_sequential(a, b) + np.float32(1.0)


@pytest.mark.parametrize("mutant", [_dropped_last_term, _sign_flipped_term, _transposed_b, _started_from_one])
def test_planted_mistakes_fail_the_checks(mutant):
    rng = np.random.default_rng(21)
    ai = rng.integers(-4, 5, size=(48, 48))
    bi = rng.integers(-4, 5, size=(48, 48))
    a, b = ai.astype(np.float16), bi.astype(np.float16)
    want = (ai @ bi).astype(np.float32)
    bad = mutant(a, b)
    assert not np.array_equal(bad, want)  # integer known-answer test
    assert not oracle.parity_check(bad, want, 48).ok  # the GPU parity criterion


# -- the parity criterion itself -----------------------------------------------


def test_parity_check_thresholds():
    assert oracle.max_abs_bound(1024) == pytest.approx(2e-2)
    assert oracle.max_abs_bound(4096) == pytest.approx(4e-2)
    assert oracle.max_abs_bound(1027) == pytest.approx(2e-2 * math.sqrt(1027 / 1024))
    want = np.ones((4, 4), np.float32)
    assert oracle.parity_check(want, want, 16).ok
    off = want.copy()
    off[0, 0] += 0.5
    assert not oracle.parity_check(off, want, 1024).ok  # max-abs violation
    nan = want.copy()
    nan[1, 1] = np.nan
    assert not oracle.parity_check(nan, want, 1024).ok


def test_generators_are_seeded_and_follow_the_reference_recipe():
    a1, b1 = make_demo_inputs(m=5, n=6, k=7, seed=7)
    rng = np.random.default_rng(7)
    assert np.array_equal(a1, rng.uniform(-1, 1, size=(5, 7)).astype(np.float16))
    assert np.array_equal(b1, rng.uniform(-1, 1, size=(7, 6)).astype(np.float16))
    for name in CONFIGS:
        x1, y1 = make_inputs(name, seed=3, m=8, n=8, k=8)
        x2, y2 = make_inputs(name, seed=3, m=8, n=8, k=8)
        assert np.array_equal(x1, x2) and np.array_equal(y1, y2)


@pytest.mark.parametrize("m,n,k", [(16, 16, 16), (17, 19, 18), (33, 20, 40)])
def test_lane_structured_simulation_is_the_same_fold(m, n, k):
    a, b = make_demo_inputs(m=m, n=n, k=k, seed=5)
    got = oracle.simulate_lane_structure(a, b)
    assert np.array_equal(got.view(np.uint32), oracle.gemm_bruteforce(a, b).view(np.uint32))


# -- masked tile access (hc/simulator.py:1304-1357, 1416-1458) ---------------------


def _tile_load_elementwise(src, origins, shape, mask, fill):
    """Per-element restatement: element (t, r, c) is active iff its source
    coordinate lies inside src (and the mask allows it)."""
    th, tw = shape
    n = len(origins)
    out = np.full((n, th, tw), fill, dtype=src.dtype)
    act = np.zeros((n, th, tw), dtype=bool)
    for t, (r0, c0) in enumerate(origins):
        for r in range(th):
            for c in range(tw):
                i, j = r0 + r, c0 + c
                if 0 <= i < src.shape[0] and 0 <= j < src.shape[1] and (mask is None or mask[t, r, c]):
                    out[t, r, c] = src[i, j]
                    act[t, r, c] = True
    return out, act


def _copy_loaded_value_reference_form(src, r0, c0, th, tw):
    """The reference's own formulation for non-negative origins: slice the
    source (numpy clips at the edges), copy the overlap into a zero tile,
    mark it active (hc/simulator.py:1338-1357)."""
    view = src[r0 : r0 + th, c0 : c0 + tw]
    data = np.zeros((th, tw), dtype=src.dtype)
    act = np.zeros((th, tw), dtype=bool)
    data[: view.shape[0], : view.shape[1]] = view
    act[: view.shape[0], : view.shape[1]] = True
    return data, act


@pytest.mark.parametrize("dtype", [np.float16, np.float32, np.int64])
def test_tile_load_oracle_matches_elementwise_and_reference_slicing(dtype):
    rng = np.random.default_rng(5)
    src = rng.integers(-1000, 1000, size=(23, 31)).astype(dtype)
    origins = np.array([[0, 0], [7, 9], [20, 28], [22, 30], [23, 0], [0, 31], [-3, -2], [-1, 25], [40, 40]])
    mask = rng.random((len(origins), 5, 6)) < 0.7
    for m in (None, mask):
        got, act = oracle.tile_load(src, origins, (5, 6), mask=m, fill=7)
        want, wact = _tile_load_elementwise(src, origins, (5, 6), m, 7)
        assert np.array_equal(got, want) and np.array_equal(act, wact)
    got, act = oracle.tile_load(src, origins, (5, 6), fill=0)
    for t, (r0, c0) in enumerate(origins):
        if r0 >= 0 and c0 >= 0:
            d, a = _copy_loaded_value_reference_form(src, r0, c0, 5, 6)
            assert np.array_equal(got[t], d) and np.array_equal(act[t], a)


def test_tile_load_oracle_known_answers():
    src = np.arange(20, dtype=np.float32).reshape(4, 5)
    got, act = oracle.tile_load(src, [[2, 3], [-1, -1], [10, 0], [1, 1]], (3, 3), fill=-1)
    assert got[0].tolist() == [[13, 14, -1], [18, 19, -1], [-1, -1, -1]]
    assert act[0].sum() == 4
    assert got[1].tolist() == [[-1, -1, -1], [-1, 0, 1], [-1, 5, 6]]
    assert not act[2].any() and np.all(got[2] == -1)
    assert np.array_equal(got[3], src[1:4, 1:4]) and act[3].all()  # interior tile = plain slice
    # with_inactive keeps active payloads, replaces inactive ones (doc/langref.md:577-580)
    m = np.zeros((4, 3, 3), dtype=bool)
    m[3, 1, 1] = True
    got, act = oracle.tile_load(src, [[2, 3], [-1, -1], [10, 0], [1, 1]], (3, 3), mask=m, fill=9)
    assert act.sum() == 1 and got[3, 1, 1] == src[2, 2] and np.sum(got == 9) == 4 * 9 - 1


def test_tile_store_oracle_matches_elementwise_and_leaves_the_rest():
    rng = np.random.default_rng(6)
    origins = np.array([[0, 0], [5, 11], [18, 27], [-2, 3], [30, 30], [10, -4]])
    tiles = rng.integers(1, 100, size=(len(origins), 6, 7)).astype(np.float32)
    mask = rng.random(tiles.shape) < 0.6
    for m in (None, mask):
        dst = np.full((21, 30), np.nan, dtype=np.float32)
        oracle.tile_store(dst, origins, tiles, mask=m)
        want = np.full((21, 30), np.nan, dtype=np.float32)
        for t, (r0, c0) in enumerate(origins):
            for r in range(6):
                for c in range(7):
                    i, j = r0 + r, c0 + c
                    if 0 <= i < 21 and 0 <= j < 30 and (m is None or m[t, r, c]):
                        want[i, j] = tiles[t, r, c]
        assert np.array_equal(np.isnan(dst), np.isnan(want))
        assert np.array_equal(dst[~np.isnan(dst)], want[~np.isnan(want)])


def test_tile_store_then_load_round_trips_inside_the_view():
    rng = np.random.default_rng(7)
    dst = np.zeros((17, 19), dtype=np.float16)
    origins = np.array([[0, 0], [8, 10], [12, 14]])
    tiles = rng.standard_normal((3, 8, 10)).astype(np.float16)
    oracle.tile_store(dst, origins[:2], tiles[:2])
    back, act = oracle.tile_load(dst, origins[:2], (8, 10))
    assert np.array_equal(back[act], tiles[:2][act])
    assert act[0].all() and act[1].sum() == min(8, 17 - 8) * min(10, 19 - 10)
