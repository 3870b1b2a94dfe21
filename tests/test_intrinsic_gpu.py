"""The gfx950 matrix-core intrinsics' lane contract, on the GPU.

For ``mfma_gfx950`` (32x32x16) and ``mfma16_gfx950`` (16x16x32), in float16
and bfloat16: the op their ``amdgpu-gfx950`` lowering creates is executed for
one wave (``hc.gfx950.intrinsics.run_wave`` -> ``hcg_mfma_step``) and each of
the 64 lanes' accumulators is compared with what the intrinsic's fallback
body computes for that lane (``fallback_wave``), on the same tiles, masks and
input accumulators:

* small integers (every summation order exact): bit-exact, and equal to the
  exact integer result placed by the stated lane layout; inactive entries
  hold NaN, so one that leaked into a sum would show;
* seeded normal values: both within the float32 summation bound
  gamma_{k+1} * (|acc| + |A| |B|) of the exact (float64) result, where
  gamma_n = n u / (1 - n u), u = 2^-24 (the hardware adds in another order
  than the fallback's ascending fold, so only the bound is shared).

The DSL kernel written on 16x16x32 fragments also runs through the unchanged
launch call against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

import hc_oracle as oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _cases():
    from hc.gfx950 import kernels as k

    return {
        "32x32x16": (k.mfma_gfx950, 32, 16, k.lane_acc_rows, k.lane_column),
        "16x16x32": (k.mfma16_gfx950, 16, 32, k.lane16_acc_rows, k.lane16_column),
    }


def _operands(mn: int, k: int, dtype: str, seed: int, ints: bool):
    from hc.gfx950.workloads import f32_to_bf16_bits

    rng = np.random.default_rng(seed)
    if ints:
        a = rng.integers(-8, 9, (mn, k)).astype(np.float32)
        b = rng.integers(-8, 9, (k, mn)).astype(np.float32)
        acc = rng.integers(-64, 65, (64, mn * mn // 64)).astype(np.float32)
    else:
        a = rng.normal(0, 1, (mn, k)).astype(np.float32)
        b = rng.normal(0, 1, (k, mn)).astype(np.float32)
        acc = rng.normal(0, 4, (64, mn * mn // 64)).astype(np.float32)
    am = rng.random(a.shape) < 0.8
    bm = rng.random(b.shape) < 0.8
    if dtype == "float16":
        a, b = a.astype(np.float16), b.astype(np.float16)
        nan = np.float16(np.nan)
        a_val = np.where(am, a, nan)
        b_val = np.where(bm, b, nan)
        a0 = np.where(am, a, np.float16(0)).astype(np.float64)
        b0 = np.where(bm, b, np.float16(0)).astype(np.float64)
    else:
        a, b = f32_to_bf16_bits(a), f32_to_bf16_bits(b)
        nan_bits = np.uint16(0x7FC0)
        a_val = np.where(am, a, nan_bits)
        b_val = np.where(bm, b, nan_bits)
        a0 = oracle.bf16_bits_to_f32(np.where(am, a, np.uint16(0))).astype(np.float64)
        b0 = oracle.bf16_bits_to_f32(np.where(bm, b, np.uint16(0))).astype(np.float64)
    return a_val, b_val, am, bm, acc, a0, b0


def _per_lane(c: np.ndarray, rows_of, col_of, regs: int) -> np.ndarray:
    """The (64, regs) lane-major view of an output tile."""
    out = np.empty((64, regs), dtype=c.dtype)
    for lane in range(64):
        for r, row in enumerate(rows_of(lane)):
            out[lane, r] = c[row, col_of(lane)]
    return out


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape", ["32x32x16", "16x16x32"])
def test_every_lane_matches_the_fallback_on_integers(shape, dtype):
    from hc.gfx950 import intrinsics

    fn, mn, k, rows_of, col_of = _cases()[shape]
    regs = mn * mn // 64
    print(f"case {fn.__name__} {dtype} integers", flush=True)
    for seed in range(3):
        a, b, am, bm, acc, a0, b0 = _operands(mn, k, dtype, seed, ints=True)
        dev = intrinsics.run_wave(fn, a, b, acc, dtype=dtype, a_mask=am, b_mask=bm, wave_size=64, arch="gfx950")
        ref = intrinsics.fallback_wave(fn, a, b, acc, dtype=dtype, a_mask=am, b_mask=bm, wave_size=64,
                                       arch="gfx950")
        assert np.array_equal(dev, ref), (seed, np.argwhere(dev != ref)[:5])
        exact = acc.astype(np.float64) + _per_lane(a0 @ b0, rows_of, col_of, regs)
        assert np.array_equal(dev.astype(np.float64), exact)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape", ["32x32x16", "16x16x32"])
def test_every_lane_within_the_float32_bound_on_normals(shape, dtype):
    from hc.gfx950 import intrinsics

    fn, mn, k, rows_of, col_of = _cases()[shape]
    regs = mn * mn // 64
    n = k + 1  # k products and the input accumulator
    gamma = n * 2.0**-24 / (1 - n * 2.0**-24)
    print(f"case {fn.__name__} {dtype} normals", flush=True)
    for seed in range(3):
        a, b, am, bm, acc, a0, b0 = _operands(mn, k, dtype, 100 + seed, ints=False)
        dev = intrinsics.run_wave(fn, a, b, acc, dtype=dtype, a_mask=am, b_mask=bm, wave_size=64, arch="gfx950")
        ref = intrinsics.fallback_wave(fn, a, b, acc, dtype=dtype, a_mask=am, b_mask=bm, wave_size=64,
                                       arch="gfx950")
        acc64 = acc.astype(np.float64)
        exact = acc64 + _per_lane(a0 @ b0, rows_of, col_of, regs)
        bound = gamma * (np.abs(acc64) + _per_lane(np.abs(a0) @ np.abs(b0), rows_of, col_of, regs))
        assert np.all(np.abs(ref - exact) <= bound), "fallback outside the sequential-fold bound"
        worst = np.max(np.abs(dev - exact) / np.maximum(bound, 1e-300))
        assert worst <= 1.0, f"device lane outside the float32 bound (worst {worst:.3f} of the bound)"
        assert not np.array_equal(dev, np.full_like(dev, np.nan))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_the_16x16x32_dsl_kernel_through_the_launch_surface(dtype):
    import hc
    from hc.gfx950 import kernels
    from hc.gfx950.workloads import make_inputs

    fn = kernels.tiled_gfx950_mfma16_matmul if dtype == "float16" else kernels.tiled_gfx950_mfma16_matmul_bf16
    cfg = "c5_ragged_f16" if dtype == "float16" else "c3_8192_bf16"
    a, b = make_inputs(cfg, seed=3, m=300, n=260, k=97)
    print(f"case {fn.__name__} 300x260x97", flush=True)
    if dtype == "float16":
        c = np.full((300, 260), np.nan, dtype=np.float32)
        hc.simulator.launch(fn, a, b, c)
    else:
        from hc.gfx950.workloads import to_torch

        dev = torch.device("cuda", 0)
        ta, tb = to_torch(a, dtype, dev), to_torch(b, dtype, dev)
        tc = torch.full((300, 260), float("nan"), dtype=torch.float32, device=dev)
        hc.simulator.launch(fn, ta, tb, tc)
        torch.cuda.synchronize()
        c = tc.cpu().numpy()
    code = oracle.F16 if dtype == "float16" else oracle.BF16
    rep = oracle.parity_check(c, oracle.gemm_sequential(a, b, code), 97)
    assert rep.ok, str(rep)
