"""Synthetic GEMM workloads (seeded inputs) for the benchmark, the smoke test
and the parity tests.

Each configuration draws from one ``np.random.default_rng(seed)``, A first and
then B, in float64, then casts: ``astype(np.float16)`` for fp16 (round to
nearest even), or float64 -> float32 -> bfloat16 (round to nearest even on
the float32 bits) for bf16.  This mirrors the reference's input helper
(examples/amdgpu_gfx11_wmma_matmul.py:351-361: one generator, A then B,
uniform(-1, 1), cast to float16).

bf16 operands are returned as uint16 bit patterns (numpy has no bfloat16);
``to_torch`` turns them into ``torch.bfloat16`` device tensors.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class GemmConfig:
    name: str
    m: int
    n: int
    k: int
    dtype: str  # "float16" | "bfloat16"
    a_dist: tuple[str, float]  # ("uniform", half-width) | ("normal", sigma)
    b_dist: tuple[str, float]
    description: str

    @property
    def flops(self) -> int:
        return 2 * self.m * self.n * self.k

    @property
    def algorithmic_bytes(self) -> int:
        """2-byte A and B read once, float32 C written once (never read)."""
        return 2 * self.m * self.k + 2 * self.k * self.n + 4 * self.m * self.n


# BASELINE.json "configs", in order.
CONFIGS: dict[str, GemmConfig] = {
    "c1_128_f16": GemmConfig(
        "c1_128_f16", 128, 128, 128, "float16", ("normal", 1.0), ("normal", 1.0),
        "fp16 GEMM M=N=K=128, A,B ~ N(0,1), the reference example's CPU-runnable case",
    ),
    "c2_4096_f16": GemmConfig(
        "c2_4096_f16", 4096, 4096, 4096, "float16", ("uniform", 1.0), ("uniform", 1.0),
        "fp16 GEMM M=N=K=4096, A,B ~ U[-1,1] (square, compute-bound)",
    ),
    "c3_8192_bf16": GemmConfig(
        "c3_8192_bf16", 8192, 8192, 8192, "bfloat16", ("normal", 0.02), ("normal", 0.02),
        "bf16 GEMM M=N=K=8192, A,B ~ N(0,0.02) (large, compute-bound)",
    ),
    "c4_skinny_f16": GemmConfig(
        "c4_skinny_f16", 16, 8192, 8192, "float16", ("normal", 1.0), ("normal", 0.02),
        "fp16 GEMM M=16 N=8192 K=8192, A ~ N(0,1), B ~ N(0,0.02) (decode-style, HBM-bound)",
    ),
    "c5_ragged_f16": GemmConfig(
        "c5_ragged_f16", 4095, 3001, 1027, "float16", ("uniform", 1.0), ("uniform", 1.0),
        "fp16 GEMM M=4095 N=3001 K=1027, A,B ~ U[-1,1] (masked tails in M, N and K)",
    ),
}


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (finite inputs).

    In uint32: a finite float32's bits are at most 0xFF7FFFFF, so adding at
    most 0x8000 cannot wrap."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + (0x7FFF + ((u >> 16) & 1))) >> 16).astype(np.uint16)


def _draw(rng: np.random.Generator, dist: tuple[str, float], shape: tuple[int, int]) -> np.ndarray:
    kind, scale = dist
    if kind == "uniform":
        return rng.uniform(-scale, scale, size=shape)
    if kind == "normal":
        return rng.normal(0.0, scale, size=shape)
    raise ValueError(f"unknown distribution {kind}")


def _cast(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float16":
        return x.astype(np.float16)
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x.astype(np.float32))
    raise ValueError(f"unknown dtype {dtype}")


def make_inputs(
    cfg: GemmConfig | str,
    seed: int = 0,
    *,
    m: int | None = None,
    n: int | None = None,
    k: int | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """Seeded (A, B) for a configuration; m/n/k override the extents."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    mm, nn, kk = m or cfg.m, n or cfg.n, k or cfg.k
    rng = np.random.default_rng(seed)
    a = _cast(_draw(rng, cfg.a_dist, (mm, kk)), cfg.dtype)
    b = _cast(_draw(rng, cfg.b_dist, (kk, nn)), cfg.dtype)
    return a, b


def make_demo_inputs(*, m: int = 32, n: int = 32, k: int = 32, seed: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """The reference example's inputs: one generator, A then B, U[-1,1] -> fp16
    (examples/amdgpu_gfx11_wmma_matmul.py:351-361)."""
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1.0, 1.0, size=(m, k)).astype(np.float16)
    b = rng.uniform(-1.0, 1.0, size=(k, n)).astype(np.float16)
    return a, b


def to_torch(x: np.ndarray, dtype: str, device) -> "object":
    """Host operand -> torch device tensor (bf16 from its uint16 bits)."""
    import torch

    if dtype == "bfloat16":
        t = torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to(device)
