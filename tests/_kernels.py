"""Kernels with the reference example's launch signature, for the launch
surface tests.

``tiled_gfx11_wmma_matmul`` has the name, buffer annotations and geometry of
the reference's kernel (examples/amdgpu_gfx11_wmma_matmul.py:301-311:
work_shape (ceil_div(M, 16) * 32, ceil_div(N, 16)), group_shape (32, 1),
subgroup_size 32, a: Buffer[M, K, f16], b: Buffer[K, N, f16],
c: Buffer[M, N, f32]); its body is a stand-in, since the gfx950 target lowers
the whole kernel and never executes the body.
"""

from __future__ import annotations

import numpy as np

from hc import Buffer, kernel, sym
from hc.symbols import ceil_div

M = sym.M
N = sym.N
K = sym.K


@kernel(work_shape=(ceil_div(M, 16) * 32, ceil_div(N, 16)), group_shape=(32, 1), subgroup_size=32)
def tiled_gfx11_wmma_matmul(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    raise AssertionError("lowered as a whole; the body never runs")


@kernel(work_shape=(ceil_div(M, 16) * 32, ceil_div(N, 16)), group_shape=(32, 1), subgroup_size=32)
def some_other_kernel(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    raise AssertionError("never runs")


@kernel(work_shape=(ceil_div(M, 16) * 32,), group_shape=(32,), subgroup_size=32)
def tiled_gfx950_mfma_matmul(group, x: Buffer[M, np.float16]) -> None:
    """Known GEMM name but not a contraction signature."""
    raise AssertionError("never runs")
