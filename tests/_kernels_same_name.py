"""A kernel with the reference kernel's name, geometry and signature whose
body is not the GEMM: its accumulate step doubles every product.  The gfx950
target must reject it (dispatch never goes by name)."""

from __future__ import annotations

import numpy as np

from hc import Buffer, WorkGroup, WorkItem, kernel, sym, vector_type

from ._kernels import (GEOMETRY, ROWS_PER_LANE, TILE, _lower_wmma, a_fragment, b_fragment, lane_rows, store_acc,
                       tile_origin, zero_acc)

M = sym.M
N = sym.N
K = sym.K


@kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"wave_size", "arch"},
                  result_types=(vector_type((ROWS_PER_LANE,), np.float32),))
def wmma_doubled(group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    _ = (a_frag, b_frag, arch)
    a_tile = a_tile.with_inactive(value=np.float16(0))
    b_tile = b_tile.with_inactive(value=np.float16(0))
    rows = lane_rows(lane, wave_size)
    out = np.empty((len(rows),), dtype=np.float32)
    for i, row in enumerate(rows):
        s = np.float32(acc_frag[i])
        for kk in range(TILE):
            s += np.float32(2) * np.float32(a_tile[row, kk]) * np.float32(b_tile[kk, lane % TILE])
        out[i] = s
    return group.vload(out, shape=(len(rows),))


@wmma_doubled.lower(target="amdgpu-gfx11")
def _lower(ctx, group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    # A well-formed WMMA lowering: only the fallback's doubled product is wrong.
    return _lower_wmma(ctx, group, a_tile, b_tile, a_frag, b_frag, acc_frag, lane=lane, wave_size=wave_size,
                       arch=arch)


@kernel.func(scope=WorkGroup)
def doubled_step(group, a_tile, b_tile, acc):
    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        return wmma_doubled(group, a_tile, b_tile, a_fragment(wi, a_tile), b_fragment(wi, b_tile), acc[:, lane, 0],
                            lane=lane, wave_size=32, arch="gfx11")

    return lanes()


@kernel(**GEOMETRY)
def tiled_gfx11_wmma_matmul(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = tile_origin(group.group_id[0], group.group_id[1])
    acc = zero_acc(group)
    for k0 in range(0, a.shape[1], TILE):
        a_tile = group.load(a[row0 : row0 + TILE, k0 : k0 + TILE], shape=(TILE, TILE))
        b_tile = group.load(b[k0 : k0 + TILE, col0 : col0 + TILE], shape=(TILE, TILE))
        acc = doubled_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)

