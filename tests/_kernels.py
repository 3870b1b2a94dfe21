"""The reference example's kernel, restated in the hc DSL, for the launch
surface tests.

The reference module cannot be imported here (Python >= 3.12 and a missing
native dependency), so this module states the same DSL program:
examples/amdgpu_gfx11_wmma_matmul.py's wave32 WMMA contract -- intrinsic
``wmma_gfx11`` with a fallback body (:144-190), a verify hook (:193-197) and
an ``amdgpu-gfx11`` lowering (:200-228), the lane helpers (:231-298) -- and
the kernel ``tiled_gfx11_wmma_matmul`` (:301-326) with its geometry
(work_shape (ceil_div(M, 16) * 32, ceil_div(N, 16)), group_shape (32, 1),
subgroup_size 32).  Lane l of the 16x16x16 step owns column l % 16 and rows
l // 16, l // 16 + 2, ..., 14 + l // 16 of the tile.

The other kernels are near misses that the gfx950 target must reject.
"""

from __future__ import annotations

import numpy as np

from hc import Buffer, WorkGroup, WorkItem, idx_type, kernel, sym, tensor_type, undef_type, vector_type
from hc.symbols import ceil_div

M = sym.M
N = sym.N
K = sym.K

LANES = 32
TILE = 16
ROWS_PER_LANE = TILE * TILE // LANES  # 8 accumulator floats per lane


def lane_rows(lane: int, wave_size: int) -> tuple[int, ...]:
    return tuple(range(lane // 16, TILE, wave_size // 16))


@kernel.intrinsic(
    scope=WorkItem,
    effects="pure",
    const_attrs={"wave_size", "arch"},
    operand_types=(
        undef_type(),
        tensor_type((TILE, TILE), np.float16),
        tensor_type((TILE, TILE), np.float16),
        vector_type((TILE,), np.float16),
        vector_type((TILE,), np.float16),
        vector_type((ROWS_PER_LANE,), np.float32),
        idx_type(),
    ),
    result_types=(vector_type((ROWS_PER_LANE,), np.float32),),
)
def wmma_gfx11(group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    """One lane's accumulators after a 16x16x16 step: a sequential float32
    fold over k of the lane's rows against its column (inactive entries +0)."""
    _ = (a_frag, b_frag)
    a_tile = a_tile.with_inactive(value=np.float16(0))
    b_tile = b_tile.with_inactive(value=np.float16(0))
    rows = lane_rows(lane, wave_size)
    col = lane % TILE
    out = np.empty((len(rows),), dtype=np.float32)
    for i, row in enumerate(rows):
        s = np.float32(acc_frag[i])
        for kk in range(TILE):
            s += np.float32(a_tile[row, kk]) * np.float32(b_tile[kk, col])
        out[i] = s
    return group.vload(out, shape=(len(rows),))


@wmma_gfx11.verify
def _verify_wmma(sig, target):
    _ = target
    if sig.scope is not WorkItem:
        raise ValueError("wmma_gfx11 must execute in WorkItem scope")
    if sig.kwarg("arch") != "gfx11" or sig.kwarg("wave_size") != LANES:
        raise ValueError("wmma_gfx11 expects arch='gfx11' and wave_size=32")
    lane = sig.kwarg("lane")
    if not isinstance(lane, int) or not 0 <= lane < LANES:
        raise ValueError("wmma_gfx11 lane must be in [0, 32)")
    for index, is_tensor, shape, dtype in ((1, True, (TILE, TILE), np.float16), (2, True, (TILE, TILE), np.float16),
                                           (3, False, (TILE,), np.float16), (4, False, (TILE,), np.float16),
                                           (5, False, (ROWS_PER_LANE,), np.float32)):
        value = sig.arg(index)
        if (value.is_tensor() if is_tensor else value.is_vector()) is False:
            raise ValueError(f"operand {index} has the wrong kind")
        if value.shape != shape or value.type != np.dtype(dtype):
            raise ValueError(f"operand {index} must be {shape} {np.dtype(dtype).name}")


@wmma_gfx11.lower(target="amdgpu-gfx11")
def _lower_wmma(ctx, group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    _ = (group, a_tile, b_tile, lane)
    op = ctx.builder.create("amdgpu.wmma", results=[ctx.result_type(0)], operands=[a_frag, b_frag, acc_frag],
                            attrs={"arch": arch, "wave_size": wave_size, "m": TILE, "n": TILE, "k": TILE},
                            loc=ctx.loc)
    return op.result(0)


@kernel.func(scope=WorkItem)
def a_fragment(wi, a_tile):
    return a_tile[wi.local_id()[0] % TILE, :].vec().with_inactive(value=np.float16(0))


@kernel.func(scope=WorkItem)
def b_fragment(wi, b_tile):
    return b_tile[:, wi.local_id()[0] % TILE].vec().with_inactive(value=np.float16(0))


@kernel.func(scope=WorkGroup)
def zero_acc(group):
    @group.workitems
    def init(wi):
        _ = wi
        return group.vzeros(shape=(ROWS_PER_LANE,), dtype=np.float32)

    return init()


@kernel.func(scope=WorkGroup)
def wmma_step(group, a_tile, b_tile, acc):
    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        return wmma_gfx11(group, a_tile, b_tile, a_fragment(wi, a_tile), b_fragment(wi, b_tile), acc[:, lane, 0],
                          lane=lane, wave_size=LANES, arch="gfx11")

    return lanes()


@kernel.func(scope=WorkGroup)
def store_acc(group, c, row0, col0, acc) -> None:
    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        col = col0 + lane % TILE
        group.store(c[row0 + lane // 16 : row0 + TILE : LANES // 16, col : col + 1], acc[:, lane, :])

    lanes()


def tile_origin(tile_row: int, tile_col: int) -> tuple[int, int]:
    return tile_row * TILE, tile_col * TILE


GEOMETRY = dict(work_shape=(ceil_div(M, TILE) * LANES, ceil_div(N, TILE)), group_shape=(LANES, 1),
                subgroup_size=LANES)


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
        acc = wmma_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


# --------------------------------------------------------------------------
# Near misses
# --------------------------------------------------------------------------


@kernel.func(scope=WorkGroup)
def store_transposed(group, c, row0, col0, acc) -> None:
    """Writes the tile's (row, col) accumulator to C[col0 + row, row0 + col]."""

    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        row = row0 + lane % TILE
        group.store(c[row : row + 1, col0 + lane // 16 : col0 + TILE : LANES // 16], acc[:, lane, :].vec((1, 8)))

    lanes()


@kernel(**GEOMETRY)
def transposed_store_kernel(
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
        acc = wmma_step(group, a_tile, b_tile, acc)
    store_transposed(group, c, row0, col0, acc)


@kernel(**GEOMETRY)
def k_step_32_kernel(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = tile_origin(group.group_id[0], group.group_id[1])
    acc = zero_acc(group)
    for k0 in range(0, a.shape[1], 32):
        a_tile = group.load(a[row0 : row0 + TILE, k0 : k0 + TILE], shape=(TILE, TILE))
        b_tile = group.load(b[k0 : k0 + TILE, col0 : col0 + TILE], shape=(TILE, TILE))
        acc = wmma_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


@kernel(**GEOMETRY)
def no_accumulate_kernel(
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
    store_acc(group, c, row0, col0, acc)


@kernel(**GEOMETRY)
def short_k_kernel(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = tile_origin(group.group_id[0], group.group_id[1])
    acc = zero_acc(group)
    for k0 in range(0, a.shape[1] - TILE, TILE):
        a_tile = group.load(a[row0 : row0 + TILE, k0 : k0 + TILE], shape=(TILE, TILE))
        b_tile = group.load(b[k0 : k0 + TILE, col0 : col0 + TILE], shape=(TILE, TILE))
        acc = wmma_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


@kernel(work_shape=(ceil_div(M, 32) * LANES, ceil_div(N, TILE)), group_shape=(LANES, 1), subgroup_size=LANES)
def half_grid_kernel(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    """Launches one workgroup per 32 rows but covers 16: half of C stays unwritten."""
    row0, col0 = tile_origin(group.group_id[0], group.group_id[1])
    acc = zero_acc(group)
    for k0 in range(0, a.shape[1], TILE):
        a_tile = group.load(a[row0 : row0 + TILE, k0 : k0 + TILE], shape=(TILE, TILE))
        b_tile = group.load(b[k0 : k0 + TILE, col0 : col0 + TILE], shape=(TILE, TILE))
        acc = wmma_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


@kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"wave_size", "arch"},
                  result_types=(vector_type((ROWS_PER_LANE,), np.float32),))
def wmma_unlowered(group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    """The same arithmetic as wmma_gfx11, with no lowering registered."""
    _ = (a_frag, b_frag, arch)
    a_tile = a_tile.with_inactive(value=np.float16(0))
    b_tile = b_tile.with_inactive(value=np.float16(0))
    rows = lane_rows(lane, wave_size)
    out = np.empty((len(rows),), dtype=np.float32)
    for i, row in enumerate(rows):
        s = np.float32(acc_frag[i])
        for kk in range(TILE):
            s += np.float32(a_tile[row, kk]) * np.float32(b_tile[kk, lane % TILE])
        out[i] = s
    return group.vload(out, shape=(len(rows),))


@kernel.func(scope=WorkGroup)
def unlowered_step(group, a_tile, b_tile, acc):
    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        return wmma_unlowered(group, a_tile, b_tile, a_fragment(wi, a_tile), b_fragment(wi, b_tile),
                              acc[:, lane, 0], lane=lane, wave_size=LANES, arch="gfx11")

    return lanes()


@kernel(**GEOMETRY)
def unlowered_kernel(
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
        acc = unlowered_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


@kernel(**GEOMETRY)
def some_other_kernel(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    raise AssertionError("not a contraction")


@kernel(work_shape=(ceil_div(M, 16) * 32,), group_shape=(32,), subgroup_size=32)
def tiled_gfx950_mfma_matmul(group, x: Buffer[M, np.float16]) -> None:
    """The package kernel's name, but not a contraction signature."""
    raise AssertionError("never runs")


# Near misses in the arithmetic: the same structure, with intrinsics whose
# fallback bodies accumulate more narrowly than float32.  On small integer
# inputs they agree with A @ B; the launch must still reject them, because
# the GPU kernel would accumulate in float32 and return other results than
# the simulator gives for them.


def _narrow_fold(a_tile, b_tile, acc_frag, lane, wave_size, fold_type, clamp, out_type):
    a_tile = a_tile.with_inactive(value=np.float16(0))
    b_tile = b_tile.with_inactive(value=np.float16(0))
    rows = lane_rows(lane, wave_size)
    out = np.empty((len(rows),), dtype=out_type)
    with np.errstate(over="ignore"):  # float16 sums overflow on the wide probe
        for i, row in enumerate(rows):
            s = fold_type(acc_frag[i])
            for kk in range(TILE):
                s = fold_type(s + fold_type(a_tile[row, kk]) * fold_type(b_tile[kk, lane % TILE]))
            out[i] = min(max(s, -clamp), clamp) if clamp else s
    return out


def _lower_as_wmma(ctx, group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    return _lower_wmma(ctx, group, a_tile, b_tile, a_frag, b_frag, acc_frag, lane=lane, wave_size=wave_size,
                       arch=arch)


@kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"wave_size", "arch"},
                  result_types=(vector_type((ROWS_PER_LANE,), np.float32),))
def wmma_f16_fold(group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    """Sums in float16, returns float32."""
    _ = (a_frag, b_frag, arch)
    out = _narrow_fold(a_tile, b_tile, acc_frag, lane, wave_size, np.float16, None, np.float32)
    return group.vload(out, shape=(len(out),))


@kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"wave_size", "arch"},
                  result_types=(vector_type((ROWS_PER_LANE,), np.float32),))
def wmma_clamped(group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    """Sums in float32, clamps each result to [-4096, 4096]."""
    _ = (a_frag, b_frag, arch)
    out = _narrow_fold(a_tile, b_tile, acc_frag, lane, wave_size, np.float32, np.float32(4096), np.float32)
    return group.vload(out, shape=(len(out),))


@kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"wave_size", "arch"},
                  result_types=(vector_type((ROWS_PER_LANE,), np.float32),))
def wmma_f16_result(group, a_tile, b_tile, a_frag, b_frag, acc_frag, *, lane, wave_size, arch):
    """Sums in float32, returns the accumulator rounded to float16 (while it
    declares a float32 result, so only the value it returns shows it)."""
    _ = (a_frag, b_frag, arch)
    out = _narrow_fold(a_tile, b_tile, acc_frag, lane, wave_size, np.float32, None, np.float16)
    return group.vload(out, shape=(len(out),))


for _narrow in (wmma_f16_fold, wmma_clamped, wmma_f16_result):
    _narrow.lower(target="amdgpu-gfx11")(_lower_as_wmma)


@kernel.func(scope=WorkGroup)
def f16_fold_step(group, a_tile, b_tile, acc):
    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        return wmma_f16_fold(group, a_tile, b_tile, a_fragment(wi, a_tile), b_fragment(wi, b_tile),
                             acc[:, lane, 0], lane=lane, wave_size=LANES, arch="gfx11")

    return lanes()


@kernel.func(scope=WorkGroup)
def clamped_step(group, a_tile, b_tile, acc):
    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        return wmma_clamped(group, a_tile, b_tile, a_fragment(wi, a_tile), b_fragment(wi, b_tile),
                            acc[:, lane, 0], lane=lane, wave_size=LANES, arch="gfx11")

    return lanes()


@kernel.func(scope=WorkGroup)
def f16_result_step(group, a_tile, b_tile, acc):
    @group.workitems
    def lanes(wi):
        lane = wi.local_id()[0]
        return wmma_f16_result(group, a_tile, b_tile, a_fragment(wi, a_tile), b_fragment(wi, b_tile),
                               acc[:, lane, 0], lane=lane, wave_size=LANES, arch="gfx11")

    return lanes()


@kernel(**GEOMETRY)
def f16_fold_kernel(
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
        acc = f16_fold_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


@kernel(**GEOMETRY)
def clamped_kernel(
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
        acc = clamped_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


@kernel(**GEOMETRY)
def f16_result_kernel(
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
        acc = f16_result_step(group, a_tile, b_tile, acc)
    store_acc(group, c, row0, col0, acc)


# A wave64 kernel whose intrinsic states the 32x32x16 arithmetic but whose
# amdgpu-gfx950 lowering declares another instruction (32x32x8): the launch
# must refuse it, since the op it would run is not the one the fallback states.

from hc.gfx950 import kernels as _gfx  # noqa: E402
from hc.gfx950.kernels import init_acc, store_tile  # noqa: E402


@kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"wave_size", "arch"},
                  result_types=(vector_type((_gfx.ACC_REGS,), np.float32),))
def mfma_k8_gfx950(group, a_tile, b_tile, acc_frag, *, lane, wave_size, arch):
    """The 32x32x16 fallback of mfma_gfx950."""
    _ = (wave_size, arch)
    values = _gfx._lane_fold(a_tile, b_tile, acc_frag, _gfx.lane_acc_rows(lane), _gfx.lane_column(lane), _gfx.MFMA_K)
    return group.vload(values, shape=(_gfx.ACC_REGS,))


@mfma_k8_gfx950.lower(target="amdgpu-gfx950")
def _lower_k8(ctx, group, a_tile, b_tile, acc_frag, *, lane, wave_size, arch):
    _ = (group, lane)
    op = ctx.builder.create("rocdl.mfma.f32.32x32x8", results=[ctx.result_type(0)],
                            operands=[a_tile, b_tile, acc_frag],
                            attrs={"arch": arch, "wave_size": wave_size, "m": 32, "n": 32, "k": 8}, loc=ctx.loc)
    return op.result(0)


@kernel.func(scope=WorkGroup)
def k8_step(group, a_tile, b_tile, acc):
    @group.workitems
    def wave(wi):
        lane = wi.local_id()[0]
        return mfma_k8_gfx950(group, a_tile, b_tile, acc[:, lane, 0], lane=lane, wave_size=64, arch="gfx950")

    return wave()


@kernel(work_shape=(ceil_div(M, 32) * 64, ceil_div(N, 32)), group_shape=(64, 1), subgroup_size=64)
def wrong_shape_kernel(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = group.group_id[0] * 32, group.group_id[1] * 32
    acc = init_acc(group)
    for k0 in range(0, a.shape[1], 16):
        a_tile = group.load(a[row0 : row0 + 32, k0 : k0 + 16], shape=(32, 16))
        b_tile = group.load(b[k0 : k0 + 16, col0 : col0 + 32], shape=(16, 32))
        acc = k8_step(group, a_tile, b_tile, acc)
    store_tile(group, c, row0, col0, acc)
