"""The gfx950 GEMM written in the hc DSL (wave64, MFMA 32x32x16 and 16x16x32 fragments).

This is the kernel-definition side of the gfx950 path: the same structure as
the reference's wave32 WMMA example (examples/amdgpu_gfx11_wmma_matmul.py:
intrinsic with a fallback body :144-190, verify hook :193-197, lowering hook
:200-228, helpers :231-298, kernel :301-326) re-expressed for one 64-lane
wavefront per 32x32 output tile and the CDNA4 instruction
``v_mfma_f32_32x32x16_{f16,bf16}``.  The launch does not interpret it: the
gfx950 target recognises the tiled contraction (statement structure plus a
recorded CPU run through these helpers and the intrinsic's fallback body) and
lowers the whole kernel to the hand-written HIP kernels of libhcg_gfx950.so
(256x256 macro tiles of these fragments).  The fallback body
states the per-lane arithmetic precisely.

MFMA 32x32x16 register layout for lane l in [0, 64):
  A fragment: row l % 32, k = 8 * (l // 32) .. +7   (8 x 16-bit)
  B fragment: column l % 32, same k                  (8 x 16-bit)
  accumulator register r in [0, 16): row 8*(r//4) + 4*(l//32) + r%4,
  column l % 32.
MFMA 16x16x32 (``mfma16_gfx950``, the streaming kernels' instruction):
  A fragment: row l % 16, k = 8 * (l // 16) .. +7; B: column l % 16, same k
  accumulator register r in [0, 4): row 4*(l//16) + r, column l % 16.

Each intrinsic's ``amdgpu-gfx950`` lowering creates the op of its
instruction; ``hc.gfx950.intrinsics.run_wave`` records that op through the
lowering and executes it for one wave on the GPU (``hcg_mfma_step``), so the
fallback body's statement of every lane is checked against the hardware.
"""

from __future__ import annotations

import numpy as np

from ..core import Buffer, WorkGroup, WorkItem, bfloat16, kernel, vector_type
from ..symbols import ceil_div, sym
from ._contract import TARGET_NAME

WAVE_LANES = 64
MFMA_M = 32
MFMA_N = 32
MFMA_K = 16
ACC_REGS = MFMA_M * MFMA_N // WAVE_LANES  # 16 float32 per lane
GFX_ARCH = "gfx950"

M = sym.M
N = sym.N
K = sym.K


def lane_acc_rows(lane: int) -> tuple[int, ...]:
    """Output rows held by ``lane``'s 16 accumulator registers, in order."""
    return tuple(8 * (r // 4) + 4 * (lane // 32) + (r % 4) for r in range(ACC_REGS))


def lane_column(lane: int) -> int:
    return lane % MFMA_N


def lane_k_range(lane: int) -> range:
    return range(8 * (lane // 32), 8 * (lane // 32) + 8)


MFMA16_M = 16
MFMA16_N = 16
MFMA16_K = 32
ACC16_REGS = MFMA16_M * MFMA16_N // WAVE_LANES  # 4 float32 per lane


def lane16_acc_rows(lane: int) -> tuple[int, ...]:
    """Output rows of ``lane``'s 4 accumulator registers (16x16x32)."""
    return tuple(4 * (lane // 16) + r for r in range(ACC16_REGS))


def lane16_column(lane: int) -> int:
    return lane % MFMA16_N


def _lane_fold(a_tile, b_tile, acc_frag, rows, col, depth):
    """Accumulators of one lane: register i continues acc_frag[i] with the
    products of A row rows[i] and B column col, k ascending, in float32
    (inactive tile entries +0)."""
    a_tile = a_tile.with_inactive(value=0)
    b_tile = b_tile.with_inactive(value=0)
    values = np.empty((len(rows),), dtype=np.float32)
    for index, row in enumerate(rows):
        accum = np.float32(acc_frag[index])
        for k_idx in range(depth):
            accum += np.float32(a_tile[row, k_idx]) * np.float32(b_tile[k_idx, col])
        values[index] = accum
    return values


@kernel.intrinsic(
    scope=WorkItem,
    effects="pure",
    const_attrs={"wave_size", "arch"},
    operand_types=None,
    result_types=(vector_type((ACC_REGS,), np.float32),),
)
def mfma_gfx950(group, a_tile, b_tile, acc_frag, *, lane, wave_size, arch):
    """Fallback body: lane ``lane``'s 16 accumulators after one 32x32x16 step.

    Inactive (out-of-bounds) tile entries count as +0; each accumulator adds
    its 16 products in ascending k in float32.
    """
    values = _lane_fold(a_tile, b_tile, acc_frag, lane_acc_rows(lane), lane_column(lane), MFMA_K)
    return group.vload(values, shape=(ACC_REGS,))


@mfma_gfx950.verify
def _verify_mfma(sig, target):
    _ = target
    if sig.scope is not WorkItem:
        raise ValueError("mfma_gfx950 must execute in WorkItem scope")
    if sig.kwarg("arch") != GFX_ARCH:
        raise ValueError(f"mfma_gfx950 expects arch={GFX_ARCH!r}")
    if sig.kwarg("wave_size") != WAVE_LANES:
        raise ValueError(f"mfma_gfx950 expects wave_size={WAVE_LANES}")
    lane = sig.kwarg("lane")
    if not isinstance(lane, int) or not 0 <= lane < WAVE_LANES:
        raise ValueError(f"mfma_gfx950 lane must be in [0, {WAVE_LANES})")
    a, b = sig.arg(1), sig.arg(2)
    if a.shape != (MFMA_M, MFMA_K) or b.shape != (MFMA_K, MFMA_N):
        raise ValueError("mfma_gfx950 expects a 32x16 A tile and a 16x32 B tile")
    if a.type != b.type:
        raise ValueError("mfma_gfx950 operands must share one element type")


@mfma_gfx950.lower(target=TARGET_NAME)
def _lower_mfma(ctx, group, a_tile, b_tile, acc_frag, *, lane, wave_size, arch):
    _ = (group, lane)
    op = ctx.builder.create(
        "rocdl.mfma.f32.32x32x16",
        results=[ctx.result_type(0)],
        operands=[a_tile, b_tile, acc_frag],
        attrs={"arch": arch, "wave_size": wave_size, "m": MFMA_M, "n": MFMA_N, "k": MFMA_K},
        loc=ctx.loc,
    )
    return op.result(0)


@kernel.intrinsic(
    scope=WorkItem,
    effects="pure",
    const_attrs={"wave_size", "arch"},
    operand_types=None,
    result_types=(vector_type((ACC16_REGS,), np.float32),),
)
def mfma16_gfx950(group, a_tile, b_tile, acc_frag, *, lane, wave_size, arch):
    """Fallback body: lane ``lane``'s 4 accumulators after one 16x16x32 step
    (rows 4*(lane//16) .. +3 of column lane % 16; inactive entries +0; 32
    products per accumulator, ascending k, float32)."""
    values = _lane_fold(a_tile, b_tile, acc_frag, lane16_acc_rows(lane), lane16_column(lane), MFMA16_K)
    return group.vload(values, shape=(ACC16_REGS,))


@mfma16_gfx950.verify
def _verify_mfma16(sig, target):
    _ = target
    if sig.scope is not WorkItem:
        raise ValueError("mfma16_gfx950 must execute in WorkItem scope")
    if sig.kwarg("arch") != GFX_ARCH:
        raise ValueError(f"mfma16_gfx950 expects arch={GFX_ARCH!r}")
    if sig.kwarg("wave_size") != WAVE_LANES:
        raise ValueError(f"mfma16_gfx950 expects wave_size={WAVE_LANES}")
    lane = sig.kwarg("lane")
    if not isinstance(lane, int) or not 0 <= lane < WAVE_LANES:
        raise ValueError(f"mfma16_gfx950 lane must be in [0, {WAVE_LANES})")
    a, b = sig.arg(1), sig.arg(2)
    if a.shape != (MFMA16_M, MFMA16_K) or b.shape != (MFMA16_K, MFMA16_N):
        raise ValueError("mfma16_gfx950 expects a 16x32 A tile and a 32x16 B tile")
    if a.type != b.type:
        raise ValueError("mfma16_gfx950 operands must share one element type")


@mfma16_gfx950.lower(target=TARGET_NAME)
def _lower_mfma16(ctx, group, a_tile, b_tile, acc_frag, *, lane, wave_size, arch):
    _ = (group, lane)
    op = ctx.builder.create(
        "rocdl.mfma.f32.16x16x32",
        results=[ctx.result_type(0)],
        operands=[a_tile, b_tile, acc_frag],
        attrs={"arch": arch, "wave_size": wave_size, "m": MFMA16_M, "n": MFMA16_N, "k": MFMA16_K},
        loc=ctx.loc,
    )
    return op.result(0)


@kernel.func(scope=WorkGroup)
def init_acc(group):
    @group.workitems
    def init(wi):
        _ = wi
        return group.vzeros(shape=(ACC_REGS,), dtype=np.float32)

    return init()


@kernel.func(scope=WorkGroup)
def issue_mfma_tile(group, a_tile, b_tile, acc):
    @group.workitems
    def wave(wi):
        lane = wi.local_id()[0]
        return mfma_gfx950(group, a_tile, b_tile, acc[:, lane, 0], lane=lane, wave_size=WAVE_LANES, arch=GFX_ARCH)

    return wave()


@kernel.func(scope=WorkGroup)
def store_tile(group, c, row0, col0, acc) -> None:
    @group.workitems
    def wave(wi):
        lane = wi.local_id()[0]
        col = col0 + lane_column(lane)
        for r in range(ACC_REGS):
            row = row0 + 8 * (r // 4) + 4 * (lane // 32) + (r % 4)
            group.store(c[row : row + 1, col : col + 1], acc[r : r + 1, lane, :])

    wave()


_GEOMETRY = dict(
    work_shape=(ceil_div(M, MFMA_M) * WAVE_LANES, ceil_div(N, MFMA_N)),
    group_shape=(WAVE_LANES, 1),
    subgroup_size=WAVE_LANES,
)


@kernel(**_GEOMETRY)
def tiled_gfx950_mfma_matmul(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = group.group_id[0] * MFMA_M, group.group_id[1] * MFMA_N
    acc = init_acc(group)
    for k0 in range(0, a.shape[1], MFMA_K):
        a_tile = group.load(a[row0 : row0 + MFMA_M, k0 : k0 + MFMA_K], shape=(MFMA_M, MFMA_K))
        b_tile = group.load(b[k0 : k0 + MFMA_K, col0 : col0 + MFMA_N], shape=(MFMA_K, MFMA_N))
        acc = issue_mfma_tile(group, a_tile, b_tile, acc)
    store_tile(group, c, row0, col0, acc)


@kernel(**_GEOMETRY)
def tiled_gfx950_mfma_matmul_bf16(
    group,
    a: Buffer[M, K, bfloat16],
    b: Buffer[K, N, bfloat16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = group.group_id[0] * MFMA_M, group.group_id[1] * MFMA_N
    acc = init_acc(group)
    for k0 in range(0, a.shape[1], MFMA_K):
        a_tile = group.load(a[row0 : row0 + MFMA_M, k0 : k0 + MFMA_K], shape=(MFMA_M, MFMA_K))
        b_tile = group.load(b[k0 : k0 + MFMA_K, col0 : col0 + MFMA_N], shape=(MFMA_K, MFMA_N))
        acc = issue_mfma_tile(group, a_tile, b_tile, acc)
    store_tile(group, c, row0, col0, acc)



# -- the same contraction on 16x16x32 fragments (one wave per 16x16 tile) ------


@kernel.func(scope=WorkGroup)
def init_acc16(group):
    @group.workitems
    def init(wi):
        _ = wi
        return group.vzeros(shape=(ACC16_REGS,), dtype=np.float32)

    return init()


@kernel.func(scope=WorkGroup)
def issue_mfma16_tile(group, a_tile, b_tile, acc):
    @group.workitems
    def wave(wi):
        lane = wi.local_id()[0]
        return mfma16_gfx950(group, a_tile, b_tile, acc[:, lane, 0], lane=lane, wave_size=WAVE_LANES, arch=GFX_ARCH)

    return wave()


@kernel.func(scope=WorkGroup)
def store_tile16(group, c, row0, col0, acc) -> None:
    @group.workitems
    def wave(wi):
        lane = wi.local_id()[0]
        row = row0 + 4 * (lane // 16)
        col = col0 + lane16_column(lane)
        group.store(c[row : row + ACC16_REGS, col : col + 1], acc[:, lane, :])

    wave()


_GEOMETRY16 = dict(
    work_shape=(ceil_div(M, MFMA16_M) * WAVE_LANES, ceil_div(N, MFMA16_N)),
    group_shape=(WAVE_LANES, 1),
    subgroup_size=WAVE_LANES,
)


@kernel(**_GEOMETRY16)
def tiled_gfx950_mfma16_matmul(
    group,
    a: Buffer[M, K, np.float16],
    b: Buffer[K, N, np.float16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = group.group_id[0] * MFMA16_M, group.group_id[1] * MFMA16_N
    acc = init_acc16(group)
    for k0 in range(0, a.shape[1], MFMA16_K):
        a_tile = group.load(a[row0 : row0 + MFMA16_M, k0 : k0 + MFMA16_K], shape=(MFMA16_M, MFMA16_K))
        b_tile = group.load(b[k0 : k0 + MFMA16_K, col0 : col0 + MFMA16_N], shape=(MFMA16_K, MFMA16_N))
        acc = issue_mfma16_tile(group, a_tile, b_tile, acc)
    store_tile16(group, c, row0, col0, acc)


@kernel(**_GEOMETRY16)
def tiled_gfx950_mfma16_matmul_bf16(
    group,
    a: Buffer[M, K, bfloat16],
    b: Buffer[K, N, bfloat16],
    c: Buffer[M, N, np.float32],
) -> None:
    row0, col0 = group.group_id[0] * MFMA16_M, group.group_id[1] * MFMA16_N
    acc = init_acc16(group)
    for k0 in range(0, a.shape[1], MFMA16_K):
        a_tile = group.load(a[row0 : row0 + MFMA16_M, k0 : k0 + MFMA16_K], shape=(MFMA16_M, MFMA16_K))
        b_tile = group.load(b[k0 : k0 + MFMA16_K, col0 : col0 + MFMA16_N], shape=(MFMA16_K, MFMA16_N))
        acc = issue_mfma16_tile(group, a_tile, b_tile, acc)
    store_tile16(group, c, row0, col0, acc)
