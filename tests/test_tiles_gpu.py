"""GPU parity of the masked tile gather / scatter (include/hcg_tile_ops.h)
against the oracle's restatement of the hc tile semantics
(hc/simulator.py:1304-1357, 1416-1458; doc/langref.md:530-596).

Bit-exact: these are copies.  Cases: 2-, 4- and 8-byte elements, contiguous
and column-sliced views (row stride > cols, 2-byte aligned starts), tile
origins inside, on and beyond every edge (negative ones too), mask= operands,
fill values (NaN included), guard bands around the store target, and empty
batches.
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest

import hc_oracle as oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DEV = "cuda:0"

DTYPES = {
    "float16": (torch.float16, np.float16),
    "bfloat16": (torch.bfloat16, None),
    "float32": (torch.float32, np.float32),
    "int64": (torch.int64, np.int64),
}


def _source(rng, rows, cols, name):
    tdt, ndt = DTYPES[name]
    if name == "bfloat16":
        x = torch.from_numpy(rng.standard_normal((rows, cols)).astype(np.float32)).to(torch.bfloat16)
        return x, x.view(torch.int16).numpy()
    if name == "int64":
        x = rng.integers(-(1 << 40), 1 << 40, size=(rows, cols)).astype(np.int64)
    else:
        x = rng.standard_normal((rows, cols)).astype(ndt)
    return torch.from_numpy(x), x


def _bits(t):
    """Host bits of a device tensor, as the integer type of its width."""
    ints = {2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    return t.cpu().view(ints).numpy()


def _origins(rng, n, rows, cols, th, tw):
    o = np.stack([rng.integers(-th, rows + 2, n), rng.integers(-tw, cols + 2, n)], axis=1)
    # plus the corners and exactly-on-the-edge tiles
    extra = [[0, 0], [rows - th, cols - tw], [rows - 1, cols - 1], [rows, 0], [0, cols], [-th, -tw]]
    return np.concatenate([o, np.array(extra)]).astype(np.int64)


@pytest.mark.parametrize("name", list(DTYPES))
@pytest.mark.parametrize("shape", [(16, 16), (17, 19), (1, 1), (3, 40), (32, 8)])
@pytest.mark.parametrize("sliced", [False, True])
def test_tile_load_matches_oracle(name, shape, sliced):
    import hc.gfx950 as g

    rng = np.random.default_rng(zlib.crc32(f"{name}{shape}{sliced}".encode()))
    rows, cols = 45, 77
    full_t, full_n = _source(rng, rows, cols + 5, name)
    if sliced:
        src_t, src_n = full_t[:, 3 : 3 + cols], full_n[:, 3 : 3 + cols]
    else:
        src_t, src_n = full_t[:, :cols].contiguous(), np.ascontiguousarray(full_n[:, :cols])
    th, tw = shape
    origins = _origins(rng, 40, rows, cols, th, tw)
    mask = rng.random((len(origins), th, tw)) < 0.75
    src_dev = (full_t.to(DEV)[:, 3 : 3 + cols]) if sliced else src_t.to(DEV)
    print(f"case tile_load {name} {shape} sliced={sliced}", flush=True)
    for m in (None, mask):
        fill = -3
        tiles, act = g.tile_load(src_dev, torch.from_numpy(origins).to(DEV), shape,
                                 mask=None if m is None else torch.from_numpy(m).to(DEV), fill=fill)
        torch.cuda.synchronize()
        if name == "bfloat16":
            fill_bits = torch.tensor([fill], dtype=torch.bfloat16).view(torch.int16).item()
            want, wact = oracle.tile_load(src_n, origins, shape, mask=m, fill=fill_bits)
        else:
            want, wact = oracle.tile_load(src_n, origins, shape, mask=m, fill=fill)
            want = want.view({2: np.int16, 4: np.int32, 8: np.int64}[want.itemsize])
        assert np.array_equal(act.cpu().numpy(), wact)
        assert np.array_equal(_bits(tiles), want)


def test_tile_load_nan_fill_and_zero_tiles():
    import hc.gfx950 as g

    src = torch.arange(12, dtype=torch.float32, device=DEV).reshape(3, 4)
    tiles, act = g.tile_load(src, [[2, 2]], (2, 3), fill=float("nan"))
    got = tiles.cpu().numpy()
    assert got[0, 0, 0] == 10 and got[0, 0, 1] == 11 and np.isnan(got[0, 0, 2]) and np.isnan(got[0, 1]).all()
    assert act.cpu().numpy().sum() == 2
    empty, eact = g.tile_load(src, torch.zeros((0, 2), dtype=torch.int64), (4, 4))
    assert empty.shape == (0, 4, 4) and eact.shape == (0, 4, 4)


@pytest.mark.parametrize("name", ["float16", "float32", "int64"])
@pytest.mark.parametrize("shape", [(16, 16), (5, 9), (2, 33)])
def test_tile_store_matches_oracle_and_leaves_the_guard_band(name, shape):
    import hc.gfx950 as g

    rng = np.random.default_rng(zlib.crc32(f"{name}{shape}".encode()))
    rows, cols = 40, 70
    th, tw = shape
    # Non-overlapping tile grid over (and past) the view, shuffled, plus a
    # few tiles wholly outside it.
    grid = [[r, c] for r in range(-th, rows + th, th) for c in range(-tw, cols + tw, tw)]
    origins = np.array(grid, dtype=np.int64)[rng.permutation(len(grid))]
    _, ndt = DTYPES[name]
    tiles_n = (rng.integers(1, 1000, size=(len(origins), th, tw))).astype(ndt)
    mask = rng.random(tiles_n.shape) < 0.6
    print(f"case tile_store {name} {shape}", flush=True)
    for m in (None, mask):
        sentinel = -7
        guard = torch.full((rows + 4, cols + 9), sentinel, dtype=DTYPES[name][0], device=DEV)
        view = guard[2 : 2 + rows, 5 : 5 + cols]
        g.tile_store(view, torch.from_numpy(origins).to(DEV), torch.from_numpy(tiles_n).to(DEV),
                     mask=None if m is None else torch.from_numpy(m).to(DEV))
        torch.cuda.synchronize()
        want = np.full((rows + 4, cols + 9), sentinel, dtype=ndt)
        oracle.tile_store(want[2 : 2 + rows, 5 : 5 + cols], origins, tiles_n, mask=m)
        assert np.array_equal(guard.cpu().numpy(), want)


def test_tile_store_then_load_round_trip_bf16():
    import hc.gfx950 as g

    rng = np.random.default_rng(3)
    dst = torch.zeros((33, 47), dtype=torch.bfloat16, device=DEV)
    origins = torch.tensor([[0, 0], [16, 16], [16, 40]], dtype=torch.int64, device=DEV)
    tiles = torch.from_numpy(rng.standard_normal((3, 17, 7)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    g.tile_store(dst, origins, tiles)
    back, act = g.tile_load(dst, origins, (17, 7))
    torch.cuda.synchronize()
    a = act.cpu()
    assert torch.equal(back.cpu()[a], tiles.cpu()[a])
    assert a[0].all() and a[1].sum().item() == 17 * 7 and a[2].sum().item() == 17 * 7
