"""The C ABI library: it is built, loads, exports every entry point that
include/hcg_gemm.h and include/hcg_tile_ops.h declare, and rejects bad
arguments on the host before any HIP call (no GPU needed for these)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from hc.gfx950 import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("hcg_gemm.h", "hcg_tile_ops.h", "hcg_mfma.h")]


def declared_functions() -> list[str]:
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(hcg_\w+)\s*\(", text, re.M)))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted(_native.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    assert os.path.exists(_native.LIB_PATH), "run 5_amd/csrc/build.py (or __graft_entry__.build())"
    lib = _native.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.hcg_version() == 100


def test_probe_library_exports_what_its_header_declares():
    from hc.gfx950 import probe

    text = open(os.path.join(ROOT, "include", "hcg_probe.h")).read()
    declared = sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(hcg_\w+)\s*\(", text, re.M)))
    assert declared == sorted(probe.EXPORTS)
    assert os.path.exists(probe.LIB_PATH), "run 5_amd/csrc/build.py"
    lib = probe.load()
    for name in declared:
        assert hasattr(lib, name), name
    # bad arguments are rejected on the host, before any launch
    assert lib.hcg_probe_mfma(2, 1, 1, 0x1000, 0x1000, None) == 1
    assert "dtype" in lib.hcg_probe_last_error().decode()
    assert lib.hcg_probe_mfma16(0, 6, 1, 0x1000, 0x1000, None) == 1
    assert "multiple of 4" in lib.hcg_probe_last_error().decode()
    assert lib.hcg_probe_read(0x1000, 4096, 24, 8, 1, 4, 0x1000, None) == 1
    assert "power of two" in lib.hcg_probe_last_error().decode()
    assert lib.hcg_probe_read(0x1000, 4096, 256, 8, 1, 3, 0x1000, None) == 1
    assert "unroll" in lib.hcg_probe_last_error().decode()
    assert lib.hcg_probe_write(0x1000, 100, 4, 0, None) == 1


@pytest.mark.parametrize(
    "args,match",
    [
        ((0, 5, None, 0, None, 0, None, 0, 1, 1, 1, None), "dtype must be"),
        ((10, 0, None, 0, None, 0, None, 0, 1, 1, 1, None), "unknown algo"),
        ((0, 0, None, 0, None, 0, None, 0, -1, 1, 1, None), "negative extent"),
        ((2, 0, None, 0, None, 0, None, 0, 129, 1, 1, None), "needs M <= 128"),
        ((0, 0, None, 0, None, 0, None, 0, 2, 2, 2, None), "C is NULL"),
        ((0, 0, 0x1000, 2, 0x1000, 2, 0x1000, 1, 2, 2, 2, None), r"ldc \(1\) < N \(2\)"),
        ((0, 0, 0x1000, 1, 0x1000, 2, 0x1000, 2, 2, 2, 2, None), r"lda \(1\) < K \(2\)"),
        ((0, 0, 0x1000, 2, 0x1000, 1, 0x1000, 2, 2, 2, 2, None), r"ldb \(1\) < N \(2\)"),
        ((0, 0, None, 0, None, 0, None, 0, 1 << 31, 1, 1, None), "extent above 2\\^30"),
    ],
)
def test_invalid_arguments_are_rejected_on_the_host(args, match):
    lib = _native.load()
    assert lib.hcg_gemm_algo(*args) == _native.HCG_EINVAL
    assert re.search(match, _native.last_error(lib))


def test_empty_output_is_a_noop_and_clears_the_error():
    lib = _native.load()
    lib.hcg_gemm_algo(0, 5, None, 0, None, 0, None, 0, 1, 1, 1, None)
    assert _native.last_error(lib)
    assert lib.hcg_gemm(0, None, 0, None, 0, None, 0, 0, 5, 5, None) == _native.HCG_OK
    assert _native.last_error(lib) == ""


@pytest.mark.parametrize(
    "args,match",
    [
        ((3, 0x1000, 4, 4, 4, 0x1000, 1, 2, 2, None, 0, 0x1000, None, None), "elem_bytes must be 2, 4 or 8"),
        ((2, 0x1000, 4, -1, 4, 0x1000, 1, 2, 2, None, 0, 0x1000, None, None), "negative extent"),
        ((2, None, 4, 4, 4, 0x1000, 1, 2, 2, None, 0, 0x1000, None, None), "view pointer is NULL"),
        ((2, 0x1000, 3, 4, 4, 0x1000, 1, 2, 2, None, 0, 0x1000, None, None), r"ld \(3\) < cols \(4\)"),
        ((2, 0x1000, 4, 4, 4, None, 1, 2, 2, None, 0, 0x1000, None, None), "origins is NULL"),
        ((2, 0x1000, 4, 4, 4, 0x1000, 1, 2, 2, None, 0, None, None, None), "out is NULL"),
    ],
)
def test_tile_load_rejects_bad_arguments_on_the_host(args, match):
    lib = _native.load()
    assert lib.hcg_tile_load(*args) == _native.HCG_EINVAL
    assert re.search(match, _native.last_error(lib))


def test_tile_ops_with_nothing_to_do_launch_nothing():
    lib = _native.load()
    # no tiles, empty tiles, and a store into an empty view
    assert lib.hcg_tile_load(2, 0x1000, 4, 4, 4, None, 0, 2, 2, None, 0, None, None, None) == _native.HCG_OK
    assert lib.hcg_tile_load(4, 0x1000, 4, 4, 4, 0x1000, 3, 0, 5, None, 0, None, None, None) == _native.HCG_OK
    assert lib.hcg_tile_store(8, None, 0, 0, 0, 0x1000, 2, 2, 2, 0x1000, None, None) == _native.HCG_OK
    assert lib.hcg_tile_store(2, 0x1000, 4, 4, 4, 0x1000, 1, 2, 2, None, None, None) == _native.HCG_EINVAL
    assert "tiles is NULL" in _native.last_error(lib)


def test_device_tensor_binding_is_built_and_leaves_other_cases_to_python():
    """_hcg_torch (the compiled binding of hcg_gemm_algo for device tensors)
    is built beside the library and returns -1, launching nothing, for
    tensors it does not take (here CPU tensors)."""
    torch = pytest.importorskip("torch")
    from hc.gfx950 import _hcg_torch

    a = torch.zeros((4, 4), dtype=torch.float16)
    assert _hcg_torch.gemm(a, a, torch.zeros((4, 4)), 0) == -1


def test_loading_the_library_leaves_the_garbage_collector_alone():
    """Opening the library (and importing the package) neither freezes nor
    disables Python's cyclic garbage collector: that stays the caller's
    choice.  Runs in a fresh interpreter, where nothing has loaded it yet."""
    import subprocess
    import sys

    code = (
        "import gc, sys; sys.path[:0] = [%r];"
        "before = (gc.get_freeze_count(), gc.isenabled(), gc.get_threshold());"
        "import hc, hc.gfx950; from hc.gfx950 import _native; _native.load();"
        "after = (gc.get_freeze_count(), gc.isenabled(), gc.get_threshold());"
        "assert before == after, (before, after); print('ok')"
    ) % os.path.join(ROOT, "5_amd")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stderr


def test_operand_query_without_device_memory():
    """hcg_operand_in_place decides on the host.  Rows 16-byte aligned: in
    place; an odd address: copied; a tail whose extra bytes stay in the last
    element's 4 KB page: in place without asking the runtime; a tail that
    crosses into the next page of memory the runtime does not know (here host
    memory): copied."""
    lib = _native.load()
    q = lib.hcg_operand_in_place
    assert q(0x10000, 4, 8, 8) == 1  # aligned rows
    assert q(0x10001, 1, 3, 3) == 0  # odd address
    # 1 x 3 at 0x10002: last byte 0x10007, the 16-byte pieces read to 0x10021
    assert q(0x10002, 1, 3, 3) == 1
    # rows at 2-byte alignment ending 2 bytes before a page boundary: the
    # pieces read past it, into a page the runtime knows nothing about
    buf = ctypes.create_string_buffer(3 * 4096)
    page = (ctypes.addressof(buf) + 4095) & ~4095
    assert q(page + 4096 - 2 * 11 - 2, 1, 11, 11) == 0
    assert q(None, 1, 1, 1) == -1 and "NULL" in _native.last_error(lib)
    assert q(0x10000, 2, 8, 7) == -1 and "ld 7" in _native.last_error(lib)


@pytest.mark.parametrize(
    "args,match",
    [
        ((2, 32, 32, 16, 0x1000, 0x1000, None, None, 0x1000, 0x1000, None), "dtype must be"),
        ((0, 32, 32, 8, 0x1000, 0x1000, None, None, 0x1000, 0x1000, None), "32 x 32 x 8"),
        ((1, 16, 16, 16, 0x1000, 0x1000, None, None, 0x1000, 0x1000, None), "16 x 16 x 16"),
        ((0, 16, 16, 32, None, 0x1000, None, None, 0x1000, 0x1000, None), "must not be NULL"),
        ((0, 32, 32, 16, 0x1000, 0x1000, None, None, 0x1000, None, None), "must not be NULL"),
    ],
)
def test_mfma_step_rejects_bad_arguments_on_the_host(args, match):
    lib = _native.load()
    assert lib.hcg_mfma_step(*args) == _native.HCG_EINVAL
    assert re.search(match, _native.last_error(lib))


def test_stamps_library_is_built_apart_and_its_records_reduce():
    """The timestamped build exports hcg_stamps_set (the product library does
    not), and breakdown() reduces records: two CUs of one XCD, one running two
    workgroups in sequence, at a 2.0 GHz shader clock."""
    import numpy as np

    from hc.gfx950 import stamps

    assert os.path.exists(stamps.LIB_PATH), "run 5_amd/csrc/build.py"
    assert not hasattr(_native.load(), "hcg_stamps_set")
    assert hasattr(ctypes.CDLL(stamps.LIB_PATH), "hcg_stamps_set")

    def rec(t0, t1, t2, t3, cu):
        return [t0, t1, t2, t3, 2 * (t2 - t1) * 10, 2 * (t3 - t0) * 10, 3, cu << 8]

    r = np.array([rec(1000, 1100, 2100, 2300, 1), rec(1010, 1110, 2010, 2210, 2), rec(2400, 2500, 3500, 3700, 1),
                  [0] * 8], dtype=np.uint64)
    out = stamps.breakdown(r)
    assert out["workgroups"] == 3
    assert out["span_us"] == 27.0
    assert out["k_loop_us"] == {"mean": 29.0 / 3, "min": 9.0, "max": 10.0}
    assert out["per_xcd"][0]["xcd"] == 3 and abs(out["per_xcd"][0]["clock_mhz"] - 2000) < 1e-9
    assert out["cu_rounds"] == {"cus": 2, "max_per_cu": 2, "min_per_cu": 1, "mean_gap_us": 1.0}
    assert out["start_spread_us"] == 0.1


def test_stamps_buffer_splits_into_two_consecutive_launches():
    """Records of two launches of a 3-workgroup grid: slot 1 (the earlier
    launch here) at records 3..5, slot 0 (later) at 0..2; workgroup 1 of the
    later launch never wrote (a padding workgroup)."""
    import numpy as np

    from hc.gfx950 import stamps

    def rec(t0, t3, slot, grid=3):
        return [t0, t0 + 10, t3 - 10, t3, 0, 0, 5 | (grid << 8) | (slot << 48), 0]

    buf = np.zeros((8, 8), dtype=np.uint64)
    buf[0] = rec(2000, 2900, 0)
    buf[2] = rec(2010, 2950, 0)
    buf[3] = rec(1000, 1800, 1)
    buf[4] = rec(1005, 1850, 1)
    buf[5] = rec(1010, 1900, 1)
    (prev, prev_wg), (last, last_wg) = stamps.split_launches(buf)
    assert list(prev_wg) == [0, 1, 2] and list(last_wg) == [0, 2]
    assert int(prev[:, 3].max()) == 1900 and int(last[:, 0].min()) == 2000
