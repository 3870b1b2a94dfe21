"""Hardware ceilings of the GPU a benchmark runs on (libhcg_probe.so, the C
ABI of include/hcg_probe.h): pure MFMA issue with its shader clock, and
streaming HBM reads and writes.  Measurement only; the GEMM path never
loads this library.

Every figure is taken in the board's sustained state: a probe first runs
back to back for ``warm_s`` seconds (the clock settles ~25 ms into a fresh
load), then a timed run of launches is bracketed by HIP events on the
launch stream.
"""

from __future__ import annotations

import ctypes
import os
import threading
import time
from typing import Any

from .._errors import BackendError

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhcg_probe.so")
EXPORTS = ("hcg_probe_mfma", "hcg_probe_mfma16", "hcg_probe_read", "hcg_probe_write", "hcg_probe_last_error")

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise BackendError(f"{LIB_PATH} is not built; run 5_amd/csrc/build.py")
            try:
                import torch  # noqa: F401  (one HIP runtime with torch)
            except ImportError:
                pass
            lib = ctypes.CDLL(LIB_PATH)
            i64, vp, c_int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
            lib.hcg_probe_mfma.argtypes = [c_int, c_int, c_int, vp, vp, vp]
            lib.hcg_probe_mfma.restype = c_int
            lib.hcg_probe_mfma16.argtypes = [c_int, c_int, c_int, vp, vp, vp]
            lib.hcg_probe_mfma16.restype = c_int
            lib.hcg_probe_read.argtypes = [vp, i64, c_int, i64, c_int, c_int, vp, vp]
            lib.hcg_probe_read.restype = c_int
            lib.hcg_probe_write.argtypes = [vp, i64, c_int, c_int, vp]
            lib.hcg_probe_write.restype = c_int
            lib.hcg_probe_last_error.argtypes = []
            lib.hcg_probe_last_error.restype = ctypes.c_char_p
            _lib = lib
        return _lib


def _check(lib: ctypes.CDLL, rc: int, what: str) -> None:
    if rc != 0:
        raise BackendError(f"{what} failed ({rc}): {lib.hcg_probe_last_error().decode()}")


def _timed(torch: Any, stream: Any, launch: Any, warm_s: float, launches: int) -> float:
    """Seconds per launch over `launches` back-to-back launches, after
    `warm_s` seconds of the same load."""
    t0 = time.perf_counter()
    while True:
        with torch.cuda.stream(stream):
            for _ in range(4):
                launch()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_s:
            break
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(launches):
            launch()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / launches


def mfma(torch: Any, stream: Any, dtype: int = 0, warm_s: float = 0.3, launches: int = 20,
         iters: int = 2048, per_cu: int = 1, small: bool = False) -> dict:
    """Pure MFMA issue on every CU (`per_cu` 4-wave workgroups per CU, 8
    independent 32x32x16 chains per wave, or with `small` 16 chains of
    16x16x32, the same flops): TFLOP/s, the fraction of the CUs' issue rate
    at the measured mean clock (the launch lasts as long as the slowest
    XCD's clock allows, so this stays below 1), shader cycles per MFMA
    inside the loop (32 for 32x32x16 and 16 for 16x16x32 at the full issue
    rate), and the shader clock (cycles over 100 MHz real-time ticks, per
    workgroup)."""
    lib = load()
    dev = torch.cuda.current_device()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks = cus * per_cu
    sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    clocks = torch.zeros(2 * blocks, dtype=torch.int64, device="cuda")

    entry = lib.hcg_probe_mfma16 if small else lib.hcg_probe_mfma

    def launch() -> None:
        _check(lib, entry(dtype, iters, blocks, sink.data_ptr(), clocks.data_ptr(), stream.cuda_stream),
               "hcg_probe_mfma16" if small else "hcg_probe_mfma")

    seconds = _timed(torch, stream, launch, warm_s, launches)
    flops = blocks * 4 * 8 * iters * 2 * 32 * 32 * 16
    c = clocks.view(blocks, 2).double().cpu()
    mhz = (c[:, 0] / (c[:, 1] / 100e6) / 1e6)
    tflops = flops / seconds / 1e12
    # 4096 fp16/bf16 flop per clock per CU (four SIMDs, one 32x32x16 MFMA
    # per 32 clocks each)
    issue = tflops * 1e12 / (cus * 4096 * float(mhz.mean()) * 1e6)
    chains = 16 if small else 8
    return {"dtype": "f16" if dtype == 0 else "bf16", "tflops": tflops, "issue_frac": issue,
            "cycles_per_mfma": float(c[:, 0].mean()) / (iters * chains),
            "us_per_launch": seconds * 1e6, "clock_mhz": float(mhz.mean()),
            "clock_mhz_min": float(mhz.min()), "clock_mhz_max": float(mhz.max()),
            "shape": f"{blocks} workgroups x 4 waves x {chains} chains x {iters} rounds of "
                     f"v_mfma_f32_{'16x16x32' if small else '32x32x16'}"}


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def read(torch: Any, stream: Any, pitch: int, width: int, nbytes: int, row_splits: int, unroll: int,
         warm_s: float = 0.1, launches: int = 20) -> dict:
    """Streaming read of `nbytes` as rows of `pitch` bytes in strips of
    `width`.  Launches rotate over enough copies (more than twice the 256 MB
    Infinity Cache in total) that every launch reads HBM."""
    lib = load()
    rows = nbytes // pitch
    copies = max(1, -(-2 * MALL_BYTES // (rows * pitch)) + 1)
    bufs = [torch.full((rows * pitch // 4,), 7, dtype=torch.int32, device="cuda") for _ in range(copies)]
    nstrips = pitch // width
    sink = torch.empty(nstrips * row_splits * 256, dtype=torch.int32, device="cuda")
    turn = [0]

    def launch() -> None:
        buf = bufs[turn[0] % copies]
        turn[0] += 1
        _check(lib, lib.hcg_probe_read(buf.data_ptr(), pitch, width, rows, row_splits, unroll, sink.data_ptr(),
                                       stream.cuda_stream), "hcg_probe_read")

    seconds = _timed(torch, stream, launch, warm_s, launches)
    del bufs
    return {"gbs": rows * pitch / seconds / 1e9, "us_per_launch": seconds * 1e6, "pitch": pitch, "width": width,
            "bytes": rows * pitch, "copies": copies, "workgroups": nstrips * row_splits, "unroll": unroll}


def write(torch: Any, stream: Any, nbytes: int, blocks: int, nontemporal: bool, warm_s: float = 0.1,
          launches: int = 10) -> dict:
    """Streaming 16-byte stores over `nbytes`."""
    lib = load()
    buf = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda")

    def launch() -> None:
        _check(lib, lib.hcg_probe_write(buf.data_ptr(), nbytes, blocks, int(nontemporal), stream.cuda_stream),
               "hcg_probe_write")

    seconds = _timed(torch, stream, launch, warm_s, launches)
    del buf
    return {"gbs": nbytes / seconds / 1e9, "us_per_launch": seconds * 1e6, "bytes": nbytes, "workgroups": blocks,
            "nontemporal": nontemporal}


def ceilings(torch: Any, stream: Any) -> dict:
    """What this board sustains, measured now: pure MFMA issue (fp16 and
    bf16, random operands; and fp16 as 16x16x32), streaming HBM read (1 GiB, contiguous and in
    1 KB strips of 16 KB rows; and at the skinny GEMM's size, 128 MiB of
    16 KB rows in 256-byte strips, the pattern its kernel streams B in) and
    streaming HBM write (1 GiB).  Each read figure is the best of a few
    launch shapes; every launch reads HBM (rotating copies)."""
    gib, mib = 1 << 30, 1 << 20
    out: dict = {"mfma_f16": mfma(torch, stream, 0), "mfma_bf16": mfma(torch, stream, 1),
                 "mfma16_f16": mfma(torch, stream, 0, small=True)}
    reads = [read(torch, stream, 4096, 4096, gib, 2048, 8), read(torch, stream, 16384, 1024, gib, 16, 8)]
    out["hbm_read"] = max(reads, key=lambda r: r["gbs"])
    c4 = [read(torch, stream, 16384, 256, 128 * mib, 4, 4), read(torch, stream, 4096, 4096, 128 * mib, 256, 8)]
    out["hbm_read_128mib"] = max(c4, key=lambda r: r["gbs"])
    writes = [write(torch, stream, gib, 256, True), write(torch, stream, gib, 512, False)]
    out["hbm_write"] = max(writes, key=lambda r: r["gbs"])
    return out
