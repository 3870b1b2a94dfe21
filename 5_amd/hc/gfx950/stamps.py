"""Where a GEMM launch's time goes, from per-workgroup timestamps.

libhcg_gfx950_stamps.so is the GEMM library built from the same sources with
``-DHCG_STAMPS`` (5_amd/csrc/build.py): there the tiled kernel
(``gemm_dma_kernel``) and the streaming kernel (``gemm_stream_kernel``) store,
per workgroup, the 100 MHz constant clock at its start, at the end of its
prologue, at the end of its K loop and at its end (its stores acknowledged),
the shader clock cycles of its K loop and of its whole run, its XCD id and its
HW_ID (CU, shader engine) -- one 8-word record per workgroup into a buffer
that ``hcg_stamps_set`` names.  ``run`` drives a workload through that
library in the sustained state (after ``warm_s`` of back-to-back launches) and
``breakdown`` reduces the last launch's records:

* ``span_us``: first workgroup start to last workgroup end; ``events_us``
  the same launch timed by HIP events around it, so the difference is the
  dispatch's own start and end;
* per workgroup (mean, min, max): ``prologue_us``, ``k_loop_us``,
  ``epilogue_us`` and ``k_loop_cycles``;
* per XCD: workgroups, mean shader clock (cycles over constant-clock time),
  first start and last end relative to the launch's first start;
* ``cu_rounds``: workgroups per CU in sequence and the mean gap between
  one's end and the next one's start on the same CU;
* ``gap_after_previous_launch_us``: from the previous launch's last
  workgroup end to this launch's first workgroup start (launches alternate
  between two record areas), and ``launch_period_us`` between their starts.

The product library never carries this code; only ``bench.py --stamps``
loads the stamps library (in its own process).
"""

from __future__ import annotations

import ctypes
import os
import time
from typing import Any

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhcg_gfx950_stamps.so")
WORDS = 8
REALTIME_HZ = 100e6


def load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run 5_amd/csrc/build.py")
    import torch  # noqa: F401  (one HIP runtime with torch)

    lib = ctypes.CDLL(LIB_PATH)
    i64, vp, c_int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    lib.hcg_gemm_algo.argtypes = [c_int, c_int, vp, i64, vp, i64, vp, i64, i64, i64, i64, vp]
    lib.hcg_gemm_algo.restype = c_int
    lib.hcg_stamps_set.argtypes = [vp, i64]
    lib.hcg_stamps_set.restype = c_int
    lib.hcg_last_error.argtypes = []
    lib.hcg_last_error.restype = ctypes.c_char_p
    return lib


def _stats(x: np.ndarray) -> dict[str, float]:
    return {"mean": float(np.mean(x)), "min": float(np.min(x)), "max": float(np.max(x))}


def breakdown(records: np.ndarray) -> dict[str, Any]:
    """Reduce (workgroups, 8) uint64 records (unwritten rows all zero)."""
    rec = records[records[:, 3] != 0].astype(np.int64)
    if rec.size == 0:
        return {"workgroups": 0}
    t0, t1, t2, t3 = (rec[:, i] for i in range(4))
    base = int(t0.min())
    us = 1e6 / REALTIME_HZ
    out: dict[str, Any] = {
        "workgroups": int(rec.shape[0]),
        "span_us": float((t3.max() - base) * us),
        "prologue_us": _stats((t1 - t0) * us),
        "k_loop_us": _stats((t2 - t1) * us),
        "epilogue_us": _stats((t3 - t2) * us),
        "k_loop_cycles": _stats(rec[:, 4]),
        "start_spread_us": None,
    }
    xcc = rec[:, 6] & 0xF  # (bits 47:8 the grid size, bit 48 the record slot)
    clock = rec[:, 5] / np.maximum(t3 - t0, 1) * REALTIME_HZ / 1e6
    per_xcd = []
    for x in sorted(set(int(v) for v in xcc)):
        sel = xcc == x
        per_xcd.append({
            "xcd": x,
            "workgroups": int(sel.sum()),
            "clock_mhz": float(np.mean(clock[sel])),
            "first_start_us": float((t0[sel].min() - base) * us),
            "last_end_us": float((t3[sel].max() - base) * us),
            "k_loop_us_mean": float(np.mean((t2 - t1)[sel]) * us),
        })
    out["per_xcd"] = per_xcd
    ends = [d["last_end_us"] for d in per_xcd]
    out["xcd_end_spread_us"] = float(max(ends) - min(ends))
    # CU identity: XCD and HW_ID bits 15:8 (CU, SH and SE ids).
    cu = (xcc << 8) | ((rec[:, 7] >> 8) & 0xFF)
    counts: dict[int, list[int]] = {}
    for i, key in enumerate(cu.tolist()):
        counts.setdefault(key, []).append(i)
    rounds = [len(v) for v in counts.values()]
    gaps = []
    for idx in counts.values():
        order = sorted(idx, key=lambda i: t0[i])
        gaps.extend(float((t0[b] - t3[a]) * us) for a, b in zip(order, order[1:]))
    out["cu_rounds"] = {"cus": len(counts), "max_per_cu": max(rounds), "min_per_cu": min(rounds),
                        "mean_gap_us": float(np.mean(gaps)) if gaps else None}
    first_round = [min(idx, key=lambda i: t0[i]) for idx in counts.values()]
    out["start_spread_us"] = float((max(t0[i] for i in first_round) - base) * us)
    return out


def split_launches(buffer: np.ndarray) -> list[tuple[np.ndarray, np.ndarray]]:
    """The (records, workgroup indices) of the launches in a stamps buffer,
    earlier launch first.  Consecutive launches alternate between two record
    areas: record b of slot s sits at s * grid + b, and word 6 carries the
    slot (bit 48) and the grid size (bits 47:8); unwritten records are zero.
    The later launch is the one whose workgroups end last."""
    index = np.nonzero(buffer[:, 3])[0]
    recs = buffer[index]
    slot = (recs[:, 6] >> np.uint64(48)) & np.uint64(1)
    grid = (recs[:, 6] >> np.uint64(8)) & np.uint64((1 << 40) - 1)
    wg = index.astype(np.int64) - (slot * grid).astype(np.int64)
    areas = [(recs[slot == s], wg[slot == s]) for s in (0, 1)]
    areas = [a for a in areas if a[0].size]
    areas.sort(key=lambda a: int(a[0][:, 3].max()))
    return areas


def run(torch: Any, cfg_name: str, *, warm_s: float = 0.3, copies: int = 1, algo: int = 0,
        records: int = 1 << 16, lda: int = 0, ldb: int = 0, ldc: int = 0, m: int | None = None,
        n: int | None = None, k: int | None = None, raw: bool = False) -> dict[str, Any]:
    """Sustained launches of a workload through the stamps library; the
    breakdown of the last one.  ``copies`` > 1 rotates A and B over that many
    copies (operands streamed from HBM rather than the Infinity Cache);
    ``lda``/``ldb``/``ldc`` > 0 place the operands in rows of that many
    elements (views of wider buffers) instead of tight rows; ``m``/``n``/``k``
    change the workload's extents (its input recipe kept); ``raw`` adds the
    last launch's records as ``records`` (workgroup index -> 8 words)."""
    from .workloads import CONFIGS, make_inputs, to_torch

    cfg = CONFIGS[cfg_name]
    lib = load()
    dev = torch.device("cuda", torch.cuda.current_device())
    a, b = make_inputs(cfg, seed=0, m=m, n=n, k=k)
    mm, kk = a.shape
    nn = b.shape[1]

    def placed(t: Any, ld: int) -> Any:
        if ld <= 0:
            return t
        buf = torch.zeros((t.shape[0], ld), dtype=t.dtype, device=dev)
        buf[:, : t.shape[1]] = t
        return buf[:, : t.shape[1]]

    tas = [placed(to_torch(a, cfg.dtype, dev), lda) for _ in range(copies)]
    tbs = [placed(to_torch(b, cfg.dtype, dev), ldb) for _ in range(copies)]
    tc = placed(torch.empty((mm, nn), dtype=torch.float32, device=dev), ldc)
    buf = torch.zeros(records * WORDS, dtype=torch.int64, device=dev)
    code = 0 if cfg.dtype == "float16" else 1
    stream = torch.cuda.current_stream(dev)

    def launch(i: int) -> None:
        ta, tb = tas[i % copies], tbs[i % copies]
        rc = lib.hcg_gemm_algo(algo, code, ta.data_ptr(), ta.stride(0), tb.data_ptr(), tb.stride(0), tc.data_ptr(),
                               tc.stride(0), mm, nn, kk, stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"hcg_gemm_algo failed ({rc}): {lib.hcg_last_error().decode()}")

    if lib.hcg_stamps_set(buf.data_ptr(), records) != 0:
        raise RuntimeError(lib.hcg_last_error().decode())
    try:
        i = 0
        t_end = time.perf_counter() + warm_s
        while time.perf_counter() < t_end:
            for _ in range(10):
                launch(i)
                i += 1
            torch.cuda.synchronize()
        buf.zero_()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(9):
            launch(i)
            i += 1
        start.record(stream)
        launch(i)
        end.record(stream)
        torch.cuda.synchronize()
    finally:
        lib.hcg_stamps_set(None, 0)
    recs = buf.view(records, WORDS).cpu().numpy().view(np.uint64)
    launches = split_launches(recs)
    last, last_wg = launches[-1]
    out = breakdown(last)
    if len(launches) == 2:
        prev = launches[0][0]
        us = 1e6 / REALTIME_HZ
        p_end, l_start, p_start = int(prev[:, 3].max()), int(last[:, 0].min()), int(prev[:, 0].min())
        out["gap_after_previous_launch_us"] = (l_start - p_end) * us
        out["previous_launch_span_us"] = (p_end - p_start) * us
        out["launch_period_us"] = (l_start - p_start) * us
    out["events_us"] = start.elapsed_time(end) * 1e3
    if raw:
        out["records"] = {int(b): [int(x) for x in r] for b, r in zip(last_wg, last)}
    out["workload"] = cfg_name
    out["operand_copies"] = copies
    out["ld"] = [tas[0].stride(0), tbs[0].stride(0), tc.stride(0)]
    out["shape"] = [mm, nn, kk]
    out["k_steps_of_32"] = -(-kk // 32)
    return out
