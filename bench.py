"""Benchmark of the hc GEMM hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                    [--no-cpu-baseline] [--no-extra]

A step is one launch of the GEMM C = A @ B over the workload's synthetic
inputs (already resident in HBM).  The headline workload is BASELINE.json's
metric configuration, fp16 M=N=K=4096; ``value`` is TFLOP/s
(2*M*N*K per step).  One JSON line is printed with:

* ``roofline``: the dominant kernel's algorithmic flops per launch divided by
  its average launch time (HIP events on the launch stream, over the timed
  region), against MI355X's dense fp16 MFMA peak (2516.6 TFLOP/s = 256 CUs x
  2.4 GHz x 4096 flop/clk/CU);
* ``cpu_baseline``: the C oracle (the reference simulator's float32 fold,
  restated; OpenMP) timed on this host on a bounded sample of rows of the
  same workload (kind "port");
* ``skinny``: the M=16 decode-shaped GEMM in GB/s of algorithmic
  bytes against the 8 TB/s HBM peak, timed while rotating through enough
  copies of B that every launch streams B from HBM, not from the 256 MB
  Infinity Cache (warm, same-buffer numbers are reported beside it);
* ``others``: the remaining BASELINE.json configurations, TFLOP/s, each
  also ``cold``: A and B rotated over copies larger than the Infinity Cache
  (``cold`` at the top level is the headline workload's; ``value`` is the
  warm figure, the same operands every launch);
* ``board``: graphics (per XCD too) and memory clocks and socket power
  sampled from the driver while the headline workload runs;
* ``ceiling``: what this board sustains, measured in the same run by the
  probes of libhcg_probe.so (include/hcg_probe.h): pure MFMA issue (TFLOP/s
  and shader clock), streaming HBM read and write (GB/s); ``roofline``,
  ``skinny`` and each of ``others`` (warm and cold; against the MFMA ceiling
  of its input type) carry ``frac_of_ceiling`` beside ``frac`` (which stays
  against the 2516.6 TFLOP/s and 8 TB/s nameplate peaks).

``--ceilings-only`` runs just the probes (for rocprofv3).  ``--stamps
WORKLOAD`` runs a workload through the timestamped build of the library and
prints where one sustained launch's time goes (hc/gfx950/stamps.py).
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "5_amd"))

PEAK_F16_TFLOPS = 2516.6  # dense fp16/bf16 MFMA, MI355X
PEAK_HBM_GBS = 8000.0
METRIC = "TFLOP/s + % MFMA fp16 peak at 4096³ GEMM; GB/s at M=16 skinny, 1 MI355X"
MALL_BYTES = 256 * 1024 * 1024
LAST_ENQUEUE_S = [0.0]  # host seconds to enqueue the last timed run of launches


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=400)
    p.add_argument("--min-warm-ms", type=float, default=60.0,
                   help="keep warming up (untimed) until at least this much sustained load has run")
    p.add_argument("--workload", default="c2_4096_f16")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true")
    p.add_argument("--no-ceilings", action="store_true")
    p.add_argument("--ceilings-only", action="store_true", help="run only the hardware ceiling probes")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU time of the baseline sample")
    p.add_argument("--profile-only", action="store_true",
                   help="run only --steps launches of the workload's GEMM (for rocprofv3), print nothing else")
    p.add_argument("--queue-ahead", type=int, default=0, metavar="N",
                   help="with --profile-only: afterwards, hold the GPU in a sleep kernel while N more launches "
                        "are enqueued, so they run back to back even when the host enqueues slower than the GPU "
                        "runs (as under a tracer), and print their event time per launch")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="run 5 device-to-device copies of MIB MiB (calibrates FETCH_SIZE/WRITE_SIZE) and exit")
    p.add_argument("--stamps", metavar="WORKLOAD",
                   help="run WORKLOAD through the timestamped build of the library (libhcg_gfx950_stamps.so) "
                        "and print where its last sustained launch's time goes, per workgroup and per XCD")
    p.add_argument("--stamps-copies", type=int, default=0, metavar="N",
                   help="with --stamps: rotate A and B over N copies (default: 5 for c4_skinny_f16, whose B the "
                        "bench streams from HBM, else 1)")
    return p.parse_args()


def measured_traffic(kernel: str, workload: str) -> tuple[int | None, str | None]:
    """Memory-side bytes per launch from the committed rocprofv3 summary
    profiles/<kernel>_<workload>.md (FETCH_SIZE and WRITE_SIZE runs, each
    scaled by a plain-copy calibration; the L2's traffic to the fabric, of
    which the Infinity Cache may serve part), or (None, None) if absent."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}.md")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1]), os.path.relpath(path, ROOT)
    return None, None


def dtype_short(name: str) -> str:
    return {"float16": "f16", "bfloat16": "bf16"}[name]


WARM_S = 0.06  # overwritten from --min-warm-ms in main()


def time_launches(torch, stream, fn, steps: int, warmup: int) -> tuple[float, float]:
    """(event seconds per launch, host seconds per step) over `steps` launches.

    Before timing: `warmup` launches, then more until WARM_S seconds of
    sustained load have run.  Under a fresh load the board's clock needs
    about 25 ms to settle (a 4096^3 launch takes ~165 us in the first
    milliseconds and ~115 us after), so the timed launches measure the
    sustained state."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    # A collection of Python's cyclic garbage collector can stall the host for
    # tens of ms while the GPU drains its queue and idles: inside the timed
    # enqueue loop the events would time that gap, and between the warm-up
    # and the timed launches the idle board's clock drops and the first timed
    # launches run slow.  So collect before the warm-up and keep the
    # collector off until the timed launches are enqueued.
    gc.collect()
    gc.disable()
    try:
        t_w = time.perf_counter()
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                fn()
        torch.cuda.synchronize()
        while time.perf_counter() - t_w < WARM_S:
            with torch.cuda.stream(stream):
                for _ in range(10):
                    fn()
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            start.record(stream)
            for _ in range(steps):
                fn()
            end.record(stream)
        t_enq = time.perf_counter()
    finally:
        gc.enable()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    LAST_ENQUEUE_S[0] = t_enq - t0
    return start.elapsed_time(end) * 1e-3 / steps, (t1 - t0) / steps


def median_launch(torch, stream, fn, launches: int) -> float:
    """Median seconds of single launches, each bracketed by its own pair of
    HIP events (run after time_launches, so the clock has settled)."""
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(launches)]
    with torch.cuda.stream(stream):
        for start, end in pairs:
            start.record(stream)
            fn()
            end.record(stream)
    torch.cuda.synchronize()
    times = sorted(start.elapsed_time(end) * 1e-3 for start, end in pairs)
    return times[len(times) // 2]


def _smi_handle(amdsmi, torch):
    handles = amdsmi.amdsmi_get_processor_handles()
    if len(handles) == 1:
        return handles[0]
    props = torch.cuda.get_device_properties(0)
    for h in handles:
        bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)  # "dddd:bb:dd.f"
        dom, bus, rest = bdf.split(":")
        if int(dom, 16) == props.pci_domain_id and int(bus, 16) == props.pci_bus_id and int(rest.split(".")[0], 16) == props.pci_device_id:
            return h
    raise RuntimeError("no amdsmi handle matches cuda:0")


def board_state(torch, stream, fn, seconds: float) -> dict:
    """Clocks and power the driver reports while ``fn`` runs back to back.

    The SMU refreshes the gpu_metrics table (read through amdsmi) about once
    a second, so ``seconds`` of launches follow the timed region and a
    thread reads the table every 20 ms; the values reported come from the
    last refresh made at least 1.05 s into the load, whose averaging window
    therefore lies under load.  ``current_gfxclk`` is the SMU's clock
    setting: the effective shader clock under a power limit can be lower
    (compare ``achieved`` with the MFMA rate).  Only reads are made.
    Returns {"error": ...} where amdsmi is unavailable."""
    import threading

    try:
        import amdsmi

        amdsmi.amdsmi_init()
    except Exception as exc:  # reported, never fatal
        return {"error": f"amdsmi unavailable: {exc}"}
    try:
        handle = _smi_handle(amdsmi, torch)
        samples: list[tuple[float, dict]] = []
        errors: list[str] = []
        stop = threading.Event()
        t0 = time.perf_counter()

        def sampler():
            while not stop.is_set():
                try:
                    samples.append((time.perf_counter() - t0, amdsmi.amdsmi_get_gpu_metrics_info(handle)))
                except Exception as exc:
                    errors.append(str(exc))
                    return
                stop.wait(0.02)

        t = threading.Thread(target=sampler, daemon=True)
        t.start()
        with torch.cuda.stream(stream):
            while time.perf_counter() - t0 < seconds:
                for _ in range(20):
                    fn()
                stream.synchronize()
        stop.set()
        t.join(timeout=5)
        if not samples:
            return {"error": errors[0] if errors else "no gpu_metrics sample"}
        first_ts = samples[0][1].get("firmware_timestamp")
        under_load = [m for ts, m in samples if ts >= 1.05 and m.get("firmware_timestamp") != first_ts]
        pick = under_load[-1] if under_load else samples[-1][1]

        def num(x):
            return x if isinstance(x, (int, float)) and not isinstance(x, bool) and x < 0xFFFF else None

        xcd = pick.get("current_gfxclks")
        out = {
            "sclk_mhz": num(pick.get("current_gfxclk")),
            "sclk_per_xcd_mhz": [num(v) for v in xcd] if isinstance(xcd, (list, tuple)) else None,
            "mclk_mhz": num(pick.get("current_uclk")),
            "socket_power_w": num(pick.get("current_socket_power")),
            "gfx_activity_pct": num(pick.get("average_gfx_activity")),
            "under_load": bool(under_load),
            "method": (f"amdsmi gpu_metrics (SMU-reported, refreshed ~1/s) read every 20 ms over {seconds:.1f} s of "
                       "back-to-back launches after the timed region; last refresh >= 1.05 s into the load"),
        }
        if errors:
            out["error"] = errors[0]
        return out
    except Exception as exc:
        return {"error": f"amdsmi query failed: {exc}"}
    finally:
        try:
            amdsmi.amdsmi_shut_down()
        except Exception:
            pass


def cpu_baseline(cfg, a, b, target_s: float) -> dict:
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import hc_oracle

    threads = hc_oracle.default_threads()
    dt = hc_oracle.F16 if cfg.dtype == "float16" else hc_oracle.BF16
    rows = 16
    elapsed = 0.0
    while True:
        idx = np.arange(rows, dtype=np.int64)
        t0 = time.perf_counter()
        hc_oracle.gemm_c_rows(a, b, idx, dt, threads=threads)
        elapsed = time.perf_counter() - t0
        if elapsed >= target_s / 4 or rows >= cfg.m:
            break
        rows = min(cfg.m, max(rows * 2, int(rows * (target_s / 4) / max(elapsed, 1e-3))))
    # The timed sample: rows near the target size, repeated when even all
    # rows of the workload finish well inside the target time.
    rows = min(cfg.m, max(16, int(rows * target_s / max(elapsed, 1e-3) / 2)))
    reps = 1
    if rows == cfg.m and elapsed * rows / max(1, len(idx)) < target_s / 2:
        reps = max(1, int(target_s / max(elapsed * rows / len(idx), 1e-3)))
    idx = np.arange(rows, dtype=np.int64)
    t0 = time.perf_counter()
    for _ in range(reps):
        hc_oracle.gemm_c_rows(a, b, idx, dt, threads=threads)
    elapsed = time.perf_counter() - t0
    flops = 2.0 * rows * cfg.n * cfg.k * reps
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"rows 0..{rows - 1} of {cfg.name} ({rows}x{cfg.n}x{cfg.k}) x {reps}, {elapsed:.1f} s, "
        f"C oracle (sequential fp32 fold, OpenMP over row blocks) on {os.cpu_count()} host CPUs",
        "single_thread": single_thread_baseline(cfg, a, b, dt),
        "simulator_shape": simulator_shape_baseline(cfg),
    }


def single_thread_baseline(cfg, a, b, dt) -> dict:
    """The same C oracle on one host thread, over a fixed sample of 256 rows
    (about 2 s on these hosts)."""
    import numpy as np

    import hc_oracle

    rows = min(cfg.m, 256)
    idx = np.arange(rows, dtype=np.int64)
    t0 = time.perf_counter()
    hc_oracle.gemm_c_rows(a, b, idx, dt, threads=1)
    elapsed = time.perf_counter() - t0
    return {
        "value": 2.0 * rows * cfg.n * cfg.k / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "sample": f"rows 0..{rows - 1} of {cfg.name} ({rows}x{cfg.n}x{cfg.k}), {elapsed:.2f} s",
    }


def simulator_shape_baseline(cfg) -> dict:
    """The reference's own CPU path shape: per-lane NumPy scalar MACs.

    Times hc_oracle.simulate_lane_structure (one Python-level float32 MAC per
    lane, row and k, workgroup by workgroup, as hc.simulator executes the
    kernel's fallback bodies) on the 128^3 configuration, on one core, and
    projects that rate linearly to the headline workload.
    """
    import hc_oracle
    from hc.gfx950.workloads import make_inputs

    a, b = make_inputs("c1_128_f16", seed=0)
    t0 = time.perf_counter()
    hc_oracle.simulate_lane_structure(a, b)
    elapsed = time.perf_counter() - t0
    rate = 2.0 * 128**3 / elapsed
    return {
        "value": rate / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "sample": f"c1_128_f16 (128x128x128) in {elapsed:.2f} s, Python per-lane float32 MACs",
        "projected_headline_s": 2.0 * cfg.m * cfg.n * cfg.k / rate,
    }


def bench_skinny(torch, g, stream, steps: int, warmup: int) -> dict:
    from hc.gfx950.workloads import CONFIGS, make_inputs, to_torch

    cfg = CONFIGS["c4_skinny_f16"]
    dev = torch.device("cuda", 0)
    a, b = make_inputs(cfg, seed=0)
    ta = to_torch(a, cfg.dtype, dev)
    tb0 = to_torch(b, cfg.dtype, dev)
    copies = max(3, math.ceil(2 * MALL_BYTES / tb0.numel() / 2) + 1)
    tbs = [tb0] + [tb0.clone() for _ in range(copies - 1)]
    tc = torch.empty((cfg.m, cfg.n), dtype=torch.float32, device=dev)
    it = {"i": 0}

    def rotating():
        tb = tbs[it["i"] % copies]
        it["i"] += 1
        g.gemm(ta, tb, out=tc, algo="skinny")

    cold, _ = time_launches(torch, stream, rotating, steps, warmup)
    warm, _ = time_launches(torch, stream, lambda: g.gemm(ta, tb0, out=tc, algo="skinny"), steps, warmup)
    gbs = cfg.algorithmic_bytes / cold / 1e9
    return {
        "workload": cfg.name,
        "M": cfg.m,
        "N": cfg.n,
        "K": cfg.k,
        "value": gbs,
        "unit": "GB/s",
        "us_per_launch": cold * 1e6,
        "frac_hbm_peak": gbs / PEAK_HBM_GBS,
        "algorithmic_bytes": cfg.algorithmic_bytes,
        "b_copies_rotated": copies,
        "warm_same_buffer_GBs": cfg.algorithmic_bytes / warm / 1e9,
        "note": "time per launch includes the split-K reduce kernel",
    }


def first_use(torch, g, stream) -> dict:
    """Cost per call of the small C1 GEMM (128^3 fp16) from the first call
    of this process on: the first call (it loads the library's code object
    onto the GPU), then calls 2-100 and 101-1000, each block enqueued back
    to back and timed on the host up to a synchronize.  Runs before any
    other GEMM of the process."""
    from hc.gfx950.workloads import CONFIGS, make_inputs, to_torch

    cfg = CONFIGS["c1_128_f16"]
    dev = torch.device("cuda", 0)
    a, b = make_inputs(cfg, seed=0)
    ta, tb = to_torch(a, cfg.dtype, dev), to_torch(b, cfg.dtype, dev)
    tc = torch.empty((cfg.m, cfg.n), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    out = {}
    with torch.cuda.stream(stream):
        for label, count in (("first_call_ms", 1), ("calls_2_100_us", 99), ("calls_101_1000_us", 900)):
            t0 = time.perf_counter()
            for _ in range(count):
                g.gemm(ta, tb, out=tc)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            out[label] = dt * 1e3 if count == 1 else dt / count * 1e6
    out["method"] = ("fresh process; host time per call of hc.gfx950.gemm on device tensors, blocks of calls "
                     "enqueued back to back up to a synchronize")
    return out


def bench_cold(torch, g, stream, name: str, steps: int, warmup: int) -> dict:
    """Event time per launch with A and B rotated over copies that total at
    least twice the 256 MB Infinity Cache, so every launch reads its operands
    from HBM (the warm figures reuse one pair of operands, which then stays
    in the Infinity Cache when it fits)."""
    from hc.gfx950.workloads import CONFIGS, make_inputs, to_torch

    cfg = CONFIGS[name]
    dev = torch.device("cuda", 0)
    a, b = make_inputs(cfg, seed=0)
    ta0, tb0 = to_torch(a, cfg.dtype, dev), to_torch(b, cfg.dtype, dev)
    pair = 2 * (ta0.numel() + tb0.numel())
    copies = max(2, math.ceil(2 * MALL_BYTES / pair))
    tas = [ta0] + [ta0.clone() for _ in range(copies - 1)]
    tbs = [tb0] + [tb0.clone() for _ in range(copies - 1)]
    tc = torch.empty((cfg.m, cfg.n), dtype=torch.float32, device=dev)
    it = {"i": 0}

    def rotating():
        i = it["i"] % copies
        it["i"] += 1
        g.gemm(tas[i], tbs[i], out=tc)

    t, _ = time_launches(torch, stream, rotating, steps, warmup)
    del tas, tbs
    return {"value": cfg.flops / t / 1e12, "unit": "TFLOP/s", "us_per_launch": t * 1e6, "operand_copies": copies,
            "operand_bytes_rotated": copies * pair}


def bench_config(torch, g, stream, name: str, steps: int, warmup: int) -> dict:
    from hc.gfx950.workloads import CONFIGS, make_inputs, to_torch

    cfg = CONFIGS[name]
    dev = torch.device("cuda", 0)
    a, b = make_inputs(cfg, seed=0)
    ta, tb = to_torch(a, cfg.dtype, dev), to_torch(b, cfg.dtype, dev)
    tc = torch.empty((cfg.m, cfg.n), dtype=torch.float32, device=dev)
    t, _ = time_launches(torch, stream, lambda: g.gemm(ta, tb, out=tc), steps, warmup)
    tf = cfg.flops / t / 1e12
    return {"value": tf, "unit": "TFLOP/s", "us_per_launch": t * 1e6, "frac_peak": tf / PEAK_F16_TFLOPS}


def main() -> int:
    args = parse_args()
    global WARM_S
    WARM_S = max(0.0, args.min_warm_ms) / 1e3
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X; "
            "the GEMM would shard by N or M with no exchange, and no multi-GPU run is part of this build",
            file=sys.stderr,
        )
        return 2
    import torch

    import hc.gfx950 as g
    from hc.gfx950.workloads import CONFIGS, make_inputs, to_torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    # The process's first full garbage collection after torch is imported
    # scans ~170k objects and stops the host for 40-50 ms a few hundred calls
    # in, while the GPU idles.  Collect once now and freeze what survives (the
    # imported modules and their data, which live as long as the process), so
    # no later collection rescans them.  The library leaves this to its caller.
    gc.collect()
    gc.freeze()
    cfg = CONFIGS[args.workload]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.stamps:
        from hc.gfx950 import stamps

        name = args.stamps
        copies = args.stamps_copies or (5 if name == "c4_skinny_f16" else 1)
        log(f"stamps: {name}, operands rotated over {copies} cop{'y' if copies == 1 else 'ies'}")
        out = stamps.run(torch, name, copies=copies, warm_s=max(0.3, WARM_S), algo=2 if name == "c4_skinny_f16" else 0)
        print(json.dumps({"stamps": out}), flush=True)
        return 0
    stream = torch.cuda.Stream(device=dev)
    if args.copy_probe:
        n = args.copy_probe * 1024 * 1024 // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 5 x {args.copy_probe} MiB device-to-device")
        return 0
    if args.ceilings_only:
        from hc.gfx950 import probe

        print(json.dumps({"ceiling": probe.ceilings(torch, stream)}), flush=True)
        return 0
    if args.profile_only:
        a, b = make_inputs(cfg, seed=0)
        ta, tb = to_torch(a, cfg.dtype, dev), to_torch(b, cfg.dtype, dev)
        tc = torch.empty((cfg.m, cfg.n), dtype=torch.float32, device=dev)
        # HBM-bound shapes rotate over copies of B larger than the Infinity
        # Cache in total, as in the timed benchmark.
        tbs = [tb]
        if cfg.m <= 16:
            copies = max(3, math.ceil(2 * MALL_BYTES / tb.numel() / 2) + 1)
            tbs += [tb.clone() for _ in range(copies - 1)]
        with torch.cuda.stream(stream):
            for i in range(args.steps):
                g.gemm(ta, tbs[i % len(tbs)], out=tc)
        torch.cuda.synchronize()
        log(f"profile-only: {args.steps} launches of {cfg.name}")
        if args.queue_ahead > 0:
            # 200 us of sleep per launch to enqueue (a kernel tracer's host
            # cost per launch is far below that), counted in shader cycles at
            # 2.4 GHz, the highest clock: the sleep lasts at least that long.
            n = args.queue_ahead
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                torch.cuda._sleep(int(n * 200e-6 * 2.4e9))
                start.record(stream)
                for i in range(n):
                    g.gemm(ta, tbs[i % len(tbs)], out=tc)
                end.record(stream)
            torch.cuda.synchronize()
            log(f"queued ahead: {n} launches of {cfg.name}, events {start.elapsed_time(end) * 1e3 / n:.2f} us per launch")
        return 0
    log(f"bench: {torch.cuda.get_device_name(0)}, workload {cfg.name}")
    fresh = first_use(torch, g, stream) if not args.no_extra else None

    a, b = make_inputs(cfg, seed=0)
    ta, tb = to_torch(a, cfg.dtype, dev), to_torch(b, cfg.dtype, dev)
    tc = torch.empty((cfg.m, cfg.n), dtype=torch.float32, device=dev)

    def step():
        g.gemm(ta, tb, out=tc)

    per_launch, host_per_step = time_launches(torch, stream, step, args.steps, args.warmup)
    tflops = cfg.flops / per_launch / 1e12
    enqueue_s = LAST_ENQUEUE_S[0]
    log(f"bench: {cfg.name}: {per_launch * 1e6:.1f} us/launch, {tflops:.1f} TFLOP/s "
        f"(host enqueue of the {args.steps} launches: {enqueue_s * 1e3:.2f} ms)")
    is_skinny = cfg.m <= 16
    kernel_name = "gemm_stream_kernel" if is_skinny else "gemm_dma_kernel"
    if is_skinny:
        achieved = cfg.algorithmic_bytes / per_launch / 1e9
        roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": achieved / PEAK_HBM_GBS, "traffic": None}
    else:
        roofline = {"bound": "mfma", "achieved": tflops, "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                    "frac": tflops / PEAK_F16_TFLOPS, "traffic": None}
    roofline["kernel"] = kernel_name
    roofline["traffic"], roofline["traffic_source"] = measured_traffic(kernel_name, cfg.name)
    roofline["per_launch_us"] = per_launch * 1e6
    roofline["median_single_launch_us"] = median_launch(torch, stream, step, 200) * 1e6
    roofline["timing"] = ("warm: the same A and B every launch" if not is_skinny else
                          "cold: B rotated over copies larger than the Infinity Cache")
    roofline["algorithmic_per_launch"] = cfg.algorithmic_bytes if is_skinny else cfg.flops

    result = {
        "metric": METRIC,
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "min_warm_ms": args.min_warm_ms,
        "ms_per_step": host_per_step * 1e3,
        "host_enqueue_ms": enqueue_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_short(cfg.dtype),
        "data": "synthetic",
        "config": {
            "workload": cfg.name,
            "M": cfg.m,
            "N": cfg.n,
            "K": cfg.k,
            "inputs": f"{cfg.dtype}, A~{cfg.a_dist}, B~{cfg.b_dist}, seed 0",
            "accumulate": "f32",
            "output": "f32",
            "layout": "row-major A (MxK), B (KxN), C (MxN)",
        },
        "pct_mfma_fp16_peak": 100.0 * tflops / PEAK_F16_TFLOPS,
        "roofline": roofline,
        "board": board_state(torch, stream, step, 2.5),
    }
    del ta, tb, tc
    if not args.no_extra and not is_skinny and cfg.flops >= 1e9:  # (a launch-bound 128^3 GEMM has no cold case)
        log(f"bench: {cfg.name} cold (operands rotated)")
        cold = bench_cold(torch, g, stream, cfg.name, args.steps, args.warmup)
        cold["note"] = "value uses the warm figure; this one reads A and B from HBM on every launch"
        result["cold"] = cold
    if not args.no_extra:
        log("bench: skinny M=16 (rotating B buffers)")
        result["skinny"] = bench_skinny(torch, g, stream, max(20, args.steps), max(5, args.warmup // 2))
        others = {}
        for name in CONFIGS:
            if name in (cfg.name, "c4_skinny_f16"):
                continue
            log(f"bench: {name}")
            others[name] = bench_config(torch, g, stream, name, max(20, args.steps // 4), 5)
            if name != "c1_128_f16":
                others[name]["cold"] = bench_cold(torch, g, stream, name, max(20, args.steps // 4), 5)
        result["others"] = others
    if fresh is not None:
        result["first_use"] = fresh
    if not args.no_ceilings:
        log("bench: hardware ceilings (probes)")
        from hc.gfx950 import probe

        ceiling = probe.ceilings(torch, stream)
        result["ceiling"] = ceiling
        key, unit_key = ("hbm_read_128mib", "gbs") if is_skinny else ("mfma_f16", "tflops")
        roofline["frac_of_ceiling"] = roofline["achieved"] / ceiling[key][unit_key]
        roofline["ceiling_source"] = f"ceiling.{key}"
        if "skinny" in result:
            sk = result["skinny"]
            sk["frac_of_ceiling"] = sk["value"] / ceiling["hbm_read_128mib"]["gbs"]
            sk["ceiling_source"] = "ceiling.hbm_read_128mib"
        # The other compute-bound workloads against the same board's MFMA
        # ceiling of their input type.
        for name, other in result.get("others", {}).items():
            mkey = "mfma_bf16" if CONFIGS[name].dtype == "bfloat16" else "mfma_f16"
            for entry in (other, other.get("cold")):
                if entry:
                    entry["frac_of_ceiling"] = entry["value"] / ceiling[mkey]["tflops"]
                    entry["ceiling_source"] = f"ceiling.{mkey}"
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle)")
        result["cpu_baseline"] = cpu_baseline(cfg, a, b, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
