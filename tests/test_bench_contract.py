"""bench.py's contract on the CPU: more than one GPU is refused with a
message before any device work, a machine without a GPU gets a clear error,
and the committed profiles/ summaries carry the per-launch traffic figure
that the JSON line's roofline.traffic reads."""

from __future__ import annotations

import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _bench_module():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    assert spec.loader is not None
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused_with_a_message():
    out = subprocess.run([sys.executable, BENCH, "--gpus", "2", "--steps", "3"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 2
    assert "--gpus 2 is not supported" in out.stderr and "one MI355X" in out.stderr
    assert out.stdout == ""


def test_without_a_gpu_the_bench_says_so():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    out = subprocess.run([sys.executable, BENCH, "--steps", "3"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 1 and "needs a GPU" in out.stderr


@pytest.mark.parametrize("kernel,workload", [("gemm_dma_kernel", "c2_4096_f16"), ("gemm_dma_kernel", "c3_8192_bf16"),
                                             ("gemm_stream_kernel", "c4_skinny_f16"),
                                             ("gemm_dma_kernel", "c5_ragged_f16")])
def test_committed_profiles_give_the_traffic_per_launch(kernel, workload):
    bench = _bench_module()
    traffic, source = bench.measured_traffic(kernel, workload)
    assert source == os.path.join("profiles", f"{kernel}_{workload}.md")
    from hc.gfx950.workloads import CONFIGS

    # Traffic is at least the algorithmic bytes (the L2s re-read operands)
    # and at most a few times them.
    algorithmic = CONFIGS[workload].algorithmic_bytes
    assert algorithmic <= traffic <= 4 * algorithmic
