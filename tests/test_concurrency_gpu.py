"""Launches from several host threads, and HIP-graph capture and replay.

The reference runs concurrent launches from two threads
(tests/test_simulator.py:1113-1125); here each thread drives its own stream
through the C ABI.  Graph capture: the kernels take no host-side action
inside a launch except on a stream's first use of a workspace size (an
allocation), so after one warm-up call on the capture stream every path --
tiled, skinny split-K (workspace partials + reduce), tiled split-K, ragged
operands read in place, the narrow kernel (split partials), a peeled shape
(tiled bulk + streaming remainder, two launches sharing the workspace),
unaligned B rows and odd K on the streaming kernels -- records into a
graph; and, in a process that turns in-place reads of unaligned rows off,
so do the repack kernel and the register-staged streaming forms.  Every
replay is checked against the eager result, with eager work between
replays.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

import hc_oracle as oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DEV = "cuda:0"


def _dev(x, dtype="float16"):
    from hc.gfx950.workloads import to_torch

    return to_torch(x, dtype, torch.device(DEV))


CASES = [
    ("tiled", 1024, 768, 512),
    ("skinny", 16, 4096, 4096),
    ("ragged", 1000, 601, 333),
    ("splitk", 512, 512, 16384),
    ("narrow", 2048, 13, 4096),
    ("peel", 4111, 4096, 1024),
    ("unaligned_b", 16, 8191, 4096),
    ("odd_k_narrow", 4096, 40, 4095),
]


def _inputs(name, m, n, k, seed):
    from hc.gfx950.workloads import make_inputs

    cfg = "c4_skinny_f16" if name in ("skinny", "unaligned_b") else "c2_4096_f16"
    return make_inputs(cfg, seed=seed, m=m, n=n, k=k)


def test_two_host_threads_each_with_a_stream():
    import hc.gfx950 as g

    jobs = []
    for i, (name, m, n, k) in enumerate(CASES * 2):
        a, b = _inputs(name, m, n, k, seed=100 + i)
        jobs.append((a, b, _dev(a), _dev(b), torch.empty((m, n), dtype=torch.float32, device=DEV)))
    errors = []
    barrier = threading.Barrier(2)

    def worker(part):
        try:
            s = torch.cuda.Stream(device=DEV)
            barrier.wait()
            with torch.cuda.stream(s):
                for _ in range(5):
                    for _, _, ta, tb, tc in part:
                        g.gemm(ta, tb, out=tc)
            s.synchronize()
        except Exception as exc:  # surfaced below
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(jobs[i::2],)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for a, b, _, _, tc in jobs:
        rep = oracle.parity_check(tc.cpu().numpy(), oracle.gemm_c(a, b), a.shape[1])
        assert rep.ok, str(rep)


def test_two_host_threads_sharing_one_stream():
    """Both threads enqueue onto one stream, alternating shapes whose
    library workspaces differ in size, so a call can find the stream's buffer
    too small and replace it while the other thread's call is between taking
    that buffer and launching on it (the library's workspace lock covers both)."""
    import hc.gfx950 as g

    shapes = [("skinny", 16, 2048, 2048), ("splitk", 512, 512, 16384), ("narrow", 2048, 13, 4096),
              ("ragged", 1000, 601, 333), ("splitk", 768, 768, 12288)]
    jobs = []
    for i, (name, m, n, k) in enumerate(shapes * 2):
        a, b = _inputs(name, m, n, k, seed=300 + i)
        jobs.append((a, b, _dev(a), _dev(b), torch.empty((m, n), dtype=torch.float32, device=DEV)))
    shared = torch.cuda.Stream(device=DEV)
    errors = []
    barrier = threading.Barrier(2)

    def worker(part):
        try:
            barrier.wait()
            with torch.cuda.stream(shared):
                for _ in range(10):
                    for _, _, ta, tb, tc in part:
                        g.gemm(ta, tb, out=tc)
        except Exception as exc:  # surfaced below
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(jobs[i::2],)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    shared.synchronize()
    assert not errors, errors
    for a, b, _, _, tc in jobs:
        rep = oracle.parity_check(tc.cpu().numpy(), oracle.gemm_c(a, b), a.shape[1])
        assert rep.ok, str(rep)


@pytest.mark.parametrize("name,m,n,k", CASES)
def test_graph_capture_replays_match_eager(name, m, n, k):
    import hc.gfx950 as g

    a, b = _inputs(name, m, n, k, seed=7)
    ta, tb = _dev(a), _dev(b)
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    s = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(s):
        g.gemm(ta, tb, out=out)  # warm-up: allocates this stream's workspace if the path needs one
    s.synchronize()
    eager = out.clone()
    rep = oracle.parity_check(eager.cpu().numpy(), oracle.gemm_c(a, b), k)
    assert rep.ok, str(rep)
    print(f"case graph {name} m={m} n={n} k={k}", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        g.gemm(ta, tb, out=out)
    # Eager calls with other operands on the capturing stream, issued so
    # that they can overlap the replays (which run on the current stream):
    # they must not share the scratch the graph holds.
    a2, b2 = _inputs(name, m, n, k, seed=8)
    ta2, tb2 = _dev(a2), _dev(b2)
    want2 = oracle.gemm_c(a2, b2)
    outs2 = []
    for i in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            outs2.append(g.gemm(ta2, tb2))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
    for i, o in enumerate(outs2):
        rep = oracle.parity_check(o.cpu().numpy(), want2, k)
        assert rep.ok, f"eager call {i}: {rep}"


def test_graph_capture_of_the_repack_and_register_staged_paths():
    """With HCG_UNALIGNED_DMA=0 (a fresh process: the library reads it
    once) unaligned rows take the fallback paths: A and B repacked into the
    workspace before the tiled kernel, B register-staged in the streaming
    kernel, A register-staged and B repacked in the narrow kernel.  Each is
    captured after a warm-up call and replayed, with eager calls on other
    operands on the capturing stream between replays."""
    import os
    import subprocess
    import sys
    import textwrap

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{os.path.join(root, "5_amd")!r}, {os.path.join(root, "oracle")!r}]
        import torch
        import hc.gfx950 as g, hc_oracle as oracle
        from hc.gfx950.workloads import make_inputs, to_torch
        dev = torch.device("cuda:0")
        for name, m, n, k in [("repacked", 1000, 601, 333), ("staged_b", 16, 8191, 4096),
                              ("staged_a", 4096, 13, 4095), ("narrow_repacked_b", 2048, 40, 4095)]:
            print("case graph fallback", name, m, n, k, flush=True)
            a, b = make_inputs("c2_4096_f16", seed=7, m=m, n=n, k=k)
            ta, tb = to_torch(a, "float16", dev), to_torch(b, "float16", dev)
            out = torch.empty((m, n), dtype=torch.float32, device=dev)
            s = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(s):
                g.gemm(ta, tb, out=out)
            s.synchronize()
            eager = out.clone()
            assert oracle.parity_check(eager.cpu().numpy(), oracle.gemm_c(a, b), k).ok, name
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                g.gemm(ta, tb, out=out)
            a2, b2 = make_inputs("c2_4096_f16", seed=8, m=m, n=n, k=k)
            ta2, tb2 = to_torch(a2, "float16", dev), to_torch(b2, "float16", dev)
            want2 = oracle.gemm_c(a2, b2)
            for i in range(3):
                out.fill_(float("nan"))
                torch.cuda.synchronize()
                with torch.cuda.stream(s):
                    o2 = g.gemm(ta2, tb2)
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, eager), (name, i)
                assert oracle.parity_check(o2.cpu().numpy(), want2, k).ok, (name, i)
    """)
    print("case graph capture with HCG_UNALIGNED_DMA=0", flush=True)
    env = dict(os.environ, HCG_UNALIGNED_DMA="0")
    proc = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_graph_replays_stay_valid_after_the_stream_needs_a_larger_workspace():
    """A captured graph keeps the workspace address it was captured with:
    when a later eager call on the same stream needs a larger workspace,
    the library allocates a new one and keeps the captured one alive, so
    replays still compute the right result."""
    import hc.gfx950 as g

    s = torch.cuda.Stream(device=DEV)
    a, b = _inputs("skinny", 16, 4096, 4096, seed=31)
    ta, tb = _dev(a), _dev(b)
    out = torch.empty((16, 4096), dtype=torch.float32, device=DEV)
    with torch.cuda.stream(s):
        g.gemm(ta, tb, out=out)
    s.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        g.gemm(ta, tb, out=out)
    # a split-K call whose partials (8 x 512 x 512 floats) exceed the
    # captured workspace, on the capturing stream
    big_a, big_b = _inputs("tiled", 512, 512, 16384, seed=32)
    tba, tbb = _dev(big_a), _dev(big_b)
    with torch.cuda.stream(s):
        big = g.gemm(tba, tbb)
    s.synchronize()
    rep = oracle.parity_check(big.cpu().numpy(), oracle.gemm_c(big_a, big_b), 16384)
    assert rep.ok, str(rep)
    print("case graph replay after workspace growth", flush=True)
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
