"""Build recipe for the gfx950 GEMM library.

    python 5_amd/csrc/build.py [-v]

compiles 5_amd/csrc/hcg_gemm.hip, hcg_tile.hip and hcg_mfma.hip (kernels +
the C ABI declared in include/hcg_gemm.h, include/hcg_tile_ops.h and
include/hcg_mfma.h) with hipcc for
gfx950 into
5_amd/hc/gfx950/libhcg_gfx950.so, next to the Python code that loads it
(and, with -DHCG_STAMPS, libhcg_gfx950_stamps.so, whose GEMM kernels record
per-workgroup timestamps for bench.py --stamps), and hcg_probe.hip (the hardware ceiling probes of include/hcg_probe.h, used
by bench.py) into 5_amd/hc/gfx950/libhcg_probe.so, and hcg_torch.cpp (host
code: the device-tensor binding of hcg_gemm_algo as a Python extension,
linked against libhcg_gfx950.so) with g++ against the installed PyTorch into
5_amd/hc/gfx950/_hcg_torch<EXT_SUFFIX>.
hipcc cross-compiles, so this runs on a machine without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
SRCS = [os.path.join(HERE, f) for f in ("hcg_gemm.hip", "hcg_tile.hip", "hcg_mfma.hip")]
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(PKG, "hc", "gfx950", "libhcg_gfx950.so")
# The same sources with -DHCG_STAMPS: the tiled and streaming kernels record
# per-workgroup timestamps (bench.py --stamps); never loaded by the package.
STAMPS_OUT = os.path.join(PKG, "hc", "gfx950", "libhcg_gfx950_stamps.so")
PROBE_SRCS = [os.path.join(HERE, "hcg_probe.hip")]
PROBE_OUT = os.path.join(PKG, "hc", "gfx950", "libhcg_probe.so")
TORCH_SRC = os.path.join(HERE, "hcg_torch.cpp")
TORCH_OUT = os.path.join(PKG, "hc", "gfx950", "_hcg_torch" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++20",
        "-fPIC",
        "-shared",
        # Packed fp32 VALU forms stay disabled for all device code.
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        f"-I{INCLUDE}",
        "-Wall",
    ]


def _start(srcs: list[str], out: str, extra: list[str], verbose: bool) -> tuple[subprocess.Popen, str]:
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cmd = [hipcc(), *flags(), *extra, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
    return proc, out


def _finish(job: tuple[subprocess.Popen, str], verbose: bool) -> str:
    proc, out = job
    _, stderr = proc.communicate()
    # The host pass does not know the device-only target feature; that
    # warning is expected and harmless.  Anything else is shown.
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    err = "\n".join(line for line in stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(out)} ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)
    os.replace(out + ".tmp", out)
    return out


def _compile_torch_binding(verbose: bool) -> str:
    """g++ on hcg_torch.cpp: PyTorch's headers and libraries, the HIP headers
    (host code only), and libhcg_gfx950.so found next to the module."""
    import torch.utils.cpp_extension as cpp

    import torch

    tmp = TORCH_OUT + ".tmp"
    # The C++ ABI the installed torch was built with (its headers' std::string
    # layout must match ours).
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
           "-DTORCH_EXTENSION_NAME=_hcg_torch", "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *(f"-I{p}" for p in cpp.include_paths()), f"-I{sysconfig.get_paths()['include']}",
           "-I/opt/rocm/include", f"-I{INCLUDE}", TORCH_SRC, "-o", tmp,
           *(f"-L{p}" for p in cpp.library_paths()), "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", f"-L{os.path.dirname(OUT)}", "-l:libhcg_gfx950.so", "-Wl,-rpath,$ORIGIN",
           *(f"-Wl,-rpath,{p}" for p in cpp.library_paths())]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, TORCH_OUT)
    return TORCH_OUT


def build(verbose: bool = False) -> str:
    """Builds the GEMM library, its timestamped variant, the probe library
    and the device-tensor binding (the three hipcc runs in parallel);
    returns the first."""
    jobs = [_start(SRCS, OUT, [], verbose), _start(SRCS, STAMPS_OUT, ["-DHCG_STAMPS"], verbose),
            _start(PROBE_SRCS, PROBE_OUT, [], verbose)]
    outs = [_finish(job, verbose) for job in jobs]
    _compile_torch_binding(verbose)
    return outs[0]


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
