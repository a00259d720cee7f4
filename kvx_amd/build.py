"""Build libkvx_amd.so (the C-ABI library with the gfx950 HIP kernels) in-tree.

Usage: python -m kvx_amd.build   (or kvx_amd.build.build() from Python)

Every source is compiled with hipcc for gfx950 only.  Device-code flags:
  -fhip-fp32-correctly-rounded-divide-sqrt  the FP8 quantizing cast divides by
                                            the scale and must round exactly;
  -fno-gpu-flush-denormals-to-zero          keep f32 subnormals (bit-exact
                                            casts of tiny values);
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                            no packed-FP32 instructions.
The library links with -Bsymbolic so its own entry points never resolve to a
same-named symbol from another loaded library, and exports only kvx_* symbols
(csrc/exports.map).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO / "include"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libkvx_amd.so"

# The kernel families live in kernels_*.hip (one translation unit each, all
# including kernels.h) so that they compile in parallel.
SOURCES = ["abi.cpp", "launch.cpp", "dispatch.hip"] + sorted(
    p.name for p in CSRC.glob("kernels_*.hip"))
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the kvx_amd build needs ROCm")
    return path


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature;
    # that line is expected and carries no information.
    noise = "not a recognized feature for this target"
    stderr = "\n".join(l for l in proc.stderr.splitlines() if noise not in l
                       and "ignoring feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n"
                           f"{proc.stdout}\n{proc.stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr, flush=True)


def build_jobs() -> int:
    """Parallel compiler processes: MAX_JOBS when set, else one per CPU (at
    most 16)."""
    env = os.environ.get("MAX_JOBS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return max(1, min(16, os.cpu_count() or 1))


def build(verbose: bool = False) -> Path:
    """Compile every source and link LIB_PATH.  Always rebuilds."""
    OBJ_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    objs = [str(OBJ_DIR / (src + ".o")) for src in SOURCES]
    for stale in OBJ_DIR.glob("*.o"):
        if str(stale) not in objs:
            stale.unlink()
    jobs = [[cc, *COMMON_FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", obj]
            for src, obj in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=build_jobs()) as pool:
        for f in [pool.submit(_run, cmd, verbose) for cmd in jobs]:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs,
          "-Wl,-Bsymbolic", "-Wl,--no-undefined",
          f"-Wl,--version-script={CSRC / 'exports.map'}"], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


PROBE_SRC = CSRC / "stream_probe.hip"
PROBE_LIB = PKG_DIR / "libkvx_amd_probe.so"


def build_probe(verbose: bool = False) -> Path:
    """Compile the streaming-probe library (plain copy / read / write
    kernels that bench.py times beside the KV kernels)."""
    cc = hipcc()
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    _run([cc, *COMMON_FLAGS, "-shared", "-x", "hip", str(PROBE_SRC), "-o", str(tmp)], verbose)
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


BENCH_SRC = CSRC / "kvx_bench.cpp"
BENCH_BIN = PKG_DIR / "kvx_bench"


def build_bench(verbose: bool = False) -> Path:
    """Compile the kvx_bench command line (host code over libkvx_amd.so,
    found next to it at run time)."""
    cc = hipcc()
    tmp = BENCH_BIN.with_suffix(".tmp")
    _run([cc, "-O2", "-std=c++17", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}", str(BENCH_SRC),
          "-o", str(tmp), f"-L{PKG_DIR}", "-lkvx_amd", "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, BENCH_BIN)
    return BENCH_BIN


TORCH_OPS_SRC = CSRC / "torch_ops.cpp"
TORCH_OPS_LIB = PKG_DIR / "libkvx_amd_torch.so"


def build_torch_ops(verbose: bool = False) -> Path:
    """Compile the PyTorch-ROCm op library (csrc/torch_ops.cpp) against the
    installed torch and link it to libkvx_amd.so (found next to it at run
    time).  Host code only: g++ with torch's and ROCm's headers."""
    import torch

    if torch.version.hip is None:
        raise RuntimeError("the torch op library needs a ROCm build of PyTorch")
    tdir = Path(torch.__file__).resolve().parent
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cxx = shutil.which("g++") or "g++"
    tmp = TORCH_OPS_LIB.with_suffix(".so.tmp")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          f"-I{INCLUDE}", f"-I{tdir / 'include'}",
          f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
          f"-I{rocm / 'include'}", str(TORCH_OPS_SRC), "-o", str(tmp),
          f"-L{PKG_DIR}", "-lkvx_amd", f"-L{tdir / 'lib'}", "-lc10", "-lc10_hip",
          "-ltorch_cpu", "-ltorch_hip", f"-L{rocm / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, TORCH_OPS_LIB)
    return TORCH_OPS_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_bench(verbose="-v" in sys.argv))
    print(build_probe(verbose="-v" in sys.argv))
    print(build_torch_ops(verbose="-v" in sys.argv))
