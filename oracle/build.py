"""Build recipe for the CPU oracle and the reference-compiled checkers.

TEST INFRASTRUCTURE ONLY.

  oracle/_build/libkvx_oracle.so     this repository's C restatement
                                     (kvx_oracle.c), gcc -O2 -fopenmp.
  oracle/_ref/libkvx_ref_abi.so      the reference's own kvx_abi.c, compiled
                                     unmodified from /root/reference (pure
                                     C11, validation only): the status-code
                                     oracle for the kvx_abi.h entry points.
  oracle/_ref/kvx_abi_test_ref       the reference's tests/kvx_abi_test.c
                                     linked with its own kvx_abi.c (sanity).
  oracle/_ref/kvx_abi_test_kvx_amd   the same test compiled against the
                                     reference's kvx_abi.h but linked with
                                     kvx_amd/libkvx_amd.so: the drop-in check.

The reference's kernel file (kernels/kvx_paged_kv.cu) needs nvcc and the CUDA
runtime headers, which this image lacks, so it is not built; its semantics
are restated in kvx_oracle.c.  _ref/ is built only where /root/reference
exists; nothing is copied from it into the repository.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
BUILD = HERE / "_build"
REF_OUT = HERE / "_ref"
REFERENCE = Path(os.environ.get("KVX_REFERENCE_ROOT", "/root/reference"))
ORACLE_LIB = BUILD / "libkvx_oracle.so"
REF_ABI_LIB = REF_OUT / "libkvx_ref_abi.so"
REF_TEST_REF = REF_OUT / "kvx_abi_test_ref"
REF_TEST_OURS = REF_OUT / "kvx_abi_test_kvx_amd"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build_oracle() -> Path:
    BUILD.mkdir(exist_ok=True)
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run(["gcc", "-std=c11", "-O3", "-fopenmp", "-fPIC", "-shared", "-Wall",
          "-o", str(tmp), str(HERE / "kvx_oracle.c"), "-lm"])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def build_ref(kvx_lib: Path | None = None) -> list[Path]:
    """Compile the reference's C ABI files where they lie.  Returns the
    artefacts built; empty when the reference tree is absent."""
    abi_c = REFERENCE / "kvx_abi.c"
    test_c = REFERENCE / "tests" / "kvx_abi_test.c"
    if not abi_c.exists():
        return []
    REF_OUT.mkdir(exist_ok=True)
    inc = f"-I{REFERENCE}"
    _run(["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-Wl,-Bsymbolic", inc,
          "-o", str(REF_ABI_LIB), str(abi_c)])
    out = [REF_ABI_LIB]
    if test_c.exists():
        _run(["gcc", "-std=c11", "-O0", "-UNDEBUG", inc, "-o", str(REF_TEST_REF),
              str(test_c), str(abi_c)])
        out.append(REF_TEST_REF)
        if kvx_lib is not None and kvx_lib.exists():
            _run(["gcc", "-std=c11", "-O0", "-UNDEBUG", inc, "-o", str(REF_TEST_OURS),
                  str(test_c), str(kvx_lib), f"-Wl,-rpath,{kvx_lib.parent}"])
            out.append(REF_TEST_OURS)
    return out


def build(kvx_lib: Path | None = None) -> list[Path]:
    return [build_oracle(), *build_ref(kvx_lib)]


if __name__ == "__main__":
    sys.path.insert(0, str(REPO))
    from kvx_amd.abi import LIB_PATH

    for p in build(LIB_PATH):
        print(p)
