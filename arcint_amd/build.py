"""Builds libqmm.so (HIP, gfx950) in-tree, and the CPU oracle for the tests.

    python -m arcint_amd.build            # library + oracle
    python -m arcint_amd.build --lib      # library only

The library is compiled with hipcc for gfx950 only; every HIP source gets
packed-fp32 code generation switched off (-packed-fp32-ops), the objects go
to arcint_amd/_build/ and the shared library to arcint_amd/libqmm.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqmm.so")
ORACLE_DIR = os.path.join(ROOT, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]

# per-source extras: the few-column GEMV consumes its MFMA results on the VALU, so they are
# written to VGPRs directly (no accumulation-register reads)
FILE_FLAGS = {"k_gemv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_lib() -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
    objs = []
    jobs = []
    for s in srcs:
        o = os.path.join(BUILD, s + ".o")
        objs.append(o)
        lang = ["-x", "hip"]
        jobs.append([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(s, []), *lang, "-c", os.path.join(CSRC, s), "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        list(ex.map(_run, jobs))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> str:
    _run(["make", "-s", "-C", ORACLE_DIR])
    return os.path.join(ORACLE_DIR, "liborc.so")


def main(argv: list[str]) -> int:
    if "--oracle" not in argv:
        print(build_lib())
    if "--lib" not in argv:
        print(build_oracle())
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
