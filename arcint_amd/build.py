"""Builds libqmm.so (HIP, gfx950) in-tree, and the CPU oracle for the tests.

    python -m arcint_amd.build            # library + oracle
    python -m arcint_amd.build --lib      # library only
    python -m arcint_amd.build --sanitize # host code under ASan/UBSan (tests/sanitize.sh)
    python -m arcint_amd.build --red K    # mutation build K (tests/red/run_red.py)

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


def build_lib(out: str = LIB, build_dir: str = BUILD, extra: list[str] | None = None,
              link_extra: list[str] | None = None) -> str:
    """Compiles every source of csrc/ and links `out`.  `extra` goes on every compile line
    (test builds: host-only sanitizers, a mutation define), `link_extra` on the link line."""
    os.makedirs(build_dir, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
    objs = []
    jobs = []
    for s in srcs:
        o = os.path.join(build_dir, s + ".o")
        objs.append(o)
        lang = ["-x", "hip"]
        jobs.append([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(s, []), *(extra or []), *lang, "-c", os.path.join(CSRC, s),
                     "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        list(ex.map(_run, jobs))
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *(link_extra or []), "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


# Test builds (tests/sanitize.sh, tests/red/run_red.py), never loaded by the product path:
#  * sanitized: the host code (layout packing, tensor I/O, dispatch) under AddressSanitizer and
#    UndefinedBehaviorSanitizer; the device code is built as usual (-Xarch_host keeps the
#    sanitizers off the GPU code);
#  * mutation k: QMM_RED=k plants one known mistake in one kernel family, which the GPU parity
#    suite must catch.
SAN_DIR = os.path.join(HERE, "_build_san")
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=undefined"]


def build_sanitized() -> str:
    return build_lib(os.path.join(SAN_DIR, "libqmm.so"), os.path.join(SAN_DIR, "obj"), SAN_FLAGS,
                     ["-fsanitize=address", "-fsanitize=undefined"])


def build_red(k: int) -> str:
    d = os.path.join(HERE, "_build_red")
    return build_lib(os.path.join(d, f"libqmm_red{k}.so"), os.path.join(d, f"obj{k}"), [f"-DQMM_RED={k}"])


def build_oracle() -> str:
    _run(["make", "-s", "-C", ORACLE_DIR])
    return os.path.join(ORACLE_DIR, "liborc.so")


def main(argv: list[str]) -> int:
    if "--sanitize" in argv:
        print(build_sanitized())
        return 0
    if "--red" in argv:
        print(build_red(int(argv[argv.index("--red") + 1])))
        return 0
    if "--oracle" not in argv:
        print(build_lib())
    if "--lib" not in argv:
        print(build_oracle())
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
