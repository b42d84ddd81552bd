"""Mutation builds against the GPU parity suite: every planted mistake must turn it red.

    python tests/red/run_red.py --build          # here: libqmm_red{k}.so for every k (CPU, hipcc)
    python tests/red/run_red.py                  # on a GPU: the suite against each build

Build k of arcint_amd.build --red compiles the library with QMM_RED=k, which plants one known,
in-bounds mistake in one kernel family (qmm_internal.h lists them).  For each k the GPU tests run
against that library (QMM_LIB) until MAXFAIL of them fail; the run prints the failing tests and
exits non-zero if some mutation left the suite green.  Not collected by pytest (the suite is
meant to fail here).
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
MUTATIONS = {
    1: "dequant: Q4_K sub-block j takes sub-block j ^ 1's scale and min",
    2: "q8_0 activation quantizer rounds ties away from zero instead of to even",
    3: "v_dot4 GEMV (Q4_0): the last block of every group dropped",
    4: "MFMA GEMV (Q4_0/Q8_0/IQ4_NL): rows 32-63 use rows 0-31's block scale in the magic-bias subtract",
    5: "Q4_K GEMM: sub-block scales of neighbouring sub-blocks swapped",
    6: "streaming GEMM (Q4_0/Q8_0/IQ4_NL): rows 32-63 take rows 0-31's block scale",
    7: "MoE route: every routed task runs on the next expert",
    8: "fused MoE GEMV (few tokens): every pair runs on the next expert",
}
MAXFAIL = 3


def lib(k: int) -> str:
    return os.path.join(ROOT, "arcint_amd", "_build_red", f"libqmm_red{k}.so")


def main(argv: list[str]) -> int:
    sys.path.insert(0, ROOT)
    if "--build" in argv:
        from arcint_amd import build
        for k in MUTATIONS:
            print(build.build_red(k), flush=True)
        return 0
    green = []
    for k, what in MUTATIONS.items():
        print(f"[red {k}] {what}", flush=True)
        if not os.path.exists(lib(k)):
            print(f"[red {k}] {lib(k)} is not built (--build)", flush=True)
            return 2
        env = dict(os.environ, QMM_LIB=lib(k))
        cmd = [sys.executable, "-u", "-m", "pytest", os.path.join(ROOT, "tests"), "-m", "gpu", "-q", "-rf",
               f"--maxfail={MAXFAIL}", "--timeout", "120", "--timeout-method", "thread", "-p", "no:cacheprovider"]
        r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=900)
        failed = re.findall(r"^FAILED (\S+)", r.stdout, flags=re.M)
        summary = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else ""
        print(f"[red {k}] rc={r.returncode} {summary}", flush=True)
        for f in failed:
            print(f"[red {k}]   FAILED {f}", flush=True)
        if not failed:
            green.append(k)
    if green:
        print(f"mutations the suite did not catch: {green}", flush=True)
        return 1
    print("every mutation turned the suite red", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
