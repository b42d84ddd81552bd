#!/bin/bash
# Runs the device-free tests against the host code of libqmm (layout packing, tensor I/O, plans,
# the load replay) and the CPU oracle, both built with AddressSanitizer and
# UndefinedBehaviorSanitizer; CPU only.  The GPU code of that build is compiled as usual.
set -euo pipefail
cd "$(dirname "$0")/.."
python -m arcint_amd.build --sanitize > /dev/null
make -s -C oracle liborc_san.so
RT="$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)"
export QMM_LIB="$PWD/arcint_amd/_build_san/libqmm.so" QMM_ORACLE_LIB="$PWD/oracle/liborc_san.so"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1 UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
LD_PRELOAD="$RT" python -m pytest tests/test_layout.py tests/test_oracle.py tests/test_oracle_glu.py \
    tests/test_oracle_moe.py tests/test_abi.py tests/test_gguf.py tests/test_gemv_bounds.py -q -m "not gpu" \
    -p no:cacheprovider "$@"
