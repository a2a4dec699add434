#!/bin/bash
# The CPU test suite (pytest -m "not gpu") against sanitised builds of the
# oracle and of the library's host code: AddressSanitizer + UBSan (clang,
# shared runtime, UBSan errors fatal). Python itself is not instrumented, so
# the ASan runtime is preloaded; leak checking is off (the interpreter and
# the HIP runtime keep allocations until exit). Run from the repository root:
#   tests/sanitize_cpu.sh
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/.." && pwd)
make -C "$ROOT/oracle" asan
make -C "$ROOT/omni-rs_amd" -j8 asan
RT=$(dirname "$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)")
[ -f "$RT/libclang_rt.asan-x86_64.so" ] || RT=$(ls -d /opt/rocm/lib/llvm/lib/clang/*/lib/linux | head -1)
export LD_PRELOAD="$RT/libclang_rt.asan-x86_64.so"
export LD_LIBRARY_PATH="$RT:/opt/rocm/llvm/lib${LD_LIBRARY_PATH:+:$LD_LIBRARY_PATH}"
export ASAN_OPTIONS="detect_leaks=0:detect_odr_violation=0:alloc_dealloc_mismatch=0:abort_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
export OMNI_INT8_LIBRARY="$ROOT/omni-rs_amd/_asan/libomni_int8.so"
export OMNI_ORACLE_LIBRARY="$ROOT/oracle/_asan/liboracle_int8.so"
cd "$ROOT"
python -m pytest tests -m "not gpu" -q -p no:cacheprovider "$@"
