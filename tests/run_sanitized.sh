#!/bin/bash
# Runs the CPU tests against AddressSanitizer + UndefinedBehaviorSanitizer
# builds of the host libraries (triton-ext_amd/lib_asan) and the oracle
# (oracle/_asan).  CPU only: nothing here touches a GPU.
set -eo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
make -s -C "$ROOT/triton-ext_amd" sanitize
make -s -C "$ROOT/oracle" sanitize
RT="$(/opt/rocm/lib/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)"
[ -f "$RT" ] || RT="$(ls /opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)"
export TX_LIB_DIR="$ROOT/triton-ext_amd/lib_asan" TX_ORACLE_LIB="$ROOT/oracle/_asan/liboracle.so"
# Python itself is not instrumented: its allocations are not leaks of ours
export ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1:verify_asan_link_order=0"
export UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1"
cd "$ROOT"
LD_PRELOAD="$RT" python -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
