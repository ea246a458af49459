#!/bin/bash
# CPU test suite under AddressSanitizer + UndefinedBehaviorSanitizer: the library's host code
# (planner, validation, entry points) and the C oracle are rebuilt instrumented and the
# `-m "not gpu"` tests run against those builds.  No GPU is used.
#   bash tests/sanitize.sh [extra pytest args]
set -euo pipefail
REPO="$(cd "$(dirname "${BASH_SOURCE[0]}")/.." && pwd)"
PKG="$REPO/qwen3-embedding-webgpu-prepacked_amd"
make -s -C "$PKG" asan
make -s -C "$REPO/oracle" asan
RT="$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)"
if [ ! -f "$RT" ]; then
  RT="$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -n 1)"
fi
export QATTN_LIB="$PKG/_build/asan/libqattn.so"
export QATTN_ORACLE_LIB="$REPO/oracle/_build/asan/liboracle.so"
# CPython and numpy are not instrumented: leak reports from their allocations are noise.
export ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
cd "$REPO"
LD_PRELOAD="$RT" python -m pytest tests/ -x -q -m "not gpu" -p no:cacheprovider "$@"
