#!/bin/bash
# Host code under AddressSanitizer + UBSan, on the CPU (no GPU is used and
# device code is not instrumented):
#   1. the oracle, built with gcc's runtimes, under its tests;
#   2. the library's host paths (the GGUF parser, every entry point's
#      argument checks), built with clang's runtime, under the GGUF and ABI
#      tests.
# Each suite runs in its own process with its runtime preloaded; any report
# fails the run (halt_on_error).  Usage: bash tests/sanitize.sh
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/.." && pwd)
cd "$ROOT"
make -s -C oracle sanitize
make -s -C breadv2_amd/csrc -j8 sanitize
export ASAN_OPTIONS=detect_leaks=0:halt_on_error=1:abort_on_error=1
export UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1
GCC_ASAN=$(gcc -print-file-name=libasan.so)
CLANG_ASAN=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -n 1)
echo "== oracle (gcc ASan + UBSan)"
BREAD_ORACLE_LIB="$ROOT/oracle/_san/liboracle.so" LD_PRELOAD="$GCC_ASAN" \
    python -m pytest -q -m "not gpu" -p no:cacheprovider tests/test_oracle.py
echo "== library host code (clang ASan + UBSan)"
BREAD_MOE_LIB="$ROOT/breadv2_amd/_san/libbread_moe.so" LD_PRELOAD="$CLANG_ASAN" \
    python -m pytest -q -m "not gpu" -p no:cacheprovider tests/test_gguf.py tests/test_abi.py
