#!/bin/bash
# The CPU test tier with the host code under AddressSanitizer + UndefinedBehaviorSanitizer: the
# core, the runtime and the oracle rebuilt with -fsanitize=address,undefined (g++; no GPU code is
# sanitized), the sanitizer runtimes preloaded into python, any report fatal. Extra arguments go to
# pytest (e.g. -k test_host).
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
make -C "$ROOT/ggml-loader_amd" -j8 asan
make -C "$ROOT/oracle" asan
export GGML_LOADER_LIB_DIR="$ROOT/ggml-loader_amd/_asan/lib"
export GGML_LOADER_ORACLE_SO="$ROOT/oracle/_asan/libggml-cpu-oracle.so"
export ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1"
export UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1"
export LD_PRELOAD="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)"
cd "$ROOT"
exec python -m pytest tests -x -q -m "not gpu" -p no:cacheprovider "$@"
