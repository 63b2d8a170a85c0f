#!/bin/bash
# Runs the CPU test suite against an AddressSanitizer + UndefinedBehaviorSanitizer build of the
# oracle (oracle/_san/libva_oracle.so; the Python interpreter itself is not instrumented, so the
# ASan runtime is preloaded).  CPU only: nothing here touches a GPU.
set -eo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
ROOT="$(dirname "$HERE")"
make -s -C "$HERE" sanitize
ASAN_RT="$(gcc -print-file-name=libasan.so)"
UBSAN_RT="$(gcc -print-file-name=libubsan.so)"
cd "$ROOT"
export VA_ORACLE_LIB="$HERE/_san/libva_oracle.so"
export VA_SANITIZE=1  # tests that compile their own host harness build it sanitized too
# Python and numpy are not instrumented: leaks at exit are theirs, not the oracle's
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:print_summary=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
LD_PRELOAD="$ASAN_RT:$UBSAN_RT" python3 -c "import sys; sys.path.insert(0, '.'); from oracle import oracle; \
import ctypes; l = oracle.lib(); ctypes.CDLL(None).__asan_init; print('oracle:', oracle.LIB)"
LD_PRELOAD="$ASAN_RT:$UBSAN_RT" python3 -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
