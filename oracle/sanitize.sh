#!/bin/bash
# Runs the oracle's own CPU tests (tests/test_oracle.py, tests/test_golden.py,
# CPU cases) against sanitizer builds of oracle/refcpu.c:
#   1. AddressSanitizer + UndefinedBehaviorSanitizer (errors are fatal);
#   2. ThreadSanitizer (the 32-thread row-read pool and the row-parallel
#      MatMulVec run under it).
# The sanitizer runtime is preloaded into the Python process, and REFCPU_LIB
# points oracle/refcpu.py at the sanitizer build; each run first checks that
# the process really mapped that build.  torch runs single-threaded
# (OMP_NUM_THREADS=1): its OpenMP pool is not instrumented and would only add
# reports about torch itself.  Exit status: 0 when both runs pass.
set -u
HERE="$(cd "$(dirname "$0")" && pwd)"
ROOT="$(dirname "$HERE")"
make -s -C "$HERE" asan tsan || exit 1
export UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1  # the build also sets -fno-sanitize-recover
cd "$ROOT" || exit 1

run() {  # name, runtime library, lib, options variable, options
    local name=$1 rt=$2 lib=$3 optvar=$4 opts=$5
    echo "== $name"
    env OMP_NUM_THREADS=1 LD_PRELOAD="$rt" "$optvar=$opts" REFCPU_LIB="$lib" python -c "
import sys; sys.path.insert(0, '.')
from oracle import refcpu as R
R.lib()
assert '$(basename "$lib")' in open('/proc/self/maps').read(), 'sanitizer build not mapped'
print('mapped', R.LIB_PATH)" || return 1
    env OMP_NUM_THREADS=1 LD_PRELOAD="$rt" "$optvar=$opts" REFCPU_LIB="$lib" \
        python -m pytest tests/test_oracle.py tests/test_golden.py -q -s -m "not gpu" \
        -p no:cacheprovider
}

run "ASan + UBSan" "$(gcc -print-file-name=libasan.so)" "$HERE/librefcpu_asan.so" \
    ASAN_OPTIONS "detect_leaks=0:halt_on_error=1" || exit 1
run "TSan" "$(gcc -print-file-name=libtsan.so)" "$HERE/librefcpu_tsan.so" \
    TSAN_OPTIONS "halt_on_error=1:report_signal_unsafe=0" || exit 1
echo "sanitizers: clean"
