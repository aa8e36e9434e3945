#!/bin/bash
# CPU test suite (pytest -m "not gpu") against sanitizer builds of the host
# code: the fp64 checker's OpenMP loops under TSan (oracle/tsan_driver.c, run
# by make sanitize), then the checker and the operator library's host side
# (descriptor checks, planning, workspace carving) under ASan + UBSan.  Python itself is not instrumented,
# so the runtimes are preloaded and leak reports (CPython's) are off.
# Usage: bash oracle/run_sanitized.sh   (from the repository root)
set -e
R=$(cd "$(dirname "$0")/.." && pwd)
make -s -C "$R/oracle" sanitize   # builds the ASan checker; builds and runs the TSan driver
python3 "$R/race_attention_amd/build.py" --sanitize
ASAN_RT=$(gcc -print-file-name=libasan.so)
UBSAN_RT=$(gcc -print-file-name=libubsan.so)
cd "$R"
echo "== ASan + UBSan: oracle and library host code"
ASAN_OPTIONS=detect_leaks=0:halt_on_error=1 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \
LD_PRELOAD="$ASAN_RT $UBSAN_RT" RACE_ORACLE_LIB="$R/oracle/_san/liborace_asan.so" \
RACE_ATTENTION_LIB="$R/race_attention_amd/_san/librace_attention_asan.so" \
    python3 -m pytest tests -q -m "not gpu" -p no:cacheprovider
echo "== TSan: every OpenMP loop of the oracle (LLVM libomp + Archer), via make sanitize above"
