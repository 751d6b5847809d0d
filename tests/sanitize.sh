#!/bin/bash
# CPU sanitizer run: builds the host runtime (libzealot_hip.so) and the oracle
# with AddressSanitizer + UndefinedBehaviorSanitizer and runs the CPU tests
# that exercise them (the oracle's pins, the checkpoint image parser with its
# malformed images, the C ABI's argument checks) against those builds.
# Python itself is not instrumented, so the ASan runtime is preloaded into it.
# CPU only: no GPU is used.
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
make -s -C "$ROOT/zealot_amd/csrc" asan
make -s -C "$ROOT/oracle" asan
export ZL_LIBRARY="$ROOT/zealot_amd/lib/asan/libzealot_hip.so"
export ZL_ORACLE_LIBRARY="$ROOT/oracle/_asan/libzl_oracle.so"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
LD_PRELOAD="$(gcc -print-file-name=libasan.so)" \
  python -m pytest -q -m "not gpu" -p no:cacheprovider \
  "$ROOT/tests/test_oracle.py" "$ROOT/tests/test_checkpoint_format.py" "$ROOT/tests/test_abi.py" "$@"
