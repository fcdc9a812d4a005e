#!/bin/bash
# The CPU tests that reach the library's host code (ABI argument checks, the
# .slhw loader, the EventLog file side, the CCOS host paths, the malformed-file
# cases of test_host_fuzz.py) against the host sanitizer build of libslha
# (AddressSanitizer + UndefinedBehaviorSanitizer on the host C++; build with
# `python3 slhav2_amd/build.py sanitize`). Any report aborts the run.
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/.." && pwd)
LIB="$ROOT/slhav2_amd/libslha_asan.so"
[ -f "$LIB" ] || python3 "$ROOT/slhav2_amd/build.py" sanitize
RT=$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)
export SLHA_LIBRARY="$LIB"
# Python and torch are not instrumented: their allocator pairings and leaks
# are not this library's; everything in libslha is checked.
export ASAN_OPTIONS=detect_leaks=0:halt_on_error=1:abort_on_error=1:alloc_dealloc_mismatch=0:new_delete_type_mismatch=0
export UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1
cd "$ROOT"
LD_PRELOAD="$RT" python3 -m pytest -q -m "not gpu" -p no:cacheprovider \
    tests/test_abi_cpu.py tests/test_eventlog.py tests/test_learned.py tests/test_ccos.py \
    tests/test_host_fuzz.py "$@"
