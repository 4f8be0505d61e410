#!/bin/bash
# Host-side sanitizer run on the CPU (no GPU needed): builds the library's
# host code and the oracle with AddressSanitizer + UndefinedBehaviorSanitizer
# (make targets `asan`) and runs the CPU tests that exercise them - the GGUF
# parser on well-formed and malformed files, the C-ABI argument checks and
# failure paths, and the oracle tests - with the compiler's shared ASan
# runtime preloaded into Python. Any report fails the run.
set -euo pipefail
ROOT=$(cd "$(dirname "${BASH_SOURCE[0]}")/.." && pwd)
make -s -C "$ROOT/inferno.jl_amd" -j"$(nproc)" asan
make -s -C "$ROOT/oracle" asan
RT=$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)
export LD_PRELOAD="$RT"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1:verify_asan_link_order=0"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
export INFERNO_HIP_LIB="$ROOT/inferno.jl_amd/lib/asan/libinferno_hip.so"
export INFERNO_ORACLE_LIB="$ROOT/oracle/_asan/liboracle.so"
cd "$ROOT"
# the instrumented builds and the ASan runtime are the ones this process maps
python - <<'PY'
import sys
sys.path[:0] = ["inferno.jl_amd", "oracle"]
import inferno_hip, oracle
inferno_hip.load(); oracle.lib()
maps = open("/proc/self/maps").read()
for want in ("libclang_rt.asan-x86_64.so", "lib/asan/libinferno_hip.so", "_asan/liboracle.so"):
    assert want in maps, want
print("sanitizer builds loaded")
PY
python -m pytest tests/test_gguf.py tests/test_abi.py tests/test_oracle_quant.py tests/test_oracle_accept.py \
    tests/test_oracle_sampler.py tests/test_host_logic.py -q -m "not gpu" -p no:cacheprovider "$@"
