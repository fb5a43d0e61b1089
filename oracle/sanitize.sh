#!/usr/bin/env bash
# Host-side sanitizer runs of the checkers and the C++ host mirror, on the CPU (no GPU code is
# instrumented, and nothing here launches a kernel):
#   1. the oracle built with AddressSanitizer + UndefinedBehaviorSanitizer, loaded by the whole
#      CPU test suite (pytest -m "not gpu");
#   2. the C++ host mirror (sketchpad_amd/host) compiled into its test binary with both
#      sanitizers on the host code, running the binary's CPU cases (--cpu-only).
# Outputs go to oracle/build/sanitize/. Needs the product library built first
# (python -m sketchpad_amd.build).
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
root="$(dirname "$here")"
out="$here/build/sanitize"
mkdir -p "$out"
san_preload="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)"

echo "[sanitize] oracle under the CPU test suite"
gcc -O1 -g -fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer \
    -mavx2 -mfma -ffp-contract=off -fopenmp -fPIC -shared -std=c11 \
    "$here/sp_oracle.c" -o "$out/libsp_oracle.so" -lm
SP_ORACLE_LIB="$out/libsp_oracle.so" ASAN_OPTIONS=detect_leaks=0 \
    LD_PRELOAD="$san_preload${LD_PRELOAD:+ $LD_PRELOAD}" \
    python -m pytest "$root/tests" -q -m "not gpu" -p no:cacheprovider

echo "[sanitize] host mirror CPU cases"
/opt/rocm/bin/hipcc --offload-arch=gfx950 -O1 -g -std=c++17 -fPIC \
    -Xclang -target-feature -Xclang -packed-fp32-ops \
    -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined \
    -I"$root/include" -I"$root/sketchpad_amd/csrc" -I"$root/sketchpad_amd/host" -I"$here" \
    -x hip "$root/tests/cpp/test_paged_attention.cpp" "$root/tests/cpp/test_batching.cpp" \
    "$root/sketchpad_amd/host/paged_attention.cpp" "$root/sketchpad_amd/host/ragged_batch.cpp" \
    -o "$out/test_paged_attention" \
    -L"$root/sketchpad_amd/lib" -lsketchpad_attn -L"$here/build" -lsp_oracle \
    -Wl,-rpath,"$root/sketchpad_amd/lib" -Wl,-rpath,"$here/build"
ASAN_OPTIONS=detect_leaks=0 "$out/test_paged_attention" --cpu-only
echo "[sanitize] clean"
