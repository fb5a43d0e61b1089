#!/usr/bin/env bash
# Build the CPU oracle (test infrastructure; never linked by the product) into oracle/build/.
# -mavx2 -mfma instead of -march=native: the library is built here and run on the GPU box's host.
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
mkdir -p "$here/build"
gcc -O3 -mavx2 -mfma -ffp-contract=off -fopenmp -fPIC -shared -std=c11 -Wall -Wextra -Wno-unused-parameter \
    "$here/sp_oracle.c" -o "$here/build/libsp_oracle.so.tmp" -lm
mv "$here/build/libsp_oracle.so.tmp" "$here/build/libsp_oracle.so"
