#!/bin/bash
# Builds the CPU oracle (test infrastructure) into oracle/_build/libfst_oracle.so.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
mkdir -p "$here/_build"
gcc -O2 -fopenmp -ffp-contract=off -fno-fast-math -std=gnu11 -fPIC -shared \
    -Wall -Wextra -Wno-unused-function \
    "$here/fst_oracle.c" -o "$here/_build/libfst_oracle.so.tmp" -lm
mv "$here/_build/libfst_oracle.so.tmp" "$here/_build/libfst_oracle.so"
