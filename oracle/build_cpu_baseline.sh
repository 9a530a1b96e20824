#!/bin/bash
# Builds the benchmark's CPU baseline (oracle/fst_cpu_baseline.c) for the host
# it runs on: -O3 -march=native, OpenMP, fp32.  Usage: build_cpu_baseline.sh OUT.so
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
out="${1:-$here/_build/libfst_cpu_baseline.so}"
mkdir -p "$(dirname "$out")"
gcc -O3 -march=native -fopenmp -std=gnu11 -fPIC -shared -Wall -Wextra \
    "$here/fst_cpu_baseline.c" -o "$out.tmp" -lm
mv "$out.tmp" "$out"
