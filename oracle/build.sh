#!/usr/bin/env bash
# Builds the CPU oracle (test infrastructure) into oracle/_build/liboracle.so.
# The reference's own path cannot be compiled here (CUDA inline PTX + CUB,
# no nvcc), so no oracle/_ref build exists.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
mkdir -p "$here/_build"
gcc -O2 -fPIC -shared -fopenmp -std=c11 -Wall -Wextra -Wno-unused-parameter \
    "$here/oracle.c" -o "$here/_build/liboracle.so.tmp"
mv "$here/_build/liboracle.so.tmp" "$here/_build/liboracle.so"
