#!/bin/sh
# Builds the C restatement of the oracle (test infrastructure only).
# The reference itself (Objective-C++ over Metal/MPSGraph, MLIR/StableHLO
# fetched by scripts/setup_deps.sh) cannot be compiled here, so there is no
# oracle/_ref build; see the oracle package docstring.
# -ffp-contract=off: every a * b + c rounds after the product, as the
# restated programs do (no fused multiply-add the programs do not ask for).
set -e
here="$(cd "$(dirname "$0")" && pwd)"
mkdir -p "$here/lib"
gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp -fPIC -shared -o "$here/lib/liboracle_c.so.tmp" "$here/c/oracle.c" -lm
mv "$here/lib/liboracle_c.so.tmp" "$here/lib/liboracle_c.so"
