#!/bin/sh
# Builds the CPU oracle (test infrastructure only) into oracle/librefcpu.so.
# -mavx2 -mfma (not AVX-512) keeps the reference's 8-wide SIMD; no FMA
# contraction so every fused multiply-add is an explicit one.
set -e
cd "$(dirname "$0")"
gcc -O3 -mavx2 -mfma -ffp-contract=off -fno-fast-math -fPIC -shared -pthread \
    -Wall -o librefcpu.so.tmp refcpu.c -lm
mv librefcpu.so.tmp librefcpu.so
