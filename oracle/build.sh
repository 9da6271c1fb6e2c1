#!/bin/sh
# Builds the CPU oracle (test infrastructure only) into oracle/librefcpu.so.
# -mavx2 -mfma (not AVX-512) keeps the reference's 8-wide SIMD; no FMA
# contraction so every fused multiply-add is an explicit one.
#
# SANITIZE=1 oracle/build.sh builds the same library with AddressSanitizer
# and UndefinedBehaviorSanitizer (host code only; gcc, no GPU code involved).
# Python does not link libasan itself, so preload it for the CPU tests:
#   SANITIZE=1 oracle/build.sh
#   LD_PRELOAD=$(gcc -print-file-name=libasan.so) ASAN_OPTIONS=detect_leaks=0 \
#     python -m pytest tests -m "not gpu" -q
#   oracle/build.sh        # back to the normal build
set -e
cd "$(dirname "$0")"
SAN=""
if [ "${SANITIZE:-0}" = "1" ]; then
  SAN="-fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer -g"
fi
gcc -O3 -mavx2 -mfma -ffp-contract=off -fno-fast-math -fPIC -shared -pthread \
    -Wall $SAN -o librefcpu.so.tmp refcpu.c -lm
mv librefcpu.so.tmp librefcpu.so
