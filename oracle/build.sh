#!/bin/sh
# Builds the CPU oracle (test infrastructure only) into oracle/liboracle.so.
# -ffp-contract=off: no fused multiply-add, so every fp32 op rounds once (runtime/detrt/core.py:1-17).
set -e
cd "$(dirname "$0")"
gcc -O2 -fopenmp -ffp-contract=off -fno-fast-math -fPIC -shared -fvisibility=hidden uwc_oracle.c -o liboracle.so.tmp -lm
mv liboracle.so.tmp liboracle.so
