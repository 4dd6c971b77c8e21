#!/bin/sh
# Builds the gfx950 HIP library (the C-ABI of include/uwc.h) into uwc_amd/libuwc_hip.so.
#   -ffp-contract=off        no fused multiply-add: detrt's fp32 steps round once each
#   -packed-fp32-ops off     no v_pk_*_f32 from the compiler
set -e
cd "$(dirname "$0")"
OUT=../uwc_amd/libuwc_hip.so
/opt/rocm/bin/hipcc --offload-arch=gfx950 -O3 -std=c++17 -fPIC -shared -ffp-contract=off \
  -Xclang -target-feature -Xclang -packed-fp32-ops -Wno-unused-result -I../../include ${UWC_HIPCC_EXTRA} \
  uwc_abi.hip uwc_commit.hip uwc_gemm.hip uwc_gemm256.hip uwc_noise.hip uwc_quant.hip uwc_side.hip uwc_skinny.hip \
  uwc_layer.hip uwc_attn.hip uwc_sha.hip -o "$OUT.tmp"
mv "$OUT.tmp" "$OUT"
