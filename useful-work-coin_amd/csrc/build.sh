#!/bin/sh
# Builds the gfx950 HIP library (the C-ABI of include/uwc.h) into uwc_amd/libuwc_hip.so: every
# source compiled to an object in parallel, then one link.
#   -ffp-contract=off        no fused multiply-add: detrt's fp32 steps round once each
#   -packed-fp32-ops off     no v_pk_*_f32 from the compiler
set -e
cd "$(dirname "$0")"
OUT=../uwc_amd/libuwc_hip.so
HIPCC=/opt/rocm/bin/hipcc
# the header's hash, which uwc_header_sha() returns and the Python binding checks at load
SHA=$(sha256sum ../../include/uwc.h | cut -c1-16)
FLAGS="--offload-arch=gfx950 -O3 -std=c++17 -fPIC -ffp-contract=off -Xclang -target-feature -Xclang -packed-fp32-ops -Wno-unused-result -I../../include -DUWC_HEADER_SHA=\"$SHA\" ${UWC_HIPCC_EXTRA}"
TMP=$(mktemp -d)
trap 'rm -rf "$TMP"' EXIT
pids=""
for f in uwc_*.hip; do
  $HIPCC $FLAGS -c "$f" -o "$TMP/${f%.hip}.o" &
  pids="$pids $!"
done
fail=0
for p in $pids; do
  wait "$p" || fail=1
done
if [ "$fail" -ne 0 ]; then
  echo "build.sh: a source failed to compile" >&2
  exit 1
fi
$HIPCC --offload-arch=gfx950 -shared -fPIC "$TMP"/*.o -o "$OUT.tmp"
mv "$OUT.tmp" "$OUT"
