#!/bin/bash
# Builds oracle/_ref/libref_cpu.so from the reference's own CPU routines
# (see ref_shim.cpp for the line ranges).  Test infrastructure only.
# Usage: build_ref.sh [reference_root]   (default /root/reference)
set -euo pipefail
REF=${1:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
OUT="$HERE/_ref"
if [ ! -d "$REF/FINAL_CLEAN_CODE" ]; then
    echo "build_ref: $REF not present, skipping oracle/_ref" >&2
    exit 0
fi
TMP=$(mktemp -d)
trap 'rm -rf "$TMP"' EXIT
excerpt() {  # file first last out expected-first-line-prefix
    sed -n "$2,$3p" "$REF/$1" > "$TMP/$4"
    head -1 "$TMP/$4" | grep -q "^$5" || {
        echo "build_ref: $1:$2 does not start with '$5'" >&2; exit 1; }
}
excerpt FINAL_CLEAN_CODE/tests/test_layernorm.cu 8 24 ln_cpu.inc "static void layernorm_cpu("
excerpt NEW_code/tests/test_embedding.cu 16 41 emb_cpu.inc "static void embedding_forward_cpu("
excerpt FINAL_CLEAN_CODE/tests/test_fusion_benchmark.cu 8 12 fill_pattern.inc "static void fill_pattern("
excerpt FINAL_CLEAN_CODE/tests/test_model_reference.cu 49 68 ln_f64.inc "static void layernorm("
excerpt NEW_code/tests/test_softmax_ce.cu 26 75 softmax_ce.inc "static void softmax_cpu("
mkdir -p "$OUT"
g++ -std=c++17 -O2 -ffp-contract=off -fPIC -shared -I"$TMP" \
    "$HERE/ref_shim.cpp" -o "$OUT/libref_cpu.so"
echo "build_ref: wrote $OUT/libref_cpu.so"
