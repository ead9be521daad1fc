#!/bin/bash
# Builds the reference's own PLD proposer from its sources where they lie (engine/src/pld.cu is plain C++17
# despite its extension: engine/include/pld.h:5) into oracle/_ref/libpld_ref.so, for the oracle's parity tests
# and the CPU baseline.  Test infrastructure only; needs /root/reference (absent on GPU boxes, where the built
# library travels with the tree).
set -e
REF=${QWS_REFERENCE:-/root/reference}
OUT=$(cd "$(dirname "$0")" && pwd)/_ref
[ -f "$REF/engine/src/pld.cu" ] || { echo "reference sources not found under $REF: nothing built"; exit 0; }
mkdir -p "$OUT"
g++ -x c++ -std=c++17 -O2 -shared -fPIC -I"$REF/engine/include" "$REF/engine/src/pld.cu" -o "$OUT/libpld_ref.so"
echo "$OUT/libpld_ref.so"
