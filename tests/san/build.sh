#!/bin/bash
# Build tests/san/_build/san_driver: the library (every source) plus
# san_driver.cpp with AddressSanitizer and UndefinedBehaviorSanitizer on the
# host code (the .hip files' device code is compiled as usual and not
# instrumented: -Xarch_host before each -fsanitize), for a CPU run.
set -euo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
CSRC="$HERE/../../juno_amd/csrc"
OUT="$HERE/_build"
mkdir -p "$OUT"
rm -f "$OUT"/*.o "$OUT/san_driver"
HIPCC="${HIPCC:-/opt/rocm/bin/hipcc}"
SAN=(-fsanitize=address -fsanitize=undefined -fno-sanitize-recover=undefined)
HSAN=()
for f in "${SAN[@]}"; do HSAN+=(-Xarch_host "$f"); done
DBG=(-fno-omit-frame-pointer -g -O1)
NOPK=(-Xclang -target-feature -Xclang -packed-fp32-ops)
objs=()
for f in jh_api.cpp jh_gguf.cpp; do
    o="$OUT/${f%.*}.o"
    "$HIPCC" -std=c++17 -fPIC "${SAN[@]}" "${DBG[@]}" -c "$CSRC/$f" -o "$o"
    objs+=("$o")
done
for f in jh_gemv.hip jh_gemv_staged.hip jh_quant.hip jh_mfma.hip jh_decode.hip; do
    o="$OUT/${f%.*}.o"
    "$HIPCC" --offload-arch=gfx950 -std=c++17 -fPIC "${NOPK[@]}" "${HSAN[@]}" "${DBG[@]}" -c "$CSRC/$f" -o "$o" &
    objs+=("$o")
done
wait
"$HIPCC" -std=c++17 "${SAN[@]}" "${DBG[@]}" -c "$HERE/san_driver.cpp" -o "$OUT/san_driver.o"
"$HIPCC" --offload-arch=gfx950 "${HSAN[@]}" "$OUT/san_driver.o" "${objs[@]}" -o "$OUT/san_driver"
echo "$OUT/san_driver"
