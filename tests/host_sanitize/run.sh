#!/usr/bin/env bash
# Build the library's host code (store.hip, host_rows.hip, runtime.hip) under a sanitizer and run
# driver.cpp against it, on the CPU:  bash tests/host_sanitize/run.sh address|thread
# The objects and the driver go to $TMPDIR (default /tmp), never into the repository.
set -euo pipefail
SAN=${1:-address}
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
OUT=${TMPDIR:-/tmp}/evs-sanitize-$SAN
CS=$ROOT/everserve_amd/csrc
CXX=/opt/rocm/llvm/bin/clang++
mkdir -p "$OUT"
for f in store host_rows runtime; do
  /opt/rocm/bin/hipcc -O1 -g -std=c++17 -fPIC --offload-arch=gfx950 -Xclang -target-feature \
    -Xclang -packed-fp32-ops -I"$ROOT/include" -I"$CS" -Xarch_host -fsanitize=$SAN \
    -c "$CS/$f.hip" -o "$OUT/$f.o"
done
$CXX -O1 -g -std=c++17 -fsanitize=$SAN -c "$HERE/driver.cpp" -o "$OUT/driver.o"
$CXX -fsanitize=$SAN "$OUT/driver.o" "$OUT/store.o" "$OUT/host_rows.o" "$OUT/runtime.o" \
  -L/opt/rocm/lib -lamdhip64 -lpthread -Wl,-rpath,/opt/rocm/lib -o "$OUT/driver"
"$OUT/driver"
