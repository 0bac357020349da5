#!/bin/bash
# Host-code sanitizer run (CPU only, no GPU needed): the library's host C++
# (raggedroute_amd/csrc/*.cpp: operator wrappers, dispatch, chain entries,
# graphs, the route-trace reader) and the CPU oracle are built with
# AddressSanitizer + UndefinedBehaviorSanitizer by g++/gcc and linked with the
# normally built HIP objects; the CPU test tier (-m "not gpu": oracle against
# the golden vectors, host contracts of every C-ABI entry, the route-trace
# reader on the fixture and on planted errors) then runs against that build.
# Any sanitizer report ends the run with a failure.
#
#   bash tests/sanitize.sh
set -euo pipefail
REPO=$(cd "$(dirname "$0")/.." && pwd)
OUT="$REPO/_build/sanitize"
ROCM=${ROCM_PATH:-/opt/rocm}
SAN="-fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer -g -O1"
mkdir -p "$OUT"
cd "$REPO"
python raggedroute_amd/build.py > /dev/null   # the HIP objects (and _build/*.hip.o)
for src in raggedroute_amd/csrc/*.cpp; do
  g++ $SAN -std=c++17 -fPIC -Wall -D__HIP_PLATFORM_AMD__ -Iinclude -Iraggedroute_amd/csrc \
      -I"$ROCM/include" -c "$src" -o "$OUT/$(basename "$src").o"
done
g++ $SAN -shared -o "$OUT/libraggedroute_amd.so" "$OUT"/*.cpp.o _build/*.hip.o \
    -L"$ROCM/lib" -lamdhip64 -Wl,-rpath,"$ROCM/lib"
gcc $SAN -std=c11 -ffp-contract=off -fPIC -shared -o "$OUT/liboracle.so" oracle/oracle.c -lm
export LD_PRELOAD="$(gcc -print-file-name=libasan.so):$(gcc -print-file-name=libubsan.so)"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1:halt_on_error=1
export UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1
export RR_LIBRARY="$OUT/libraggedroute_amd.so" RR_ORACLE_LIBRARY="$OUT/liboracle.so"
python -m pytest tests -m "not gpu" -q -p no:cacheprovider "$@"
