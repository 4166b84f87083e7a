#!/bin/bash
# AddressSanitizer and UndefinedBehaviorSanitizer over the host code the CPU
# tests drive: the oracle's C restatement (oracle/adi_oracle.c, built with
# gcc) and the host side of libadi_hip.so (the GGUF reader and its
# malformed-file rejections, the tensor checks, the C ABI's argument checks;
# built with hipcc, sanitizers on the host pass only). Each build goes to
# $OUT and the CPU tests load it in place of the in-tree library through
# ADI_ORACLE_LIBRARY / ADI_HIP_LIBRARY, with the matching sanitizer runtime
# preloaded (gcc's for the oracle, clang's for the HIP library: one runtime
# per process). Any sanitizer report aborts the test process.
#
#     bash tests/sanitize.sh            # about three minutes on 8 cores
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/.." && pwd)
OUT=${OUT:-${TMPDIR:-/tmp}/adi_sanitize}
mkdir -p "$OUT/obj"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1:halt_on_error=1
export UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1

echo "== oracle (gcc, -fsanitize=address,undefined)"
gcc -std=c11 -O1 -g -fPIC -ffp-contract=off -fopenmp -fno-omit-frame-pointer \
    -fsanitize=address,undefined -fno-sanitize-recover=undefined \
    -shared -o "$OUT/liboracle.so" "$ROOT/oracle/adi_oracle.c" -lm
# libstdc++ is preloaded with the runtime: C++ code that throws (the compiled
# reference's rejections, the library's own error paths) needs the runtime's
# __cxa_throw interceptor to find it at start-up
STDCXX=$(gcc -print-file-name=libstdc++.so.6)
GCC_ASAN=$(gcc -print-file-name=libasan.so)
ADI_ORACLE_LIBRARY="$OUT/liboracle.so" LD_PRELOAD="$GCC_ASAN $STDCXX" \
    python -m pytest "$ROOT/tests/test_oracle_cpu.py" "$ROOT/tests/test_attention_cpu.py" \
    "$ROOT/tests/test_decode_cpu.py" -q -p no:cacheprovider -m "not gpu"

echo "== libadi_hip.so host code (hipcc, host pass -fsanitize=address,undefined)"
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
FLAGS=(-O1 -g -std=c++20 -fPIC --offload-arch=gfx950 -I "$ROOT/include" -I "$ROOT/adi_amd/csrc"
       -Xclang -target-feature -Xclang -packed-fp32-ops -fno-omit-frame-pointer
       -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined
       -Xarch_host -fno-sanitize-recover=undefined)
objs=()
for src in "$ROOT"/adi_amd/csrc/*.hip "$ROOT"/adi_amd/csrc/*.cpp; do
    obj="$OUT/obj/$(basename "$src").o"
    lang=()
    [[ "$src" == *.cpp ]] && lang=(-x hip)
    "$HIPCC" "${FLAGS[@]}" "${lang[@]}" -c "$src" -o "$obj" 2>"$obj.log" &
    objs+=("$obj")
done
wait
"$HIPCC" -shared --offload-arch=gfx950 -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined \
    -shared-libasan -o "$OUT/libadi_hip.so" "${objs[@]}"
CLANG_ASAN=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)
ADI_HIP_LIBRARY="$OUT/libadi_hip.so" LD_PRELOAD="$CLANG_ASAN $STDCXX" \
    python -m pytest "$ROOT/tests/test_gguf_cpu.py" "$ROOT/tests/test_capi_cpu.py" \
    -q -p no:cacheprovider -m "not gpu"
echo "== sanitizers clean"
