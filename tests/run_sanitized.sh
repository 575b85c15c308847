#!/bin/bash
# Host code under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU (no
# GPU needed, none used).
#
#   1. the C oracle, built with gcc and the sanitizers, runs the oracle tests
#      (every oracle function against its pins);
#   2. libtbhip.so with the sanitizers on its host code only (device code as in
#      the product) runs the C-ABI tests that need no GPU: exported symbols,
#      argument validation before any GPU call, decoder config errors.
#
# Builds go to /tmp (nothing in the tree changes).  Usage, from the repo root:
#   bash tests/run_sanitized.sh
set -euo pipefail
cd "$(dirname "$0")/.."
OUT=${TB_SAN_DIR:-/tmp/tb_sanitized}
mkdir -p "$OUT"

echo "== oracle (gcc, -fsanitize=address,undefined)"
gcc -O1 -g -fPIC -fopenmp -ffp-contract=off -fno-omit-frame-pointer \
    -fsanitize=address,undefined -fno-sanitize-recover=undefined \
    -shared -o "$OUT/liboracle.so" oracle/tb_oracle.c -lm
GCC_RT="$(gcc -print-file-name=libasan.so):$(gcc -print-file-name=libubsan.so)"
ASAN_OPTIONS=detect_leaks=0:halt_on_error=1 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \
    TB_ORACLE_SO="$OUT/liboracle.so" LD_PRELOAD="$GCC_RT" \
    python -m pytest -q -p no:cacheprovider -m "not gpu" \
        tests/test_oracle.py tests/test_oracle_v2.py tests/test_oracle_sample.py tests/test_spec_host.py

echo "== libtbhip.so, host code under the sanitizers"
python -m torchburn_amd.build --host-sanitize "$OUT/libtbhip.so"
CLANG_RT=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -n 1)
ASAN_OPTIONS=detect_leaks=0:halt_on_error=1 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \
    TB_LIB_SO="$OUT/libtbhip.so" LD_PRELOAD="$CLANG_RT" \
    python -m pytest -q -p no:cacheprovider -m "not gpu" tests/test_capi.py
echo "== sanitized runs clean"
