#!/usr/bin/env bash
# Host-side sanitizer runs of the block manager and the C ABI's host paths.
#
# Builds libkrillhip.so twice, once with AddressSanitizer and once with
# ThreadSanitizer on the host code of capi.cpp and block_manager.cpp (the
# kernel objects are the ones the Makefile built, not instrumented: device
# code cannot be), and runs the host-only-pool tests against each copy:
# tests/test_block_manager.py (including the 8-thread hammer) and
# tests/test_abi.py.  The copies live in a temporary tree, so the package's
# own library is never replaced.  CPU only; exits non-zero on any report.
#
# Usage: krill_amd/csrc/sanitize.sh [address|thread ...]   (default: both)
set -euo pipefail

HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
ROOT="$(cd "$HERE/../.." && pwd)"
CXX=${CXX:-/opt/rocm/llvm/bin/clang++}
ARCH=${ARCH:-gfx950}
RT="$("$CXX" -print-resource-dir)/lib/linux"
SANS=("$@")
[ ${#SANS[@]} -eq 0 ] && SANS=(address thread)

for o in kv_ops attn_valu attn_mfma scratch; do
  [ -f "$HERE/_build/$o.o" ] || { echo "missing $HERE/_build/$o.o: run make in $HERE first" >&2; exit 2; }
done

for san in "${SANS[@]}"; do
  case "$san" in
    address) rtlib="$RT/libclang_rt.asan-x86_64.so"; env_opts=(ASAN_OPTIONS=detect_leaks=0:abort_on_error=1) ;;
    thread) rtlib="$RT/libclang_rt.tsan-x86_64.so"; env_opts=(TSAN_OPTIONS=halt_on_error=1:report_signal_unsafe=0) ;;
    *) echo "unknown sanitizer $san" >&2; exit 2 ;;
  esac
  out="$HERE/_build/san_$san"
  mkdir -p "$out"
  echo "== $san: build"
  # capi.cpp is HIP source (device helpers in kdev.hpp): instrument its host half only
  "$CXX" -x hip --offload-arch="$ARCH" -std=c++17 -O1 -g -fPIC -fno-omit-frame-pointer \
    -Xarch_host -fsanitize="$san" -c "$HERE/capi.cpp" -o "$out/capi.o" 2>&1 | grep -v "option-ignored\|packed-fp32" || true
  "$CXX" -std=c++17 -O1 -g -fPIC -fno-omit-frame-pointer -fsanitize="$san" \
    -c "$HERE/block_manager.cpp" -o "$out/block_manager.o"
  "$CXX" -shared -fPIC --hip-link --offload-arch="$ARCH" -fsanitize="$san" -shared-libsan -o "$out/libkrillhip.so" \
    "$out/capi.o" "$out/block_manager.o" "$HERE/_build/kv_ops.o" "$HERE/_build/attn_valu.o" "$HERE/_build/attn_mfma.o" "$HERE/_build/scratch.o"

  tree="$(mktemp -d)"
  trap 'rm -rf "$tree"' EXIT
  mkdir -p "$tree/krill_amd"
  cp "$ROOT"/krill_amd/*.py "$tree/krill_amd/"
  cp "$out/libkrillhip.so" "$tree/krill_amd/"
  cp -r "$ROOT/include" "$ROOT/tests" "$ROOT/oracle" "$ROOT/pytest.ini" "$tree/"
  echo "== $san: tests"
  (cd "$tree" && env "${env_opts[@]}" LD_PRELOAD="$rtlib" python3 -m pytest -q -p no:cacheprovider \
    tests/test_block_manager.py tests/test_abi.py) 2>&1 | tee "$out/report.txt"
  if grep -q "ERROR: AddressSanitizer\|WARNING: ThreadSanitizer" "$out/report.txt"; then
    echo "== $san: sanitizer report (see $out/report.txt)" >&2
    exit 1
  fi
  rm -rf "$tree"
  trap - EXIT
  echo "== $san: clean"
done
