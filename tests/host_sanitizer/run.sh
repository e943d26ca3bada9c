#!/bin/bash
# Host ASan / UBSan check of libqgemm.so on the CPU (no GPU needed or used):
# sanitized build, the CPU test suite against it, then the random-argument fuzz.
set -eo pipefail
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
python3 "$HERE/build.py"
ASAN_SO=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)
export LD_PRELOAD=$ASAN_SO ASAN_OPTIONS=detect_leaks=0:halt_on_error=1 UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
cd "$ROOT"
python3 -c "
import importlib, pathlib, sys
sys.path.insert(0, '$ROOT')
q = importlib.import_module('355_1_trans_amd'); q.LIB_PATH = pathlib.Path('$HERE/_out/libqgemm.so')
import pytest
sys.exit(pytest.main(['-x', '-q', '-m', 'not gpu', 'tests', '-p', 'no:cacheprovider']))
"
for seed in 1 2 3; do python3 "$HERE/fuzz.py" "$HERE/_out/libqgemm.so" $seed 3000; done
