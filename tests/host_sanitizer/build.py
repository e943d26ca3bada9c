"""Host-sanitized build of libqgemm.so for the CPU checks in this folder.

The device code is built as usual; the host side (argument validation,
planning, routing, the host layout helpers) is built with AddressSanitizer
and UndefinedBehaviorSanitizer (`-Xarch_host` keeps the sanitizers off the
GPU code).  Output: tests/host_sanitizer/_out/libqgemm.so.  CPU only -- no
GPU is touched by anything in this folder.
"""
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
CSRC = ROOT / "355_1_trans_amd" / "csrc"
OUT = HERE / "_out"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined"]
FLAGS = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", *SAN, "-Xarch_host", "-fno-omit-frame-pointer", "-I", str(ROOT / "include"),
         "-I", str(CSRC)]


def _cc(src):
    obj = OUT / (src.stem + ".o")
    res = subprocess.run(["/opt/rocm/bin/hipcc", *FLAGS, "-c", str(src), "-o", str(obj)], capture_output=True,
                         text=True)
    if res.returncode:
        raise SystemExit(f"{src.name}:\n{res.stderr[-4000:]}")
    return str(obj)


def main():
    OUT.mkdir(exist_ok=True)
    with ThreadPoolExecutor(8) as ex:
        objs = list(ex.map(_cc, sorted(CSRC.glob("*.hip"))))
    subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-shared", "-fPIC", *SAN, "-o",
                    str(OUT / "libqgemm.so"), *objs], check=True)
    print(OUT / "libqgemm.so")


if __name__ == "__main__":
    sys.exit(main())
