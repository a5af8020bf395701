"""Build libkvcache_amd.so (gfx950) and the C++ test programs, in-tree.

    python -m kvcache_amd.build            # library + C++ tests
    python -m kvcache_amd.build --lib-only

Sources: kvcache_amd/csrc/*.hip (device + ABI) and *.cpp (host-only C++).
Objects go to kvcache_amd/_build/, the library to kvcache_amd/libkvcache_amd.so,
test programs (tests/cpp/*.cpp) to kvcache_amd/_build/bin/.  When the reference
tree is present, its test programs that use only the API this library replaces
(tests/test_kv_manager.cu) are compiled unchanged against include/kvc into
kvcache_amd/_build/bin/ref_<name>: the drop-in check (built, never committed).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libkvcache_amd.so"
INCLUDE = ROOT / "include"
TESTS_CPP = ROOT / "tests" / "cpp"
REFERENCE = Path(os.environ.get("KVC_REFERENCE", "/root/reference"))
# reference test programs whose only includes are headers this library replaces
REFERENCE_TESTS = ["tests/test_kv_manager.cu"]

ARCH = os.environ.get("KVC_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
# kernarg preload: the first two kernel arguments arrive in scalar registers at wave
# start (the decode kernels take their work list there, so the entry is read without
# waiting for the parameter block); the compiler keeps a fallback that loads them.
DEVICE_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-mllvm", "-amdgpu-kernarg-preload-count=2"]
HOST_FLAGS = ["-x", "c++", "-O2", "-std=c++17", "-fPIC", "-Wall"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    flags = DEVICE_FLAGS if src.suffix == ".hip" else HOST_FLAGS
    _run([HIPCC, *flags, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)])
    return obj


def build_library(jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          "-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(tmp, LIB)
    return LIB


def build_cpp_tests() -> list[Path]:
    """C++ programs written against include/kvc/*.h, linked to the library."""
    out_dir = BUILD / "bin"
    out_dir.mkdir(parents=True, exist_ok=True)
    built = []
    for src in sorted(TESTS_CPP.glob("*.cpp")):
        exe = out_dir / src.stem
        _run([HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", f"-I{INCLUDE}", str(src), "-o", str(exe), f"-L{PKG}",
              "-lkvcache_amd", "-Wl,-rpath,$ORIGIN/../..", "-Wl,-rpath,/opt/rocm/lib"])
        built.append(exe)
    return built


def build_reference_tests() -> list[Path]:
    """The reference's own test programs, source unchanged, against include/kvc."""
    out_dir = BUILD / "bin"
    out_dir.mkdir(parents=True, exist_ok=True)
    built = []
    for rel in REFERENCE_TESTS:
        src = REFERENCE / rel
        if not src.exists():
            continue
        exe = out_dir / ("ref_" + src.stem)
        _run([HIPCC, "-x", "c++", "-O2", "-std=c++17", f"-I{INCLUDE / 'kvc'}", str(src), "-o", str(exe), f"-L{PKG}",
              "-lkvcache_amd", "-Wl,-rpath,$ORIGIN/../..", "-Wl,-rpath,/opt/rocm/lib"])
        built.append(exe)
    return built


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    a = ap.parse_args(argv)
    print(f"built {build_library(a.jobs)}")
    if not a.lib_only:
        for exe in build_cpp_tests() + build_reference_tests():
            print(f"built {exe}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
