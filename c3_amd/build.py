"""Build recipe for the gfx950 backend (no cmake needed).

Products, all in-tree under c3_amd/lib/ (git-ignored, shipped with the tree):
  *.hsaco        gfx950 code objects, one per kernel family (hipcc --genco)
  libc3hip.so    host C-ABI library (include/c3hip.h) that loads them
  libc3core.so   C++ dispatch layer (registry, hot-path manager, JIT cache)
  c3core_tests   C++ unit-test runner for the dispatch layer (CPU only)
  san/c3core_tests_{tsan,asan}  the same tests with the dispatch layer built
                 under ThreadSanitizer / AddressSanitizer (host code)
and the oracle (test infrastructure) under oracle/liboracle.so.

Run:  python -m c3_amd.build   (or __graft_entry__.build()).
"""
from __future__ import annotations

import os
import shlex
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "c3_amd"
CSRC = PKG / "csrc"
LIB = PKG / "lib"
INCLUDE = ROOT / "include"
ORACLE = ROOT / "oracle"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed fp32 ops stay off in all device code; hipcc would otherwise form
# v_pk_* fp32 instructions from ordinary float code.
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
DEVICE_FLAGS = ["--genco", "--no-gpu-bundle-output", f"--offload-arch={ARCH}", "-O3", "-std=c++17", *NO_PACKED_FP32]

KERNELS = ["elementwise", "gemm_f32", "gemm_bf16", "reduce", "loss"]
RUNTIME_SOURCES = ["runtime/c3hip_runtime.cpp", "runtime/c3hip_ops.cpp", "runtime/c3hip_loss.cpp"]
HOST_SOURCES = sorted(p.name for p in (CSRC / "host" / "src").glob("*.cpp"))
TESTS_CPP = ROOT / "tests" / "cpp"


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed ({proc.returncode}): {shlex.join(cmd)}")


def build_code_objects() -> list[Path]:
    LIB.mkdir(parents=True, exist_ok=True)
    jobs = []
    for k in KERNELS:
        src = CSRC / "kernels" / f"{k}.hip"
        out = LIB / f"{k}.hsaco"
        jobs.append(([HIPCC, *DEVICE_FLAGS, f"-I{CSRC / 'kernels'}", str(src), "-o", str(out)], out))
    with ThreadPoolExecutor(max_workers=min(4, len(jobs))) as ex:
        list(ex.map(lambda j: _run(j[0]), jobs))
    return [j[1] for j in jobs]


def build_runtime() -> Path:
    out = LIB / "libc3hip.so"
    srcs = [str(CSRC / s) for s in RUNTIME_SOURCES]
    # Host-only C++: no device code in these files, so hipcc only supplies the
    # HIP headers and links libamdhip64.  c3hip_noalloc.hip holds a static
    # device array (the no-alloc entry point's scratch), so it is compiled as
    # HIP for gfx950 and its fat binary is linked into the library.
    noalloc_obj = LIB / "c3hip_noalloc.o"
    _run([HIPCC, "-x", "hip", f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-c", "-Wall",
          *NO_PACKED_FP32, f"-I{INCLUDE}", f"-I{CSRC / 'runtime'}", str(CSRC / "runtime" / "c3hip_noalloc.hip"),
          "-o", str(noalloc_obj)])
    cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{INCLUDE}", f"-I{CSRC / 'runtime'}",
           *srcs, "-x", "none", str(noalloc_obj), f"--offload-arch={ARCH}", "-o", str(out), "-ldl"]
    _run(cmd)
    return out


def build_core() -> Path:
    """libc3core.so: the C++ dispatch layer (registry, hot-path manager, region
    registry, JIT cache, engine, backward capture) over libc3hip.so."""
    out = LIB / "libc3core.so"
    srcs = [str(CSRC / "host" / "src" / s) for s in HOST_SOURCES]
    cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{CSRC / 'host' / 'include'}", f"-I{INCLUDE}",
           *srcs, "-o", str(out), f"-L{LIB}", "-lc3hip", "-Wl,-rpath,$ORIGIN", "-lpthread"]
    _run(cmd)
    return out


def build_core_tests() -> Path:
    """tests/cpp/c3core_tests: unit-test runner of the dispatch layer."""
    out = TESTS_CPP / "c3core_tests"
    cmd = [HIPCC, "-O1", "-std=c++17", "-Wall", f"-I{CSRC / 'host' / 'include'}", f"-I{INCLUDE}", f"-I{TESTS_CPP}",
           f"-I{ORACLE}", str(TESTS_CPP / "test_c3core.cpp"), "-o", str(out), f"-L{LIB}", "-lc3core", "-lc3hip",
           f"-L{ORACLE}", "-loracle", f"-Wl,-rpath,{LIB}", f"-Wl,-rpath,{ORACLE}", "-Wl,-rpath,$ORIGIN/../../c3_amd/lib",
           "-Wl,-rpath,$ORIGIN/../../oracle", "-lpthread"]
    _run(cmd)
    return out


SANITIZERS = {"tsan": ["-Xarch_host", "-fsanitize=thread"],
              "asan": ["-Xarch_host", "-fsanitize=address", "-fno-omit-frame-pointer"]}


def build_sanitized_tests() -> list[Path]:
    """tests/cpp/san/c3core_tests_{tsan,asan}: the dispatch layer's sources and
    its unit tests in one executable, host code built with ThreadSanitizer or
    AddressSanitizer (device code is not instrumented; the CPU tests launch
    none)."""
    out_dir = TESTS_CPP / "san"
    out_dir.mkdir(parents=True, exist_ok=True)
    srcs = [str(CSRC / "host" / "src" / s) for s in HOST_SOURCES]
    jobs = []
    for name, flags in SANITIZERS.items():
        out = out_dir / f"c3core_tests_{name}"
        jobs.append(([HIPCC, "-O1", "-g", "-std=c++17", *flags, f"-I{CSRC / 'host' / 'include'}", f"-I{INCLUDE}",
                      f"-I{TESTS_CPP}", f"-I{ORACLE}", str(TESTS_CPP / "test_c3core.cpp"), *srcs, "-o", str(out),
                      f"-L{LIB}", "-lc3hip", f"-L{ORACLE}", "-loracle", "-Wl,-rpath,$ORIGIN/../../../c3_amd/lib",
                      "-Wl,-rpath,$ORIGIN/../../../oracle", "-lpthread"], out))
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        list(ex.map(lambda j: _run(j[0]), jobs))
    return [j[1] for j in jobs]


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ORACLE), "liboracle.so"])
    return ORACLE / "liboracle.so"


def build_all(verbose: bool = False) -> None:
    built = []
    built += build_code_objects()
    built.append(build_runtime())
    built.append(build_core())
    built.append(build_oracle())
    built.append(build_core_tests())
    built += build_sanitized_tests()
    if verbose:
        for b in built:
            print(f"built {b.relative_to(ROOT)} ({b.stat().st_size} bytes)")


if __name__ == "__main__":
    build_all(verbose=True)
