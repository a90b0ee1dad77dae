"""Runs the C++ unit tests of the dispatch layer (tests/cpp/test_c3core.cpp),
one pytest case per C++ test.  CPU tests use host tensors and a test kernel
factory; gpu_* tests run the registry / hot-path / backward-capture flow on
HIP device tensors with the real gfx950 kernels and check them against the
oracle."""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "c3core_tests"


def _names():
    if not BIN.exists():
        return []
    out = subprocess.run([str(BIN), "--list"], capture_output=True, text=True, timeout=60)
    return [n for n in out.stdout.split() if n]


NAMES = _names()
CPU_NAMES = [n for n in NAMES if not n.startswith("gpu_")]
GPU_NAMES = [n for n in NAMES if n.startswith("gpu_")]


def _run(name, tmp_path):
    env = dict(os.environ)
    env["C3_AOT_CACHE_DIR"] = str(tmp_path)  # keep the JIT cache out of $HOME
    p = subprocess.run([str(BIN), name], capture_output=True, text=True, timeout=600, env=env)
    assert p.returncode == 0 and f"PASS {name}" in p.stdout, p.stdout + p.stderr


def test_binary_built():
    assert BIN.exists(), "tests/cpp/c3core_tests is not built: run __graft_entry__.build()"
    assert CPU_NAMES and GPU_NAMES


@pytest.mark.parametrize("name", CPU_NAMES)
def test_cpp(name, tmp_path):
    _run(name, tmp_path)


@pytest.mark.gpu
@pytest.mark.parametrize("name", GPU_NAMES)
def test_cpp_gpu(name, tmp_path):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    _run(name, tmp_path)


@pytest.mark.parametrize("san", ["tsan", "asan"])
def test_cpu_tests_under_sanitizer(san, tmp_path):
    """Every CPU C++ test, with the dispatch layer (registry, hot-path
    manager's background compiles, backward capture, JIT cache, caching pool)
    built under ThreadSanitizer or AddressSanitizer: all pass and the
    sanitizer reports nothing."""
    exe = ROOT / "tests" / "cpp" / "san" / f"c3core_tests_{san}"
    assert exe.exists(), f"{exe} is not built: run __graft_entry__.build()"
    env = dict(os.environ)
    env["C3_AOT_CACHE_DIR"] = str(tmp_path)
    env["TSAN_OPTIONS"] = "halt_on_error=1 second_deadlock_stack=1"
    env["ASAN_OPTIONS"] = "halt_on_error=1 detect_leaks=1"
    p = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    out = p.stdout + p.stderr
    assert "Sanitizer" not in out, out[-4000:]
    assert p.returncode == 0, out[-4000:]
    assert out.count("PASS ") == len(CPU_NAMES), out[-2000:]
