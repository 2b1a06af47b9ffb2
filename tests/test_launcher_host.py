"""The launch ring of the library (stwo-ml_amd/csrc/launcher.h) on the host: every
submitted closure runs once, in submission order, across ring wrap-around; the first
error is kept and cleared once taken; the thread sleeps when idle and wakes on the next
submission; destruction drains what is queued; a closure of almost a slot's size keeps
its bytes; errors stay with the ring whose launch returned them.  Host work stands in for the HIP launches, so no GPU is needed."""
import ctypes as C
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "native", "launcher_host.cpp")
OUT = os.path.join(ROOT, "tests", "native", "_build", "liblauncher_host.so")
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.fixture(scope="module")
def lt():
    deps = [SRC, os.path.join(ROOT, "stwo-ml_amd", "csrc", "launcher.h")]
    if not os.path.exists(OUT) or os.path.getmtime(OUT) < max(os.path.getmtime(d) for d in deps):
        if not os.path.exists(CLANG):
            pytest.skip("clang++ from ROCm not available")
        os.makedirs(os.path.dirname(OUT), exist_ok=True)
        subprocess.run([CLANG, "-O2", "-std=c++17", "-shared", "-fPIC", "-pthread", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include", "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-o", OUT, SRC,
                        "-lamdhip64"], check=True)
    lib = C.CDLL(OUT)
    for f in ("lt_order", "lt_destroy_pending"):
        getattr(lib, f).argtypes = [C.c_int]
    return lib


def test_order_and_wraparound(lt):
    assert lt.lt_order(5) == 0
    assert lt.lt_order(1000) == 0  # about four times the ring


def test_first_error_kept(lt):
    assert lt.lt_error() == 0


def test_sleep_and_wake(lt):
    assert lt.lt_sleep_wake() == 0


def test_destroy_drains(lt):
    assert lt.lt_destroy_pending(300) == 0


def test_large_closure(lt):
    assert lt.lt_big_closure() == 0


def test_errors_stay_with_their_ring(lt):
    assert lt.lt_errors_per_ring() == 0

