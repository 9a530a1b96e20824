"""The FSTEngine-shaped C++ adapter compiles against the public headers with
g++ and behaves as the reference members do (host side on CPU; end to end on
the GPU)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpp", "adapter_check.cpp")
OUT = os.path.join(ROOT, "tests", "cpp", "_build", "adapter_check")


def build(fa):
    fa.lib()
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    libdir = os.path.dirname(fa.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), SRC,
                    "-L", libdir, "-lfst_hip", "-Wl,-rpath," + libdir, "-o", OUT], check=True)
    return OUT


def test_adapter_compiles_and_reports_missing_gpu(fa):
    exe = build(fa)
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK):
        pytest.skip("a GPU is visible")
    r = subprocess.run([exe, "cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ADAPTER CPU OK" in r.stdout


@pytest.mark.gpu
def test_adapter_end_to_end_on_gpu(fa):
    exe = build(fa)
    print("[gpu-test] adapter_check gpu", flush=True)
    r = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ADAPTER GPU OK" in r.stdout
