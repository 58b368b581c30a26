"""The C++ host API (include/viper/*.h, viper_amd/host/*.cpp) through its own
C++ test programs (tests/cpp/), built by __graft_entry__.build()."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "bin")


def _run(name, timeout):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} not built: run __graft_entry__.build()")
    p = subprocess.run([exe], capture_output=True, text=True, timeout=timeout)
    print(p.stdout[-4000:])
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert "PASS" in p.stdout


def test_host_api_registry_and_validation():
    _run("test_host_api", 60)


@pytest.mark.gpu
def test_host_api_gpu_parity():
    _run("test_host_api_gpu", 170)
