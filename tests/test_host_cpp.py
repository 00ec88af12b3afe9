"""The C++ host layer (include/kvmem_hip/kvmem_hip.hpp) through its own C++
test program, tests/cpp/test_host.cpp, built in-tree by __graft_entry__.build()."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "build", "test_host")


def _run(mode, timeout):
    assert os.path.exists(EXE), "run __graft_entry__.build() first"
    r = subprocess.run([EXE, mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_host_layer_cpu():
    out = _run("--cpu", 60)
    assert out.count("PASS") == 8


@pytest.mark.gpu
def test_host_layer_gpu():
    out = _run("--gpu", 110)
    assert out.count("PASS") == 12
