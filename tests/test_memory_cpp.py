"""The llama.cpp hooks, the memory-factory hook and RecallMemory's
memory-backend side (include/kvmem_hip/llama_kvmem_hooks.h,
kvmem_memory.hpp) through tests/cpp/test_memory.cpp, which plays the engine
with its own tensor and model types."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "build", "test_memory")


def _run(mode, timeout):
    assert os.path.exists(EXE), "run __graft_entry__.build() first"
    r = subprocess.run([EXE, mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_hooks_cpu():
    assert _run("--cpu", 60).count("PASS") == 1


@pytest.mark.gpu
def test_hooks_gpu():
    assert _run("--gpu", 110).count("PASS") == 1
