"""The adapter glue (conversions, the MemoryTransfer forwarder, the scorer
on the reference's own RawKvStore) compiled against the reference's public
headers and linked with its host library from oracle/_ref, through
tests/cpp/test_reference_boundary.cpp.  Skipped where that program was not
built (no reference tree at build time)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "build", "test_reference_boundary")


def _run(mode, timeout):
    if not os.path.exists(EXE):
        pytest.skip("reference boundary test not built (no reference tree at build time)")
    r = subprocess.run([EXE, mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_boundary_cpu():
    assert _run("--cpu", 60).count("PASS") == 2


@pytest.mark.gpu
def test_boundary_gpu():
    assert _run("--gpu", 110).count("PASS") == 2
