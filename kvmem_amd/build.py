"""Build the in-tree native libraries.

  kvmem_amd/libkvrecall.so   HIP kernels + the C ABI of include/kvrecall.h (gfx950)
  kvmem_amd/libkvmem_hip.so  C++ host layer (include/kvmem_hip/*.hpp, llama_kvmem_hooks.h) over it
  tests/cpp/build/test_host  C++ test of the host layer (links the oracle as checker)
  oracle/liboracle.so        the CPU restatement used by tests (checker only)
  oracle/_ref/*.so           the reference's own host sources, when present
  tests/cpp/build/test_reference_boundary
                             the adapter glue against the reference's headers
                             and host library (test only, when present)

Every call recompiles (no stale-object reuse).  Objects are compiled in
parallel and linked with hipcc.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kvmem_amd", "csrc")
LIB = os.path.join(ROOT, "kvmem_amd", "libkvrecall.so")
HOST_LIB = os.path.join(ROOT, "kvmem_amd", "libkvmem_hip.so")
HOST_SRCS = [os.path.join(ROOT, "kvmem_amd", "host", f) for f in ("kvmem_hip.cpp", "kvmem_memory.cpp", "kvmem_hooks.cpp")]
HOST_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_host.cpp")
HOST_TEST = os.path.join(ROOT, "tests", "cpp", "build", "test_host")
ORACLE = os.path.join(ROOT, "oracle")
ARCH = os.environ.get("KVR_OFFLOAD_ARCH", "gfx950")

SOURCES = ["kvr_kernels.hip", "kvr_attention.hip", "kvr_scratch.hip", "kvr_capi.cpp", "kvr_policy.cpp"]
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # Packed FP32 VALU ops stay disabled: the compiler's own v_pk_* forms are
    # not used anywhere in this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose: bool):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l
                    and "not a recognized feature for this target" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_library(verbose: bool = False) -> str:
    hipcc = _hipcc()
    tmp = tempfile.mkdtemp(prefix="kvr_build_")
    try:
        objs = []
        cmds = []
        for src in SOURCES:
            obj = os.path.join(tmp, os.path.splitext(src)[0] + ".o")
            objs.append(obj)
            cmds.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
            for f in [ex.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp_lib = LIB + ".tmp"
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp_lib, *objs], verbose)
        os.replace(tmp_lib, LIB)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return LIB


def build_host(verbose: bool = False) -> str:
    """The C++ host layer: host code only, linked against libkvrecall.so."""
    hipcc = _hipcc()
    tmp = HOST_LIB + ".tmp"
    _run([hipcc, "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
          *HOST_SRCS, "-o", tmp, "-L", os.path.dirname(LIB), "-lkvrecall", "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


MEMORY_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_memory.cpp")
MEMORY_TEST = os.path.join(ROOT, "tests", "cpp", "build", "test_memory")


def _build_cpp_test(src: str, exe: str, verbose: bool) -> str:
    """A C++ test program against the host layer, the C ABI and the oracle."""
    hipcc = _hipcc()
    os.makedirs(os.path.dirname(exe), exist_ok=True)
    tmp = exe + ".tmp"
    libdir = os.path.dirname(LIB)
    _run([hipcc, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"), "-I", ORACLE, src,
          "-o", tmp, "-L", libdir, "-lkvmem_hip", "-lkvrecall", "-L", ORACLE, "-loracle",
          f"-Wl,-rpath,{libdir}", f"-Wl,-rpath,{ORACLE}", "-Wl,-rpath,$ORIGIN/../../../kvmem_amd",
          "-Wl,-rpath,$ORIGIN/../../../oracle", "-ldl"], verbose)
    os.replace(tmp, exe)
    return exe


def build_host_test(verbose: bool = False) -> str:
    """tests/cpp/test_host.cpp and tests/cpp/test_memory.cpp."""
    _build_cpp_test(MEMORY_TEST_SRC, MEMORY_TEST, verbose)
    return _build_cpp_test(HOST_TEST_SRC, HOST_TEST, verbose)


REF_INCLUDE = os.path.join(os.environ.get("KVR_REFERENCE_ROOT", "/root/reference"), "kvmem", "include")
REF_LIB = os.path.join(ORACLE, "_ref", "libkvmem_ref.so")
BOUNDARY_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_reference_boundary.cpp")
BOUNDARY_TEST = os.path.join(ROOT, "tests", "cpp", "build", "test_reference_boundary")


def build_boundary_test(verbose: bool = False) -> str:
    """tests/cpp/test_reference_boundary.cpp: the adapter glue compiled against
    the reference's own headers and linked with its host library (oracle/_ref).
    Built only where the reference tree is present; test-only."""
    if not (os.path.isdir(REF_INCLUDE) and os.path.exists(REF_LIB)):
        return ""
    hipcc = _hipcc()
    os.makedirs(os.path.dirname(BOUNDARY_TEST), exist_ok=True)
    tmp = BOUNDARY_TEST + ".tmp"
    libdir = os.path.dirname(LIB)
    refdir = os.path.dirname(REF_LIB)
    _run([hipcc, "-O2", "-std=c++17", "-Wall", "-I", REF_INCLUDE, "-I", os.path.join(ROOT, "include"),
          BOUNDARY_TEST_SRC, "-o", tmp, "-L", libdir, "-lkvmem_hip", "-lkvrecall", "-L", refdir, "-lkvmem_ref",
          "-Wl,-rpath,$ORIGIN/../../../kvmem_amd", "-Wl,-rpath,$ORIGIN/../../../oracle/_ref"], verbose)
    os.replace(tmp, BOUNDARY_TEST)
    return BOUNDARY_TEST


def build_oracle(verbose: bool = False) -> None:
    jobs = str(min(8, os.cpu_count() or 1))
    _run(["make", "-C", ORACLE, "-B", f"-j{jobs}", "all"], verbose)


def build_all(verbose: bool = False) -> None:
    build_library(verbose)
    build_host(verbose)
    build_oracle(verbose)
    build_host_test(verbose)
    build_boundary_test(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print(LIB)
