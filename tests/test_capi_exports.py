"""The C-ABI library loads and exports every entry point that
include/kvrecall.h declares; host-only helpers behave.  No device compute."""
import ctypes as C
import os
import subprocess
import sys

import pytest

from kvmem_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_built_in_tree():
    assert os.path.exists(_capi.LIB_PATH), "run __graft_entry__.build() first"


def test_every_declared_symbol_is_exported():
    lib = C.CDLL(_capi.LIB_PATH)
    declared = _capi.header_symbols()
    assert len(declared) >= 25
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python view binds each of them with a signature
    assert sorted(_capi._SIGNATURES) == declared


def test_exports_match_nm():
    out = subprocess.run(["nm", "-D", "--defined-only", _capi.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T kvr_" in line}
    assert exported == set(_capi.header_symbols())


def test_status_strings_and_workspace_arithmetic():
    lib = _capi.lib()
    assert lib.kvr_status_string(_capi.OK) == b"ok"
    assert lib.kvr_status_string(_capi.ERR_BUDGET).startswith(b"mandatory")
    # logits: 1 lane x 1 row x 32 heads x 512 pages x 8 B = 131072; two
    # statistics per softmax row: 32 x 16 B = 512; qpack 8192 -> 256-aligned
    assert lib.kvr_workspace_bytes(1, 512, 1, 32, 8, 128) == 131072 + 512 + 8192
    assert lib.kvr_workspace_bytes(0, 7, 1, 1, 1, 1) == 256 + 256 + 256


def test_null_context_is_rejected():
    lib = _capi.lib()
    assert lib.kvr_check(None, None) == _capi.ERR_INVALID
    assert b"null context" in lib.kvr_last_error()
    assert lib.kvr_destroy(None) == _capi.OK


def test_header_compiles_as_c():
    """include/kvrecall.h is plain C: it compiles with gcc -std=c99."""
    src = '#include "kvrecall.h"\nint main(void){kvr_status s = KVR_OK; return (int)s;}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        "-x", "c", "-"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stdout


def test_struct_layouts_match_header(tmp_path):
    """The ctypes mirrors of the descriptor structs have the C sizes and
    field offsets of include/kvrecall.h."""
    structs = {"kvr_key_history": _capi.KeyHistory, "kvr_query": _capi.Query, "kvr_plane": _capi.Plane,
               "kvr_layer_recall": _capi.LayerRecall, "kvr_rope": _capi.Rope,
               "kvr_attention_sample": _capi.AttentionSample, "kvr_page_graph": _capi.PageGraph}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "kvrecall.h"', 'int main(void) {']
    for cname, py in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ['return 0;', '}']
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    for cname, py in structs.items():
        assert int(got[cname]) == C.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(py, fname).offset, (cname, fname)
