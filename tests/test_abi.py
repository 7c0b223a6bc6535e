"""The C ABI library: it loads without a GPU and exports what include/g4hip.h declares."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "g4hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g4_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("g4_init", "g4_alloc", "g4_upload", "g4_download", "g4_w4_load",
                 "g4_w4_linear", "g4_w4_dequant", "g4_ple_create", "g4_ple_gather",
                 "g4_bf16_head"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import g4hip
    if not os.path.exists(g4hip.LIB_PATH):
        pytest.fail("libg4hip.so is not built (python3 gemma4-js_amd/build.py)")
    out = subprocess.run(["nm", "-D", "--defined-only", g4hip.LIB_PATH],
                         stdout=subprocess.PIPE, text=True, check=True).stdout
    exported = set(l.split()[-1] for l in out.splitlines() if l.strip())
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    # the Python binding describes exactly the declared set
    assert sorted(g4hip.SIGNATURES) == declared_functions()
    # nothing else leaks out with a g4_ prefix
    extra = sorted(n for n in exported if n.startswith("g4_") and n not in declared_functions())
    assert not extra, extra


def test_library_loads_and_rejects_use_before_init():
    import g4hip
    L = g4hip.lib()
    import ctypes
    p = ctypes.c_void_p()
    assert L.g4_alloc(16, ctypes.byref(p)) == g4hip.G4_E_STATE
    assert b"g4_init" in L.g4_last_error()
