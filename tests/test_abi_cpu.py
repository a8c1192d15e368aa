"""CPU-side checks of the C-ABI boundary (no GPU needed, no compute calls):
every function declared in include/*.h is exported by libhip_bridge.so, the ctypes bindings
(ziglm_amd/bridge.py for hip_bridge.h, ziglm_amd/gguf.py for zl_gguf.h) cover exactly those
functions, and the library loads without initialising a device."""
import os
import re
import subprocess

import pytest

from ziglm_amd import bridge, gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {"hip_bridge.h": "hip_", "zl_gguf.h": "zl_"}


def declared_functions(header=None):
    names = set()
    for h, prefix in HEADERS.items():
        if header and h != header:
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text))
    return sorted(names)


def test_header_parses():
    names = declared_functions()
    assert "hip_qk_norm_rope_kv" in names and "hip_embed_lookup_batch" in names
    assert len(names) >= 50


def test_library_exports_every_declared_symbol():
    if not os.path.exists(bridge.LIB_PATH):
        pytest.fail("libhip_bridge.so is not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", bridge.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT ((?:hip|zl)_\w+)$", out, flags=re.M))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_matches_header():
    assert sorted(bridge.SIGNATURES) == declared_functions("hip_bridge.h")
    assert sorted(gguf.SIGNATURES) == declared_functions("zl_gguf.h")
    gguf.lib()  # binds every zl_ symbol


def test_library_loads_and_binds():
    b = bridge.load()
    assert "gfx950" in b.version()
    assert b.hip_bridge_last_error() == 0
    assert b.hip_bridge_error_string(-2).decode().startswith("unsupported")
