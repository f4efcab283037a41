"""The C ABI library loads without a GPU and exports every entry point the
header declares, and the Python binding declares the same set."""
import os
import re
import subprocess

from golem_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "golem_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "gx_matmul_q4_0" in names and "gx_matmul_q6_k" in names and "gx_quantize_q8_0" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    lib = capi.load()  # loads without a device: no call is made
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (gx_[a-z0-9_]+)", out))
    assert set(declared()) <= exported


def test_binding_matches_header():
    assert sorted(capi.exported_names()) == declared()


def test_last_error_callable_without_device():
    assert isinstance(capi.last_error(), str)
