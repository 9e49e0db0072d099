"""CPU checks of the C-ABI boundary: the built library loads and exports every
symbol include/seeker_hip.h declares, and the Python binding covers them.
No compute call is made (there is no GPU here)."""
import ctypes as C
import os
import re
import subprocess

from seeker_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "seeker_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(sh_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ["sh_engine_create", "sh_model_load_gguf", "sh_kv_truncate", "sh_forward_full", "sh_spec_step",
              "sh_accept_sample", "sh_gemv_quant", "sh_kv_compact", "sh_last_error"]:
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(N.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", N.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (sh_[a-z0-9_]+)", out))
    assert set(declared_symbols()) <= exported


def test_python_binding_covers_header():
    assert set(declared_symbols()) == set(N.SIGNATURES)


def test_version_string():
    assert N.lib().sh_version().decode().startswith("seeker-hip")


def test_gfx950_code_object_present():
    # the HIP fat binary inside the library names its gfx950 code object
    data = open(N.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
