"""CPU checks of the C ABI: the library loads without a GPU and exports every
entry point include/wm_hip.h declares (no compute calls are made here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wm_hip.h")
LIB = os.path.join(ROOT, "whitematter_amd", "libwm_hip.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(wm_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    fns = declared_functions()
    for name in ("wm_init", "wm_binary", "wm_binary_bwd", "wm_unary", "wm_unary_bwd", "wm_reduce",
                 "wm_reduce_bwd", "wm_softmax_fwd", "wm_softmax_bwd", "wm_log_softmax_fwd",
                 "wm_log_softmax_bwd", "wm_fill", "wm_f32_to_f16_rtz", "wm_f16_to_f32"):
        assert name in fns


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    missing = [f for f in declared_functions() if not hasattr(lib, f)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_binding_matches_header():
    """Every header entry point has a ctypes signature in the binding."""
    from whitematter_amd import _lib
    missing = [f for f in declared_functions() if f not in _lib._SIGS and f != "wm_last_error"]
    assert not missing, missing


def test_header_compiles_as_c():
    """The header is plain C (no torch / HIP types in the signatures)."""
    import subprocess
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "t.c")
        with open(src, "w") as f:
            f.write('#include "wm_hip.h"\nint main(void){return (int)sizeof(&wm_binary);}\n')
        r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                            "-c", src, "-o", os.path.join(d, "t.o")], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
