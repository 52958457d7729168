"""CPU checks of the C ABI: the library loads without a GPU and exports every
entry point the headers in include/ declare (no compute calls are made here)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))
LIB = os.path.join(ROOT, "whitematter_amd", "libwm_hip.so")


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(wm_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_header_declares_entry_points():
    fns = declared_functions()
    for name in ("wm_init", "wm_binary", "wm_binary_bwd", "wm_unary", "wm_unary_bwd", "wm_reduce",
                 "wm_reduce_bwd", "wm_softmax_fwd", "wm_softmax_bwd", "wm_log_softmax_fwd",
                 "wm_log_softmax_bwd", "wm_fill", "wm_f32_to_f16_rtz", "wm_f16_to_f32",
                 "wm_sgd_step", "wm_adam_step", "wm_adamw_step", "wm_rmsprop_step", "wm_grad_sumsq_accumulate",
                 "wm_clip_grad_norm_scale", "wm_clip_grad_value", "wm_grad_unscale"):
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


@pytest.mark.parametrize("header", [os.path.basename(h) for h in HEADERS])
def test_header_compiles_as_c(header):
    """Each header is plain C (no torch / HIP types in the signatures)."""
    import subprocess
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "t.c")
        with open(src, "w") as f:
            f.write('#include "%s"\nint main(void){return 0;}\n' % header)
        r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                            "-c", src, "-o", os.path.join(d, "t.o")], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
