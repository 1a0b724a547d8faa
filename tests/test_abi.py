"""C-ABI conformance on the CPU: the library loads, exports every entry point
that include/hip_bridge.h declares, and the structs keep the reference's
layouts (native/mlx_bridge.h:50-54, native/state_table.h:11-13)."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hip_bridge.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:rs|hb)_[A-Za-z0-9_]+)\s*\(", text)))


def test_header_declares_reference_surface():
    names = declared_functions()
    # the reference graph API, weight store and kernel entry (native/mlx_bridge.h:8-43,64)
    for n in ["rs_mlx_create", "rs_mlx_destroy", "rs_mlx_input", "rs_mlx_op", "rs_mlx_finish", "rs_mlx_version",
              "rs_mlx_cleanup", "rs_mlx_weights_create", "rs_mlx_weights_destroy", "rs_mlx_weights_load",
              "rs_mlx_parameter", "rs_mlx_kernel", "rs_mlx_weight_bytes"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    import hip_bridge

    lib = hip_bridge.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    out = subprocess.run(["nm", "-D", "--defined-only", hip_bridge.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\b((?:rs|hb)_[A-Za-z0-9_]+)$", out, flags=re.M))
    assert set(declared_functions()) <= exported


def test_struct_layouts_compile():
    src = r"""
#include <stddef.h>
#include "hip_bridge.h"
_Static_assert(sizeof(rs_qwen_config) == 132, "config");
_Static_assert(offsetof(rs_qwen_config, epsilon) == 124, "epsilon");
_Static_assert(sizeof(rs_qwen_layer) == 8, "layer");
_Static_assert(sizeof(StateId) == 40, "state id");
int main(void) { return 0; }
"""
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "layout.c")
        open(p, "w").write(src)
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), p, "-o", os.path.join(d, "a.out")],
                       check=True)


def test_failed_calls_report_and_never_throw():
    import hip_bridge

    lib = hip_bridge.load()
    err = C.create_string_buffer(64)
    # null graph handle: -1 with a message, no exception across the ABI
    assert lib.rs_mlx_input(None, 0, None, None, 0, err, 64) == -1
    assert err.value == b"invalid input descriptor"
    assert lib.rs_mlx_op(None, 0, None, 0, 0, 0.0, err, 64) == -1
    assert lib.rs_mlx_finish(None, 0, None, 0, err, 64) == -1
    # messages are truncated to the caller's capacity and NUL-terminated
    tiny = C.create_string_buffer(b"\xff" * 8)
    assert lib.rs_mlx_input(None, 0, None, None, 0, tiny, 8) == -1
    assert tiny.raw[:8] == b"invalid\x00"
    assert lib.rs_mlx_version().startswith(b"hip_bridge")
