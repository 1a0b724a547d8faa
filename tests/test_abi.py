"""C-ABI conformance on the CPU: the library loads, exports every entry point
that include/hip_bridge.h declares, and the structs keep the reference's
layouts (native/mlx_bridge.h:50-54, native/state_table.h:11-13)."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import numpy as np
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


def test_header_declares_session_surface():
    names = declared_functions()
    # native/mlx_bridge.h:55-57, 76-86, 94-96, 103-112, 120-133
    for n in ["rs_qwen_quant", "rs_qwen_forward"] + [
            "rs_qwen_device_" + s for s in
            ["create", "decode_batch", "step", "step_sampled", "block", "release", "snapshot", "stats", "drain",
             "destroy", "hidden_step", "hidden_block", "hidden_snapshot", "mtp_attach", "mtp_step", "mtp_release",
             "mtp_snapshot", "dspark_step", "dspark_snapshot"]] + [
            "rs_qwen_dspark_" + s for s in ["create", "destroy", "ingest", "propose", "release", "stats"]]:
        assert n in names, n


def test_session_entry_points_validate_before_device_work():
    """Descriptor, geometry, program and store checks fail with the reference's
    messages (native/qwen_model.inc:279-293, qwen_device.inc:14-29) before any
    device work, so they run without a GPU."""
    import hip_bridge
    from hip_bridge.engine import tiny_config
    from hip_bridge.session import Layer, WeightStore, layer_program

    lib = hip_bridge.load()
    err = C.create_string_buffer(1024)

    def create(store, cfg, prog=None, count=None, gpu=1, slots=4):
        prog = layer_program(cfg) if prog is None else prog
        count = cfg.layers if count is None else count
        h = lib.rs_qwen_device_create(store, gpu, C.byref(cfg), prog, count, slots, C.c_uint64(1 << 40), err, 1024)
        assert h is None
        return err.value.decode()

    target, sidecar, empty = WeightStore(5, 0), WeightStore(5, 1), WeightStore()
    cfg = tiny_config(layers=2, interval=2, chunk=8, context=64)
    assert create(target.handle, cfg, gpu=0).endswith("GPU only (gpu = 1)")
    assert create(None, cfg) == "device session descriptor"
    assert create(target.handle, cfg, slots=65) == "state table bounds"
    assert create(target.handle, cfg, count=1) == "IR layer count"
    bad = (Layer * 2)()
    bad[0].index, bad[0].mixer, bad[1].index, bad[1].mixer = 0, 1, 1, 1
    assert create(target.handle, cfg, prog=bad) == "IR layer program"
    assert create(empty.handle, cfg).startswith("weight store holds no model")
    assert create(sidecar.handle, cfg) == "not a target model store"
    for field, value, message in [("layer_group", 3, "model layer group"), ("chunk", 65, "model geometry/capacity"),
                                  ("layers", 3, "model geometry/capacity"), ("top", 9, "model geometry mismatch"),
                                  ("rope_dims", 63, "model geometry mismatch")]:
        c = tiny_config(layers=2, interval=2, chunk=8, context=64)
        setattr(c, field, value)
        assert create(target.handle, c) == message, field
    # activation profiles: this bridge computes profile 0 (BF16 activations, FP32
    # residual and accumulation) and refuses the FP32 profile 1 instead of
    # running it in BF16; the reference's own profile checks keep their order
    fp32 = ("activation precision 1 (FP32) is not built into this bridge: it computes BF16 activations with an "
            "FP32 residual stream and FP32 accumulation (activation precision 0)")
    c = tiny_config(layers=2, interval=2, chunk=8, context=64, activation_precision=1)
    assert create(target.handle, c) == fp32
    c.compiled_decode = 1
    assert create(target.handle, c) == fp32
    c.activation_precision = 0
    assert create(target.handle, c) == "compiled decode requires FP32"  # native/qwen_device.inc:19
    c.compiled_decode, c.fused_attention = 0, 2
    assert create(target.handle, c) == "Metal reference attention requires FP32/context512"
    c = tiny_config(layers=2, interval=2, chunk=8, context=64, activation_precision=2)
    assert create(target.handle, c) == "model geometry mismatch"
    e = C.create_string_buffer(256)
    assert lib.hb_engine_create(C.byref(tiny_config(activation_precision=1)), 2, 64, 8, 16, 1, 0, e, 256) is None
    assert e.value.decode() == fp32
    # per-module overrides: recorded, validated; a synthetic store (4-bit g64 by construction) refuses others
    assert lib.rs_qwen_quant(target.handle, b"x", 48, 4, err, 1024) == -1
    assert err.value == b"invalid model quantization"
    assert lib.rs_qwen_quant(target.handle, b"language_model.lm_head", 64, 8, err, 1024) == 0
    assert create(target.handle, cfg) == ("device session: a synthetic store is 4-bit group 64; quantization "
                                          "overrides apply to checkpoint stores")
    # the stateless forward refuses projection diagnostics and wrong state lengths
    tok = np.zeros(2, np.uint32)
    logits = np.zeros(cfg.vocab, np.float32)
    new = np.zeros(8, np.float32)
    rc = lib.rs_qwen_forward(target.handle, 1, C.byref(cfg), layer_program(cfg), cfg.layers,
                             tok.ctypes.data_as(C.c_void_p), 2, 0, None, 0, new.ctypes.data_as(C.c_void_p), 8,
                             logits.ctypes.data_as(C.c_void_p), cfg.vocab, 0, None, 0, None, 0, err, 1024)
    assert rc == -1 and err.value == b"model state length"
    c = tiny_config(layers=2, interval=2, chunk=8, context=64, activation_precision=1)
    rc = lib.rs_qwen_forward(target.handle, 1, C.byref(c), layer_program(c), c.layers, tok.ctypes.data_as(C.c_void_p),
                             2, 0, None, 0, new.ctypes.data_as(C.c_void_p), 8, logits.ctypes.data_as(C.c_void_p),
                             c.vocab, 0, None, 0, None, 0, err, 1024)
    assert rc == -1 and err.value.decode() == fp32
    # DSpark is not part of this bridge: every entry fails with a message
    assert lib.rs_qwen_dspark_create(None, b"p", 0, 1, 1, err, 1024) is None and b"DSpark" in err.value
    assert lib.rs_qwen_dspark_stats(None, None, 0, err, 1024) == -1
    # handles: null session / id descriptors
    assert lib.rs_qwen_device_release(None, None, err, 1024) == -1 and err.value == b"release descriptor"
    assert lib.rs_qwen_device_stats(None, None, 74, err, 1024) == -1


def test_fused_deltanet_step_refuses_other_geometries():
    """hb_gdn_decode covers conv width 4, 128-wide heads and two value heads
    per key head; any other geometry is refused with a message before any
    device work (the engine then runs hb_gdn_prep + hb_gdn_recurrence), so this
    runs without a GPU."""
    import hip_bridge

    lib = hip_bridge.load()
    err = C.create_string_buffer(256)
    fake = C.c_void_p(256)  # never dereferenced: the geometry check comes first

    def call(hk, hv, dk, dv, conv):
        rc = lib.hb_gdn_decode(fake, 8192, fake, fake, 64, fake, fake, fake, fake, fake, None, None, fake, 1, hk, hv,
                               dk, dv, conv, 4, fake, None, None, None, None, 0, 0, None, None, 0, None, None, None,
                               err, 256)
        return rc, err.value.decode()

    want = "hb_gdn_decode: the fused step needs conv width 4, 128-wide heads and two value heads per key head"
    for geom in [(16, 16, 128, 128, 4), (16, 32, 128, 128, 3), (16, 32, 64, 128, 4), (16, 32, 128, 64, 4),
                 (8, 32, 128, 128, 4)]:
        assert call(*geom) == (-1, want), geom
