"""ctypes front end of libhip_bridge.so (the C ABI in include/hip_bridge.h).

This is the host-side mirror a Python caller uses; the Rust host of the
reference binds the same symbols through `extern "C"` blocks
(src/serving/native_device.rs:1087-1207, src/serving/native_mlx.rs:574-636).
The library is required: there is no CPU fallback, and loading fails loudly
when it is missing.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libhip_bridge.so")
ERR_CAP = 1024

_lib = None


class HipBridgeError(RuntimeError):
    pass


def build(jobs: int = 8) -> str:
    """Compile libhip_bridge.so for gfx950 (recompiles every source each call)."""
    subprocess.run(["make", "-s", "-B", "-C", PKG_DIR, f"-j{jobs}"], check=True)
    return LIB_PATH


def _err():
    return C.create_string_buffer(ERR_CAP)


def _declare(L):
    vp, sz, i, u32, f = C.c_void_p, C.c_size_t, C.c_int, C.c_uint32, C.c_float
    cp = C.c_char_p
    sig = {
        # graph API (native/mlx_bridge.h)
        "rs_mlx_create": (vp, [i, cp, sz]),
        "rs_mlx_destroy": (None, [vp]),
        "rs_mlx_input": (i, [vp, i, vp, vp, sz, cp, sz]),
        "rs_mlx_op": (i, [vp, i, vp, sz, i, f, cp, sz]),
        "rs_mlx_finish": (i, [vp, u32, vp, sz, cp, sz]),
        "rs_mlx_version": (cp, []),
        "rs_mlx_cleanup": (None, []),
        "rs_mlx_weights_create": (vp, [cp, sz]),
        "rs_mlx_weights_destroy": (None, [vp]),
        "rs_mlx_weights_load": (i, [vp, cp, cp, sz]),
        "hb_safetensors_check": (i, [cp, C.POINTER(sz), cp, sz]),
        "rs_mlx_parameter": (i, [vp, vp, cp, vp, sz, i, cp, sz]),
        "rs_mlx_kernel": (i, [vp, i, vp, sz, vp, sz, vp, sz, cp, sz]),
        "rs_mlx_weight_bytes": (i, [vp, cp, vp, sz, i, sz, vp, sz, cp, sz]),
        # device-pointer API
        "hb_device_count": (i, []),
        "hb_device_name": (cp, [i]),
        "hb_malloc": (vp, [sz, cp, sz]),
        "hb_free": (i, [vp]),
        "hb_memcpy_h2d": (i, [vp, vp, sz, cp, sz]),
        "hb_memcpy_d2h": (i, [vp, vp, sz, cp, sz]),
        "hb_memcpy_d2d": (i, [vp, vp, sz, vp, cp, sz]),
        "hb_memset": (i, [vp, i, sz, vp, cp, sz]),
        "hb_stream_read_sink_bytes": (sz, [i]),
        "hb_stream_read": (i, [vp, sz, vp, i, i, vp, cp, sz]),
        "hb_stream_copy": (i, [vp, vp, sz, i, vp, cp, sz]),
        "hb_stream_read_chunked": (i, [vp, sz, sz, vp, i, vp, cp, sz]),
        "hb_stream_copy_chunked": (i, [vp, vp, sz, sz, vp, cp, sz]),
        "hb_synchronize": (i, [vp, cp, sz]),
        "hb_stream_create": (vp, [cp, sz]),
        "hb_stream_destroy": (None, [vp]),
        "hb_event_create": (vp, [cp, sz]),
        "hb_event_destroy": (None, [vp]),
        "hb_event_record": (i, [vp, vp, cp, sz]),
        "hb_event_elapsed": (i, [vp, vp, C.POINTER(f), cp, sz]),
        "hb_graph_begin": (i, [vp, cp, sz]),
        "hb_graph_end": (vp, [vp, cp, sz]),
        "hb_graph_launch": (i, [vp, vp, cp, sz]),
        "hb_graph_destroy": (None, [vp]),
        "hb_q4_tile": (i, [vp, vp, vp, vp, vp, i, i, vp, cp, sz]),
        "hb_qmm": (i, [vp, vp, vp, vp, vp, i, i, i, i, i, i, i, i, vp, cp, sz]),
        "hb_pack_tables": (i, [vp, vp, vp, i, i, i, vp, vp, vp, vp, vp, vp, vp, cp, sz]),
        "hb_attn_prep": (i, [vp, i, vp, i, i, vp, vp, vp, vp, i, i, i, i, i, f, f, vp, vp, vp, vp, cp, sz]),
        "hb_attn_workspace_floats": (sz, [i, i, i, i, i, i, i]),
        "hb_paged_attention": (i, [vp, vp, vp, vp, i, vp, vp, vp, vp, i, i, i, i, i, i, i, i, f, i, vp, vp, vp,
                                   vp, cp, sz]),
        "hb_gdn_prep": (i, [vp, i, vp, vp, i, vp, vp, vp, vp, vp, vp, vp, vp, i, i, i, i, i, i, i, vp, vp, vp, vp,
                            vp, vp, cp, sz]),
        "hb_gdn_recurrence": (i, [vp, vp, vp, vp, vp, vp, i, i, i, i, i, vp, vp, vp, vp, vp, vp, vp, i, i, vp, vp,
                                  i, vp, vp, vp, cp, sz]),
        "hb_gdn_decode": (i, [vp, i, vp, vp, i, vp, vp, vp, vp, vp, vp, vp, vp, i, i, i, i, i, i, i, vp, vp, vp, vp,
                              vp, i, i, vp, vp, i, vp, vp, vp, cp, sz]),
        "hb_gdn_chunked": (i, [vp, vp, vp, vp, vp, vp, i, i, i, i, i, vp, vp, vp, vp, vp, i, vp, vp, vp, cp, sz]),
        "hb_random_q4": (i, [C.c_uint64, i, i, f, vp, vp, vp, vp, cp, sz]),
        "hb_random_normal": (i, [C.c_uint64, sz, f, f, i, vp, vp, cp, sz]),
        "hb_random_uniform": (i, [C.c_uint64, sz, f, f, i, vp, vp, cp, sz]),
        "hb_random_ints": (i, [C.c_uint64, sz, u32, vp, vp, cp, sz]),
        "hb_moe_route": (i, [vp, i, i, i, i, vp, vp, vp, vp, vp, vp, vp, vp, cp, sz]),
        "hb_moe_items_capacity": (sz, [i, i, i]),
        "hb_moe_grouped_qmm": (i, [vp, i, vp, vp, i, vp, vp, vp, vp, i, i, i, i, vp, vp, cp, sz]),
        "hb_moe_combine": (i, [vp, vp, vp, vp, i, i, i, i, i, vp, vp, cp, sz]),
        "hb_argmax_margin": (i, [vp, i, i, i, vp, vp, vp, vp, vp, cp, sz]),
        "hb_qmm_select": (i, [vp, i, i, vp, vp, i, i, vp, sz, vp, vp, vp, C.POINTER(i), vp, cp, sz]),
        "hb_qmm_select_workspace_bytes": (sz, [i, i]),
        "hb_argmax_workspace_bytes": (sz, [i, i]),
        "hb_argmax_margin_noalloc": (i, [vp, i, i, i, vp, vp, vp, vp, cp, sz]),
        "hb_argmax_noalloc_limit_bytes": (sz, []),
        "hb_mtp_plan": (i, [vp, vp, i, vp, vp, i, vp, i, i, vp, vp, vp, vp, vp, vp, cp, sz]),
        "hb_embed_gather": (i, [vp, i, vp, vp, vp, i, vp, vp, cp, sz]),
        "hb_rmsnorm": (i, [vp, i, vp, i, i, f, vp, i, vp, vp, cp, sz]),
        "hb_rmsnorm_gs": (i, [vp, i, vp, i, i, f, vp, i, vp, vp, cp, sz]),
        "hb_qmm_gs": (i, [vp, vp, vp, vp, i, i, i, i, i, vp, vp, cp, sz]),
        "hb_engine_create": (vp, [vp, i, i, i, i, C.c_uint64, i, cp, sz]),
        "hb_engine_create_named": (vp, [vp, i, i, i, i, vp, vp, cp, sz]),
        "hb_engine_destroy": (None, [vp]),
        "hb_engine_info": (i, [vp, vp, sz, cp, sz]),
        "hb_session_info": (i, [vp, vp, sz, cp, sz]),
        "hb_engine_tensor_shape": (i, [vp, i, vp, vp, vp, cp, sz]),
        "hb_engine_export": (i, [vp, i, vp, vp, vp, cp, sz]),
        "hb_engine_forward": (i, [vp, i, vp, vp, vp, vp, vp, vp, vp, vp, i, vp, i, cp, sz]),
        "hb_engine_mtp_forward": (i, [vp, i, vp, vp, vp, vp, i, vp, vp, i, cp, sz]),
        "hb_engine_read": (i, [vp, i, sz, vp, sz, cp, sz]),
        "hb_engine_synthetic_context": (i, [vp, i, vp, C.c_uint64, cp, sz]),
        "hb_engine_trace": (i, [vp, i, cp, sz]),
        "hb_engine_profile": (i, [vp, i, cp, sz]),
        "hb_engine_profile_read": (i, [vp, i, vp, sz, cp, sz]),
        "hb_decode_create": (vp, [vp, i, f, vp, i, cp, sz]),
        "hb_decode_destroy": (None, [vp]),
        "hb_decode_admit": (i, [vp, i, i, u32, i, i, cp, sz]),
        "hb_decode_set_drafts": (i, [vp, i, vp, i, cp, sz]),
        "hb_decode_step": (i, [vp, vp, cp, sz]),
        "hb_decode_stats": (i, [vp, vp, sz, cp, sz]),
        "hb_decode_output": (i, [vp, i, vp, sz, vp, vp, cp, sz]),
        # model entry points and device sessions (native/mlx_bridge.h:55-133)
        "hb_weights_synthetic": (i, [vp, C.c_uint64, i, cp, sz]),
        "rs_qwen_quant": (i, [vp, cp, i, i, cp, sz]),
        "rs_qwen_forward": (i, [vp, i, vp, vp, sz, vp, sz, sz, vp, sz, vp, sz, vp, sz, i, vp, sz, vp, sz, cp, sz]),
        "rs_qwen_device_create": (vp, [vp, i, vp, vp, sz, sz, C.c_uint64, cp, sz]),
        "rs_qwen_device_destroy": (None, [vp]),
        "rs_qwen_device_decode_batch": (i, [vp, vp, vp, sz, vp, vp, sz, cp, sz]),
        "rs_qwen_device_step": (i, [vp, vp, sz, vp, sz, vp, vp, sz, vp, sz, cp, sz]),
        "rs_qwen_device_step_sampled": (i, [vp, vp, sz, vp, sz, vp, vp, cp, sz]),
        "rs_qwen_device_block": (i, [vp, vp, sz, vp, sz, vp, vp, sz, cp, sz]),
        "rs_qwen_device_hidden_step": (i, [vp, vp, sz, vp, sz, vp, vp, sz, cp, sz]),
        "rs_qwen_device_hidden_block": (i, [vp, vp, sz, vp, sz, vp, vp, sz, cp, sz]),
        "rs_qwen_device_ragged_step": (i, [vp, vp, vp, sz, vp, sz, i, vp, vp, vp, vp, sz, cp, sz]),
        "rs_qwen_device_release": (i, [vp, vp, cp, sz]),
        "rs_qwen_device_snapshot": (i, [vp, vp, vp, sz, cp, sz]),
        "rs_qwen_device_hidden_snapshot": (i, [vp, vp, vp, sz, cp, sz]),
        "rs_qwen_device_stats": (i, [vp, vp, sz, cp, sz]),
        "rs_qwen_device_drain": (i, [vp, vp, cp, sz]),
        "rs_qwen_device_mtp_attach": (i, [vp, vp, cp, sz]),
        "rs_qwen_device_mtp_step": (i, [vp, vp, vp, i, sz, vp, sz, vp, vp, sz, i, cp, sz]),
        "rs_qwen_device_mtp_release": (i, [vp, vp, cp, sz]),
        "rs_qwen_device_mtp_snapshot": (i, [vp, vp, vp, sz, cp, sz]),
        "rs_qwen_dspark_create": (vp, [vp, cp, i, sz, C.c_uint64, cp, sz]),
        "rs_qwen_dspark_stats": (i, [vp, vp, sz, cp, sz]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def load():
    """Load libhip_bridge.so (fails loudly when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipBridgeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        _lib = _declare(C.CDLL(LIB_PATH))
    return _lib


def _arg(a):
    if isinstance(a, DeviceBuffer):
        return C.c_void_p(a.ptr)
    if isinstance(a, Stream):
        return a.handle
    return a


def call(fn_name, *args):
    """Call an int-returning entry point with a trailing (error, capacity) pair.
    DeviceBuffer and Stream arguments are passed as their device pointer / handle."""
    err = _err()
    rc = getattr(load(), fn_name)(*[_arg(a) for a in args], err, ERR_CAP)
    if rc != 0:
        raise HipBridgeError(f"{fn_name}: {err.value.decode(errors='replace')}")
    return rc


# ------------------------------------------------------------------ device memory
class DeviceBuffer:
    """Owning handle of a device allocation (bytes)."""

    def __init__(self, nbytes: int):
        err = _err()
        self.nbytes = int(nbytes)
        self.ptr = load().hb_malloc(max(self.nbytes, 4), err, ERR_CAP)
        if not self.ptr:
            raise HipBridgeError(f"hb_malloc({nbytes}): {err.value.decode(errors='replace')}")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        call("hb_memcpy_h2d", C.c_void_p(self.ptr + offset), a.ctypes.data_as(C.c_void_p), a.nbytes)

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        call("hb_memcpy_d2h", out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset), out.nbytes)
        return out

    def zero(self, stream=None):
        call("hb_memset", C.c_void_p(self.ptr), 0, self.nbytes, stream)

    def free(self):
        if getattr(self, "ptr", None):
            load().hb_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize(stream=None):
    call("hb_synchronize", stream)


class Stream:
    def __init__(self):
        err = _err()
        self.handle = load().hb_stream_create(err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(err.value.decode(errors="replace"))

    def __del__(self):
        if getattr(self, "handle", None):
            load().hb_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        err = _err()
        self.handle = load().hb_event_create(err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(err.value.decode(errors="replace"))

    def record(self, stream=None):
        call("hb_event_record", self.handle, stream.handle if isinstance(stream, Stream) else stream)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("hb_event_elapsed", self.handle, end.handle, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        if getattr(self, "handle", None):
            load().hb_event_destroy(self.handle)
            self.handle = None


class CapturedGraph:
    """Work issued on `stream` between begin() and end() becomes one replayable graph."""

    def __init__(self, stream: "Stream"):
        self.stream = stream
        self.handle = None
        call("hb_graph_begin", stream.handle)

    def end(self):
        err = _err()
        self.handle = load().hb_graph_end(self.stream.handle, err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(f"hb_graph_end: {err.value.decode(errors='replace')}")
        return self

    def launch(self):
        call("hb_graph_launch", self.handle, self.stream.handle)

    def __del__(self):
        if getattr(self, "handle", None):
            load().hb_graph_destroy(self.handle)
            self.handle = None


# ------------------------------------------------------------------ operators
LAYOUT_MLX = 0
LAYOUT_Q4T = 1


def _s(stream):
    return stream.handle if isinstance(stream, Stream) else stream


def q4_tile(w, scales, biases, w_tiled, sb_tiled, N, K, stream=None):
    """Checkpoint-format 4-bit g64 weights -> the tiled MFMA layout (device buffers)."""
    call("hb_q4_tile", _p(w), _p(scales), _p(biases), _p(w_tiled), _p(sb_tiled), N, K, _s(stream))


class TiledWeight:
    """A 4-bit group-64 matrix resident in HBM in the tiled layout."""

    def __init__(self, packed, scales_bits, biases_bits, stream=None):
        self.N, words = packed.shape
        self.K = words * 8
        raw = DeviceBuffer.from_array(packed)
        s = DeviceBuffer.from_array(scales_bits)
        b = DeviceBuffer.from_array(biases_bits)
        self.w = DeviceBuffer(packed.nbytes)
        self.sb = DeviceBuffer(scales_bits.nbytes * 2)
        q4_tile(raw, s, b, self.w, self.sb, self.N, self.K, stream)
        synchronize(_s(stream))

    @property
    def nbytes(self):
        return self.w.nbytes + self.sb.nbytes


def qmm(x, w, scales, biases, y, M, N, K, group=64, bits=4, layout=LAYOUT_Q4T, y_f32=False, ldy=None,
        stream=None, out_mode=None):
    """y = x . W^T on device buffers (x bf16 [M][K], y bf16/f32 [M][ldy]); out_mode 0 bf16,
    1 f32, 2 f32 accumulate (default from y_f32)."""
    mode = int(y_f32) if out_mode is None else out_mode
    call("hb_qmm", _p(x), _p(w), _p(scales), _p(biases), _p(y), M, N, K, group, bits, layout, mode, ldy or N,
         _s(stream))


def qmm_tiled(x, tw: TiledWeight, y, M, y_f32=False, ldy=None, stream=None):
    qmm(x, tw.w, tw.sb, None, y, M, tw.N, tw.K, 64, 4, LAYOUT_Q4T, y_f32, ldy, stream)


def _p(b):
    if b is None:
        return None
    if isinstance(b, DeviceBuffer):
        return C.c_void_p(b.ptr)
    return C.c_void_p(int(b))


# ------------------------------------------------------------------ graph API
class GraphHandle:
    """Thin wrapper over rs_mlx_create/input/op/kernel/finish."""

    def __init__(self, gpu: int = 1):
        err = _err()
        self.handle = load().rs_mlx_create(gpu, err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(err.value.decode(errors="replace"))
        self.count = 0
        self.shapes = []

    def input(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        dtype = {np.dtype(np.float32): 0, np.dtype(np.int32): 1, np.dtype(np.uint32): 2}[a.dtype]
        shape = np.array(a.shape, dtype=np.int32)
        call("rs_mlx_input", self.handle, dtype, a.ctypes.data_as(C.c_void_p), shape.ctypes.data_as(C.c_void_p),
             len(a.shape))
        self.count += 1
        return self.count - 1

    def op(self, code: int, inputs, group: int = 0, epsilon: float = 0.0) -> int:
        ids = np.array(inputs, dtype=np.uint32)
        call("rs_mlx_op", self.handle, code, ids.ctypes.data_as(C.c_void_p), len(ids), group, epsilon)
        self.count += 1
        return self.count - 1

    def kernel(self, code: int, inputs, ints=(), floats=(), outputs: int = 1):
        ids = np.array(inputs, dtype=np.uint32)
        iv = np.array(ints, dtype=np.int32)
        fv = np.array(floats, dtype=np.float32)
        call("rs_mlx_kernel", self.handle, code, ids.ctypes.data_as(C.c_void_p), len(ids),
             iv.ctypes.data_as(C.c_void_p) if len(iv) else None, len(iv),
             fv.ctypes.data_as(C.c_void_p) if len(fv) else None, len(fv))
        first = self.count
        self.count += outputs
        return list(range(first, first + outputs)) if outputs > 1 else first

    def finish(self, node: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        call("rs_mlx_finish", self.handle, node, out.ctypes.data_as(C.c_void_p), out.size)
        return out

    def __del__(self):
        if getattr(self, "handle", None):
            load().rs_mlx_destroy(self.handle)
            self.handle = None


# ------------------------------------------------------------------ step operators
def pack_tables(row_tokens, positions, block_table, max_pages, rows, page, cu_seqlens, token_row, token_pos,
                kv_slot, context, status, stream=None):
    call("hb_pack_tables", _p(row_tokens), _p(positions), _p(block_table), max_pages, rows, page, _p(cu_seqlens),
         _p(token_row), _p(token_pos), _p(kv_slot), _p(context), _p(status), _s(stream))


def attn_prep(qg, ld_qg, kv, ld_kv, kv_off, q_norm, k_norm, token_pos, kv_slot, tokens, q_heads, kv_heads,
              head_dim, rotary, theta, eps, qout, kcache, vcache, stream=None):
    call("hb_attn_prep", _p(qg), ld_qg, _p(kv), ld_kv, kv_off, _p(q_norm), _p(k_norm), _p(token_pos), _p(kv_slot),
         tokens, q_heads, kv_heads, head_dim, rotary, theta, eps, _p(qout), _p(kcache), _p(vcache), _s(stream))


def attn_workspace_floats(rows, kv_heads, head_dim, max_tokens, group, max_context, split_len):
    return int(load().hb_attn_workspace_floats(rows, kv_heads, head_dim, max_tokens, group, max_context, split_len))


def paged_attention(q, kcache, vcache, block_table, max_pages, cu_seqlens, context, token_row, qg, ld_qg, rows,
                    tokens, max_tokens, max_context, q_heads, kv_heads, head_dim, scale, split_len, work_o, work_ml,
                    out, stream=None):
    call("hb_paged_attention", _p(q), _p(kcache), _p(vcache), _p(block_table), max_pages, _p(cu_seqlens),
         _p(context), _p(token_row), _p(qg), ld_qg, rows, tokens, max_tokens, max_context, q_heads, kv_heads,
         head_dim, scale, split_len, _p(work_o), _p(work_ml), _p(out), _s(stream))
