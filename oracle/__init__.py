"""ctypes front end of the CPU oracle (oracle.c) and of the reference-oracle shim.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, always as the checker. The product
library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB names another build of oracle.c (the sanitizer tests load an
# ASan/UBSan build through it)
LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build(reference: bool = True) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "oracle"], check=True)
    if reference:
        subprocess.run(["make", "-s", "-B", "-C", HERE, "ref"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(reference=False)
        L = C.CDLL(LIB_PATH)
        sz, i, d = C.c_size_t, C.c_int, C.c_double
        L.orc_code.restype = C.c_uint
        L.orc_code.argtypes = [_u32p, sz, i]
        L.orc_qmm.argtypes = [_f32p, sz, _u32p, _f32p, _f32p, sz, sz, i, i, _f64p, i]
        L.orc_dequant.argtypes = [_u32p, _f32p, _f32p, sz, sz, i, i, _f64p]
        L.orc_rms.argtypes = [_f32p, C.c_void_p, sz, sz, d, _f64p]
        L.orc_silu.argtypes = [_f32p, sz, _f64p]
        L.orc_sigmoid.restype = d
        L.orc_sigmoid.argtypes = [d]
        L.orc_rope.argtypes = [_f32p, i, i, i, i, _i32p, d, _f64p]
        L.orc_paged_attention.argtypes = [_f32p, _f32p, _f32p, _i32p, i, _i32p, _i32p, i, i, i, i, i, d,
                                          C.c_void_p, _f64p]
        L.orc_gated_delta.argtypes = [_f32p] * 6 + [i] * 6 + [_f64p, _f64p]
        L.orc_gdn.argtypes = [_f32p] * 8 + [i] * 6 + [C.c_void_p, C.c_void_p, _f64p, _f64p]
        L.orc_route_topk.argtypes = [_f32p, i, i, i, _i32p, _f64p]
        L.orc_expert_permute.argtypes = [_i32p, i, i, i, _i32p, _i32p, _i32p]
        L.orc_gather_qmm.argtypes = [_f32p, i, _u32p, _f32p, _f32p, i, i, i, i, i, _i32p, i, _f64p, i]
        L.orc_qmm4_f32.argtypes = [_f32p, sz, _u32p, _f32p, _f32p, sz, sz, _f32p, i]
        L.orc_gather_qmm4_f32.argtypes = [_f32p, i, _u32p, _f32p, _f32p, i, i, i, _i32p, i, _f32p, i]
        L.orc_mix.argtypes = [_f32p, _f32p, i, i, i, _f64p]
        L.orc_winner.argtypes = [_f32p, sz, C.POINTER(C.c_uint32), C.POINTER(C.c_float)]
        L.orc_plan.argtypes = [_f32p, sz, C.c_void_p, sz, C.c_void_p, C.c_void_p, sz, sz, _u32p,
                               C.POINTER(sz), C.POINTER(sz), C.POINTER(C.c_int)]
        L.orc_pack_tables.argtypes = [_i32p, _i32p, _i32p, i, i, i, _i32p, _i32p, _i32p, _i32p, _i32p]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_max_threads.restype = i
        _lib = L
    return _lib


def ref():
    """The reference's own scalar oracles (built in this container), or None."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = C.CDLL(REF_PATH)
        sz, i, d = C.c_size_t, C.c_int, C.c_double
        R.ref_projection.argtypes = [_f32p, sz, _u32p, _f32p, _f32p, sz, sz, i, i, _f64p]
        R.ref_embedding.argtypes = [_u32p, _f32p, _f32p, sz, sz, i, i, _f64p]
        R.ref_rms.argtypes = [_f32p, sz, C.c_void_p, sz, d, _f64p]
        R.ref_silu.argtypes = [_f32p, sz, _f64p]
        R.ref_rope.argtypes = [_f32p, i, i, i, i, i, d, _f64p]
        R.ref_delta.argtypes = [_f32p] * 8 + [i] * 6 + [_f64p] * 4
        R.ref_routing.argtypes = [_f32p, _i32p, i, i, i, _f64p]
        R.ref_attention.argtypes = [_f32p, _f32p, _f32p, i, i, i, i, i, _f64p]
        R.ref_table_create.restype = C.c_void_p
        R.ref_table_create.argtypes = [C.c_uint64, sz, C.c_uint64]
        R.ref_table_destroy.argtypes = [C.c_void_p]
        for name in ("reserve",):
            getattr(R, f"ref_table_{name}").argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p]
        R.ref_table_publish.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        R.ref_table_get.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(C.c_int)]
        R.ref_table_rollback.argtypes = [C.c_void_p, C.c_void_p]
        R.ref_table_release.argtypes = [C.c_void_p, C.c_void_p]
        R.ref_table_bytes.restype = C.c_uint64
        R.ref_table_bytes.argtypes = [C.c_void_p]
        R.ref_table_residents.restype = sz
        R.ref_table_residents.argtypes = [C.c_void_p]
        R.ref_table_clear.argtypes = [C.c_void_p]
        _ref = R
    return _ref


class OracleError(ValueError):
    pass


def _check(rc):
    if rc != 0:
        raise OracleError("oracle rejected descriptor")


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- bf16 helpers
def bf16_round(a) -> np.ndarray:
    """Round float32 values to bf16 (nearest-even) and widen back to float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.view(np.float32)


def to_bf16_bits(a) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bf16_bits(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- quantisation
def quantize_affine(w, group=64, bits=4):
    """Min/max affine quantiser producing LSB-first packed codes and bf16-exact
    scales/biases. The reference never quantises (its checkpoints are
    pre-quantised), so this is only a generator of valid inputs.
    Returns (packed u32 [N, K*bits/32], scales f32 [N,K/g], biases f32 [N,K/g])."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    g = w.reshape(n, k // group, group)
    lo, hi = g.min(-1), g.max(-1)
    levels = (1 << bits) - 1
    scale = bf16_round(np.maximum((hi - lo) / levels, 1e-8))
    bias = bf16_round(lo)
    q = np.clip(np.rint((g - bias[..., None]) / scale[..., None]), 0, levels).astype(np.uint64)
    q = q.reshape(n, k)
    return pack_codes(q, bits), scale.astype(np.float32), bias.astype(np.float32)


def pack_codes(q, bits):
    """LSB-first bit stream per row (native/projection_reference.h:16)."""
    q = np.asarray(q, dtype=np.uint64)
    n, k = q.shape
    words = k * bits // 32
    out = np.zeros((n, words), dtype=np.uint64)
    for c in range(k):
        bit = c * bits
        word, shift = bit // 32, bit % 32
        out[:, word] |= (q[:, c] << np.uint64(shift)) & np.uint64(0xFFFFFFFF)
        if shift + bits > 32:
            out[:, word + 1] |= q[:, c] >> np.uint64(32 - shift)
    return out.astype(np.uint32)


# ---------------------------------------------------------------- operators
def qmm(x, packed, scales, biases, group=64, bits=4, threads=0):
    x = f32(x)
    rows, width = x.shape
    outputs = packed.shape[0]
    y = np.zeros((rows, outputs), dtype=np.float64)
    _check(lib().orc_qmm(x, rows, np.ascontiguousarray(packed, np.uint32), f32(scales), f32(biases),
                         outputs, width, group, bits, y, threads))
    return y


def qmm4_f32(x, packed, scales, biases, threads=0):
    """FP32 form of qmm for 4-bit g64 (the CPU baseline's timing path)."""
    x = f32(x)
    rows, width = x.shape
    outputs = packed.shape[0]
    y = np.zeros((rows, outputs), dtype=np.float32)
    _check(lib().orc_qmm4_f32(x, rows, np.ascontiguousarray(packed, np.uint32), f32(scales), f32(biases), outputs,
                              width, y, threads))
    return y


def dequant(packed, scales, biases, width, group=64, bits=4):
    rows = packed.shape[0]
    y = np.zeros((rows, width), dtype=np.float64)
    _check(lib().orc_dequant(np.ascontiguousarray(packed, np.uint32), f32(scales), f32(biases), rows, width,
                             group, bits, y))
    return y


def rms(x, weight=None, eps=1e-6):
    x = f32(x)
    width = x.shape[-1]
    y = np.zeros(x.shape, dtype=np.float64)
    w = f32(weight) if weight is not None else None
    _check(lib().orc_rms(x, w.ctypes.data if w is not None else None, x.size // width, width, eps, y))
    return y


def silu(x):
    x = f32(x)
    y = np.zeros(x.shape, dtype=np.float64)
    _check(lib().orc_silu(x, x.size, y))
    return y


def rope(x, positions, rotary=64, theta=1e7):
    """x [tokens, heads, dim]; positions [tokens]."""
    x = f32(x)
    t, h, d = x.shape
    y = np.zeros(x.shape, dtype=np.float64)
    _check(lib().orc_rope(x, t, h, d, rotary, np.ascontiguousarray(positions, np.int32), theta, y))
    return y


def paged_attention(q, kcache, vcache, block_table, cu_seqlens, context, scale, gate=None):
    q = f32(q)
    total, hq, dim = q.shape
    pages, hkv, page, _ = kcache.shape
    out = np.zeros(q.shape, dtype=np.float64)
    g = f32(gate) if gate is not None else None
    bt = np.ascontiguousarray(block_table, np.int32)
    _check(lib().orc_paged_attention(q, f32(kcache), f32(vcache), bt, bt.shape[1],
                                     np.ascontiguousarray(cu_seqlens, np.int32),
                                     np.ascontiguousarray(context, np.int32), len(context), hq, hkv, dim, page,
                                     scale, g.ctypes.data if g is not None else None, out))
    return out


def gated_delta(q, k, v, decay, beta, state):
    b, t, hk, dk = q.shape
    hv, dv = v.shape[2], v.shape[3]
    out = np.zeros((b, t, hv, dv), dtype=np.float64)
    st = np.zeros((b, hv, dv, dk), dtype=np.float64)
    _check(lib().orc_gated_delta(f32(q), f32(k), f32(v), f32(decay), f32(beta), f32(state), b, t, hk, hv, dk,
                                 dv, out, st))
    return out, st


def gdn(qkv, history, conv_w, a, b, alog, dt, state, hk, hv, dk, dv):
    t = qkv.shape[0]
    kernel = conv_w.shape[1]
    channels = qkv.shape[1]
    act = np.zeros((t, channels), dtype=np.float64)
    hist = np.zeros((kernel - 1, channels), dtype=np.float64)
    out = np.zeros((t, hv, dv), dtype=np.float64)
    st = np.zeros((hv, dv, dk), dtype=np.float64)
    _check(lib().orc_gdn(f32(qkv), f32(history), f32(conv_w), f32(a), f32(b), f32(alog), f32(dt), f32(state), t,
                         hk, hv, dk, dv, kernel, act.ctypes.data, hist.ctypes.data, out, st))
    return act, hist, out, st


def route_topk(logits, top):
    logits = f32(logits)
    rows, experts = logits.shape
    idx = np.zeros((rows, top), dtype=np.int32)
    w = np.zeros((rows, top), dtype=np.float64)
    _check(lib().orc_route_topk(logits, rows, experts, top, idx, w))
    return idx, w


def expert_permute(idx, experts):
    idx = np.ascontiguousarray(idx, np.int32)
    tokens, top = idx.shape
    order = np.zeros(tokens * top, dtype=np.int32)
    inverse = np.zeros(tokens * top, dtype=np.int32)
    offsets = np.zeros(experts + 1, dtype=np.int32)
    _check(lib().orc_expert_permute(idx, tokens, top, experts, order, inverse, offsets))
    return order, inverse, offsets


def gather_qmm(x, packed, scales, biases, idx, group=64, bits=4, threads=0):
    x = f32(x)
    rows, width = x.shape
    experts, outputs = packed.shape[0], packed.shape[1]
    idx = np.ascontiguousarray(idx, np.int32)
    top = idx.shape[1]
    y = np.zeros((rows, top, outputs), dtype=np.float64)
    _check(lib().orc_gather_qmm(x, rows, np.ascontiguousarray(packed, np.uint32), f32(scales), f32(biases),
                                experts, outputs, width, group, bits, idx, top, y, threads))
    return y


def gather_qmm4_f32(x, packed, scales, biases, idx, threads=0):
    """FP32 form of gather_qmm for 4-bit g64 (the CPU baseline's timing path)."""
    x = f32(x)
    rows, width = x.shape
    experts, outputs = packed.shape[0], packed.shape[1]
    idx = np.ascontiguousarray(idx, np.int32)
    top = idx.shape[1]
    y = np.zeros((rows, top, outputs), dtype=np.float32)
    _check(lib().orc_gather_qmm4_f32(x, rows, np.ascontiguousarray(packed, np.uint32), f32(scales), f32(biases),
                                     experts, outputs, width, idx, top, y, threads))
    return y


def mix(experts, scores):
    e = f32(experts)
    rows, top, width = e.shape
    y = np.zeros((rows, width), dtype=np.float64)
    _check(lib().orc_mix(e, f32(scores), rows, top, width, y))
    return y


def winner(logits):
    logits = f32(logits)
    tok = C.c_uint32()
    margin = C.c_float()
    _check(lib().orc_winner(logits, logits.size, C.byref(tok), C.byref(margin)))
    return int(tok.value), float(margin.value)


def plan(initial, draft, rows, eos, remaining):
    initial = f32(initial)
    vocab = initial.size
    draft = np.ascontiguousarray(draft, np.uint32)
    rows = f32(rows).reshape(-1) if len(draft) else np.zeros(1, np.float32)
    eos = np.ascontiguousarray(eos, np.uint32)
    emitted = np.zeros(len(draft) + 1, dtype=np.uint32)
    n, acc, term = C.c_size_t(), C.c_size_t(), C.c_int()
    if len(draft) and rows.size != len(draft) * vocab:
        raise OracleError("verifier row vocabulary")
    _check(lib().orc_plan(initial, vocab, draft.ctypes.data if len(draft) else None, len(draft),
                          rows.ctypes.data if len(draft) else None, eos.ctypes.data if len(eos) else None,
                          len(eos), remaining, emitted, C.byref(n), C.byref(acc), C.byref(term)))
    return [int(t) for t in emitted[: n.value]], int(acc.value), bool(term.value)


def pack_tables(row_tokens, positions, block_table, page=16):
    row_tokens = np.ascontiguousarray(row_tokens, np.int32)
    positions = np.ascontiguousarray(positions, np.int32)
    bt = np.ascontiguousarray(block_table, np.int32)
    rows = len(row_tokens)
    total = int(row_tokens.sum())
    cu = np.zeros(rows + 1, np.int32)
    token_row = np.zeros(max(total, 1), np.int32)
    token_pos = np.zeros(max(total, 1), np.int32)
    kv_slot = np.zeros(max(total, 1), np.int32)
    context = np.zeros(max(rows, 1), np.int32)
    _check(lib().orc_pack_tables(row_tokens, positions, bt, bt.shape[1], rows, page, cu, token_row, token_pos,
                                 kv_slot, context))
    return dict(cu_seqlens=cu, token_row=token_row[:total], token_pos=token_pos[:total], kv_slot=kv_slot[:total],
                context=context[:rows])
