"""Host-side affine quantiser and seeded synthetic workloads.

The reference never quantises at run time (its checkpoints arrive already
quantised, src/serving/weights.rs:146-395), so this module only produces valid
inputs in the checkpoint format: LSB-first packed codes per row with bf16
scales and biases per group (native/projection_reference.h:16).
"""
from __future__ import annotations

import numpy as np

SEED = 20261201


def bf16_bits(a) -> np.ndarray:
    """float32 -> bf16 bit patterns (round to nearest even)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(bits) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(a) -> np.ndarray:
    return bf16_value(bf16_bits(a))


def quantize_affine(w, group: int = 64, bits: int = 4):
    """Min/max affine quantisation of w [N, K].

    Returns (packed uint32 [N, K*bits/32], scales bf16-bits [N, K/g], biases bf16-bits [N, K/g]),
    where the dequantised weight is scale * code + bias with code in [0, 2^bits)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % group == 0 and (k * bits) % 32 == 0
    g = w.reshape(n, k // group, group)
    lo, hi = g.min(-1), g.max(-1)
    levels = (1 << bits) - 1
    scale = bf16_round(np.maximum((hi - lo) / levels, 1e-8))
    bias = bf16_round(lo)
    q = np.clip(np.rint((g - bias[..., None]) / scale[..., None]), 0, levels).astype(np.uint32).reshape(n, k)
    return pack(q, bits), bf16_bits(scale), bf16_bits(bias)


def pack(q, bits: int) -> np.ndarray:
    """LSB-first bit stream per row."""
    q = np.asarray(q, dtype=np.uint64)
    n, k = q.shape
    if 32 % bits == 0:
        per = 32 // bits
        q = q.reshape(n, k // per, per)
        shifts = (np.arange(per, dtype=np.uint64) * np.uint64(bits))
        return (q << shifts).sum(-1).astype(np.uint32)
    words = k * bits // 32
    out = np.zeros((n, words), dtype=np.uint64)
    for c in range(k):
        bit = c * bits
        word, shift = bit // 32, bit % 32
        out[:, word] |= (q[:, c] << np.uint64(shift)) & np.uint64(0xFFFFFFFF)
        if shift + bits > 32:
            out[:, word + 1] |= q[:, c] >> np.uint64(32 - shift)
    return out.astype(np.uint32)


def qgemv_workload(m=8, n=6144, k=2048, group=64, bits=4, seed=SEED):
    """x bf16 [m,k] ~ N(0,1); W [n,k] ~ N(0,0.02) quantised to bits/group."""
    rng = np.random.default_rng(seed)
    x = bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    packed, scales, biases = quantize_affine(w, group, bits)
    return x, packed, scales, biases
