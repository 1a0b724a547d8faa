// Device helpers shared by the 4-bit MFMA kernels (dense and grouped).
#pragma once
#include "hb_common.h"

namespace hb {

// Workgroup barrier that orders LDS only: global loads in flight (the next
// operands) stay in flight across it, where __syncthreads() first waits for
// every outstanding memory operation of the wave.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// bf16 (128 + code) for the 8 codes of one interleaved word, in k order: the
// interleaved word keeps codes 2j and 2j+1 in the two 16-bit halves of (w >> 4j),
// and 0x4300 | q is the bf16 bit pattern of 128 + q for q < 128.
__device__ inline bf16x8 q4_offset_bf16(uint32_t w) {
  u32x4 d;
  d[0] = (w & 0x000F000Fu) | 0x43004300u;
  d[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  d[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  d[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8, d);
}

// Same as one v_and_or_b32 per dword (after its shift): 7 VALU ops per word
// instead of 11. gfx9 VOP3 takes no literal and one scalar operand, so the
// nibble mask rides in a VGPR and the bf16 offset pattern in an SGPR; with the
// constants hidden in registers the compiler selects v_and_or_b32 from plain
// code. (Hand-written inline asm for it hides the VGPR write from the
// compiler's hazard tracking: an MFMA issued right after could read the
// operand before the write landed, which produced garbage outputs.)
struct Q4Consts {
  uint32_t mask;   // 0x000F000F (VGPR)
  uint32_t magic;  // 0x43004300 (SGPR)
};

__device__ inline Q4Consts q4_consts() {
  Q4Consts c{0x000F000Fu, 0x43004300u};
  asm volatile("" : "+v"(c.mask), "+s"(c.magic));
  return c;
}

__device__ inline uint32_t and_or_b32(uint32_t a, uint32_t mask, uint32_t magic) { return (a & mask) | magic; }

__device__ inline bf16x8 q4_offset_bf16_s(uint32_t w, Q4Consts c) {
  u32x4 d;
  d[0] = and_or_b32(w, c.mask, c.magic);
  d[1] = and_or_b32(w >> 4, c.mask, c.magic);
  d[2] = and_or_b32(w >> 8, c.mask, c.magic);
  d[3] = and_or_b32(w >> 12, c.mask, c.magic);
  return __builtin_bit_cast(bf16x8, d);
}

__device__ inline f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ inline bf16x8 bf16x8_ones() {
  const u32x4 ones_bits = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  return __builtin_bit_cast(bf16x8, ones_bits);
}

// One 64-wide group of the tiled layout: the A fragments of two MFMA steps
// (xa0, xa1), the lane's weight words for the group (w0, w1) and its packed
// (scale, bias) bf16 pair. Returns s * sum x*(128+q) + (b - 128 s) * sum x for
// the lane's 4 accumulator rows.
__device__ inline f32x4 q4_group_dot(bf16x8 xa0, bf16x8 xa1, uint32_t w0, uint32_t w1, uint32_t sb) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const bf16x8 ones = bf16x8_ones();
  f32x4 ax = mfma16(xa0, ones, zero);
  ax = mfma16(xa1, ones, ax);
  f32x4 acc = mfma16(xa0, q4_offset_bf16(w0), zero);
  acc = mfma16(xa1, q4_offset_bf16(w1), acc);
  const float s = bf16_to_f32(bf16_t(sb & 0xFFFFu));
  const float bp = bf16_to_f32(bf16_t(sb >> 16)) - 128.f * s;
  f32x4 out;
#pragma unroll
  for (int r = 0; r < 4; ++r) out[r] = s * acc[r] + bp * ax[r];
  return out;
}

// Same with the per-row sums of x over the group (ax) supplied by the caller,
// e.g. computed once while staging x, which halves the MFMA work.
__device__ inline f32x4 q4_group_dot_ax(bf16x8 xa0, bf16x8 xa1, uint32_t w0, uint32_t w1, uint32_t sb, f32x4 ax) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc = mfma16(xa0, q4_offset_bf16(w0), zero);
  acc = mfma16(xa1, q4_offset_bf16(w1), acc);
  const float s = bf16_to_f32(bf16_t(sb & 0xFFFFu));
  const float bp = bf16_to_f32(bf16_t(sb >> 16)) - 128.f * s;
  f32x4 out;
#pragma unroll
  for (int r = 0; r < 4; ++r) out[r] = s * acc[r] + bp * ax[r];
  return out;
}

// Per-group sums of bf16 activations (the sum over each 64-column group of x
// that the tiled 4-bit projections scale by b - 128 s). One fixed order
// everywhere they are computed, so every producer and consumer gets the same
// bits: a thread holding 8 consecutive columns (one packed uint4) adds them as
// pairs, (((lo0 + hi0) + (lo1 + hi1)) + ...) from zero, and the 8 lanes of an
// aligned group combine with sum8_lanes.
__device__ inline float bf16x8_pair_sum(uint4 v) {
  const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
  float sum = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) sum += bf16_to_f32(bf16_t(vw[q] & 0xFFFFu)) + bf16_to_f32(bf16_t(vw[q] >> 16));
  return sum;
}

// Sum over the eight lanes of an aligned group: each lane adds its partner at
// distance 1, then 2, then its mirror in the group of 8; every step adds the
// same two operands as the xor butterfly (1, 2, 4), so the group's total is
// the same value, without an LDS round trip.
__device__ inline float sum8_lanes(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  return v;
}

}  // namespace hb
