// Device helpers of greedy selection shared by the argmax kernels and the
// vocabulary-head GEMM's fused selection epilogue: the f32 total-order key
// (native/selection.h:3-13: -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN by
// bit pattern) and a mergeable (best, index, second best) summary.
#pragma once
#include "hb_common.h"

namespace hb {
namespace {

__device__ inline uint32_t total_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline float key_value(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __builtin_bit_cast(float, u);
}

// top1 = (key, index), top2 = key of the best element other than top1's index.
struct Top2 {
  uint32_t k1;
  uint32_t i1;
  uint32_t k2;
  bool has2;
};

__device__ inline bool better(uint32_t ka, uint32_t ia, uint32_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

__device__ inline Top2 merge(const Top2& a, const Top2& b) {
  // an empty side carries i1 == UINT32_MAX
  if (b.i1 == 0xFFFFFFFFu) return a;
  if (a.i1 == 0xFFFFFFFFu) return b;
  Top2 r;
  const Top2& w = better(a.k1, a.i1, b.k1, b.i1) ? a : b;
  const Top2& l = better(a.k1, a.i1, b.k1, b.i1) ? b : a;
  r.k1 = w.k1;
  r.i1 = w.i1;
  // second best: the loser's top1 or the winner's top2
  r.k2 = l.k1;
  r.has2 = true;
  if (w.has2 && w.k2 > r.k2) r.k2 = w.k2;
  return r;
}

}  // namespace
}  // namespace hb
