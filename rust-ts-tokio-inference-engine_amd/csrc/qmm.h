// Affine-quantised matmul y[M,N] = x[M,K] . W[N,K]^T with W = s*q + b per group.
// Reference semantics: mx::quantized_matmul(x, W, s, b, transpose=true, group,
// bits, "affine") at native/qwen_model.inc:34 and native/mlx_bridge.cpp:72,75.
#pragma once
#include "hb_common.h"

namespace hb {

// Device weight layouts.
enum WeightLayout : int {
  kLayoutMlx = 0,          // LSB-first bit stream per row (the checkpoint format)
  kLayoutQ4Interleaved = 1 // 4-bit only: per 32-bit word, codes 0,2,4,6 in bits 0-15 and
                           // 1,3,5,7 in bits 16-31 (nibble i/2 of each half), so one
                           // mask yields two adjacent codes in the two bf16 halves.
};

// MLX 4-bit words -> interleaved words (n words, device pointers).
void q4_interleave(const uint32_t* in, uint32_t* out, size_t n, hipStream_t stream);

// y (bf16 or f32) = x (bf16 [M][K], row stride K) . W^T.
// 4-bit g64 interleaved weights use the MFMA path; everything else the generic path.
void qmm(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* scales, const bf16_t* biases,
         int N, int group, int bits, int layout, void* y, bool y_f32, int ldy, hipStream_t stream);

}  // namespace hb
