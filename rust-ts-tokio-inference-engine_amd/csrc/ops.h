// Small elementwise / normalisation kernels used by the graph API and the
// decode step (f32 and bf16 variants).
#pragma once
#include <array>

#include "hb_common.h"

namespace hb {

constexpr int kMaxRank = 4;
using Dims = std::array<int64_t, kMaxRank>;

// dst[i] = bf16(src[i])
void f32_to_bf16_n(const float* src, bf16_t* dst, size_t n, hipStream_t s);
// dst[i] = f32(src[i]) for bf16 (is_f16=false) or f16 (is_f16=true) sources
void half_to_f32_n(const uint16_t* src, float* dst, size_t n, bool is_f16, hipStream_t s);
void f16_to_bf16_n(const uint16_t* src, bf16_t* dst, size_t n, hipStream_t s);

// Broadcast binary op on f32 tensors of rank <= 4 (shapes right-aligned and
// padded to rank 4; stride 0 on broadcast axes). op: 0 add, 1 multiply, 2 a - b.
void binary_f32(int op, const float* a, Dims astride, const float* b, Dims bstride, float* y, Dims shape,
                hipStream_t s);

// y[b][m][n] = sum_k a[b][m][k] * w[b'][k][n] (f32, batch broadcast of w when wb == 1)
void matmul_f32(const float* a, const float* w, float* y, int batch, int wbatch, int M, int N, int K, hipStream_t s);

// RMSNorm over the last axis: y = x * rsqrt(mean(x^2) + eps) * (weight or 1).
void rms_norm_f32(const float* x, const float* weight, float* y, int rows, int width, float eps, hipStream_t s);

// y = x * sigmoid(x)
void silu_f32(const float* x, float* y, size_t n, hipStream_t s);

}  // namespace hb
