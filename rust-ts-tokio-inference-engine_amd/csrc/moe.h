// Sparse MoE block over packed ragged tokens (Qwen::moe, native/qwen_model.inc:75-100).
#pragma once
#include "hb_common.h"

namespace hb {

constexpr int kMoeMaxPairs = 4096;  // tokens * top handled by one routing workgroup

// Router: per token, top-k of the first `experts` logits under IEEE total order
// (lowest index first on ties), weights = softmax renormalised over the
// selection; then a stable counting sort of the flattened (token, slot) pairs
// by expert: order[offsets[e] + i] is the i-th pair of expert e in pair order,
// inverse[p] its position. Reference: softmax/argpartition/take_along_axis at
// qwen_model.inc:77-79 and argsort at :81 (whose tie order MLX leaves open).
// active (optional): receives the number of routed experts with a pair.
// items (moe_items_capacity int32): the grouped GEMM's work list, items[0] =
// count, then slot << 16 | tile for the shared expert's 16-token tiles (slot 0)
// and every routed expert's 16-pair tiles (slot e + 1); after the list, one
// 64-byte record per tile (expert, first output row, rows, source tokens) in
// the order the persistent grouped GEMM walks them.
size_t moe_items_capacity(int tokens, int experts, int top);
void moe_route(const float* logits, int ld_logits, int tokens, int experts, int top, int32_t* idx, float* weights,
               int32_t* counts, int32_t* offsets, int32_t* order, int32_t* inverse, int32_t* items,
               hipStream_t stream, int32_t* active = nullptr);

// Grouped affine 4-bit GEMM over experts. Weights are [experts+1] matrices of
// n_rows x K in the tiled layout (index `experts` is the shared expert);
// routed expert e multiplies its counts[e] pairs, the shared expert all tokens
// in chunks of 16. Output rows are in sorted pair order, shared rows follow at
// P + token (P = tokens * top).
//   swiglu = 1: A = x[token] (bf16 [tokens][K]); the matrix interleaves gate and up
//     rows per 16-row tile (8 gate rows then the 8 matching up rows) and the
//     output is silu(gate) * up, bf16 [P + tokens][n_rows / 2]
//     (Qwen::expert up/gate and silu(gate)*up, qwen_model.inc:85-93);
//   swiglu = 0: A = x[row] (bf16 [P + tokens][K], sorted order), output bf16 [P + tokens][n_rows].
// items: the work list moe_route wrote (null selects the non-persistent kernels).
void moe_grouped_qmm(const bf16_t* x, int K, const uint32_t* w_tiled, const bf16_t* sb_tiled, int n_rows,
                     const int32_t* counts, const int32_t* offsets, const int32_t* order, const int32_t* items,
                     int experts, int top, int tokens, int swiglu, bf16_t* y, hipStream_t stream);

// residual[t] += sum_j weights[t][j] * down[inverse[t*top+j]] + sigmoid(logits[t][sg_col]) * down[P + t]
// (weighted mixture and shared-expert merge, qwen_model.inc:95-98). f32 residual [tokens][hidden].
// Optional fused RMSNorm of the updated residual rows (the next layer's input
// norm): out = bf16(x * rsqrt(mean(x^2) + eps) * w), also f32 into out_f32
// when given; bit-identical to rmsnorm() over the residual.
struct CombineNorm {
  const float* w = nullptr;
  float eps = 0.f;
  bf16_t* out = nullptr;
  int ld_out = 0;
  float* out_f32 = nullptr;
  float* gsum = nullptr;  // optional: per-64-column group sums of out, f32 [T][hidden / 64] (as rmsnorm())
};
void moe_combine(const bf16_t* down, const float* weights, const int32_t* inverse, const float* logits,
                 int ld_logits, int sg_col, int top, int tokens, int hidden, float* residual, hipStream_t stream,
                 const CombineNorm* norm = nullptr);

// out[0] = number of experts with counts[e] > 0 (the routed experts whose
// weights one grouped GEMM launch reads).
void moe_count_active(const int32_t* counts, int experts, int32_t* out, hipStream_t stream);

}  // namespace hb
