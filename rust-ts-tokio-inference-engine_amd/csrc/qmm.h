// Affine-quantised matmul y[M,N] = x[M,K] . W[N,K]^T with W = s*q + b per group.
// Reference semantics: mx::quantized_matmul(x, W, s, b, transpose=true, group,
// bits, "affine") at native/qwen_model.inc:34 and native/mlx_bridge.cpp:72,75.
#pragma once
#include "hb_common.h"

namespace hb {

// Device weight layouts.
enum WeightLayout : int {
  kLayoutMlx = 0,    // checkpoint format: LSB-first bit stream per row, scales/biases [N][K/g]
  kLayoutQ4Tiled = 1 // 4-bit group-64, MFMA-native tiles (see q4_tile)
};

// Repacks MLX 4-bit g64 weights into the tiled device layout:
//   w_tiled [N/16][K/128][64 lanes][4 words]: lane l = 16*qt + r holds, for row
//     16*tile + r and the group pair (2p, 2p+1), words 2qt and 2qt+1 of group 2p
//     then of group 2p+1, each word with its codes in interleaved order
//     (codes 0,2,4,6 in bits 0-15, codes 1,3,5,7 in bits 16-31);
//   sb_tiled [N/16][K/128][16 rows][4] bf16 = (s_2p, b_2p, s_2p+1, b_2p+1).
// Requires N % 16 == 0 and K % 128 == 0. Both outputs have the input sizes.
void q4_tile(const uint32_t* w_mlx, const bf16_t* scales, const bf16_t* biases, uint32_t* w_tiled,
             bf16_t* sb_tiled, int N, int K, hipStream_t stream);

// y (row stride ldy) = x (bf16 [M][K]) . W^T; out_mode 0: y bf16, 1: y f32,
// 2: y f32 += result (adds a projection straight into an f32 residual stream).
// kLayoutQ4Tiled: w = w_tiled, scales = sb_tiled, biases unused (may be null).
// kLayoutMlx: any bits in {2,3,4,5,6,8}, group in {32,64,128} (generic kernel).
// gsum (optional, tiled layout): the per-64-column group sums of x, f32
// [M][K / 64], as the kernel that wrote x computed them (rmsnorm(), the MoE
// combine's fused norm); the streamed projection then reads them instead of
// recomputing them. Results are the same bits either way.
void qmm(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* scales, const bf16_t* biases,
         int N, int group, int bits, int layout, void* y, int out_mode, int ldy, hipStream_t stream,
         const float* gsum = nullptr);

// Greedy selection fused into a tiled 4-bit projection (the vocabulary head):
// per token the argmax winner, margin and non-finite status over columns
// [0, vocab) of x . W^T, without writing the product. Covers 16 < M <= 256,
// K = 2048, N % 256 == 0 when the grid fills the GPU; false (nothing
// launched) otherwise. `part` holds qmm_select_workspace(M, N) bytes.
size_t qmm_select_workspace(int M, int N);
bool qmm_select(const bf16_t* x, int M, int K, const uint32_t* w_tiled, const bf16_t* sb_tiled, int N, int vocab,
                void* part, size_t part_bytes, uint32_t* winner, float* margin, int32_t* status, hipStream_t stream);

}  // namespace hb
