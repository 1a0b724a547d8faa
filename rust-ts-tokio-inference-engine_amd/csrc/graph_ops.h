// Fused operators of the graph API (rs_mlx_kernel op codes 1-6,
// native/mlx_bridge.cpp:141-167; callers src/serving/native_ops.rs:53-244).
// General f32 shapes: these serve the reference's graph callers and its
// operator tests, not the decode step (which runs the engine's kernels).
#pragma once
#include "hb_common.h"

namespace hb {

// op 1, mx::fast::rope(x, dims, traditional = false, base, scale = 1, offset):
// x f32 [rows][L][D] (rows = all leading axes); position of row l is
// offset + l; pairs (i, i + dims/2) for i < dims/2 rotate by
// (offset + l) * base^(-2i/dims); columns >= dims are copied.
void graph_rope(const float* x, float* y, int rows, int L, int D, int dims, int offset, float base, hipStream_t s);

// op 2, mx::fast::scaled_dot_product_attention(q, k, v, scale, causal):
// q [B][Hq][Tq][D], k [B][Hkv][Tk][D], v [B][Hkv][Tk][Dv] f32, Hq % Hkv == 0
// (query head h reads kv head h / (Hq / Hkv)); causal: query i sees keys
// j <= i + Tk - Tq. scores [B][Hq][Tq][Tk] is scratch. out [B][Hq][Tq][Dv].
void graph_sdpa(const float* q, const float* k, const float* v, float* scores, float* out, int B, int Hq, int Hkv,
                int Tq, int Tk, int D, int Dv, float scale, bool causal, hipStream_t s);

// op 3, the gated delta rule per token t (native/mlx_bridge.cpp:144-156):
//   S *= decay_t; mem = S k_t; delta = (v_t - mem) * beta_t; S += delta k_t^T;
//   y_t = S q_t
// q, k [B][T][Hk][Dk], v [B][T][Hv][Dv], decay, beta [B][T][Hv], state
// [B][Hv][Dv][Dk] (value head h reads key head h / (Hv / Hk)). Writes y
// [B][T][Hv][Dv] and the final state into state_out.
void graph_gated_delta(const float* q, const float* k, const float* v, const float* decay, const float* beta,
                       const float* state, float* y, float* state_out, int B, int T, int Hk, int Hv, int Dk, int Dv,
                       hipStream_t s);

// op 4, softmax then top-k with renormalised scores (native/mlx_bridge.cpp:158-163):
// logits f32 [rows][E] -> idx u32 [rows][top] (descending probability, lower
// index first on ties), scores f32 [rows][top].
void graph_route_topk(const float* logits, uint32_t* idx, float* scores, int rows, int E, int top, hipStream_t s);

// op 5, mx::gather_qmm(x, w, scales, biases, rhs_indices = idx, transpose = true,
// group, bits, "affine"): x f32 [rows][K], w u32 [E][N][K*bits/32] (LSB-first
// codes), scales/biases f32 [E][N][K/group], idx u32 [rows][top] (checked
// < E by the caller) -> y f32 [rows][top][N].
void graph_gather_qmm(const float* x, const uint32_t* w, const float* scales, const float* biases,
                      const uint32_t* idx, float* y, int rows, int top, int N, int K, int group, int bits,
                      hipStream_t s);

// op 6, sum over j of experts[r][j][n] * scores[r][j] -> y f32 [rows][N].
void graph_mix(const float* experts, const float* scores, float* y, int rows, int top, int N, hipStream_t s);

}  // namespace hb
