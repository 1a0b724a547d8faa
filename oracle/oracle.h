/*
 * CPU oracle for the continuous-batching decode step of the hybrid Qwen decoder.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/, the
 * smoke() entry point and bench.py's cpu_baseline leg may load it. The product
 * path (libhip_bridge.so) never links, loads or calls it.
 *
 * Every function restates the reference semantics in plain C with FP64
 * accumulation (except the two FP32 forms of the 4-bit products, which time
 * the CPU baseline and check nothing); each cites the reference file:line it
 * follows. Inputs that the
 * GPU path receives as bf16 are handed to the oracle as the identical values
 * widened to float, so both sides see bit-identical operands.
 *
 * Return convention: 0 on success, -1 on an invalid descriptor (the reference
 * oracles throw std::invalid_argument in the same places).
 */
#ifndef ORACLE_H
#define ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* A1 affine quantisation: code of column `col` in a LSB-first packed row.
 * native/projection_reference.h:16 (word/shift extraction, words may straddle). */
unsigned orc_code(const uint32_t* row, size_t col, int bits);

/* y[r*outputs+o] = sum_c x[r*width+c] * (s*q + b)  (FP64).
 * native/projection_reference.h:8-22; MLX quantized_matmul(transpose=true) at
 * native/qwen_model.inc:34 and native/mlx_bridge.cpp:72,75. Any row count. */
int orc_qmm(const float* x, size_t rows, const uint32_t* packed, const float* scales,
            const float* biases, size_t outputs, size_t width, int group, int bits,
            double* y, int threads);

/* FP32 restatement of the same product for 4-bit group-64 weights (the CPU
 * baseline's timing path, not a parity reference): per output row and group
 * the 64 weights s*q + b are formed once in f32 and applied to every token
 * row, f32 accumulation, OpenMP over output rows. y f32 [rows][outputs]. */
int orc_qmm4_f32(const float* x, size_t rows, const uint32_t* packed, const float* scales,
                 const float* biases, size_t outputs, size_t width, float* y, int threads);

/* The grouped form of orc_qmm4_f32: y[(r*top+j)][o] = x[r] . W_e[o] with
 * e = idx[r*top+j] over experts [experts][outputs][width]; every (expert,
 * output row) pair dequantises its row once for all the tokens routed to it. */
int orc_gather_qmm4_f32(const float* x, int rows, const uint32_t* packed, const float* scales,
                        const float* biases, int experts, int outputs, int width, const int32_t* idx,
                        int top, float* y, int threads);

/* Dequantised rows (embedding gather). native/projection_reference.h:23-30,
 * native/qwen_model.inc:306-309. */
int orc_dequant(const uint32_t* packed, const float* scales, const float* biases,
                size_t rows, size_t width, int group, int bits, double* out);

/* RMSNorm, weight optional. native/operator_reference.h:11-14, qwen_model.inc:19-32. */
int orc_rms(const float* x, const float* weight, size_t rows, size_t width, double eps,
            double* y);
/* x*sigmoid(x). native/operator_reference.h:9-10. */
int orc_silu(const float* x, size_t n, double* y);
double orc_sigmoid(double x);

/* Non-traditional partial RoPE on x[tokens][heads][dim] with per-token absolute
 * positions. native/operator_reference.h:15-18 (angle = pos * theta^(-2j/rotary)). */
int orc_rope(const float* x, int tokens, int heads, int dim, int rotary,
             const int32_t* positions, double theta, double* y);

/* Ragged paged GQA attention with causal mask inside each row's new tokens and
 * optional sigmoid output gate.
 *   q      [total_tokens][hq][dim]
 *   kcache [pages][hkv][page][dim], vcache likewise
 *   block_table [rows][max_pages], cu_seqlens [rows+1], context [rows]
 *   (context = visible length after the new tokens are appended)
 *   gate   [total_tokens][hq][dim] or NULL
 * native/attention_reference.h:8-21 (FP64 softmax, kv head h/(hq/hkv),
 * visible = offset + row + 1); gate: native/qwen_model.inc:151-152. */
int orc_paged_attention(const float* q, const float* kcache, const float* vcache,
                        const int32_t* block_table, int max_pages, const int32_t* cu_seqlens,
                        const int32_t* context, int rows, int hq, int hkv, int dim, int page,
                        double scale, const float* gate, double* out);

/* Gated delta recurrence on already-normalised operands (rs_mlx_kernel op 3).
 * q,k [b][t][hk][dk], v [b][t][hv][dv], decay,beta [b][t][hv], state [b][hv][dv][dk].
 * native/mlx_bridge.cpp:143-156; native/qwen_model.inc:191-200. */
int orc_gated_delta(const float* q, const float* k, const float* v, const float* decay,
                    const float* beta, const float* state, int b, int t, int hk, int hv,
                    int dk, int dv, double* out, double* state_out);

/* Full Gated DeltaNet mixer core for one sequence: causal depthwise conv with
 * rolling history, SiLU, q/k normalisation, gates, recurrence.
 *   qkv [t][channels], history [kernel-1][channels], conv_w [channels][kernel],
 *   a,b [t][hv], alog,dt [hv], state [hv][dv][dk]
 * native/operator_reference.h:20-44; qwen_model.inc:154-206. */
int orc_gdn(const float* qkv, const float* history, const float* conv_w, const float* a,
            const float* b, const float* alog, const float* dt, const float* state, int t,
            int hk, int hv, int dk, int dv, int kernel, double* activated,
            double* history_out, double* out, double* state_out);

/* Router: softmax over experts (FP64), top-k chosen on logits under IEEE total
 * order with the lower index first on ties, weights renormalised over the
 * selection. idx/weights are [rows][top] in descending order.
 * native/qwen_model.inc:77-79; native/operator_reference.h:48-57. */
int orc_route_topk(const float* logits, int rows, int experts, int top, int32_t* idx,
                   double* weights);

/* Stable counting sort of the flattened (token, slot) pairs by expert.
 * order[p] = flat index (t*top+j) of the p-th pair in expert order, inverse is
 * its inverse permutation, offsets[e] = first pair of expert e (size experts+1).
 * Closed form of the argsort in native/qwen_model.inc:81 with stability fixed. */
int orc_expert_permute(const int32_t* idx, int tokens, int top, int experts, int32_t* order,
                       int32_t* inverse, int32_t* offsets);

/* Per-(token,slot) expert projection. x [rows][width], packed [experts][outputs][words],
 * scales/biases [experts][outputs][groups], idx [rows][top] -> y [rows][top][outputs].
 * native/mlx_bridge.cpp:164-166 (gather_qmm), qwen_model.inc:35-56. */
int orc_gather_qmm(const float* x, int rows, const uint32_t* packed, const float* scales,
                   const float* biases, int experts, int outputs, int width, int group, int bits,
                   const int32_t* idx, int top, double* y, int threads);

/* Weighted sum over slots: y[r] = sum_j scores[r][j] * e[r][j]. native/mlx_bridge.cpp:167. */
int orc_mix(const float* experts, const float* scores, int rows, int top, int width, double* y);

/* Greedy winner under f32 total order (lowest index on ties) plus top1-top2 margin.
 * Rejects empty or non-finite rows. src/serving/native_speculative.rs:45-73,
 * native/selection.h:5-13. */
int orc_winner(const float* logits, size_t n, uint32_t* token, float* margin);

/* MTP acceptance plan. src/serving/native_speculative.rs:74-128.
 * rows is [n_draft][vocab]; emitted has capacity n_draft+1. */
int orc_plan(const float* initial, size_t vocab, const uint32_t* draft, size_t n_draft,
             const float* rows, const uint32_t* eos, size_t n_eos, size_t remaining,
             uint32_t* emitted, size_t* n_emitted, size_t* accepted, int* terminal);

/* Ragged packing tables (closed form). For row r with row_tokens[r] new tokens
 * starting at absolute position positions[r]:
 *   cu_seqlens[r+1] = cu_seqlens[r] + row_tokens[r]
 *   token_row[i] = r, token_pos[i] = positions[r] + j
 *   kv_slot[i]  = block_table[r][pos/page]*page + pos%page
 *   context[r]  = positions[r] + row_tokens[r]
 * Generalises the concat packer of native/qwen_batch.inc:2-50 to ragged rows. */
int orc_pack_tables(const int32_t* row_tokens, const int32_t* positions,
                    const int32_t* block_table, int max_pages, int rows, int page,
                    int32_t* cu_seqlens, int32_t* token_row, int32_t* token_pos,
                    int32_t* kv_slot, int32_t* context);

/* bf16 helpers (round-to-nearest-even, NaN preserved). */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t x);

/* Thread count the oracle will use for threads<=0. */
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
