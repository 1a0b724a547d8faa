// Gated GQA attention over a paged bf16 KV cache (ragged decode / MTP verify).
// Reference semantics: Qwen::attention, native/qwen_model.inc:101-153;
// FP64 oracle native/attention_reference.h:8-21.
#pragma once
#include "hb_common.h"

namespace hb {

// Cache layouts (one attention layer):
//   K: [pages][kv_heads][page][head_dim]   bf16 (key-major rows)
//   V: [pages][kv_heads][head_dim][page]   bf16 (transposed within a page)
constexpr int kPage = 16;

struct AttnGeom {
  int q_heads, kv_heads, head_dim;
  int rotary;       // partial RoPE dims (64 of 256)
  float theta;      // RoPE base (1e7)
  float eps;        // q/k RMSNorm epsilon
};

// Per packed token i: q = rope(rms(q_i, q_norm)), k = rope(rms(k_i, k_norm)),
// v as is; k and v are written to kv_slot[i] of the paged cache.
//   qg  bf16 [T][q_heads][2*head_dim] (q then gate per head), row stride ld_qg
//   kv  bf16 [T][...]: k at kv + i*ld_kv, v at kv + i*ld_kv + kv_off (each kv_heads*head_dim)
//   qout bf16 [T][q_heads][head_dim]
void attn_prep(const bf16_t* qg, int ld_qg, const bf16_t* kv, int ld_kv, int kv_off, const float* q_norm,
               const float* k_norm, const int32_t* token_pos, const int32_t* kv_slot, int tokens, const AttnGeom& g,
               bf16_t* qout, bf16_t* kcache, bf16_t* vcache, hipStream_t stream);

// Split-K partial attention. Query token t of row r (0 <= t < T_r) sits at
// absolute position context[r] - T_r + t and sees keys 0..that position. A
// piece is (row, group of 16 (token, q head) pairs, split, kv head) over keys
// [split * split_len, min((split + 1) * split_len, context[r])): the cut
// depends on the row alone, so a row's result never depends on its batch.
//   work_o  f32 [rows][kv_heads][row_groups][splits][16][head_dim]
//   work_ml f32 [rows][kv_heads][row_groups][splits][16][2]   (running max, sum)
//   plan    int32 [attn_plan_ints]: [0] piece count, then the pieces as
//           (row * row_groups + group, split * kv_heads + kv head) pairs from 2 on
// row_groups = ceil(max_tokens * group / 16), splits = ceil(max_context / split_len).
struct AttnWork {
  int rows, max_tokens, row_groups, splits, split_len;
  float* work_o;
  float* work_ml;
  int32_t* plan;
};
size_t attn_work_floats_o(int rows, int kv_heads, int head_dim, int max_tokens, int group, int max_context,
                          int split_len);
size_t attn_plan_ints(int rows, int kv_heads, int row_groups, int splits);
// Lists the step's pieces: whole pieces first, then the rows' shorter last
// pieces by decreasing length (one wave each, dispatched in list order, so
// the longest work starts first). One list serves every attention layer of
// the step.
void attn_plan(const int32_t* cu_seqlens, const int32_t* context, const AttnGeom& g, const AttnWork& w,
               hipStream_t stream);
void paged_attention(const bf16_t* q, const bf16_t* kcache, const bf16_t* vcache, const int32_t* block_table,
                     int max_pages, const int32_t* cu_seqlens, const int32_t* context, const AttnGeom& g, float scale,
                     const AttnWork& w, hipStream_t stream);

// out[i][h] = sigmoid(gate[i][h]) * combine over splits; bf16 [T][q_heads][head_dim].
void attn_combine(const AttnWork& w, const int32_t* token_row, const int32_t* cu_seqlens, const int32_t* context,
                  const bf16_t* qg, int ld_qg, int tokens, const AttnGeom& g, bf16_t* out, hipStream_t stream);

}  // namespace hb
