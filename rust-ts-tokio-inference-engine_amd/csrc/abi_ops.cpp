// Additive device-pointer entry points for the per-step operators (packing,
// attention, recurrence, MoE, selection). Each validates its descriptor and
// launches on the caller's stream; results stay in HBM.
#include "../../include/hip_bridge.h"
#include "attention.h"
#include "deltanet.h"
#include "hb_common.h"
#include "moe.h"
#include "pack.h"
#include "synth.h"

using namespace hb;

extern "C" int hb_random_q4(uint64_t seed, int N, int K, float std_dev, uint32_t* w, void* scales, void* biases,
                            void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    random_q4(seed, N, K, std_dev, w, static_cast<bf16_t*>(scales), static_cast<bf16_t*>(biases), as_stream(stream));
  });
}

extern "C" int hb_random_normal(uint64_t seed, size_t n, float std_dev, float mean, int dtype, void* out,
                                void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] { random_normal(seed, n, std_dev, mean, dtype, out, as_stream(stream)); });
}

extern "C" int hb_random_uniform(uint64_t seed, size_t n, float lo, float hi, int dtype, void* out, void* stream,
                                 char* error, size_t capacity) {
  return guarded(error, capacity, [&] { random_uniform(seed, n, lo, hi, dtype, out, as_stream(stream)); });
}

extern "C" int hb_random_ints(uint64_t seed, size_t n, uint32_t bound, uint32_t* out, void* stream, char* error,
                              size_t capacity) {
  return guarded(error, capacity, [&] { random_ints(seed, n, bound, out, as_stream(stream)); });
}

extern "C" size_t hb_moe_items_capacity(int tokens, int experts, int top) {
  return moe_items_capacity(tokens, experts, top);
}

extern "C" int hb_moe_route(const float* logits, int ld_logits, int tokens, int experts, int top, int32_t* idx,
                            float* weights, int32_t* counts, int32_t* offsets, int32_t* order, int32_t* inverse,
                            int32_t* items, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    moe_route(logits, ld_logits, tokens, experts, top, idx, weights, counts, offsets, order, inverse, items,
              as_stream(stream));
  });
}

extern "C" int hb_moe_grouped_qmm(const void* x, int K, const uint32_t* w_tiled, const void* sb_tiled, int n_rows,
                                  const int32_t* counts, const int32_t* offsets, const int32_t* order,
                                  const int32_t* items, int experts, int top, int tokens, int swiglu, void* y,
                                  void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    moe_grouped_qmm(static_cast<const bf16_t*>(x), K, w_tiled, static_cast<const bf16_t*>(sb_tiled), n_rows, counts,
                    offsets, order, items, experts, top, tokens, swiglu, static_cast<bf16_t*>(y),
                    as_stream(stream));
  });
}

extern "C" int hb_moe_combine(const void* down, const float* weights, const int32_t* inverse, const float* logits,
                              int ld_logits, int sg_col, int top, int tokens, int hidden, float* residual,
                              void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    moe_combine(static_cast<const bf16_t*>(down), weights, inverse, logits, ld_logits, sg_col, top, tokens, hidden,
                residual, as_stream(stream));
  });
}

extern "C" int hb_pack_tables(const int32_t* row_tokens, const int32_t* positions, const int32_t* block_table,
                              int max_pages, int rows, int page, int32_t* cu_seqlens, int32_t* token_row,
                              int32_t* token_pos, int32_t* kv_slot, int32_t* context, int32_t* status, void* stream,
                              char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    pack_tables(row_tokens, positions, block_table, max_pages, rows, page, cu_seqlens, token_row, token_pos,
                kv_slot, context, status, as_stream(stream));
  });
}

extern "C" int hb_attn_prep(const void* qg, int ld_qg, const void* kv, int ld_kv, int kv_off, const float* q_norm,
                            const float* k_norm, const int32_t* token_pos, const int32_t* kv_slot, int tokens,
                            int q_heads, int kv_heads, int head_dim, int rotary, float theta, float eps, void* qout,
                            void* kcache, void* vcache, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(qg && kv && q_norm && k_norm && token_pos && kv_slot && qout && kcache && vcache,
            "hb_attn_prep: null pointer");
    require(q_heads > 0 && kv_heads > 0 && tokens >= 0, "hb_attn_prep: invalid geometry");
    const AttnGeom g{q_heads, kv_heads, head_dim, rotary, theta, eps};
    attn_prep(static_cast<const bf16_t*>(qg), ld_qg, static_cast<const bf16_t*>(kv), ld_kv, kv_off, q_norm, k_norm,
              token_pos, kv_slot, tokens, g, static_cast<bf16_t*>(qout), static_cast<bf16_t*>(kcache),
              static_cast<bf16_t*>(vcache), as_stream(stream));
  });
}

extern "C" size_t hb_attn_workspace_floats(int rows, int kv_heads, int head_dim, int max_tokens, int group,
                                           int max_context, int split_len) {
  if (rows <= 0 || kv_heads <= 0 || head_dim <= 0 || max_tokens <= 0 || group <= 0 || max_context <= 0 ||
      split_len <= 0)
    return 0;
  const int rgs = (max_tokens * group + 15) / 16, splits = (max_context + split_len - 1) / split_len;
  return attn_work_floats_o(rows, kv_heads, head_dim, max_tokens, group, max_context, split_len) +
         attn_plan_ints(rows, kv_heads, rgs, splits);
}

extern "C" int hb_paged_attention(const void* q, const void* kcache, const void* vcache, const int32_t* block_table,
                                  int max_pages, const int32_t* cu_seqlens, const int32_t* context,
                                  const int32_t* token_row, const void* qg, int ld_qg, int rows, int tokens,
                                  int max_tokens, int max_context, int q_heads, int kv_heads, int head_dim,
                                  float scale, int split_len, float* work_o, float* work_ml, void* out, void* stream,
                                  char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(q && kcache && vcache && block_table && cu_seqlens && context && token_row && qg && work_o && work_ml &&
                out,
            "hb_paged_attention: null pointer");
    require(rows > 0 && tokens >= 0 && max_tokens > 0 && max_context > 0 && q_heads % kv_heads == 0,
            "hb_paged_attention: invalid geometry");
    require(max_context <= max_pages * kPage, "hb_paged_attention: max_context exceeds the block table");
    const AttnGeom g{q_heads, kv_heads, head_dim, 0, 0.f, 0.f};
    const int group = q_heads / kv_heads;
    require(split_len > 0, "hb_paged_attention: split_len must be positive");
    const int rgs = (max_tokens * group + 15) / 16, splits = (max_context + split_len - 1) / split_len;
    // the piece list sits after the partial outputs in work_o
    int32_t* plan = reinterpret_cast<int32_t*>(
        work_o + attn_work_floats_o(rows, kv_heads, head_dim, max_tokens, group, max_context, split_len));
    AttnWork w{rows, max_tokens, rgs, splits, split_len, work_o, work_ml, plan};
    const hipStream_t s = as_stream(stream);
    attn_plan(cu_seqlens, context, g, w, s);
    paged_attention(static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(kcache),
                    static_cast<const bf16_t*>(vcache), block_table, max_pages, cu_seqlens, context, g, scale, w, s);
    attn_combine(w, token_row, cu_seqlens, context, static_cast<const bf16_t*>(qg), ld_qg, tokens, g,
                 static_cast<bf16_t*>(out), s);
  });
}

extern "C" int hb_gdn_prep(const void* qkv, int ld_qkv, const void* a, const void* b, int ld_ab, const float* conv_w,
                           const float* a_log, const float* dt_bias, void* window, const int32_t* hist_off,
                           const int32_t* src_slot, const int32_t* dst_slot, const int32_t* cu_seqlens, int rows,
                           int key_heads, int value_heads, int key_dim, int value_dim, int conv, int max_tokens,
                           float* q_hat, float* k_hat, float* v, float* decay, float* beta, void* stream, char* error,
                           size_t capacity) {
  return guarded(error, capacity, [&] {
    require(qkv && a && b && conv_w && a_log && dt_bias && window && hist_off && cu_seqlens && q_hat && k_hat && v &&
                decay && beta,
            "hb_gdn_prep: null pointer");
    require(key_heads > 0 && value_heads > 0 && max_tokens > 0, "hb_gdn_prep: invalid geometry");
    const GdnGeom g{key_heads, value_heads, key_dim, value_dim, conv, max_tokens};
    gdn_prep(static_cast<const bf16_t*>(qkv), ld_qkv, static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
             ld_ab, conv_w, a_log, dt_bias, static_cast<bf16_t*>(window), hist_off, GdnSlots{src_slot, dst_slot},
             cu_seqlens, rows, g, q_hat, k_hat, v, decay, beta, as_stream(stream));
  });
}

extern "C" int hb_gdn_recurrence(const float* q_hat, const float* k_hat, const float* v, const float* decay,
                                 const float* beta, const int32_t* cu_seqlens, int rows, int key_heads,
                                 int value_heads, int key_dim, int value_dim, float* state, const int32_t* src_slot,
                                 const int32_t* dst_slot, float* log_k, float* log_delta, float* log_g,
                                 const int32_t* log_count, int log_cap, int speculative, float* o_out, const void* z,
                                 int ld_z, const float* norm_w, void* y_out, void* stream, char* error,
                                 size_t capacity) {
  return guarded(error, capacity, [&] {
    require(q_hat && k_hat && v && decay && beta && cu_seqlens && state, "hb_gdn_recurrence: null pointer");
    require(key_heads > 0 && value_heads > 0, "hb_gdn_recurrence: invalid geometry");
    const GdnGeom g{key_heads, value_heads, key_dim, value_dim, 0, 0};
    const GdnLog log{log_k, log_delta, log_g};
    gdn_recurrence(q_hat, k_hat, v, decay, beta, cu_seqlens, rows, g, state, GdnSlots{src_slot, dst_slot}, log,
                   log_count, log, log_cap, speculative, o_out, static_cast<const bf16_t*>(z), ld_z, norm_w,
                   static_cast<bf16_t*>(y_out), as_stream(stream));
  });
}

extern "C" int hb_gdn_decode(const void* qkv, int ld_qkv, const void* a, const void* b, int ld_ab, const float* conv_w,
                             const float* a_log, const float* dt_bias, void* window, const int32_t* hist_off,
                             const int32_t* src_slot, const int32_t* dst_slot, const int32_t* cu_seqlens, int rows,
                             int key_heads, int value_heads, int key_dim, int value_dim, int conv, int max_tokens,
                             float* state, float* log_k, float* log_delta, float* log_g, const int32_t* log_count,
                             int log_cap, int speculative, float* o_out, const void* z, int ld_z, const float* norm_w,
                             void* y_out, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(qkv && a && b && conv_w && a_log && dt_bias && window && hist_off && cu_seqlens && state,
            "hb_gdn_decode: null pointer");
    require(key_heads > 0 && value_heads > 0 && max_tokens > 0, "hb_gdn_decode: invalid geometry");
    const GdnGeom g{key_heads, value_heads, key_dim, value_dim, conv, max_tokens};
    const GdnLog log{log_k, log_delta, log_g};
    const bool fused =
        gdn_decode(static_cast<const bf16_t*>(qkv), ld_qkv, static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
                   ld_ab, conv_w, a_log, dt_bias, static_cast<bf16_t*>(window), hist_off, cu_seqlens, rows, g, state,
                   GdnSlots{src_slot, dst_slot}, log, log_count, log, log_cap, speculative, o_out,
                   static_cast<const bf16_t*>(z), ld_z, norm_w, static_cast<bf16_t*>(y_out), as_stream(stream));
    require(fused, "hb_gdn_decode: the fused step needs conv width 4, 128-wide heads and two value heads per key head");
  });
}

extern "C" int hb_gdn_chunked(const float* q_hat, const float* k_hat, const float* v, const float* decay,
                              const float* beta, const int32_t* cu_seqlens, int rows, int key_heads, int value_heads,
                              int key_dim, int value_dim, float* state, const int32_t* src_slot,
                              const int32_t* dst_slot, float* o_out, const void* z, int ld_z, const float* norm_w,
                              void* y_out, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(q_hat && k_hat && v && decay && beta && cu_seqlens && state, "hb_gdn_chunked: null pointer");
    require(key_heads > 0 && value_heads > 0, "hb_gdn_chunked: invalid geometry");
    const GdnGeom g{key_heads, value_heads, key_dim, value_dim, 0, 0};
    gdn_chunked(q_hat, k_hat, v, decay, beta, cu_seqlens, rows, g, state, GdnSlots{src_slot, dst_slot}, o_out,
                static_cast<const bf16_t*>(z), ld_z, norm_w, static_cast<bf16_t*>(y_out), as_stream(stream));
  });
}
