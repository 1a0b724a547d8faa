// Additive device-pointer entry points for the per-step operators (packing,
// attention, recurrence, MoE, selection). Each validates its descriptor and
// launches on the caller's stream; results stay in HBM.
#include "../../include/hip_bridge.h"
#include "attention.h"
#include "hb_common.h"
#include "pack.h"

using namespace hb;

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
  return attn_work_floats_o(rows, kv_heads, head_dim, max_tokens, group, max_context, split_len);
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
    AttnWork w{rows, max_tokens, (max_tokens * group + 15) / 16, (max_context + split_len - 1) / split_len,
               split_len, work_o, work_ml};
    const hipStream_t s = as_stream(stream);
    paged_attention(static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(kcache),
                    static_cast<const bf16_t*>(vcache), block_table, max_pages, cu_seqlens, context, g, scale, w, s);
    attn_combine(w, token_row, cu_seqlens, context, static_cast<const bf16_t*>(qg), ld_qg, tokens, g,
                 static_cast<bf16_t*>(out), s);
  });
}
