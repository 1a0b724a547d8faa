// C-ABI for greedy selection, acceptance, norms, the decode engine and the
// speculative decode loop (declared in include/hip_bridge.h).
#include <algorithm>
#include <cstring>
#include <vector>

#include "qmm.h"
#include "decode.h"
#include "engine.h"
#include "norm.h"
#include "select.h"

using namespace hb;

extern "C" size_t hb_argmax_workspace_bytes(int rows, int vocab) { return argmax_workspace_bytes(rows, vocab); }

extern "C" int hb_argmax_margin(const float* logits, int ld, int rows, int vocab, uint32_t* winner, float* margin,
                                int32_t* status, void* workspace, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(rows >= 0 && vocab > 0 && ld >= vocab, "hb_argmax_margin: invalid geometry");
    argmax_margin(logits, ld, rows, vocab, winner, margin, status, as_stream(stream), workspace);
  });
}

extern "C" size_t hb_argmax_noalloc_limit_bytes(void) { return kSelectScratchBytes; }

extern "C" int hb_argmax_margin_noalloc(const float* logits, int ld, int rows, int vocab, uint32_t* winner,
                                        float* margin, int32_t* status, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(rows >= 0 && vocab > 0 && ld >= vocab, "hb_argmax_margin_noalloc: invalid geometry");
    require(argmax_workspace_bytes(rows, vocab) <= kSelectScratchBytes,
            "hb_argmax_margin_noalloc: rows x ceil(vocab / 8192) exceeds the 65536 summaries of the 1 MiB static "
            "scratch");
    if (rows == 0) return;
    argmax_margin(logits, ld, rows, vocab, winner, margin, status, as_stream(stream), select_scratch());
  });
}

extern "C" size_t hb_qmm_select_workspace_bytes(int rows, int n) { return qmm_select_workspace(rows, n); }

extern "C" int hb_qmm_select(const void* x, int rows, int K, const uint32_t* w_tiled, const void* sb_tiled, int n,
                             int vocab, void* workspace, size_t workspace_bytes, uint32_t* winner, float* margin,
                             int32_t* status, int* fused, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(fused, "hb_qmm_select: descriptor");
    *fused = qmm_select(static_cast<const bf16_t*>(x), rows, K, w_tiled, static_cast<const bf16_t*>(sb_tiled), n,
                        vocab, workspace, workspace_bytes, winner, margin, status, as_stream(stream))
                 ? 1
                 : 0;
  });
}

extern "C" int hb_mtp_plan(const uint32_t* draft, const int32_t* n_draft, int max_draft, const uint32_t* target,
                           const uint32_t* eos, int n_eos, const int32_t* remaining, int rows, int vocab,
                           uint32_t* emitted, int32_t* n_emitted, int32_t* accepted, int32_t* terminal,
                           int32_t* status, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(rows >= 0 && vocab > 0, "hb_mtp_plan: invalid geometry");
    mtp_plan(draft, n_draft, max_draft, target, eos, n_eos, remaining, rows, vocab, emitted, n_emitted, accepted,
             terminal, status, as_stream(stream));
  });
}

extern "C" int hb_embed_gather(const uint32_t* tokens, int count, const uint32_t* w, const void* scales,
                               const void* biases, int hidden, float* out, void* stream, char* error,
                               size_t capacity) {
  return guarded(error, capacity, [&] {
    embed_gather(tokens, count, w, static_cast<const bf16_t*>(scales), static_cast<const bf16_t*>(biases), hidden, out,
                 as_stream(stream));
  });
}

extern "C" int hb_rmsnorm(const float* x, int ld_x, const float* weight, int rows, int hidden, float epsilon,
                          void* out, int ld_out, float* out_f32, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(hidden > 0 && ld_x >= hidden && ld_out >= hidden, "hb_rmsnorm: invalid geometry");
    rmsnorm(x, ld_x, weight, rows, hidden, epsilon, static_cast<bf16_t*>(out), ld_out, as_stream(stream), out_f32);
  });
}

extern "C" int hb_rmsnorm_gs(const float* x, int ld_x, const float* weight, int rows, int hidden, float epsilon,
                             void* out, int ld_out, float* gsum, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(hidden > 0 && ld_x >= hidden && ld_out >= hidden && gsum, "hb_rmsnorm_gs: invalid geometry");
    rmsnorm(x, ld_x, weight, rows, hidden, epsilon, static_cast<bf16_t*>(out), ld_out, as_stream(stream), nullptr,
            gsum);
  });
}

extern "C" int hb_qmm_gs(const void* x, const uint32_t* w_tiled, const void* sb_tiled, void* y, int M, int N, int K,
                         int out_mode, int ld_y, const float* gsum, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(gsum, "hb_qmm_gs: null group sums");
    qmm(static_cast<const bf16_t*>(x), M, K, w_tiled, static_cast<const bf16_t*>(sb_tiled), nullptr, N, 64, 4,
        kLayoutQ4Tiled, y, out_mode, ld_y, as_stream(stream), gsum);
  });
}

// ------------------------------------------------------------------ engine
extern "C" void* hb_engine_create(const rs_qwen_config* config, int max_rows, int max_context, int max_row_tokens,
                                  int max_step_tokens, uint64_t seed, int mtp, char* error, size_t capacity) {
  Engine* e = nullptr;
  const int rc = guarded(error, capacity, [&] {
    require(config, "hb_engine_create: null config");
    e = new Engine(*config, max_rows, max_context, max_row_tokens, max_step_tokens, seed, mtp != 0);
  });
  return rc == 0 ? e : nullptr;
}

extern "C" void hb_engine_destroy(void* engine) { delete static_cast<Engine*>(engine); }

extern "C" int hb_engine_info(void* engine, uint64_t* out, size_t count, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && out && count >= 4, "hb_engine_info: descriptor");
    auto& e = *static_cast<Engine*>(engine);
    const uint64_t v[5] = {e.weight_bytes(), e.state_bytes(), uint64_t(e.max_pages()),
                           reinterpret_cast<uint64_t>(e.stream()), e.fused_heads()};
    std::memcpy(out, v, std::min(count, size_t(5)) * sizeof(uint64_t));
  });
}

extern "C" int hb_engine_tensor_shape(void* engine, int id, int32_t* rows, int32_t* cols, int32_t* q4, char* error,
                                      size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && rows && cols && q4, "hb_engine_tensor_shape: descriptor");
    int N, K;
    bool q;
    static_cast<Engine*>(engine)->tensor_shape(id, N, K, q);
    *rows = N;
    *cols = K;
    *q4 = q;
  });
}

extern "C" int hb_engine_export(void* engine, int id, void* w, void* scales, void* biases, char* error,
                                size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && w, "hb_engine_export: descriptor");
    auto& e = *static_cast<Engine*>(engine);
    int N, K;
    bool q;
    e.tensor_shape(id, N, K, q);
    require(!q || (scales && biases), "hb_engine_export: scales/biases needed for a 4-bit tensor");
    e.export_tensor(id, w, scales, biases);
    HB_CHECK(hipStreamSynchronize(e.stream()));
  });
}

namespace {
StepRows step_rows(int rows, const int32_t* row_tokens, const int32_t* positions, const int32_t* seq,
                   const int32_t* src_slot, const int32_t* dst_slot, const int32_t* hist_off,
                   const int32_t* log_count, const uint32_t* tokens) {
  require(rows > 0 && row_tokens && positions && seq && tokens, "step: null table");
  StepRows s;
  s.rows = rows;
  s.row_tokens.assign(row_tokens, row_tokens + rows);
  s.positions.assign(positions, positions + rows);
  s.seq.assign(seq, seq + rows);
  s.src_slot = src_slot ? std::vector<int32_t>(src_slot, src_slot + rows) : s.seq;
  s.dst_slot = dst_slot ? std::vector<int32_t>(dst_slot, dst_slot + rows) : s.seq;
  s.hist_off = hist_off ? std::vector<int32_t>(hist_off, hist_off + rows) : std::vector<int32_t>(rows, 0);
  s.log_count = log_count ? std::vector<int32_t>(log_count, log_count + rows) : std::vector<int32_t>(rows, 0);
  long total = 0;
  for (int r = 0; r < rows; ++r) {
    require(row_tokens[r] >= 0, "step: negative row token count");
    total += row_tokens[r];
  }
  require(total > 0 && total < (1l << 30), "step: token count");
  s.tokens.assign(tokens, tokens + total);
  return s;
}
}  // namespace

extern "C" int hb_engine_forward(void* engine, int rows, const int32_t* row_tokens, const int32_t* positions,
                                 const int32_t* seq, const int32_t* src_slot, const int32_t* dst_slot,
                                 const int32_t* hist_off, const int32_t* log_count, const uint32_t* tokens,
                                 int speculative, const int32_t* logit_rows, int n_logit_rows, char* error,
                                 size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && n_logit_rows >= 0 && (n_logit_rows == 0 || logit_rows), "hb_engine_forward: descriptor");
    auto& e = *static_cast<Engine*>(engine);
    const StepRows s = step_rows(rows, row_tokens, positions, seq, src_slot, dst_slot, hist_off, log_count, tokens);
    for (int i = 0; i < n_logit_rows; ++i)
      require(logit_rows[i] >= 0 && logit_rows[i] < s.total(), "hb_engine_forward: logit row outside the step");
    e.forward(s, speculative != 0, std::vector<int32_t>(logit_rows, logit_rows + n_logit_rows));
    HB_CHECK(hipStreamSynchronize(e.stream()));
  });
}

extern "C" int hb_engine_mtp_forward(void* engine, int rows, const int32_t* row_tokens, const int32_t* positions,
                                     const int32_t* seq, const uint32_t* tokens, int hidden_source,
                                     const int32_t* hidden_idx, const int32_t* logit_rows, int n_logit_rows,
                                     char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && hidden_idx && n_logit_rows >= 0 && (n_logit_rows == 0 || logit_rows) &&
                (hidden_source == 0 || hidden_source == 1),
            "hb_engine_mtp_forward: descriptor");
    auto& e = *static_cast<Engine*>(engine);
    const StepRows s = step_rows(rows, row_tokens, positions, seq, nullptr, nullptr, nullptr, nullptr, tokens);
    const int T = s.total();
    for (int i = 0; i < T; ++i)
      require(hidden_idx[i] >= 0 && hidden_idx[i] < e.max_step_tokens(), "hb_engine_mtp_forward: hidden row");
    for (int i = 0; i < n_logit_rows; ++i)
      require(logit_rows[i] >= 0 && logit_rows[i] < T, "hb_engine_mtp_forward: logit row outside the step");
    e.mtp_forward(s, hidden_source ? e.mtp_hidden_f32() : e.hidden_f32(), std::vector<int32_t>(hidden_idx, hidden_idx + T),
                  std::vector<int32_t>(logit_rows, logit_rows + n_logit_rows));
    HB_CHECK(hipStreamSynchronize(e.stream()));
  });
}

// which: 0 hidden f32 [T][H], 1 MTP hidden f32 [T][H], 2 logits f32 [n][V],
// 3 winners u32 [n], 4 margins f32 [n], 5 selection status i32 [n],
// 6 residual trace f32 [L+1][max_step_tokens][H]
extern "C" int hb_engine_read(void* engine, int which, size_t offset, void* out, size_t bytes, char* error,
                              size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && out, "hb_engine_read: descriptor");
    auto& e = *static_cast<Engine*>(engine);
    const Geom& g = e.geom();
    const size_t Tm = size_t(e.max_step_tokens());
    const void* src = nullptr;
    size_t limit = 0;
    switch (which) {
      case 0: src = e.hidden_f32(); limit = Tm * g.H * 4; break;
      case 1: src = e.mtp_hidden_f32(); limit = Tm * g.H * 4; break;
      case 2:
        require(e.logits_valid(),
                "hb_engine_read: the last vocabulary-head pass fused the selection and wrote no logits");
        src = e.logits();
        limit = Tm * g.V * 4;
        break;
      case 3: src = e.winners(); limit = Tm * 4; break;
      case 4: src = e.margins(); limit = Tm * 4; break;
      case 5: src = e.sel_status(); limit = Tm * 4; break;
      case 6:
        require(e.trace(), "hb_engine_read: tracing was never enabled");
        src = e.trace();
        limit = size_t(g.L + 1) * Tm * g.H * 4;
        break;
      case 7:
        require(e.mid_trace(), "hb_engine_read: tracing was never enabled");
        src = e.mid_trace();
        limit = size_t(g.L + 1) * Tm * g.H * 4;
        break;
      default: throw std::invalid_argument("hb_engine_read: unknown buffer");
    }
    require(offset <= limit && bytes <= limit - offset, "hb_engine_read: range outside the buffer");
    HB_CHECK(hipStreamSynchronize(e.stream()));
    if (which == 2) {  // rows of V logits out of the padded [n][vocab_rows] buffer
      const size_t row = size_t(g.V) * 4, pitch = size_t(g.vocab_rows()) * 4;
      require(offset % row == 0 && bytes % row == 0, "hb_engine_read: logits are read in whole rows");
      require((offset / row + bytes / row) * pitch <= size_t(Tm) * pitch, "hb_engine_read: range outside the buffer");
      HB_CHECK(hipMemcpy2D(out, row, static_cast<const char*>(src) + offset / row * pitch, pitch, row, bytes / row,
                           hipMemcpyDeviceToHost));
      return;
    }
    HB_CHECK(hipMemcpy(out, static_cast<const char*>(src) + offset, bytes, hipMemcpyDeviceToHost));
  });
}

extern "C" int hb_engine_profile(void* engine, int enable, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine, "hb_engine_profile: descriptor");
    static_cast<Engine*>(engine)->set_profile(enable);
  });
}

// out[0..4) = launches, summed milliseconds, summed tokens, summed routed experts touched
extern "C" int hb_engine_profile_read(void* engine, int kind, double* out, size_t count, char* error,
                                      size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && out && count >= 4, "hb_engine_profile_read: descriptor");
    const ProbeStats s = static_cast<Engine*>(engine)->profile_read(kind);
    out[0] = s.launches;
    out[1] = s.ms;
    out[2] = s.tokens;
    out[3] = s.active;
    if (count >= 5) out[4] = s.bytes;
  });
}

extern "C" int hb_engine_trace(void* engine, int enable, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine, "hb_engine_trace: descriptor");
    static_cast<Engine*>(engine)->set_trace(enable != 0);
  });
}

extern "C" int hb_engine_synthetic_context(void* engine, int rows, const int32_t* positions, uint64_t seed,
                                           char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(engine && positions, "hb_engine_synthetic_context: descriptor");
    static_cast<Engine*>(engine)->synthetic_context(rows, positions, seed);
  });
}

// ------------------------------------------------------------------ decode loop
extern "C" void* hb_decode_create(void* engine, int width, float gate_margin, const uint32_t* eos, int n_eos,
                                  char* error, size_t capacity) {
  DecodeLoop* d = nullptr;
  const int rc = guarded(error, capacity, [&] {
    require(engine && n_eos >= 0 && (n_eos == 0 || eos), "hb_decode_create: descriptor");
    d = new DecodeLoop(*static_cast<Engine*>(engine), width, gate_margin, std::vector<uint32_t>(eos, eos + n_eos));
  });
  return rc == 0 ? d : nullptr;
}

extern "C" void hb_decode_destroy(void* loop) { delete static_cast<DecodeLoop*>(loop); }

extern "C" int hb_decode_admit(void* loop, int seq, int position, uint32_t pending, int budget, int hist_off,
                               char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(loop, "hb_decode_admit: descriptor");
    static_cast<DecodeLoop*>(loop)->admit(seq, position, pending, budget, hist_off);
  });
}

extern "C" int hb_decode_set_drafts(void* loop, int seq, const uint32_t* tokens, int count, char* error,
                                    size_t capacity) {
  return guarded(error, capacity, [&] {
    require(loop, "hb_decode_set_drafts: descriptor");
    static_cast<DecodeLoop*>(loop)->set_drafts(seq, tokens, count);
  });
}

extern "C" int hb_decode_step(void* loop, int32_t* emitted, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(loop && emitted, "hb_decode_step: descriptor");
    const int n = static_cast<DecodeLoop*>(loop)->step();
    *emitted = n;
  });
}

// stats[0..9): steps, emitted, target tokens, proposed, accepted, MTP calls, MTP tokens, finished, live rows
extern "C" int hb_decode_stats(void* loop, uint64_t* stats, size_t count, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(loop && stats && count >= 9, "hb_decode_stats: descriptor");
    auto& d = *static_cast<DecodeLoop*>(loop);
    const DecodeStats& s = d.stats();
    const uint64_t v[9] = {s.steps,     s.emitted,    s.target_tokens, s.proposed,          s.accepted,
                           s.mtp_calls, s.mtp_tokens, s.finished,      uint64_t(d.live())};
    std::memcpy(stats, v, sizeof v);
  });
}

extern "C" int hb_decode_output(void* loop, int seq, uint32_t* tokens, size_t capacity_tokens, int32_t* count,
                                int32_t* position, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(loop && count, "hb_decode_output: descriptor");
    auto& d = *static_cast<DecodeLoop*>(loop);
    const auto& out = d.output(seq);
    require(!tokens || out.size() <= capacity_tokens, "hb_decode_output: capacity");
    if (tokens) std::copy(out.begin(), out.end(), tokens);
    *count = int32_t(out.size());
    if (position) *position = d.position(seq);
  });
}
