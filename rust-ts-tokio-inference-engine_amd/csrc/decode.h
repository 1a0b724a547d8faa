// Continuous-batching greedy decode with MTP speculation over the Engine.
//
// Per step every live row feeds the block [pending, d1..dn] (pending = the
// last emitted token, not yet in the target state; d = drafts) through one
// packed target forward. Device selection and the acceptance plan
// (src/serving/native_speculative.rs:74-128) then emit t_0..t_m, where t_i
// is the target's greedy token after block input i. The accepted prefix
// [pending, d1..d_m] is committed by the recurrent log and the conv history
// offset (no second target pass), t_m becomes the new pending token, and the
// MTP head is refreshed over the committed positions with the target's
// hidden rows; deeper drafts are margin-gated autoregressive MTP steps
// (src/serving/native_mtp_decode.rs:124-295, gate 1.25).
//
// The reference replays the emitted tokens through the target when a draft
// is rejected, and verifies a block whose first token is the target's known
// next token. Here the last emitted token opens the next block instead, so
// each step costs one target forward. Greedy decoding is lossless, so the
// emitted stream is the target's greedy stream either way.
#pragma once
#include <cstdint>
#include <vector>

#include "engine.h"

namespace hb {

struct DecodeStats {
  uint64_t steps = 0, emitted = 0, target_tokens = 0, proposed = 0, accepted = 0, mtp_calls = 0, mtp_tokens = 0,
           finished = 0;
};

class DecodeLoop {
 public:
  // width = block width (1 disables drafting; k drafts -> width k+1, at most 9).
  DecodeLoop(Engine& engine, int width, float gate_margin, std::vector<uint32_t> eos);
  ~DecodeLoop();
  DecodeLoop(const DecodeLoop&) = delete;
  DecodeLoop& operator=(const DecodeLoop&) = delete;

  // A sequence whose first `position` tokens are in the target state (and,
  // with MTP, in the draft KV); `pending` is its last emitted token and
  // `hist_off` the row count of the last forward that wrote its conv window
  // (the prefill chunk length; 0 for a synthetic context).
  void admit(int seq, int position, uint32_t pending, int budget, int hist_off);
  // Overrides the drafts of a row for its next step (external drafter).
  void set_drafts(int seq, const uint32_t* tokens, int n);
  // One decode step over all live rows; returns the tokens emitted.
  int step();
  int live() const;
  const DecodeStats& stats() const { return stats_; }
  // Tokens emitted so far by the sequence in `seq` (pending included last).
  const std::vector<uint32_t>& output(int seq) const;
  int position(int seq) const;

 private:
  struct Row {
    bool used = false, done = true;
    int position = 0, budget = 0, emitted = 0, hist_off = 0, log_count = 0;
    uint32_t pending = 0;
    std::vector<uint32_t> drafts, out;
    bool external = false;
  };
  void refresh_and_draft(const std::vector<int>& live, const std::vector<int>& cu, const std::vector<int>& commit);
  Row& row(int seq);

  Engine& e_;
  int width_;
  float gate_;
  std::vector<uint32_t> eos_;
  std::vector<Row> rows_;
  DecodeStats stats_;
  // device plan buffers
  uint32_t *d_draft_ = nullptr, *d_target_ = nullptr, *d_eos_ = nullptr, *d_emitted_ = nullptr;
  int32_t *d_ndraft_ = nullptr, *d_remaining_ = nullptr, *d_tidx_ = nullptr, *d_nemit_ = nullptr,
          *d_accepted_ = nullptr, *d_terminal_ = nullptr, *d_status_ = nullptr;
  int32_t *d_in_ = nullptr, *d_out_ = nullptr;  // the blocks the pointers above live in
  size_t in_n_ = 0, out_n_ = 0;
  int32_t* h_ = nullptr;  // pinned staging: [in | out | selection block]
  size_t h_cap_ = 0;
};

}  // namespace hb
