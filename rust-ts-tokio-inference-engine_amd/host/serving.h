// Host layer over the C ABI of include/hip_bridge.h: the part of the
// reference's Rust serving crate that drives device sessions, restated in C++
// for a host without Rust (the Rust caller binds the same symbols through
// `extern "C"` blocks, src/serving/native_device.rs:1087-1207).
//
//   StepIr / select / winner_with_margin  model_ir.rs:28-61, choices.rs:65-79,
//                                         native_speculative.rs:45-73
//   PreparedBatch / CompletedBatch        batch_transaction.rs:67-252: row and
//       resident bounds, cohorts of equal (kind, position, tokens) geometry in
//       first-appearance order, results restored to input order, an atomic
//       commit (a failed row publishes nothing and releases every provisional
//       state)
//   Device                                native_device.rs:820-1086: the
//       step/block/sampled/decode_batch calls with their receipt checks and
//       validate_batch, plus the ragged extension (one packed forward for rows
//       of any position and block length)
//   ScheduledDevice                       native_device_scheduler.rs:147-199:
//       the packed predicate (several decode rows at one position > 0 share
//       one decode_batch) or, in ragged mode, one ragged step per batch
//   mtp_transaction                       judges/native_cpp_bench.cpp:87-132
//
// Errors are exceptions (Failure); every published StateId is owned by a
// Lifetime and released exactly once, when its last holder drops it.
#pragma once
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

#include "../../include/hip_bridge.h"

namespace hbhost {

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};
inline void ensure(bool ok, const std::string& what) {
  if (!ok) throw Failure(what);
}

enum class StepKind { Prefill, Decode };

// A validated step: 1..max_tokens tokens below the vocabulary, one for a
// decode step, ending within the context (model_ir.rs:28-61; the reference
// bounds are 8 tokens and context 512).
struct StepIr {
  StepKind kind = StepKind::Decode;
  size_t position = 0;
  std::vector<uint32_t> tokens;
  static StepIr compile(StepKind kind, size_t position, std::vector<uint32_t> tokens, uint32_t vocabulary,
                        size_t max_tokens = 8, size_t context = 512);
  size_t len() const { return tokens.size(); }
};

// Greedy choice, lowest index on ties under the f32 total order; with a mask,
// the best allowed id (choices.rs:65-79). Non-finite logits fail.
uint32_t select(const float* logits, size_t n, const std::vector<uint32_t>* allowed);
// (winner, top1 - top2) with +inf for a single value (native_speculative.rs:45-73).
std::pair<uint32_t, float> winner_with_margin(const float* logits, size_t n);

struct StepInput {
  uint64_t sequence = 0;
  size_t position = 0;
  StepKind kind = StepKind::Decode;
  std::vector<uint32_t> tokens;
  size_t remaining_output_tokens = 1;
  bool prompt_complete = true;
  std::optional<std::vector<uint32_t>> allowed_tokens;
};

struct StepOutput {
  uint64_t sequence = 0;
  std::optional<uint32_t> next_token;
  uint64_t state_bytes = 0;
};

struct Cohort {
  StepKind kind;
  size_t position, tokens;
  std::vector<size_t> rows;  // input indices
};

// A row's result: its new state and either logits or a device-selected token.
template <class P>
struct RowResult {
  P state;
  std::variant<std::vector<float>, uint32_t> selection;
};

template <class P>
class CompletedBatch {
 public:
  CompletedBatch(std::map<uint64_t, P>* committed, std::vector<std::pair<uint64_t, P>> states,
                 std::vector<StepOutput> outputs)
      : committed_(committed), states_(std::move(states)), outputs_(std::move(outputs)) {}
  // Publishes every row's state at once; nothing fallible happens here.
  std::vector<StepOutput> commit() && {
    for (auto& [id, s] : states_) (*committed_)[id] = std::move(s);
    return std::move(outputs_);
  }

 private:
  std::map<uint64_t, P>* committed_;
  std::vector<std::pair<uint64_t, P>> states_;
  std::vector<StepOutput> outputs_;
};

template <class P>
class PreparedBatch {
 public:
  // batch_transaction.rs:67-134. `row_bound` is the reference's 3 for its
  // physical batches; the ragged path raises it to the session's slots.
  static PreparedBatch prepare(std::vector<StepInput> batch, std::map<uint64_t, P>& committed,
                               const std::function<P()>& empty, uint32_t vocabulary, size_t row_bound = 3,
                               size_t max_tokens = 8, size_t context = 512) {
    ensure(!batch.empty() && batch.size() <= row_bound, "batch row bound");
    size_t fresh = 0;
    for (const auto& r : batch) fresh += committed.count(r.sequence) ? 0 : 1;
    ensure(committed.size() + fresh <= row_bound, "batch resident bound");
    PreparedBatch p(committed, vocabulary);
    std::vector<uint64_t> seen;
    for (auto& item : batch) {
      ensure(std::find(seen.begin(), seen.end(), item.sequence) == seen.end(), "batch duplicate/history");
      seen.push_back(item.sequence);
      ensure(item.remaining_output_tokens >= 1 && item.remaining_output_tokens <= 128, "batch output bound");
      auto it = committed.find(item.sequence);
      P parent = it != committed.end() ? it->second : empty();
      ensure(parent.position() == item.position, "batch parent position");
      if (item.allowed_tokens) {
        const auto& m = *item.allowed_tokens;
        ensure(!m.empty() && m.size() <= 32 &&
                   std::all_of(m.begin(), m.end(), [&](uint32_t t) { return t < vocabulary; }),
               "batch token mask");
      }
      StepIr ir = StepIr::compile(item.kind, item.position, std::move(item.tokens), vocabulary, max_tokens, context);
      const size_t index = p.rows_.size();
      auto g = std::find_if(p.cohorts_.begin(), p.cohorts_.end(), [&](const Cohort& c) {
        return c.kind == ir.kind && c.position == ir.position && c.tokens == ir.len();
      });
      if (g != p.cohorts_.end())
        g->rows.push_back(index);
      else
        p.cohorts_.push_back(Cohort{ir.kind, ir.position, ir.len(), {index}});
      p.rows_.push_back(Row{item.sequence, std::move(parent), std::move(ir), item.prompt_complete,
                            std::move(item.allowed_tokens)});
    }
    return p;
  }

  const std::vector<Cohort>& cohorts() const { return cohorts_; }
  std::vector<uint64_t> sequences() const {
    std::vector<uint64_t> s;
    for (const auto& r : rows_) s.push_back(r.sequence);
    return s;
  }

  // One executor call per cohort; it returns that cohort's results in order
  // (batch_transaction.rs:140-174).
  template <class F>
  CompletedBatch<P> execute_grouped(F&& executor) && {
    std::vector<Row> rows = take();
    std::vector<std::optional<RowResult<P>>> results(rows.size());
    for (const Cohort& c : cohorts_) {
      std::vector<std::pair<P, StepIr>> inputs;
      for (size_t i : c.rows) inputs.emplace_back(rows[i].parent, rows[i].ir);
      std::vector<RowResult<P>> out = executor(std::move(inputs));
      ensure(out.size() == c.rows.size(), "batch cohort cardinality");
      for (size_t j = 0; j < c.rows.size(); ++j) results[c.rows[j]] = std::move(out[j]);
    }
    return finish(std::move(rows), std::move(results));
  }

  // One executor call for every row at once, in input order (the ragged
  // extension: one packed forward whatever the rows' geometries).
  template <class F>
  CompletedBatch<P> execute_packed(F&& executor) && {
    std::vector<Row> rows = take();
    std::vector<std::pair<P, StepIr>> inputs;
    std::vector<bool> unconstrained;
    for (const Row& r : rows) {
      inputs.emplace_back(r.parent, r.ir);
      unconstrained.push_back(!r.allowed);
    }
    std::vector<RowResult<P>> out = executor(std::move(inputs), unconstrained);
    ensure(out.size() == rows.size(), "batch cohort cardinality");
    std::vector<std::optional<RowResult<P>>> results;
    for (auto& o : out) results.emplace_back(std::move(o));
    return finish(std::move(rows), std::move(results));
  }

  // One executor call per row, in input order; the flag allows a
  // device-selected token when the row has no mask (batch_transaction.rs:177-235).
  template <class F>
  CompletedBatch<P> execute_receipts(F&& executor) && {
    std::vector<Row> rows = take();
    std::vector<std::optional<RowResult<P>>> results;
    for (const Row& r : rows) results.emplace_back(executor(r.parent, r.ir, !r.allowed));
    return finish(std::move(rows), std::move(results));
  }

 private:
  struct Row {
    uint64_t sequence;
    P parent;
    StepIr ir;
    bool complete;
    std::optional<std::vector<uint32_t>> allowed;
  };
  PreparedBatch(std::map<uint64_t, P>& committed, uint32_t vocabulary)
      : committed_(&committed), vocabulary_(vocabulary) {}

  // Executing consumes the batch, as Rust's `execute(self)` does: the rows
  // (and the parent copies they hold) leave this object, so a failure drops
  // them together with every staged result.
  std::vector<Row> take() { return std::move(rows_); }

  // The receipt checks of every row, then the staged outputs
  // (batch_transaction.rs:186-235). Any failure drops every staged state.
  CompletedBatch<P> finish(std::vector<Row> rows, std::vector<std::optional<RowResult<P>>> results) {
    std::vector<std::pair<uint64_t, P>> states;
    std::vector<StepOutput> outputs;
    for (size_t i = 0; i < rows.size(); ++i) {
      ensure(results[i].has_value(), "batch missing row");
      RowResult<P>& res = *results[i];
      const Row& row = rows[i];
      ensure(res.state.position() == row.ir.position + row.ir.len(), "batch result position");
      std::optional<uint32_t> next;
      if (auto* logits = std::get_if<std::vector<float>>(&res.selection)) {
        ensure(logits->size() == vocabulary_, "batch result logits");
        if (row.complete) {
          next = select(logits->data(), logits->size(), row.allowed ? &*row.allowed : nullptr);
        } else {
          for (float v : *logits) ensure(std::isfinite(v), "batch result logits");
        }
      } else {
        const uint32_t token = std::get<uint32_t>(res.selection);
        ensure(!row.allowed && token < vocabulary_, "invalid device-selected token");
        if (row.complete) next = token;
      }
      outputs.push_back(StepOutput{row.sequence, next, uint64_t(res.state.bytes())});
      states.emplace_back(row.sequence, std::move(res.state));
    }
    return CompletedBatch<P>(committed_, std::move(states), std::move(outputs));
  }

  std::map<uint64_t, P>* committed_;
  uint32_t vocabulary_;
  std::vector<Row> rows_;
  std::vector<Cohort> cohorts_;
};

// ------------------------------------------------------------------ device
// Ownership of one published StateId: released (target or draft table) when
// the last holder drops it (native_device.rs:13-22 Lifetime).
struct Lifetime {
  void* session;
  StateId id;
  bool draft;
  Lifetime(void* s, StateId i, bool d) : session(s), id(i), draft(d) {}
  Lifetime(const Lifetime&) = delete;
  Lifetime& operator=(const Lifetime&) = delete;
  ~Lifetime();
  void detach() { session = nullptr; }  // ownership passed on: never released here
};

struct DeviceState {
  uint64_t owner = 0;       // the executor that produced it
  size_t hidden_rows = 0;   // hidden rows kept for the MTP head
  std::shared_ptr<Lifetime> token;  // empty: a fresh sequence at position 0
  size_t position() const { return token ? size_t(token->id.position) : 0; }
  size_t bytes() const { return token ? size_t(token->id.bytes) : 0; }
  const StateId* id() const { return token ? &token->id : nullptr; }
};

// Rust's Architecture::state_len: the fixed-capacity recurrent + KV floats of
// one version, independent of its position (native_qwen.rs:196-204).
size_t state_len(const rs_qwen_config& c);
// Bytes of an MTP draft version holding `rows` hidden rows: the draft layer's
// KV at full context plus the rows (native_mtp_device.rs:45-48 at this geometry).
size_t mtp_state_bytes(const rs_qwen_config& c, size_t rows);

class Device {
 public:
  Device(void* session, const rs_qwen_config& c);
  const rs_qwen_config& config() const { return c_; }
  uint64_t owner() const { return owner_; }
  void* session() const { return session_; }
  DeviceState empty() const { return DeviceState{owner_, 0, nullptr}; }

  struct Step {
    DeviceState state;
    std::vector<float> logits;
  };
  // device_forward: step (last-token logits), block (every token's logits),
  // with or without hidden rows, then the receipt checks.
  Step execute(const DeviceState& parent, const StepIr& ir, bool all_logits = false, bool hidden = false) const;
  // device_forward_sampled: the greedy token chosen on the device.
  std::pair<DeviceState, uint32_t> execute_sampled(const DeviceState& parent, const StepIr& ir) const;
  // validate_batch + batch_forward (native_device.rs:959-1086).
  std::vector<Step> decode_batch(const std::vector<DeviceState>& parents, const std::vector<uint32_t>& tokens) const;
  // The ragged step: rows with their own parents, positions and blocks.
  struct RaggedRow {
    DeviceState state;
    std::vector<uint32_t> winners;  // one per token (all_tokens) or the last token
    std::vector<float> margins;
    std::vector<float> logits;      // same rows, when requested
  };
  std::vector<RaggedRow> ragged(const std::vector<DeviceState>& parents, const std::vector<std::vector<uint32_t>>& blocks,
                                bool all_tokens, bool with_logits) const;
  // validate_batch (native_device.rs:959-979) with the row bound as a parameter.
  void validate_batch(const std::vector<DeviceState>& parents, const std::vector<uint32_t>& tokens,
                      size_t row_bound = 3) const;

 private:
  void* session_;
  rs_qwen_config c_;
  uint64_t owner_;
};

// validate_batch on bare (owner, position) pairs, for host-only checks.
void validate_batch_geometry(uint64_t owner, const std::vector<std::pair<uint64_t, size_t>>& parents,
                             const std::vector<uint32_t>& tokens, uint32_t vocabulary, size_t context,
                             size_t row_bound = 3);

class ScheduledDevice {
 public:
  enum class Packing { Scalar, Physical, Ragged };
  ScheduledDevice(const Device& device, Packing packing, size_t row_bound = 3)
      : dev_(device), packing_(packing), row_bound_(row_bound) {}
  // One scheduler step over a batch of sequences (native_device_scheduler.rs:103-199).
  std::vector<StepOutput> step(std::vector<StepInput> batch);
  struct Counters {
    uint64_t packed_calls = 0, packed_rows = 0, scalar_calls = 0, ragged_calls = 0, ragged_rows = 0;
  };
  const Counters& counters() const { return counters_; }
  std::map<uint64_t, DeviceState>& states() { return states_; }

 private:
  const Device& dev_;
  Packing packing_;
  size_t row_bound_;
  Counters counters_;
  std::map<uint64_t, DeviceState> states_;
};

// ------------------------------------------------------------------ MTP
struct MtpResult {
  StateId target_state{}, draft_state{};
  std::vector<uint32_t> emitted;
  uint32_t learned_proposed = 0, learned_accepted = 0, target_calls = 0, draft_calls = 0, reused_target_tokens = 0,
           replayed_target_tokens = 0, target_forward_tokens = 0;
  bool terminal = false;
};
// One speculative transaction over the public ABI (judges/native_cpp_bench.cpp:
// 87-132): margin-gated MTP drafts from the draft state, one hidden_block
// verify from the target parent, greedy acceptance, reuse of the verified
// block on a full accept or a hidden_step replay of the emitted prefix, then
// the MTP refresh over the committed positions. target_logits/draft_logits
// receive the committed target's last logits and the refreshed draft logits.
// The caller owns both returned states.
MtpResult mtp_transaction(const Device& dev, const StateId& target_previous, const StateId& draft_previous,
                          uint32_t seed, uint32_t first, float first_margin, size_t width, size_t budget,
                          const std::vector<uint32_t>& eos, float gate, std::vector<float>& target_logits,
                          std::vector<float>& draft_logits);

}  // namespace hbhost
