// Device sessions: immutable, generation-checked state versions over the
// decode engine (DeviceSession / device_step / the batched packer / the MTP
// operator, native/qwen_device.inc:5-75, native/qwen_batch.inc:2-50,
// native/qwen_mtp.inc:2-63).
//
// A version is not a copy of the state. It owns a recurrent slot (per
// DeltaNet layer: fp32 state and conv history), a page list into the paged
// KV pools and optionally hidden rows. A child step reads its parent's slot
// and writes its own, so the parent never changes; KV pages are shared with
// the parent copy-on-write (see PagePool).
#pragma once
#include <memory>
#include <vector>

#include "engine.h"
#include "page_pool.h"
#include "state_table.h"

namespace hb {

// Reference state length in floats (qwen_state_count, native/qwen_model.inc:268-271):
// fixed-capacity, independent of the position.
size_t reference_state_count(const rs_qwen_config& c);

struct Version {
  int row = -1;          // block-table row, and row block of the hidden pool
  int slot = -1;         // recurrent slot (target versions only)
  int hist_off = 0;      // window row where the committed conv history starts
  int hidden_rows = 0;   // f32 rows kept in the hidden pool (0 = none)
  std::vector<int32_t> pages;
};

class DeviceSession {
 public:
  // slots and bytes: the combined resident budget of both tables
  // (native/qwen_device.inc:31-33). The engine holds the seeded synthetic model.
  // A checkpoint store passes its tensors as `named` (the seed is then unused).
  DeviceSession(const rs_qwen_config& c, size_t slots, uint64_t bytes, uint64_t owner, uint64_t seed,
                std::shared_ptr<const NamedWeights> named = nullptr);
  ~DeviceSession();

  const rs_qwen_config& config() const { return c_; }
  Engine& engine() { return *eng_; }
  int max_row_tokens() const { return row_cap_; }

  // device_step (native/qwen_device.inc:40-49): one row, count <= 8 tokens.
  StateId step(const StateId* previous, size_t position, const uint32_t* tokens, size_t count, float* logits,
               size_t logits_count, float* trace, size_t trace_count, bool all_logits, bool hidden,
               uint32_t* sampled);
  // Equal-position one-token rows in one packed forward (native/qwen_batch.inc:2-50).
  void decode_batch(const StateId* parents, const uint32_t* tokens, size_t batch, StateId* outputs, float* logits,
                    size_t logits_count);
  // Ragged rows: any parents and positions, row_tokens[r] tokens each.
  // flags: 1 = per-token results (else the last token of each row), 2 = keep hidden rows.
  void ragged(const StateId* parents, const uint32_t* row_tokens, size_t rows, const uint32_t* tokens,
              size_t total, int flags, StateId* outputs, uint32_t* winners, float* margins, float* logits,
              size_t logits_count);
  void release(const StateId& id);
  void snapshot(const StateId& id, float* out, size_t count);
  void hidden_snapshot(const StateId& id, float* out, size_t count);
  void stats(uint64_t* out, size_t count);
  uint64_t drain();
  // Import of a full reference-layout state as a published root version (the
  // stateless rs_qwen_forward path).
  StateId import(size_t position, const float* state, size_t count);

  void mtp_attach(std::shared_ptr<const NamedWeights> named_mtp = nullptr);
  StateId mtp_step(const StateId* previous, const StateId& source, int draft_source, size_t row,
                   const uint32_t* tokens, size_t count, float* logits, size_t logits_count);
  void mtp_release(const StateId& id);
  void mtp_snapshot(const StateId& id, float* out, size_t count);

 private:
  struct Child {
    StateId id{};
    Version v;
    PagePool::Plan plan;
    const Version* parent = nullptr;
    int tokens = 0, position = 0;
  };
  void check_budget(size_t add, uint64_t bytes) const;
  void take_resources(Child& ch, bool target);
  void free_version(const Version& v);
  void abandon(std::vector<Child>& kids, bool drafts);
  void run_target(std::vector<Child>& kids, const std::vector<uint32_t>& tokens, bool all_rows, float* trace);
  void read_rows(int n, float* logits, uint32_t* winners, float* margins);
  void keep_hidden(Child& ch, const float* src_rows);
  uint64_t charge(size_t tokens, bool hidden) const;

  rs_qwen_config c_;
  std::unique_ptr<Engine> eng_;
  size_t slots_;
  uint64_t limit_;
  int row_cap_;
  VersionTable<Version> table_, drafts_;
  PagePool pages_;
  std::vector<int> free_rows_, free_slots_;
  float* hidden_pool_ = nullptr;  // device f32 [slots][row_cap][H]
  float* trace_buf_ = nullptr;    // device f32 [L][5][row_cap][H], on demand
  bool mtp_ = false;
  // counters (stats layout, native/qwen_device.inc:62)
  uint64_t exports_ = 0, uploads_ = 0, steps_ = 0, calls_ = 0, completed_ = 0, graph_ns_ = 0, wait_ns_ = 0,
           export_ns_ = 0, wall_ns_ = 0, peak_ = 0;
};

}  // namespace hb
