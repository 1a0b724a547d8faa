// Host layer over the C ABI: device executor with its receipt checks, the
// scheduler step and the MTP transaction (declarations and reference
// citations in serving.h).
#include "serving.h"

#include <atomic>
#include <cstring>
#include <limits>

namespace hbhost {
namespace {

// Every native call passes a zeroed 1024-byte buffer and turns -1 into the
// message it holds (native_device.rs:136, native_status).
struct Err {
  char text[1024] = {};
};
void native(int rc, const Err& e, const char* call) {
  if (rc != 0) throw Failure(std::string(call) + ": " + e.text);
}

// Owners of the host executors (distinct from the session's table owners).
uint64_t next_owner() {
  static std::atomic<uint64_t> next{1};
  return next.fetch_add(1);
}

// f32 total order key: -0 below +0, larger values larger keys.
int32_t total_key(float v) {
  int32_t i;
  std::memcpy(&i, &v, 4);
  return i < 0 ? int32_t(uint32_t(i) ^ 0x7fffffffu) : i;
}

bool all_finite(const std::vector<float>& v) {
  return std::all_of(v.begin(), v.end(), [](float x) { return std::isfinite(x); });
}

}  // namespace

StepIr StepIr::compile(StepKind kind, size_t position, std::vector<uint32_t> tokens, uint32_t vocabulary,
                       size_t max_tokens, size_t context) {
  ensure(vocabulary > 0 && vocabulary <= 300000 && !tokens.empty() && tokens.size() <= max_tokens &&
             std::all_of(tokens.begin(), tokens.end(), [&](uint32_t t) { return t < vocabulary; }),
         "IR token geometry");
  ensure(kind != StepKind::Decode || tokens.size() == 1, "decode IR requires one token");
  ensure(position <= context && tokens.size() <= context - position, "IR context bound");
  return StepIr{kind, position, std::move(tokens)};
}

uint32_t select(const float* logits, size_t n, const std::vector<uint32_t>* allowed) {
  ensure(n > 0, "invalid logits");
  for (size_t i = 0; i < n; ++i) ensure(std::isfinite(logits[i]), "invalid logits");
  if (!allowed) {
    uint32_t best = 0;
    for (size_t i = 1; i < n; ++i)
      if (total_key(logits[i]) > total_key(logits[best])) best = uint32_t(i);
    return best;
  }
  std::optional<uint32_t> win;
  for (uint32_t id : *allowed) {
    ensure(id < n, "invalid legal token");
    if (!win || total_key(logits[id]) > total_key(logits[*win]) ||
        (total_key(logits[id]) == total_key(logits[*win]) && id < *win))
      win = id;
  }
  ensure(win.has_value(), "empty legal token set");
  return *win;
}

std::pair<uint32_t, float> winner_with_margin(const float* logits, size_t n) {
  ensure(n > 0 && n <= 300000 && std::isfinite(logits[0]), "greedy logits finite/shape");
  uint32_t best = 0;
  float best_val = logits[0], second = -std::numeric_limits<float>::infinity();
  for (size_t i = 1; i < n; ++i) {
    const float v = logits[i];
    ensure(std::isfinite(v), "greedy logits finite/shape");
    if (total_key(v) > total_key(best_val)) {
      second = best_val;
      best = uint32_t(i);
      best_val = v;
    } else if (total_key(v) > total_key(second)) {
      second = v;
    }
  }
  return {best, std::isfinite(second) ? best_val - second : std::numeric_limits<float>::infinity()};
}

Lifetime::~Lifetime() {
  if (!session) return;
  Err e;
  if (draft)
    (void)rs_qwen_device_mtp_release(session, &id, e.text, sizeof e.text);
  else
    (void)rs_qwen_device_release(session, &id, e.text, sizeof e.text);
}

size_t state_len(const rs_qwen_config& c) {
  const size_t full = size_t(c.layers / c.interval), linear = size_t(c.layers) - full;
  return linear * (size_t(c.conv - 1) * size_t(2 * c.key_heads * c.key_dim + c.value_heads * c.value_dim) +
                   size_t(c.value_heads) * c.value_dim * c.key_dim) +
         full * 2 * size_t(c.kv_heads) * size_t(c.context) * c.head_dim;
}

size_t mtp_state_bytes(const rs_qwen_config& c, size_t rows) {
  return size_t(c.context) * 2 * c.kv_heads * c.head_dim * 4 + rows * size_t(c.hidden) * 4;
}

Device::Device(void* session, const rs_qwen_config& c) : session_(session), c_(c), owner_(next_owner()) {
  ensure(session != nullptr, "device session handle");
}

Device::Step Device::execute(const DeviceState& parent, const StepIr& ir, bool all_logits, bool hidden) const {
  ensure(parent.owner == owner_, "foreign device state");
  const size_t rows = all_logits ? ir.len() : 1;
  std::vector<float> logits(rows * size_t(c_.vocab));
  StateId id{};
  Err e;
  const StateId* prev = parent.id();
  int rc;
  if (hidden)
    rc = all_logits ? rs_qwen_device_hidden_block(session_, prev, parent.position(), ir.tokens.data(), ir.len(), &id,
                                                  logits.data(), logits.size(), e.text, sizeof e.text)
                    : rs_qwen_device_hidden_step(session_, prev, parent.position(), ir.tokens.data(), ir.len(), &id,
                                                 logits.data(), logits.size(), e.text, sizeof e.text);
  else
    rc = all_logits ? rs_qwen_device_block(session_, prev, parent.position(), ir.tokens.data(), ir.len(), &id,
                                           logits.data(), logits.size(), e.text, sizeof e.text)
                    : rs_qwen_device_step(session_, prev, parent.position(), ir.tokens.data(), ir.len(), &id,
                                          logits.data(), logits.size(), nullptr, 0, e.text, sizeof e.text);
  native(rc, e, "device step");
  // own the child before any fallible receipt check
  DeviceState next{owner_, hidden ? ir.len() : 0, std::make_shared<Lifetime>(session_, id, false)};
  ensure(id.position == parent.position() + ir.len() &&
             id.bytes == (state_len(c_) + (hidden ? ir.len() * size_t(c_.hidden) : 0)) * 4 && all_finite(logits),
         "invalid device receipt");
  return Step{std::move(next), std::move(logits)};
}

std::pair<DeviceState, uint32_t> Device::execute_sampled(const DeviceState& parent, const StepIr& ir) const {
  ensure(parent.owner == owner_, "foreign device state");
  StateId id{};
  uint32_t token = 0;
  Err e;
  native(rs_qwen_device_step_sampled(session_, parent.id(), parent.position(), ir.tokens.data(), ir.len(), &id, &token,
                                     e.text, sizeof e.text),
         e, "device sampled step");
  DeviceState next{owner_, 0, std::make_shared<Lifetime>(session_, id, false)};
  ensure(id.position == parent.position() + ir.len() && id.bytes == state_len(c_) * 4 &&
             token < uint32_t(c_.vocab),
         "invalid device sampled receipt");
  return {std::move(next), token};
}

void validate_batch_geometry(uint64_t owner, const std::vector<std::pair<uint64_t, size_t>>& parents,
                             const std::vector<uint32_t>& tokens, uint32_t vocabulary, size_t context,
                             size_t row_bound) {
  ensure(!parents.empty() && parents.size() <= row_bound && parents.size() == tokens.size(), "batch row geometry");
  const size_t position = parents[0].second;
  ensure(position >= 1 && position < context, "batch decode position");
  for (size_t i = 0; i < parents.size(); ++i)
    ensure(parents[i].first == owner && parents[i].second == position && tokens[i] < vocabulary,
           "batch parent owner/token geometry");
}

void Device::validate_batch(const std::vector<DeviceState>& parents, const std::vector<uint32_t>& tokens,
                            size_t row_bound) const {
  std::vector<std::pair<uint64_t, size_t>> g;
  for (const auto& p : parents) g.emplace_back(p.owner, p.position());
  validate_batch_geometry(owner_, g, tokens, uint32_t(c_.vocab), size_t(c_.context), row_bound);
}

std::vector<Device::Step> Device::decode_batch(const std::vector<DeviceState>& parents,
                                               const std::vector<uint32_t>& tokens) const {
  validate_batch(parents, tokens);
  std::vector<StateId> old;
  for (const auto& p : parents) {
    ensure(p.id() != nullptr, "batch parent without a published state");
    old.push_back(*p.id());
  }
  std::vector<StateId> ids(parents.size());
  std::vector<float> logits(parents.size() * size_t(c_.vocab));
  Err e;
  native(rs_qwen_device_decode_batch(session_, old.data(), tokens.data(), parents.size(), ids.data(), logits.data(),
                                     logits.size(), e.text, sizeof e.text),
         e, "decode batch");
  std::vector<Step> out;
  for (const StateId& id : ids) out.push_back(Step{DeviceState{owner_, 0, std::make_shared<Lifetime>(session_, id, false)}, {}});
  const size_t position = parents[0].position() + 1;
  for (const StateId& id : ids)
    ensure(id.position == position && id.bytes == parents.size() * state_len(c_) * 4, "invalid batch receipt");
  ensure(all_finite(logits), "invalid batch receipt");
  for (size_t r = 0; r < out.size(); ++r)
    out[r].logits.assign(logits.begin() + r * size_t(c_.vocab), logits.begin() + (r + 1) * size_t(c_.vocab));
  return out;
}

std::vector<Device::RaggedRow> Device::ragged(const std::vector<DeviceState>& parents,
                                              const std::vector<std::vector<uint32_t>>& blocks, bool all_tokens,
                                              bool with_logits) const {
  ensure(!parents.empty() && parents.size() == blocks.size(), "ragged row geometry");
  std::vector<StateId> old;
  std::vector<uint32_t> row_tokens, tokens;
  for (size_t r = 0; r < parents.size(); ++r) {
    ensure(parents[r].owner == owner_, "foreign device state");
    old.push_back(parents[r].id() ? *parents[r].id() : StateId{0, 0, 0, 0, 0});
    row_tokens.push_back(uint32_t(blocks[r].size()));
    tokens.insert(tokens.end(), blocks[r].begin(), blocks[r].end());
  }
  const size_t n_out = all_tokens ? tokens.size() : parents.size();
  std::vector<StateId> ids(parents.size());
  std::vector<uint32_t> winners(n_out);
  std::vector<float> margins(n_out), logits(with_logits ? n_out * size_t(c_.vocab) : 0);
  Err e;
  native(rs_qwen_device_ragged_step(session_, old.data(), row_tokens.data(), parents.size(), tokens.data(),
                                    tokens.size(), all_tokens ? 1 : 0, ids.data(), winners.data(), margins.data(),
                                    with_logits ? logits.data() : nullptr, logits.size(), e.text, sizeof e.text),
         e, "ragged step");
  std::vector<RaggedRow> out;
  for (const StateId& id : ids)
    out.push_back(RaggedRow{DeviceState{owner_, 0, std::make_shared<Lifetime>(session_, id, false)}, {}, {}, {}});
  size_t k = 0;
  for (size_t r = 0; r < parents.size(); ++r) {
    const StateId& id = ids[r];
    ensure(id.position == parents[r].position() + blocks[r].size() && id.bytes == state_len(c_) * 4,
           "invalid ragged receipt");
    const size_t n = all_tokens ? blocks[r].size() : 1;
    out[r].winners.assign(winners.begin() + k, winners.begin() + k + n);
    out[r].margins.assign(margins.begin() + k, margins.begin() + k + n);
    for (uint32_t w : out[r].winners) ensure(w < uint32_t(c_.vocab), "invalid ragged receipt");
    if (with_logits)
      out[r].logits.assign(logits.begin() + k * size_t(c_.vocab), logits.begin() + (k + n) * size_t(c_.vocab));
    k += n;
  }
  ensure(all_finite(logits), "invalid ragged receipt");
  return out;
}

std::vector<StepOutput> ScheduledDevice::step(std::vector<StepInput> batch) {
  const Device& dev = dev_;
  const uint32_t V = uint32_t(dev.config().vocab);
  const size_t T = packing_ == Packing::Ragged ? size_t(dev.config().chunk) : 8;
  auto prepared = PreparedBatch<DeviceState>::prepare(std::move(batch), states_, [&] { return dev.empty(); }, V,
                                                      row_bound_, T, size_t(dev.config().context));
  if (packing_ == Packing::Ragged) {
    Counters& cnt = counters_;
    auto completed = std::move(prepared).execute_packed(
        [&](std::vector<std::pair<DeviceState, StepIr>> rows, const std::vector<bool>& unconstrained) {
          const bool masked = std::find(unconstrained.begin(), unconstrained.end(), false) != unconstrained.end();
          std::vector<DeviceState> parents;
          std::vector<std::vector<uint32_t>> blocks;
          for (auto& [s, ir] : rows) {
            parents.push_back(s);
            blocks.push_back(ir.tokens);
          }
          auto res = dev.ragged(parents, blocks, false, masked);
          cnt.ragged_calls += 1;
          cnt.ragged_rows += res.size();
          std::vector<RowResult<DeviceState>> out;
          for (size_t r = 0; r < res.size(); ++r) {
            if (unconstrained[r])
              out.push_back(RowResult<DeviceState>{std::move(res[r].state), res[r].winners[0]});
            else
              out.push_back(RowResult<DeviceState>{std::move(res[r].state), std::move(res[r].logits)});
          }
          return out;
        });
    return std::move(completed).commit();
  }
  const bool physical = packing_ == Packing::Physical;
  Counters& cnt = counters_;
  auto completed = std::move(prepared).execute_grouped([&](std::vector<std::pair<DeviceState, StepIr>> rows) {
    std::vector<RowResult<DeviceState>> out;
    const bool packed = physical && rows.size() > 1 && rows[0].second.kind == StepKind::Decode &&
                        rows[0].second.position > 0;
    if (packed) {
      std::vector<DeviceState> parents;
      std::vector<uint32_t> tokens;
      for (auto& [s, ir] : rows) {
        parents.push_back(s);
        tokens.push_back(ir.tokens[0]);
      }
      auto res = dev.decode_batch(parents, tokens);
      cnt.packed_calls += 1;
      cnt.packed_rows += res.size();
      for (auto& r : res) out.push_back(RowResult<DeviceState>{std::move(r.state), std::move(r.logits)});
    } else {
      for (auto& [s, ir] : rows) {
        auto r = dev.execute(s, ir);
        cnt.scalar_calls += 1;
        out.push_back(RowResult<DeviceState>{std::move(r.state), std::move(r.logits)});
      }
    }
    return out;
  });
  return std::move(completed).commit();
}

MtpResult mtp_transaction(const Device& dev, const StateId& target_previous, const StateId& draft_previous,
                          uint32_t seed, uint32_t first, float first_margin, size_t width, size_t budget,
                          const std::vector<uint32_t>& eos, float gate, std::vector<float>& target_logits,
                          std::vector<float>& draft_logits) {
  const rs_qwen_config& c = dev.config();
  void* s = dev.session();
  const size_t V = size_t(c.vocab), context = size_t(c.context);
  ensure(target_previous.position == draft_previous.position && target_previous.position < context &&
             target_logits.size() == V && draft_logits.size() == V,
         "transaction descriptor");
  auto is_eos = [&](uint32_t t) { return std::find(eos.begin(), eos.end(), t) != eos.end(); };
  const size_t count = std::min({width, budget, context - size_t(target_previous.position)});
  ensure(count >= 1 && count <= 8, "transaction width");
  const size_t kv_bytes = mtp_state_bytes(c, 0);
  // drafts: the first learned draft always, deeper ones while the margins pass the gate
  std::shared_ptr<Lifetime> branch;
  std::vector<uint32_t> proposed{seed};
  std::vector<float> scores(V);
  uint32_t next = first;
  float confidence = first_margin;
  uint32_t draft_calls = 0;
  while (proposed.size() < count && !is_eos(proposed.back())) {
    if (proposed.size() >= 2 && confidence < gate) break;
    proposed.push_back(next);
    if (proposed.size() < count && !is_eos(next) && confidence >= gate) {
      const StateId& parent = branch ? branch->id : draft_previous;
      ensure(parent.bytes >= kv_bytes, "draft bytes");
      const size_t rows = (parent.bytes - kv_bytes) / (size_t(c.hidden) * 4);
      ensure(rows >= 1 && rows <= 64 && parent.bytes == mtp_state_bytes(c, rows), "draft hidden rows");
      StateId updated{};
      Err e;
      native(rs_qwen_device_mtp_step(s, &parent, &parent, 1, rows - 1, &next, 1, &updated, scores.data(), V, 0, e.text,
                                     sizeof e.text),
             e, "MTP draft step");
      branch = std::make_shared<Lifetime>(s, updated, true);
      std::tie(next, confidence) = winner_with_margin(scores.data(), V);
      ++draft_calls;
    } else {
      break;
    }
  }
  branch.reset();
  // verify the block from the target parent
  std::vector<float> block(V * proposed.size());
  StateId block_id{};
  {
    Err e;
    native(rs_qwen_device_hidden_block(s, &target_previous, size_t(target_previous.position), proposed.data(),
                                       proposed.size(), &block_id, block.data(), block.size(), e.text, sizeof e.text),
           e, "verify block");
  }
  auto verified = std::make_shared<Lifetime>(s, block_id, false);
  std::vector<uint32_t> row_winners;
  for (size_t i = 0; i < proposed.size(); ++i) row_winners.push_back(winner_with_margin(block.data() + i * V, V).first);
  std::vector<uint32_t> emitted;
  size_t accepted = 0;
  bool terminal = false;
  for (size_t i = 0; i < proposed.size(); ++i) {
    const uint32_t authoritative = i == 0 ? seed : row_winners[i - 1];
    emitted.push_back(authoritative);
    terminal = is_eos(authoritative);
    if (proposed[i] != authoritative || terminal) {
      accepted += proposed[i] == authoritative;
      break;
    }
    ++accepted;
  }
  ensure(!emitted.empty() && emitted.size() <= budget, "committed output");
  // commit: reuse the verified block on a full accept, else replay the emitted prefix
  std::shared_ptr<Lifetime> committed;
  uint32_t target_calls = 1;
  const bool reusable = accepted == proposed.size();
  if (reusable) {
    std::copy_n(block.data() + (proposed.size() - 1) * V, V, target_logits.data());
    committed = verified;
  } else {
    verified.reset();
    StateId replay{};
    Err e;
    native(rs_qwen_device_hidden_step(s, &target_previous, size_t(target_previous.position), emitted.data(),
                                      emitted.size(), &replay, target_logits.data(), V, e.text, sizeof e.text),
           e, "replay step");
    committed = std::make_shared<Lifetime>(s, replay, false);
    ++target_calls;
  }
  // refresh the draft head over the committed positions
  std::vector<uint32_t> shifted(emitted.begin() + 1, emitted.end());
  shifted.push_back(winner_with_margin(target_logits.data(), V).first);
  StateId next_draft{};
  {
    Err e;
    native(rs_qwen_device_mtp_step(s, &draft_previous, &committed->id, 0, 0, shifted.data(), shifted.size(),
                                   &next_draft, draft_logits.data(), V, 0, e.text, sizeof e.text),
           e, "MTP refresh");
  }
  ++draft_calls;
  MtpResult r;
  r.target_state = committed->id;
  r.draft_state = next_draft;
  r.emitted = emitted;
  r.learned_proposed = uint32_t(proposed.size() - 1);
  r.learned_accepted = uint32_t(accepted ? accepted - 1 : 0);
  r.target_calls = target_calls;
  r.draft_calls = draft_calls;
  r.target_forward_tokens = uint32_t(proposed.size() + (reusable ? 0 : emitted.size()));
  r.terminal = terminal;
  r.reused_target_tokens = reusable ? uint32_t(proposed.size()) : 0;
  r.replayed_target_tokens = reusable ? 0 : uint32_t(emitted.size());
  committed->detach();  // the caller owns both published states
  return r;
}

}  // namespace hbhost
