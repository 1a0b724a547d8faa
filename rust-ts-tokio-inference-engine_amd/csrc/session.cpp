// Device sessions over the decode engine (see session.h).
#include "session.h"

#include <algorithm>
#include <chrono>

namespace hb {

namespace {

constexpr size_t kStats = 17 + 19 * 3;  // native/qwen_device.inc:62; 19 operator stages

uint64_t now_ns() {
  return uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(
                      std::chrono::steady_clock::now().time_since_epoch())
                      .count());
}

bool same_id(const StateId& a, const StateId& b) {
  return a.owner == b.owner && a.slot == b.slot && a.generation == b.generation && a.position == b.position &&
         a.bytes == b.bytes;
}

}  // namespace

size_t reference_state_count(const rs_qwen_config& c) {
  const size_t full = size_t(c.layers / c.interval), linear = size_t(c.layers) - full;
  const size_t conv = size_t(c.conv - 1) * (2 * size_t(c.key_heads) * c.key_dim + size_t(c.value_heads) * c.value_dim);
  const size_t rec = size_t(c.value_heads) * c.value_dim * c.key_dim;
  return linear * (conv + rec) + full * 2 * size_t(c.kv_heads) * size_t(c.context) * c.head_dim;
}

// ------------------------------------------------------------------ session

DeviceSession::DeviceSession(const rs_qwen_config& c, size_t slots, uint64_t bytes, uint64_t owner, uint64_t seed,
                             std::shared_ptr<const NamedWeights> named)
    : c_(c),
      slots_(slots),
      limit_(bytes),
      row_cap_(c.chunk),
      table_(owner, slots, bytes),
      drafts_(owner + 1, slots, bytes),
      pages_(0, kPage) {
  require(c.group == 64 && c.bits == 4, "device session: the kernels take affine 4-bit group-64 weights");
  require(c.chunk >= 1 && c.chunk <= 64, "device session: chunk (tokens per row and step) outside 1..64");
  require(c.context >= 1 && c.context <= 262144, "device session: context outside 1..262144");
  eng_ = std::make_unique<Engine>(c, int(slots), c.context, row_cap_, int(slots) * row_cap_, seed, false,
                                  std::move(named));
  eng_->set_operator_profile(c.operator_profile != 0);
  pages_ = PagePool(eng_->page_count(), kPage);
  for (int r = int(slots) - 1; r >= 0; --r) free_rows_.push_back(r);
  for (int s = 2 * int(slots) - 1; s >= 0; --s) free_slots_.push_back(s);
  HB_CHECK(hipMalloc(reinterpret_cast<void**>(&hidden_pool_), slots * row_cap_ * size_t(c.hidden) * 4));
}

DeviceSession::~DeviceSession() {
  eng_.reset();  // drains the stream before anything is freed
  if (hidden_pool_) (void)hipFree(hidden_pool_);
  if (trace_buf_) (void)hipFree(trace_buf_);
}

uint64_t DeviceSession::charge(size_t tokens, bool hidden) const {
  return reference_state_count(c_) * 4 + (hidden ? tokens * size_t(c_.hidden) * 4 : 0);
}

void DeviceSession::check_budget(size_t add, uint64_t bytes) const {
  const size_t residents = table_.residents() + drafts_.residents();
  const uint64_t used = table_.bytes() + drafts_.bytes();
  if (residents + add > slots_ || bytes > limit_ - used) throw std::runtime_error("combined resident budget exhausted");
}

void DeviceSession::take_resources(Child& ch, bool target) {
  if (free_rows_.empty() || (target && free_slots_.empty())) throw std::runtime_error("session rows exhausted");
  ch.v.row = free_rows_.back();
  free_rows_.pop_back();
  if (target) {
    ch.v.slot = free_slots_.back();
    free_slots_.pop_back();
  }
  static const std::vector<int32_t> none;
  ch.plan = pages_.extend(ch.parent ? ch.parent->pages : none, ch.position, ch.tokens);
  ch.v.pages = ch.plan.pages;
}

void DeviceSession::free_version(const Version& v) {
  pages_.drop(v.pages);
  if (v.row >= 0) free_rows_.push_back(v.row);
  if (v.slot >= 0) free_slots_.push_back(v.slot);
}

void DeviceSession::abandon(std::vector<Child>& kids, bool drafts) {
  try {
    HB_CHECK(hipStreamSynchronize(eng_->stream()));
  } catch (...) {
  }
  for (Child& k : kids) {
    pages_.undo(k.plan);
    if (k.v.row >= 0) free_rows_.push_back(k.v.row);
    if (k.v.slot >= 0) free_slots_.push_back(k.v.slot);
    k.v = Version{};
    if (k.id.owner) (drafts ? drafts_ : table_).rollback(k.id);
  }
}

void DeviceSession::run_target(std::vector<Child>& kids, const std::vector<uint32_t>& tokens, bool all_rows,
                               float* trace) {
  StepRows s;
  s.rows = int(kids.size());
  std::vector<int32_t> pairs, logit_rows;
  int cu = 0;
  for (Child& k : kids) {
    s.row_tokens.push_back(k.tokens);
    s.positions.push_back(k.position);
    s.seq.push_back(k.v.row);
    s.src_slot.push_back(k.parent ? k.parent->slot : k.v.slot);
    s.dst_slot.push_back(k.v.slot);
    s.hist_off.push_back(k.parent ? k.parent->hist_off : 0);
    s.log_count.push_back(0);
    eng_->write_block_row(k.v.row, k.v.pages);
    pairs.insert(pairs.end(), k.plan.pairs.begin(), k.plan.pairs.end());
    if (all_rows)
      for (int j = 0; j < k.tokens; ++j) logit_rows.push_back(cu + j);
    else
      logit_rows.push_back(cu + k.tokens - 1);
    cu += k.tokens;
  }
  s.tokens = tokens;
  uploads_ += tokens.size() * 4 + size_t(s.rows) * 7 * 4;
  const uint64_t t0 = now_ns();
  ++calls_;
  eng_->copy_kv_pages(false, pairs);
  eng_->set_stage_trace(trace);
  try {
    eng_->forward(s, false, logit_rows);
  } catch (...) {
    eng_->set_stage_trace(nullptr);
    throw;
  }
  eng_->set_stage_trace(nullptr);
  const uint64_t t1 = now_ns();
  HB_CHECK(hipStreamSynchronize(eng_->stream()));
  const uint64_t t2 = now_ns();
  graph_ns_ += t1 - t0;
  wait_ns_ += t2 - t1;
  ++completed_;
  for (Child& k : kids) k.v.hist_off = k.tokens;
}

void DeviceSession::read_rows(int n, float* logits, uint32_t* winners, float* margins) {
  const uint64_t t0 = now_ns();
  std::vector<int32_t> status(n);
  // the finite check of the step's logits (the reference's StateValidation cut)
  eng_->op_begin();
  HB_CHECK(hipMemcpy(status.data(), eng_->sel_status(), size_t(n) * 4, hipMemcpyDeviceToHost));
  for (int32_t v : status)
    if (v) throw std::runtime_error("nonfinite logits");
  eng_->op_cut(OpStage::StateValidation);
  const int V = c_.vocab, Vp = eng_->geom().vocab_rows();
  if (logits) {
    HB_CHECK(hipMemcpy2D(logits, size_t(V) * 4, eng_->logits(), size_t(Vp) * 4, size_t(V) * 4, n,
                         hipMemcpyDeviceToHost));
    exports_ += size_t(n) * V * 4;
  }
  if (winners) HB_CHECK(hipMemcpy(winners, eng_->winners(), size_t(n) * 4, hipMemcpyDeviceToHost));
  if (margins) HB_CHECK(hipMemcpy(margins, eng_->margins(), size_t(n) * 4, hipMemcpyDeviceToHost));
  export_ns_ += now_ns() - t0;
}

void DeviceSession::keep_hidden(Child& ch, const float* src_rows) {
  const size_t H = size_t(c_.hidden);
  HB_CHECK(hipMemcpyAsync(hidden_pool_ + size_t(ch.v.row) * row_cap_ * H, src_rows, size_t(ch.tokens) * H * 4,
                          hipMemcpyDeviceToDevice, eng_->stream()));
  HB_CHECK(hipStreamSynchronize(eng_->stream()));
  ch.v.hidden_rows = ch.tokens;
}

StateId DeviceSession::step(const StateId* previous, size_t position, const uint32_t* tokens, size_t count,
                            float* logits, size_t logits_count, float* trace, size_t trace_count, bool all_logits,
                            bool hidden, uint32_t* sampled) {
  const rs_qwen_config& c = c_;
  const size_t V = size_t(c.vocab), H = size_t(c.hidden);
  require(tokens && (logits || sampled), "device step descriptor");
  if (!count || count > 8 || count > size_t(row_cap_) || position > size_t(c.context) ||
      count > size_t(c.context) - position || (sampled ? logits_count != 0 : logits_count != V * (all_logits ? count : 1)))
    throw std::invalid_argument("device step capacity");
  if ((position == 0) != (previous == nullptr)) throw std::invalid_argument("device previous state presence");
  for (size_t i = 0; i < count; ++i) require(tokens[i] < uint32_t(c.vocab), "token outside vocabulary");
  if (trace_count && (!trace || trace_count != size_t(c.layers) * 5 * count * H || sampled))
    throw std::invalid_argument("trace capacity");
  const Version* parent = nullptr;
  if (previous) {
    if (previous->position != position) throw std::invalid_argument("device position mismatch");
    parent = &table_.get(*previous);
  }
  const uint64_t bytes = charge(count, hidden);
  check_budget(1, bytes);
  if (trace_count && !trace_buf_)
    HB_CHECK(hipMalloc(reinterpret_cast<void**>(&trace_buf_), size_t(c.layers) * 5 * row_cap_ * H * 4));
  const uint64_t w0 = now_ns();
  std::vector<Child> kids(1);
  Child& k = kids[0];
  k.id = table_.reserve(position + count, bytes);
  k.parent = parent;
  k.tokens = int(count);
  k.position = int(position);
  try {
    take_resources(k, true);
    run_target(kids, std::vector<uint32_t>(tokens, tokens + count), all_logits, trace_count ? trace_buf_ : nullptr);
    const int n = all_logits ? int(count) : 1;
    std::vector<float> lg(sampled ? 0 : size_t(n) * V), tr(trace_count);
    uint32_t win = 0;
    read_rows(n, sampled ? nullptr : lg.data(), sampled ? &win : nullptr, nullptr);
    if (trace_count) HB_CHECK(hipMemcpy(tr.data(), trace_buf_, trace_count * 4, hipMemcpyDeviceToHost));
    if (hidden) keep_hidden(k, eng_->hidden_f32());
    const StateId id = k.id;
    table_.publish(id, std::move(k.v));
    ++steps_;
    if (sampled)
      *sampled = win;
    else
      std::copy(lg.begin(), lg.end(), logits);
    std::copy(tr.begin(), tr.end(), trace);
    wall_ns_ += now_ns() - w0;
    return id;
  } catch (...) {
    abandon(kids, false);
    throw;
  }
}

void DeviceSession::decode_batch(const StateId* parents, const uint32_t* tokens, size_t batch, StateId* outputs,
                                 float* logits, size_t logits_count) {
  const rs_qwen_config& c = c_;
  const size_t V = size_t(c.vocab);
  if (!parents || !tokens || !outputs || !logits || batch < 1 || batch > slots_)
    throw std::invalid_argument("batch descriptor");
  const size_t position = parents[0].position;
  if (!position || position >= size_t(c.context) || logits_count != batch * V)
    throw std::invalid_argument("batch geometry");
  std::vector<const Version*> old;
  for (size_t r = 0; r < batch; ++r) {
    if (parents[r].position != position || tokens[r] >= uint32_t(c.vocab))
      throw std::invalid_argument("batch parent/token geometry");
    old.push_back(&table_.get(parents[r]));
  }
  // each child is charged the whole batch's logical state (native/qwen_batch.inc:11)
  const uint64_t per = batch * reference_state_count(c) * 4;
  const size_t residents = table_.residents() + drafts_.residents();
  const uint64_t used = table_.bytes() + drafts_.bytes();
  if (residents + batch > slots_ || per > (limit_ - used) / batch)
    throw std::runtime_error("batch resident budget exhausted");
  const uint64_t w0 = now_ns();
  std::vector<Child> kids(batch);
  std::vector<float> lg(batch * V);
  try {
    for (size_t r = 0; r < batch; ++r) {
      kids[r].id = table_.reserve(position + 1, per);
      kids[r].parent = old[r];
      kids[r].tokens = 1;
      kids[r].position = int(position);
    }
    for (Child& k : kids) take_resources(k, true);
    run_target(kids, std::vector<uint32_t>(tokens, tokens + batch), false, nullptr);
    read_rows(int(batch), lg.data(), nullptr, nullptr);
  } catch (...) {
    abandon(kids, false);
    throw;
  }
  for (Child& k : kids) table_.publish(k.id, std::move(k.v));
  steps_ += batch;
  for (size_t r = 0; r < batch; ++r) outputs[r] = kids[r].id;
  std::copy(lg.begin(), lg.end(), logits);
  wall_ns_ += now_ns() - w0;
}

void DeviceSession::ragged(const StateId* parents, const uint32_t* row_tokens, size_t rows, const uint32_t* tokens,
                           size_t total, int flags, StateId* outputs, uint32_t* winners, float* margins,
                           float* logits, size_t logits_count) {
  const rs_qwen_config& c = c_;
  const size_t V = size_t(c.vocab);
  if (!parents || !row_tokens || !tokens || !outputs || !winners || rows < 1 || rows > slots_ || flags < 0 ||
      flags > 3)
    throw std::invalid_argument("ragged step descriptor");
  const bool per_token = flags & 1, hidden = flags & 2;
  size_t sum = 0;
  for (size_t r = 0; r < rows; ++r) {
    if (row_tokens[r] < 1 || row_tokens[r] > uint32_t(row_cap_)) throw std::invalid_argument("ragged row token count");
    sum += row_tokens[r];
  }
  const size_t n_out = per_token ? total : rows;
  if (sum != total || (logits ? logits_count != n_out * V : logits_count != 0))
    throw std::invalid_argument("ragged step capacity");
  for (size_t i = 0; i < total; ++i) require(tokens[i] < uint32_t(c.vocab), "token outside vocabulary");
  std::vector<const Version*> old(rows, nullptr);
  uint64_t bytes = 0;
  for (size_t r = 0; r < rows; ++r) {
    const size_t pos = parents[r].owner ? parents[r].position : 0;
    if (pos + row_tokens[r] > size_t(c.context)) throw std::invalid_argument("ragged context capacity");
    if (parents[r].owner) old[r] = &table_.get(parents[r]);
    for (size_t q = 0; q < r; ++q)
      if (parents[r].owner && same_id(parents[r], parents[q]))
        throw std::invalid_argument("ragged step: a parent appears twice (branch it in separate steps)");
    bytes += charge(row_tokens[r], hidden);
  }
  check_budget(rows, bytes);
  const uint64_t w0 = now_ns();
  std::vector<Child> kids(rows);
  std::vector<float> lg(logits ? n_out * V : 0), mar(n_out);
  std::vector<uint32_t> win(n_out);
  try {
    size_t cu = 0;
    for (size_t r = 0; r < rows; ++r) {
      Child& k = kids[r];
      k.position = int(parents[r].owner ? parents[r].position : 0);
      k.tokens = int(row_tokens[r]);
      k.parent = old[r];
      k.id = table_.reserve(size_t(k.position) + k.tokens, charge(k.tokens, hidden));
    }
    for (Child& k : kids) take_resources(k, true);
    // without a logits output the vocabulary head may fuse the selection
    eng_->set_logits_export(logits != nullptr);
    try {
      run_target(kids, std::vector<uint32_t>(tokens, tokens + total), per_token, nullptr);
    } catch (...) {
      eng_->set_logits_export(true);
      throw;
    }
    eng_->set_logits_export(true);
    read_rows(int(n_out), logits ? lg.data() : nullptr, win.data(), mar.data());
    if (hidden)
      for (Child& k : kids) {
        keep_hidden(k, eng_->hidden_f32() + cu * size_t(c.hidden));
        cu += k.tokens;
      }
  } catch (...) {
    abandon(kids, false);
    throw;
  }
  for (Child& k : kids) table_.publish(k.id, std::move(k.v));
  steps_ += rows;
  for (size_t r = 0; r < rows; ++r) outputs[r] = kids[r].id;
  std::copy(win.begin(), win.end(), winners);
  if (margins) std::copy(mar.begin(), mar.end(), margins);
  if (logits) std::copy(lg.begin(), lg.end(), logits);
  wall_ns_ += now_ns() - w0;
}

void DeviceSession::release(const StateId& id) {
  const Version v = table_.get(id);
  table_.release(id);
  free_version(v);
}

void DeviceSession::snapshot(const StateId& id, float* out, size_t count) {
  const Version& v = table_.get(id);
  const rs_qwen_config& c = c_;
  if (!out || count != reference_state_count(c)) throw std::invalid_argument("snapshot capacity");
  std::vector<float> host(count);
  const Geom& g = eng_->geom();
  const size_t conv = size_t(g.conv - 1) * g.conv_channels(), rec = size_t(g.Hv) * g.Dv * g.Dk,
               kv = size_t(g.Hkv) * c.context * g.D;
  size_t off = 0;
  int dn = 0, ai = 0;
  for (int l = 0; l < g.L; ++l) {
    if (g.attn(l)) {
      eng_->read_kv(ai++, v.pages, int(id.position), c.context, host.data() + off, host.data() + off + kv);
      off += 2 * kv;
    } else {
      eng_->read_recurrent(dn++, v.slot, v.hist_off, host.data() + off, host.data() + off + conv);
      off += conv + rec;
    }
  }
  if (off != count) throw std::runtime_error("snapshot accounting");
  std::copy(host.begin(), host.end(), out);
  exports_ += count * 4;
}

void DeviceSession::hidden_snapshot(const StateId& id, float* out, size_t count) {
  const Version& v = table_.get(id);
  const size_t H = size_t(c_.hidden);
  if (!out || !v.hidden_rows || count != size_t(v.hidden_rows) * H)
    throw std::invalid_argument("missing hidden or snapshot capacity");
  std::vector<float> host(count);
  HB_CHECK(hipMemcpy(host.data(), hidden_pool_ + size_t(v.row) * row_cap_ * H, count * 4, hipMemcpyDeviceToHost));
  std::copy(host.begin(), host.end(), out);
  exports_ += count * 4;
}

void DeviceSession::stats(uint64_t* out, size_t count) {
  if (!out || count != kStats) throw std::invalid_argument("stats capacity");
  size_t free_b = 0, total_b = 0;
  HB_CHECK(hipMemGetInfo(&free_b, &total_b));
  const uint64_t active = total_b - free_b;
  peak_ = std::max(peak_, active);
  std::fill(out, out + count, uint64_t(0));
  out[0] = table_.residents() + drafts_.residents();
  out[1] = table_.bytes() + drafts_.bytes();
  out[2] = exports_;
  out[3] = uploads_;
  out[4] = steps_;
  out[5] = active;  // device bytes in use (every allocation on the device)
  out[6] = peak_;
  out[7] = calls_;
  out[8] = completed_;
  out[9] = graph_ns_;
  out[10] = wait_ns_;
  out[11] = export_ns_;
  out[12] = wall_ns_;
  out[13] = completed_;  // one evaluation group per forward
  // [14..16] compiled graph entries / misses / calls: none; [17..] operator
  // stages (calls, host ns, wait ns), zero unless the session was created
  // with the operator profile
  const auto& ops = eng_->operator_metrics();
  for (int i = 0; i < kOpStages; ++i) {
    out[17 + 3 * i] = ops[i].calls;
    out[18 + 3 * i] = ops[i].host_ns;
    out[19 + 3 * i] = ops[i].wait_ns;
  }
}

uint64_t DeviceSession::drain() {
  const uint64_t invalidated = table_.residents() + drafts_.residents();
  HB_CHECK(hipStreamSynchronize(eng_->stream()));
  table_.for_each([&](const Version& v) { free_version(v); });
  drafts_.for_each([&](const Version& v) { free_version(v); });
  table_.clear();
  drafts_.clear();
  if (table_.residents() || table_.bytes() || drafts_.residents() || drafts_.bytes())
    throw std::runtime_error("device drain residual");
  return invalidated;
}

StateId DeviceSession::import(size_t position, const float* state, size_t count) {
  const rs_qwen_config& c = c_;
  if (!state || count != reference_state_count(c)) throw std::invalid_argument("model state length");
  if (!position || position > size_t(c.context)) throw std::invalid_argument("model state position");
  const uint64_t bytes = charge(0, false);
  check_budget(1, bytes);
  std::vector<Child> kids(1);
  Child& k = kids[0];
  k.id = table_.reserve(position, bytes);
  k.position = 0;
  k.tokens = int(position);
  try {
    take_resources(k, true);
    eng_->write_block_row(k.v.row, k.v.pages);
    const Geom& g = eng_->geom();
    const size_t conv = size_t(g.conv - 1) * g.conv_channels(), rec = size_t(g.Hv) * g.Dv * g.Dk,
                 kv = size_t(g.Hkv) * c.context * g.D;
    size_t off = 0;
    int dn = 0, ai = 0;
    for (int l = 0; l < g.L; ++l) {
      if (g.attn(l)) {
        eng_->write_kv(ai++, k.v.pages, int(position), c.context, state + off, state + off + kv);
        off += 2 * kv;
      } else {
        eng_->write_recurrent(dn++, k.v.slot, state + off, state + off + conv);
        off += conv + rec;
      }
    }
    k.v.hist_off = 0;
    uploads_ += count * 4;
  } catch (...) {
    abandon(kids, false);
    throw;
  }
  const StateId id = k.id;
  table_.publish(id, std::move(k.v));
  return id;
}

void DeviceSession::mtp_attach(std::shared_ptr<const NamedWeights> named_mtp) {
  if (mtp_ || table_.residents() || drafts_.residents())
    throw std::invalid_argument("MTP attach must precede admission");
  eng_->enable_mtp(std::move(named_mtp));
  mtp_ = true;
}

StateId DeviceSession::mtp_step(const StateId* previous, const StateId& source, int draft_source, size_t row,
                                const uint32_t* tokens, size_t count, float* logits, size_t logits_count) {
  const rs_qwen_config& c = c_;
  const size_t V = size_t(c.vocab), H = size_t(c.hidden);
  if (!tokens || !logits || draft_source < 0 || draft_source > 1 || !count || count > 8 || count > size_t(row_cap_))
    throw std::invalid_argument("MTP descriptor");
  if (!mtp_ || logits_count != V) throw std::invalid_argument("MTP unavailable or vocabulary capacity");
  const size_t position = previous ? previous->position : 0;
  if (position > size_t(c.context) || count > size_t(c.context) - position)
    throw std::invalid_argument("MTP context capacity");
  for (size_t i = 0; i < count; ++i)
    if (tokens[i] >= uint32_t(c.vocab)) throw std::invalid_argument("MTP token vocabulary");
  const Version* old = previous ? &drafts_.get(*previous) : nullptr;
  const Version& input = draft_source ? drafts_.get(source) : table_.get(source);
  if (!input.hidden_rows) throw std::invalid_argument("MTP hidden source");
  const size_t rows = size_t(input.hidden_rows);
  if (row > rows || count > rows - row) throw std::invalid_argument("MTP hidden row capacity");
  if (draft_source) {
    if (!previous || !same_id(*previous, source) || count != 1 || row + 1 != rows)
      throw std::invalid_argument("MTP autoregressive parent identity");
  } else if (source.position < rows || source.position - rows + row != position) {
    throw std::invalid_argument("MTP target hidden alignment");
  }
  const Geom& g = eng_->geom();
  const uint64_t bytes = uint64_t(c.context) * 2 * g.Hkv * g.D * 4 + count * H * 4;
  check_budget(1, bytes);
  const uint64_t w0 = now_ns();
  std::vector<Child> kids(1);
  Child& k = kids[0];
  k.id = drafts_.reserve(position + count, bytes);
  k.parent = old;
  k.tokens = int(count);
  k.position = int(position);
  std::vector<float> lg(V);
  try {
    take_resources(k, false);
    eng_->write_block_row(k.v.row, k.v.pages);
    eng_->copy_kv_pages(true, k.plan.pairs);
    StepRows s;
    s.rows = 1;
    s.row_tokens = {int(count)};
    s.positions = {int(position)};
    s.seq = {k.v.row};
    s.src_slot = {0};
    s.dst_slot = {0};
    s.hist_off = {0};
    s.log_count = {0};
    s.tokens.assign(tokens, tokens + count);
    std::vector<int32_t> idx(count);
    for (size_t i = 0; i < count; ++i) idx[i] = int32_t(size_t(input.row) * row_cap_ + row + i);
    const uint64_t t0 = now_ns();
    ++calls_;
    eng_->mtp_forward(s, hidden_pool_, idx, {int(count) - 1});
    const uint64_t t1 = now_ns();
    HB_CHECK(hipStreamSynchronize(eng_->stream()));
    graph_ns_ += t1 - t0;
    wait_ns_ += now_ns() - t1;
    ++completed_;
    read_rows(1, lg.data(), nullptr, nullptr);
    keep_hidden(k, eng_->mtp_hidden_f32());
  } catch (...) {
    abandon(kids, true);
    throw;
  }
  const StateId id = k.id;
  drafts_.publish(id, std::move(k.v));
  std::copy(lg.begin(), lg.end(), logits);
  wall_ns_ += now_ns() - w0;
  return id;
}

void DeviceSession::mtp_release(const StateId& id) {
  const Version v = drafts_.get(id);
  drafts_.release(id);
  free_version(v);
}

void DeviceSession::mtp_snapshot(const StateId& id, float* out, size_t count) {
  const Version& v = drafts_.get(id);
  const Geom& g = eng_->geom();
  const size_t kv = size_t(g.Hkv) * c_.context * g.D, H = size_t(c_.hidden);
  if (!out || count != id.bytes / 4 || count != 2 * kv + size_t(v.hidden_rows) * H)
    throw std::invalid_argument("MTP snapshot capacity");
  std::vector<float> host(count);
  eng_->read_kv(eng_->attn_layers(), v.pages, int(id.position), c_.context, host.data(), host.data() + kv);
  HB_CHECK(hipMemcpy(host.data() + 2 * kv, hidden_pool_ + size_t(v.row) * row_cap_ * H, size_t(v.hidden_rows) * H * 4,
                     hipMemcpyDeviceToHost));
  std::copy(host.begin(), host.end(), out);
  exports_ += count * 4;
}

}  // namespace hb
