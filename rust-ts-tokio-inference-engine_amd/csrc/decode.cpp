// Continuous-batching greedy decode with MTP speculation (see decode.h).
#include "decode.h"

#include <algorithm>

#include "norm.h"
#include "select.h"

namespace hb {

namespace {
constexpr int kMaxEos = 16;
}

DecodeLoop::DecodeLoop(Engine& engine, int width, float gate_margin, std::vector<uint32_t> eos)
    : e_(engine), width_(width), gate_(gate_margin), eos_(std::move(eos)) {
  require(width >= 1 && width <= 9, "decode: block width must be in 1..9");
  require(int(eos_.size()) <= kMaxEos, "decode: at most 16 EOS tokens");
  for (uint32_t t : eos_) require(t < uint32_t(engine.geom().V), "decode: EOS outside the vocabulary");
  const int R = engine.max_rows(), md = std::max(width - 1, 1);
  rows_.resize(R);
  auto alloc = [](size_t bytes) {
    void* p = nullptr;
    HB_CHECK(hipMalloc(&p, std::max<size_t>(bytes, 4)));
    return p;
  };
  // plan inputs and outputs are single blocks with fixed regions (capacity R),
  // so each crosses the bus in one copy:
  //   in  = [drafts R*md | n_draft R | remaining R | target index R*(md+1)]
  //   out = [emitted R*(md+1) | n_emitted R | accepted R | terminal R | status R]
  in_n_ = size_t(R) * md + 2 * size_t(R) + size_t(R) * (md + 1);
  out_n_ = size_t(R) * (md + 1) + 4 * size_t(R);
  d_in_ = static_cast<int32_t*>(alloc(in_n_ * 4));
  d_out_ = static_cast<int32_t*>(alloc(out_n_ * 4));
  d_draft_ = reinterpret_cast<uint32_t*>(d_in_);
  d_ndraft_ = d_in_ + size_t(R) * md;
  d_remaining_ = d_ndraft_ + R;
  d_tidx_ = d_remaining_ + R;
  d_emitted_ = reinterpret_cast<uint32_t*>(d_out_);
  d_nemit_ = d_out_ + size_t(R) * (md + 1);
  d_accepted_ = d_nemit_ + R;
  d_terminal_ = d_accepted_ + R;
  d_status_ = d_terminal_ + R;
  d_target_ = static_cast<uint32_t*>(alloc(size_t(R) * (md + 1) * 4));
  d_eos_ = static_cast<uint32_t*>(alloc(kMaxEos * 4));
  if (!eos_.empty()) HB_CHECK(hipMemcpy(d_eos_, eos_.data(), eos_.size() * 4, hipMemcpyHostToDevice));
  // host staging: [in | out | selection block (3 * max_step_tokens)]
  h_cap_ = in_n_ + out_n_ + size_t(3) * e_.max_step_tokens() + 64;
  HB_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_), h_cap_ * 4, hipHostMallocDefault));
}

DecodeLoop::~DecodeLoop() {
  (void)hipStreamSynchronize(e_.stream());
  for (void* p : {static_cast<void*>(d_in_), static_cast<void*>(d_out_), static_cast<void*>(d_target_),
                  static_cast<void*>(d_eos_)})
    (void)hipFree(p);
  if (h_) (void)hipHostFree(h_);
}

DecodeLoop::Row& DecodeLoop::row(int seq) {
  require(seq >= 0 && seq < int(rows_.size()), "decode: sequence slot out of range");
  return rows_[seq];
}

void DecodeLoop::admit(int seq, int position, uint32_t pending, int budget, int hist_off) {
  Row& r = row(seq);
  require(!r.used || r.done, "decode: sequence slot is live");
  require(position >= 0 && position < e_.max_context(), "decode: position outside the context");
  require(budget > 0, "decode: budget must be positive");
  require(pending < uint32_t(e_.geom().V), "decode: pending token outside the vocabulary");
  require(hist_off >= 0 && hist_off <= e_.max_row_tokens() && hist_off <= position, "decode: history offset");
  r = Row{};
  r.hist_off = hist_off;
  r.used = true;
  r.done = std::find(eos_.begin(), eos_.end(), pending) != eos_.end();
  r.position = position;
  r.pending = pending;
  r.budget = budget;
  r.out.push_back(pending);
}

void DecodeLoop::set_drafts(int seq, const uint32_t* tokens, int n) {
  Row& r = row(seq);
  require(r.used && !r.done, "decode: drafts for a row that is not live");
  require(n >= 0 && n <= width_ - 1 && (n == 0 || tokens), "decode: draft count exceeds the block width");
  for (int i = 0; i < n; ++i) require(tokens[i] < uint32_t(e_.geom().V), "decode: draft outside the vocabulary");
  r.drafts.assign(tokens, tokens + n);
  r.external = true;
}

int DecodeLoop::live() const {
  int n = 0;
  for (const Row& r : rows_) n += r.used && !r.done;
  return n;
}

const std::vector<uint32_t>& DecodeLoop::output(int seq) const {
  require(seq >= 0 && seq < int(rows_.size()) && rows_[seq].used, "decode: unknown sequence slot");
  return rows_[seq].out;
}

int DecodeLoop::position(int seq) const {
  require(seq >= 0 && seq < int(rows_.size()) && rows_[seq].used, "decode: unknown sequence slot");
  return rows_[seq].position;
}

int DecodeLoop::step() {
  const int md = std::max(width_ - 1, 1);
  std::vector<int> live;
  for (int s = 0; s < int(rows_.size()); ++s)
    if (rows_[s].used && !rows_[s].done) live.push_back(s);
  if (live.empty()) return 0;
  const int B = int(live.size());

  StepRows sr;
  sr.rows = B;
  std::vector<int32_t> logit_rows;
  std::vector<int> cu(B + 1, 0);
  for (int i = 0; i < B; ++i) {
    Row& r = rows_[live[i]];
    const int remaining = r.budget - r.emitted;
    const int ctx_room = e_.max_context() - r.position - 1;
    const int n = std::min<int>({int(r.drafts.size()), remaining, ctx_room, e_.max_row_tokens() - 1});
    r.drafts.resize(std::max(n, 0));
    const int len = 1 + int(r.drafts.size());
    require(ctx_room >= 0, "decode: context exhausted");
    sr.row_tokens.push_back(len);
    sr.positions.push_back(r.position);
    sr.seq.push_back(live[i]);
    sr.src_slot.push_back(live[i]);
    sr.dst_slot.push_back(live[i]);
    sr.hist_off.push_back(r.hist_off);
    sr.log_count.push_back(r.log_count);
    sr.tokens.push_back(r.pending);
    for (uint32_t d : r.drafts) sr.tokens.push_back(d);
    cu[i + 1] = cu[i] + len;
  }
  const int T = cu[B];
  require(T <= e_.max_step_tokens(), "decode: step exceeds the packed token capacity");
  for (int t = 0; t < T; ++t) logit_rows.push_back(t);

  // plan inputs: drafts, counts, budgets and the packed index of each target winner
  HB_CHECK(hipStreamSynchronize(e_.stream()));
  const int R = e_.max_rows();
  uint32_t* hd = reinterpret_cast<uint32_t*>(h_);
  int32_t* hn = h_ + size_t(R) * md;
  int32_t* hrem = hn + R;
  int32_t* hti = hrem + R;
  for (int i = 0; i < B; ++i) {
    const Row& r = rows_[live[i]];
    const int n = int(r.drafts.size());
    for (int j = 0; j < md; ++j) hd[size_t(i) * md + j] = j < n ? r.drafts[j] : 0u;
    hn[i] = n;
    hrem[i] = r.budget - r.emitted;
    for (int j = 0; j <= md; ++j) hti[size_t(i) * (md + 1) + j] = cu[i] + std::min(j, n);
  }
  hipStream_t st = e_.stream();
  HB_CHECK(hipMemcpyAsync(d_in_, h_, in_n_ * 4, hipMemcpyHostToDevice, st));

  e_.set_logits_export(false);  // the loop reads only the selection
  try {
    e_.forward(sr, true, logit_rows);
  } catch (...) {
    e_.set_logits_export(true);
    throw;
  }
  e_.set_logits_export(true);
  gather_rows_i32(reinterpret_cast<const int32_t*>(e_.winners()), 1, d_tidx_, B * (md + 1), 1,
                  reinterpret_cast<int32_t*>(d_target_), 1, st);
  mtp_plan(d_draft_, d_ndraft_, md, d_target_, d_eos_, int(eos_.size()), d_remaining_, B, e_.geom().V, d_emitted_,
           d_nemit_, d_accepted_, d_terminal_, d_status_, st);
  // results: emitted [B][md+1], n_emitted, accepted, terminal, plan status, selection status [T]
  int32_t* o = h_ + in_n_;
  int32_t* o_emit = o;
  int32_t* o_n = o_emit + size_t(R) * (md + 1);
  int32_t* o_acc = o_n + R;
  int32_t* o_term = o_acc + R;
  int32_t* o_st = o_term + R;
  int32_t* o_sel = o + out_n_;
  HB_CHECK(hipMemcpyAsync(o, d_out_, out_n_ * 4, hipMemcpyDeviceToHost, st));
  HB_CHECK(hipMemcpyAsync(o_sel, e_.sel_status(), size_t(T) * 4, hipMemcpyDeviceToHost, st));
  HB_CHECK(hipStreamSynchronize(st));
  for (int t = 0; t < T; ++t) require(o_sel[t] == 0, "decode: nonfinite target logits");
  for (int i = 0; i < B; ++i) require(o_st[i] == 0, "decode: malformed acceptance row");

  int total = 0;
  std::vector<int> commit(B);
  for (int i = 0; i < B; ++i) {
    Row& r = rows_[live[i]];
    const int m = o_n[i];
    require(m >= 1 && m <= int(r.drafts.size()) + 1, "decode: acceptance emitted an invalid count");
    const uint32_t* em = reinterpret_cast<const uint32_t*>(o_emit) + size_t(i) * (md + 1);
    stats_.proposed += r.drafts.size();
    stats_.accepted += o_acc[i];
    // inputs [pending, d1..d_{m-1}] are consistent with the emitted prefix: commit them
    commit[i] = m;
    r.position += m;
    r.hist_off = m;
    r.log_count = m;
    r.emitted += m;
    for (int j = 0; j < m; ++j) r.out.push_back(em[j]);
    r.pending = em[m - 1];
    r.drafts.clear();
    r.external = false;
    if (o_term[i] || r.emitted >= r.budget || r.position >= e_.max_context()) {
      r.done = true;
      ++stats_.finished;
    }
    total += m;
  }
  stats_.steps += 1;
  stats_.emitted += total;
  stats_.target_tokens += T;
  if (width_ > 1 && e_.has_mtp()) refresh_and_draft(live, cu, commit);
  return total;
}

// MTP refresh over the committed positions (pairs of the target's hidden row
// at position q and the token at q+1), then margin-gated autoregressive drafts
// (native_mtp_decode.rs:145-170: the first learned draft is always proposed,
// a deeper one only when the previous and its own top-1/top-2 margins reach
// the gate).
void DecodeLoop::refresh_and_draft(const std::vector<int>& live, const std::vector<int>& cu,
                                   const std::vector<int>& commit) {
  hipStream_t st = e_.stream();
  StepRows sr;
  std::vector<int32_t> hidden_idx, logit_rows;
  std::vector<int> who;
  for (size_t i = 0; i < live.size(); ++i) {
    const int s = live[i];
    const Row& r = rows_[s];
    if (r.done) continue;
    const int m = commit[i];
    sr.row_tokens.push_back(m);
    sr.positions.push_back(r.position - m);
    sr.seq.push_back(s);
    sr.src_slot.push_back(s);
    sr.dst_slot.push_back(s);
    sr.hist_off.push_back(0);
    sr.log_count.push_back(0);
    for (int j = 0; j < m; ++j) {
      sr.tokens.push_back(r.out[r.out.size() - m + j]);
      hidden_idx.push_back(cu[i] + j);
    }
    logit_rows.push_back(int32_t(sr.tokens.size()) - 1);
    who.push_back(s);
  }
  if (who.empty()) return;
  sr.rows = int(who.size());
  const int n = int(who.size());
  std::vector<float> margin(n);
  std::vector<int32_t> prev = logit_rows;  // MTP hidden row of each live draft chain
  auto run = [&](const StepRows& step, const float* hidden, const std::vector<int32_t>& idx,
                 const std::vector<int32_t>& rows_out, std::vector<uint32_t>& tok, std::vector<float>& marg) {
    e_.set_logits_export(false);
    try {
      e_.mtp_forward(step, hidden, idx, rows_out);
    } catch (...) {
      e_.set_logits_export(true);
      throw;
    }
    e_.set_logits_export(true);
    // winners, margins and status are consecutive regions of Tm entries: one copy
    const int k = int(rows_out.size());
    const size_t Tm = size_t(e_.max_step_tokens());
    int32_t* hs = h_ + in_n_ + out_n_;
    HB_CHECK(hipMemcpyAsync(hs, e_.winners(), (2 * Tm + k) * 4, hipMemcpyDeviceToHost, st));
    HB_CHECK(hipStreamSynchronize(st));
    tok.assign(reinterpret_cast<uint32_t*>(hs), reinterpret_cast<uint32_t*>(hs) + k);
    marg.assign(reinterpret_cast<float*>(hs + Tm), reinterpret_cast<float*>(hs + Tm) + k);
    for (int j = 0; j < k; ++j) require(hs[2 * Tm + j] == 0, "decode: nonfinite MTP logits");
    stats_.mtp_calls += 1;
    stats_.mtp_tokens += step.total();
  };
  std::vector<uint32_t> tok;
  run(sr, e_.hidden_f32(), hidden_idx, logit_rows, tok, margin);
  auto limit = [&](const Row& r) {
    return std::min({width_ - 1, r.budget - r.emitted, e_.max_context() - r.position - 1, e_.max_row_tokens() - 1});
  };
  auto is_eos = [&](uint32_t t) { return std::find(eos_.begin(), eos_.end(), t) != eos_.end(); };
  std::vector<int> chain(n);
  for (int k = 0; k < n; ++k) {
    Row& r = rows_[who[k]];
    if (limit(r) >= 1) r.drafts.push_back(tok[k]);
    chain[k] = k;
  }
  for (int depth = 1; depth < width_ - 1; ++depth) {
    StepRows ar;
    std::vector<int32_t> idx, out_rows;
    std::vector<int> next;
    for (int c : chain) {
      Row& r = rows_[who[c]];
      if (int(r.drafts.size()) != depth || int(r.drafts.size()) >= limit(r) || is_eos(r.drafts.back()) ||
          !(margin[c] >= gate_))
        continue;
      ar.row_tokens.push_back(1);
      ar.positions.push_back(r.position + depth - 1);
      ar.seq.push_back(who[c]);
      ar.src_slot.push_back(who[c]);
      ar.dst_slot.push_back(who[c]);
      ar.hist_off.push_back(0);
      ar.log_count.push_back(0);
      ar.tokens.push_back(r.drafts.back());
      idx.push_back(prev[c]);
      out_rows.push_back(int32_t(out_rows.size()));
      next.push_back(c);
    }
    if (next.empty()) break;
    ar.rows = int(next.size());
    std::vector<uint32_t> t2;
    std::vector<float> m2;
    run(ar, e_.mtp_hidden_f32(), idx, out_rows, t2, m2);
    std::vector<int> kept;
    for (size_t j = 0; j < next.size(); ++j) {
      const int c = next[j];
      Row& r = rows_[who[c]];
      prev[c] = int32_t(j);
      margin[c] = m2[j];
      if (!(m2[j] >= gate_)) continue;  // too uncertain to propose
      r.drafts.push_back(t2[j]);
      kept.push_back(c);
    }
    chain = kept;
  }
}

}  // namespace hb
