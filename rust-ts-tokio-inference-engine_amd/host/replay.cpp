// Replays the reference's host-side call sequences against libhip_bridge.so.
//
//   replay transaction  host only: the Rust unit tests of the batch
//                       transaction (batch_transaction.rs:253-480), validate_batch
//                       (native_device.rs:1001-1016), the selection vectors
//                       (judges/device_selection.cpp:8-11, native_speculative.rs:
//                       349-415) and the step IR bounds (model_ir.rs:28-61)
//   replay abi          the adversarial protocol of judges/device_abi.cpp at its
//                       own 40-layer geometry, with gpu = 1 and a seeded store:
//                       forged, stale and malformed descriptors fail, output
//                       sentinels stay untouched, resident/byte/step stats stay 0
//   replay scheduler    ScheduledDevice over a small session: scalar, physical
//                       (decode_batch) and ragged packing emit the same tokens,
//                       batch order does not matter, a failed batch publishes
//                       nothing and every version is released at the end
//   replay mtp          the C++ MTP transaction loop of judges/native_cpp_bench.cpp
//                       emits the greedy stream, under the 1.25 margin gate and
//                       with every draft forced
// Prints "PASS <scenario> checks=<n>" and exits 0, or the failure and exits 1.
#include <cstdio>
#include <cstring>
#include <iostream>
#include <limits>
#include <string>

#include "serving.h"

using namespace hbhost;

namespace {

size_t checks = 0;
void check(bool ok, const std::string& what) {
  ++checks;
  if (!ok) throw Failure("check failed: " + what);
}
template <class F>
void fails(F&& f, const std::string& what) {
  ++checks;
  try {
    f();
  } catch (const Failure&) {
    return;
  }
  throw Failure("expected a failure: " + what);
}

// ------------------------------------------------------------ transaction
struct Fake {
  size_t pos = 0;
  uint32_t tag = 0;
  std::shared_ptr<int> lease = std::make_shared<int>(0);
  size_t position() const { return pos; }
  size_t bytes() const { return 16; }
};
Fake fstate(size_t p, uint32_t t) { return Fake{p, t, std::make_shared<int>(0)}; }
std::map<uint64_t, Fake> fparents() { return {{1, fstate(2, 11)}, {2, fstate(2, 22)}}; }
StepInput frow(uint64_t seq) {
  StepInput r;
  r.sequence = seq;
  r.position = 2;
  r.kind = StepKind::Decode;
  r.tokens = {uint32_t(seq)};
  r.remaining_output_tokens = 8;
  return r;
}
RowResult<Fake> advance(const Fake& old, const StepIr& ir) {
  uint32_t sum = 0;
  for (uint32_t t : ir.tokens) sum += t;
  Fake next = fstate(old.pos + ir.len(), old.tag + sum);
  std::vector<float> logits(16, 0.f);
  logits[next.tag % 16] = 1.f;
  return RowResult<Fake>{next, logits};
}
void unchanged(const std::map<uint64_t, Fake>& m) {
  check(m.at(1).pos == 2 && m.at(1).tag == 11 && m.at(2).pos == 2 && m.at(2).tag == 22, "parents unchanged");
  check(m.at(1).lease.use_count() == 1 && m.at(2).lease.use_count() == 1, "no parent lease retained");
}
std::function<Fake()> empty_fake = [] { return fstate(0, 0); };

void scenario_transaction() {
  // token receipts commit atomically and refuse invalid or masked tokens
  for (int mode = 0; mode < 4; ++mode) {
    auto map = fparents();
    StepInput second = frow(2);
    if (mode == 2) second.allowed_tokens = std::vector<uint32_t>{1};
    bool ok = true;
    try {
      auto p = PreparedBatch<Fake>::prepare({frow(1), second}, map, empty_fake, 16);
      auto done = std::move(p).execute_receipts([&](const Fake& old, const StepIr& ir, bool unconstrained) {
        const uint32_t token = ir.tokens[0] == 2 && mode == 1 ? 16 : 1;
        if (ir.tokens[0] == 2 && mode == 3) throw Failure("injected late failure");
        if (mode == 2 && ir.tokens[0] == 2) check(!unconstrained, "masked rows are constrained");
        return RowResult<Fake>{fstate(old.pos + ir.len(), 42), token};
      });
      auto outputs = std::move(done).commit();
      for (auto& o : outputs) check(o.next_token == 1u, "receipt token");
      check(map.at(1).pos == 3 && map.at(2).pos == 3, "committed positions");
    } catch (const Failure&) {
      ok = false;
    }
    check(ok == (mode == 0), "receipt mode " + std::to_string(mode));
    if (mode) unchanged(map);
  }
  // invalid batches fail before any execution
  for (int mode = 0; mode < 9; ++mode) {
    auto map = fparents();
    std::vector<StepInput> batch{frow(1), frow(2)};
    switch (mode) {
      case 0: batch[1].sequence = 1; break;
      case 1: batch[1].position = std::numeric_limits<size_t>::max(); break;
      case 2: batch[1].tokens = {16}; break;
      case 3: batch[1].tokens = {}; break;
      case 4: batch[1].remaining_output_tokens = 0; break;
      case 5: batch[1].remaining_output_tokens = 129; break;
      case 6: batch[1].allowed_tokens = std::vector<uint32_t>{}; break;
      case 7: batch[1].allowed_tokens = std::vector<uint32_t>{16}; break;
      default: batch.push_back(frow(1)); batch.push_back(frow(2)); break;
    }
    fails([&] { (void)PreparedBatch<Fake>::prepare(batch, map, empty_fake, 16); }, "invalid batch " + std::to_string(mode));
    unchanged(map);
  }
  {
    auto map = fparents();
    map[3] = fstate(0, 0);
    fails([&] { (void)PreparedBatch<Fake>::prepare({frow(4)}, map, empty_fake, 16); }, "resident bound");
    fails([&] { (void)PreparedBatch<Fake>::prepare({}, map, empty_fake, 16); }, "empty batch");
  }
  // cohorts describe geometry without reordering rows
  {
    auto map = fparents();
    StepInput third = frow(3);
    third.kind = StepKind::Prefill;
    third.position = 0;
    third.tokens = {3, 4};
    third.prompt_complete = false;
    auto p = PreparedBatch<Fake>::prepare({frow(2), third, frow(1)}, map, empty_fake, 16);
    check(p.cohorts().size() == 2 && p.cohorts()[0].rows == std::vector<size_t>{0, 2} &&
              p.cohorts()[1].rows == std::vector<size_t>{1},
          "cohort rows");
    check(p.sequences() == std::vector<uint64_t>{2, 3, 1}, "input order kept");
    // grouped execution restores input order
    auto outs = std::move(p).execute_grouped([](std::vector<std::pair<Fake, StepIr>> rows) {
      std::vector<RowResult<Fake>> r;
      for (auto& [s, ir] : rows) r.push_back(advance(s, ir));
      return r;
    });
    auto o = std::move(outs).commit();
    check(o.size() == 3 && o[0].sequence == 2 && o[1].sequence == 3 && o[2].sequence == 1, "outputs in input order");
    check(!o[1].next_token && o[0].next_token == uint32_t((22 + 2) % 16), "incomplete prompt selects nothing");
    check(map.at(3).pos == 2 && map.at(1).pos == 3, "grouped commit");
  }
  // a later row's failure drops the provisionals and keeps every parent
  {
    auto map = fparents();
    std::vector<std::weak_ptr<int>> leases;
    int calls = 0;
    auto p = PreparedBatch<Fake>::prepare({frow(1), frow(2)}, map, empty_fake, 16);
    fails(
        [&] {
          (void)std::move(p).execute_receipts([&](const Fake& old, const StepIr& ir, bool) {
            if (++calls == 2) throw Failure("injected later-row backend failure");
            auto r = advance(old, ir);
            leases.push_back(r.state.lease);
            return r;
          });
        },
        "later-row failure");
    unchanged(map);
    for (auto& w : leases) check(w.expired(), "provisional released");
  }
  // malformed results cannot create a commit
  for (int mode = 0; mode < 3; ++mode) {
    auto map = fparents();
    int calls = 0;
    auto p = PreparedBatch<Fake>::prepare({frow(1), frow(2)}, map, empty_fake, 16);
    fails(
        [&] {
          (void)std::move(p).execute_receipts([&](const Fake& old, const StepIr& ir, bool) {
            auto r = advance(old, ir);
            if (++calls == 2) {
              auto& lg = std::get<std::vector<float>>(r.selection);
              if (mode == 0)
                r.state.pos += 1;
              else if (mode == 1)
                lg[0] = std::numeric_limits<float>::quiet_NaN();
              else
                lg.pop_back();
            }
            return r;
          });
        },
        "malformed result " + std::to_string(mode));
    unchanged(map);
  }
  // a completed batch that is dropped is a rollback, not a commit
  {
    auto map = fparents();
    {
      auto p = PreparedBatch<Fake>::prepare({frow(1), frow(2)}, map, empty_fake, 16);
      auto done = std::move(p).execute_receipts([](const Fake& old, const StepIr& ir, bool) { return advance(old, ir); });
      (void)done;
    }
    unchanged(map);
  }
  // validate_batch (native_device.rs:1001-1016), vocabulary 16, context 512
  validate_batch_geometry(1, {{1, 8}, {1, 8}}, {1, 2}, 16, 512);
  ++checks;
  using G = std::vector<std::pair<uint64_t, size_t>>;
  const std::vector<std::pair<G, std::vector<uint32_t>>> bad = {
      {{}, {}}, {{{1, 8}}, {}}, {{{2, 8}}, {1}}, {{{1, 0}}, {1}}, {{{1, 512}}, {1}}, {{{1, 8}}, {16}},
      {{{1, 8}, {1, 9}}, {1, 2}}, {G(4, {1, 8}), std::vector<uint32_t>(4, 1)}};
  for (size_t i = 0; i < bad.size(); ++i)
    fails([&] { validate_batch_geometry(1, bad[i].first, bad[i].second, 16, 512); }, "validate_batch " + std::to_string(i));
  // selection under the f32 total order (judges/device_selection.cpp:8-11)
  const float f = std::numeric_limits<float>::denorm_min();
  const float rows[4][4] = {{-0.f, +0.f, -f, -0.f}, {+0.f, -0.f, -f, -f}, {-2.f, -1.f, -1.f, -3.f}, {f, 0.f, f, -f}};
  const uint32_t want[4] = {1, 0, 1, 0};
  for (int i = 0; i < 4; ++i) {
    check(select(rows[i], 4, nullptr) == want[i], "total-order argmax row " + std::to_string(i));
    check(winner_with_margin(rows[i], 4).first == want[i], "winner row " + std::to_string(i));
  }
  const float w1[] = {-0.f, 0.f, -1.f};
  check(winner_with_margin(w1, 3).first == 1, "winner(-0, 0, -1)");
  const float w2[] = {0.5f, 3.25f, 1.75f, -2.0f};
  auto [t2, m2] = winner_with_margin(w2, 4);
  check(t2 == 1 && std::abs(m2 - 1.5f) < 1e-6f, "margin 1.5");
  const float w3[] = {2.f, 4.f, 4.f};
  auto [t3, m3] = winner_with_margin(w3, 3);
  check(t3 == 1 && m3 == 0.f, "tied margin 0");
  for (int n = 1; n <= 512; ++n) {
    std::vector<float> v(n);
    for (int i = 0; i < n; ++i) v[i] = float((i * 17 + n * 31) % 23) - 11.f;
    check(winner_with_margin(v.data(), n).first == select(v.data(), n, nullptr), "tie break under pressure");
  }
  const std::vector<uint32_t> allowed{5, 2};
  const float masked[] = {9.f, 0.f, 3.f, 0.f, 0.f, 3.f};
  check(select(masked, 6, &allowed) == 2, "masked tie goes to the lower id");
  const float nan_row[] = {0.f, std::numeric_limits<float>::quiet_NaN()};
  fails([&] { (void)select(nan_row, 2, nullptr); }, "non-finite logits");
  // step IR bounds (model_ir.rs:28-61)
  (void)StepIr::compile(StepKind::Decode, 511, {99}, 100);
  ++checks;
  fails([] { (void)StepIr::compile(StepKind::Decode, 0, {1, 2}, 100); }, "decode of two tokens");
  fails([] { (void)StepIr::compile(StepKind::Prefill, 0, {100}, 100); }, "token outside the vocabulary");
  fails([] { (void)StepIr::compile(StepKind::Prefill, 0, {}, 100); }, "empty step");
  fails([] { (void)StepIr::compile(StepKind::Prefill, 0, std::vector<uint32_t>(9, 1), 100); }, "nine tokens");
  fails([] { (void)StepIr::compile(StepKind::Decode, 512, {1}, 100); }, "context bound");
}

// ------------------------------------------------------------ device helpers
struct Err {
  char text[1024] = {};
};

rs_qwen_config small_config() {
  rs_qwen_config c{};
  c.hidden = 256, c.layers = 2, c.vocab = 512, c.q_heads = 8, c.kv_heads = 1, c.head_dim = 256, c.key_heads = 2,
  c.value_heads = 4, c.key_dim = 128, c.value_dim = 128, c.conv = 4, c.interval = 2, c.experts = 8, c.top = 2,
  c.intermediate = 128, c.shared = 128, c.group = 64, c.bits = 4, c.context = 96, c.chunk = 8, c.rope_dims = 64,
  c.activation_precision = 0, c.layer_group = 1, c.validation_interval = 1, c.epsilon = 1e-6f, c.theta = 1e7f;
  return c;
}

std::vector<rs_qwen_layer> program(const rs_qwen_config& c) {
  std::vector<rs_qwen_layer> l(size_t(c.layers));
  for (int i = 0; i < c.layers; ++i) l[i] = {uint32_t(i), uint32_t((i + 1) % c.interval == 0)};
  return l;
}

struct Store {
  void* h;
  Store(uint64_t seed, int part) {
    Err e;
    h = rs_mlx_weights_create(e.text, sizeof e.text);
    if (!h || hb_weights_synthetic(h, seed, part, e.text, sizeof e.text)) throw Failure(std::string("store: ") + e.text);
  }
  ~Store() { rs_mlx_weights_destroy(h); }
};

struct Session {
  void* h;
  Session(void* store, const rs_qwen_config& c, size_t slots, uint64_t bytes) {
    Err e;
    auto layers = program(c);
    h = rs_qwen_device_create(store, 1, &c, layers.data(), layers.size(), slots, bytes, e.text, sizeof e.text);
    if (!h) throw Failure(std::string("session: ") + e.text);
  }
  ~Session() { rs_qwen_device_destroy(h); }
  std::vector<uint64_t> stats() const {
    std::vector<uint64_t> s(74);
    Err e;
    if (rs_qwen_device_stats(h, s.data(), 74, e.text, sizeof e.text)) throw Failure(std::string("stats: ") + e.text);
    return s;
  }
};

// ------------------------------------------------------------ abi
void scenario_abi() {
  // judges/device_abi.cpp:7: the reference's own 40-layer geometry
  rs_qwen_config c = {2048, 40, 248320, 16, 2, 256, 16, 32, 128, 128, 4, 4, 256, 8, 512, 512, 64,
                      4,    512, 8,    64, 1, 1,   0,  0,  0,   0,   0, 2, 32,  0,   1e-6f, 10000000.f};
  std::vector<rs_qwen_layer> layers(40);
  for (unsigned i = 0; i < 40; ++i) layers[i] = {i, uint32_t((i + 1) % 4 == 0)};
  Err e;
  char* error = e.text;
  const size_t cap = sizeof e.text;
  Store fake(20261201, 0);  // a seeded store stands in for the reference's empty one
  // this bridge computes the BF16 activation profile only: the judge's FP32
  // descriptor is refused with a message, and the protocol runs at profile 0
  check(!rs_qwen_device_create(fake.h, 1, &c, layers.data(), 40, 2, 1 << 28, error, cap) &&
            std::string(error).rfind("activation precision 1 (FP32)", 0) == 0,
        "FP32 profile refused");
  c.activation_precision = 0;
  check(!rs_qwen_device_create(nullptr, 1, &c, layers.data(), 40, 2, 1 << 28, error, cap), "null store");
  auto bad = c;
  bad.interval = 0;
  check(!rs_qwen_device_create(fake.h, 1, &bad, layers.data(), 40, 2, 1 << 28, error, cap), "interval 0");
  check(!rs_qwen_device_create(fake.h, 1, &c, layers.data(), 40, 65, 1 << 28, error, cap), "65 slots");
  check(!rs_qwen_device_create(fake.h, 0, &c, layers.data(), 40, 2, 1 << 28, error, cap), "no CPU sessions here");
  for (int value : {-1, 3, 2147483647}) {
    bad = c;
    bad.expert_kernel = value;
    check(!rs_qwen_device_create(fake.h, 1, &bad, layers.data(), 40, 2, 1 << 28, error, cap), "expert kernel mode");
    bad = c;
    bad.validation_mode = value;
    check(!rs_qwen_device_create(fake.h, 1, &bad, layers.data(), 40, 2, 1 << 28, error, cap), "validation mode");
  }
  bad = c;
  bad.activation_precision = 0;
  bad.compiled_decode = 1;
  check(!rs_qwen_device_create(fake.h, 1, &bad, layers.data(), 40, 2, 1 << 28, error, cap), "compiled decode FP32");
  bad = c;
  bad.fused_attention = 2;
  bad.context = 1024;
  check(!rs_qwen_device_create(fake.h, 1, &bad, layers.data(), 40, 2, 1 << 28, error, cap), "attention context512");
  bad = c;
  bad.fused_attention = 2;
  bad.activation_precision = 0;
  check(!rs_qwen_device_create(fake.h, 1, &bad, layers.data(), 40, 2, 1 << 28, error, cap), "attention FP32");
  void* session = rs_qwen_device_create(fake.h, 1, &c, layers.data(), 40, 2, 1 << 28, error, cap);
  check(session != nullptr, std::string("session at the reference geometry: ") + error);
  // DSpark descriptors fail and preserve outputs
  check(!rs_qwen_dspark_create(nullptr, "missing", 0, 4, 1024, error, cap), "dspark null session");
  check(!rs_qwen_dspark_create(session, "missing", 0, 4, 1024, error, cap), "dspark missing");
  for (int head : {-1, 4}) check(!rs_qwen_dspark_create(session, "missing", head, 4, 1024, error, cap), "dspark head");
  bad = c;
  bad.validation_mode = 0;
  void* unchecked = rs_qwen_device_create(fake.h, 1, &bad, layers.data(), 40, 2, 1 << 28, error, cap);
  check(unchecked != nullptr, "unchecked session");
  check(!rs_qwen_dspark_create(unchecked, "missing", 0, 4, 1024, error, cap), "dspark on unchecked");
  rs_qwen_device_destroy(unchecked);
  StateId ds_sentinel{9, 9, 9, 9, 9};
  uint32_t ds_id = 999;
  float ds_conf = 999;
  uint64_t ds_stats[2]{9, 9};
  check(rs_qwen_dspark_ingest(nullptr, nullptr, nullptr, &ds_sentinel, error, cap) != 0 && ds_sentinel.owner == 9,
        "dspark ingest");
  check(rs_qwen_dspark_propose(nullptr, nullptr, 1, 4, &ds_id, &ds_conf, 1, error, cap) != 0 && ds_id == 999 &&
            ds_conf == 999,
        "dspark propose");
  check(rs_qwen_dspark_release(nullptr, nullptr, error, cap) != 0, "dspark release");
  check(rs_qwen_dspark_stats(nullptr, ds_stats, 2, error, cap) != 0 && ds_stats[0] == 9, "dspark stats");
  check(rs_qwen_device_dspark_snapshot(session, nullptr, &ds_conf, 1, error, cap) != 0 && ds_conf == 999,
        "dspark snapshot");
  check(rs_qwen_device_dspark_step(session, nullptr, 0, &ds_id, 1, &ds_sentinel, &ds_conf, 1, 2, error, cap) != 0 &&
            ds_sentinel.owner == 9,
        "dspark step");
  std::vector<float> logits(size_t(c.vocab));
  uint32_t invalid = uint32_t(c.vocab);
  StateId output{9, 9, 9, 9, 9};
  uint64_t stats[74];
  auto zero_stats = [&] {
    return rs_qwen_device_stats(session, stats, 74, error, cap) == 0 && stats[0] == 0 && stats[1] == 0 &&
           stats[4] == 0;
  };
  for (size_t i = 0; i < 14000; ++i) {
    StateId foreign{i + 1, i % 64, i + 1, 1, 4};
    check(rs_qwen_device_release(session, &foreign, error, cap) != 0, "foreign release");
    check(rs_qwen_device_step(session, &foreign, 1, &invalid, 1, &output, logits.data(), logits.size(), nullptr, 0,
                              error, cap) != 0,
          "foreign parent");
    check(rs_qwen_device_step(session, nullptr, 0, &invalid, 1, &output, logits.data(), logits.size(), nullptr, 0,
                              error, cap) != 0,
          "token outside the vocabulary");
    check(output.owner == 9 && output.slot == 9 && output.generation == 9, "output sentinel");
    check(zero_stats(), "stats stay zero");
  }
  check(rs_qwen_device_step(session, nullptr, 512, &invalid, 1, &output, logits.data(), logits.size(), nullptr, 0,
                            error, cap) != 0,
        "position at the context end");
  check(rs_qwen_device_stats(session, stats, 73, error, cap) != 0, "stats count 73");
  uint32_t valid = 0;
  float scalar = 0;
  StateId forged{999, 0, 1, 1, 4};
  check(rs_qwen_device_step(session, nullptr, 0, &valid, 1, &output, logits.data(), logits.size(), &scalar, 1, error,
                            cap) != 0,
        "trace capacity");
  check(rs_qwen_device_step(session, nullptr, 0, &valid, 1, nullptr, logits.data(), logits.size(), nullptr, 0, error,
                            cap) != 0,
        "null output");
  check(rs_qwen_device_step(session, nullptr, 0, nullptr, 1, &output, logits.data(), logits.size(), nullptr, 0, error,
                            cap) != 0,
        "null tokens");
  check(rs_qwen_device_step(session, nullptr, 0, &valid, 0, &output, logits.data(), logits.size(), nullptr, 0, error,
                            cap) != 0,
        "zero tokens");
  check(rs_qwen_device_step(session, nullptr, 0, &valid, 9, &output, logits.data(), logits.size(), nullptr, 0, error,
                            cap) != 0,
        "nine tokens");
  check(rs_qwen_device_step(session, nullptr, 0, &valid, 1, &output, logits.data(), 1, nullptr, 0, error, cap) != 0,
        "logits capacity");
  check(rs_qwen_device_snapshot(session, &forged, &scalar, 1, error, cap) != 0, "forged snapshot");
  check(rs_qwen_device_snapshot(session, &forged, nullptr, 1, error, cap) != 0, "snapshot without output");
  uint64_t invalidated = 99;
  check(rs_qwen_device_drain(session, &invalidated, error, cap) == 0 && invalidated == 0, "drain");
  check(zero_stats(), "stats after drain");
  for (size_t n = 0; n <= 10; ++n) {
    std::vector<uint32_t> ids(n, invalid);
    std::vector<float> rows(size_t(c.vocab) * std::min(n, size_t(8)));
    check(rs_qwen_device_block(session, nullptr, 0, ids.data(), n, &output, rows.data(), rows.size(), error, cap) != 0,
          "block of " + std::to_string(n));
    check(output.owner == 9 && output.slot == 9 && output.generation == 9, "block sentinel");
  }
  check(rs_qwen_device_block(session, nullptr, 0, &valid, 1, &output, &scalar, 1, error, cap) != 0, "block capacity");
  check(rs_qwen_device_block(session, &forged, 1, &valid, 1, &output, logits.data(), logits.size(), error, cap) != 0,
        "forged block parent");
  check(rs_qwen_device_block(session, nullptr, 0, &valid, 1, nullptr, logits.data(), logits.size(), error, cap) != 0,
        "block null output");
  check(zero_stats(), "stats after blocks");
  StateId batch_outputs[3] = {{9, 9, 9, 9, 9}, {9, 9, 9, 9, 9}, {9, 9, 9, 9, 9}};
  uint32_t batch_tokens[3] = {0, 0, 0};
  StateId batch_parents[3] = {{999, 0, 1, 1, 4}, {999, 1, 1, 1, 4}, {999, 2, 1, 1, 4}};
  std::vector<float> batch_logits(size_t(c.vocab) * 3);
  for (size_t it = 0; it < 10000; ++it) {
    for (size_t count = 0; count <= 4; ++count)
      check(rs_qwen_device_decode_batch(session, batch_parents, batch_tokens, count, batch_outputs,
                                        batch_logits.data(), size_t(c.vocab) * std::min(count, size_t(3)), error,
                                        cap) != 0,
            "forged batch");
    check(batch_outputs[0].owner == 9 && batch_outputs[1].owner == 9 && batch_outputs[2].owner == 9, "batch sentinel");
  }
  check(rs_qwen_device_decode_batch(session, nullptr, batch_tokens, 3, batch_outputs, batch_logits.data(),
                                    batch_logits.size(), error, cap) != 0,
        "batch null parents");
  check(rs_qwen_device_decode_batch(session, batch_parents, nullptr, 3, batch_outputs, batch_logits.data(),
                                    batch_logits.size(), error, cap) != 0,
        "batch null tokens");
  check(rs_qwen_device_decode_batch(session, batch_parents, batch_tokens, 3, nullptr, batch_logits.data(),
                                    batch_logits.size(), error, cap) != 0,
        "batch null outputs");
  check(rs_qwen_device_decode_batch(session, batch_parents, batch_tokens, 3, batch_outputs, batch_logits.data(), 1,
                                    error, cap) != 0,
        "batch logits capacity");
  check(zero_stats(), "stats after batches");
  rs_qwen_device_destroy(session);
  rs_qwen_device_destroy(nullptr);
}

// ------------------------------------------------------------ scheduler
std::vector<uint32_t> prompt_tokens(uint32_t seed, size_t n, uint32_t vocab) {
  std::vector<uint32_t> t(n);
  uint64_t x = 0x9E3779B97F4A7C15ull * (seed + 1);
  for (auto& v : t) {
    x ^= x << 13, x ^= x >> 7, x ^= x << 17;
    v = uint32_t(x % vocab);
  }
  return t;
}

// Prefill (chunks of 8) then `steps` greedy decode steps for each sequence;
// each scheduler step carries every live sequence, in `order`.
std::map<uint64_t, std::vector<uint32_t>> drive(ScheduledDevice& sd, const std::vector<std::vector<uint32_t>>& prompts,
                                                const std::vector<uint64_t>& order, size_t steps) {
  std::map<uint64_t, std::vector<uint32_t>> out;
  std::map<uint64_t, size_t> done;
  bool more = true;
  while (more) {  // prefill rounds: one chunk of every unfinished prompt per step
    more = false;
    std::vector<StepInput> batch;
    for (uint64_t s : order) {
      const auto& p = prompts[s - 1];
      const size_t at = done[s];
      if (at >= p.size()) continue;
      const size_t n = std::min<size_t>(8, p.size() - at);
      StepInput in;
      in.sequence = s;
      in.position = at;
      in.kind = StepKind::Prefill;
      in.tokens.assign(p.begin() + at, p.begin() + at + n);
      in.remaining_output_tokens = steps;
      in.prompt_complete = at + n == p.size();
      batch.push_back(in);
      done[s] = at + n;
      more = true;
    }
    if (batch.empty()) break;
    for (auto& o : sd.step(batch))
      if (o.next_token) out[o.sequence].push_back(*o.next_token);
  }
  for (size_t k = 1; k < steps; ++k) {
    std::vector<StepInput> batch;
    for (uint64_t s : order) {
      StepInput in;
      in.sequence = s;
      in.position = sd.states().at(s).position();
      in.kind = StepKind::Decode;
      in.tokens = {out[s].back()};
      in.remaining_output_tokens = steps - k;
      batch.push_back(in);
    }
    for (auto& o : sd.step(batch)) out[o.sequence].push_back(*o.next_token);
  }
  return out;
}

// A prompt through step calls of at most 8 tokens: the last state and logits.
Device::Step prefill(const Device& dev, const std::vector<uint32_t>& p) {
  DeviceState s = dev.empty();
  std::vector<float> logits;
  for (size_t at = 0; at < p.size(); at += 8) {
    const size_t k = std::min<size_t>(8, p.size() - at);
    auto r = dev.execute(s, StepIr::compile(StepKind::Prefill, at, {p.begin() + at, p.begin() + at + k},
                                            uint32_t(dev.config().vocab), 8, size_t(dev.config().context)));
    s = r.state;
    logits = std::move(r.logits);
  }
  return Device::Step{s, logits};
}

void scenario_scheduler() {
  const rs_qwen_config c = small_config();
  Store store(23, 0);
  Session sess(store.h, c, 16, uint64_t(1) << 40);
  Device dev(sess.h, c);
  const std::vector<std::vector<uint32_t>> prompts = {prompt_tokens(1, 11, 512), prompt_tokens(2, 11, 512),
                                                      prompt_tokens(3, 5, 512)};
  const size_t steps = 7;
  std::map<uint64_t, std::vector<uint32_t>> scalar, physical, reversed, ragged;
  {
    ScheduledDevice sd(dev, ScheduledDevice::Packing::Scalar);
    scalar = drive(sd, prompts, {1, 2, 3}, steps);
    check(sd.counters().packed_calls == 0 && sd.counters().scalar_calls > 0, "scalar counters");
  }
  check(sess.stats()[0] == 0, "scalar states released");
  {
    ScheduledDevice sd(dev, ScheduledDevice::Packing::Physical);
    physical = drive(sd, prompts, {1, 2, 3}, steps);
    // rows 1 and 2 share every decode position: one decode_batch per step
    check(sd.counters().packed_calls == steps - 1 && sd.counters().packed_rows == 2 * (steps - 1),
          "physical counters");
  }
  {
    ScheduledDevice sd(dev, ScheduledDevice::Packing::Physical);
    reversed = drive(sd, prompts, {3, 2, 1}, steps);
  }
  {
    ScheduledDevice sd(dev, ScheduledDevice::Packing::Ragged, 16);
    ragged = drive(sd, prompts, {2, 3, 1}, steps);
    check(sd.counters().ragged_calls > 0 && sd.counters().packed_calls == 0 && sd.counters().scalar_calls == 0,
          "ragged counters");
  }
  for (uint64_t s = 1; s <= 3; ++s) {
    check(scalar[s].size() == steps, "stream length");
    check(physical[s] == scalar[s], "physical packing emits the scalar stream, sequence " + std::to_string(s));
    check(reversed[s] == scalar[s], "batch order does not change the stream, sequence " + std::to_string(s));
    check(ragged[s] == scalar[s], "ragged packing emits the scalar stream, sequence " + std::to_string(s));
  }
  // packed and scalar logits of the same decode rows are bit-identical
  {
    auto a = prefill(dev, prompts[0]);
    auto b = prefill(dev, prompts[1]);
    const uint32_t ta = select(a.logits.data(), a.logits.size(), nullptr);
    const uint32_t tb = select(b.logits.data(), b.logits.size(), nullptr);
    auto batch = dev.decode_batch({a.state, b.state}, {ta, tb});
    auto sa = dev.execute(a.state, StepIr::compile(StepKind::Decode, 11, {ta}, 512, 8, 96));
    auto sb = dev.execute(b.state, StepIr::compile(StepKind::Decode, 11, {tb}, 512, 8, 96));
    check(batch[0].logits == sa.logits && batch[1].logits == sb.logits, "decode_batch logits equal scalar steps");
    // the ragged step mixes a decode row, a 4-token verify block and a prefill chunk
    auto rows = dev.ragged({a.state, b.state, dev.empty()}, {{ta}, {tb, 7, 9, 11}, prompts[2]}, true, true);
    check(rows[0].logits == sa.logits, "ragged decode row equals the scalar step");
    auto blk = dev.execute(b.state, StepIr::compile(StepKind::Prefill, 11, {tb, 7, 9, 11}, 512, 8, 96), true);
    check(rows[1].logits == blk.logits, "ragged verify block equals the block call");
    for (size_t j = 0; j < 4; ++j)
      check(rows[1].winners[j] == select(blk.logits.data() + j * 512, 512, nullptr), "ragged winners");
    // validate_batch refuses rows of a foreign executor or unequal positions before any native call
    Device other(sess.h, c);
    fails([&] { (void)dev.decode_batch({a.state, rows[2].state}, {1, 2}); }, "unequal positions");
    fails([&] { (void)other.decode_batch({a.state, b.state}, {1, 2}); }, "foreign executor");
    fails([&] { (void)dev.decode_batch({a.state, b.state, a.state, b.state}, {1, 2, 3, 4}); }, "four rows");
  }
  check(sess.stats()[0] == 0, "every version released");
  // a batch that fails in its second cohort publishes nothing and releases the first cohort's children
  {
    std::map<uint64_t, DeviceState> committed;
    auto r1 = prefill(dev, prompts[0]);
    auto r3 = prefill(dev, prompts[2]);
    committed[1] = r1.state;
    committed[3] = r3.state;
    const uint64_t before = sess.stats()[0];
    StepInput a, b;
    a.sequence = 1, a.position = 11, a.tokens = {1};
    b.sequence = 3, b.position = 5, b.tokens = {2};
    auto p = PreparedBatch<DeviceState>::prepare({a, b}, committed, [&] { return dev.empty(); }, 512);
    int calls = 0;
    fails(
        [&] {
          (void)std::move(p).execute_grouped([&](std::vector<std::pair<DeviceState, StepIr>> rows) {
            if (++calls == 2) throw Failure("injected second-cohort failure");
            std::vector<RowResult<DeviceState>> out;
            for (auto& [s, ir] : rows) {
              auto r = dev.execute(s, ir);
              out.push_back(RowResult<DeviceState>{std::move(r.state), std::move(r.logits)});
            }
            return out;
          });
        },
        "second cohort failure");
    check(sess.stats()[0] == before, "first cohort's child released");
    check(committed.at(1).position() == 11 && committed.at(3).position() == 5, "parents kept");
  }
  check(sess.stats()[0] == 0, "every version released after the failure");
}

// ------------------------------------------------------------ mtp
std::vector<uint32_t> greedy_stream(const Device& dev, const std::vector<uint32_t>& prompt, size_t n) {
  const size_t V = size_t(dev.config().vocab);
  auto start = prefill(dev, prompt);
  DeviceState s = start.state;
  std::vector<float> logits = std::move(start.logits);
  std::vector<uint32_t> out;
  while (out.size() < n) {
    const uint32_t t = winner_with_margin(logits.data(), V).first;
    out.push_back(t);
    auto r = dev.execute(s, StepIr::compile(StepKind::Decode, s.position(), {t}, uint32_t(V), 8,
                                            size_t(dev.config().context)));
    s = r.state;
    logits = r.logits;
  }
  return out;
}

// judges/native_cpp_bench.cpp:134-165 with the transaction of serving.cpp
std::vector<uint32_t> mtp_stream(const Device& dev, const std::vector<uint32_t>& prompt, size_t cap, size_t width,
                                 float gate, uint64_t& proposed, uint64_t& accepted) {
  void* s = dev.session();
  const size_t V = size_t(dev.config().vocab);
  std::vector<float> tl(V), dl(V);
  std::shared_ptr<Lifetime> target, draft;
  Err e;
  for (size_t off = 0; off < prompt.size(); off += 8) {
    const size_t n = std::min<size_t>(8, prompt.size() - off);
    StateId next{};
    if (rs_qwen_device_hidden_step(s, target ? &target->id : nullptr, off, prompt.data() + off, n, &next, tl.data(), V,
                                   e.text, sizeof e.text))
      throw Failure(std::string("prefill: ") + e.text);
    target = std::make_shared<Lifetime>(s, next, false);
    std::vector<uint32_t> shifted(prompt.begin() + off + 1, prompt.begin() + off + n);
    shifted.push_back(off + n < prompt.size() ? prompt[off + n] : winner_with_margin(tl.data(), V).first);
    StateId dn{};
    if (rs_qwen_device_mtp_step(s, draft ? &draft->id : nullptr, &target->id, 0, 0, shifted.data(), n, &dn, dl.data(), V,
                                0, e.text, sizeof e.text))
      throw Failure(std::string("MTP prefill: ") + e.text);
    draft = std::make_shared<Lifetime>(s, dn, true);
  }
  std::vector<uint32_t> out;
  while (out.size() < cap) {
    const uint32_t seed = winner_with_margin(tl.data(), V).first;
    auto [first, margin] = winner_with_margin(dl.data(), V);
    MtpResult r = mtp_transaction(dev, target->id, draft->id, seed, first, margin, width, cap - out.size(), {}, gate,
                                  tl, dl);
    target = std::make_shared<Lifetime>(s, r.target_state, false);
    draft = std::make_shared<Lifetime>(s, r.draft_state, true);
    check(!r.emitted.empty() && r.emitted.size() <= 9 && r.emitted.size() <= cap - out.size(), "receipt capacity");
    check(r.learned_accepted <= r.learned_proposed && r.learned_proposed < width && r.target_calls >= 1 &&
              r.target_calls <= 2,
          "receipt counters");
    out.insert(out.end(), r.emitted.begin(), r.emitted.end());
    proposed += r.learned_proposed;
    accepted += r.learned_accepted;
  }
  return out;
}

void scenario_mtp() {
  rs_qwen_config c = small_config();
  c.context = 96;
  Store store(23, 0), sidecar(23, 1);
  Session sess(store.h, c, 16, uint64_t(1) << 40);
  Err e;
  if (rs_qwen_device_mtp_attach(sess.h, sidecar.h, e.text, sizeof e.text))
    throw Failure(std::string("MTP attach: ") + e.text);
  Device dev(sess.h, c);
  for (uint32_t p = 0; p < 3; ++p) {
    const auto prompt = prompt_tokens(10 + p, 11 + 3 * p, 512);
    const size_t cap = 24;
    const auto greedy = greedy_stream(dev, prompt, cap);
    uint64_t proposed = 0, accepted = 0;
    const auto gated = mtp_stream(dev, prompt, cap, 4, 1.25f, proposed, accepted);
    check(gated == greedy, "gated MTP stream equals greedy, prompt " + std::to_string(p));
    uint64_t fp = 0, fa = 0;
    const auto forced = mtp_stream(dev, prompt, cap, 4, 0.f, fp, fa);
    check(forced == greedy, "forced MTP stream equals greedy, prompt " + std::to_string(p));
    check(fp >= proposed && fp > 0, "forced drafts proposed");
    std::printf("mtp prompt %u: gated %llu/%llu accepted, forced %llu/%llu accepted\n", p,
                (unsigned long long)accepted, (unsigned long long)proposed, (unsigned long long)fa,
                (unsigned long long)fp);
  }
  check(sess.stats()[0] == 0, "every target and draft version released");
}

}  // namespace

int main(int argc, char** argv) {
  const std::string what = argc > 1 ? argv[1] : "";
  try {
    if (what == "transaction")
      scenario_transaction();
    else if (what == "abi")
      scenario_abi();
    else if (what == "scheduler")
      scenario_scheduler();
    else if (what == "mtp")
      scenario_mtp();
    else {
      std::fprintf(stderr, "usage: replay transaction|abi|scheduler|mtp\n");
      return 2;
    }
  } catch (const std::exception& ex) {
    std::printf("FAIL %s after %zu checks: %s\n", what.c_str(), checks, ex.what());
    return 1;
  }
  std::printf("PASS %s checks=%zu\n", what.c_str(), checks);
  return 0;
}
