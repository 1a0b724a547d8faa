// C-ABI of the device sessions (native/mlx_bridge.h:50-133): rs_qwen_quant,
// rs_qwen_forward, rs_qwen_device_*, the MTP operator, and failing DSpark
// stubs. Conventions: 0 / -1 with the message in the caller's buffer, no
// exception across the ABI, outputs written only after success.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <memory>

#include "graph.h"
#include "session.h"

using namespace hb;

namespace {

// Owner ids come in pairs (target table, draft table); 0 is never an owner.
uint64_t next_owner() {
  static std::atomic<uint64_t> next{1};
  const uint64_t owner = next.fetch_add(2);
  if (owner == 0 || owner >= UINT64_MAX - 2) throw std::overflow_error("session owner exhausted");
  return owner;
}

DeviceSession& session_of(void* handle) {
  if (!handle) throw std::invalid_argument("invalid device session handle");
  return *static_cast<DeviceSession*>(handle);
}

WeightStore& store_of(void* store) {
  if (!store) throw std::invalid_argument("invalid weight store handle");
  return *static_cast<WeightStore*>(store);
}

// Geometry and mode checks of qwen_forward_core (native/qwen_model.inc:279-293),
// with the step bound widened to 64 tokens for ragged chunks.
void validate_model(const rs_qwen_config& c, const rs_qwen_layer* layers, size_t count) {
  if (c.hidden <= 0 || c.hidden > 8192 || c.layers <= 0 || c.layers > 64 || c.vocab <= 0 || c.vocab > 300000 ||
      c.interval <= 0 || c.layers % c.interval || c.context <= 0 || c.context > 262144 || c.chunk <= 0 ||
      c.chunk > 64)
    throw std::invalid_argument("model geometry/capacity");
  if (c.layer_group != 1 && c.layer_group != 4 && c.layer_group != 10 && c.layer_group != 40)
    throw std::invalid_argument("model layer group");
  if (c.fused_recurrent < 0 || c.fused_recurrent > 1) throw std::invalid_argument("recurrent kernel mode");
  if (c.execution_timing < 0 || c.execution_timing > 1) throw std::invalid_argument("execution timing mode");
  if (c.expert_kernel < 0 || c.expert_kernel > 2) throw std::invalid_argument("expert kernel mode");
  if (c.compiled_decode < 0 || c.compiled_decode > 1) throw std::invalid_argument("compiled decode mode");
  // mode combinations the reference refuses at session creation (native/qwen_device.inc:19-25)
  if (c.compiled_decode && c.activation_precision != 1) throw std::invalid_argument("compiled decode requires FP32");
  if (c.operator_profile < 0 || c.operator_profile > 1 || (c.operator_profile && (c.compiled_decode || c.execution_timing)))
    throw std::invalid_argument("operator profile requires GPU/eager/timing off");
  if (c.fused_attention < 0 || c.fused_attention > 2) throw std::invalid_argument("fused attention mode");
  if (c.fused_attention == 2 && (c.context != 512 || c.activation_precision != 1))
    throw std::invalid_argument("Metal reference attention requires FP32/context512");
  if (c.validation_mode < 0 || c.validation_mode > 2 || c.validation_interval < 1 || c.validation_interval > 1000000)
    throw std::invalid_argument("validation mode");
  if (!layers || count != size_t(c.layers)) throw std::invalid_argument("IR layer count");
  for (size_t i = 0; i < count; ++i)
    if (layers[i].index != i || layers[i].mixer > 1 || layers[i].mixer != uint32_t((i + 1) % c.interval == 0))
      throw std::invalid_argument("IR layer program");
  for (int d : {c.q_heads, c.kv_heads, c.head_dim, c.key_heads, c.value_heads, c.key_dim, c.value_dim, c.conv,
                c.experts, c.top, c.intermediate, c.shared})
    if (d <= 0 || d > 8192) throw std::invalid_argument("model dimension bounds");
  if (c.activation_precision < 0 || c.activation_precision > 1 || c.q_heads % c.kv_heads ||
      c.value_heads % c.key_heads || c.conv < 2 || c.top > c.experts || c.rope_dims <= 0 || c.rope_dims > c.head_dim ||
      c.rope_dims % 2 || !std::isfinite(c.epsilon) || c.epsilon <= 0 || !std::isfinite(c.theta) || c.theta <= 1)
    throw std::invalid_argument("model geometry mismatch");
  // After the reference's own checks, so its messages keep their order: the
  // FP32 activation profile is refused rather than run in BF16.
  if (c.activation_precision == 1) throw std::invalid_argument(kFp32ProfileRefused);
}

// The store must describe a model the session can build on the device: a
// seeded synthetic model, or checkpoint tensors loaded by rs_mlx_weights_load
// (the target's names under language_model.model / language_model.lm_head, the
// MTP sidecar's under language_model.mtp). A sidecar's norms are never shifted
// (native/qwen_mtp.inc:30); the target's follow the store's flag.
struct ModelSource {
  uint64_t seed = 0;
  std::shared_ptr<const NamedWeights> named;
};

ModelSource model_source(const WeightStore& w, int part) {
  ModelSource m;
  if (w.synthetic) {
    // seeded weights are generated 4-bit g64; overrides need checkpoint tensors
    for (const auto& [module, q] : w.quant)
      if (q.first != 64 || q.second != 4)
        throw std::invalid_argument("device session: a synthetic store is 4-bit group 64; quantization overrides "
                                    "apply to checkpoint stores");
    if (w.part != part) throw std::invalid_argument(part ? "not an MTP sidecar store" : "not a target model store");
    m.seed = w.seed;
    return m;
  }
  if (w.arrays.empty())
    throw std::invalid_argument("weight store holds no model (load a checkpoint or mark it with hb_weights_synthetic)");
  const bool sidecar = std::any_of(w.arrays.begin(), w.arrays.end(),
                                   [](const auto& kv) { return kv.first.rfind("language_model.mtp.", 0) == 0; });
  if (part && !sidecar) throw std::invalid_argument("not an MTP sidecar store");
  auto named = std::make_shared<NamedWeights>();
  named->arrays = w.arrays;
  named->quant = w.quant;  // per-module (group, bits) overrides (rs_qwen_quant)
  named->shift = part == 0 && w.has_shift;
  m.named = std::move(named);
  return m;
}

}  // namespace

// Engine over checkpoint stores (no reference counterpart: the engine-level
// entry the parity tests use to check the assembled tensors and the forward).
extern "C" void* hb_engine_create_named(const rs_qwen_config* config, int max_rows, int max_context,
                                        int max_row_tokens, int max_step_tokens, void* weights, void* mtp_weights,
                                        char* error, size_t capacity) {
  Engine* e = nullptr;
  const int rc = guarded(error, capacity, [&] {
    if (!config || !weights) throw std::invalid_argument("hb_engine_create_named: descriptor");
    const ModelSource m = model_source(store_of(weights), 0);
    if (!m.named) throw std::invalid_argument("hb_engine_create_named: not a checkpoint store");
    std::shared_ptr<const NamedWeights> side;
    if (mtp_weights) {
      side = model_source(store_of(mtp_weights), 1).named;
      if (!side) throw std::invalid_argument("hb_engine_create_named: the MTP store is not a checkpoint store");
    }
    e = new Engine(*config, max_rows, max_context, max_row_tokens, max_step_tokens, 0, mtp_weights != nullptr,
                   m.named, side);
  });
  return rc == 0 ? e : nullptr;
}

extern "C" int hb_weights_synthetic(void* store, uint64_t seed, int part, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    auto& w = store_of(store);
    if (part < 0 || part > 1) throw std::invalid_argument("synthetic store part");
    if (!w.arrays.empty()) throw std::invalid_argument("store already holds named arrays");
    w.synthetic = true;
    w.seed = seed;
    w.part = part;
    w.forward_cache.reset();
  });
}

extern "C" int rs_qwen_quant(void* store, const char* module, int group, int bits, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!store || !module || !(group == 32 || group == 64 || group == 128) ||
        !(bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8))
      throw std::invalid_argument("invalid model quantization");
    store_of(store).quant[std::string(module)] = {group, bits};
  });
}

extern "C" void* rs_qwen_device_create(void* weights, int gpu, const rs_qwen_config* config,
                                       const rs_qwen_layer* layers, size_t count, size_t slots, uint64_t bytes,
                                       char* error, size_t capacity) {
  DeviceSession* result = nullptr;
  guarded(error, capacity, [&] {
    if (!weights || !config || !layers) throw std::invalid_argument("device session descriptor");
    if (gpu != 1) throw std::invalid_argument("device session: this bridge runs on the GPU only (gpu = 1)");
    if (!slots || slots > 64 || !bytes) throw std::invalid_argument("state table bounds");
    validate_model(*config, layers, count);
    ModelSource m = model_source(store_of(weights), 0);
    result = new DeviceSession(*config, slots, bytes, next_owner(), m.seed, std::move(m.named));
  });
  return result;
}

extern "C" void rs_qwen_device_destroy(void* handle) { delete static_cast<DeviceSession*>(handle); }

extern "C" int rs_qwen_device_step(void* h, const StateId* previous, size_t position, const uint32_t* tokens,
                                   size_t count, StateId* output, float* logits, size_t logits_count, float* trace,
                                   size_t trace_count, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!output) throw std::invalid_argument("device step descriptor");
    *output = session_of(h).step(previous, position, tokens, count, logits, logits_count, trace, trace_count, false,
                                 false, nullptr);
  });
}

extern "C" int rs_qwen_device_step_sampled(void* h, const StateId* previous, size_t position, const uint32_t* tokens,
                                           size_t count, StateId* output, uint32_t* token, char* error,
                                           size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!output || !token) throw std::invalid_argument("device step descriptor");
    *output = session_of(h).step(previous, position, tokens, count, nullptr, 0, nullptr, 0, false, false, token);
  });
}

extern "C" int rs_qwen_device_block(void* h, const StateId* previous, size_t position, const uint32_t* tokens,
                                    size_t count, StateId* output, float* logits, size_t logits_count, char* error,
                                    size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!output) throw std::invalid_argument("device step descriptor");
    *output =
        session_of(h).step(previous, position, tokens, count, logits, logits_count, nullptr, 0, true, false, nullptr);
  });
}

extern "C" int rs_qwen_device_hidden_step(void* h, const StateId* previous, size_t position, const uint32_t* tokens,
                                          size_t count, StateId* output, float* logits, size_t logits_count,
                                          char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!output) throw std::invalid_argument("device step descriptor");
    *output =
        session_of(h).step(previous, position, tokens, count, logits, logits_count, nullptr, 0, false, true, nullptr);
  });
}

extern "C" int rs_qwen_device_hidden_block(void* h, const StateId* previous, size_t position, const uint32_t* tokens,
                                           size_t count, StateId* output, float* logits, size_t logits_count,
                                           char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!output) throw std::invalid_argument("device step descriptor");
    *output =
        session_of(h).step(previous, position, tokens, count, logits, logits_count, nullptr, 0, true, true, nullptr);
  });
}

extern "C" int rs_qwen_device_decode_batch(void* h, const StateId* parents, const uint32_t* tokens, size_t batch,
                                           StateId* outputs, float* logits, size_t logits_count, char* error,
                                           size_t capacity) {
  return guarded(error, capacity,
                 [&] { session_of(h).decode_batch(parents, tokens, batch, outputs, logits, logits_count); });
}

extern "C" int rs_qwen_device_ragged_step(void* h, const StateId* parents, const uint32_t* row_tokens, size_t rows,
                                          const uint32_t* tokens, size_t total_tokens, int flags, StateId* outputs,
                                          uint32_t* winners, float* margins, float* logits, size_t logits_count,
                                          char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    session_of(h).ragged(parents, row_tokens, rows, tokens, total_tokens, flags, outputs, winners, margins, logits,
                         logits_count);
  });
}

extern "C" int rs_qwen_device_release(void* h, const StateId* id, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!id) throw std::invalid_argument("release descriptor");
    session_of(h).release(*id);
  });
}

extern "C" int rs_qwen_device_snapshot(void* h, const StateId* id, float* output, size_t count, char* error,
                                       size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!id || !output) throw std::invalid_argument("snapshot descriptor");
    session_of(h).snapshot(*id, output, count);
  });
}

extern "C" int rs_qwen_device_hidden_snapshot(void* h, const StateId* id, float* output, size_t count, char* error,
                                              size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!id || !output) throw std::invalid_argument("hidden snapshot descriptor");
    session_of(h).hidden_snapshot(*id, output, count);
  });
}

extern "C" int rs_qwen_device_stats(void* h, uint64_t* output, size_t count, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!output) throw std::invalid_argument("stats capacity");
    std::vector<uint64_t> v(count);
    session_of(h).stats(v.data(), count);
    std::copy(v.begin(), v.end(), output);
  });
}

// Bridge diagnostics beside the reference's stats: [0] vocabulary-head passes
// of this session that fused the greedy selection (wrote no logits).
extern "C" int hb_session_info(void* h, uint64_t* output, size_t count, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!output || count < 1) throw std::invalid_argument("session info descriptor");
    output[0] = session_of(h).engine().fused_heads();
  });
}

extern "C" int rs_qwen_device_drain(void* h, uint64_t* invalidated, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!invalidated) throw std::invalid_argument("drain descriptor");
    *invalidated = session_of(h).drain();
  });
}

extern "C" int rs_qwen_device_mtp_attach(void* h, void* weights, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!h || !weights) throw std::invalid_argument("MTP attach descriptor");
    auto& s = session_of(h);
    s.mtp_attach(model_source(store_of(weights), 1).named);
  });
}

extern "C" int rs_qwen_device_mtp_step(void* h, const StateId* previous, const StateId* source, int draft_source,
                                       size_t row, const uint32_t* tokens, size_t count, StateId* output,
                                       float* logits, size_t logits_count, int diagnostics, char* error,
                                       size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!source || !output || diagnostics < 0 || diagnostics > 1) throw std::invalid_argument("MTP descriptor");
    *output = session_of(h).mtp_step(previous, *source, draft_source, row, tokens, count, logits, logits_count);
  });
}

extern "C" int rs_qwen_device_mtp_release(void* h, const StateId* id, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!id) throw std::invalid_argument("MTP release descriptor");
    session_of(h).mtp_release(*id);
  });
}

extern "C" int rs_qwen_device_mtp_snapshot(void* h, const StateId* id, float* output, size_t count, char* error,
                                           size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!id || !output) throw std::invalid_argument("MTP snapshot capacity");
    session_of(h).mtp_snapshot(*id, output, count);
  });
}

// Stateless forward over a full reference-layout state (qwen_forward_core):
// the state is imported as a version of a session kept with the store,
// stepped, snapshotted and released.
extern "C" int rs_qwen_forward(void* store, int gpu, const rs_qwen_config* config, const rs_qwen_layer* layers,
                               size_t layer_count, const uint32_t* tokens, size_t count, size_t offset,
                               const float* old_state, size_t old_count, float* new_state, size_t new_count,
                               float* logits, size_t logits_count, int projection_checks,
                               const uint32_t* projection_outputs, size_t projection_output_count, float* trace,
                               size_t trace_count, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!store || !config || !layers || !tokens || !new_state || !logits)
      throw std::invalid_argument("invalid model descriptor");
    if (gpu != 1) throw std::invalid_argument("rs_qwen_forward: this bridge runs on the GPU only (gpu = 1)");
    const rs_qwen_config& c = *config;
    validate_model(c, layers, layer_count);
    if (!count || count > size_t(c.chunk) || count > 8 || offset > size_t(c.context) ||
        offset + count > size_t(c.context) || logits_count != size_t(c.vocab))
      throw std::invalid_argument("model geometry/capacity");
    const size_t n = reference_state_count(c);
    if (new_count != n || (offset ? (old_count != n || !old_state) : old_count != 0))
      throw std::invalid_argument("model state length");
    if (projection_checks || projection_output_count || projection_outputs)
      throw std::invalid_argument("projection diagnostics are not built into this bridge");
    auto& w = store_of(store);
    const ModelSource m = model_source(w, 0);
    std::vector<uint8_t> key(sizeof(rs_qwen_config));
    std::memcpy(key.data(), config, sizeof(rs_qwen_config));
    if (!w.forward_cache || w.forward_key != key) {
      w.forward_cache.reset();
      w.forward_cache = std::shared_ptr<void>(new DeviceSession(c, 2, UINT64_MAX / 2, next_owner(), m.seed, m.named),
                                              [](void* p) { delete static_cast<DeviceSession*>(p); });
      w.forward_key = key;
    }
    auto& s = *static_cast<DeviceSession*>(w.forward_cache.get());
    std::vector<float> lg(logits_count), st(n), tr(trace_count);
    StateId parent{}, child{};
    bool have_parent = false, have_child = false;
    try {
      if (offset) {
        parent = s.import(offset, old_state, old_count);
        have_parent = true;
      }
      child = s.step(have_parent ? &parent : nullptr, offset, tokens, count, lg.data(), lg.size(),
                     trace_count ? tr.data() : nullptr, trace_count, false, false, nullptr);
      have_child = true;
      s.snapshot(child, st.data(), n);
    } catch (...) {
      if (have_child) s.release(child);
      if (have_parent) s.release(parent);
      throw;
    }
    s.release(child);
    if (have_parent) s.release(parent);
    std::copy(st.begin(), st.end(), new_state);
    std::copy(lg.begin(), lg.end(), logits);
    if (trace_count) std::copy(tr.begin(), tr.end(), trace);
  });
}

// DSpark drafter (native/mlx_bridge.h:120-133): not part of this bridge.
namespace {
const char* const kNoDspark = "the DSpark drafter is not built into this bridge";
}

extern "C" int rs_qwen_device_dspark_step(void*, const StateId*, size_t, const uint32_t*, size_t, StateId*, float*,
                                          size_t, int, char* error, size_t capacity) {
  report(error, capacity, kNoDspark);
  return -1;
}
extern "C" void* rs_qwen_dspark_create(void*, const char*, int, size_t, uint64_t, char* error, size_t capacity) {
  report(error, capacity, kNoDspark);
  return nullptr;
}
extern "C" void rs_qwen_dspark_destroy(void*) {}
extern "C" int rs_qwen_dspark_ingest(void*, const StateId*, const StateId*, StateId*, char* error, size_t capacity) {
  report(error, capacity, kNoDspark);
  return -1;
}
extern "C" int rs_qwen_dspark_propose(void*, const StateId*, uint32_t, size_t, uint32_t*, float*, size_t,
                                      char* error, size_t capacity) {
  report(error, capacity, kNoDspark);
  return -1;
}
extern "C" int rs_qwen_dspark_release(void*, const StateId*, char* error, size_t capacity) {
  report(error, capacity, kNoDspark);
  return -1;
}
extern "C" int rs_qwen_dspark_stats(void*, uint64_t*, size_t, char* error, size_t capacity) {
  report(error, capacity, kNoDspark);
  return -1;
}
extern "C" int rs_qwen_device_dspark_snapshot(void*, const StateId*, float*, size_t, char* error, size_t capacity) {
  report(error, capacity, kNoDspark);
  return -1;
}
