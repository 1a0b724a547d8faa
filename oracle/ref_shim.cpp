// Build-time shim that compiles the reference's own header-only scalar oracles
// (native/projection_reference.h, native/operator_reference.h,
// native/attention_reference.h, native/state_table.h) in place under
// /root/reference and exposes them through plain C entry points, so the tests
// can cross-check the C restatement in oracle.c against the reference code
// itself. Built into oracle/_ref/ (git-ignored) only where /root/reference is
// present; nothing from the reference is copied into this repository.
//
// TEST INFRASTRUCTURE ONLY.
#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

#include "attention_reference.h"
#include "operator_reference.h"
#include "projection_reference.h"
#include "state_table.h"

namespace {
template <class F>
int guarded(F f) {
  try {
    f();
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}
std::vector<float> vec(const float* p, size_t n) { return p ? std::vector<float>(p, p + n) : std::vector<float>(); }
void out(const std::vector<double>& v, double* dst) { std::memcpy(dst, v.data(), v.size() * sizeof(double)); }
}  // namespace

extern "C" {
int ref_projection(const float* x, size_t rows, const uint32_t* packed, const float* scales,
                   const float* biases, size_t outputs, size_t width, int group, int bits, double* y) {
  return guarded([&] {
    const size_t words = width * bits / 32, groups = width / group;
    auto r = projection_reference(vec(x, rows * width), std::vector<uint32_t>(packed, packed + outputs * words),
                                  vec(scales, outputs * groups), vec(biases, outputs * groups), rows, outputs,
                                  width, group, bits);
    out(r, y);
  });
}
int ref_embedding(const uint32_t* packed, const float* scales, const float* biases, size_t rows, size_t width,
                  int group, int bits, double* y) {
  return guarded([&] {
    const size_t words = width * bits / 32, groups = width / group;
    auto r = embedding_reference(std::vector<uint32_t>(packed, packed + rows * words), vec(scales, rows * groups),
                                 vec(biases, rows * groups), rows, width, group, bits);
    out(r, y);
  });
}
int ref_rms(const float* x, size_t n, const float* weight, size_t width, double eps, double* y) {
  return guarded([&] { out(scalar_reference::rms(vec(x, n), vec(weight, weight ? width : 0), width, eps), y); });
}
int ref_silu(const float* x, size_t n, double* y) {
  return guarded([&] { out(scalar_reference::silu(vec(x, n)), y); });
}
// x layout [heads][tokens][dim] as in the reference oracle.
int ref_rope(const float* x, int heads, int tokens, int dim, int rotary, int offset, double theta, double* y) {
  return guarded([&] {
    out(scalar_reference::rope(vec(x, size_t(heads) * tokens * dim), heads, tokens, dim, rotary, offset, theta), y);
  });
}
int ref_delta(const float* qkv, const float* history, const float* conv, const float* a, const float* b,
              const float* alog, const float* dt, const float* initial, int tokens, int hk, int hv, int dk, int dv,
              int kernel, double* activated, double* history_out, double* output, double* state) {
  return guarded([&] {
    const size_t channels = size_t(2) * hk * dk + size_t(hv) * dv;
    auto r = scalar_reference::delta(vec(qkv, tokens * channels), vec(history, (kernel - 1) * channels),
                                     vec(conv, channels * kernel), vec(a, size_t(tokens) * hv),
                                     vec(b, size_t(tokens) * hv), vec(alog, hv), vec(dt, hv),
                                     vec(initial, size_t(hv) * dv * dk), tokens, hk, hv, dk, dv, kernel);
    out(r.activated, activated);
    out(r.history, history_out);
    out(r.output, output);
    out(r.state, state);
  });
}
int ref_routing(const float* logits, const int32_t* selected, int rows, int experts, int top, double* weights) {
  return guarded([&] {
    auto r = scalar_reference::routing(vec(logits, size_t(rows) * experts),
                                       std::vector<int32_t>(selected, selected + size_t(rows) * top), rows, experts,
                                       top);
    out(r.weights, weights);
  });
}
// q [heads][tokens][dim], k/v [kv_heads][offset+tokens][dim].
int ref_attention(const float* q, const float* k, const float* v, int heads, int kv_heads, int tokens, int offset,
                  int dim, double* y) {
  return guarded([&] {
    const size_t n = size_t(offset) + tokens;
    out(attention_reference(vec(q, size_t(heads) * tokens * dim), vec(k, size_t(kv_heads) * n * dim),
                            vec(v, size_t(kv_heads) * n * dim), heads, kv_heads, tokens, offset, dim),
        y);
  });
}

// StateTable<int> driven by scripted operations for differential tests.
void* ref_table_create(uint64_t owner, size_t slots, uint64_t bytes) {
  try {
    return new StateTable<int>(owner, slots, bytes);
  } catch (const std::exception&) {
    return nullptr;
  }
}
void ref_table_destroy(void* t) { delete static_cast<StateTable<int>*>(t); }
int ref_table_reserve(void* t, uint64_t position, uint64_t bytes, StateId* id) {
  return guarded([&] { *id = static_cast<StateTable<int>*>(t)->reserve(position, bytes); });
}
int ref_table_publish(void* t, const StateId* id, int value) {
  return guarded([&] { static_cast<StateTable<int>*>(t)->publish(*id, value); });
}
int ref_table_get(void* t, const StateId* id, int* value) {
  return guarded([&] { *value = static_cast<StateTable<int>*>(t)->get(*id); });
}
int ref_table_rollback(void* t, const StateId* id) {
  return guarded([&] { static_cast<StateTable<int>*>(t)->rollback(*id); });
}
int ref_table_release(void* t, const StateId* id) {
  return guarded([&] { static_cast<StateTable<int>*>(t)->release(*id); });
}
uint64_t ref_table_bytes(void* t) { return static_cast<StateTable<int>*>(t)->bytes(); }
size_t ref_table_residents(void* t) { return static_cast<StateTable<int>*>(t)->residents(); }
void ref_table_clear(void* t) { static_cast<StateTable<int>*>(t)->clear(); }
}
