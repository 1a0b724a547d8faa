// Decode engine for the hybrid Qwen decoder (see engine.h).
//
// Layer program (Qwen::attention / Qwen::recurrent / Qwen::moe and the layer
// loop of qwen_forward_core, native/qwen_model.inc:101-206, 321-352):
//   h = rms(x, input_layernorm)
//   x += attention(h) | deltanet(h)         (projection output accumulated into x)
//   h = rms(x, post_attention_layernorm)
//   x += moe(h) + sigmoid(shared_gate(h)) * shared_expert(h)
// The residual stream x is fp32; every matmul input is bf16.
#include "engine.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <numeric>
#include <random>

#include "moe.h"
#include "norm.h"
#include "ops.h"
#include "pack.h"
#include "qmm.h"
#include "select.h"
#include "synth.h"

namespace hb {

namespace {
constexpr int kMoeChunk = 256;  // tokens per routing workgroup (top-10 -> 2560 pairs)
constexpr float kWeightStd = 0.02f;
size_t round256(size_t b) { return (b + 255) / 256 * 256; }
}  // namespace

Geom geom_from(const rs_qwen_config& c) {
  if (c.activation_precision != 0) throw std::invalid_argument(kFp32ProfileRefused);
  Geom g{};
  g.H = c.hidden;
  g.L = c.layers;
  g.V = c.vocab;
  g.Hq = c.q_heads;
  g.Hkv = c.kv_heads;
  g.D = c.head_dim;
  g.Hk = c.key_heads;
  g.Hv = c.value_heads;
  g.Dk = c.key_dim;
  g.Dv = c.value_dim;
  g.conv = c.conv;
  g.interval = c.interval;
  g.E = c.experts;
  g.top = c.top;
  g.I = c.intermediate;
  g.rotary = c.rope_dims;
  g.eps = c.epsilon;
  g.theta = c.theta;
  return g;
}

int tensor_id(int layer, int slot) { return 16 + layer * kTLayerStride + slot; }
int tensor_id_global(int which) { return which; }

int StepRows::total() const { return std::accumulate(row_tokens.begin(), row_tokens.end(), 0); }

void* Engine::dalloc(size_t bytes, size_t* counter) {
  void* p = nullptr;
  HB_CHECK(hipMalloc(&p, round256(std::max<size_t>(bytes, 4))));
  allocations_.push_back(p);
  if (counter) *counter += bytes;
  return p;
}

void Engine::tensor_shape(int id, int& N, int& K, bool& q4) const {
  const Geom& g = g_;
  q4 = false;
  K = 0;
  if (id < 16) {
    switch (id) {
      case 0: N = g.V; K = g.H; q4 = true; return;
      case 1: case 3: case 4: case 6: N = g.H; return;
      case 2: N = g.vocab_rows(); K = g.H; q4 = true; return;
      case 5: N = g.H; K = 2 * g.H; q4 = true; return;
    }
    throw std::invalid_argument("unknown tensor id");
  }
  const int layer = (id - 16) / kTLayerStride, slot = (id - 16) % kTLayerStride;
  require(layer <= g.L, "tensor id: layer out of range");
  const bool attn = layer == g.L ? true : g.attn(layer);
  switch (slot) {
    case kTInNorm: case kTPostNorm: N = g.H; return;
    case kTInProj: N = attn ? g.attn_in_rows() : g.dn_in_rows(); K = g.H; q4 = true; return;
    case kTOutProj: N = g.H; K = attn ? g.Hq * g.D : g.Hv * g.Dv; q4 = true; return;
    case kTConvW: N = g.conv_channels() * g.conv; return;
    case kTALog: case kTDtBias: N = g.Hv; return;
    case kTGNorm: N = g.Dv; return;
    case kTQNorm: case kTKNorm: N = g.D; return;
    case kTRouter: N = g.router_rows(); K = g.H; q4 = true; return;
    case kTGateUp: N = (g.E + 1) * 2 * g.I; K = g.H; q4 = true; return;
    case kTDown: N = (g.E + 1) * g.H; K = g.I; q4 = true; return;
  }
  throw std::invalid_argument("unknown tensor slot");
}

static int vector_kind(int id) {
  if (id < 16) return 0;
  const int slot = (id - 16) % kTLayerStride;
  if (slot == kTConvW) return 1;
  if (slot == kTALog) return 2;
  if (slot == kTDtBias) return 3;
  return 0;
}

void Engine::export_tensor(int id, void* w, void* s, void* b) {
  if (named_) {
    export_named(id, w, s, b);
    return;
  }
  int N, K;
  bool q4;
  tensor_shape(id, N, K, q4);
  const uint64_t sd = seed_ * 1000003ull + uint64_t(id);
  if (q4) {
    random_q4(sd, N, K, kWeightStd, static_cast<uint32_t*>(w), static_cast<bf16_t*>(s), static_cast<bf16_t*>(b),
              stream_);
  } else {
    float* out = static_cast<float*>(w);
    switch (vector_kind(id)) {
      case 0: random_normal(sd, N, 0.02f, 1.f, 0, out, stream_); break;
      case 1: random_normal(sd, N, 0.3f, 0.f, 0, out, stream_); break;
      case 2: random_uniform(sd, N, 0.f, 1.f, 0, out, stream_); break;
      default: HB_CHECK(hipMemsetAsync(out, 0, size_t(N) * 4, stream_)); break;
    }
  }
}

void Engine::gen_slot(Q4T& m, GSlot& gs, int id, int N, int K) {
  gs = generic_slot(id);
  if (gs.on()) {  // read in place from the store; the tiled form stays empty
    m.N = N;
    m.K = K;
    return;
  }
  gen_q4(m, id, N, K, kWeightStd);
}

void Engine::project(const Q4T& m, const GSlot& g, const bf16_t* x, int M, void* y, int out_mode, int ldy,
                     const float* gsum) {
  if (!g.on()) {
    qmm(x, M, m.K, m.w, m.sb, nullptr, m.N, 64, 4, kLayoutQ4Tiled, y, out_mode, ldy, stream_, gsum);
    return;
  }
  for (const QMod& q : g.mods) {
    void* yc = out_mode == 0 ? static_cast<void*>(static_cast<bf16_t*>(y) + q.col)
                             : static_cast<void*>(static_cast<float*>(y) + q.col);
    qmm(x, M, q.K, q.w, q.s, q.b, q.rows, q.group, q.bits, kLayoutMlx, yc, out_mode, ldy, stream_);
  }
}

void Engine::embed(int T) {
  if (w_.g_emb.on())
    embed_generic(d_tokens_, T, w_.g_emb.mods[0], x_, stream_);
  else
    embed_gather(d_tokens_, T, w_.emb_w, w_.emb_s, w_.emb_b, g_.H, x_, stream_);
}

void Engine::gen_q4(Q4T& m, int id, int N, int K, float) {
  m.N = N;
  m.K = K;
  m.w = static_cast<uint32_t*>(dalloc(size_t(N) * K / 2, &weight_bytes_));
  m.sb = static_cast<bf16_t*>(dalloc(size_t(N) * (K / 64) * 4, &weight_bytes_));
  require(size_t(N) * K / 2 <= gen_cap_, "weight generation scratch too small");
  export_tensor(id, gen_w_, gen_s_, gen_b_);
  q4_tile(gen_w_, gen_s_, gen_b_, m.w, m.sb, N, K, stream_);
}

float* Engine::gen_vec(int id, int n, int) {
  float* p = static_cast<float*>(dalloc(size_t(n) * 4, &weight_bytes_));
  export_tensor(id, p, nullptr, nullptr);
  return p;
}

void Engine::alloc_weights() {
  const Geom& g = g_;
  // scratch for the largest checkpoint-layout tensor
  size_t largest = 0;
  for (int id = 0; id < 16 + (g.L + 1) * kTLayerStride; ++id) {
    int N, K;
    bool q4;
    try {
      tensor_shape(id, N, K, q4);
    } catch (const std::exception&) {
      continue;
    }
    if (q4) largest = std::max(largest, size_t(N) * K / 2);
  }
  gen_cap_ = largest;
  gen_w_ = static_cast<uint32_t*>(dalloc(largest, nullptr));
  gen_s_ = static_cast<bf16_t*>(dalloc(largest / 16, nullptr));
  gen_b_ = static_cast<bf16_t*>(dalloc(largest / 16, nullptr));

  w_.g_emb = generic_slot(tensor_id_global(0));
  if (!w_.g_emb.on()) {
    w_.emb_w = static_cast<uint32_t*>(dalloc(size_t(g.V) * g.H / 2, &weight_bytes_));
    w_.emb_s = static_cast<bf16_t*>(dalloc(size_t(g.V) * (g.H / 64) * 2, &weight_bytes_));
    w_.emb_b = static_cast<bf16_t*>(dalloc(size_t(g.V) * (g.H / 64) * 2, &weight_bytes_));
    export_tensor(tensor_id_global(0), w_.emb_w, w_.emb_s, w_.emb_b);
  }

  for (int l = 0; l < g.L; ++l) w_.layers.push_back(make_layer(l, g.attn(l)));
  w_.final_norm = gen_vec(tensor_id_global(1), g.H, 0);
  gen_slot(w_.lm_head, w_.g_head, tensor_id_global(2), g.vocab_rows(), g.H);
  if (mtp_) build_mtp_weights();
  HB_CHECK(hipStreamSynchronize(stream_));
}

LayerW Engine::make_layer(int l, bool attn) {
  const Geom& g = g_;
  LayerW L;
  L.attn = attn;
  L.in_norm = gen_vec(tensor_id(l, kTInNorm), g.H, 0);
  L.post_norm = gen_vec(tensor_id(l, kTPostNorm), g.H, 0);
  gen_slot(L.in_proj, L.g_in, tensor_id(l, kTInProj), attn ? g.attn_in_rows() : g.dn_in_rows(), g.H);
  gen_slot(L.out_proj, L.g_out, tensor_id(l, kTOutProj), g.H, attn ? g.Hq * g.D : g.Hv * g.Dv);
  if (attn) {
    L.q_norm = gen_vec(tensor_id(l, kTQNorm), g.D, 0);
    L.k_norm = gen_vec(tensor_id(l, kTKNorm), g.D, 0);
  } else {
    L.conv_w = gen_vec(tensor_id(l, kTConvW), g.conv_channels() * g.conv, 1);
    L.a_log = gen_vec(tensor_id(l, kTALog), g.Hv, 2);
    L.dt_bias = gen_vec(tensor_id(l, kTDtBias), g.Hv, 3);
    L.gnorm = gen_vec(tensor_id(l, kTGNorm), g.Dv, 0);
  }
  gen_slot(L.router, L.g_router, tensor_id(l, kTRouter), g.router_rows(), g.H);
  gen_slot(L.gate_up, L.g_gate_up, tensor_id(l, kTGateUp), (g.E + 1) * 2 * g.I, g.H);
  gen_slot(L.down, L.g_down, tensor_id(l, kTDown), (g.E + 1) * g.H, g.I);
  HB_CHECK(hipStreamSynchronize(stream_));
  return L;
}

void Engine::build_mtp_weights() {
  const Geom& g = g_;
  w_.mtp_pre_e = gen_vec(tensor_id_global(3), g.H, 0);
  w_.mtp_pre_h = gen_vec(tensor_id_global(4), g.H, 0);
  if (named_mtp_) {
    // the sidecar's fc may be a dense BF16 matrix (native_mtp.rs:121-123)
    const auto it = named_mtp_->arrays.find("language_model.mtp.fc.weight");
    if (it != named_mtp_->arrays.end() && it->second->dtype == kBF16) {
      const Tensor& t = *it->second;
      require(t.shape == std::vector<int32_t>{g.H, 2 * g.H}, "checkpoint: MTP dense fc must be [hidden, 2 hidden]");
      w_.mtp_fc_dense = static_cast<const bf16_t*>(t.data);
    }
  }
  if (!w_.mtp_fc_dense) gen_slot(w_.mtp_fc, w_.g_mtp_fc, tensor_id_global(5), g.H, 2 * g.H);
  w_.mtp_norm = gen_vec(tensor_id_global(6), g.H, 0);
  w_.mtp_layer = make_layer(g.L, true);
  w_.has_mtp = true;
}

void Engine::alloc_kv_pool() {
  const Geom& g = g_;
  const size_t kv_elems = size_t(pages_) * g.Hkv * kPage * g.D;
  kc_.push_back(static_cast<bf16_t*>(dalloc(kv_elems * 2, &state_bytes_)));
  vc_.push_back(static_cast<bf16_t*>(dalloc(kv_elems * 2, &state_bytes_)));
  HB_CHECK(hipMemsetAsync(kc_.back(), 0, kv_elems * 2, stream_));
  HB_CHECK(hipMemsetAsync(vc_.back(), 0, kv_elems * 2, stream_));
}

void Engine::sync_pool_table() {
  std::vector<bf16_t*> t;
  for (size_t i = 0; i < kc_.size(); ++i) {
    t.push_back(kc_[i]);
    t.push_back(vc_[i]);
  }
  HB_CHECK(hipStreamSynchronize(stream_));
  HB_CHECK(hipMemcpy(d_pools_, t.data(), t.size() * sizeof(bf16_t*), hipMemcpyHostToDevice));
}

void Engine::enable_mtp(std::shared_ptr<const NamedWeights> named_mtp) {
  require(!w_.has_mtp, "engine: the MTP head is already built");
  require(!named_ == !named_mtp, "engine: the MTP head's weights come from the target model's kind of source");
  named_mtp_ = std::move(named_mtp);
  build_mtp_weights();
  alloc_kv_pool();
  sync_pool_table();
  mtp_ = true;
}

void Engine::write_block_row(int row, const std::vector<int32_t>& pages) {
  require(row >= 0 && row < max_rows_ && int(pages.size()) <= max_pages_, "block table row");
  for (int32_t p : pages) require(p >= 0 && p < pages_, "block table: page outside the pool");
  if (pages.empty()) return;
  HB_CHECK(hipStreamSynchronize(stream_));
  HB_CHECK(hipMemcpy(block_table_ + size_t(row) * max_pages_, pages.data(), pages.size() * 4, hipMemcpyHostToDevice));
}

void Engine::copy_kv_pages(bool mtp, const std::vector<int32_t>& pairs) {
  const int n = int(pairs.size() / 2);
  if (n == 0) return;
  require(pairs.size() % 2 == 0 && n <= pairs_cap_, "copy_kv_pages: pair list");
  require(!mtp || w_.has_mtp, "copy_kv_pages: no MTP pool");
  for (int32_t p : pairs) require(p >= 0 && p < pages_, "copy_kv_pages: page outside the pool");
  HB_CHECK(hipStreamSynchronize(stream_));
  HB_CHECK(hipMemcpy(d_pairs_, pairs.data(), pairs.size() * 4, hipMemcpyHostToDevice));
  const Geom& g = g_;
  const int first = mtp ? 2 * n_attn_ : 0, count = mtp ? 2 : 2 * n_attn_;
  if (count == 0) return;
  copy_pages(d_pools_ + first, count, d_pairs_, n, g.Hkv * kPage * g.D, nullptr, stream_);
}

void Engine::read_recurrent(int dn, int slot, int hist_off, float* conv, float* state) {
  const Geom& g = g_;
  require(dn >= 0 && dn < int(dn_state_.size()) && slot >= 0 && slot < 2 * max_rows_ && hist_off >= 0 &&
              hist_off <= max_row_tokens_,
          "read_recurrent: layer / slot");
  const int C = g.conv_channels(), H = g.conv - 1;
  const size_t window_row = size_t(g.conv - 1 + max_row_tokens_) * C;
  HB_CHECK(hipStreamSynchronize(stream_));
  std::vector<bf16_t> w(size_t(H) * C);
  HB_CHECK(hipMemcpy(w.data(), dn_window_[dn] + size_t(slot) * window_row + size_t(hist_off) * C, w.size() * 2,
                     hipMemcpyDeviceToHost));
  for (size_t i = 0; i < w.size(); ++i) conv[i] = bf16_to_f32(w[i]);
  // device layout [Hv][key c][value i] -> reference [Hv][value i][key c]
  const size_t per = size_t(g.Dk) * g.Dv;
  std::vector<float> s(size_t(g.Hv) * per);
  HB_CHECK(hipMemcpy(s.data(), dn_state_[dn] + size_t(slot) * g.Hv * per, s.size() * 4, hipMemcpyDeviceToHost));
  for (int h = 0; h < g.Hv; ++h)
    for (int c = 0; c < g.Dk; ++c)
      for (int i = 0; i < g.Dv; ++i) state[h * per + size_t(i) * g.Dk + c] = s[h * per + size_t(c) * g.Dv + i];
}

void Engine::write_recurrent(int dn, int slot, const float* conv, const float* state) {
  const Geom& g = g_;
  require(dn >= 0 && dn < int(dn_state_.size()) && slot >= 0 && slot < 2 * max_rows_, "write_recurrent: layer / slot");
  const int C = g.conv_channels(), H = g.conv - 1;
  const size_t window_row = size_t(g.conv - 1 + max_row_tokens_) * C;
  std::vector<bf16_t> w(size_t(H) * C);
  for (size_t i = 0; i < w.size(); ++i) w[i] = f32_to_bf16(conv[i]);
  const size_t per = size_t(g.Dk) * g.Dv;
  std::vector<float> s(size_t(g.Hv) * per);
  for (int h = 0; h < g.Hv; ++h)
    for (int c = 0; c < g.Dk; ++c)
      for (int i = 0; i < g.Dv; ++i) s[h * per + size_t(c) * g.Dv + i] = state[h * per + size_t(i) * g.Dk + c];
  HB_CHECK(hipStreamSynchronize(stream_));
  HB_CHECK(hipMemcpy(dn_window_[dn] + size_t(slot) * window_row, w.data(), w.size() * 2, hipMemcpyHostToDevice));
  HB_CHECK(hipMemcpy(dn_state_[dn] + size_t(slot) * g.Hv * per, s.data(), s.size() * 4, hipMemcpyHostToDevice));
}

void Engine::write_kv(int pool, const std::vector<int32_t>& pages, int position, int context, const float* k,
                      const float* v) {
  const Geom& g = g_;
  require(pool >= 0 && pool < int(kc_.size()) && position >= 0 && position <= context &&
              int(pages.size()) * kPage >= position,
          "write_kv: pool / pages");
  for (int32_t p : pages) require(p >= 0 && p < pages_, "write_kv: page outside the pool");
  const size_t plane = size_t(context) * g.D, page_elems = size_t(g.Hkv) * kPage * g.D;
  const int n = (position + kPage - 1) / kPage;
  std::vector<bf16_t> kp(page_elems), vp(page_elems);
  HB_CHECK(hipStreamSynchronize(stream_));
  for (int j = 0; j < n; ++j) {
    std::fill(kp.begin(), kp.end(), bf16_t(0));
    std::fill(vp.begin(), vp.end(), bf16_t(0));
    for (int t = 0; t < kPage && j * kPage + t < position; ++t) {
      const size_t pos = size_t(j) * kPage + t;
      for (int h = 0; h < g.Hkv; ++h)
        for (int d = 0; d < g.D; ++d) {
          kp[(size_t(h) * kPage + t) * g.D + d] = f32_to_bf16(k[h * plane + pos * g.D + d]);
          vp[(size_t(h) * g.D + d) * kPage + t] = f32_to_bf16(v[h * plane + pos * g.D + d]);
        }
    }
    HB_CHECK(hipMemcpy(kc_[pool] + size_t(pages[j]) * page_elems, kp.data(), page_elems * 2, hipMemcpyHostToDevice));
    HB_CHECK(hipMemcpy(vc_[pool] + size_t(pages[j]) * page_elems, vp.data(), page_elems * 2, hipMemcpyHostToDevice));
  }
}

void Engine::read_kv(int pool, const std::vector<int32_t>& pages, int position, int context, float* k, float* v) {
  const Geom& g = g_;
  require(pool >= 0 && pool < int(kc_.size()) && position >= 0 && position <= context &&
              int(pages.size()) * kPage >= position,
          "read_kv: pool / pages");
  for (int32_t p : pages) require(p >= 0 && p < pages_, "read_kv: page outside the pool");
  const size_t plane = size_t(context) * g.D;
  std::fill(k, k + g.Hkv * plane, 0.f);
  std::fill(v, v + g.Hkv * plane, 0.f);
  const int n = (position + kPage - 1) / kPage;
  if (n == 0) return;
  const size_t page_elems = size_t(g.Hkv) * kPage * g.D;
  HB_CHECK(hipStreamSynchronize(stream_));
  std::vector<bf16_t> kp(page_elems), vp(page_elems);
  for (int j = 0; j < n; ++j) {
    HB_CHECK(hipMemcpy(kp.data(), kc_[pool] + size_t(pages[j]) * page_elems, page_elems * 2, hipMemcpyDeviceToHost));
    HB_CHECK(hipMemcpy(vp.data(), vc_[pool] + size_t(pages[j]) * page_elems, page_elems * 2, hipMemcpyDeviceToHost));
    for (int t = 0; t < kPage && j * kPage + t < position; ++t) {
      const size_t pos = size_t(j) * kPage + t;
      for (int h = 0; h < g.Hkv; ++h)
        for (int d = 0; d < g.D; ++d) {
          // K page [Hkv][16][D], V page [Hkv][D][16]
          k[h * plane + pos * g.D + d] = bf16_to_f32(kp[(size_t(h) * kPage + t) * g.D + d]);
          v[h * plane + pos * g.D + d] = bf16_to_f32(vp[(size_t(h) * g.D + d) * kPage + t]);
        }
    }
  }
}

Engine::Engine(const rs_qwen_config& cfg, int max_rows, int max_context, int max_row_tokens, int max_step_tokens,
               uint64_t seed, bool mtp, std::shared_ptr<const NamedWeights> named,
               std::shared_ptr<const NamedWeights> named_mtp)
    : g_(geom_from(cfg)),
      seed_(seed),
      named_(std::move(named)),
      named_mtp_(std::move(named_mtp)),
      max_rows_(max_rows),
      max_context_(max_context),
      max_row_tokens_(max_row_tokens),
      max_step_tokens_(max_step_tokens),
      mtp_(mtp) {
  const Geom& g = g_;
  require(max_rows > 0 && max_rows <= 1024 && max_context > 0 && max_row_tokens > 0 && max_step_tokens > 0,
          "engine: invalid capacity");
  require(g.H % 128 == 0 && g.I % 128 == 0 && g.D == 256 && g.Dk == 128 && g.Dv == 128,
          "engine: hidden and intermediate must be multiples of 128, head_dim 256, key/value dims 128");
  require(g.Hq % g.Hkv == 0 && g.Hv % g.Hk == 0 && g.interval > 0 && g.L > 0,
          "engine: head grouping / layer program");
  require(g.V % 16 == 0 && (g.Hq * g.D) % 128 == 0 && (g.Hv * g.Dv) % 128 == 0, "engine: vocabulary / widths");
  require(g.conv_channels() % 256 == 0 && (g.Hk * g.Dk) % 256 == 0 && g.Hv <= 256,
          "engine: conv channels and key width must be multiples of 256");
  require(g.E >= 1 && g.top >= 1 && g.top <= g.E && g.top <= 16, "engine: experts / top");
  require(cfg.shared == 0 || cfg.shared == cfg.intermediate, "engine: the shared expert width must equal the expert width");
  require(!mtp || !named_ == !named_mtp_, "engine: a checkpoint model's MTP head needs the MTP sidecar's tensors");
  if (named_) {
    // a checkpoint's default quantization; synthetic weights are 4-bit g64
    require((cfg.group == 32 || cfg.group == 64 || cfg.group == 128) &&
                (cfg.bits == 2 || cfg.bits == 3 || cfg.bits == 4 || cfg.bits == 5 || cfg.bits == 6 || cfg.bits == 8),
            "engine: invalid model quantization");
    qgroup_ = cfg.group;
    qbits_ = cfg.bits;
  }
  HB_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  alloc_weights();

  // pools
  int n_attn = 0;
  for (int l = 0; l < g.L; ++l) n_attn += g.attn(l);
  const int n_dn = g.L - n_attn;
  const int slots = 2 * max_rows;
  max_pages_ = (max_context + kPage - 1) / kPage;
  pages_ = max_rows * max_pages_;
  n_attn_ = n_attn;
  for (int i = 0; i < n_attn + (mtp ? 1 : 0); ++i) alloc_kv_pool();
  d_pools_ = static_cast<bf16_t**>(dalloc(size_t(2) * (n_attn + 1) * sizeof(bf16_t*), nullptr));
  pairs_cap_ = std::max(max_rows, max_pages_);
  d_pairs_ = static_cast<int32_t*>(dalloc(size_t(2) * pairs_cap_ * 4, nullptr));
  sync_pool_table();
  const int C = g.conv_channels();
  for (int i = 0; i < n_dn; ++i) {
    dn_state_.push_back(static_cast<float*>(dalloc(size_t(slots) * g.Hv * g.Dv * g.Dk * 4, &state_bytes_)));
    dn_window_.push_back(
        static_cast<bf16_t*>(dalloc(size_t(slots) * (g.conv - 1 + max_row_tokens) * C * 2, &state_bytes_)));
    dn_log_k_.push_back(static_cast<float*>(dalloc(size_t(slots) * max_row_tokens * g.Hv * g.Dk * 4, &state_bytes_)));
    dn_log_d_.push_back(static_cast<float*>(dalloc(size_t(slots) * max_row_tokens * g.Hv * g.Dv * 4, &state_bytes_)));
    dn_log_g_.push_back(static_cast<float*>(dalloc(size_t(slots) * max_row_tokens * g.Hv * 4, &state_bytes_)));
    HB_CHECK(hipMemsetAsync(dn_state_.back(), 0, size_t(slots) * g.Hv * g.Dv * g.Dk * 4, stream_));
    HB_CHECK(hipMemsetAsync(dn_window_.back(), 0, size_t(slots) * (g.conv - 1 + max_row_tokens) * C * 2, stream_));
  }
  // block table: disjoint pages per sequence slot, in a seeded random order
  std::vector<int32_t> perm(pages_);
  std::iota(perm.begin(), perm.end(), 0);
  std::mt19937_64 rng(seed ^ 0x5EEDull);
  std::shuffle(perm.begin(), perm.end(), rng);
  block_table_ = static_cast<int32_t*>(dalloc(size_t(pages_) * 4, nullptr));
  HB_CHECK(hipMemcpy(block_table_, perm.data(), size_t(pages_) * 4, hipMemcpyHostToDevice));

  // step tables
  const int Tm = max_step_tokens, R = max_rows;
  auto ialloc = [&](size_t n) { return static_cast<int32_t*>(dalloc(n * 4, &work_bytes_)); };
  // the per-row tables and the tokens form one block uploaded by one copy:
  // [row_tokens | positions | seq | src | dst | hist_off | log_count] (R each), tokens (Tm)
  d_tab_ = ialloc(size_t(7) * R + Tm);
  d_row_tokens_ = d_tab_;
  d_positions_ = d_tab_ + R;
  d_seq_ = d_tab_ + 2 * R;
  d_src_ = d_tab_ + 3 * R;
  d_dst_ = d_tab_ + 4 * R;
  d_hist_ = d_tab_ + 5 * R;
  d_logc_ = d_tab_ + 6 * R;
  d_tokens_ = reinterpret_cast<uint32_t*>(d_tab_ + 7 * R);
  d_cu_ = ialloc(R + 1);
  d_ctx_ = ialloc(R);
  d_status_ = ialloc(1);
  d_tok_row_ = ialloc(Tm);
  d_tok_pos_ = ialloc(Tm);
  d_slot_ = ialloc(Tm);
  d_sel_idx_ = ialloc(Tm);
  d_bt_rows_ = ialloc(size_t(R) * max_pages_);
  h_pinned_cap_ = size_t(8) * R + 4 * size_t(Tm) + 64;
  HB_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_pinned_), h_pinned_cap_ * 4 * kStageSlots, hipHostMallocDefault));
  for (hipEvent_t& e : stage_ev_) HB_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));

  // work buffers
  auto falloc = [&](size_t n) { return static_cast<float*>(dalloc(n * 4, &work_bytes_)); };
  auto balloc = [&](size_t n) { return static_cast<bf16_t*>(dalloc(n * 2, &work_bytes_)); };
  const int proj_w = std::max({g.dn_in_rows(), g.attn_in_rows(), 2 * g.H});
  x_ = falloc(size_t(Tm) * g.H);
  hn_f32_ = falloc(size_t(Tm) * g.H);
  mtp_h_f32_ = falloc(size_t(Tm) * g.H);
  mtp_in_f32_ = falloc(size_t(Tm) * g.H);
  h_ = balloc(size_t(Tm) * g.H);
  hn_ = balloc(size_t(Tm) * g.H);
  sel_h_ = balloc(size_t(Tm) * g.H);
  proj_ = balloc(size_t(Tm) * proj_w);
  q_ = balloc(size_t(Tm) * g.Hq * g.D);
  aout_ = balloc(size_t(Tm) * g.Hq * g.D);
  const size_t awo = attn_work_floats_o(R, g.Hkv, g.D, max_row_tokens, g.Hq / g.Hkv, max_context, attn_split_);
  attn_wo_ = falloc(awo);
  attn_wml_ = falloc(awo / g.D * 2);
  {
    const int rgs = (max_row_tokens * (g.Hq / g.Hkv) + 15) / 16;
    const int splits = (max_context + attn_split_ - 1) / attn_split_;
    attn_plan_ = static_cast<int32_t*>(dalloc(attn_plan_ints(R, g.Hkv, rgs, splits) * 4, &work_bytes_));
  }
  gq_ = falloc(size_t(Tm) * g.Hk * g.Dk);
  gk_ = falloc(size_t(Tm) * g.Hk * g.Dk);
  gv_ = falloc(size_t(Tm) * g.Hv * g.Dv);
  gg_ = falloc(size_t(Tm) * g.Hv);
  gb_ = falloc(size_t(Tm) * g.Hv);
  if (g.H % 64 == 0) hgs_ = falloc(size_t(Tm) * (g.H / 64));
  y_ = balloc(size_t(Tm) * g.Hv * g.Dv);
  const int chunk = std::min(Tm, kMoeChunk);
  rlog_ = falloc(size_t(chunk) * g.router_rows());
  moe_idx_ = ialloc(size_t(chunk) * g.top);
  moe_w_ = falloc(size_t(chunk) * g.top);
  moe_counts_ = ialloc(g.E);
  moe_offsets_ = ialloc(g.E + 1);
  moe_order_ = ialloc(size_t(chunk) * g.top);
  moe_inverse_ = ialloc(size_t(chunk) * g.top);
  moe_items_ = ialloc(moe_items_capacity(chunk, g.E, g.top));
  act_ = balloc(size_t(chunk) * (g.top + 1) * g.I);
  dout_ = balloc(size_t(chunk) * (g.top + 1) * g.H);
  logits_ = falloc(size_t(Tm) * g.vocab_rows());
  // selection results in one block [winners | margins | status] (Tm each), read back by one copy
  sel_block_ = ialloc(size_t(3) * Tm);
  winners_ = reinterpret_cast<uint32_t*>(sel_block_);
  margins_ = reinterpret_cast<float*>(sel_block_ + Tm);
  sel_status_ = sel_block_ + 2 * Tm;
  sel_ws_ = dalloc(argmax_workspace_bytes(Tm, g.V), &work_bytes_);
  sel_part_bytes_ = qmm_select_workspace(std::min(Tm, 256), g.vocab_rows());
  sel_part_ = dalloc(sel_part_bytes_, &work_bytes_);
  HB_CHECK(hipStreamSynchronize(stream_));
}

Engine::~Engine() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (Probe& p : probe_)
    for (hipEvent_t e : p.ev) (void)hipEventDestroy(e);
  for (void* p : allocations_) (void)hipFree(p);
  for (hipEvent_t e : stage_ev_)
    if (e) (void)hipEventDestroy(e);
  if (h_pinned_) (void)hipHostFree(h_pinned_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

int32_t* Engine::stage_begin() {
  const int k = stage_next_;
  stage_next_ = (k + 1) % kStageSlots;
  if (stage_used_[k]) HB_CHECK(hipEventSynchronize(stage_ev_[k]));  // its last copies have executed
  stage_cur_ = k;
  return h_pinned_ + size_t(k) * h_pinned_cap_;
}

void Engine::stage_end() {
  HB_CHECK(hipEventRecord(stage_ev_[stage_cur_], stream_));
  stage_used_[stage_cur_] = true;
}

void Engine::upload_tables(const StepRows& s) {
  const int B = s.rows, T = s.total();
  require(B > 0 && B <= max_rows_, "step: row count outside 1..max_rows");
  require(T > 0 && T <= max_step_tokens_, "step: token count outside 1..max_step_tokens");
  require(int(s.row_tokens.size()) == B && int(s.positions.size()) == B && int(s.seq.size()) == B &&
              int(s.src_slot.size()) == B && int(s.dst_slot.size()) == B && int(s.hist_off.size()) == B &&
              int(s.log_count.size()) == B && int(s.tokens.size()) == T,
          "step: table sizes");
  for (int r = 0; r < B; ++r) {
    require(s.row_tokens[r] >= 0 && s.row_tokens[r] <= max_row_tokens_, "step: row token count");
    require(s.positions[r] >= 0 && s.positions[r] + s.row_tokens[r] <= max_context_, "step: context capacity");
    require(s.seq[r] >= 0 && s.seq[r] < max_rows_, "step: sequence slot");
    require(s.src_slot[r] >= 0 && s.src_slot[r] < 2 * max_rows_ && s.dst_slot[r] >= 0 &&
                s.dst_slot[r] < 2 * max_rows_,
            "step: state slot");
    require(s.hist_off[r] >= 0 && s.hist_off[r] <= max_row_tokens_ && s.log_count[r] >= 0 &&
                s.log_count[r] <= max_row_tokens_,
            "step: history offset / log count");
  }
  for (uint32_t t : s.tokens) require(t < uint32_t(g_.V), "step: token outside vocabulary");
  step_rows_ = B;
  step_tokens_ = T;
  step_logs_ = std::any_of(s.log_count.begin(), s.log_count.end(), [](int32_t c) { return c != 0; });
  step_ctx_sum_ = 0;
  for (int r = 0; r < B; ++r) step_ctx_sum_ += s.positions[r] + s.row_tokens[r];
  // one copy: the staging slot mirrors the device table block (regions of R)
  int32_t* const h = stage_begin();
  const int R = max_rows_;
  const std::vector<int32_t>* cols[7] = {&s.row_tokens, &s.positions, &s.seq, &s.src_slot,
                                         &s.dst_slot,   &s.hist_off,  &s.log_count};
  for (int k = 0; k < 7; ++k) std::copy(cols[k]->begin(), cols[k]->end(), h + size_t(k) * R);
  std::copy(s.tokens.begin(), s.tokens.end(), reinterpret_cast<uint32_t*>(h + size_t(7) * R));
  HB_CHECK(hipMemcpyAsync(d_tab_, h, (size_t(7) * R + T) * 4, hipMemcpyHostToDevice, stream_));
  stage_end();
  // per-step block table rows, gathered from the sequence slots
  gather_rows_i32(block_table_, max_pages_, d_seq_, B, max_pages_, d_bt_rows_, max_pages_, stream_);
  pack_tables(d_row_tokens_, d_positions_, d_bt_rows_, max_pages_, B, kPage, d_cu_, d_tok_row_, d_tok_pos_, d_slot_,
              d_ctx_, d_status_, stream_);
  if (n_attn_ > 0 || w_.has_mtp) {  // one piece list per step, shared by every attention layer
    int max_t = 1, max_ctx = 1;
    for (int r = 0; r < B; ++r) {
      max_t = std::max(max_t, s.row_tokens[r]);
      max_ctx = std::max(max_ctx, s.positions[r] + s.row_tokens[r]);
    }
    const AttnGeom ag{g_.Hq, g_.Hkv, g_.D, g_.rotary, g_.theta, g_.eps};
    const int group = g_.Hq / g_.Hkv;
    attn_work_ = AttnWork{B, max_t, (max_t * group + 15) / 16, (max_ctx + attn_split_ - 1) / attn_split_,
                          attn_split_, attn_wo_, attn_wml_, attn_plan_};
    attn_plan(d_cu_, d_ctx_, ag, attn_work_, stream_);
  }
}

void Engine::op_begin() {
  if (op_profile_)
    op_start_ = uint64_t(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
}

void Engine::op_cut(OpStage stage) {
  if (!op_profile_) return;
  auto now = [] {
    return uint64_t(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
  };
  const uint64_t host_end = now();
  HB_CHECK(hipStreamSynchronize(stream_));
  const uint64_t end = now();
  OpMetrics& m = ops_[int(stage)];
  ++m.calls;
  m.host_ns += host_end - op_start_;
  m.wait_ns += end - host_end;
}

void Engine::moe_block(const LayerW& w, int T, const CombineNorm* next, bool cut_norm) {
  const Geom& g = g_;
  if (cut_norm) op_begin();
  rmsnorm(x_, g.H, w.post_norm, T, g.H, g.eps, h_, g.H, stream_);
  if (cut_norm) op_cut(OpStage::ResidualNorm);
  for (int c0 = 0; c0 < T; c0 += kMoeChunk) {
    const int n = std::min(kMoeChunk, T - c0);
    const bf16_t* hc = h_ + size_t(c0) * g.H;
    op_begin();
    project(w.router, w.g_router, hc, n, rlog_, 1, w.router.N);
    const bool sampled = probe_sample(0);
    int32_t* census = sampled && probe_[0].n < kProbeCap ? census_ + probe_[0].n : nullptr;
    moe_route(rlog_, w.router.N, n, g.E, g.top, moe_idx_, moe_w_, moe_counts_, moe_offsets_, moe_order_,
              moe_inverse_, moe_items_, stream_, census);
    op_cut(OpStage::MoeRouting);
    op_begin();
    probe_begin(0, sampled);
    if (w.g_gate_up.on()) {
      const auto& m = w.g_gate_up.mods;  // experts' gate, up, then the shared expert's
      moe_generic_gate_up(hc, g.H, moe_order_, moe_idx_, g.top, n * g.top, n, m[0], m[1], m[2], m[3], act_, stream_);
    } else {
      moe_grouped_qmm(hc, g.H, w.gate_up.w, w.gate_up.sb, 2 * g.I, moe_counts_, moe_offsets_, moe_order_,
                      moe_items_, g.E, g.top, n, 1, act_, stream_);
    }
    probe_end(0, n, sampled, 0);
    op_cut(OpStage::MoeUpGate);
    op_begin();
    probe_begin(1, sampled);
    if (w.g_down.on()) {
      const auto& m = w.g_down.mods;
      moe_generic_down(act_, moe_order_, moe_idx_, g.top, n * g.top, n, m[0], m[1], dout_, stream_);
    } else {
      moe_grouped_qmm(act_, g.I, w.down.w, w.down.sb, g.H, moe_counts_, moe_offsets_, moe_order_, moe_items_, g.E,
                      g.top, n, 0, dout_, stream_);
    }
    probe_end(1, n, sampled);
    op_cut(OpStage::MoeDown);
    op_begin();
    CombineNorm cn;
    if (next) {  // this chunk's rows of the fused norm output
      cn = *next;
      cn.out += size_t(c0) * cn.ld_out;
      if (cn.out_f32) cn.out_f32 += size_t(c0) * g.H;
      if (cn.gsum) cn.gsum += size_t(c0) * (g.H / 64);
    }
    moe_combine(dout_, moe_w_, moe_inverse_, rlog_, w.router.N, g.E, g.top, n, g.H, x_ + size_t(c0) * g.H, stream_,
                next ? &cn : nullptr);
    op_cut(OpStage::MoeMerge);
  }
}

void Engine::layer_forward(const LayerW& w, int attn_index, int dn_index, int T, int B, int max_t, bool speculative,
                           bool mtp_pool, bool normed_in, const CombineNorm* next) {
  const Geom& g = g_;
  // the input norm (here, or fused into the previous layer's MoE combine)
  // also writes the group sums the in-projection reads
  if (!normed_in) {
    if (!mtp_pool) op_begin();
    rmsnorm(x_, g.H, w.in_norm, T, g.H, g.eps, h_, g.H, stream_, nullptr, hgs_);
    if (!mtp_pool) op_cut(OpStage::InputNorm);
  }
  // stage trace: [h | r | residual | mlp | x] of this layer, each [T][H]
  float* const st = stage_trace_ && !mtp_pool ? stage_trace_ + size_t(trace_layer_) * 5 * T * g.H : nullptr;
  const size_t TH = size_t(T) * g.H;
  const Dims flat{1, 1, 1, int64_t(TH)}, unit{0, 0, 0, 1};
  if (st) {
    half_to_f32_n(h_, st, TH, false, stream_);
    HB_CHECK(hipMemcpyAsync(st + TH, x_, TH * 4, hipMemcpyDeviceToDevice, stream_));
  }
  if (w.attn) {
    const int rows = g.attn_in_rows();
    op_begin();
    project(w.in_proj, w.g_in, h_, T, proj_, 0, rows, hgs_);
    const AttnGeom ag{g.Hq, g.Hkv, g.D, g.rotary, g.theta, g.eps};
    const int pool = mtp_pool ? int(kc_.size()) - 1 : attn_index;
    attn_prep(proj_, rows, proj_ + g.Hq * 2 * g.D, rows, g.Hkv * g.D, w.q_norm, w.k_norm, d_tok_pos_, d_slot_, T, ag,
              q_, kc_[pool], vc_[pool], stream_);
    op_cut(OpStage::AttentionProjection);
    op_begin();
    require(attn_work_.rows == B && attn_work_.max_tokens >= max_t, "engine: attention piece list of another step");
    const bool sampled = probe_sample(2);
    probe_begin(2, sampled, false);
    paged_attention(q_, kc_[pool], vc_[pool], d_bt_rows_, max_pages_, d_cu_, d_ctx_, ag, 1.f / std::sqrt(float(g.D)),
                    attn_work_, stream_);
    probe_last(2, sampled);
    attn_combine(attn_work_, d_tok_row_, d_cu_, d_ctx_, proj_, rows, T, ag, aout_, stream_);
    // K and V of every context token, then q, gate and the output per packed token (bf16)
    probe_end(2, T, sampled, step_ctx_sum_ * g.Hkv * g.D * 2 * 2 + double(T) * g.Hq * g.D * 2 * 3);
    op_cut(OpStage::AttentionReduction);
    op_begin();
    project(w.out_proj, w.g_out, aout_, T, x_, 2, g.H);
    op_cut(OpStage::AttentionOutput);
  } else {
    const int rows = g.dn_in_rows();
    op_begin();
    project(w.in_proj, w.g_in, h_, T, proj_, 0, rows, hgs_);
    op_cut(OpStage::RecurrentProjection);
    const GdnGeom gg{g.Hk, g.Hv, g.Dk, g.Dv, g.conv, max_row_tokens_};
    const GdnSlots slots{d_src_, d_dst_};
    const GdnLog log{dn_log_k_[dn_index], dn_log_d_[dn_index], dn_log_g_[dn_index]};
    const bool chunked = !speculative && !step_logs_ && max_t >= kChunkedRowTokens;  // prefill: 64-token chunks on MFMA
    const bool sampled = probe_sample(3);
    const double state_bytes = double(B) * g.Hv * g.Dk * g.Dv * 4 * 2;  // read and written once per (row, head)
    const double C = 2.0 * g.Hk * g.Dk + g.Hv * g.Dv;                   // conv channels
    probe_begin(3, sampled);  // taken by the recurrence's launch (the prep and the chunked form are not timed)
    op_begin();
    if (!chunked && gdn_decode(proj_, rows, proj_ + g.a_col(), proj_ + g.b_col(), rows, w.conv_w, w.a_log,
                               w.dt_bias, dn_window_[dn_index], d_hist_, d_cu_, B, gg, dn_state_[dn_index], slots,
                               log, d_logc_, log, max_row_tokens_, speculative ? 1 : 0, nullptr, proj_ + g.z_col(),
                               rows, w.gnorm, y_, stream_)) {
      // decode steps, the prep and the recurrence in one launch: per token the conv input (bf16) read and
      // written to the window, a and b, z and the gated output y (bf16); per row the conv history read and
      // rewritten
      probe_end(3, T, sampled,
                state_bytes + double(T) * (C * 2 * 2 + 2.0 * g.Hv * 2 + 2.0 * g.Hv * g.Dv * 2) +
                    double(B) * C * (g.conv - 1) * 2 * 2);
      op_cut(OpStage::RecurrentUpdate);
    } else {
      gdn_prep(proj_, rows, proj_ + g.a_col(), proj_ + g.b_col(), rows, w.conv_w, w.a_log, w.dt_bias,
               dn_window_[dn_index], d_hist_, slots, d_cu_, B, gg, gq_, gk_, gv_, gg_, gb_, stream_);
      op_cut(OpStage::RecurrentPrepare);
      op_begin();
      if (chunked)
        gdn_chunked(gq_, gk_, gv_, gg_, gb_, d_cu_, B, gg, dn_state_[dn_index], slots, nullptr, proj_ + g.z_col(),
                    rows, w.gnorm, y_, stream_);
      else
        gdn_recurrence(gq_, gk_, gv_, gg_, gb_, d_cu_, B, gg, dn_state_[dn_index], slots, log, d_logc_, log,
                       max_row_tokens_, speculative ? 1 : 0, nullptr, proj_ + g.z_col(), rows, w.gnorm, y_, stream_);
      // per token q_hat, k_hat, v, decay and beta (f32), z (bf16) and the gated output y (bf16)
      probe_end(3, T, sampled,
                state_bytes + double(T) * (2.0 * g.Hk * g.Dk * 4 + g.Hv * g.Dv * 4 + 2.0 * g.Hv * 4 +
                                           2.0 * g.Hv * g.Dv * 2));
      op_cut(OpStage::RecurrentUpdate);
    }
    op_begin();
    project(w.out_proj, w.g_out, y_, T, x_, 2, g.H);
    op_cut(OpStage::RecurrentOutput);
  }
  if (tracing_)
    HB_CHECK(hipMemcpyAsync(mid_trace_ + size_t(mtp_pool ? g.L : trace_layer_) * max_step_tokens_ * g.H, x_,
                            TH * 4, hipMemcpyDeviceToDevice, stream_));
  if (st) {  // residual = x after the mixer; r = residual - x before it
    HB_CHECK(hipMemcpyAsync(st + 2 * TH, x_, TH * 4, hipMemcpyDeviceToDevice, stream_));
    binary_f32(2, st + 2 * TH, unit, st + TH, unit, st + TH, flat, stream_);
  }
  moe_block(w, T, next, !mtp_pool);
  if (st) {  // x = layer output; mlp = x - residual
    HB_CHECK(hipMemcpyAsync(st + 4 * TH, x_, TH * 4, hipMemcpyDeviceToDevice, stream_));
    binary_f32(2, st + 4 * TH, unit, st + 2 * TH, unit, st + 3 * TH, flat, stream_);
  }
}

void Engine::upload_index(const std::vector<int32_t>& idx) {
  require(idx.size() <= size_t(max_step_tokens_), "index list longer than the step capacity");
  int32_t* h = stage_begin();
  std::copy(idx.begin(), idx.end(), h);
  HB_CHECK(hipMemcpyAsync(d_sel_idx_, h, idx.size() * 4, hipMemcpyHostToDevice, stream_));
  stage_end();
}

void Engine::lm_head_select(const bf16_t*, const std::vector<int32_t>& rows) {
  const Geom& g = g_;
  const int n = int(rows.size());
  if (n == 0) return;
  require(n <= max_step_tokens_, "lm_head: too many rows");
  upload_index(rows);
  // bf16 rows gathered as pairs of 16-bit values
  gather_rows_i32(reinterpret_cast<const int32_t*>(hn_), g.H / 2, d_sel_idx_, n, g.H / 2,
                  reinterpret_cast<int32_t*>(sel_h_), g.H / 2, stream_);
  head_select(n);
}

void Engine::head_select(int n) {
  const Geom& g = g_;
  const int Vp = g.vocab_rows();
  if (!logits_export_ && n <= 256 && !w_.g_head.on() &&
      qmm_select(sel_h_, n, g.H, w_.lm_head.w, w_.lm_head.sb, Vp, g.V, sel_part_, sel_part_bytes_, winners_,
                 margins_, sel_status_, stream_)) {
    logits_valid_ = false;
    ++fused_heads_;
    return;
  }
  project(w_.lm_head, w_.g_head, sel_h_, n, logits_, 1, Vp);
  logits_valid_ = true;
  argmax_margin(logits_, Vp, n, g.V, winners_, margins_, sel_status_, stream_, sel_ws_);
}

void Engine::set_profile(int stride) {
  require(stride >= 0, "profile: negative sampling stride");
  if (stride && !census_) {
    census_ = static_cast<int32_t*>(dalloc(size_t(kProbeCap) * 4, nullptr));
    for (Probe& p : probe_) {
      p.ev.resize(2 * kProbeCap);
      for (hipEvent_t& e : p.ev) HB_CHECK(hipEventCreate(&e));
    }
  }
  profile_stride_ = stride;
  for (Probe& p : probe_) p.n = 0, p.tokens = 0, p.bytes = 0, p.calls = 0;
}

void Engine::probe_begin(int k, bool sampled, bool one_launch) {
  Probe& p = probe_[k];
  launch_events() = LaunchEvents{};
  if (sampled && p.n < kProbeCap) launch_events() = LaunchEvents{p.ev[2 * p.n], one_launch ? p.ev[2 * p.n + 1] : nullptr};
}

void Engine::probe_last(int k, bool sampled) {
  Probe& p = probe_[k];
  if (sampled && p.n < kProbeCap) launch_events().stop = p.ev[2 * p.n + 1];
}

bool Engine::probe_sample(int k) {
  return profile_stride_ > 0 && probe_[k].calls++ % uint64_t(profile_stride_) == 0;
}

void Engine::probe_end(int k, int tokens, bool sampled, double bytes) {
  Probe& p = probe_[k];
  const LaunchEvents left = launch_events();
  launch_events() = LaunchEvents{};
  if (!sampled || p.n >= kProbeCap || left.start || left.stop) return;
  p.tokens += tokens;
  p.bytes += bytes;
  p.n += 1;
}

ProbeStats Engine::profile_read(int k) {
  require(k >= 0 && k < kProbes && census_, "profile: probes were never enabled");
  HB_CHECK(hipStreamSynchronize(stream_));
  Probe& p = probe_[k];
  ProbeStats s{};
  s.launches = p.n;
  s.tokens = p.tokens;
  for (int i = 0; i < p.n; ++i) {
    float ms = 0.f;
    HB_CHECK(hipEventElapsedTime(&ms, p.ev[2 * i], p.ev[2 * i + 1]));
    s.ms += ms;
  }
  const int nc = probe_[0].n;
  std::vector<int32_t> c(nc);
  if (nc) HB_CHECK(hipMemcpy(c.data(), census_, size_t(nc) * 4, hipMemcpyDeviceToHost));
  for (int32_t v : c) s.active += v;
  s.bytes = p.bytes;
  return s;
}

void Engine::set_trace(bool on) {
  if (on && !trace_) trace_ = static_cast<float*>(dalloc(size_t(g_.L + 1) * max_step_tokens_ * g_.H * 4, nullptr));
  if (on && !mid_trace_)
    mid_trace_ = static_cast<float*>(dalloc(size_t(g_.L + 1) * max_step_tokens_ * g_.H * 4, nullptr));
  tracing_ = on;
}

void Engine::trace_point(int i, int T) {
  if (!tracing_) return;
  HB_CHECK(hipMemcpyAsync(trace_ + size_t(i) * max_step_tokens_ * g_.H, x_, size_t(T) * g_.H * 4,
                          hipMemcpyDeviceToDevice, stream_));
}

void Engine::clear_fresh_rows(const StepRows& s) {
  const Geom& g = g_;
  const size_t state_row = size_t(g.Hv) * g.Dv * g.Dk;
  const size_t window_row = size_t(g.conv - 1 + max_row_tokens_) * g.conv_channels();
  for (int r = 0; r < s.rows; ++r) {
    if (s.positions[r] != 0) continue;
    require(s.log_count[r] == 0 && s.hist_off[r] == 0, "step: a row at position 0 has no pending history");
    for (size_t i = 0; i < dn_state_.size(); ++i) {
      HB_CHECK(hipMemsetAsync(dn_state_[i] + size_t(s.src_slot[r]) * state_row, 0, state_row * 4, stream_));
      HB_CHECK(hipMemsetAsync(dn_window_[i] + size_t(s.src_slot[r]) * window_row, 0, window_row * 2, stream_));
    }
  }
}

void Engine::forward(const StepRows& s, bool speculative, const std::vector<int32_t>& logit_rows) {
  const Geom& g = g_;
  upload_tables(s);
  clear_fresh_rows(s);
  const int T = s.total(), B = s.rows;
  int max_t = 0;
  for (int r = 0; r < B; ++r) max_t = std::max(max_t, s.row_tokens[r]);
  op_begin();
  embed(T);
  op_cut(OpStage::Embedding);
  trace_point(0, T);
  int ai = 0, di = 0;
  // each layer's MoE combine also writes the next norm: the next layer's input
  // norm into h_, after the last layer the final norm into hn_ / hn_f32_
  for (int l = 0; l < g.L; ++l) {
    const LayerW& w = w_.layers[l];
    trace_layer_ = l;
    CombineNorm next;
    next.eps = g.eps;
    if (l + 1 < g.L) {
      next.w = w_.layers[l + 1].in_norm;
      next.out = h_;
      next.ld_out = g.H;
      next.gsum = hgs_;
    } else {
      next.w = w_.final_norm;
      next.out = hn_;
      next.ld_out = g.H;
      next.out_f32 = hn_f32_;
    }
    layer_forward(w, ai, di, T, B, max_t, speculative, false, l > 0, &next);
    trace_point(l + 1, T);
    if (w.attn)
      ++ai;
    else
      ++di;
  }
  op_begin();
  lm_head_select(hn_, logit_rows);
  op_cut(OpStage::FinalProjection);
}

void Engine::mtp_forward(const StepRows& s, const float* hidden_src, const std::vector<int32_t>& hidden_idx,
                         const std::vector<int32_t>& logit_rows) {
  const Geom& g = g_;
  require(w_.has_mtp, "engine: no MTP head");
  upload_tables(s);
  const int T = s.total(), B = s.rows;
  require(int(hidden_idx.size()) == T, "mtp: one hidden row per token");
  int max_t = 0;
  for (int r = 0; r < B; ++r) max_t = std::max(max_t, s.row_tokens[r]);
  upload_index(hidden_idx);
  gather_rows_f32(hidden_src, g.H, d_sel_idx_, T, g.H, mtp_in_f32_, g.H, stream_);
  embed(T);
  // fc([rms(embed, pre_fc_norm_embedding) | rms(hidden, pre_fc_norm_hidden)]), native/qwen_mtp.inc:38-39
  rmsnorm(x_, g.H, w_.mtp_pre_e, T, g.H, g.eps, proj_, 2 * g.H, stream_);
  rmsnorm(mtp_in_f32_, g.H, w_.mtp_pre_h, T, g.H, g.eps, proj_ + g.H, 2 * g.H, stream_);
  if (w_.mtp_fc_dense)
    dense_bf16(proj_, T, 2 * g.H, w_.mtp_fc_dense, g.H, x_, 1, g.H, stream_);
  else
    project(w_.mtp_fc, w_.g_mtp_fc, proj_, T, x_, 1, g.H);
  trace_point(0, T);
  CombineNorm next;  // the MTP head's final norm, fused into its MoE combine
  next.w = w_.mtp_norm;
  next.eps = g.eps;
  next.out = hn_;
  next.ld_out = g.H;
  next.out_f32 = mtp_h_f32_;
  layer_forward(w_.mtp_layer, 0, 0, T, B, max_t, false, true, false, &next);
  trace_point(1, T);
  // lm_head over the MTP hidden rows (the target lm_head, native/qwen_mtp.inc:46)
  const int n = int(logit_rows.size());
  if (n) {
    upload_index(logit_rows);
  // bf16 rows gathered as pairs of 16-bit values
  gather_rows_i32(reinterpret_cast<const int32_t*>(hn_), g.H / 2, d_sel_idx_, n, g.H / 2,
                  reinterpret_cast<int32_t*>(sel_h_), g.H / 2, stream_);
    head_select(n);
  }
}

void Engine::synthetic_context(int n, const int32_t* positions, uint64_t seed) {
  const Geom& g = g_;
  require(n > 0 && n <= max_rows_, "synthetic_context: rows");
  for (int r = 0; r < n; ++r) require(positions[r] >= 0 && positions[r] <= max_context_, "synthetic_context: position");
  const size_t kv_elems = size_t(pages_) * g.Hkv * kPage * g.D;
  uint64_t sd = seed;
  for (size_t i = 0; i < kc_.size(); ++i) {
    random_normal(++sd, kv_elems, 1.f, 0.f, 4, kc_[i], stream_);
    random_normal(++sd, kv_elems, 1.f, 0.f, 4, vc_[i], stream_);
  }
  const int slots = 2 * max_rows_;
  const int C = g.conv_channels();
  for (size_t i = 0; i < dn_state_.size(); ++i) {
    random_normal(++sd, size_t(slots) * g.Hv * g.Dv * g.Dk, 0.01f, 0.f, 0, dn_state_[i], stream_);
    random_normal(++sd, size_t(slots) * (g.conv - 1 + max_row_tokens_) * C, 1.f, 0.f, 4, dn_window_[i], stream_);
  }
  HB_CHECK(hipStreamSynchronize(stream_));
}

}  // namespace hb
