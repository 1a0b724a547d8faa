// Engine weights from checkpoint tensors (rs_mlx_weights_load): each fused
// engine tensor is assembled in the checkpoint layout (u32 codes [N][K/8], bf16
// scales and biases [N][K/64]) from the named MLX tensors the reference's model
// code reads (native/qwen_model.inc:34-206,306-373, qwen_mtp.inc:37-45), then
// tiled like the synthetic weights.
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "engine.h"

namespace hb {

namespace {

const char* kModel = "language_model.model";
const char* kMtp = "language_model.mtp";

std::string shape_text(const std::vector<int32_t>& s) {
  std::string t = "[";
  for (size_t i = 0; i < s.size(); ++i) t += (i ? "," : "") + std::to_string(s[i]);
  return t + "]";
}

}  // namespace

const NamedWeights& Engine::source_of(int id) const {
  // the MTP tensors (global ids 3..6 and the MTP layer) live in the sidecar
  const bool mtp_part = (id >= 3 && id <= 6) || (id >= 16 && (id - 16) / kTLayerStride == g_.L);
  require(named_ && (!mtp_part || named_mtp_), "checkpoint: no named source for this tensor");
  return mtp_part ? *named_mtp_ : *named_;
}

std::pair<int, int> Engine::quant_of(const NamedWeights& src, const std::string& module) const {
  const auto it = src.quant.find(module);
  return it == src.quant.end() ? std::pair<int, int>{qgroup_, qbits_} : it->second;
}

// The modules each matrix tensor is assembled from (the names the reference's
// linear / expert calls read, native/qwen_model.inc:34-206,306-373 and
// qwen_mtp.inc:37-45), in the order of their output columns.
std::vector<Engine::ModSpec> Engine::slot_modules(int id) const {
  const Geom& g = g_;
  if (id == 0) return {{std::string(kModel) + ".embed_tokens", 0, g.V, g.H, 0}};
  if (id == 2) return {{"language_model.lm_head", 0, g.V, g.H, 0}};
  if (id == 5) return {{std::string(kMtp) + ".fc", 0, g.H, 2 * g.H, 0}};
  require(id >= 16, "checkpoint: not a matrix tensor");
  const int layer = (id - 16) / kTLayerStride, slot = (id - 16) % kTLayerStride;
  const bool attn = layer == g.L ? true : g.attn(layer);
  const std::string p =
      layer == g.L ? std::string(kMtp) + ".layers.0" : std::string(kModel) + ".layers." + std::to_string(layer);
  switch (slot) {
    case kTInProj:
      if (attn) {
        const int q = g.Hq * 2 * g.D, kv = g.Hkv * g.D;
        return {{p + ".self_attn.q_proj", 0, q, g.H, 0},
                {p + ".self_attn.k_proj", 0, kv, g.H, q},
                {p + ".self_attn.v_proj", 0, kv, g.H, q + kv}};
      } else {
        const int C = g.conv_channels(), Z = g.Hv * g.Dv;
        return {{p + ".linear_attn.in_proj_qkv", 0, C, g.H, 0},
                {p + ".linear_attn.in_proj_z", 0, Z, g.H, C},
                {p + ".linear_attn.in_proj_a", 0, g.Hv, g.H, C + Z},
                {p + ".linear_attn.in_proj_b", 0, g.Hv, g.H, C + Z + g.Hv}};
      }
    case kTOutProj:
      return {{p + (attn ? ".self_attn.o_proj" : ".linear_attn.out_proj"), 0, g.H,
               attn ? g.Hq * g.D : g.Hv * g.Dv, 0}};
    case kTRouter: return {{p + ".mlp.gate", 0, g.E, g.H, 0}, {p + ".mlp.shared_expert_gate", 0, 1, g.H, g.E}};
    case kTGateUp:
      return {{p + ".mlp.switch_mlp.gate_proj", g.E, g.I, g.H, 0},
              {p + ".mlp.switch_mlp.up_proj", g.E, g.I, g.H, 0},
              {p + ".mlp.shared_expert.gate_proj", 0, g.I, g.H, 0},
              {p + ".mlp.shared_expert.up_proj", 0, g.I, g.H, 0}};
    case kTDown:
      return {{p + ".mlp.switch_mlp.down_proj", g.E, g.H, g.I, 0}, {p + ".mlp.shared_expert.down_proj", 0, g.H, g.I, 0}};
    default: break;
  }
  throw std::invalid_argument("checkpoint: not a matrix slot");
}

GSlot Engine::generic_slot(int id) const {
  GSlot out;
  if (!named_) return out;
  const NamedWeights& src = source_of(id);
  const std::vector<ModSpec> mods = slot_modules(id);
  // the sidecar's dense BF16 fc has its own path
  if (id == 5) {
    const auto it = src.arrays.find(mods[0].name + ".weight");
    if (it != src.arrays.end() && it->second->dtype == kBF16) return out;
  }
  bool other = false;
  for (const ModSpec& m : mods) other |= quant_of(src, m.name) != std::pair<int, int>{64, 4};
  if (!other) return out;
  for (const ModSpec& m : mods) {
    const auto [group, bits] = quant_of(src, m.name);
    require(m.K % group == 0 && (size_t(m.K) * bits) % 32 == 0,
            ("checkpoint: " + m.name + ": K is not a whole number of groups / words").c_str());
    std::vector<int32_t> ws, ss;
    if (m.lead) ws.push_back(m.lead), ss.push_back(m.lead);
    ws.push_back(m.rows), ws.push_back(int32_t(size_t(m.K) * bits / 32));
    ss.push_back(m.rows), ss.push_back(m.K / group);
    auto find = [&](const std::string& name, int dtype, const std::vector<int32_t>& shape) -> const Tensor& {
      const auto it = src.arrays.find(name);
      if (it == src.arrays.end()) throw std::invalid_argument("checkpoint: missing tensor " + name);
      const Tensor& t = *it->second;
      if (t.dtype != dtype || t.shape != shape)
        throw std::invalid_argument("checkpoint: tensor " + name + " is " + shape_text(t.shape) + " dtype " +
                                    std::to_string(t.dtype) + ", " + std::to_string(bits) + "-bit group " +
                                    std::to_string(group) + " needs " + shape_text(shape) + " dtype " +
                                    std::to_string(dtype));
      return t;
    };
    QMod q;
    q.w = static_cast<const uint32_t*>(find(m.name + ".weight", kU32, ws).data);
    q.s = static_cast<const bf16_t*>(find(m.name + ".scales", kBF16, ss).data);
    q.b = static_cast<const bf16_t*>(find(m.name + ".biases", kBF16, ss).data);
    q.rows = m.rows, q.K = m.K, q.group = group, q.bits = bits, q.lead = m.lead, q.col = m.col;
    out.mods.push_back(q);
  }
  return out;
}

void Engine::export_named(int id, void* wv, void* sv, void* bv) {
  const Geom& g = g_;
  int N, K;
  bool q4;
  tensor_shape(id, N, K, q4);
  // the MTP tensors (global ids 3..6 and the MTP layer) live in the sidecar
  const bool mtp_part = (id >= 3 && id <= 6) || (id >= 16 && (id - 16) / kTLayerStride == g.L);
  require(!mtp_part || named_mtp_, "checkpoint: the MTP sidecar's tensors are not attached");
  const NamedWeights& src = source_of(id);

  auto find = [&](const std::string& name, int dtype, const std::vector<int32_t>& shape) -> const Tensor& {
    const auto it = src.arrays.find(name);
    if (it == src.arrays.end()) throw std::invalid_argument("checkpoint: missing tensor " + name);
    const Tensor& t = *it->second;
    if (t.dtype != dtype || t.shape != shape)
      throw std::invalid_argument("checkpoint: tensor " + name + " is " + shape_text(t.shape) + " dtype " +
                                  std::to_string(t.dtype) + ", the model needs " + shape_text(shape) + " dtype " +
                                  std::to_string(dtype));
    return t;
  };

  if (!q4) {
    // f32 vector: norms (+1 for shifted checkpoints), conv taps, A_log, dt_bias
    float* out = static_cast<float*>(wv);
    std::string name;
    bool shifted = false;
    int conv = 0;
    if (id == 1) {
      name = std::string(kModel) + ".norm.weight", shifted = true;
    } else if (id == 3) {
      name = std::string(kMtp) + ".pre_fc_norm_embedding.weight", shifted = true;
    } else if (id == 4) {
      name = std::string(kMtp) + ".pre_fc_norm_hidden.weight", shifted = true;
    } else if (id == 6) {
      name = std::string(kMtp) + ".norm.weight", shifted = true;
    } else {
      const int layer = (id - 16) / kTLayerStride, slot = (id - 16) % kTLayerStride;
      const std::string p =
          layer == g.L ? std::string(kMtp) + ".layers.0" : std::string(kModel) + ".layers." + std::to_string(layer);
      switch (slot) {
        case kTInNorm: name = p + ".input_layernorm.weight", shifted = true; break;
        case kTPostNorm: name = p + ".post_attention_layernorm.weight", shifted = true; break;
        case kTQNorm: name = p + ".self_attn.q_norm.weight", shifted = true; break;
        case kTKNorm: name = p + ".self_attn.k_norm.weight", shifted = true; break;
        case kTGNorm: name = p + ".linear_attn.norm.weight"; break;  // never shifted (qwen_model.inc:203)
        case kTALog: name = p + ".linear_attn.A_log"; break;
        case kTDtBias: name = p + ".linear_attn.dt_bias"; break;
        case kTConvW: name = p + ".linear_attn.conv1d.weight", conv = g.conv; break;
        default: throw std::invalid_argument("checkpoint: unknown vector slot");
      }
    }
    const auto it = src.arrays.find(name);
    if (it == src.arrays.end()) throw std::invalid_argument("checkpoint: missing tensor " + name);
    const Tensor& t = *it->second;
    if (t.dtype != kF32 && t.dtype != kBF16 && t.dtype != kF16)
      throw std::invalid_argument("checkpoint: tensor " + name + " must be f32, bf16 or f16");
    if (size_t(t.elements) != size_t(N)) throw std::invalid_argument("checkpoint: tensor " + name + " size");
    if (conv) {
      // MLX layout [C, W, 1]; raw checkpoints [C, 1, W] (qwen_model.inc:166)
      const int C = N / conv;
      const bool mlx = t.shape == std::vector<int32_t>{C, conv, 1};
      const bool raw = t.shape == std::vector<int32_t>{C, 1, conv};
      if (!mlx && !raw) throw std::invalid_argument("checkpoint: conv1d weight shape " + shape_text(t.shape));
    } else if (t.shape.size() != 1) {
      throw std::invalid_argument("checkpoint: tensor " + name + " must be a vector");
    }
    // small: widened on the host (both conv layouts list tap w of channel c at c * W + w)
    HB_CHECK(hipStreamSynchronize(stream_));
    std::vector<uint8_t> raw(t.elements * dtype_size(t.dtype));
    HB_CHECK(hipMemcpy(raw.data(), t.data, raw.size(), hipMemcpyDeviceToHost));
    std::vector<float> v(t.elements);
    for (size_t i = 0; i < t.elements; ++i) {
      if (t.dtype == kF32) {
        std::memcpy(&v[i], raw.data() + 4 * i, 4);
      } else {
        uint16_t h;
        std::memcpy(&h, raw.data() + 2 * i, 2);
        v[i] = t.dtype == kBF16 ? bf16_to_f32(h) : float(reinterpret_cast<const _Float16&>(h));
      }
      if (shifted && src.shift && !mtp_part) v[i] += 1.f;  // the sidecar is never shifted (qwen_mtp.inc:30)
    }
    HB_CHECK(hipMemcpy(out, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return;
  }

  // q4: assemble rows into (codes, scales, biases), then zero the padding rows
  uint8_t* w = static_cast<uint8_t*>(wv);
  uint8_t* s = static_cast<uint8_t*>(sv);
  uint8_t* b = static_cast<uint8_t*>(bv);
  const size_t wrow = size_t(K) / 2, srow = size_t(K) / 64 * 2;  // bytes per row
  size_t filled = 0;
  // rows of tensor `name` (leading dims flattened, `rows` in all) as blocks of
  // `block` rows, placed every `dst_stride` rows from dst_row
  auto place = [&](const std::string& name, std::vector<int32_t> lead, int rows_per, size_t dst_row,
                   size_t block, size_t dst_stride) {
    std::vector<int32_t> ws = lead, ss = lead;
    ws.push_back(rows_per);
    ws.push_back(K / 8);
    ss.push_back(rows_per);
    ss.push_back(K / 64);
    const Tensor& tw = find(name + ".weight", kU32, ws);
    const Tensor& ts = find(name + ".scales", kBF16, ss);
    const Tensor& tb = find(name + ".biases", kBF16, ss);
    size_t rows = size_t(rows_per);
    for (int32_t d : lead) rows *= size_t(d);
    require(rows % block == 0, "checkpoint: row blocks");
    const size_t blocks = rows / block;
    require(dst_row + (blocks - 1) * dst_stride + block <= size_t(N), "checkpoint: rows past the fused tensor");
    HB_CHECK(hipMemcpy2DAsync(w + dst_row * wrow, dst_stride * wrow, tw.data, block * wrow, block * wrow, blocks,
                              hipMemcpyDeviceToDevice, stream_));
    HB_CHECK(hipMemcpy2DAsync(s + dst_row * srow, dst_stride * srow, ts.data, block * srow, block * srow, blocks,
                              hipMemcpyDeviceToDevice, stream_));
    HB_CHECK(hipMemcpy2DAsync(b + dst_row * srow, dst_stride * srow, tb.data, block * srow, block * srow, blocks,
                              hipMemcpyDeviceToDevice, stream_));
    filled = std::max(filled, dst_row + (blocks - 1) * dst_stride + block);
  };
  auto rows_of = [&](const std::string& name, int rows, size_t at) {
    place(name, {}, rows, at, size_t(rows), size_t(rows));
    return at + size_t(rows);
  };

  if (id == 0) {
    rows_of(std::string(kModel) + ".embed_tokens", g.V, 0);
  } else if (id == 2) {
    rows_of("language_model.lm_head", g.V, 0);  // the target's head, also under the MTP head
  } else if (id == 5) {
    rows_of(std::string(kMtp) + ".fc", g.H, 0);
  } else {
    const int layer = (id - 16) / kTLayerStride, slot = (id - 16) % kTLayerStride;
    const bool attn = layer == g.L ? true : g.attn(layer);
    const std::string p =
        layer == g.L ? std::string(kMtp) + ".layers.0" : std::string(kModel) + ".layers." + std::to_string(layer);
    switch (slot) {
      case kTInProj:
        if (attn) {
          size_t at = rows_of(p + ".self_attn.q_proj", g.Hq * 2 * g.D, 0);  // q then gate per head
          at = rows_of(p + ".self_attn.k_proj", g.Hkv * g.D, at);
          rows_of(p + ".self_attn.v_proj", g.Hkv * g.D, at);
        } else {
          size_t at = rows_of(p + ".linear_attn.in_proj_qkv", g.conv_channels(), 0);
          at = rows_of(p + ".linear_attn.in_proj_z", g.Hv * g.Dv, at);
          at = rows_of(p + ".linear_attn.in_proj_a", g.Hv, at);
          rows_of(p + ".linear_attn.in_proj_b", g.Hv, at);
        }
        break;
      case kTOutProj: rows_of(p + (attn ? ".self_attn.o_proj" : ".linear_attn.out_proj"), g.H, 0); break;
      case kTRouter: rows_of(p + ".mlp.shared_expert_gate", 1, rows_of(p + ".mlp.gate", g.E, 0)); break;
      case kTGateUp: {
        // each 16-row tile: 8 gate rows, then the matching 8 up rows
        const size_t I2 = 2 * size_t(g.I);
        place(p + ".mlp.switch_mlp.gate_proj", {g.E}, g.I, 0, 8, 16);
        place(p + ".mlp.switch_mlp.up_proj", {g.E}, g.I, 8, 8, 16);
        place(p + ".mlp.shared_expert.gate_proj", {}, g.I, size_t(g.E) * I2, 8, 16);
        place(p + ".mlp.shared_expert.up_proj", {}, g.I, size_t(g.E) * I2 + 8, 8, 16);
        break;
      }
      case kTDown:
        place(p + ".mlp.switch_mlp.down_proj", {g.E}, g.H, 0, size_t(g.E) * g.H, size_t(g.E) * g.H);
        rows_of(p + ".mlp.shared_expert.down_proj", g.H, size_t(g.E) * g.H);
        break;
      default: throw std::invalid_argument("checkpoint: unknown matrix slot");
    }
  }
  // padding rows: zero codes, scales and biases (outputs nobody reads)
  if (filled < size_t(N)) {
    HB_CHECK(hipMemsetAsync(w + filled * wrow, 0, (size_t(N) - filled) * wrow, stream_));
    HB_CHECK(hipMemsetAsync(s + filled * srow, 0, (size_t(N) - filled) * srow, stream_));
    HB_CHECK(hipMemsetAsync(b + filled * srow, 0, (size_t(N) - filled) * srow, stream_));
  }
}

}  // namespace hb
