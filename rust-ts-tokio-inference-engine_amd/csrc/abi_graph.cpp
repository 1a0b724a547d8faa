// Graph API (rs_mlx_*) over HIP. The reference builds lazy MLX graphs
// (native/mlx_bridge.cpp:33-174); here every node is a device tensor and ops run
// eagerly on the graph's stream, so finish() is one synchronisation plus one
// device-to-host copy. Validation messages and limits follow the reference
// (256 nodes, rank 1..4, dims 1..8192, output element count must match).
#include <fstream>
#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/hip_bridge.h"
#include "graph.h"
#include "safetensors.h"
#include "ops.h"
#include "qmm.h"

using namespace hb;

namespace hb {

size_t dtype_size(int dtype) {
  switch (dtype) {
    case kF32:
    case kI32:
    case kU32:
      return 4;
    case kF16:
    case kBF16:
      return 2;
  }
  throw std::invalid_argument("invalid dtype");
}

Tensor::~Tensor() {
  if (owned && data) (void)hipFree(data);
}

std::shared_ptr<Tensor> Tensor::make(int dtype, std::vector<int32_t> shape) {
  auto t = std::make_shared<Tensor>();
  t->dtype = dtype;
  t->shape = std::move(shape);
  t->elements = 1;
  for (auto d : t->shape) t->elements *= size_t(d);
  const size_t bytes = std::max<size_t>(t->elements * dtype_size(dtype), 4);
  HB_CHECK(hipMalloc(&t->data, bytes));
  return t;
}

Graph::Graph(bool g) : gpu(g) {
  int n = 0;
  require(hipGetDeviceCount(&n) == hipSuccess && n > 0, "no HIP device available");
  HB_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
}

Graph::~Graph() {
  if (stream) {
    (void)hipStreamSynchronize(stream);
    (void)hipStreamDestroy(stream);
  }
}

const Tensor& Graph::at(uint32_t id) const {
  if (id >= nodes.size()) throw std::invalid_argument("invalid node reference");
  return *nodes[id];
}

void Graph::push(std::shared_ptr<Tensor> t) {
  if (nodes.size() >= kMaxNodes) throw std::invalid_argument("node cap");
  nodes.push_back(std::move(t));
}

// f32 view of a node (converted when the node holds f16/bf16).
std::shared_ptr<Tensor> Graph::as_f32(const std::shared_ptr<Tensor>& t) {
  if (t->dtype == kF32) return t;
  require(t->dtype == kF16 || t->dtype == kBF16, "expected a floating node");
  auto out = Tensor::make(kF32, t->shape);
  half_to_f32_n(static_cast<const uint16_t*>(t->data), static_cast<float*>(out->data), t->elements,
                t->dtype == kF16, stream);
  return out;
}

// bf16 copy of a floating node.
std::shared_ptr<Tensor> Graph::as_bf16(const std::shared_ptr<Tensor>& t) {
  if (t->dtype == kBF16) return t;
  auto out = Tensor::make(kBF16, t->shape);
  if (t->dtype == kF32)
    f32_to_bf16_n(static_cast<const float*>(t->data), static_cast<bf16_t*>(out->data), t->elements, stream);
  else if (t->dtype == kF16)
    f16_to_bf16_n(static_cast<const uint16_t*>(t->data), static_cast<bf16_t*>(out->data), t->elements, stream);
  else
    throw std::invalid_argument("expected a floating node");
  return out;
}


}  // namespace hb

namespace {

Graph& graph_of(void* g) {
  if (!g) throw std::invalid_argument("invalid graph handle");
  return *static_cast<Graph*>(g);
}

// Numpy-style broadcast of two shapes (rank <= 4).
void broadcast(const Tensor& a, const Tensor& b, std::vector<int32_t>& out, Dims& as, Dims& bs, Dims& shape) {
  const size_t rank = std::max(a.shape.size(), b.shape.size());
  out.assign(rank, 1);
  for (size_t i = 0; i < rank; ++i) {
    const int64_t da = i < rank - a.shape.size() ? 1 : a.shape[i - (rank - a.shape.size())];
    const int64_t db = i < rank - b.shape.size() ? 1 : b.shape[i - (rank - b.shape.size())];
    if (da != db && da != 1 && db != 1) throw std::invalid_argument("shapes do not broadcast");
    out[i] = int32_t(std::max(da, db));
  }
  auto strides = [&](const Tensor& t, Dims& s) {
    s.fill(0);
    int64_t stride = 1;
    for (int i = int(t.shape.size()) - 1; i >= 0; --i) {
      const int ax = kMaxRank - int(t.shape.size()) + i;
      s[ax] = t.shape[i] == 1 ? 0 : stride;
      stride *= t.shape[i];
    }
  };
  strides(a, as);
  strides(b, bs);
  shape.fill(1);
  for (size_t i = 0; i < rank; ++i) shape[kMaxRank - rank + i] = out[i];
}

}  // namespace

extern "C" void* rs_mlx_create(int gpu, char* error, size_t capacity) {
  Graph* g = nullptr;
  guarded(error, capacity, [&] { g = new Graph(gpu != 0); });
  return g;
}

extern "C" void rs_mlx_destroy(void* graph) { delete static_cast<Graph*>(graph); }

extern "C" const char* rs_mlx_version(void) { return "hip_bridge-gfx950-0.1"; }

extern "C" void rs_mlx_cleanup(void) {}

extern "C" int rs_mlx_input(void* graph, int dtype, const void* data, const int32_t* shape, size_t rank, char* error,
                            size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!graph || !data || !shape || rank == 0 || rank > 4) throw std::invalid_argument("invalid input descriptor");
    auto& g = graph_of(graph);
    if (g.nodes.size() >= kMaxNodes) throw std::invalid_argument("node cap");
    std::vector<int32_t> dims(shape, shape + rank);
    if (std::any_of(dims.begin(), dims.end(), [](int32_t d) { return d <= 0 || d > 8192; }))
      throw std::invalid_argument("invalid dimension");
    if (dtype < 0 || dtype > 2) throw std::invalid_argument("invalid input dtype");
    auto t = Tensor::make(dtype, dims);
    HB_CHECK(hipMemcpyAsync(t->data, data, t->elements * 4, hipMemcpyHostToDevice, g.stream));
    g.push(std::move(t));
  });
}

extern "C" int rs_mlx_op(void* graph, int op, const uint32_t* inputs, size_t count, int group, float epsilon,
                         char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!graph || !inputs) throw std::invalid_argument("invalid operation descriptor");
    auto& g = graph_of(graph);
    if (g.nodes.size() >= kMaxNodes) throw std::invalid_argument("node cap");
    const bool quantized = op == 3 || op == 102 || op == 103 || op == 104 || op == 105 || op == 106 || op == 108;
    if (count != (quantized ? 4u : 2u)) throw std::invalid_argument("invalid operand count");
    for (size_t i = 0; i < count; ++i)
      if (inputs[i] >= g.nodes.size()) throw std::invalid_argument("invalid node reference");
    auto a = g.nodes[inputs[0]];
    auto b = g.nodes[inputs[1]];
    if (op == 0 || op == 1) {
      auto af = g.as_f32(a), bf = g.as_f32(b);
      std::vector<int32_t> shape;
      Dims as, bs, sh;
      broadcast(*af, *bf, shape, as, bs, sh);
      auto y = Tensor::make(kF32, shape);
      binary_f32(op, static_cast<float*>(af->data), as, static_cast<float*>(bf->data), bs,
                 static_cast<float*>(y->data), sh, g.stream);
      g.push(y);
    } else if (op == 2) {
      auto af = g.as_f32(a), bf = g.as_f32(b);
      require(af->shape.size() >= 2 && bf->shape.size() >= 2, "matmul rank");
      const int M = af->shape[af->shape.size() - 2], K = af->shape.back();
      const int K2 = bf->shape[bf->shape.size() - 2], N = bf->shape.back();
      require(K == K2, "matmul inner dimension");
      int batch = 1, wbatch = 1;
      for (size_t i = 0; i + 2 < af->shape.size(); ++i) batch *= af->shape[i];
      for (size_t i = 0; i + 2 < bf->shape.size(); ++i) wbatch *= bf->shape[i];
      require(wbatch == 1 || wbatch == batch, "matmul batch");
      std::vector<int32_t> shape(af->shape.begin(), af->shape.end() - 1);
      shape.push_back(N);
      auto y = Tensor::make(kF32, shape);
      matmul_f32(static_cast<float*>(af->data), static_cast<float*>(bf->data), static_cast<float*>(y->data), batch,
                 wbatch, M, N, K, g.stream);
      g.push(y);
    } else if (op == 4) {
      auto af = g.as_f32(a), wf = g.as_f32(b);
      const int width = af->shape.back();
      require(wf->elements == size_t(width), "rms_norm weight width");
      auto y = Tensor::make(kF32, af->shape);
      rms_norm_f32(static_cast<float*>(af->data), static_cast<float*>(wf->data), static_cast<float*>(y->data),
                   int(af->elements / width), width, epsilon, g.stream);
      g.push(y);
    } else if (quantized) {
      const int bits = op == 3 ? 4 : op - 100;
      auto s = g.nodes[inputs[2]], bi = g.nodes[inputs[3]];
      require(a->shape.size() == 2 && b->shape.size() == 2 && s->shape.size() == 2 && s->shape == bi->shape,
              "Q4 dtype/rank mismatch");
      require(b->dtype == kU32 && a->dtype != kI32 && a->dtype != kU32, "Q4 dtype/rank mismatch");
      require(group == 32 || group == 64 || group == 128, "unsupported affine quantization");
      const int M = a->shape[0], K = a->shape[1], N = b->shape[0];
      require(K % group == 0 && int64_t(b->shape[1]) * 32 == int64_t(K) * bits && s->shape[0] == N &&
                  s->shape[1] == K / group,
              "Q4 packed shape mismatch");
      auto xb = g.as_bf16(a), sb = g.as_bf16(s), bb = g.as_bf16(bi);
      auto y = Tensor::make(kF32, {M, N});
      if (bits == 4 && group == 64 && N % 16 == 0 && K % 128 == 0) {
        auto wt = Tensor::make(kU32, b->shape);
        auto sbt = Tensor::make(kBF16, {N, 2 * (K / 64)});
        q4_tile(b->as<uint32_t>(), sb->as<bf16_t>(), bb->as<bf16_t>(), wt->as<uint32_t>(), sbt->as<bf16_t>(), N, K,
                g.stream);
        qmm(xb->as<bf16_t>(), M, K, wt->as<uint32_t>(), sbt->as<bf16_t>(), nullptr, N, group, bits, kLayoutQ4Tiled,
            y->data, true, N, g.stream);
        g.keep(wt);
        g.keep(sbt);
      } else {
        qmm(static_cast<bf16_t*>(xb->data), M, K, static_cast<uint32_t*>(b->data), static_cast<bf16_t*>(sb->data),
            static_cast<bf16_t*>(bb->data), N, group, bits, kLayoutMlx, y->data, true, N, g.stream);
      }
      g.keep(xb);
      g.keep(sb);
      g.keep(bb);
      g.push(y);
    } else {
      throw std::invalid_argument("unknown operation");
    }
  });
}

extern "C" int rs_mlx_finish(void* graph, uint32_t output, void* data, size_t elements, char* error,
                             size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!graph || !data) throw std::invalid_argument("invalid output descriptor");
    auto& g = graph_of(graph);
    auto node = g.nodes.at(output);
    if (node->elements != elements) throw std::invalid_argument("output size mismatch");
    auto value = (node->dtype == kF16 || node->dtype == kBF16) ? g.as_f32(node) : node;
    HB_CHECK(hipStreamSynchronize(g.stream));
    std::vector<uint8_t> staging(elements * 4);
    HB_CHECK(hipMemcpy(staging.data(), value->data, elements * 4, hipMemcpyDeviceToHost));
    std::memcpy(data, staging.data(), elements * 4);
  });
}

extern "C" void* rs_mlx_weights_create(char* error, size_t capacity) {
  WeightStore* s = nullptr;
  guarded(error, capacity, [&] { s = new WeightStore; });
  return s;
}

extern "C" void rs_mlx_weights_destroy(void* store) { delete static_cast<WeightStore*>(store); }

// Loads every tensor of a safetensors file into the store as a device array
// (native/mlx_bridge.cpp:108-118): a name already held is an error, and so is
// any malformed header (safetensors.h); nothing is stored unless the whole
// file loads. A store holding any "mtp." tensor or a conv1d weight in the raw
// [C, 1, W] layout is marked shifted: its norm weights are offsets from 1.
extern "C" int rs_mlx_weights_load(void* store, const char* file, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!store || !file) throw std::invalid_argument("invalid weight load descriptor");
    auto& w = *static_cast<WeightStore*>(store);
    if (w.synthetic) throw std::invalid_argument("store describes a synthetic model");
    const SafeFile sf = read_safetensors_header(file);
    std::ifstream in(file, std::ios::binary);
    if (!in) throw std::invalid_argument("cannot open weight file");
    std::map<std::string, std::shared_ptr<Tensor>> staged;
    bool shift = false;
    std::vector<char> host;
    for (const SafeTensor& t : sf.tensors) {
      if (w.arrays.count(t.name) || staged.count(t.name)) throw std::invalid_argument("duplicate native parameter");
      auto tensor = Tensor::make(t.dtype, t.shape);
      const size_t bytes = size_t(t.end - t.begin);
      host.resize(bytes);
      in.seekg(std::streamoff(sf.payload + t.begin));
      if (!in.read(host.data(), std::streamsize(bytes))) throw std::invalid_argument("truncated tensor data");
      HB_CHECK(hipMemcpy(tensor->data, host.data(), bytes, hipMemcpyHostToDevice));
      const bool raw_conv = t.name.size() >= 13 && t.name.compare(t.name.size() - 13, 13, "conv1d.weight") == 0 &&
                            t.shape.back() != 1;
      if (t.name.find("mtp.") != std::string::npos || raw_conv) shift = true;
      staged.emplace(t.name, std::move(tensor));
    }
    for (auto& [name, tensor] : staged) w.arrays.emplace(name, std::move(tensor));
    if (shift) w.has_shift = true;
    w.forward_cache.reset();
  });
}

extern "C" int hb_safetensors_check(const char* file, size_t* tensors, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!file || !tensors) throw std::invalid_argument("hb_safetensors_check: descriptor");
    *tensors = read_safetensors_header(file).tensors.size();
  });
}

extern "C" int rs_mlx_parameter(void* graph, void* store, const char* name, const int32_t* shape, size_t rank,
                                int dtype, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!graph || !store || !name || !shape || rank == 0 || rank > 4)
      throw std::invalid_argument("invalid parameter descriptor");
    auto& g = graph_of(graph);
    auto& w = *static_cast<WeightStore*>(store);
    auto it = w.arrays.find(name);
    if (it == w.arrays.end()) throw std::invalid_argument("unknown parameter");
    const auto& v = *it->second;
    if (g.nodes.size() >= kMaxNodes || v.shape.size() != rank || !std::equal(shape, shape + rank, v.shape.begin()))
      throw std::invalid_argument("parameter shape mismatch");
    if (dtype < 0 || dtype > 4 || v.dtype != dtype) throw std::invalid_argument("parameter dtype mismatch");
    g.push(it->second);
  });
}

extern "C" int rs_mlx_weight_bytes(void* store, const char* name, const int32_t* shape, size_t rank, int dtype,
                                   size_t offset, uint8_t* output, size_t count, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!store || !name || !shape || rank == 0 || rank > 4 || dtype < 0 || dtype > 4 || !output || count == 0 ||
        count > 4 * 1024 * 1024)
      throw std::invalid_argument("weight byte export descriptor");
    auto& w = *static_cast<WeightStore*>(store);
    auto it = w.arrays.find(name);
    if (it == w.arrays.end()) throw std::invalid_argument("unknown parameter");
    const auto& v = *it->second;
    const size_t nbytes = v.elements * dtype_size(v.dtype);
    if (v.shape.size() != rank || v.dtype != dtype || offset > nbytes || count > nbytes - offset)
      throw std::invalid_argument("weight byte export bounds/type");
    for (size_t i = 0; i < rank; ++i)
      if (shape[i] != v.shape[i]) throw std::invalid_argument("weight byte export shape");
    std::vector<uint8_t> staging(count);
    HB_CHECK(hipMemcpy(staging.data(), static_cast<uint8_t*>(v.data) + offset, count, hipMemcpyDeviceToHost));
    std::memcpy(output, staging.data(), count);
  });
}
