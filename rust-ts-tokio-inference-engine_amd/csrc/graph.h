// Device tensors and the eager graph behind the rs_mlx_* entry points.
#pragma once
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "hb_common.h"

namespace hb {

enum Dtype : int { kF32 = 0, kI32 = 1, kU32 = 2, kF16 = 3, kBF16 = 4 };
constexpr size_t kMaxNodes = 256;  // native/mlx_bridge.cpp:46

size_t dtype_size(int dtype);

struct Tensor {
  void* data = nullptr;
  int dtype = kF32;
  std::vector<int32_t> shape;
  size_t elements = 0;
  bool owned = true;
  Tensor() = default;
  Tensor(const Tensor&) = delete;
  Tensor& operator=(const Tensor&) = delete;
  ~Tensor();
  static std::shared_ptr<Tensor> make(int dtype, std::vector<int32_t> shape);
  template <class T>
  T* as() const {
    return static_cast<T*>(data);
  }
};

struct Graph {
  bool gpu;
  hipStream_t stream = nullptr;
  std::vector<std::shared_ptr<Tensor>> nodes;
  std::vector<std::shared_ptr<Tensor>> scratch;  // temporaries kept alive until destroy
  explicit Graph(bool gpu);
  ~Graph();
  const Tensor& at(uint32_t id) const;
  void push(std::shared_ptr<Tensor> t);
  void keep(std::shared_ptr<Tensor> t) { scratch.push_back(std::move(t)); }
  std::shared_ptr<Tensor> as_f32(const std::shared_ptr<Tensor>& t);
  std::shared_ptr<Tensor> as_bf16(const std::shared_ptr<Tensor>& t);
};

// rs_mlx_weights_* store: named device tensors, per-module quantisation
// overrides (rs_qwen_quant) and, for the benchmark model, a seeded synthetic
// descriptor (hb_weights_synthetic) from which device sessions generate the
// random-init weights on the device.
struct WeightStore {
  std::map<std::string, std::shared_ptr<Tensor>> arrays;
  std::map<std::string, std::pair<int, int>> quant;  // module -> (group, bits)
  bool has_shift = false;  // norm weights are offsets from 1 (native/mlx_bridge.cpp:115)
  bool synthetic = false;
  uint64_t seed = 0;
  int part = 0;                          // 0 target model, 1 MTP sidecar
  std::shared_ptr<void> forward_cache;   // session reused by rs_qwen_forward
  std::vector<uint8_t> forward_key;      // its configuration bytes
};

}  // namespace hb
