// rs_mlx_kernel: the fused-operator graph entry (native/mlx_bridge.cpp:132-174).
// op 7 silu and op 8 flat concat are served here; the remaining codes are
// routed to the hot-path kernels as they are wired in.
#include <vector>

#include "../../include/hip_bridge.h"
#include "graph.h"
#include "ops.h"

using namespace hb;

extern "C" int rs_mlx_kernel(void* graph, int op, const uint32_t* inputs, size_t count, const int32_t* ints,
                             size_t ni, const float* floats, size_t nf, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (!graph || !inputs) throw std::invalid_argument("invalid kernel descriptor");
    auto& g = *static_cast<Graph*>(graph);
    auto at = [&](size_t n) -> std::shared_ptr<Tensor> {
      if (n >= count) throw std::invalid_argument("kernel operand missing");
      if (inputs[n] >= g.nodes.size()) throw std::invalid_argument("invalid node reference");
      return g.nodes[inputs[n]];
    };
    (void)ints;
    (void)ni;
    (void)floats;
    (void)nf;
    std::vector<std::shared_ptr<Tensor>> outputs;
    if (op == 7) {
      auto x = g.as_f32(at(0));
      auto y = Tensor::make(kF32, x->shape);
      silu_f32(x->as<float>(), y->as<float>(), x->elements, g.stream);
      outputs.push_back(y);
    } else if (op == 8) {
      auto a = g.as_f32(at(0)), b = g.as_f32(at(1));
      auto y = Tensor::make(kF32, {int32_t(a->elements + b->elements)});
      HB_CHECK(hipMemcpyAsync(y->data, a->data, a->elements * 4, hipMemcpyDeviceToDevice, g.stream));
      HB_CHECK(hipMemcpyAsync(y->as<float>() + a->elements, b->data, b->elements * 4, hipMemcpyDeviceToDevice,
                              g.stream));
      outputs.push_back(y);
    } else {
      throw std::invalid_argument("unsupported native kernel");
    }
    if (g.nodes.size() + outputs.size() > kMaxNodes) throw std::invalid_argument("kernel node cap");
    for (auto& o : outputs) g.push(o);
  });
}
