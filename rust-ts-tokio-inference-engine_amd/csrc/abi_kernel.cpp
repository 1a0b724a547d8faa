// rs_mlx_kernel: the fused-operator graph entry (native/mlx_bridge.cpp:132-174).
// Op codes, operand order and integer/float arguments follow the reference;
// the operand checks are the ones its Rust callers apply before building the
// node (src/serving/native_ops.rs:53-244), so a malformed descriptor fails
// here with a message instead of reaching a kernel.
//   1 rope(x; dims, offset; base)             -> x's shape
//   2 sdpa(q, k, v; causal; scale)            -> [B][Hq][Tq][Dv]
//   3 gated delta(q, k, v, decay, beta, state) -> y [B][T][Hv][Dv], state [B][Hv][Dv][Dk]
//   4 route(logits; top)                      -> idx u32 [rows][top], scores [rows][top]
//   5 gather qmm(x, w, scales, biases, idx; group, bits) -> [rows][top][N]
//   6 mix(experts, scores)                    -> [rows][N]
//   7 silu(x), 8 flat concat(a, b)
#include <cmath>
#include <vector>

#include "../../include/hip_bridge.h"
#include "graph.h"
#include "graph_ops.h"
#include "ops.h"

using namespace hb;

namespace {

bool is_float(int dtype) { return dtype == kF32 || dtype == kF16 || dtype == kBF16; }

int64_t product(const std::vector<int32_t>& s, size_t from, size_t to) {
  int64_t p = 1;
  for (size_t i = from; i < to; ++i) p *= s[i];
  return p;
}

}  // namespace

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
    auto integer = [&](size_t n) {
      if (!ints || n >= ni) throw std::invalid_argument("kernel integer missing");
      return ints[n];
    };
    auto scalar = [&](size_t n) {
      if (!floats || n >= nf) throw std::invalid_argument("kernel scalar missing");
      return floats[n];
    };
    auto f32 = [&](size_t n) {
      auto t = at(n);
      require(is_float(t->dtype), "kernel operand must be floating point");
      auto f = g.as_f32(t);
      if (f != t) g.keep(f);
      return f;
    };
    std::vector<std::shared_ptr<Tensor>> outputs;
    if (op == 1) {
      auto x = f32(0);
      const int dims = integer(0), offset = integer(1);
      const float base = scalar(0);
      const auto& s = x->shape;
      require(s.size() >= 2 && s.size() <= 4 && dims > 0 && dims % 2 == 0 && dims <= s.back() && offset >= 0 &&
                  offset <= 262144 && std::isfinite(base) && base > 0.f,
              "invalid RoPE descriptor");
      auto y = Tensor::make(kF32, s);
      graph_rope(x->as<float>(), y->as<float>(), int(product(s, 0, s.size() - 2)), s[s.size() - 2], s.back(), dims,
                 offset, base, g.stream);
      outputs.push_back(y);
    } else if (op == 2) {
      auto q = f32(0), k = f32(1), v = f32(2);
      const bool causal = integer(0) != 0;
      const float scale = scalar(0);
      const auto &qs = q->shape, &ks = k->shape, &vs = v->shape;
      require(qs.size() == 4 && ks.size() == 4 && vs.size() == 4, "attention dtype/rank");
      require(qs[0] == ks[0] && ks[0] == vs[0] && ks[1] == vs[1] && ks[1] > 0 && qs[1] % ks[1] == 0 &&
                  ks[2] == vs[2] && ks[2] > 0 && qs[3] == ks[3] && qs[2] <= ks[2] && std::isfinite(scale) &&
                  scale > 0.f,
              "attention shape/scale mismatch");
      auto scores = Tensor::make(kF32, {qs[0], qs[1], qs[2], ks[2]});
      auto y = Tensor::make(kF32, {qs[0], qs[1], qs[2], vs[3]});
      graph_sdpa(q->as<float>(), k->as<float>(), v->as<float>(), scores->as<float>(), y->as<float>(), qs[0], qs[1],
                 ks[1], qs[2], ks[2], qs[3], vs[3], scale, causal, g.stream);
      g.keep(scores);
      outputs.push_back(y);
    } else if (op == 3) {
      auto q = f32(0), k = f32(1), v = f32(2), decay = f32(3), beta = f32(4), state = f32(5);
      const auto &qs = q->shape, &vs = v->shape;
      require(qs.size() == 4 && q->shape == k->shape && vs.size() == 4, "gated-delta dtype/rank");
      const int B = qs[0], T = qs[1], Hk = qs[2], Dk = qs[3], Hv = vs[2], Dv = vs[3];
      require(T <= 128 && vs[0] == B && vs[1] == T && Hk > 0 && Hv % Hk == 0 &&
                  decay->shape == std::vector<int32_t>{B, T, Hv} && beta->shape == std::vector<int32_t>{B, T, Hv} &&
                  state->shape == std::vector<int32_t>{B, Hv, Dv, Dk},
              "gated-delta state/head mismatch");
      auto y = Tensor::make(kF32, {B, T, Hv, Dv});
      auto s = Tensor::make(kF32, {B, Hv, Dv, Dk});
      graph_gated_delta(q->as<float>(), k->as<float>(), v->as<float>(), decay->as<float>(), beta->as<float>(),
                        state->as<float>(), y->as<float>(), s->as<float>(), B, T, Hk, Hv, Dk, Dv, g.stream);
      outputs.push_back(y);
      outputs.push_back(s);
    } else if (op == 4) {
      auto logits = f32(0);
      const int top = integer(0);
      const auto& ls = logits->shape;
      require(ls.size() == 2 && top > 0 && top <= ls[1], "invalid expert top-k");
      auto idx = Tensor::make(kU32, {ls[0], top});
      auto scores = Tensor::make(kF32, {ls[0], top});
      graph_route_topk(logits->as<float>(), idx->as<uint32_t>(), scores->as<float>(), ls[0], ls[1], top, g.stream);
      outputs.push_back(idx);
      outputs.push_back(scores);
    } else if (op == 5) {
      const int group = integer(0), bits = integer(1);
      require((bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8) &&
                  (group == 32 || group == 64 || group == 128),
              "unsupported expert quantization");
      auto x = f32(0);
      auto w = at(1), idx = at(4);
      auto sc_raw = at(2), bi_raw = at(3);
      const auto &xs = x->shape, &ws = w->shape, &is = idx->shape;
      require(xs.size() == 2 && w->dtype == kU32 && ws.size() == 3 && is_float(sc_raw->dtype) &&
                  sc_raw->dtype == bi_raw->dtype && sc_raw->shape.size() == 3 && sc_raw->shape == bi_raw->shape &&
                  idx->dtype == kU32 && is.size() == 2 && is[0] == xs[0],
              "expert dtype/rank mismatch");
      require(xs[1] % group == 0 && int64_t(ws[2]) * 32 == int64_t(xs[1]) * bits &&
                  sc_raw->shape == std::vector<int32_t>{ws[0], ws[1], xs[1] / group},
              "expert packed shape mismatch");
      // the indices select weight rows: every one must name an expert
      std::vector<uint32_t> host(idx->elements);
      if (!host.empty()) {
        HB_CHECK(hipMemcpyAsync(host.data(), idx->data, host.size() * 4, hipMemcpyDeviceToHost, g.stream));
        HB_CHECK(hipStreamSynchronize(g.stream));
      }
      for (uint32_t e : host) require(e < uint32_t(ws[0]), "untrusted or out-of-range expert indices");
      auto sc = f32(2), bi = f32(3);
      auto y = Tensor::make(kF32, {xs[0], is[1], ws[1]});
      graph_gather_qmm(x->as<float>(), w->as<uint32_t>(), sc->as<float>(), bi->as<float>(), idx->as<uint32_t>(),
                       y->as<float>(), xs[0], is[1], ws[1], xs[1], group, bits, g.stream);
      outputs.push_back(y);
    } else if (op == 6) {
      auto ex = f32(0), sc = f32(1);
      const auto &es = ex->shape, &ss = sc->shape;
      require(es.size() == 3 && ss.size() == 2 && ss[0] == es[0] && ss[1] == es[1], "expert mix shape/dtype mismatch");
      auto y = Tensor::make(kF32, {es[0], es[2]});
      graph_mix(ex->as<float>(), sc->as<float>(), y->as<float>(), es[0], es[1], es[2], g.stream);
      outputs.push_back(y);
    } else if (op == 7) {
      auto x = f32(0);
      auto y = Tensor::make(kF32, x->shape);
      silu_f32(x->as<float>(), y->as<float>(), x->elements, g.stream);
      outputs.push_back(y);
    } else if (op == 8) {
      auto a = f32(0), b = f32(1);
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
