// Checkpoint-layout (MLX) projections for quantization overrides and dense
// BF16 modules; see generic.h. One wave per output value: the 64 lanes split
// K, dequantize their codes in place and reduce.
#include "generic.h"

namespace hb {
namespace {

constexpr int kGenWaves = 4;

// weight (row, column c) of a module: s * q + b, q the bits-wide code at bit
// c * bits of the row's LSB-first stream (codes of 3, 5 or 6 bits may straddle
// two words)
__device__ inline float deq(const QMod& m, size_t row, int c) {
  const uint32_t* r = m.w + row * m.words_per_row();
  const size_t bit = size_t(c) * m.bits;
  const size_t word = bit >> 5;
  const unsigned shift = unsigned(bit & 31);
  uint64_t v = r[word];
  if (shift + m.bits > 32) v |= uint64_t(r[word + 1]) << 32;
  const float q = float(uint32_t(v >> shift) & ((1u << m.bits) - 1u));
  const size_t g = row * (m.K / m.group) + c / m.group;
  return bf16_to_f32(m.s[g]) * q + bf16_to_f32(m.b[g]);
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ __launch_bounds__(64 * kGenWaves) void moe_generic_gate_up_kernel(
    const bf16_t* __restrict__ x, int ldx, const int32_t* __restrict__ order, const int32_t* __restrict__ idx, int top,
    int P, QMod gate, QMod up, QMod sgate, QMod sup, bf16_t* __restrict__ act) {
  const int lane = threadIdx.x & 63, n = blockIdx.x * kGenWaves + (threadIdx.x >> 6), j = blockIdx.y;
  const int I = gate.rows;
  if (n >= I) return;  // uniform over the wave
  // the row's modules (workgroup-uniform choice)
  const bool routed = j < P;
  const int p = routed ? order[j] : 0;
  const int token = routed ? p / top : j - P;
  const size_t row = routed ? size_t(idx[p]) * I + n : size_t(n);
  const QMod g = routed ? gate : sgate, u = routed ? up : sup;
  const bf16_t* xr = x + size_t(token) * ldx;
  float ga = 0.f, ua = 0.f;
  for (int c = lane; c < gate.K; c += 64) {
    const float xv = bf16_to_f32(xr[c]);
    ga += xv * deq(g, row, c);
    ua += xv * deq(u, row, c);
  }
  ga = wave_sum(ga);
  ua = wave_sum(ua);
  if (lane == 0) act[size_t(j) * I + n] = f32_to_bf16(ga / (1.f + __expf(-ga)) * ua);
}

__global__ __launch_bounds__(64 * kGenWaves) void moe_generic_down_kernel(
    const bf16_t* __restrict__ act, const int32_t* __restrict__ order, const int32_t* __restrict__ idx, int top, int P,
    QMod down, QMod sdown, bf16_t* __restrict__ dout) {
  const int lane = threadIdx.x & 63, n = blockIdx.x * kGenWaves + (threadIdx.x >> 6), j = blockIdx.y;
  const int H = down.rows, I = down.K;
  if (n >= H) return;
  const bool routed = j < P;
  const QMod d = routed ? down : sdown;
  const size_t row = routed ? size_t(idx[order[j]]) * H + n : size_t(n);
  const bf16_t* ar = act + size_t(j) * I;
  float acc = 0.f;
  for (int c = lane; c < I; c += 64) acc += bf16_to_f32(ar[c]) * deq(d, row, c);
  acc = wave_sum(acc);
  if (lane == 0) dout[size_t(j) * H + n] = f32_to_bf16(acc);
}

__global__ __launch_bounds__(256) void embed_generic_kernel(const uint32_t* __restrict__ tokens, QMod emb,
                                                            float* __restrict__ x) {
  const int t = blockIdx.x;
  const size_t row = tokens[t];
  for (int c = threadIdx.x; c < emb.K; c += 256) x[size_t(t) * emb.K + c] = deq(emb, row, c);
}

template <int OUT>
__global__ __launch_bounds__(64 * kGenWaves) void dense_bf16_kernel(const bf16_t* __restrict__ x, int K,
                                                                    const bf16_t* __restrict__ W, int N,
                                                                    void* __restrict__ y, int ldy) {
  const int lane = threadIdx.x & 63, n = blockIdx.x * kGenWaves + (threadIdx.x >> 6), m = blockIdx.y;
  if (n >= N) return;
  const bf16_t* xr = x + size_t(m) * K;
  const bf16_t* wr = W + size_t(n) * K;
  float acc = 0.f;
  for (int c = lane; c < K; c += 64) acc += bf16_to_f32(xr[c]) * bf16_to_f32(wr[c]);
  acc = wave_sum(acc);
  if (lane) return;
  const size_t o = size_t(m) * ldy + n;
  if (OUT == 0)
    static_cast<bf16_t*>(y)[o] = f32_to_bf16(acc);
  else if (OUT == 1)
    static_cast<float*>(y)[o] = acc;
  else
    static_cast<float*>(y)[o] += acc;
}

void check_mod(const QMod& m, const char* what) {
  require(m.w && m.s && m.b && m.rows > 0 && m.K > 0, what);
  require((m.group == 32 || m.group == 64 || m.group == 128) && m.K % m.group == 0, what);
  require(m.bits == 2 || m.bits == 3 || m.bits == 4 || m.bits == 5 || m.bits == 6 || m.bits == 8, what);
  require((size_t(m.K) * m.bits) % 32 == 0, what);
}

}  // namespace

void moe_generic_gate_up(const bf16_t* x, int ldx, const int32_t* order, const int32_t* idx, int top, int P, int T,
                         const QMod& gate, const QMod& up, const QMod& sgate, const QMod& sup, bf16_t* act,
                         hipStream_t stream) {
  for (const QMod* m : {&gate, &up, &sgate, &sup}) check_mod(*m, "moe_generic_gate_up: module descriptor");
  require(up.rows == gate.rows && sgate.rows == gate.rows && sup.rows == gate.rows, "moe_generic_gate_up: widths");
  require(up.K == gate.K && sgate.K == gate.K && sup.K == gate.K && ldx >= gate.K, "moe_generic_gate_up: K");
  require(top > 0 && P == T * top, "moe_generic_gate_up: pairs");
  if (T == 0) return;
  hipLaunchKernelGGL(moe_generic_gate_up_kernel, dim3((gate.rows + kGenWaves - 1) / kGenWaves, P + T),
                     dim3(64 * kGenWaves), 0, stream, x, ldx, order, idx, top, P, gate, up, sgate, sup, act);
  HB_CHECK(hipGetLastError());
}

void moe_generic_down(const bf16_t* act, const int32_t* order, const int32_t* idx, int top, int P, int T,
                      const QMod& down, const QMod& sdown, bf16_t* dout, hipStream_t stream) {
  check_mod(down, "moe_generic_down: module descriptor");
  check_mod(sdown, "moe_generic_down: module descriptor");
  require(sdown.rows == down.rows && sdown.K == down.K, "moe_generic_down: shapes");
  require(top > 0 && P == T * top, "moe_generic_down: pairs");
  if (T == 0) return;
  hipLaunchKernelGGL(moe_generic_down_kernel, dim3((down.rows + kGenWaves - 1) / kGenWaves, P + T),
                     dim3(64 * kGenWaves), 0, stream, act, order, idx, top, P, down, sdown, dout);
  HB_CHECK(hipGetLastError());
}

void embed_generic(const uint32_t* tokens, int T, const QMod& emb, float* x, hipStream_t stream) {
  check_mod(emb, "embed_generic: module descriptor");
  if (T == 0) return;
  hipLaunchKernelGGL(embed_generic_kernel, dim3(T), dim3(256), 0, stream, tokens, emb, x);
  HB_CHECK(hipGetLastError());
}

void dense_bf16(const bf16_t* x, int M, int K, const bf16_t* W, int N, void* y, int out_mode, int ldy,
                hipStream_t stream) {
  require(x && W && y && M >= 0 && N > 0 && K > 0 && ldy >= N, "dense_bf16: shape");
  require(out_mode >= 0 && out_mode <= 2, "dense_bf16: output mode");
  if (M == 0) return;
  const dim3 grid((N + kGenWaves - 1) / kGenWaves, M), block(64 * kGenWaves);
  if (out_mode == 0)
    hipLaunchKernelGGL(dense_bf16_kernel<0>, grid, block, 0, stream, x, K, W, N, y, ldy);
  else if (out_mode == 1)
    hipLaunchKernelGGL(dense_bf16_kernel<1>, grid, block, 0, stream, x, K, W, N, y, ldy);
  else
    hipLaunchKernelGGL(dense_bf16_kernel<2>, grid, block, 0, stream, x, K, W, N, y, ldy);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
