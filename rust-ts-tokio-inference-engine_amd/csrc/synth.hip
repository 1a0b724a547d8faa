// Seeded synthetic tensors generated on the device: the benchmark model is
// random-init and 44 GB of 4-bit weights cannot be produced on the host in
// reasonable time. Values come from a counter-based generator (splitmix64 of
// seed and element index), so any slice can be regenerated independently;
// normals use the Box-Muller transform.
#include "synth.h"

namespace hb {
namespace {

__device__ inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Two independent uniforms in (0, 1] and [0, 1) from one 64-bit hash.
__device__ inline void uniform2(uint64_t seed, uint64_t i, float& u1, float& u2) {
  const uint64_t h = splitmix64(seed * 0xD1B54A32D192ED03ull + i);
  u1 = (float((h >> 40) & 0xFFFFFFull) + 1.f) * (1.f / 16777216.f);
  u2 = float((h >> 16) & 0xFFFFFFull) * (1.f / 16777216.f);
}

__device__ inline float normal(uint64_t seed, uint64_t i) {
  float u1, u2;
  uniform2(seed, i >> 1, u1, u2);
  const float r = sqrtf(-2.f * logf(u1));
  float s, c;
  sincosf(6.28318530717958647692f * u2, &s, &c);
  return (i & 1) ? r * s : r * c;
}

// One thread per 64-wide group: draw the group, affine-quantise it to 4 bits
// (scale = (max-min)/15 and bias = min, both rounded to bf16; code =
// clamp(rint((w - bias) / scale), 0, 15)) and pack 8 codes per word LSB first.
__global__ void random_q4_kernel(uint64_t seed, int N, int K, float std_dev, uint32_t* __restrict__ w,
                                 bf16_t* __restrict__ s, bf16_t* __restrict__ b) {
  const size_t gidx = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  const int G = K / 64;
  if (gidx >= size_t(N) * G) return;
  const size_t row = gidx / G;
  const int g = int(gidx % G);
  const uint64_t first = uint64_t(row) * K + uint64_t(g) * 64;
  float v[64];
  float lo = INFINITY, hi = -INFINITY;
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    v[j] = normal(seed, first + j) * std_dev;
    lo = fminf(lo, v[j]);
    hi = fmaxf(hi, v[j]);
  }
  const bf16_t sb = f32_to_bf16(fmaxf((hi - lo) / 15.f, 1e-8f));
  const bf16_t bb = f32_to_bf16(lo);
  const float scale = bf16_to_f32(sb), bias = bf16_to_f32(bb);
  s[gidx] = sb;
  b[gidx] = bb;
  uint32_t* out = w + size_t(row) * (K / 8) + g * 8;
#pragma unroll
  for (int wd = 0; wd < 8; ++wd) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float q = fminf(fmaxf(rintf((v[wd * 8 + j] - bias) / scale), 0.f), 15.f);
      word |= uint32_t(q) << (4 * j);
    }
    out[wd] = word;
  }
}

__global__ void random_normal_kernel(uint64_t seed, size_t n, float std_dev, float mean, int dtype, void* out) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  const float v = mean + std_dev * normal(seed, i);
  if (dtype == 0)
    static_cast<float*>(out)[i] = v;
  else
    static_cast<bf16_t*>(out)[i] = f32_to_bf16(v);
}

__global__ void random_uniform_kernel(uint64_t seed, size_t n, float lo, float hi, int dtype, void* out) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  float u1, u2;
  uniform2(seed, i, u1, u2);
  const float v = lo + (hi - lo) * u2;
  if (dtype == 0)
    static_cast<float*>(out)[i] = v;
  else
    static_cast<bf16_t*>(out)[i] = f32_to_bf16(v);
}

__global__ void random_ints_kernel(uint64_t seed, size_t n, uint32_t bound, uint32_t* out) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  out[i] = uint32_t(splitmix64(seed * 0xD1B54A32D192ED03ull + i) % bound);
}

inline unsigned blocks(size_t n) { return unsigned((n + 255) / 256); }

}  // namespace

void random_q4(uint64_t seed, int N, int K, float std_dev, uint32_t* w, bf16_t* s, bf16_t* b, hipStream_t stream) {
  require(w && s && b, "random_q4: null pointer");
  require(N > 0 && K > 0 && K % 64 == 0, "random_q4: K must be a multiple of 64");
  const size_t groups = size_t(N) * (K / 64);
  hipLaunchKernelGGL(random_q4_kernel, dim3(blocks(groups)), dim3(256), 0, stream, seed, N, K, std_dev, w, s, b);
  HB_CHECK(hipGetLastError());
}

void random_normal(uint64_t seed, size_t n, float std_dev, float mean, int dtype, void* out, hipStream_t stream) {
  require(out && (dtype == 0 || dtype == 4), "random_normal: dtype must be 0 (f32) or 4 (bf16)");
  if (!n) return;
  hipLaunchKernelGGL(random_normal_kernel, dim3(blocks(n)), dim3(256), 0, stream, seed, n, std_dev, mean, dtype, out);
  HB_CHECK(hipGetLastError());
}

void random_uniform(uint64_t seed, size_t n, float lo, float hi, int dtype, void* out, hipStream_t stream) {
  require(out && (dtype == 0 || dtype == 4), "random_uniform: dtype must be 0 (f32) or 4 (bf16)");
  if (!n) return;
  hipLaunchKernelGGL(random_uniform_kernel, dim3(blocks(n)), dim3(256), 0, stream, seed, n, lo, hi, dtype, out);
  HB_CHECK(hipGetLastError());
}

void random_ints(uint64_t seed, size_t n, uint32_t bound, uint32_t* out, hipStream_t stream) {
  require(out && bound > 0, "random_ints: invalid arguments");
  if (!n) return;
  hipLaunchKernelGGL(random_ints_kernel, dim3(blocks(n)), dim3(256), 0, stream, seed, n, bound, out);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
