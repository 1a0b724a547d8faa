#include "ops.h"

namespace hb {
namespace {

constexpr int kBlock = 256;
inline unsigned blocks_for(size_t n) { return unsigned((n + kBlock - 1) / kBlock); }

__global__ void f32_to_bf16_kernel(const float* __restrict__ src, bf16_t* __restrict__ dst, size_t n) {
  size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) dst[i] = f32_to_bf16(src[i]);
}

__device__ inline float f16_bits_to_f32(uint16_t v) { return float(__builtin_bit_cast(_Float16, v)); }

__global__ void half_to_f32_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst, size_t n, bool f16) {
  size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) dst[i] = f16 ? f16_bits_to_f32(src[i]) : bf16_to_f32(src[i]);
}

__global__ void f16_to_bf16_kernel(const uint16_t* __restrict__ src, bf16_t* __restrict__ dst, size_t n) {
  size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) dst[i] = f32_to_bf16(f16_bits_to_f32(src[i]));
}

struct BinArgs {
  int64_t shape[kMaxRank], as[kMaxRank], bs[kMaxRank];
};

__global__ void binary_kernel(int op, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y,
                              BinArgs d, size_t n) {
  size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  size_t r = i;
  int64_t ao = 0, bo = 0;
  for (int ax = kMaxRank - 1; ax >= 0; --ax) {
    const int64_t c = int64_t(r % size_t(d.shape[ax]));
    r /= size_t(d.shape[ax]);
    ao += c * d.as[ax];
    bo += c * d.bs[ax];
  }
  const float u = a[ao], v = b[bo];
  y[i] = op == 0 ? u + v : op == 1 ? u * v : u - v;
}

__global__ void matmul_kernel(const float* __restrict__ a, const float* __restrict__ w, float* __restrict__ y, int wb,
                              int M, int N, int K) {
  __shared__ float ta[16][17], tw[16][17];
  const int bz = blockIdx.z, row = blockIdx.y * 16 + threadIdx.y, col = blockIdx.x * 16 + threadIdx.x;
  const float* ab = a + size_t(bz) * M * K;
  const float* wbp = w + (wb == 1 ? 0 : size_t(bz) * K * N);
  float acc = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    const int ka = k0 + threadIdx.x, kw = k0 + threadIdx.y;
    ta[threadIdx.y][threadIdx.x] = (row < M && ka < K) ? ab[size_t(row) * K + ka] : 0.f;
    tw[threadIdx.y][threadIdx.x] = (kw < K && col < N) ? wbp[size_t(kw) * N + col] : 0.f;
    __syncthreads();
    for (int kk = 0; kk < 16; ++kk) acc += ta[threadIdx.y][kk] * tw[kk][threadIdx.x];
    __syncthreads();
  }
  if (row < M && col < N) y[size_t(bz) * M * N + size_t(row) * N + col] = acc;
}

__global__ void rms_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, int width,
                           float eps) {
  const int row = blockIdx.x;
  const float* xr = x + size_t(row) * width;
  float s = 0.f;
  for (int c = threadIdx.x; c < width; c += blockDim.x) s += xr[c] * xr[c];
  __shared__ float part[kBlock / 64];
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < int(blockDim.x >> 6); ++i) tot += part[i];
  const float inv = 1.f / sqrtf(tot / float(width) + eps);
  for (int c = threadIdx.x; c < width; c += blockDim.x) y[size_t(row) * width + c] = xr[c] * inv * (w ? w[c] : 1.f);
}

__global__ void silu_kernel(const float* __restrict__ x, float* __restrict__ y, size_t n) {
  size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) {
    const float v = x[i];
    y[i] = v / (1.f + expf(-v));
  }
}

}  // namespace

void f32_to_bf16_n(const float* src, bf16_t* dst, size_t n, hipStream_t s) {
  if (!n) return;
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(blocks_for(n)), dim3(kBlock), 0, s, src, dst, n);
  HB_CHECK(hipGetLastError());
}

void half_to_f32_n(const uint16_t* src, float* dst, size_t n, bool is_f16, hipStream_t s) {
  if (!n) return;
  hipLaunchKernelGGL(half_to_f32_kernel, dim3(blocks_for(n)), dim3(kBlock), 0, s, src, dst, n, is_f16);
  HB_CHECK(hipGetLastError());
}

void f16_to_bf16_n(const uint16_t* src, bf16_t* dst, size_t n, hipStream_t s) {
  if (!n) return;
  hipLaunchKernelGGL(f16_to_bf16_kernel, dim3(blocks_for(n)), dim3(kBlock), 0, s, src, dst, n);
  HB_CHECK(hipGetLastError());
}

void binary_f32(int op, const float* a, Dims astride, const float* b, Dims bstride, float* y, Dims shape,
                hipStream_t s) {
  BinArgs d;
  size_t n = 1;
  for (int i = 0; i < kMaxRank; ++i) {
    d.shape[i] = shape[i];
    d.as[i] = astride[i];
    d.bs[i] = bstride[i];
    n *= size_t(shape[i]);
  }
  if (!n) return;
  hipLaunchKernelGGL(binary_kernel, dim3(blocks_for(n)), dim3(kBlock), 0, s, op, a, b, y, d, n);
  HB_CHECK(hipGetLastError());
}

void matmul_f32(const float* a, const float* w, float* y, int batch, int wbatch, int M, int N, int K, hipStream_t s) {
  const dim3 grid((N + 15) / 16, (M + 15) / 16, batch);
  hipLaunchKernelGGL(matmul_kernel, grid, dim3(16, 16), 0, s, a, w, y, wbatch, M, N, K);
  HB_CHECK(hipGetLastError());
}

void rms_norm_f32(const float* x, const float* weight, float* y, int rows, int width, float eps, hipStream_t s) {
  if (!rows) return;
  hipLaunchKernelGGL(rms_kernel, dim3(rows), dim3(kBlock), 0, s, x, weight, y, width, eps);
  HB_CHECK(hipGetLastError());
}

void silu_f32(const float* x, float* y, size_t n, hipStream_t s) {
  if (!n) return;
  hipLaunchKernelGGL(silu_kernel, dim3(blocks_for(n)), dim3(kBlock), 0, s, x, y, n);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
