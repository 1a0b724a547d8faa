// Embedding gather + dequantisation and RMSNorm for the residual stream.
#include "norm.h"

#include "q4_device.h"

namespace hb {
namespace {

constexpr int kNormThreads = 256;

// One workgroup per token; each thread dequantises 8 columns (one packed word).
__global__ __launch_bounds__(kNormThreads) void embed_gather_kernel(const uint32_t* __restrict__ tokens,
                                                                    const uint32_t* __restrict__ w,
                                                                    const bf16_t* __restrict__ s,
                                                                    const bf16_t* __restrict__ b, int H,
                                                                    float* __restrict__ out) {
  const int t = blockIdx.x;
  const size_t row = tokens[t];
  const int words = H / 8, G = H / 64;
  for (int wd = threadIdx.x; wd < words; wd += blockDim.x) {
    const uint32_t q = w[row * words + wd];
    const int g = wd / 8;
    const float sc = bf16_to_f32(s[row * G + g]), bi = bf16_to_f32(b[row * G + g]);
#pragma unroll
    for (int j = 0; j < 8; ++j) out[size_t(t) * H + wd * 8 + j] = sc * float((q >> (4 * j)) & 0xFu) + bi;
  }
}

// 32-bit words are copied as integers (no float arithmetic touches them).
__global__ void gather_rows_kernel(const uint32_t* __restrict__ src, int ld_src, const int32_t* __restrict__ idx,
                                   int width, uint32_t* __restrict__ dst, int ld_dst) {
  const int i = blockIdx.x;
  const uint32_t* s = src + size_t(idx[i]) * ld_src;
  for (int c = threadIdx.x; c < width; c += blockDim.x) dst[size_t(i) * ld_dst + c] = s[c];
}

// One workgroup per row; a thread keeps its (up to kNormChunks) 8-column
// chunks in registers, so the row is read once.
constexpr int kNormChunks = 4;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* __restrict__ x, int ld_x,
                                                               const float* __restrict__ w, int H, float eps,
                                                               bf16_t* __restrict__ out, int ld_out,
                                                               float* __restrict__ out_f32,
                                                               float* __restrict__ gsum) {
  const int t = blockIdx.x, nch = H / 8;
  const float* xr = x + size_t(t) * ld_x;
  float v[kNormChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < nch) {
      const float4 a = reinterpret_cast<const float4*>(xr)[2 * c], b = reinterpret_cast<const float4*>(xr)[2 * c + 1];
      v[j][0] = a.x, v[j][1] = a.y, v[j][2] = a.z, v[j][3] = a.w, v[j][4] = b.x, v[j][5] = b.y, v[j][6] = b.z,
      v[j][7] = b.w;
#pragma unroll
      for (int q = 0; q < 8; ++q) ss += v[j][q] * v[j][q];
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  __shared__ float part[kNormThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
  const float inv = 1.f / sqrtf(tot / float(H) + eps);
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c >= nch) continue;
    const float4 wa = reinterpret_cast<const float4*>(w)[2 * c], wb = reinterpret_cast<const float4*>(w)[2 * c + 1];
    const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
    float y[8];
    uint32_t packed[4];
#pragma unroll
    for (int q = 0; q < 8; ++q) y[q] = v[j][q] * inv * wv[q];
#pragma unroll
    for (int q = 0; q < 4; ++q) packed[q] = uint32_t(f32_to_bf16(y[2 * q])) | (uint32_t(f32_to_bf16(y[2 * q + 1])) << 16);
    const uint4 pv = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    *reinterpret_cast<uint4*>(out + size_t(t) * ld_out + 8 * c) = pv;
    if (gsum) {  // the 8 lanes of a 64-column group are all live (H % 64 == 0)
      const float gsv = sum8_lanes(bf16x8_pair_sum(pv));
      if ((c & 7) == 0) gsum[size_t(t) * (H / 64) + c / 8] = gsv;
    }
    if (out_f32) {
      float4* o = reinterpret_cast<float4*>(out_f32 + size_t(t) * H + 8 * c);
      o[0] = make_float4(y[0], y[1], y[2], y[3]);
      o[1] = make_float4(y[4], y[5], y[6], y[7]);
    }
  }
}

}  // namespace

void embed_gather(const uint32_t* tokens, int T, const uint32_t* w, const bf16_t* s, const bf16_t* b, int H,
                  float* out, hipStream_t stream) {
  require(tokens && w && s && b && out, "embed_gather: null pointer");
  require(H % 64 == 0, "embed_gather: hidden must be a multiple of 64");
  if (T <= 0) return;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(T), dim3(kNormThreads), 0, stream, tokens, w, s, b, H, out);
  HB_CHECK(hipGetLastError());
}

void rmsnorm(const float* x, int ld_x, const float* w, int T, int H, float eps, bf16_t* out, int ld_out,
             hipStream_t stream, float* out_f32, float* gsum) {
  require(x && w && out, "rmsnorm: null pointer");
  require(H % 8 == 0 && H <= 8 * kNormThreads * kNormChunks && ld_x % 4 == 0 && ld_out % 8 == 0,
          "rmsnorm: hidden must be a multiple of 8 and at most 8192, strides 16-byte aligned");
  require(!gsum || H % 64 == 0, "rmsnorm: group sums need a hidden size that is a multiple of 64");
  if (T <= 0) return;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(kNormThreads), 0, stream, x, ld_x, w, H, eps, out, ld_out,
                     out_f32, gsum);
  HB_CHECK(hipGetLastError());
}

void gather_rows_f32(const float* src, int ld_src, const int32_t* idx, int n, int width, float* dst, int ld_dst,
                     hipStream_t stream) {
  require(src && idx && dst, "gather_rows_f32: null pointer");
  if (n <= 0) return;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(n), dim3(256), 0, stream, reinterpret_cast<const uint32_t*>(src),
                     ld_src, idx, width, reinterpret_cast<uint32_t*>(dst), ld_dst);
  HB_CHECK(hipGetLastError());
}

void gather_rows_i32(const int32_t* src, int ld_src, const int32_t* idx, int n, int width, int32_t* dst, int ld_dst,
                     hipStream_t stream) {
  gather_rows_f32(reinterpret_cast<const float*>(src), ld_src, idx, n, width, reinterpret_cast<float*>(dst), ld_dst,
                  stream);
}

}  // namespace hb
