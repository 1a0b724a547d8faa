// Affine 4-bit group-64 quantised GEMV/GEMM for gfx950.
//
// MFMA path (4-bit, group 64, interleaved layout), one 32x32 output tile per
// workgroup, v_mfma_f32_32x32x16_bf16:
//   D[m][n] += A[m][k] * B[k][n],  A = x rows (bf16), B = 128 + code (bf16, exact).
// Each lane owns weight row n = lane%32 and the k-half h = lane/32 of every
// 64-wide group: one 16-byte load brings the 32 codes it feeds to the 4 MFMA
// steps of that group. Codes become bf16 (128+q) with one mask+or per pair of
// codes, so the dequantisation costs 7 VALU ops per 8 codes. Per group the
// affine map is applied to the f32 accumulator:
//   sum_k x*(s*q+b) = s * sum_k x*(128+q) + (b - 128*s) * sum_k x
// with sum_k x (the group sums of the activation) computed once per workgroup
// into LDS. Waves split the groups of K; partial tiles are reduced in LDS.
#include "qmm.h"

namespace hb {
namespace {

__device__ inline uint32_t interleave_nibbles(uint32_t w) {
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t c = (w >> (4 * i)) & 0xFu;
    const int pos = (i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1);
    out |= c << pos;
  }
  return out;
}

__global__ void q4_interleave_kernel(const uint32_t* __restrict__ in, uint32_t* __restrict__ out, size_t n) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i < n) out[i] = interleave_nibbles(in[i]);
}

// bf16 (128 + code) for the 8 codes of one interleaved word, in k order.
__device__ inline bf16x8 q4_offset_bf16(uint32_t w) {
  u32x4 d;
  d[0] = (w & 0x000F000Fu) | 0x43004300u;
  d[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  d[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  d[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8, d);
}

__device__ inline float sum_bf16x8(uint4 v) {
  float s = 0.f;
  const uint32_t p[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += __builtin_bit_cast(float, p[i] << 16);
    s += __builtin_bit_cast(float, p[i] & 0xFFFF0000u);
  }
  return s;
}

template <bool OUT_F32>
__device__ inline void store_out(void* y, size_t i, float v) {
  if constexpr (OUT_F32)
    static_cast<float*>(y)[i] = v;
  else
    static_cast<bf16_t*>(y)[i] = f32_to_bf16(v);
}

// MB = number of live 8-row blocks in the 32-row m tile (1..4).
template <int MB, int WAVES, bool OUT_F32>
__global__ __launch_bounds__(64 * WAVES) void qmm4_g64_mfma(const bf16_t* __restrict__ x, int M, int K,
                                                            const uint32_t* __restrict__ w,
                                                            const bf16_t* __restrict__ scales,
                                                            const bf16_t* __restrict__ biases, void* __restrict__ y,
                                                            int N, int ldy) {
  constexpr int kThreads = 64 * WAVES;
  const int G = K >> 6;
  const int words = K >> 3;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nl = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 32;
  const int m0 = blockIdx.y * 32;
  const int n = min(n0 + nl, N - 1);  // clamped row for the N tail; its result is never stored
  extern __shared__ float lds[];
  float* xs = lds;           // [G][32]   group sums of x
  float* red = lds + G * 32; // [WAVES][32 m][32 n] partial tiles

  const uint32_t* wrow = w + size_t(n) * words + h * 4;
  const bf16_t* srow = scales + size_t(n) * G;
  const bf16_t* brow = biases + size_t(n) * G;
  const bool a_live = (m0 + nl) < M;
  const bf16_t* xrow = x + size_t(a_live ? m0 + nl : 0) * K + h * 32;

  int g = wave;
  uint4 wq = g < G ? *reinterpret_cast<const uint4*>(wrow + g * 8) : uint4{0, 0, 0, 0};

  for (int idx = threadIdx.x; idx < G * 32; idx += kThreads) {
    const int gg = idx >> 5, m = idx & 31;
    float s = 0.f;
    if (m < MB * 8 && m0 + m < M) {
      const uint4* p = reinterpret_cast<const uint4*>(x + size_t(m0 + m) * K + gg * 64);
#pragma unroll
      for (int c = 0; c < 8; ++c) s += sum_bf16x8(p[c]);
    }
    xs[idx] = s;
  }
  __syncthreads();

  f32x16 total = {};
  for (; g < G; g += WAVES) {
    const uint4 cur = wq;
    const int gn = g + WAVES;
    if (gn < G) wq = *reinterpret_cast<const uint4*>(wrow + gn * 8);
    const float s = bf16_to_f32(srow[g]);
    const float bp = bf16_to_f32(brow[g]) - 128.f * s;
    const uint32_t cw[4] = {cur.x, cur.y, cur.z, cur.w};
    f32x16 acc = {};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      bf16x8 a = {};
      if (a_live) a = *reinterpret_cast<const bf16x8*>(xrow + g * 64 + st * 8);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, q4_offset_bf16(cw[st]), acc, 0, 0, 0);
    }
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
      const f32x4 xv = *reinterpret_cast<const f32x4*>(xs + g * 32 + rb * 8 + h * 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) total[rb * 4 + j] += s * acc[rb * 4 + j] + bp * xv[j];
    }
  }

  // D layout: lane holds column n = lane%32, rows m = 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
  for (int rb = 0; rb < MB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[(wave * 32 + rb * 8 + h * 4 + j) * 32 + nl] = total[rb * 4 + j];
  __syncthreads();
  for (int idx = threadIdx.x; idx < MB * 8 * 32; idx += kThreads) {
    const int m = idx >> 5, nn = idx & 31;
    if (m0 + m < M && n0 + nn < N) {
      float s = 0.f;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) s += red[(wv * 32 + m) * 32 + nn];
      store_out<OUT_F32>(y, size_t(m0 + m) * ldy + n0 + nn, s);
    }
  }
}

// Any bits in {2,3,4,5,6,8}, group in {32,64,128}, MLX bit-stream layout. One
// 64-lane block per output row n and 8 rows of x; FP32 accumulation.
template <bool OUT_F32>
__global__ __launch_bounds__(64) void qmm_generic(const bf16_t* __restrict__ x, int M, int K,
                                                  const uint32_t* __restrict__ w, const bf16_t* __restrict__ scales,
                                                  const bf16_t* __restrict__ biases, void* __restrict__ y, int N,
                                                  int ldy, int group, int bits) {
  const int n = blockIdx.x, m0 = blockIdx.y * 8, lane = threadIdx.x;
  const int words = K * bits / 32, G = K / group;
  const uint32_t* row = w + size_t(n) * words;
  const uint32_t mask = (1u << bits) - 1u;
  float acc[8] = {};
  for (int c = lane; c < K; c += 64) {
    const size_t bit = size_t(c) * bits;
    const size_t word = bit >> 5;
    const unsigned shift = unsigned(bit & 31);
    uint64_t v = row[word];
    if (shift + bits > 32) v |= uint64_t(row[word + 1]) << 32;
    const float q = float(uint32_t(v >> shift) & mask);
    const int g = c / group;
    const float wv = bf16_to_f32(scales[size_t(n) * G + g]) * q + bf16_to_f32(biases[size_t(n) * G + g]);
#pragma unroll
    for (int r = 0; r < 8; ++r)
      if (m0 + r < M) acc[r] += bf16_to_f32(x[size_t(m0 + r) * K + c]) * wv;
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    float v = acc[r];
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0 && m0 + r < M) store_out<OUT_F32>(y, size_t(m0 + r) * ldy + n, v);
  }
}

template <int MB, bool OUT_F32>
void launch_mfma(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* s, const bf16_t* b, int N,
                 void* y, int ldy, hipStream_t stream) {
  constexpr int kWaves = 4;
  const dim3 grid((N + 31) / 32, (M + 31) / 32);
  const size_t lds = sizeof(float) * (size_t(K / 64) * 32 + kWaves * 32 * 32);
  hipLaunchKernelGGL((qmm4_g64_mfma<MB, kWaves, OUT_F32>), grid, dim3(64 * kWaves), lds, stream, x, M, K, w, s,
                     b, y, N, ldy);
}

template <bool OUT_F32>
void dispatch_mfma(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* s, const bf16_t* b, int N,
                   void* y, int ldy, hipStream_t stream) {
  const int live = M >= 32 ? 4 : (M + 7) / 8;
  switch (live) {
    case 1: launch_mfma<1, OUT_F32>(x, M, K, w, s, b, N, y, ldy, stream); break;
    case 2: launch_mfma<2, OUT_F32>(x, M, K, w, s, b, N, y, ldy, stream); break;
    case 3: launch_mfma<3, OUT_F32>(x, M, K, w, s, b, N, y, ldy, stream); break;
    default: launch_mfma<4, OUT_F32>(x, M, K, w, s, b, N, y, ldy, stream); break;
  }
}

}  // namespace

void q4_interleave(const uint32_t* in, uint32_t* out, size_t n, hipStream_t stream) {
  if (!n) return;
  hipLaunchKernelGGL(q4_interleave_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, in, out, n);
  HB_CHECK(hipGetLastError());
}

void qmm(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* scales, const bf16_t* biases, int N,
         int group, int bits, int layout, void* y, bool y_f32, int ldy, hipStream_t stream) {
  require(x && w && scales && biases && y, "qmm: null operand");
  require(M > 0 && N > 0 && K > 0 && ldy >= N, "qmm: invalid shape");
  require(group == 32 || group == 64 || group == 128, "qmm: group must be 32, 64 or 128");
  require(bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8, "qmm: unsupported bits");
  require(K % group == 0 && (size_t(K) * bits) % 32 == 0, "qmm: K must be a multiple of the group");
  if (layout == kLayoutQ4Interleaved) {
    require(bits == 4 && group == 64, "qmm: interleaved layout is 4-bit group-64 only");
    if (y_f32)
      dispatch_mfma<true>(x, M, K, w, scales, biases, N, y, ldy, stream);
    else
      dispatch_mfma<false>(x, M, K, w, scales, biases, N, y, ldy, stream);
  } else {
    require(layout == kLayoutMlx, "qmm: unknown weight layout");
    const dim3 grid(N, (M + 7) / 8);
    if (y_f32)
      hipLaunchKernelGGL(qmm_generic<true>, grid, dim3(64), 0, stream, x, M, K, w, scales, biases, y, N, ldy, group,
                         bits);
    else
      hipLaunchKernelGGL(qmm_generic<false>, grid, dim3(64), 0, stream, x, M, K, w, scales, biases, y, N, ldy, group,
                         bits);
  }
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
