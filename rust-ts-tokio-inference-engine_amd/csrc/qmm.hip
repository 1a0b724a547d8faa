// Affine 4-bit group-64 quantised GEMV/GEMM for gfx950.
//
// MFMA path (tiled layout, v_mfma_f32_16x16x32_bf16):
//   D[m][n] += A[m][k] * B[k][n],  A = x rows (bf16), B = 128 + code (bf16, exact).
// Codes become bf16 (128+q) with one mask+or per pair of codes (the interleaved
// word order puts codes 2j and 2j+1 in the two 16-bit halves of (w >> 4j)), so
// the dequantisation costs 7 VALU ops per 8 codes. Per group the affine map is
// applied to the f32 accumulator:
//   sum_k x*(s*q+b) = s * sum_k x*(128+q) + (b - 128*s) * sum_k x,
// where sum_k x comes from one extra MFMA against a fragment of ones, which
// lands the group sums directly in the accumulator layout.
//
// Tiling: a workgroup owns one 16-row tile of W and all of K; wave w owns PW
// consecutive group pairs. The tiled layout stores each (tile, pair) as 64
// lanes x 16 bytes in MFMA lane order, so every weight load is one contiguous
// 1 KB read and every scale/bias load a contiguous 128-byte read. All loads of
// a wave are issued before its first MFMA; partial tiles are reduced in LDS.
#include "qmm.h"
#include "proj_gemm.h"
#include "proj_stream.h"
#include "stream_gemm.h"
#include "q4_device.h"

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

__global__ void q4_tile_weights(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int K, size_t total) {
  const size_t idx = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (idx >= total) return;
  const int P = K / 128;
  const int j = int(idx & 3), lane = int((idx >> 2) & 63);
  const size_t tp = idx >> 8;  // tile * P + pair
  const int p = int(tp % P);
  const size_t tile = tp / P;
  const int r = lane & 15, qt = lane >> 4;
  const int g = 2 * p + (j >> 1), word = qt * 2 + (j & 1);
  dst[idx] = interleave_nibbles(src[(tile * 16 + r) * size_t(K / 8) + g * 8 + word]);
}

__global__ void q4_tile_sb(const bf16_t* __restrict__ s, const bf16_t* __restrict__ b, bf16_t* __restrict__ dst,
                           int K, size_t total) {
  const size_t idx = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (idx >= total) return;
  const int P = K / 128, G = K / 64;
  const int c = int(idx & 3), r = int((idx >> 2) & 15);
  const size_t tp = idx >> 6;
  const int p = int(tp % P);
  const size_t tile = tp / P;
  const int g = 2 * p + (c >> 1);
  const bf16_t* src = (c & 1) ? b : s;
  dst[idx] = src[(tile * 16 + r) * size_t(G) + g];
}

template <int OUT_F32>
__device__ inline void store_out(void* y, size_t i, float v) {
  // OUT_F32: 0 bf16 store, 1 f32 store, 2 f32 accumulate (y += v; every output
  // element is written by exactly one thread)
  if constexpr (OUT_F32 == 2)
    static_cast<float*>(y)[i] += v;
  else if constexpr (OUT_F32 == 1)
    static_cast<float*>(y)[i] = v;
  else
    static_cast<bf16_t*>(y)[i] = f32_to_bf16(v);
}

// MT = 16-row m tiles per workgroup, PW = group pairs per wave, TN = 16-row
// weight tiles per workgroup. Each wave reuses its x fragments for its TN
// weight tiles (half the x reads per weight byte at TN = 2). Per output the
// arithmetic does not depend on TN, which only changes the workgroup that
// computes a tile.
template <int MT, int PW, int TN, int OUT_F32>
__global__ __launch_bounds__(1024) void qmm4_tiled(const bf16_t* __restrict__ x, int M, int K,
                                                   const uint32_t* __restrict__ wt, const bf16_t* __restrict__ sbt,
                                                   void* __restrict__ y, int N, int ldy) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const int r16 = lane & 15, qt = lane >> 4;
  const int P = K >> 7;
  const int tile0 = blockIdx.x * TN;
  const int mbase = blockIdx.y * 16 * MT;
  const int p0 = wave * PW;

  // Every load is unconditional at a clamped, in-bounds address and masked
  // afterwards: a conditional load becomes a branch plus a full wait.
  uint4 wq[TN][PW];
  uint2 sbv[TN][PW];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const size_t tp = size_t(tile0 + j) * P + min(p0 + i, P - 1);
      wq[j][i] = *reinterpret_cast<const uint4*>(wt + (tp * 64 + lane) * 4);
      sbv[j][i] = *reinterpret_cast<const uint2*>(sbt + (tp * 16 + r16) * 4);
    }
  bf16x8 xa[MT][PW][2][2];  // [m tile][pair][group of pair][step]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const bf16_t* xrow = x + size_t(min(mbase + mt * 16 + r16, M - 1)) * K + qt * 16;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int pc = min(p0 + i, P - 1);
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int s = 0; s < 2; ++s)
          xa[mt][i][gi][s] = *reinterpret_cast<const bf16x8*>(xrow + (2 * pc + gi) * 64 + s * 8);
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const bool mlive = mbase + mt * 16 + r16 < M;
#pragma unroll
    for (int i = 0; i < PW; ++i)
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int s = 0; s < 2; ++s)
          if (!mlive || p0 + i >= P) xa[mt][i][gi][s] = bf16x8{};
  }

  const u32x4 ones_bits = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const bf16x8 ones = __builtin_bit_cast(bf16x8, ones_bits);
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 total[MT][TN];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < TN; ++j) total[mt][j] = zero;
#pragma unroll
  for (int i = 0; i < PW; ++i) {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4 ax = mfma16(xa[mt][i][gi][0], ones, zero);
        ax = mfma16(xa[mt][i][gi][1], ones, ax);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const uint32_t wwords[4] = {wq[j][i].x, wq[j][i].y, wq[j][i].z, wq[j][i].w};
          const uint32_t sbw[2] = {sbv[j][i].x, sbv[j][i].y};
          const bf16x8 b0 = q4_offset_bf16(wwords[2 * gi]);
          const bf16x8 b1 = q4_offset_bf16(wwords[2 * gi + 1]);
          const float s = bf16_to_f32(bf16_t(sbw[gi] & 0xFFFFu));
          const float bp = bf16_to_f32(bf16_t(sbw[gi] >> 16)) - 128.f * s;
          f32x4 acc = mfma16(xa[mt][i][gi][0], b0, zero);
          acc = mfma16(xa[mt][i][gi][1], b1, acc);
#pragma unroll
          for (int r = 0; r < 4; ++r) total[mt][j][r] += s * acc[r] + bp * ax[r];
        }
      }
    }
  }

  // D layout: lane holds column n = lane%16, rows m = 4*(lane/16) + r.
  extern __shared__ float red[];  // [waves][TN][MT*16][16]
  constexpr int TM = MT * 16;
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((wave * TN + j) * TM + mt * 16 + qt * 4 + r) * 16 + r16] = total[mt][j][r];
  __syncthreads();
  for (int idx = threadIdx.x; idx < TN * TM * 16; idx += blockDim.x) {
    const int j = idx / (TM * 16), m = (idx >> 4) % TM, nn = idx & 15;
    if (mbase + m < M) {
      float s = 0.f;
      for (int wv = 0; wv < waves; ++wv) s += red[((wv * TN + j) * TM + m) * 16 + nn];
      store_out<OUT_F32>(y, size_t(mbase + m) * ldy + (tile0 + j) * 16 + nn, s);
    }
  }
}

// Any bits in {2,3,4,5,6,8}, group in {32,64,128}, MLX bit-stream layout. One
// 64-lane block per output row n and 8 rows of x; FP32 accumulation.
template <int OUT_F32>
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

template <int MT, int PW, int TN, int OUT_F32>
void launch_tiled(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* sb, int N, void* y, int ldy,
                  hipStream_t stream) {
  const int P = K / 128;
  const int waves = (P + PW - 1) / PW;
  require(waves <= 16, "qmm: K too large for one workgroup");
  require(N % (16 * TN) == 0, "qmm: N must be a multiple of the workgroup's weight tiles");
  const dim3 grid(N / (16 * TN), (M + 16 * MT - 1) / (16 * MT));
  const size_t lds = sizeof(float) * size_t(waves) * TN * 16 * MT * 16;
  hipLaunchKernelGGL((qmm4_tiled<MT, PW, TN, OUT_F32>), grid, dim3(64 * waves), lds, stream, x, M, K, w, sb, y, N,
                     ldy);
}

// M <= 16 with K <= 2048: two weight tiles per workgroup where N allows
// (x[8,2048] . W[6144,2048]^T over 74 rotated weight copies replayed in a HIP
// graph: 5.44 -> 4.56 us per launch; four tiles leave too few workgroups, 5.8 us).
template <int OUT_F32>
void dispatch_tiled(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* sb, int N, void* y, int ldy,
                    hipStream_t stream) {
  const int P = K / 128;
  if (M <= 16) {
    if (P <= 16) {
      if (N % 32 == 0)
        launch_tiled<1, 1, 2, OUT_F32>(x, M, K, w, sb, N, y, ldy, stream);
      else
        launch_tiled<1, 1, 1, OUT_F32>(x, M, K, w, sb, N, y, ldy, stream);
    } else {
      launch_tiled<1, 2, 1, OUT_F32>(x, M, K, w, sb, N, y, ldy, stream);
    }
  } else {
    if (P <= 16)
      launch_tiled<2, 1, 1, OUT_F32>(x, M, K, w, sb, N, y, ldy, stream);
    else
      launch_tiled<2, 2, 1, OUT_F32>(x, M, K, w, sb, N, y, ldy, stream);
  }
}

}  // namespace

void q4_tile(const uint32_t* w_mlx, const bf16_t* scales, const bf16_t* biases, uint32_t* w_tiled, bf16_t* sb_tiled,
             int N, int K, hipStream_t stream) {
  require(w_mlx && scales && biases && w_tiled && sb_tiled, "q4_tile: null pointer");
  require(N > 0 && N % 16 == 0 && K > 0 && K % 128 == 0, "q4_tile: needs N % 16 == 0 and K % 128 == 0");
  const size_t words = size_t(N) * K / 8, sb = size_t(N) * (K / 64) * 2;
  hipLaunchKernelGGL(q4_tile_weights, dim3(unsigned((words + 255) / 256)), dim3(256), 0, stream, w_mlx, w_tiled, K,
                     words);
  HB_CHECK(hipGetLastError());
  hipLaunchKernelGGL(q4_tile_sb, dim3(unsigned((sb + 255) / 256)), dim3(256), 0, stream, scales, biases, sb_tiled, K,
                     sb);
  HB_CHECK(hipGetLastError());
}

void qmm(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* scales, const bf16_t* biases, int N,
         int group, int bits, int layout, void* y, int out_mode, int ldy, hipStream_t stream, const float* gsum) {
  require(x && w && scales && y, "qmm: null operand");
  require(out_mode >= 0 && out_mode <= 2, "qmm: output mode must be 0 (bf16), 1 (f32) or 2 (f32 accumulate)");
  require(M > 0 && N > 0 && K > 0 && ldy >= N, "qmm: invalid shape");
  require(group == 32 || group == 64 || group == 128, "qmm: group must be 32, 64 or 128");
  require(bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8, "qmm: unsupported bits");
  require(K % group == 0 && (size_t(K) * bits) % 32 == 0, "qmm: K must be a multiple of the group");
  if (layout == kLayoutQ4Tiled) {
    require(bits == 4 && group == 64, "qmm: tiled layout is 4-bit group-64 only");
    require(N % 16 == 0 && K % 128 == 0, "qmm: tiled layout needs N % 16 == 0 and K % 128 == 0");
    // more than one 16-row token tile: the streamed projection (128-row blocks
    // of 32 or 64 tokens, each weight fragment dequantized once for all token
    // tiles of its block) for shapes outside the K-sliced family; otherwise the
    // streaming kernel, which reads the weights once for all tiles (the
    // per-tile kernel re-reads them)
    if (M > 16 && !dense_sliced(N, K)) {
      bool proj = false;
      if (gsum && reinterpret_cast<uintptr_t>(gsum) % 16) gsum = nullptr;  // loaded as uint4
      if (out_mode == 2)
        proj = proj_stream<2>(x, M, K, w, scales, N, y, ldy, stream, gsum);
      else if (out_mode == 1)
        proj = proj_stream<1>(x, M, K, w, scales, N, y, ldy, stream, gsum);
      else
        proj = proj_stream<0>(x, M, K, w, scales, N, y, ldy, stream, gsum);
      if (proj) {
        HB_CHECK(hipGetLastError());
        return;
      }
    }
    if (M > 16) {
      bool done = false;
      if (out_mode == 2)
        done = stream_gemm<false, 2>(x, K, w, scales, N, nullptr, nullptr, nullptr, nullptr, 0, 0, M, 1, y, ldy, stream);
      else if (out_mode == 1)
        done = stream_gemm<false, 1>(x, K, w, scales, N, nullptr, nullptr, nullptr, nullptr, 0, 0, M, 1, y, ldy, stream);
      else
        done = stream_gemm<false, 0>(x, K, w, scales, N, nullptr, nullptr, nullptr, nullptr, 0, 0, M, 1, y, ldy, stream);
      if (done) {
        HB_CHECK(hipGetLastError());
        return;
      }
    }
    if (out_mode == 2)
      dispatch_tiled<2>(x, M, K, w, scales, N, y, ldy, stream);
    else if (out_mode == 1)
      dispatch_tiled<1>(x, M, K, w, scales, N, y, ldy, stream);
    else
      dispatch_tiled<0>(x, M, K, w, scales, N, y, ldy, stream);
  } else {
    require(layout == kLayoutMlx, "qmm: unknown weight layout");
    require(biases != nullptr, "qmm: null biases");
    const dim3 grid(N, (M + 7) / 8);
    if (out_mode == 2)
      hipLaunchKernelGGL(qmm_generic<2>, grid, dim3(64), 0, stream, x, M, K, w, scales, biases, y, N, ldy, group,
                         bits);
    else if (out_mode == 1)
      hipLaunchKernelGGL(qmm_generic<1>, grid, dim3(64), 0, stream, x, M, K, w, scales, biases, y, N, ldy, group,
                         bits);
    else
      hipLaunchKernelGGL(qmm_generic<0>, grid, dim3(64), 0, stream, x, M, K, w, scales, biases, y, N, ldy, group,
                         bits);
  }
  HB_CHECK(hipGetLastError());
}

size_t qmm_select_workspace(int M, int N) { return size_t(M) * size_t(proj_select_parts(N)) * sizeof(uint4); }

bool qmm_select(const bf16_t* x, int M, int K, const uint32_t* w_tiled, const bf16_t* sb_tiled, int N, int vocab,
                void* part, size_t part_bytes, uint32_t* winner, float* margin, int32_t* status, hipStream_t stream) {
  require(x && w_tiled && sb_tiled && part && winner && margin && status, "qmm_select: null operand");
  require(M > 0 && N > 0 && K > 0 && vocab > 0 && vocab <= N, "qmm_select: invalid shape");
  if (N % kProjRows) return false;
  require(part_bytes >= qmm_select_workspace(M, N), "qmm_select: workspace too small");
  return proj_select(x, M, K, w_tiled, sb_tiled, N, vocab, static_cast<uint4*>(part), winner, margin, status,
                     device_cus(), stream);
}

}  // namespace hb
