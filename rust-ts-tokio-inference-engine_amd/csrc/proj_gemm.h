// Dense 4-bit projection over a packed token batch where each weight fragment
// feeds two token tiles: y[M, N] = x[M, K] . W^T, W = s*q + b per group of 64,
// in the tiled layout of q4_tile. Device template: included by qmm.hip.
//
// A workgroup (8 waves) owns 256 weight rows x 32 tokens over all of K; wave w
// owns the two 16-row tiles 2w, 2w + 1 of the group. Per 128-column step a wave
// dequantizes its two tiles' fragments once and runs them against both token
// tiles, so the dequantization and scale work per MFMA is half that of the
// 16-token streaming kernel, and every A fragment read from LDS feeds two
// MFMA chains. x is staged through LDS in 1024-column chunks (two 64 KB
// buffers): chunk c + 1 is loaded during chunk c and stored at its end, one
// barrier per chunk. The arithmetic is the streaming kernel's exact form:
// s * sum x (128 + q) with bf16 128 + q operands, plus (b - 128 s) * sum x as
// one f32 MFMA per step pair over group sums computed while staging.
#pragma once
#include "hb_common.h"
#include "q4_device.h"

namespace hb {
namespace {

constexpr int kProjWaves = 8;
constexpr int kProjRows = 32 * kProjWaves;  // weight rows per workgroup
constexpr int kProjTok = 32;                // token rows per workgroup
constexpr int kProjChunk = 1024;            // x columns staged per LDS buffer
constexpr int kProjPipe = 4;                // weight steps in flight per row tile (divides the chunk's 8)
constexpr int kProjChunkU4 = kProjTok * kProjChunk / 8;           // uint4 per x chunk
constexpr int kProjPer = kProjChunkU4 / (64 * kProjWaves);        // uint4 per thread per chunk
constexpr int kProjGroups = kProjChunk / 64;                      // groups per chunk
constexpr int kProjBuf = kProjChunkU4 + kProjTok * kProjGroups / 4;  // uint4 per buffer: x + group sums
constexpr size_t kProjLds = size_t(2) * kProjBuf * 16;

// OUT 0: y bf16, 1: y f32, 2: y f32 +=. grid.x = ceil(groups / 8) * 8 *
// token pairs, with the token pairs of a row group on one XCD (workgroups are
// dealt to the 8 XCDs round-robin) so the group's weights come from HBM once.
template <int OUT>
__global__ __launch_bounds__(64 * kProjWaves, 1) void proj_gemm_kernel(const bf16_t* __restrict__ x, int M, int K,
                                                                       const uint32_t* __restrict__ wt,
                                                                       const bf16_t* __restrict__ sbt, int n_rows,
                                                                       int pairs, void* __restrict__ yv, int ldy) {
  extern __shared__ uint4 lds[];  // [2][kProjBuf]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, qt = lane >> 4;
  const int b = blockIdx.x;
  const int g = (b / 8 / pairs) * 8 + b % 8, tp = (b / 8) % pairs;
  if (g * kProjRows >= n_rows) return;  // uniform over the workgroup
  const int P = K / 128, chunks = K / kProjChunk, m0 = tp * kProjTok;
  const Q4Consts magic = q4_consts();

  const uint4* wp[2];
  const uint2* sp[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const size_t tile = size_t(g) * (kProjRows / 16) + wave * 2 + rt;
    wp[rt] = reinterpret_cast<const uint4*>(wt) + tile * P * 64 + lane;
    sp[rt] = reinterpret_cast<const uint2*>(sbt) + tile * P * 16 + r16;
  }
  // staging: thread t covers uint4 column t % 128 of rows t / 128 + 4 j (a
  // chunk row is 128 uint4); rows past M repeat row M - 1 (never stored)
  const int xc = tid & 127;
  const bf16_t* xsrc[kProjPer];
  int xdst[kProjPer];
#pragma unroll
  for (int j = 0; j < kProjPer; ++j) {
    const int r = (tid >> 7) + 4 * j;
    xsrc[j] = x + size_t(min(m0 + r, M - 1)) * K + xc * 8;
    xdst[j] = r * 128 + (xc & ~15) + ((xc & 15) ^ (r & 15));
  }
  // a chunk's x into buffer `buf` plus its per-(row, group) sums of x
  auto store_chunk = [&](const uint4 (&v)[kProjPer], int buf) {
    uint4* xs = lds + buf * kProjBuf;
    float* gs = reinterpret_cast<float*>(xs + kProjChunkU4);
#pragma unroll
    for (int j = 0; j < kProjPer; ++j) {
      xs[xdst[j]] = v[j];
      const uint32_t vw[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) sum += bf16_to_f32(bf16_t(vw[q] & 0xFFFFu)) + bf16_to_f32(bf16_t(vw[q] >> 16));
      sum += __shfl_xor(sum, 1, 64);
      sum += __shfl_xor(sum, 2, 64);
      sum += __shfl_xor(sum, 4, 64);
      const int r = (tid >> 7) + 4 * j;
      if ((xc & 7) == 0) gs[r * kProjGroups + (xc >> 3)] = sum;  // the 8 lanes of a group hold the same sum
    }
  };

  uint4 ring_w[2][kProjPipe];
  uint2 ring_s[2][kProjPipe];
#pragma unroll
  for (int q = 0; q < kProjPipe; ++q)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      ring_w[rt][q] = wp[rt][min(q, P - 1) * 64];
      ring_s[rt][q] = sp[rt][min(q, P - 1) * 16];
    }
  {
    uint4 v[kProjPer];
#pragma unroll
    for (int j = 0; j < kProjPer; ++j) v[j] = *reinterpret_cast<const uint4*>(xsrc[j]);
    store_chunk(v, 0);
  }
  __syncthreads();

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 total[2][2], bias[2][2];  // [token tile][row tile]
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) total[t][rt] = bias[t][rt] = zero;
  // A fragment column (uint4 within a 128-column step) of MFMA step j: the
  // tiled words of a lane hold k = 16 qt + 8 (j & 1) .. +7 of group j >> 1
  int acol[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acol[j] = ((j >> 1) * 8 + qt * 2 + (j & 1)) ^ r16;
  float b_even[2] = {0.f, 0.f};

  int buf = 0;
  for (int c = 0; c < chunks; ++c) {
    const bool more = c + 1 < chunks;
    uint4 xv[kProjPer];
    // the next chunk's loads go out first; a clamped re-read on the last
    // chunk keeps every load unconditional (unused)
    const int cn = more ? c + 1 : c;
#pragma unroll
    for (int j = 0; j < kProjPer; ++j) xv[j] = *reinterpret_cast<const uint4*>(xsrc[j] + cn * kProjChunk);
    const uint4* xb = lds + buf * kProjBuf;
    const float* gs = reinterpret_cast<const float*>(xb + kProjChunkU4);
#pragma unroll
    for (int s = 0; s < kProjChunk / 128; ++s) {
      const int p = c * (kProjChunk / 128) + s;
      const int slot = s % kProjPipe;  // = p % kProjPipe: a chunk is 8 steps
      bf16x8 bw[2][4];
      float s0[2], s1[2], b_mine[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const uint4 w = ring_w[rt][slot];
        const uint2 sbp = ring_s[rt][slot];
        bw[rt][0] = q4_offset_bf16_s(w.x, magic);
        bw[rt][1] = q4_offset_bf16_s(w.y, magic);
        bw[rt][2] = q4_offset_bf16_s(w.z, magic);
        bw[rt][3] = q4_offset_bf16_s(w.w, magic);
        s0[rt] = __builtin_bit_cast(float, sbp.x << 16);
        s1[rt] = __builtin_bit_cast(float, sbp.y << 16);
        const uint32_t mine = (qt & 1) ? sbp.y : sbp.x;  // (scale, bias) of this lane's group
        b_mine[rt] = __builtin_fmaf(-128.f, __builtin_bit_cast(float, mine << 16),
                                    __builtin_bit_cast(float, mine & 0xFFFF0000u));
        const int nx = min(p + kProjPipe, P - 1);  // refill; the last step again at the tail (unused)
        ring_w[rt][slot] = wp[rt][nx * 64];
        ring_s[rt][slot] = sp[rt][nx * 16];
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4* xr = xb + (16 * t + r16) * 128 + 16 * s;
        bf16x8 f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) f[j] = __builtin_bit_cast(bf16x8, xr[acol[j]]);
        const float ax = (s & 1) ? gs[(16 * t + r16) * kProjGroups + 2 * s - 2 + qt] : 0.f;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          f32x4 acc0 = mfma16(f[0], bw[rt][0], zero);
          f32x4 acc1 = mfma16(f[2], bw[rt][2], zero);
          acc0 = mfma16(f[1], bw[rt][1], acc0);
          acc1 = mfma16(f[3], bw[rt][3], acc1);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            total[t][rt][r] = __builtin_fmaf(s0[rt], acc0[r], total[t][rt][r]);
            total[t][rt][r] = __builtin_fmaf(s1[rt], acc1[r], total[t][rt][r]);
          }
          // groups 2p - 2 .. 2p + 1: lane quarter qt supplies group qt of the pair
          if (s & 1)
            bias[t][rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ax, qt < 2 ? b_even[rt] : b_mine[rt], bias[t][rt], 0,
                                                               0, 0);
        }
      }
      if (!(s & 1)) {
        b_even[0] = b_mine[0];
        b_even[1] = b_mine[1];
      }
      asm volatile("" : "+v"(total[0][0]), "+v"(total[0][1]), "+v"(total[1][0]), "+v"(total[1][1]));
      __builtin_amdgcn_sched_barrier(0);
    }
    if (more) {
      store_chunk(xv, buf ^ 1);  // the other buffer was last read before the previous barrier
      __syncthreads();
      buf ^= 1;
    }
  }

  // total[t][rt][r]: token m0 + 16 t + 4 qt + r, weight row 16 tile + r16
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int row = (g * (kProjRows / 16) + wave * 2 + rt) * 16 + r16;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * t + 4 * qt + r;
        if (m >= M) continue;
        const float v = total[t][rt][r] + bias[t][rt][r];
        const size_t o = size_t(m) * ldy + row;
        if (OUT == 0)
          static_cast<bf16_t*>(yv)[o] = f32_to_bf16(v);
        else if (OUT == 1)
          static_cast<float*>(yv)[o] = v;
        else
          static_cast<float*>(yv)[o] += v;
      }
  }
}

// Runs the projection when the shape suits it (n_rows % 256, K % 1024, at
// most two waves of workgroups over the CUs and at least half a wave); false
// otherwise, with nothing launched.
template <int OUT>
bool proj_gemm(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* sb, int n_rows, void* y, int ldy,
               int cus, hipStream_t stream) {
  if (n_rows % kProjRows || K % kProjChunk || M <= 16) return false;
  const int groups = n_rows / kProjRows, pairs = (M + kProjTok - 1) / kProjTok;
  const int units = groups * pairs;
  if (units > 2 * cus || 2 * units < cus) return false;
  const auto kernel = &proj_gemm_kernel<OUT>;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(kProjLds));
  HB_CHECK(attr);
  const dim3 grid((groups + 7) / 8 * 8 * pairs);
  hipLaunchKernelGGL(kernel, grid, dim3(64 * kProjWaves), kProjLds, stream, x, M, K, w, sb, n_rows, pairs, y, ldy);
  return true;
}

}  // namespace
}  // namespace hb
