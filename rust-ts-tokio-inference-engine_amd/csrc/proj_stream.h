// Dense 4-bit projection with x streamed through LDS: y[M, N] = x[M, K] . W^T,
// W = s*q + b per group of 64, tiled layout of q4_tile. Device template:
// included by qmm.hip.
//
// Workgroup: 8 waves, 16 TT tokens (TT token tiles) x 128 weight rows; wave w
// owns the 16-row tile w of the block over the whole K and runs every weight
// fragment it dequantizes against all TT token tiles. The costs that bound a
// decode-sized projection on gfx950 are issue slots: matrix and vector
// instructions of one SIMD barely overlap, and the vector work (the 128 + q
// operands and the per-group scaling) is most of the step. Dequantizing once
// for four token tiles instead of two cuts that share per output by a quarter.
//
// x does not fit in LDS for 64 tokens x all of K, so it streams in 256-column
// chunks through a four-buffer ring: a chunk's loads go out two chunks before
// it is read and are written to LDS (with the per-group sums of x, computed
// while writing) at the end of the chunk in between, so the first MFMA waits
// for two chunks only and no barrier waits on a load issued less than a chunk
// earlier. Weights run through a four-step register ring per wave.
//
// Per output the arithmetic is that of the two-token-tile projection and of
// the streaming kernel: s * sum x (128 + q) with bf16 128 + q operands, step
// by step, plus (b - 128 s) * sum x as one f32 MFMA per step pair, the group
// sums of x added in the same order. Results are bit-identical to theirs, so
// a row's output does not depend on which of them its batch size selects.
#pragma once
#include "hb_common.h"
#include "q4_device.h"

namespace hb {
namespace {

constexpr int kPsWaves = 8;
constexpr int kPsRows = 16 * kPsWaves;  // weight rows per workgroup
constexpr int kPsChunk = 256;           // x columns per chunk (two steps)
constexpr int kPsRowU4 = kPsChunk / 8;  // uint4 per token row per chunk
constexpr int kPsBufs = 4;              // chunks in the LDS ring
constexpr int kPsRing = 4;              // weight steps in flight per wave

template <int TT>
struct PsGeom {
  static constexpr int kTok = 16 * TT;                                // token rows per workgroup
  static constexpr int kChunkU4 = kTok * kPsRowU4;                   // x uint4 per chunk
  static constexpr int kPer = kChunkU4 / (64 * kPsWaves);            // x uint4 per thread per chunk
  static constexpr int kBufU4 = kChunkU4 + kTok * 4 / 4;             // x, then [kTok][4 groups] f32 sums
  static constexpr size_t kLds = size_t(kPsBufs) * kBufU4 * 16;
};

// PK = K / 128 in {8, 16}; OUT 0: y bf16, 1: y f32, 2: y f32 +=. GS: the
// group sums of x come from gsg (f32 [M][K / 64], written by the kernel that
// produced x, in the order bf16x8_pair_sum + sum8_lanes fix) instead of being
// computed while staging: the same values, a fifth less vector work per
// chunk. Two token
// tiles fit in 128 registers (four waves per SIMD, two workgroups per CU), four
// in 256. Workgroup b:
// XCD b % 8, j = b / 8, token block j % tblocks, row block (j / tblocks) * 8 +
// b % 8, so the token blocks of a row block run side by side on one XCD and its
// weights come from HBM once.
template <int PK, int OUT, int TT, bool GS>
__global__ __launch_bounds__(64 * kPsWaves, TT == 2 ? 4 : 2) void proj_stream_kernel(const bf16_t* __restrict__ x, int M,
                                                                       const float* __restrict__ gsg,
                                                                       const uint32_t* __restrict__ wt,
                                                                       const bf16_t* __restrict__ sbt, int n_rows,
                                                                       int tblocks, void* __restrict__ yv, int ldy) {
  using G = PsGeom<TT>;
  constexpr int K = PK * 128, kChunks = PK / 2;
  static_assert(PK % (2 * kPsBufs) == 0 && (2 * kPsBufs) % kPsRing == 0, "the unrolled body covers the ring and the buffers");
  extern __shared__ uint4 lds[];  // [kPsBufs][kBufU4]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, qt = lane >> 4;
  const int b = blockIdx.x, j8 = b / 8;
  const int tb = j8 % tblocks, rb = (j8 / tblocks) * 8 + b % 8;
  if (rb >= n_rows / kPsRows) return;  // uniform over the workgroup
  const int m0 = tb * G::kTok;
  const Q4Consts magic = q4_consts();

  // x chunk c of the token block: thread t covers uint4 (token, column) =
  // (i / 32, i % 32) for i = t + 512 k; tokens past M repeat token M - 1 (never
  // stored). Stored XOR-swizzled by token within each 16-uint4 half row. Loads
  // take a uniform base and 32-bit lane offsets (M K / 8 < 2^31).
  const int t0 = tid / kPsRowU4, cc0 = tid % kPsRowU4;
  constexpr int kRowStep = 64 * kPsWaves / kPsRowU4;  // token rows between a thread's uint4
  int xoff[G::kPer];
#pragma unroll
  for (int k = 0; k < G::kPer; ++k) xoff[k] = min(m0 + t0 + k * kRowStep, M - 1) * (K / 8) + cc0;
  const uint4* const x4 = reinterpret_cast<const uint4*>(x);
  // GS: every thread loads the 4 group sums of token tid % kTok for the chunk
  // (one uint4 of gsg) with the chunk's x, unconditionally, so the load is
  // issued with the others instead of being sunk to its use
  const int gsrow = min(m0 + tid % G::kTok, M - 1) * (K / 256);
  auto load_chunk = [&](int c, uint4 (&v)[G::kPer], uint4& g4) {
    const uint4* xc = x4 + c * kPsRowU4;
#pragma unroll
    for (int k = 0; k < G::kPer; ++k) v[k] = xc[xoff[k]];
    if constexpr (GS) g4 = reinterpret_cast<const uint4*>(gsg)[gsrow + c];
  };
  // writes chunk values into buffer `buf` with the per-group sums: each thread
  // sums its eight values, then the eight lanes of a 64-column group combine
  // (GS: the loaded sums instead). Values are copied by component, which keeps
  // the register arrays out of scratch memory.
  auto store_chunk = [&](int buf, const uint4 (&v)[G::kPer], const uint4& g4) {
    uint4* xs = lds + buf * G::kBufU4;
    float* gs = reinterpret_cast<float*>(xs + G::kChunkU4);
#pragma unroll
    for (int k = 0; k < G::kPer; ++k) {
      const int i = tid + k * 64 * kPsWaves;
      const int t = i / kPsRowU4, cc = i % kPsRowU4;
      xs[t * kPsRowU4 + (cc & 16) + ((cc & 15) ^ (t & 15))] = make_uint4(v[k].x, v[k].y, v[k].z, v[k].w);
      if constexpr (!GS) {
        const float sum = sum8_lanes(bf16x8_pair_sum(v[k]));
        if ((cc & 7) == 0) gs[t * 4 + (cc >> 3)] = sum;
      }
    }
    if constexpr (GS) reinterpret_cast<uint4*>(gs)[tid % G::kTok] = make_uint4(g4.x, g4.y, g4.z, g4.w);
  };

  // weights of this wave's row tile: wave-uniform base, lane offset
  const int tile = rb * kPsWaves + __builtin_amdgcn_readfirstlane(wave);
  const uint4* const wp = reinterpret_cast<const uint4*>(wt) + size_t(tile) * PK * 64;
  const uint2* const sp = reinterpret_cast<const uint2*>(sbt) + size_t(tile) * PK * 16;

  // prologue: x chunks 0 and 1 into LDS; the weight ring's first kPsRing steps
  uint4 vx[G::kPer];
  uint4 gv = make_uint4(0, 0, 0, 0);
  {
    uint4 v1[G::kPer];
    uint4 g1 = make_uint4(0, 0, 0, 0);
    load_chunk(0, vx, gv);
    load_chunk(1, v1, g1);
    store_chunk(0, vx, gv);
    store_chunk(1, v1, g1);
  }
  uint4 ring_w[kPsRing];
  uint2 ring_s[kPsRing];
#pragma unroll
  for (int q = 0; q < kPsRing; ++q) {
    ring_w[q] = wp[q * 64 + lane];
    ring_s[q] = sp[q * 16 + r16];
  }
  __syncthreads();

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  // A fragment column (uint4 within a step's 16) of MFMA step j: the tiled
  // words of a lane hold k = 16 qt + 8 (j & 1) .. +7 of group j >> 1
  int acol[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acol[j] = ((j >> 1) * 8 + qt * 2 + (j & 1)) ^ r16;

  f32x4 total[TT], bias[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) total[t] = bias[t] = zero;
  float b_even = 0.f;

  // body: four chunks (eight steps), so ring slots, LDS buffers and x register
  // sets are compile-time indices; chunk c = c0 + i lives in buffer i
#pragma unroll 1
  for (int c0 = 0; c0 < kChunks; c0 += kPsBufs) {
    // this body's refills: steps 2 c0 + kPsRing onwards, clamped to the last
    // steps (re-read, unused) past the end
    const uint4* const wn = wp + 2 * c0 * 64;
    const uint2* const sn = sp + 2 * c0 * 16;
#pragma unroll
    for (int i = 0; i < kPsBufs; ++i) {
      const int c = c0 + i;
      // chunk c + 2 (or the last chunk again: unused), written at the end of
      // this chunk
      load_chunk(min(c + 2, kChunks - 1), vx, gv);
      const uint4* xb = lds + i * G::kBufU4;
      const float* gs = reinterpret_cast<const float*>(xb + G::kChunkU4);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int p = (2 * i + s) % kPsRing;  // ring slot
        const uint4 w = ring_w[p];
        const uint2 sbp = ring_s[p];
        bf16x8 bw[4];
        bw[0] = q4_offset_bf16_s(w.x, magic);
        bw[1] = q4_offset_bf16_s(w.y, magic);
        bw[2] = q4_offset_bf16_s(w.z, magic);
        bw[3] = q4_offset_bf16_s(w.w, magic);
        const float s0 = __builtin_bit_cast(float, sbp.x << 16), s1 = __builtin_bit_cast(float, sbp.y << 16);
        const uint32_t mine = (qt & 1) ? sbp.y : sbp.x;  // (scale, bias) of this lane's group
        const float b_mine = __builtin_fmaf(-128.f, __builtin_bit_cast(float, mine << 16),
                                            __builtin_bit_cast(float, mine & 0xFFFF0000u));
        // refill: step 2c + s + kPsRing, or this step again past the end
        const int nx = 2 * c + s + kPsRing < PK ? 2 * i + s + kPsRing : 2 * i + s;
        ring_w[p] = wn[nx * 64 + lane];
        ring_s[p] = sn[nx * 16 + r16];
        // A fragments one token tile ahead of the MFMAs that use them (the
        // scheduling barrier per tile keeps the compiler from hoisting all of
        // them, which would not fit in the registers)
        auto frags = [&](int t, bf16x8 (&f)[4]) {
          const uint4* xr = xb + (16 * t + r16) * kPsRowU4 + 16 * s;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) f[jj] = __builtin_bit_cast(bf16x8, xr[acol[jj]]);
        };
        bf16x8 fa[4], fb[4];
        frags(0, fa);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          bf16x8(&f)[4] = (t & 1) ? fb : fa;
          if (t + 1 < TT) frags(t + 1, (t & 1) ? fa : fb);
          f32x4 acc0 = mfma16(f[0], bw[0], zero);
          f32x4 acc1 = mfma16(f[2], bw[2], zero);
          acc0 = mfma16(f[1], bw[1], acc0);
          acc1 = mfma16(f[3], bw[3], acc1);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            total[t][r] = __builtin_fmaf(s0, acc0[r], total[t][r]);
            total[t][r] = __builtin_fmaf(s1, acc1[r], total[t][r]);
          }
          // groups 4c .. 4c + 3 of this chunk: lane quarter qt supplies group qt
          if (s == 1)
            bias[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(gs[(16 * t + r16) * 4 + qt], qt < 2 ? b_even : b_mine,
                                                           bias[t], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (s == 0) b_even = b_mine;
        // materialise the running sums here: otherwise the adds sink past the
        // loop and every step's MFMA results stay live in accumulators
#pragma unroll
        for (int t = 0; t < TT; ++t) asm volatile("" : "+v"(total[t]));
        __builtin_amdgcn_sched_barrier(0);
      }
      // chunk c + 2 into the buffer chunk c - 2 used
      store_chunk((i + 2) % kPsBufs, vx, gv);
      __syncthreads();
    }
  }

  // total[t][r] + bias[t][r]: token m0 + 16 t + 4 qt + r, weight row 16 tile + r16
  const int row = tile * 16 + r16;
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 16 * t + 4 * qt + r;
      if (m >= M) continue;
      const float v = total[t][r] + bias[t][r];
      const size_t o = size_t(m) * ldy + row;
      if (OUT == 0)
        static_cast<bf16_t*>(yv)[o] = f32_to_bf16(v);
      else if (OUT == 1)
        static_cast<float*>(yv)[o] = v;
      else
        static_cast<float*>(yv)[o] += v;
    }
}

// Runs the streamed projection with TT token tiles per workgroup when the
// shape suits it (n_rows % 128, K in {1024, 2048}, M > 16); false otherwise,
// with nothing launched.
template <int OUT, int TT>
bool proj_stream_tt(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* sb, int n_rows, void* y, int ldy,
                    hipStream_t stream, const float* gsum) {
  if (n_rows % kPsRows || (K != 1024 && K != 2048) || M <= 16) return false;
  using G = PsGeom<TT>;
  const int rblocks = n_rows / kPsRows, tblocks = (M + G::kTok - 1) / G::kTok;
  const dim3 grid((rblocks + 7) / 8 * 8 * tblocks);
#define HB_PS(PKC, GSC)                                                                                           \
  {                                                                                                               \
    const auto kernel = &proj_stream_kernel<PKC, OUT, TT, GSC>;                                                   \
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),                     \
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(G::kLds)); \
    HB_CHECK(attr);                                                                                               \
    hipLaunchKernelGGL(kernel, grid, dim3(64 * kPsWaves), G::kLds, stream, x, M, gsum, w, sb, n_rows, tblocks, y, \
                       ldy);                                                                                      \
  }
  if (K == 1024) {
    if (gsum)
      HB_PS(8, true)
    else
      HB_PS(8, false)
  } else {
    if (gsum)
      HB_PS(16, true)
    else
      HB_PS(16, false)
  }
#undef HB_PS
  return true;
}

// The streamed projection for 16 < M <= 256: four token tiles per workgroup
// for 64 < M <= 128 (one workgroup per CU), two otherwise (two workgroups per
// CU at four waves per SIMD, which overlap better where there are many
// workgroups). Both give the same bits, with or without the group sums gsum
// (f32 [M][K / 64] of x, 16-byte aligned; null: computed here). The two-tile
// form computes them itself: at 128 registers the loaded sums cost it spills.
template <int OUT>
bool proj_stream(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* sb, int n_rows, void* y, int ldy,
                 hipStream_t stream, const float* gsum = nullptr) {
  if (M > 256) return false;
  return M > 64 && M <= 128 ? proj_stream_tt<OUT, 4>(x, M, K, w, sb, n_rows, y, ldy, stream, gsum)
                            : proj_stream_tt<OUT, 2>(x, M, K, w, sb, n_rows, y, ldy, stream, nullptr);
}

}  // namespace
}  // namespace hb
