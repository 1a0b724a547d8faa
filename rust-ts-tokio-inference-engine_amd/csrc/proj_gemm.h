// Dense 4-bit projection over a packed token batch where each weight fragment
// feeds two token tiles: y[M, N] = x[M, K] . W^T, W = s*q + b per group of 64,
// in the tiled layout of q4_tile. Device template: included by qmm.hip.
//
// A workgroup (8 waves) holds the x rows of one 32-token pair for all of K in
// LDS (K <= 2048: two 64 KB buffers of 1024 columns, with the per-group sums
// of x computed while staging) and streams a contiguous range of 256-row weight
// groups past them; wave w owns the two 16-row tiles 2w, 2w + 1 of a group.
// Per 128-column step a wave dequantizes its two tiles' fragments once and
// runs them against both token tiles, so the dequantization and scale work per
// MFMA is half that of the 16-token streaming kernel, and every A fragment
// read from LDS feeds two MFMA chains. The weight register ring runs across
// group boundaries (the next group's first steps load during this group's
// last), and x is staged once: no barrier after the prologue. The arithmetic
// is the streaming kernel's exact form: s * sum x (128 + q) with bf16 128 + q
// operands, plus (b - 128 s) * sum x as one f32 MFMA per step pair.
#pragma once
#include "hb_common.h"
#include "q4_device.h"
#include "select_device.h"

namespace hb {
namespace {

constexpr int kProjWaves = 8;
constexpr int kProjRows = 32 * kProjWaves;  // weight rows per group
constexpr int kProjTok = 32;                // token rows per workgroup
constexpr int kProjChunk = 1024;            // x columns per LDS buffer
constexpr int kProjChunkU4 = kProjTok * kProjChunk / 8;           // uint4 per x chunk
constexpr int kProjPer = kProjChunkU4 / (64 * kProjWaves);        // uint4 per thread per chunk
constexpr int kProjGroups = kProjChunk / 64;                      // groups per chunk
constexpr int kProjBuf = kProjChunkU4 + kProjTok * kProjGroups / 4;  // uint4 per buffer: x + group sums
constexpr size_t kProjLds = size_t(2) * kProjBuf * 16;

// PK = K / 128 in {8, 16}; OUT 0: y bf16, 1: y f32, 2: y f32 +=; 3: greedy
// selection instead of y (K = 2048 only): per token, range and wave a (best,
// index, second best, flags) summary of the wave's rows below `vocab` over the
// range into uint4 yv[token][ldy], entry range * 8 + wave (flags: 1 two or
// more candidates, 2 a non-finite value), merged by argmax_parts_kernel.
// Workgroup b: XCD b % 8, j = b / 8, token pair j % pairs, range
// (j / pairs) * 8 + b % 8 of `ranges` contiguous group ranges, so the token
// pairs of a range run side by side on one XCD and its weights come from HBM
// once.
template <int PK, int OUT, int PROJ_PIPE>
__global__ __launch_bounds__(64 * kProjWaves, 1) void proj_gemm_kernel(const bf16_t* __restrict__ x, int M,
                                                                       const uint32_t* __restrict__ wt,
                                                                       const bf16_t* __restrict__ sbt, int n_rows,
                                                                       int pairs, int ranges, void* __restrict__ yv,
                                                                       int ldy, int vocab) {
  constexpr int K = PK * 128, kChunks = K / kProjChunk, kCS = kProjChunk / 128;
  constexpr int kProjPipe = PROJ_PIPE;  // weight steps in flight per row tile
  static_assert(kChunks >= 1 && kChunks <= 2 && kCS % kProjPipe == 0, "projection geometry");
  extern __shared__ uint4 lds[];  // [2][kProjBuf]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, qt = lane >> 4;
  const int b = blockIdx.x, j8 = b / 8;
  const int tp = j8 % pairs, rr = (j8 / pairs) * 8 + b % 8;
  if (rr >= ranges) return;  // uniform over the workgroup
  const int groups = n_rows / kProjRows;
  const int g0 = int(int64_t(rr) * groups / ranges), g1 = int(int64_t(rr + 1) * groups / ranges);
  if (g0 >= g1) return;
  const int m0 = tp * kProjTok;
  const Q4Consts magic = q4_consts();

  // weights of group g, wave, row tile rt: tile 16 g + 2 wave + rt
  constexpr size_t kGroupW = size_t(kProjRows / 16) * PK * 64, kGroupS = size_t(kProjRows / 16) * PK * 16;
  const uint4* wp[2];
  const uint2* sp[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const size_t tile = size_t(g0) * (kProjRows / 16) + wave * 2 + rt;
    wp[rt] = reinterpret_cast<const uint4*>(wt) + tile * PK * 64 + lane;
    sp[rt] = reinterpret_cast<const uint2*>(sbt) + tile * PK * 16 + r16;
  }
  uint4 ring_w[2][kProjPipe];
  uint2 ring_s[2][kProjPipe];
#pragma unroll
  for (int q = 0; q < kProjPipe; ++q)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      ring_w[rt][q] = wp[rt][q * 64];
      ring_s[rt][q] = sp[rt][q * 16];
    }

  // x of the token pair, all of K: thread t covers uint4 column t % 128 of
  // rows t / 128 + 4 j of each 1024-column chunk; rows past M repeat row M - 1
  // (never stored). Group sums: the 8 lanes of a 64-column group reduce theirs.
  {
    const int xc = tid & 127;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      uint4 v[kProjPer];
#pragma unroll
      for (int j = 0; j < kProjPer; ++j) {
        const int r = (tid >> 7) + 4 * j;
        v[j] = *reinterpret_cast<const uint4*>(x + size_t(min(m0 + r, M - 1)) * K + c * kProjChunk + xc * 8);
      }
      uint4* xs = lds + c * kProjBuf;
      float* gs = reinterpret_cast<float*>(xs + kProjChunkU4);
#pragma unroll
      for (int j = 0; j < kProjPer; ++j) {
        const int r = (tid >> 7) + 4 * j;
        xs[r * 128 + (xc & ~15) + ((xc & 15) ^ (r & 15))] = v[j];
        const uint32_t vw[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) sum += bf16_to_f32(bf16_t(vw[q] & 0xFFFFu)) + bf16_to_f32(bf16_t(vw[q] >> 16));
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        sum += __shfl_xor(sum, 4, 64);
        if ((xc & 7) == 0) gs[r * kProjGroups + (xc >> 3)] = sum;
      }
    }
  }
  __syncthreads();

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  // A fragment column (uint4 within a 128-column step) of MFMA step j: the
  // tiled words of a lane hold k = 16 qt + 8 (j & 1) .. +7 of group j >> 1
  int acol[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acol[j] = ((j >> 1) * 8 + qt * 2 + (j & 1)) ^ r16;

  // OUT 3: running (best, second) per token of the lane over its rows so far
  Top2 sel[2][4];
  uint32_t sel_bad = 0;  // bit 4 t + r: a non-finite value for that token
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sel[t][r] = Top2{0u, 0xFFFFFFFFu, 0u, false};
  for (int g = g0; g < g1; ++g) {
    // the next group's pointers (this group again after the last: unused
    // cache hits, so every load stays unconditional)
    const size_t adv = g + 1 < g1 ? 1 : 0;
    const uint4* wn[2] = {wp[0] + adv * kGroupW, wp[1] + adv * kGroupW};
    const uint2* sn[2] = {sp[0] + adv * kGroupS, sp[1] + adv * kGroupS};
    f32x4 total[2][2], bias[2][2];  // [token tile][row tile]
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) total[t][rt] = bias[t][rt] = zero;
    float b_even[2] = {0.f, 0.f};
    // chunk loop kept rolled: a fully unrolled 16-step group spills
#pragma unroll 1
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
    for (int s = 0; s < kCS; ++s) {
      const int p = c * kCS + s;
      const int slot = s % kProjPipe;  // = p % kProjPipe: the ring depth divides a chunk's steps
      const uint4* xb = lds + c * kProjBuf;
      const float* gs = reinterpret_cast<const float*>(xb + kProjChunkU4);
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
        // refill the slot: this group's step p + ring, else the next group's head
        const int nx = p + kProjPipe;
        const bool here = nx < PK;
        const uint4* ws = here ? wp[rt] + nx * 64 : wn[rt] + (nx - PK) * 64;  // one load from either
        const uint2* ss = here ? sp[rt] + nx * 16 : sn[rt] + (nx - PK) * 16;
        ring_w[rt][slot] = *ws;
        ring_s[rt][slot] = *ss;
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

    // total[t][rt][r]: token m0 + 16 t + 4 qt + r, weight row 16 tile + r16
    if constexpr (OUT == 3) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const int row = (g * (kProjRows / 16) + wave * 2 + rt) * 16 + r16;
            const float v = total[t][rt][r] + bias[t][rt][r];
            if (row < vocab) {
              sel_bad |= isfinite(v) ? 0u : 1u << (4 * t + r);
              sel[t][r] = merge(sel[t][r], Top2{total_key(v), uint32_t(row), 0u, false});
            }
          }
    } else {
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
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      wp[rt] = wn[rt];
      sp[rt] = sn[rt];
    }
  }
  if constexpr (OUT == 3) {
    // per token: the 16 lanes of its quarter (lane bits 0..3 index the rows),
    // then one store per (token, range, wave) from lane r16 == 0
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) sel_bad |= uint32_t(__shfl_xor(int(sel_bad), off));
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        Top2 best = sel[t][r];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          const Top2 o{uint32_t(__shfl_xor(int(best.k1), off)), uint32_t(__shfl_xor(int(best.i1), off)),
                       uint32_t(__shfl_xor(int(best.k2), off)), __shfl_xor(int(best.has2), off) != 0};
          best = merge(best, o);
        }
        const int m = m0 + 16 * t + 4 * qt + r;
        if (r16 == 0 && m < M)
          static_cast<uint4*>(yv)[size_t(m) * ldy + rr * kProjWaves + wave] =
              make_uint4(best.k1, best.i1, best.k2, (best.has2 ? 1u : 0u) | ((sel_bad >> (4 * t + r)) & 1u) * 2u);
      }
  }
}

// Runs the projection when the shape suits it (n_rows % 256, K in {1024,
// 2048}, 16 < M <= 256, and at least half a wave of (group, token pair)
// units); false otherwise, with nothing launched. One workgroup per CU: the
// token pairs split the CUs, each pair's share of CUs splits the groups.
template <int OUT>
bool proj_gemm(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* sb, int n_rows, void* y, int ldy,
               int cus, hipStream_t stream, int vocab = 0, int* ranges_out = nullptr) {
  if (n_rows % kProjRows || (K != 1024 && K != 2048) || M <= 16 || M > 256) return false;
  if (OUT == 3 && K != 2048) return false;
  const int groups = n_rows / kProjRows, pairs = (M + kProjTok - 1) / kProjTok;
  if (2 * groups * pairs < cus) return false;
  const int ranges = std::max(1, std::min(groups, cus / pairs));
  if (ranges_out) *ranges_out = ranges;
  const dim3 grid((ranges + 7) / 8 * 8 * pairs);
#define HB_PROJ(PKC, PIPEC)                                                                                             \
  {                                                                                                              \
    const auto kernel = &proj_gemm_kernel<PKC, OUT, PIPEC>;                                                             \
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),                    \
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(kProjLds)); \
    HB_CHECK(attr);                                                                                              \
    hipLaunchKernelGGL(kernel, grid, dim3(64 * kProjWaves), kProjLds, stream, x, M, w, sb, n_rows, pairs, ranges, \
                       y, ldy, vocab);                                                                           \
  }
  if constexpr (OUT == 3) {
    HB_PROJ(16, 4)
  } else {
    if (K == 1024)
      HB_PROJ(8, 8)
    else
      HB_PROJ(16, 4)
  }
#undef HB_PROJ
  return true;
}

constexpr int kPartThreads = 256;

// Final merge of per-row partial summaries part[row][ld] (nparts used), one
// workgroup per row: winner index, margin top1 - top2 (inf with a single
// candidate) and the non-finite status, as the two-level argmax leaves them.
__global__ __launch_bounds__(kPartThreads) void argmax_parts_kernel(const uint4* __restrict__ part, int nparts,
                                                                    int ld, uint32_t* __restrict__ winner,
                                                                    float* __restrict__ margin,
                                                                    int32_t* __restrict__ status) {
  const int r = blockIdx.x, tid = threadIdx.x;
  Top2 t{0u, 0xFFFFFFFFu, 0u, false};
  uint32_t bad = 0;
  for (int c = tid; c < nparts; c += kPartThreads) {
    const uint4 p = part[size_t(r) * ld + c];
    t = merge(t, Top2{p.x, p.y, p.z, (p.w & 1u) != 0});
    bad |= p.w & 2u;
  }
  __shared__ Top2 sp[kPartThreads];
  __shared__ uint32_t sb[kPartThreads];
  sp[tid] = t;
  sb[tid] = bad;
  __syncthreads();
  for (int s = kPartThreads / 2; s > 0; s >>= 1) {
    if (tid < s) {
      sp[tid] = merge(sp[tid], sp[tid + s]);
      sb[tid] |= sb[tid + s];
    }
    __syncthreads();
  }
  if (tid == 0) {
    winner[r] = sp[0].i1;
    margin[r] = sp[0].has2 ? key_value(sp[0].k1) - key_value(sp[0].k2) : INFINITY;
    status[r] = sb[0] ? 1 : 0;
  }
}

// Entries per token of the fused selection's partial summaries (an upper
// bound: one per range and wave, at most one range per group).
inline int proj_select_parts(int n_rows) { return n_rows / kProjRows * kProjWaves; }

// Greedy selection over y = x . W^T without writing y (rows >= vocab are
// padding): winner, margin and status per token, as argmax_margin gives them
// over the same values. `part` holds M * proj_select_parts(n_rows) uint4.
// False when the projection does not cover the shape (nothing launched).
inline bool proj_select(const bf16_t* x, int M, int K, const uint32_t* w, const bf16_t* sb, int n_rows, int vocab,
                        uint4* part, uint32_t* winner, float* margin, int32_t* status, int cus, hipStream_t stream) {
  if (vocab < 1 || vocab > n_rows) return false;
  const int ld = proj_select_parts(n_rows);
  int ranges = 0;
  if (!proj_gemm<3>(x, M, K, w, sb, n_rows, part, ld, cus, stream, vocab, &ranges)) return false;
  HB_CHECK(hipGetLastError());
  hipLaunchKernelGGL(argmax_parts_kernel, dim3(M), dim3(kPartThreads), 0, stream, part, ranges * kProjWaves, ld,
                     winner, margin, status);
  HB_CHECK(hipGetLastError());
  return true;
}

}  // namespace
}  // namespace hb
