// Persistent streaming 4-bit GEMM shared by the grouped MoE GEMM (work list
// of expert tiles) and the dense projections (a single matrix over token
// tiles). Device template: included by the .hip files that launch it.
#pragma once
#include <algorithm>
#include "hb_common.h"
#include "q4_device.h"

namespace hb {
namespace {

// Weight tiles read once per launch (the grouped expert GEMMs) are loaded as
// streaming (non-temporal), codes and scale/bias pairs alike, so they do not
// displace the activations and the work list in the caches: the grouped
// gate/up launch at 128 tokens drops from 120 to 100 us (5.5 TB/s). Dense
// projections re-read a weight group from L2 for every token tile and keep
// the default policy.
template <bool NT>
__device__ inline uint4 load_weights(const uint4* p) {
  if constexpr (NT) {
    using v4u = unsigned __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    uint4 r;
    r.x = v.x;
    r.y = v.y;
    r.z = v.z;
    r.w = v.w;
    return r;
  } else {
    return *p;
  }
}
template <bool NT>
__device__ inline uint2 load_sb(const uint2* p) {
  if constexpr (NT) {
    using v2u = unsigned __attribute__((ext_vector_type(2)));
    const v2u v = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p));
    uint2 r;
    r.x = v.x;
    r.y = v.y;
    return r;
  } else {
    return *p;
  }
}

// Persistent streaming grouped GEMM. The work list (moe_sort_kernel) holds
// one item per 16-row tile of a token list: the shared expert's token tiles,
// then every routed expert's pair tiles. A unit is (item, group of 16*WAVES
// weight rows); each persistent workgroup walks units u, u + grid, ... and
// a wave owns 16 weight rows of the unit over the whole K.
//  - Weights stream through an NPIPE-deep register ring that runs across
//    units: while a wave finishes unit u it already loads unit u+grid's first
//    pairs, so its loads stay in flight through epilogues and barriers.
//  - The next unit's token rows are staged during the current unit, one
//    chunk per thread at a time, into the other half of a double-buffered LDS
//    tile (bf16 [16][K], XOR-swizzled by row, plus per-group sums): one
//    barrier per unit, no exposed staging latency.
//  - Every load is unconditional (the last unit re-reads itself), so the
//    compiler's in-order vector-memory wait counts stay exact and no step
//    waits for more than the load it consumes.
// Rows past a tile's count only feed their own output rows, which are never
// stored.
//
// SINGLE: every workgroup runs at most one unit (the host launches at least
// as many workgroups as there are units), so x is staged once into a single
// LDS buffer and nothing is prefetched for a next unit; this fits a whole K of
// 4096 (the attention and DeltaNet output projections) into one launch at any
// token count, so a row's result does not depend on the batch it is packed in.
// KS > 1 (SINGLE only): KS waves share each 16-row tile, wave slice ks taking
// steps [ks PK / KS, (ks + 1) PK / KS); the slices' partial sums meet in LDS
// and are added in slice order. A single unit per workgroup is a dependent
// chain of K / 128 steps, so one wave per SIMD walking all of K leaves the
// matrix and vector pipes idle most of the time; KS waves per SIMD cut the
// chain by KS and overlap each other's latencies.
template <int PK, int WAVES, int NPIPE, bool SWIGLU, int OUT, bool NT, bool SINGLE = false, int KS = 1>
__global__ __launch_bounds__(64 * WAVES * KS) void stream_gemm_kernel(const bf16_t* __restrict__ x,
                                                                 const uint32_t* __restrict__ wt,
                                                                 const bf16_t* __restrict__ sbt, int n_rows,
                                                                 const int32_t* __restrict__ counts,
                                                                 const int32_t* __restrict__ offsets,
                                                                 const int32_t* __restrict__ order,
                                                                 const int32_t* __restrict__ items, int E, int top,
                                                                 int T, int dense, void* __restrict__ yv, int ldy,
                                                                 int ldx, int pk_stride) {
  static_assert(KS == 1 || (SINGLE && !SWIGLU), "K slices need one unit per workgroup");
  static_assert(PK % KS == 0 && (KS == 1 || (PK / KS) % 2 == 0), "K slices of whole step pairs");
  constexpr int K = PK * 128;
  constexpr int PKS = PK / KS;  // steps per wave
  constexpr int kRowU4 = K / 8;
  constexpr int kThreads = 64 * WAVES * KS;
  constexpr int kIter = (16 * kRowU4 + kThreads - 1) / kThreads;  // x chunks per thread and unit
  // x staging schedule (see load_x): chunk `it` is loaded at step
  // it * kLdSpan / kIter and stored kLag steps later. With few chunks (16
  // waves) one chunk is live at a time and waits kStride - 1 steps; with one
  // chunk per step (4 waves) all loads go out in the first quarter of the unit
  // and are stored at its end, so each store only waits for weight loads the
  // next unit needs anyway.
  constexpr bool kSparse = kIter * 4 <= PK;
  constexpr int kLdSpan = kSparse ? PK : (PK >= 8 ? PK / 4 : 1);
  constexpr int kLag = kSparse ? PK / kIter - 1 : PK - kLdSpan;
  static_assert((kIter - 1) * kLdSpan / kIter + kLag < PK, "x staging ends inside the unit");
  constexpr int kPipe = NPIPE < PKS ? NPIPE : PKS;
  constexpr int kBuf = 16 * kRowU4 + PK * 2 * 16 / 4;  // uint4 units per LDS buffer: x tile + group sums
  extern __shared__ uint4 lds[];                        // [SINGLE ? 1 : 2][kBuf]
  const int lane = threadIdx.x & 63, wave = (threadIdx.x >> 6) % WAVES, ks = (threadIdx.x >> 6) / WAVES;
  const int r16 = lane & 15, qt = lane >> 4;
  const int P = T * top;
  const int ngroups = n_rows / (16 * WAVES);
  // dense: unit u -> (row group, token tile) with every tile of a group on the
  // same XCD (workgroups are dealt to the 8 XCDs round-robin), so the group's
  // weights come from HBM once and from that XCD's L2 for the other tiles
  const int n_tiles = (T + 15) / 16, ng8 = (ngroups + 7) / 8 * 8;
  const int n_units = dense ? ng8 * n_tiles : items[0] * ngroups;
  auto dense_group = [&](int unit) { return (unit / 8 / n_tiles) * 8 + unit % 8; };
  auto next_unit = [&](int unit) {
    if (dense)
      while (unit < n_units && dense_group(unit) >= ngroups) unit += gridDim.x;
    return unit;
  };
  // grouped: workgroup b walks the contiguous unit range [b n / grid,
  // (b + 1) n / grid), so consecutive units mostly share a token tile (the
  // ngroups row groups of one expert) and x is restaged only when it changes
  const bool contiguous = !dense;
  int u, u_end = n_units;
  if (contiguous) {
    u = int(int64_t(blockIdx.x) * n_units / gridDim.x);
    u_end = int(int64_t(blockIdx.x + 1) * n_units / gridDim.x);
  } else {
    u = next_unit(blockIdx.x);
  }
  if (u >= u_end) return;  // uniform over the workgroup
  const Q4Consts magic = q4_consts();

  // unit -> expert, output row base, live rows, this wave's tile pointers
  struct Unit {
    int slot, e, base, rows, group;
    const uint4* wp;
    const uint2* sp;
  };
  auto decode = [&](int unit) {
    Unit d;
    int it;
    if (dense) {
      d.group = dense_group(unit);
      it = (unit / 8) % n_tiles;
    } else {
      it = items[1 + unit / ngroups];
      d.group = unit % ngroups;
    }
    const int group = d.group;
    d.slot = it >> 16;
    const int m0 = (it & 0xFFFF) * 16;
    if (d.slot == 0) {
      d.e = E;
      d.base = P + m0;
      d.rows = min(16, T - m0);
    } else {
      d.e = d.slot - 1;
      d.base = offsets[d.e] + m0;
      d.rows = min(16, counts[d.e] - m0);
    }
    const size_t gt = size_t(d.e) * (n_rows / 16) + group * WAVES + wave;
    d.wp = reinterpret_cast<const uint4*>(wt) + gt * pk_stride * 64 + ks * PKS * 64 + lane;
    d.sp = reinterpret_cast<const uint2*>(sbt) + gt * pk_stride * 16 + ks * PKS * 16 + r16;
    return d;
  };
  // x staging: chunk `it` (one uint4 per thread) of a unit's 16 token rows is
  // loaded during the previous unit and written to LDS kLag steps later. A
  // vector-memory wait covers every load issued before the one it waits for,
  // so the lag is what keeps a store from draining the weight ring. With rows of >= 64 uint4 (K >= 512) a wave's chunk lies in one row, so
  // the row's source index is wave-uniform and comes through the scalar
  // cache: no vector load the weight pipeline would have to drain behind.
  auto load_x = [&](const Unit& d, int it) {
    const int i = threadIdx.x + it * kThreads;
    const int c = i % kRowU4;
    int rr = min(min(i / kRowU4, 15), d.rows - 1);
    if (kRowU4 >= 64) rr = __builtin_amdgcn_readfirstlane(rr);
    int src;
    if (SWIGLU)
      src = d.slot ? order[d.base + rr] / top : d.base - P + rr;
    else
      src = d.base + rr;
    return *reinterpret_cast<const uint4*>(x + size_t(src) * ldx + c * 8);
  };
  auto store_x = [&](const Unit& d, const uint4 v, int it, int buf) {
    uint4* xs = lds + buf * kBuf;
    float* axs = reinterpret_cast<float*>(xs + 16 * kRowU4);
    const int i = threadIdx.x + it * kThreads;
    const int r = i / kRowU4, c = i % kRowU4;
    // Rows past the tile's count hold a copy of its last row (load_x clamps):
    // they only feed output rows that are never stored, so every thread
    // writes and the store needs no branch inside the MFMA loop.
    const bool live = 16 * kRowU4 % kThreads == 0 || i < 16 * kRowU4;
    if (live) xs[r * kRowU4 + (c ^ r)] = v;
    const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) sum += bf16_to_f32(bf16_t(vw[q] & 0xFFFFu)) + bf16_to_f32(bf16_t(vw[q] >> 16));
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if (live) axs[(c >> 3) * 16 + r] = sum;  // the 8 lanes of a group hold the same sum
  };

  Unit cur = decode(u);
  uint4 wb[kPipe];
  uint2 sb[kPipe];
#pragma unroll
  for (int p = 0; p < kPipe; ++p) {
    wb[p] = load_weights<NT>(cur.wp + p * 64);
    sb[p] = load_sb<NT>(cur.sp + p * 16);
  }
#pragma unroll
  for (int it = 0; it < kIter; ++it) store_x(cur, load_x(cur, it), it, 0);
  __syncthreads();
  int buf = 0;
  for (;;) {
    const int un = SINGLE ? n_units : contiguous ? (u + 1 < u_end ? u + 1 : n_units) : next_unit(u + gridDim.x);
    const bool more = un < n_units;
    // the next unit has another token tile: stage it into the other buffer
    const bool restage = more && !(contiguous && un / ngroups == u / ngroups);
    // Without a next unit the prefetches below re-read this unit (cache hits,
    // results unused): keeping every load unconditional keeps the compiler's
    // in-order wait counts exact, so no step drains the weight pipeline.
    const Unit nxt = more ? decode(un) : cur;
    // this wave's slice: columns from 128 ks PKS, groups from 2 ks PKS
    const uint4* xr = lds + buf * kBuf + r16 * kRowU4 + ks * PKS * 16;
    const float* axs = reinterpret_cast<const float*>(lds + buf * kBuf + 16 * kRowU4) + 2 * ks * PKS * 16;
    const uint4* xf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xf[j] = xr + (((j >> 1) * 8 + qt * 2 + (j & 1)) ^ r16);
    f32x4 total = {0.f, 0.f, 0.f, 0.f};
    f32x4 bias = {0.f, 0.f, 0.f, 0.f};  // sum over groups of (b - 128 s) * sum x, by f32 MFMA
    float b_even = 0.f;                 // this lane's (b - 128 s) from the even step of a step pair
    uint4 vx[kIter];
#pragma unroll
    for (int p = 0; p < PKS; ++p) {
      if constexpr (!SINGLE) {
#pragma unroll
        for (int it = 0; it < kIter; ++it)
          if (it * kLdSpan / kIter == p) vx[it] = load_x(nxt, it);
      }
      uint4 f[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) f[q] = xf[q][16 * p];
      const uint4 w = wb[p % kPipe];
      const uint2 sbp = sb[p % kPipe];
      // refill the slot just consumed: the rest of this unit, then the next
      // unit's head (SINGLE: no next unit, and p is a compile-time step)
      if (p + kPipe < PKS) {
        wb[p % kPipe] = load_weights<NT>(cur.wp + (p + kPipe) * 64);
        sb[p % kPipe] = load_sb<NT>(cur.sp + (p + kPipe) * 16);
      } else if constexpr (!SINGLE) {
        wb[p % kPipe] = load_weights<NT>(nxt.wp + (p + kPipe - PK) * 64);
        sb[p % kPipe] = load_sb<NT>(nxt.sp + (p + kPipe - PK) * 16);
      }
      // group g: s*sum x(128+q) + (b - 128 s)*sum x. The first term is
      // accumulated by FMAs; the second is a small product over groups
      // (tokens x groups sums times groups x rows offsets) run as one
      // v_mfma_f32_16x16x4_f32 per step pair: lane quarter qt supplies group
      // 4c + qt of the pair's groups 4c..4c+3.
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      f32x4 acc0 = mfma16(__builtin_bit_cast(bf16x8, f[0]), q4_offset_bf16_s(w.x, magic), zero);
      f32x4 acc1 = mfma16(__builtin_bit_cast(bf16x8, f[2]), q4_offset_bf16_s(w.z, magic), zero);
      acc0 = mfma16(__builtin_bit_cast(bf16x8, f[1]), q4_offset_bf16_s(w.y, magic), acc0);
      acc1 = mfma16(__builtin_bit_cast(bf16x8, f[3]), q4_offset_bf16_s(w.w, magic), acc1);
      const float s0 = __builtin_bit_cast(float, sbp.x << 16), s1 = __builtin_bit_cast(float, sbp.y << 16);
      const uint32_t mine = (qt & 1) ? sbp.y : sbp.x;  // (scale, bias) of this lane's group
      const float b_mine = __builtin_fmaf(-128.f, __builtin_bit_cast(float, mine << 16),
                                          __builtin_bit_cast(float, mine & 0xFFFF0000u));
      if (p % 2 == 0) {
        b_even = b_mine;
      } else {
        const float ax = axs[(2 * p - 2 + qt) * 16 + r16];
        bias = __builtin_amdgcn_mfma_f32_16x16x4f32(ax, qt < 2 ? b_even : b_mine, bias, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        total[r] = __builtin_fmaf(s0, acc0[r], total[r]);
        total[r] = __builtin_fmaf(s1, acc1[r], total[r]);
      }
      // the next unit's x chunk goes to the other LDS buffer (free since the
      // last barrier); without a next unit it is never read
      if constexpr (!SINGLE) {
        if (restage) {
#pragma unroll
          for (int it = 0; it < kIter; ++it)
            if (it * kLdSpan / kIter + kLag == p) store_x(nxt, vx[it], it, buf ^ 1);
        }
      }
      // materialise the running sum here: otherwise the adds sink past the
      // loop and every group's MFMA results stay live in accumulators
      asm volatile("" : "+v"(total));
      __builtin_amdgcn_sched_barrier(0);
    }
    // total[r] = row qt*4 + r of the tile, weight row r16
#pragma unroll
    for (int r = 0; r < 4; ++r) total[r] += bias[r];
    if constexpr (KS > 1) {
      // slices meet in LDS (the x tile is no longer read once every wave is
      // past the barrier) and slice 0 adds them in slice order
      f32x4* red = reinterpret_cast<f32x4*>(lds);
      __syncthreads();
      red[(ks * WAVES + wave) * 64 + lane] = total;
      __syncthreads();
      if (ks == 0) {
#pragma unroll
        for (int k = 1; k < KS; ++k) {
          const f32x4 o = red[(k * WAVES + wave) * 64 + lane];
#pragma unroll
          for (int r = 0; r < 4; ++r) total[r] += o[r];
        }
      }
    }
    const int tile = cur.group * WAVES + wave;
    if (KS > 1 && ks != 0) {
      // partial sums handed to slice 0
    } else if (SWIGLU) {
      bf16_t* y = static_cast<bf16_t*>(yv);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float uu = __shfl_xor(total[r], 8, 64);
        const int m = qt * 4 + r;
        if (r16 < 8 && m < cur.rows) {
          const float g = total[r];
          y[size_t(cur.base + m) * ldy + tile * 8 + r16] = f32_to_bf16(g / (1.f + __expf(-g)) * uu);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = qt * 4 + r;
        if (m >= cur.rows) continue;
        const size_t o = size_t(cur.base + m) * ldy + tile * 16 + r16;
        if (OUT == 0)
          static_cast<bf16_t*>(yv)[o] = f32_to_bf16(total[r]);
        else if (OUT == 1)
          static_cast<float*>(yv)[o] = total[r];
        else
          static_cast<float*>(yv)[o] += total[r];
      }
    }
    if (!more) break;
    if (restage) {
      __syncthreads();  // the next tile is staged and every wave is done with this one
      buf ^= 1;
    }
    cur = nxt;
    u = un;
  }
}

// WAVES waves per workgroup (a unit covers 16 * WAVES weight rows) and a ring
// of 64 / WAVES pairs per wave: 64 KB of weights in flight per workgroup.
template <int PK, int WAVES, bool SWIGLU, int OUT, bool NT, bool SINGLE = false, int KS = 1>
void launch_stream_gemm(const bf16_t* x, const uint32_t* w, const bf16_t* sb, int n_rows, const int32_t* counts,
                        const int32_t* offsets, const int32_t* order, const int32_t* items, int E, int top, int T,
                        int dense, void* y, int ldy, int ldx, int pk_stride, hipStream_t stream, int min_grid = 0) {
  constexpr int kNPipe = 64 / (WAVES * KS);
  const auto kernel = &stream_gemm_kernel<PK, WAVES, kNPipe, SWIGLU, OUT, NT, SINGLE, KS>;
  const int lds = (SINGLE ? 1 : 2) * (16 * PK * 128 * 2 + PK * 2 * 16 * 4);
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  HB_CHECK(attr);
  static int grid = 0;
  if (!grid) {
    int dev = 0, cus = 0, per = 0;
    HB_CHECK(hipGetDevice(&dev));
    HB_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    HB_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(kernel),
                                                          64 * WAVES * KS, lds));
    grid = cus * (per > 0 ? per : 1);
  }
  hipLaunchKernelGGL(kernel, dim3(std::max(grid, min_grid)), dim3(64 * WAVES * KS), lds, stream, x, w, sb, n_rows, counts,
                     offsets, order, items, E, top, T, dense, y, ldy, ldx, pk_stride);
}

// Dense shapes whose every token count runs the K-sliced single-unit form:
// K = 4096 (the output projections, too wide for the projection kernels) and
// fewer than 4096 rows (the router: too few row blocks to fill the GPU with
// 128-row projection workgroups). The family depends on the shape only, so a
// row's result never depends on the batch it is packed in.
inline bool dense_sliced(int n_rows, int K) { return K == 4096 || n_rows < 4096; }

inline int device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    HB_CHECK(hipGetDevice(&dev));
    HB_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  }
  return cus;
}

// Persistent streaming GEMM over 256-row weight groups (n_rows % 256 == 0).
// K / 128 in {2, 4, 8, 16} runs in one pass; a larger K (a multiple of 2048)
// runs as passes over 2048-wide column blocks accumulated in f32 (OUT 1 and 2
// only). False when the shape is not covered.
template <bool SWIGLU, int OUT>
bool stream_gemm(const bf16_t* x, int K, const uint32_t* w, const bf16_t* sb, int n_rows, const int32_t* counts,
                 const int32_t* offsets, const int32_t* order, const int32_t* items, int E, int top, int T, int dense,
                 void* y, int ldy, hipStream_t stream) {
  if (n_rows % 256) return false;
  const int P = K / 128;
  // A dense matrix with fewer 256-row units than CUs (the output projections
  // and the router at a few token tiles) runs as 64-row units of 4 waves, so
  // every CU streams a share. With more units the 16-wave form is faster: one
  // wave per SIMD cannot hide its own LDS and MFMA latency over several units.
  const bool narrow = !SWIGLU && dense && (n_rows / 256) * ((T + 15) / 16) < device_cus();
#define HB_SG_LAUNCH(PKC, WV, OUTC, NTC, XO, PO)                                                              \
  launch_stream_gemm<PKC, WV, SWIGLU, OUTC, NTC>(x + (XO), w + size_t(PO) * 256, sb + size_t(PO) * 64, n_rows, \
                                                       counts, offsets, order, items, E, top, T, dense, y, ldy, K, P, \
                                                       stream)
#define HB_SG(PKC, OUTC, XO, PO)                                      \
  (narrow  ? HB_SG_LAUNCH(PKC, SWIGLU ? 16 : 4, OUTC, false, XO, PO) \
   : dense ? HB_SG_LAUNCH(PKC, 16, OUTC, false, XO, PO)               \
           : HB_SG_LAUNCH(PKC, 16, OUTC, true, XO, PO))
  // The K-sliced family (dense_sliced) in one launch with a workgroup per
  // 64-row unit (in rounds when the units outnumber the resident workgroups),
  // each 16-row tile split over K slices: a short dependent chain per wave, and
  // the same arithmetic at every token count (unlike passes over 2048-wide
  // column blocks). Other shapes keep the unsliced form below, whose per-row
  // arithmetic is that of the projection kernels.
  if constexpr (!SWIGLU) {
    if (dense && dense_sliced(n_rows, K)) {
      const int units = ((n_rows / 64 + 7) / 8 * 8) * ((T + 15) / 16);
#define HB_SG_SINGLE(PKC, KSC)                                                                                      \
  launch_stream_gemm<PKC, 4, SWIGLU, OUT, false, true, KSC>(x, w, sb, n_rows, counts, offsets, order, items, E, top, \
                                                            T, dense, y, ldy, K, P, stream, units)
      switch (P) {
        case 2: HB_SG_SINGLE(2, 1); return true;
        case 4: HB_SG_SINGLE(4, 2); return true;
        case 8: HB_SG_SINGLE(8, 4); return true;
        case 16: HB_SG_SINGLE(16, 4); return true;
        case 32: HB_SG_SINGLE(32, 4); return true;
        default: break;
      }
#undef HB_SG_SINGLE
    }
  }
  switch (P) {
    case 2: HB_SG(2, OUT, 0, 0); return true;
    case 4: HB_SG(4, OUT, 0, 0); return true;
    case 8: HB_SG(8, OUT, 0, 0); return true;
    case 16: HB_SG(16, OUT, 0, 0); return true;
    default: break;
  }
  if (SWIGLU || OUT == 0 || P % 16) return false;
  for (int c = 0; c < P / 16; ++c) {
    if (c == 0 && OUT == 1)
      HB_SG(16, 1, 0, 0);
    else
      HB_SG(16, 2, c * 2048, c * 16);
  }
  return true;
#undef HB_SG
#undef HB_SG_LAUNCH
}

}  // namespace
}  // namespace hb
