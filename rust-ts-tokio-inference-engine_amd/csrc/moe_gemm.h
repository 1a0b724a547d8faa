// Grouped 4-bit MoE GEMM over the routing work list (gate/up with the SwiGLU
// epilogue, and down). Device template: included by moe.hip.
//
// Work: a piece is (work item, 16-row weight tile) = one expert's 16 weight
// rows over all of K against the item's token rows (at most 16). The pieces
// are cut into equal contiguous ranges, one per persistent workgroup (16
// waves, one per CU). Three things keep a CU streaming weights until the
// launch ends:
//  - Staging only what an item holds. A routed expert's item holds a few
//    tokens (about 2.7 at 128 tokens, top-10 of 512), so a workgroup stages
//    the token rows of all the items its range touches into LDS once, with
//    their per-group sums, and then runs without a barrier. Only a range whose
//    rows do not fit (cap_rows) is staged in phases, two barriers each.
//  - Pieces on demand. A CU's scheduler issues its oldest waves first, so 16
//    waves given equal shares of a range finish up to a third of the launch
//    apart (measured: waves 0-3 of every SIMD at 60 us, waves 12-15 at 91 us
//    of a 100 us gate/up launch). Here every wave takes its next piece from an
//    LDS counter one piece ahead, so the favoured waves simply do more.
//  - The shared expert's token tiles (16 rows each, first in the list) are
//    walked spread among the routed tiles, so no range needs a second phase.
// Weights stream through a 4-step register ring per wave that runs on into
// the next piece; codes and scale/bias pairs are streaming (non-temporal)
// loads, read once per launch. Per output row the arithmetic is the streaming
// GEMM's: s * sum x (128 + q) per step with bf16 operands, plus
// (b - 128 s) * sum x as one f32 MFMA per step pair, groups in K order.
#pragma once
#include <algorithm>

#include "hb_common.h"
#include "q4_device.h"

namespace hb {
namespace {

template <class V>
__device__ inline V nt_load(const V* p) {
  return __builtin_nontemporal_load(p);
}
__device__ inline uint4 load_w_nt(const uint4* p) {
  using v4u = unsigned __attribute__((ext_vector_type(4)));
  const v4u v = nt_load(reinterpret_cast<const v4u*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}
__device__ inline uint2 load_sb_nt(const uint2* p) {
  using v2u = unsigned __attribute__((ext_vector_type(2)));
  const v2u v = nt_load(reinterpret_cast<const v2u*>(p));
  return uint2{v.x, v.y};
}

// The work list in walk order: the n_shared shared-expert tiles (listed
// first) go one at the head of each of n_shared blocks of the routed tiles, so
// no contiguous range of the list holds all of them. moe_walk_pos gives the
// walk position of list index li.
__host__ __device__ inline int moe_walk_pos(int li, int n_items, int n_shared) {
  const int q = (n_items - n_shared) / n_shared;
  if (li < n_shared) return li * (q + 1);
  const int r = li - n_shared;
  if (r < n_shared * q) return (r / q) * (q + 1) + r % q + 1;
  return li;
}

// Entries of the work list: (T + 15) / 16 shared tiles plus at most
// ceil(count / 16) tiles per routed expert.
__host__ __device__ inline int moe_list_capacity(int T, int E, int top) {
  return (T + 15) / 16 + E + (T * top + 15) / 16;
}

// The work records follow the list in the items buffer, 16-byte aligned: one
// 64-byte record per list entry, in walk order, written by the routing sort.
//   uint4 0: expert (E = shared), first output row, live rows (1..16), 0
//   uint4 1-2: the 16 source tokens of the rows as uint16 (gate/up reads
//              x[token]), entries past the live rows repeat the last one
//   uint4 3: zero
__host__ __device__ inline int moe_records_offset(int T, int E, int top) {
  return (1 + moe_list_capacity(T, E, top) + 3) & ~3;
}

// Writes the records (expert threads tid < E their own tiles: count v, first
// sorted row excl, first routed list index first; threads < n_shared the
// shared tiles). stok: the token of every sorted pair.
__device__ inline void moe_write_records(uint4* __restrict__ recs, const uint16_t* stok, int tid, int nthreads, int E,
                                         int T, int P, int n_shared, int n_items, int v, int excl, int first) {
  auto put = [&](int li, int e, int base, int rows, auto tok) {
    uint32_t t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = uint32_t(tok(min(2 * i, rows - 1))) | (uint32_t(tok(min(2 * i + 1, rows - 1))) << 16);
    uint4* r = recs + size_t(moe_walk_pos(li, n_items, n_shared)) * 4;
    r[0] = make_uint4(uint32_t(e), uint32_t(base), uint32_t(rows), 0u);
    r[1] = make_uint4(t[0], t[1], t[2], t[3]);
    r[2] = make_uint4(t[4], t[5], t[6], t[7]);
    r[3] = make_uint4(0u, 0u, 0u, 0u);
  };
  if (tid < E)
    for (int j = 0; j < (v + 15) / 16; ++j)
      put(n_shared + first + j, tid, excl + 16 * j, min(16, v - 16 * j),
          [&](int i) { return uint32_t(stok[excl + 16 * j + i]); });
  for (int s = tid; s < n_shared; s += nthreads)
    put(s, E, P + 16 * s, min(16, T - 16 * s), [&](int i) { return uint32_t(16 * s + i); });
}

constexpr int kMgWaves = 16;  // waves per workgroup (one workgroup per CU)
constexpr int kMgRing = 4;    // weight steps in flight per wave
constexpr int kMgRec = 64;    // records per phase: a phase holds at most cap_rows <= 64 items

// LDS: [cap_rows][K/8] uint4 x rows (XOR-swizzled by row & 15), [kMgRec][4]
// uint4 records of the phase's items, [K/64][cap_rows] f32 group sums,
// [cap_rows] source rows, [kMgRec] first staged row of each phase item, then
// the piece counter.
inline size_t moe_gemm_lds(int K, int cap_rows) {
  return size_t(cap_rows) * (size_t(K) * 2 + K / 64 * 4 + 4) + kMgRec * (64 + 4) + 16;
}

template <int PK, bool SWIGLU>
__global__ __launch_bounds__(64 * kMgWaves) void moe_gemm_kernel(const bf16_t* __restrict__ x,
                                                               const uint32_t* __restrict__ wt,
                                                               const bf16_t* __restrict__ sbt, int n_rows,
                                                               const int32_t* __restrict__ items,
                                                               const uint4* __restrict__ recs, int E, int T,
                                                               bf16_t* __restrict__ y, int ldy, int ldx,
                                                               int cap_rows) {
  constexpr int kPipe = kMgRing < PK ? kMgRing : PK;
  static_assert((PK % 2 == 0 && PK % kPipe == 0) || PK == 2, "whole step pairs; the ring divides the steps");
  constexpr int K = PK * 128;
  constexpr int kRowU4 = K / 8;
  constexpr int kG = K / 64;
  constexpr int kThreads = 64 * kMgWaves;
  extern __shared__ uint4 lds[];
  uint4* const rec_lds = lds + size_t(cap_rows) * kRowU4;
  float* const gsum = reinterpret_cast<float*>(rec_lds + kMgRec * 4);
  int* const src_tab = reinterpret_cast<int*>(gsum + size_t(kG) * cap_rows);
  int* const row_off = src_tab + cap_rows;
  int* const counter = row_off + kMgRec;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int r16 = lane & 15, qt = lane >> 4;
  const int ngroups = n_rows / (16 * kMgWaves);  // 256-row groups per expert
  const int ppi = ngroups * kMgWaves;             // pieces per item
  // this workgroup's pieces [u, u_end) of items * ppi
  const int n_all = items[0] * ppi;
  int u = int(int64_t(blockIdx.x) * n_all / gridDim.x);
  const int u_end = int(int64_t(blockIdx.x + 1) * n_all / gridDim.x);
  if (u >= u_end) return;  // uniform over the workgroup
  const int item_last = (u_end - 1) / ppi;
  const Q4Consts magic = q4_consts();

  struct Piece {
    int k, tile, base, rows;  // phase item, weight tile, first output row, live rows
    const uint4* wp;
    const uint2* sp;
  };
  auto weights_of = [&](Piece& pc, int e) {
    const size_t gt = size_t(e) * (n_rows / 16) + pc.tile;
    pc.wp = reinterpret_cast<const uint4*>(wt) + gt * PK * 64 + lane;
    pc.sp = reinterpret_cast<const uint2*>(sbt) + gt * PK * 16 + r16;
  };
  // piece g of the list, its item's record read from LDS (phase items from item0)
  auto piece_at = [&](int g, int item0) {
    Piece pc;
    const int unit = g / kMgWaves;
    pc.k = unit / ngroups - item0;
    pc.tile = (unit % ngroups) * kMgWaves + g % kMgWaves;
    const uint4 r = rec_lds[pc.k * 4];
    pc.base = __builtin_amdgcn_readfirstlane(int(r.y));
    pc.rows = __builtin_amdgcn_readfirstlane(int(r.z));
    weights_of(pc, __builtin_amdgcn_readfirstlane(int(r.x)));
    return pc;
  };
  auto grab = [&]() {
    int v = 0;
    if (lane == 0) v = atomicAdd(counter, 1);
    return __builtin_amdgcn_readfirstlane(v);
  };

  uint4 wb[kPipe];
  uint2 sb[kPipe];
  for (;;) {  // phases: whole items whose rows fit in cap_rows
    const int item0 = u / ppi;
    const int n_rec = min(item_last - item0 + 1, kMgRec);
    // The phase's records (thread t loads and stores uint4 min(t, 4 n_rec - 1):
    // unconditional, so the load is not sunk below the weight loads to a
    // conditional store) and this wave's first piece's weights, whose expert
    // the wave reads from the record itself, go out before any wait: three
    // dependent loads (the item count, the records, the x rows) precede the
    // first MFMA.
    const int rslot = min(int(threadIdx.x), 4 * n_rec - 1);
    const uint4 rv = recs[size_t(item0) * 4 + rslot];
    Piece cur;
    {
      const int g0 = min(u + wave, u_end - 1);
      const int unit = g0 / kMgWaves;
      cur.tile = (unit % ngroups) * kMgWaves + g0 % kMgWaves;
      weights_of(cur, __builtin_amdgcn_readfirstlane(int(recs[size_t(unit / ngroups) * 4].x)));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < kPipe; ++p) {
      wb[p] = load_w_nt(cur.wp + p * 64);
      sb[p] = load_sb_nt(cur.sp + p * 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    rec_lds[rslot] = rv;  // threads past 4 n_rec rewrite the last uint4 with its own value
    if (threadIdx.x == 0) *counter = kMgWaves;
    lds_barrier();

    // the phase: its first item, then items while the rows fit (every wave
    // scans the records, lane j holding item item0 + j; rows > 0, so the items
    // that fit are a prefix)
    const int rows_j = lane < n_rec ? int(rec_lds[lane * 4].z) : 0;
    int incl = rows_j;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    const int n_ph = __popcll(__ballot(lane < n_rec && (lane == 0 || incl <= cap_rows)));
    const int rows_acc = __shfl(incl, n_ph - 1, 64);
    const int u_ph_end = min(u_end, (item0 + n_ph) * ppi);
    const int n_pieces = u_ph_end - u;
    // source row of every staged row, first row of every phase item: thread
    // (wave w, lane l) covers row l % 16 of items 4 w + l / 16 + 4 kMgWaves j
    for (int kk = 4 * wave + (lane >> 4); kk < 4 * ((n_ph + 3) / 4); kk += 4 * kMgWaves) {
      const int i = lane & 15;
      const int off = __shfl(incl - rows_j, kk, 64);
      if (kk < n_ph) {
        const uint4 r0 = rec_lds[kk * 4];
        if (i == 0) row_off[kk] = off;
        if (i < int(r0.z)) {
          int src = int(r0.y) + i;
          if (SWIGLU) {
            const uint4 tk = rec_lds[kk * 4 + 1 + (i >> 3)];
            const int wi = (i >> 1) & 3;
            const uint32_t wd = wi == 0 ? tk.x : wi == 1 ? tk.y : wi == 2 ? tk.z : tk.w;
            src = int((i & 1) ? (wd >> 16) : (wd & 0xFFFFu));
          }
          src_tab[off + i] = src;
        }
      }
    }
    lds_barrier();
    // the rows, 16 bytes per thread and four at a time, with the per-group
    // sums of x (the eight lanes of a 64-column group combine by xor shuffles)
    const int n_chunks = rows_acc * kRowU4;
    for (int i0 = 0; i0 < n_chunks; i0 += 4 * kThreads) {
      uint4 v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = i0 + k * kThreads + threadIdx.x;
        const int r = min(i / kRowU4, rows_acc - 1), c = i % kRowU4;
        v[k] = *reinterpret_cast<const uint4*>(x + size_t(src_tab[r]) * ldx + c * 8);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = i0 + k * kThreads + threadIdx.x;
        const int r = min(i / kRowU4, rows_acc - 1), c = i % kRowU4;
        if (i < n_chunks) lds[r * kRowU4 + (c ^ (r & 15))] = v[k];
        const uint32_t vw[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) sum += bf16_to_f32(bf16_t(vw[q] & 0xFFFFu)) + bf16_to_f32(bf16_t(vw[q] >> 16));
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        sum += __shfl_xor(sum, 4, 64);
        if (i < n_chunks && (c & 7) == 0) gsum[(c >> 3) * cap_rows + r] = sum;
      }
    }
    lds_barrier();

    // each wave's first piece is its index (the ring holds its weights when
    // it has one); the rest come from the counter
    int my = wave;
    cur = piece_at(u + min(my, n_pieces - 1), item0);
    while (my < n_pieces) {
      // the next piece is taken now, so its first weights can follow this one's
      const int nx = grab();
      const Piece nxt = nx < n_pieces ? piece_at(u + nx, item0) : cur;
      // the item's rows, clamped to its count: rows past it only feed output
      // rows that are never stored
      const int prow = row_off[cur.k] + min(r16, cur.rows - 1);
      const uint4* xr = lds + prow * kRowU4;
      const float* axs = gsum + prow;
      const int sw = prow & 15;
      f32x4 total = {0.f, 0.f, 0.f, 0.f};
      f32x4 bias = {0.f, 0.f, 0.f, 0.f};  // sum over groups of (b - 128 s) * sum x
      float b_even = 0.f;
#pragma unroll
      for (int p = 0; p < PK; ++p) {
        uint4 f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) f[j] = xr[(16 * p + (j >> 1) * 8 + qt * 2 + (j & 1)) ^ sw];
        const uint4 w = wb[p % kPipe];
        const uint2 sbp = sb[p % kPipe];
        // refill the slot: the rest of this piece, then the next piece's head
        // (this piece again past the phase: loaded, never used)
        if (p + kPipe < PK) {
          wb[p % kPipe] = load_w_nt(cur.wp + (p + kPipe) * 64);
          sb[p % kPipe] = load_sb_nt(cur.sp + (p + kPipe) * 16);
        } else {
          wb[p % kPipe] = load_w_nt(nxt.wp + (p + kPipe - PK) * 64);
          sb[p % kPipe] = load_sb_nt(nxt.sp + (p + kPipe - PK) * 16);
        }
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 acc0 = mfma16(__builtin_bit_cast(bf16x8, f[0]), q4_offset_bf16_s(w.x, magic), zero);
        f32x4 acc1 = mfma16(__builtin_bit_cast(bf16x8, f[2]), q4_offset_bf16_s(w.z, magic), zero);
        acc0 = mfma16(__builtin_bit_cast(bf16x8, f[1]), q4_offset_bf16_s(w.y, magic), acc0);
        acc1 = mfma16(__builtin_bit_cast(bf16x8, f[3]), q4_offset_bf16_s(w.w, magic), acc1);
        const float s0 = __builtin_bit_cast(float, sbp.x << 16), s1 = __builtin_bit_cast(float, sbp.y << 16);
        const uint32_t mine = (qt & 1) ? sbp.y : sbp.x;  // (scale, bias) of this lane's group
        const float b_mine = __builtin_fmaf(-128.f, __builtin_bit_cast(float, mine << 16),
                                            __builtin_bit_cast(float, mine & 0xFFFF0000u));
        // groups 4c .. 4c + 3 of a step pair: lane quarter qt supplies group 4c + qt
        if (p % 2 == 0) {
          b_even = b_mine;
        } else {
          const float ax = axs[(2 * p - 2 + qt) * cap_rows];
          bias = __builtin_amdgcn_mfma_f32_16x16x4f32(ax, qt < 2 ? b_even : b_mine, bias, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          total[r] = __builtin_fmaf(s0, acc0[r], total[r]);
          total[r] = __builtin_fmaf(s1, acc1[r], total[r]);
        }
        // materialise the running sum here: otherwise the adds sink past the
        // loop and every step's MFMA results stay live in accumulators
        asm volatile("" : "+v"(total));
        __builtin_amdgcn_sched_barrier(0);
      }
      // total[r] = token row 4 qt + r of the item, weight row r16 of the tile
#pragma unroll
      for (int r = 0; r < 4; ++r) total[r] += bias[r];
      if (SWIGLU) {  // lane pairs (gate r16, up r16 + 8) of a tile
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float uu = __shfl_xor(total[r], 8, 64);
          const int m = qt * 4 + r;
          if (r16 < 8 && m < cur.rows) {
            const float g = total[r];
            y[size_t(cur.base + m) * ldy + cur.tile * 8 + r16] = f32_to_bf16(g / (1.f + __expf(-g)) * uu);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = qt * 4 + r;
          if (m < cur.rows) y[size_t(cur.base + m) * ldy + cur.tile * 16 + r16] = f32_to_bf16(total[r]);
        }
      }
      my = nx;
      cur = nxt;
    }
    if (u_ph_end >= u_end) break;
    u = u_ph_end;
    lds_barrier();  // every wave is done with this phase's rows and records
  }
}

// Runs the grouped GEMM over the work list when the shape suits it (K / 128
// in {2, 4, 8, 16}, n_rows % 256 == 0); false otherwise, nothing launched.
template <bool SWIGLU>
bool moe_gemm(const bf16_t* x, int K, const uint32_t* w, const bf16_t* sb, int n_rows, const int32_t* items, int E,
              int top, int T, bf16_t* y, hipStream_t stream) {
  if (n_rows % (16 * kMgWaves)) return false;
  constexpr size_t kLdsMax = 160 * 1024;
  const size_t fixed = moe_gemm_lds(K, 0), per_row = moe_gemm_lds(K, 1) - fixed;
  const int cap = int(std::min<size_t>(kMgRec, (kLdsMax - fixed) / per_row));
  if (cap < 16) return false;  // one whole item must fit
  const uint4* recs = reinterpret_cast<const uint4*>(items + moe_records_offset(T, E, top));
  const size_t lds = moe_gemm_lds(K, cap);
  const int ldy = SWIGLU ? n_rows / 2 : n_rows;
  auto launch = [&](auto kernel) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(kLdsMax));
    HB_CHECK(attr);
    static int grid = 0;
    if (!grid) {
      int dev = 0, cus = 0, per = 0;
      HB_CHECK(hipGetDevice(&dev));
      HB_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
      HB_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(kernel),
                                                            64 * kMgWaves, lds));
      grid = cus * (per > 0 ? per : 1);
    }
    launch_timed(kernel, dim3(grid), dim3(64 * kMgWaves), lds, stream, x, w, sb, n_rows, items, recs, E, T, y, ldy, K,
                 cap);
  };
  switch (K / 128) {
    case 2: launch(&moe_gemm_kernel<2, SWIGLU>); return true;
    case 4: launch(&moe_gemm_kernel<4, SWIGLU>); return true;
    case 8: launch(&moe_gemm_kernel<8, SWIGLU>); return true;
    case 16: launch(&moe_gemm_kernel<16, SWIGLU>); return true;
    default: return false;
  }
}

}  // namespace
}  // namespace hb
