// Sparse MoE block for gfx950.
//
// moe_route_kernel (one workgroup): each wave takes tokens round-robin; a lane
// holds experts lane, lane+64, ... as 64-bit keys (IEEE total-order key of the
// logit, then the complemented expert index, so the larger logit and on ties
// the lower index wins) and the top-k are k wave-wide max reductions. The
// permutation is a stable counting sort: wave 0 walks the pairs in order, 64
// at a time, finds the lanes holding the same expert with one ballot per
// expert-index bit, ranks each pair among them and bumps the per-expert count
// once per group; the counts are scanned and every pair is scattered to
// offsets[e] + rank.
//
// moe_grouped_qmm_kernel: grid (16-row weight tiles, expert slots); a slot is
// a routed expert or a 16-token chunk of the shared expert. The expert's
// weights go through the same MFMA path as the dense kernel (one tile of 16
// output rows per workgroup, waves split K and reduce in LDS), looping over the
// expert's token list 16 rows at a time.
#include "moe.h"

#include <type_traits>

#include "moe_gemm.h"
#include "q4_device.h"

namespace hb {
namespace {

__device__ inline uint32_t total_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline float key_value(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __builtin_bit_cast(float, u);
}

constexpr int kSortThreads = 1024;
constexpr int kMaxExperts = 1024;
constexpr int kTopkWaves = 4;

// One DPP step of a wave-wide u64 max: lanes of the rows in ROW_MASK combine
// with the lane CTRL selects (quad permutes, mirrors and row broadcasts are
// VALU operations, no LDS round trip).
template <int CTRL, int ROW_MASK>
__device__ inline unsigned long long dpp_max(unsigned long long v) {
  const int lo = int(uint32_t(v)), hi = int(uint32_t(v >> 32));
  const uint32_t olo = uint32_t(__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xF, false));
  const uint32_t ohi = uint32_t(__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xF, false));
  const unsigned long long o = (static_cast<unsigned long long>(ohi) << 32) | olo;
  return o > v ? o : v;
}

// Wave-wide max: pairs, quads, half rows, rows (16 lanes), then row 0 into
// row 1 and row 2 into row 3, then rows 0-1 into rows 2-3; lane 63 ends with
// the maximum, which is broadcast through scalar registers.
__device__ inline unsigned long long wave_max_dpp(unsigned long long v) {
  v = dpp_max<0xB1, 0xF>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_max<0x4E, 0xF>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_max<0x141, 0xF>(v);  // row_half_mirror
  v = dpp_max<0x140, 0xF>(v);  // row_mirror
  v = dpp_max<0x142, 0xA>(v);  // row_bcast:15
  v = dpp_max<0x143, 0xC>(v);  // row_bcast:31
  const uint32_t lo = __builtin_amdgcn_readlane(uint32_t(v), 63);
  const uint32_t hi = __builtin_amdgcn_readlane(uint32_t(v >> 32), 63);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// One wave per token: top-k of the first E logits under the total order, then
// the selection's softmax weights (largest logit first). A lane holds PER keys
// (expert lane + 64 k); each of the k rounds is a wave max over 64-bit keys
// (total-order key of the logit, complemented expert index, so on equal
// logits the lower index wins) and the winner's key is cleared. The selected
// logits are recovered from the keys, so no second read of the row.
template <int PER>
__global__ __launch_bounds__(64 * kTopkWaves) void moe_topk_kernel(const float* __restrict__ logits, int ld, int T,
                                                                   int E, int top, int32_t* __restrict__ idx,
                                                                   float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kTopkWaves + (threadIdx.x >> 6);
  if (t >= T) return;  // uniform over the wave
  const float* row = logits + size_t(t) * ld;
  unsigned long long key[PER];
  float lv[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) lv[k] = row[min(lane + 64 * k, E - 1)];  // all loads in flight at once
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = lane + 64 * k;
    key[k] = e < E ? (static_cast<unsigned long long>(total_key(lv[k])) << 32) | uint32_t(~e) : 0ull;
  }
  // lane j keeps the j-th selected logit
  float mine = 0.f, first = 0.f;
  for (int j = 0; j < top; ++j) {
    unsigned long long best = key[0];
#pragma unroll
    for (int k = 1; k < PER; ++k) best = key[k] > best ? key[k] : best;
    best = wave_max_dpp(best);
    const int e = int(~uint32_t(best & 0xFFFFFFFFu));
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (lane + 64 * k == e) key[k] = 0ull;
    const float v = key_value(uint32_t(best >> 32));
    if (j == 0) first = v;
    if (lane == j) {
      mine = v;
      idx[size_t(t) * top + j] = e;
    }
  }
  // weights: softmax renormalised over the selection (largest logit first)
  const float ex = lane < top ? __expf(mine - first) : 0.f;
  float tot = ex;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) tot += __shfl_xor(tot, off, 64);
  if (lane < top) weights[size_t(t) * top + lane] = ex / tot;
}

// Exclusive scan over the workgroup (one value per thread); *total gets the sum.
__device__ inline int block_exclusive_scan(int v, int32_t* scan, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(inc, off, 64);
    if (lane >= off) inc += u;
  }
  __syncthreads();  // scan[] may still be read by a previous call
  if (lane == 63) scan[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    const int ws = lane < nwaves ? scan[lane] : 0;
    int wi = ws;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int u = __shfl_up(wi, off, 64);
      if (lane >= off) wi += u;
    }
    if (lane < nwaves) scan[lane] = wi - ws;
    if (lane == nwaves - 1) scan[32] = wi;
  }
  __syncthreads();
  *total = scan[32];
  return scan[wave] + inc - v;
}

// Stable counting sort of the flattened (token, slot) pairs by expert (one
// workgroup): wave 0 walks the pairs in order, 64 at a time, finds the lanes
// holding the same expert with one ballot per expert-index bit, ranks each
// pair among them and bumps the per-expert count once per group; the counts
// are scanned and every pair is scattered to offsets[e] + rank.
// It also lists the grouped GEMM's work items: items[0] = count, then one
// entry per 16-row tile, slot << 16 | tile, the shared expert's token tiles
// (slot 0) first, then each routed expert e's pair tiles (slot e + 1); and
// after the list one record per item in walk order (moe_write_records).
__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(const int32_t* __restrict__ idx, int T, int top,
                                                                int E, int32_t* __restrict__ counts,
                                                                int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ order,
                                                                int32_t* __restrict__ inverse,
                                                                int32_t* __restrict__ items,
                                                                int32_t* __restrict__ active) {
  const int P = T * top;
  __shared__ int32_t sidx[kMoeMaxPairs];
  __shared__ int32_t rank[kMoeMaxPairs];
  __shared__ int32_t cnt[kMaxExperts];
  __shared__ int32_t scan[33];
  __shared__ uint16_t stok[kMoeMaxPairs];  // token of every sorted pair
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < kMaxExperts; e += blockDim.x) cnt[e] = 0;
  for (int p = tid; p < P; p += blockDim.x) sidx[p] = idx[p];
  __syncthreads();
  if (wave == 0) {
    const int bits = 32 - __builtin_clz(unsigned(E > 1 ? E - 1 : 1));
    for (int c = 0; c < P; c += 64) {
      const int p = c + lane;
      const bool valid = p < P;
      const int e = valid ? sidx[p] : 0;
      unsigned long long same = __ballot(valid);
      for (int b = 0; b < bits; ++b) {
        const unsigned long long ones = __ballot(valid && ((e >> b) & 1));
        same &= ((e >> b) & 1) ? ones : ~ones;
      }
      const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
      const int base = valid ? cnt[e] : 0;
      const int local = __popcll(same & below);
      const bool leader = valid && (same >> lane) == 1ull;  // highest lane of its group
      if (valid) rank[p] = base + local;
      if (leader) cnt[e] = base + __popcll(same);
    }
  }
  __syncthreads();
  // exclusive scan of the counts (E <= 1024, one expert per thread)
  const int v = tid < E ? cnt[tid] : 0;
  int total_pairs;
  const int excl = block_exclusive_scan(v, scan, &total_pairs);
  // work items
  const int shared_tiles = (T + 15) / 16;
  const int tiles = (v + 15) / 16;
  int total_tiles;
  const int first = block_exclusive_scan(tiles, scan, &total_tiles);
  for (int j = 0; j < tiles; ++j) items[1 + shared_tiles + first + j] = ((tid + 1) << 16) | j;
  for (int j = tid; j < shared_tiles; j += blockDim.x) items[1 + j] = j;
  if (tid == 0) items[0] = shared_tiles + total_tiles;
  if (active) {  // routed experts with at least one pair (the weights a grouped GEMM reads)
    int n_active;
    block_exclusive_scan(v > 0 ? 1 : 0, scan, &n_active);
    if (tid == 0) active[0] = n_active;
  }
  if (tid < E) {
    counts[tid] = v;
    offsets[tid] = excl;
    cnt[tid] = excl;  // reuse as offsets for the scatter
  }
  if (tid == E - 1) offsets[E] = excl + v;
  __syncthreads();
  for (int p = tid; p < P; p += blockDim.x) {
    const int dst = cnt[sidx[p]] + rank[p];
    order[dst] = p;
    inverse[p] = dst;
    stok[dst] = uint16_t(p / top);
  }
  __syncthreads();
  moe_write_records(reinterpret_cast<uint4*>(items + moe_records_offset(T, E, top)), stok, tid, blockDim.x, E, T, P,
                    shared_tiles, shared_tiles + total_tiles, v, excl, first);
}

// The same stable permutation through per-expert token bitmaps [E][W]
// (W = ceil(T / 64) words): the top-k experts of a token are distinct, so
// within an expert the pairs are ordered by token, and a pair's rank is the
// number of earlier tokens set in its expert's bitmap. Bitmaps are built with
// LDS atomic ORs (order-free, so the result is deterministic), then counts,
// offsets and work items come from block scans and every pair is placed
// independently. Needs E * W <= kBitmapWords.
constexpr int kBitmapWords = 8192;
__global__ __launch_bounds__(kSortThreads) void moe_sort_bitmap_kernel(const int32_t* __restrict__ idx, int T, int top,
                                                                       int E, int32_t* __restrict__ counts,
                                                                       int32_t* __restrict__ offsets,
                                                                       int32_t* __restrict__ order,
                                                                       int32_t* __restrict__ inverse,
                                                                       int32_t* __restrict__ items,
                                                                       int32_t* __restrict__ active) {
  extern __shared__ unsigned long long bm[];  // [E][W]
  __shared__ int32_t start[kMaxExperts];
  __shared__ int32_t scan[33];
  __shared__ uint16_t stok[kMoeMaxPairs];  // token of every sorted pair
  constexpr int kPer = kMoeMaxPairs / kSortThreads;
  const int W = (T + 63) >> 6, P = T * top, tid = threadIdx.x;
  for (int i = tid; i < E * W; i += kSortThreads) bm[i] = 0ull;
  __syncthreads();
  int pe[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) pe[k] = idx[min(tid + k * kSortThreads, P - 1)];  // loads in flight together
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int p = tid + k * kSortThreads;
    if (p < P) {
      const int t = p / top;
      atomicOr(&bm[pe[k] * W + (t >> 6)], 1ull << (t & 63));
    }
  }
  __syncthreads();
  int v = 0;
  if (tid < E)
    for (int w = 0; w < W; ++w) v += __popcll(bm[tid * W + w]);
  int total_pairs;
  const int excl = block_exclusive_scan(v, scan, &total_pairs);
  // work items
  const int shared_tiles = (T + 15) / 16;
  const int tiles = (v + 15) / 16;
  int total_tiles;
  const int first = block_exclusive_scan(tiles, scan, &total_tiles);
  for (int j = 0; j < tiles; ++j) items[1 + shared_tiles + first + j] = ((tid + 1) << 16) | j;
  for (int j = tid; j < shared_tiles; j += kSortThreads) items[1 + j] = j;
  if (tid == 0) items[0] = shared_tiles + total_tiles;
  if (active) {  // routed experts with at least one pair (the weights a grouped GEMM reads)
    int n_active;
    block_exclusive_scan(v > 0 ? 1 : 0, scan, &n_active);
    if (tid == 0) active[0] = n_active;
  }
  if (tid < E) {
    counts[tid] = v;
    offsets[tid] = excl;
    start[tid] = excl;
  }
  if (tid == E - 1) offsets[E] = excl + v;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int p = tid + k * kSortThreads;
    if (p >= P) continue;
    const int t = p / top, e = pe[k];
    const unsigned long long* b = bm + e * W;
    int rank = __popcll(b[t >> 6] & ((1ull << (t & 63)) - 1ull));
    for (int w = 0; w < (t >> 6); ++w) rank += __popcll(b[w]);
    const int dst = start[e] + rank;
    order[dst] = p;
    inverse[p] = dst;
    stok[dst] = uint16_t(t);
  }
  __syncthreads();
  moe_write_records(reinterpret_cast<uint4*>(items + moe_records_offset(T, E, top)), stok, tid, kSortThreads, E, T, P,
                    shared_tiles, shared_tiles + total_tiles, v, excl, first);
}

// PW group pairs per wave; waves = (K/128)/PW split K.
template <int PW, bool SWIGLU>
__global__ __launch_bounds__(1024) void moe_grouped_qmm_kernel(const bf16_t* __restrict__ x, int K,
                                                               const uint32_t* __restrict__ wt,
                                                               const bf16_t* __restrict__ sbt, int n_rows,
                                                               const int32_t* __restrict__ counts,
                                                               const int32_t* __restrict__ offsets,
                                                               const int32_t* __restrict__ order, int E, int top,
                                                               int T, bf16_t* __restrict__ y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const int r16 = lane & 15, qt = lane >> 4;
  const int tile = blockIdx.x, slot = blockIdx.y;
  const int P = T * top, Pk = K >> 7;
  int e, base, cnt;
  if (slot < E) {
    e = slot;
    cnt = counts[e];
    base = offsets[e];
  } else {
    e = E;
    const int chunk = slot - E;
    base = P + chunk * 16;
    cnt = min(16, T - chunk * 16);
  }
  if (cnt <= 0) return;
  const uint32_t* we = wt + size_t(e) * n_rows * (K / 8);
  const bf16_t* sbe = sbt + size_t(e) * n_rows * (K / 64) * 2;
  const int p0 = wave * PW;
  uint4 wq[PW];
  uint2 sbv[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const size_t tp = size_t(tile) * Pk + min(p0 + i, Pk - 1);
    wq[i] = *reinterpret_cast<const uint4*>(we + (tp * 64 + lane) * 4);
    sbv[i] = *reinterpret_cast<const uint2*>(sbe + (tp * 16 + r16) * 4);
  }
  extern __shared__ float red[];  // [waves][16][16]
  for (int m0 = 0; m0 < cnt; m0 += 16) {
    const int ml = min(m0 + r16, cnt - 1);
    int src;
    if (SWIGLU)
      src = slot < E ? order[base + ml] / top : base - P + ml;
    else
      src = base + ml;
    const bf16_t* xrow = x + size_t(src) * K + qt * 16;
    bf16x8 xa[PW][2][2];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int pc = min(p0 + i, Pk - 1);
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int s = 0; s < 2; ++s)
          xa[i][gi][s] = *reinterpret_cast<const bf16x8*>(xrow + (2 * pc + gi) * 64 + s * 8);
    }
    const bool mlive = m0 + r16 < cnt;
    f32x4 total = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      if (p0 + i >= Pk) continue;
      const uint32_t wwords[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
      const uint32_t sbw[2] = {sbv[i].x, sbv[i].y};
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const bf16x8 a0 = mlive ? xa[i][gi][0] : bf16x8{};
        const bf16x8 a1 = mlive ? xa[i][gi][1] : bf16x8{};
        const f32x4 d = q4_group_dot(a0, a1, wwords[2 * gi], wwords[2 * gi + 1], sbw[gi]);
#pragma unroll
        for (int r = 0; r < 4; ++r) total[r] += d[r];
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * 16 + qt * 4 + r) * 16 + r16] = total[r];
    __syncthreads();
    if (SWIGLU) {
      for (int idx = threadIdx.x; idx < 16 * 8; idx += blockDim.x) {
        const int m = idx >> 3, j = idx & 7;
        if (m0 + m < cnt) {
          float g = 0.f, u = 0.f;
          for (int wv = 0; wv < waves; ++wv) {
            g += red[(wv * 16 + m) * 16 + j];
            u += red[(wv * 16 + m) * 16 + 8 + j];
          }
          y[size_t(base + m0 + m) * (n_rows / 2) + tile * 8 + j] = f32_to_bf16(g / (1.f + __expf(-g)) * u);
        }
      }
    } else {
      for (int idx = threadIdx.x; idx < 256; idx += blockDim.x) {
        const int m = idx >> 4, nn = idx & 15;
        if (m0 + m < cnt) {
          float s = 0.f;
          for (int wv = 0; wv < waves; ++wv) s += red[(wv * 16 + m) * 16 + nn];
          y[size_t(base + m0 + m) * n_rows + tile * 16 + nn] = f32_to_bf16(s);
        }
      }
    }
    __syncthreads();
  }
}

// grid (tokens), 256 threads; a thread owns 8 consecutive columns (one 16-byte
// load per expert row), so a token's 11 rows are read in 11 wide loads.
// One workgroup of 256 threads per token; thread tid owns the 8-column
// chunks tid, tid + 256, ... With NORM the updated residual row is also
// RMS-normalised into the next layer's input. The chunk mapping and the order
// of every sum are those of rmsnorm_kernel, so the fused output is bit-identical
// to a separate rmsnorm over the residual.
constexpr int kCombineChunks = 4;  // hidden <= 8192

// NB: routed rows loaded together, the smallest of 4, 8, 10, 16 that holds top
// (every row's load in flight at once)
template <bool NORM, int NB>
__global__ __launch_bounds__(256) void moe_combine_kernel(const bf16_t* __restrict__ down,
                                                          const float* __restrict__ weights,
                                                          const int32_t* __restrict__ inverse,
                                                          const float* __restrict__ logits, int ld_logits, int sg_col,
                                                          int top, int T, int H, float* __restrict__ residual,
                                                          CombineNorm nrm) {
  const int t = blockIdx.x;
  const int P = T * top;
  const float sg = logits[size_t(t) * ld_logits + sg_col];
  const float gate = 1.f / (1.f + __expf(-sg));
  float keep[kCombineChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kCombineChunks; ++j) {
    const int c = threadIdx.x * 8 + j * 256 * 8;
    if (c >= H) break;
    float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // the shared row and the residual first, then the routed rows NB at a
    // time (the last batch re-reads its last row with weight 0), so each batch
    // costs one memory latency rather than one per row
    const uint4 v = *reinterpret_cast<const uint4*>(down + size_t(P + t) * H + c);
    float4* res = reinterpret_cast<float4*>(residual + size_t(t) * H + c);
    float4 r0 = res[0], r1 = res[1];
    for (int e0 = 0; e0 < top; e0 += NB) {
      uint4 rv[NB];
      float rw[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int e = min(e0 + u, top - 1);
        rw[u] = e0 + u < top ? weights[size_t(t) * top + e] : 0.f;
        rv[u] = *reinterpret_cast<const uint4*>(down + size_t(inverse[size_t(t) * top + e]) * H + c);
      }
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const uint32_t vw[4] = {rv[u].x, rv[u].y, rv[u].z, rv[u].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          y[2 * q] += rw[u] * bf16_to_f32(bf16_t(vw[q] & 0xFFFFu));
          y[2 * q + 1] += rw[u] * bf16_to_f32(bf16_t(vw[q] >> 16));
        }
      }
    }
    const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
    r0.x += y[0] + bf16_to_f32(bf16_t(vw[0] & 0xFFFFu)) * gate;
    r0.y += y[1] + bf16_to_f32(bf16_t(vw[0] >> 16)) * gate;
    r0.z += y[2] + bf16_to_f32(bf16_t(vw[1] & 0xFFFFu)) * gate;
    r0.w += y[3] + bf16_to_f32(bf16_t(vw[1] >> 16)) * gate;
    r1.x += y[4] + bf16_to_f32(bf16_t(vw[2] & 0xFFFFu)) * gate;
    r1.y += y[5] + bf16_to_f32(bf16_t(vw[2] >> 16)) * gate;
    r1.z += y[6] + bf16_to_f32(bf16_t(vw[3] & 0xFFFFu)) * gate;
    r1.w += y[7] + bf16_to_f32(bf16_t(vw[3] >> 16)) * gate;
    res[0] = r0;
    res[1] = r1;
    if (NORM) {
      const float r[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        keep[j][q] = r[q];
        ss += r[q] * r[q];
      }
    }
  }
  if (!NORM) return;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) tot += part[i];
  const float inv = 1.f / sqrtf(tot / float(H) + nrm.eps);
#pragma unroll
  for (int j = 0; j < kCombineChunks; ++j) {
    const int c = threadIdx.x * 8 + j * 256 * 8;
    if (c >= H) break;
    const float4 wa = reinterpret_cast<const float4*>(nrm.w + c)[0], wb = reinterpret_cast<const float4*>(nrm.w + c)[1];
    const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
    float y[8];
    uint32_t packed[4];
#pragma unroll
    for (int q = 0; q < 8; ++q) y[q] = keep[j][q] * inv * wv[q];
#pragma unroll
    for (int q = 0; q < 4; ++q) packed[q] = uint32_t(f32_to_bf16(y[2 * q])) | (uint32_t(f32_to_bf16(y[2 * q + 1])) << 16);
    const uint4 pv = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    *reinterpret_cast<uint4*>(nrm.out + size_t(t) * nrm.ld_out + c) = pv;
    if (nrm.gsum) {  // the 8 lanes of a 64-column group are all live (hidden % 64 == 0)
      const float gsv = sum8_lanes(bf16x8_pair_sum(pv));
      if ((threadIdx.x & 7) == 0) nrm.gsum[size_t(t) * (H / 64) + c / 64] = gsv;
    }
    if (nrm.out_f32) {
      float4* o = reinterpret_cast<float4*>(nrm.out_f32 + size_t(t) * H + c);
      o[0] = make_float4(y[0], y[1], y[2], y[3]);
      o[1] = make_float4(y[4], y[5], y[6], y[7]);
    }
  }
}

// Streaming grouped GEMM: a workgroup of WAVES waves covers 16*WAVES weight
// rows of one expert, a wave 16 rows over the whole K (PK = K/128 group pairs,
// 1 KB of codes per pair per wave). The expert's token rows are staged 16 at a
// time into LDS once per workgroup (bf16 [16][K], 16-byte units XOR-swizzled by
// row so the MFMA fragment reads are bank-conflict free) together with their
// per-group sums (ax, so each group needs 2 MFMAs, not 4). Only live rows are
// staged: a fragment row beyond the expert's count only feeds its own output
// row, which is never stored. Each wave then streams its pairs through an
// NPIPE-deep register pipeline, so its weight loads stay in flight while it
// computes, and the register footprint stays small enough for 8 waves per
// SIMD. Slot 0 is the shared expert (all T tokens, re-streamed per 16-token
// tile: the longest list, dispatched first), slot s >= 1 routed expert s - 1.
// The SwiGLU epilogue pairs gate row j with up row 8 + j by a lane exchange.
template <int PK, int WAVES, int NPIPE, bool SWIGLU>
__global__ __launch_bounds__(64 * WAVES) void moe_stream_kernel(const bf16_t* __restrict__ x,
                                                                const uint32_t* __restrict__ wt,
                                                                const bf16_t* __restrict__ sbt, int n_rows,
                                                                const int32_t* __restrict__ counts,
                                                                const int32_t* __restrict__ offsets,
                                                                const int32_t* __restrict__ order, int E, int top,
                                                                int T, bf16_t* __restrict__ y) {
  constexpr int K = PK * 128;
  constexpr int kRowU4 = K / 8;  // 16-byte units per staged row
  constexpr int kThreads = 64 * WAVES;
  constexpr int kIter = (16 * kRowU4 + kThreads - 1) / kThreads;  // staging units per thread
  constexpr int kPipe = NPIPE < PK ? NPIPE : PK;
  extern __shared__ uint4 xs[];                              // [16][kRowU4], unit c of row r at c ^ r
  float* axs = reinterpret_cast<float*>(xs + 16 * kRowU4);  // [K/64][16]: row sums of x per group
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, qt = lane >> 4;
  const int tile = blockIdx.x * WAVES + wave;
  const int P = T * top;
  int e, base, cnt;
  if (blockIdx.y == 0) {
    e = E;
    base = P;
    cnt = T;
  } else {
    e = blockIdx.y - 1;
    cnt = counts[e];
    base = offsets[e];
  }
  if (cnt <= 0) return;  // uniform over the workgroup
  const size_t gt = size_t(e) * (n_rows / 16) + tile;
  const uint4* wp = reinterpret_cast<const uint4*>(wt) + gt * PK * 64 + lane;
  const uint2* sp = reinterpret_cast<const uint2*>(sbt) + gt * PK * 16 + r16;
  // fragments of pair p: k = (2p+gi)*64 + qt*16 + 8s, i.e. unit 16p + (8gi + 2qt + s) of the
  // row; the swizzle only touches the low 4 bits, so p is an immediate offset
  const uint4* xr = xs + r16 * kRowU4;
  const uint4* xf[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xf[j] = xr + (((j >> 1) * 8 + qt * 2 + (j & 1)) ^ r16);
  const Q4Consts magic = q4_consts();
  for (int m0 = 0; m0 < cnt; m0 += 16) {
    const int rows = min(16, cnt - m0);
    if (m0) __syncthreads();  // the previous tile's fragment reads are done
    uint4 wb[kPipe];
    uint2 sb[kPipe];
#pragma unroll
    for (int p = 0; p < kPipe; ++p) {
      wb[p] = wp[p * 64];
      sb[p] = sp[p * 16];
    }
    // stage the tile (rows beyond `rows` re-read the last live row and are not stored):
    // lane r < 16 of every wave looks up the source row of tile row r once, the
    // units then take it by a lane exchange, so all x loads issue back to back
    const int lr = min(lane & 15, rows - 1);
    const int row_src = SWIGLU ? (blockIdx.y ? order[base + m0 + lr] / top : m0 + lr) : base + m0 + lr;
    uint4 v[kIter];
#pragma unroll
    for (int it = 0; it < kIter; ++it) {
      const int i = threadIdx.x + it * kThreads;
      const int rr = min(min(i / kRowU4, 15), rows - 1), c = i % kRowU4;
      const int src = __shfl(row_src, rr, 64);
      v[it] = *reinterpret_cast<const uint4*>(x + size_t(src) * K + c * 8);
    }
#pragma unroll
    for (int it = 0; it < kIter; ++it) {
      const int i = threadIdx.x + it * kThreads;
      const int r = i / kRowU4, c = i % kRowU4;
      const bool live = i < 16 * kRowU4 && r < rows;
      if (live) xs[r * kRowU4 + (c ^ r)] = v[it];
      // group sums: the 8 units of a 64-wide group sit in 8 consecutive lanes
      const uint32_t vw[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) sum += bf16_to_f32(bf16_t(vw[q] & 0xFFFFu)) + bf16_to_f32(bf16_t(vw[q] >> 16));
      sum += __shfl_xor(sum, 1, 64);
      sum += __shfl_xor(sum, 2, 64);
      sum += __shfl_xor(sum, 4, 64);
      if (live && (c & 7) == 0) axs[(c >> 3) * 16 + r] = sum;
    }
    __syncthreads();
    f32x4 total = {0.f, 0.f, 0.f, 0.f};
    // chunks of kPipe pairs: ring slot j holds pair pc + j; after use it is
    // refilled with pair pc + j + kPipe (the outer loop stays rolled to bound
    // the live ranges)
#pragma nounroll
    for (int pc = 0; pc < PK; pc += kPipe) {
#pragma unroll
      for (int j = 0; j < kPipe; ++j) {
        const int p = pc + j;
        uint4 f[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) f[q] = xf[q][16 * p];
        const f32x4 ax0 = *reinterpret_cast<const f32x4*>(axs + (2 * p) * 16 + qt * 4);
        const f32x4 ax1 = *reinterpret_cast<const f32x4*>(axs + (2 * p + 1) * 16 + qt * 4);
        const uint4 w = wb[j];
        const uint2 sbp = sb[j];
        if (p + kPipe < PK) {  // refill the slot just consumed
          wb[j] = wp[(p + kPipe) * 64];
          sb[j] = sp[(p + kPipe) * 16];
        }
        // group g: s*sum x(128+q) + (b - 128 s)*sum x, accumulated by FMAs
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 acc0 = mfma16(__builtin_bit_cast(bf16x8, f[0]), q4_offset_bf16_s(w.x, magic), zero);
        f32x4 acc1 = mfma16(__builtin_bit_cast(bf16x8, f[2]), q4_offset_bf16_s(w.z, magic), zero);
        acc0 = mfma16(__builtin_bit_cast(bf16x8, f[1]), q4_offset_bf16_s(w.y, magic), acc0);
        acc1 = mfma16(__builtin_bit_cast(bf16x8, f[3]), q4_offset_bf16_s(w.w, magic), acc1);
        const float s0 = __builtin_bit_cast(float, sbp.x << 16), s1 = __builtin_bit_cast(float, sbp.y << 16);
        const float b0 = __builtin_fmaf(-128.f, s0, __builtin_bit_cast(float, sbp.x & 0xFFFF0000u));
        const float b1 = __builtin_fmaf(-128.f, s1, __builtin_bit_cast(float, sbp.y & 0xFFFF0000u));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          total[r] = __builtin_fmaf(s0, acc0[r], total[r]);
          total[r] = __builtin_fmaf(b0, ax0[r], total[r]);
          total[r] = __builtin_fmaf(s1, acc1[r], total[r]);
          total[r] = __builtin_fmaf(b1, ax1[r], total[r]);
        }
        // materialise the running sum here: otherwise the adds sink past the
        // loop and every group's MFMA results stay live in accumulators
        asm volatile("" : "+v"(total));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // total[r] = row (token) qt*4 + r of the tile, weight row r16
    if (SWIGLU) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float u = __shfl_xor(total[r], 8, 64);
        const int m = qt * 4 + r;
        if (r16 < 8 && m < rows) {
          const float g = total[r];
          y[size_t(base + m0 + m) * (n_rows / 2) + tile * 8 + r16] = f32_to_bf16(g / (1.f + __expf(-g)) * u);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = qt * 4 + r;
        if (m < rows) y[size_t(base + m0 + m) * n_rows + tile * 16 + r16] = f32_to_bf16(total[r]);
      }
    }
  }
}

template <bool SWIGLU>
bool try_persist(const bf16_t* x, int K, const uint32_t* w, const bf16_t* sb, int n_rows, const int32_t* counts,
                 const int32_t* offsets, const int32_t* order, const int32_t* items, int E, int top, int T, bf16_t* y,
                 hipStream_t stream) {
  if (!items) return false;
  return moe_gemm<SWIGLU>(x, K, w, sb, n_rows, items, E, top, T, y, stream);
}

template <int PK, int WAVES, bool SWIGLU, int kNPipe = 4>
void launch_stream(const bf16_t* x, const uint32_t* w, const bf16_t* sb, int n_rows, const int32_t* counts,
                   const int32_t* offsets, const int32_t* order, int E, int top, int T, bf16_t* y,
                   hipStream_t stream) {
  const dim3 grid(n_rows / (16 * WAVES), E + 1);
  const int lds = 16 * PK * 128 * 2 + PK * 2 * 16 * 4;  // x tile + group sums (> 64 KB at K = 2048)
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_stream_kernel<PK, WAVES, kNPipe, SWIGLU>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  HB_CHECK(attr);
  hipLaunchKernelGGL((moe_stream_kernel<PK, WAVES, kNPipe, SWIGLU>), grid, dim3(64 * WAVES), lds, stream, x, w, sb,
                     n_rows, counts, offsets, order, E, top, T, y);
}

// Workgroup width: 16 waves (256 rows) when the expert has that many rows,
// else 4 (64 rows); other shapes use the K-split kernel below.
template <bool SWIGLU>
bool try_stream(const bf16_t* x, int K, const uint32_t* w, const bf16_t* sb, int n_rows, const int32_t* counts,
                const int32_t* offsets, const int32_t* order, int E, int top, int T, bf16_t* y, hipStream_t stream) {
  if (n_rows % 64) return false;
  const bool wide = n_rows % 256 == 0;
#define HB_STREAM(PK)                                                                                           \
  if (wide)                                                                                                     \
    launch_stream<PK, 16, SWIGLU>(x, w, sb, n_rows, counts, offsets, order, E, top, T, y, stream);           \
  else                                                                                                          \
    launch_stream<PK, 4, SWIGLU>(x, w, sb, n_rows, counts, offsets, order, E, top, T, y, stream);            \
  return true;
  switch (K / 128) {
    case 1: HB_STREAM(1)
    case 2: HB_STREAM(2)
    case 4: HB_STREAM(4)
    case 8: HB_STREAM(8)
    case 16: HB_STREAM(16)
    default: return false;
  }
#undef HB_STREAM
}

template <int PW, bool SWIGLU>
void launch_grouped(const bf16_t* x, int K, const uint32_t* w, const bf16_t* sb, int n_rows, const int32_t* counts,
                    const int32_t* offsets, const int32_t* order, int E, int top, int T, bf16_t* y,
                    hipStream_t stream) {
  const int waves = (K / 128 + PW - 1) / PW;
  const dim3 grid(n_rows / 16, E + (T + 15) / 16);
  hipLaunchKernelGGL((moe_grouped_qmm_kernel<PW, SWIGLU>), grid, dim3(64 * waves), sizeof(float) * waves * 256,
                     stream, x, K, w, sb, n_rows, counts, offsets, order, E, top, T, y);
}

}  // namespace

size_t moe_items_capacity(int tokens, int experts, int top) {
  return size_t(moe_records_offset(tokens, experts, top)) + 16 * size_t(moe_list_capacity(tokens, experts, top));
}

void moe_route(const float* logits, int ld_logits, int tokens, int experts, int top, int32_t* idx, float* weights,
               int32_t* counts, int32_t* offsets, int32_t* order, int32_t* inverse, int32_t* items,
               hipStream_t stream, int32_t* active) {
  require(logits && idx && weights && counts && offsets && order && inverse && items, "moe_route: null pointer");
  require(tokens <= 65535 * 16, "moe_route: too many tokens for the work-item encoding");
  require(experts > 0 && experts <= kMaxExperts, "moe_route: experts must be 1..1024");
  require(top > 0 && top <= experts && top <= 16, "moe_route: top must be 1..16 and <= experts");
  require(tokens > 0 && tokens * top <= kMoeMaxPairs, "moe_route: tokens * top exceeds one routing workgroup");
  require(ld_logits >= experts, "moe_route: logits row stride");
  const dim3 tg((tokens + kTopkWaves - 1) / kTopkWaves), tb(64 * kTopkWaves);
  const int per = (experts + 63) / 64;
  if (per <= 1)
    hipLaunchKernelGGL(moe_topk_kernel<1>, tg, tb, 0, stream, logits, ld_logits, tokens, experts, top, idx, weights);
  else if (per <= 2)
    hipLaunchKernelGGL(moe_topk_kernel<2>, tg, tb, 0, stream, logits, ld_logits, tokens, experts, top, idx, weights);
  else if (per <= 4)
    hipLaunchKernelGGL(moe_topk_kernel<4>, tg, tb, 0, stream, logits, ld_logits, tokens, experts, top, idx, weights);
  else if (per <= 8)
    hipLaunchKernelGGL(moe_topk_kernel<8>, tg, tb, 0, stream, logits, ld_logits, tokens, experts, top, idx, weights);
  else
    hipLaunchKernelGGL(moe_topk_kernel<16>, tg, tb, 0, stream, logits, ld_logits, tokens, experts, top, idx, weights);
  HB_CHECK(hipGetLastError());
  const int words = experts * ((tokens + 63) / 64);
  if (words <= kBitmapWords)
    hipLaunchKernelGGL(moe_sort_bitmap_kernel, dim3(1), dim3(kSortThreads), size_t(words) * 8, stream, idx, tokens, top,
                       experts, counts, offsets, order, inverse, items, active);
  else
    hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(kSortThreads), 0, stream, idx, tokens, top, experts, counts,
                       offsets, order, inverse, items, active);
  HB_CHECK(hipGetLastError());
}

void moe_grouped_qmm(const bf16_t* x, int K, const uint32_t* w_tiled, const bf16_t* sb_tiled, int n_rows,
                     const int32_t* counts, const int32_t* offsets, const int32_t* order, const int32_t* items,
                     int experts, int top, int tokens, int swiglu, bf16_t* y, hipStream_t stream) {
  require(x && w_tiled && sb_tiled && counts && offsets && order && y, "moe_grouped_qmm: null pointer");
  require(n_rows % 16 == 0 && K % 128 == 0 && K / 128 <= 32, "moe_grouped_qmm: needs n_rows % 16 == 0, K % 128 == 0");
  require(tokens > 0 && experts > 0 && top > 0, "moe_grouped_qmm: invalid geometry");
  const bool rows =
      swiglu ? (try_persist<true>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, items, experts, top, tokens,
                                  y, stream) ||
                try_stream<true>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, experts, top, tokens, y,
                                 stream))
             : (try_persist<false>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, items, experts, top,
                                   tokens, y, stream) ||
                try_stream<false>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, experts, top, tokens, y,
                                  stream));
  if (rows) {
    HB_CHECK(hipGetLastError());
    return;
  }
  if (swiglu) {
    if (K / 128 <= 16)
      launch_grouped<1, true>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, experts, top, tokens, y, stream);
    else
      launch_grouped<2, true>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, experts, top, tokens, y, stream);
  } else {
    if (K / 128 <= 16)
      launch_grouped<1, false>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, experts, top, tokens, y,
                               stream);
    else
      launch_grouped<2, false>(x, K, w_tiled, sb_tiled, n_rows, counts, offsets, order, experts, top, tokens, y,
                               stream);
  }
  HB_CHECK(hipGetLastError());
}

namespace {
__global__ __launch_bounds__(256) void moe_count_active_kernel(const int32_t* __restrict__ counts, int E,
                                                               int32_t* __restrict__ out) {
  int c = 0;
  for (int e = threadIdx.x; e < E; e += blockDim.x) c += counts[e] > 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  __shared__ int part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = part[0] + part[1] + part[2] + part[3];
}
}  // namespace

void moe_count_active(const int32_t* counts, int experts, int32_t* out, hipStream_t stream) {
  require(counts && out && experts > 0, "moe_count_active: descriptor");
  hipLaunchKernelGGL(moe_count_active_kernel, dim3(1), dim3(256), 0, stream, counts, experts, out);
  HB_CHECK(hipGetLastError());
}

void moe_combine(const bf16_t* down, const float* weights, const int32_t* inverse, const float* logits, int ld_logits,
                 int sg_col, int top, int tokens, int hidden, float* residual, hipStream_t stream,
                 const CombineNorm* norm) {
  require(down && weights && inverse && logits && residual, "moe_combine: null pointer");
  require(hidden % 8 == 0 && hidden <= 8 * 256 * kCombineChunks, "moe_combine: hidden must be a multiple of 8, <= 8192");
  require(!norm || (norm->w && norm->out && norm->ld_out % 8 == 0), "moe_combine: norm output");
  require(!norm || !norm->gsum || hidden % 64 == 0, "moe_combine: group sums need hidden % 64 == 0");
  require(top > 0 && top <= 16, "moe_combine: top must be 1..16");
  if (tokens <= 0) return;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(tokens), dim3(256), 0, stream, down, weights, inverse, logits, ld_logits, sg_col,
                       top, tokens, hidden, residual, norm ? *norm : CombineNorm{});
  };
  auto pick = [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    if (norm)
      launch(moe_combine_kernel<true, NB>);
    else
      launch(moe_combine_kernel<false, NB>);
  };
  if (top <= 4)
    pick(std::integral_constant<int, 4>{});
  else if (top <= 8)
    pick(std::integral_constant<int, 8>{});
  else if (top <= 10)
    pick(std::integral_constant<int, 10>{});
  else
    pick(std::integral_constant<int, 16>{});
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
