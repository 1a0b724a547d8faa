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
#include "q4_device.h"

namespace hb {
namespace {

__device__ inline uint32_t total_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

constexpr int kRouteThreads = 1024;
constexpr int kMaxExperts = 1024;

__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(const float* __restrict__ logits, int ld, int T,
                                                                  int E, int top, int32_t* __restrict__ idx,
                                                                  float* __restrict__ weights,
                                                                  int32_t* __restrict__ counts,
                                                                  int32_t* __restrict__ offsets,
                                                                  int32_t* __restrict__ order,
                                                                  int32_t* __restrict__ inverse) {
  __shared__ int32_t sidx[kMoeMaxPairs];
  __shared__ int32_t rank[kMoeMaxPairs];
  __shared__ int32_t cnt[kMaxExperts];
  __shared__ int32_t scan[kRouteThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  for (int e = tid; e < kMaxExperts; e += blockDim.x) cnt[e] = 0;
  const int per = (E + 63) / 64;
  for (int t = wave; t < T; t += nwaves) {
    const float* row = logits + size_t(t) * ld;
    unsigned long long key[kMaxExperts / 64];
#pragma unroll
    for (int k = 0; k < kMaxExperts / 64; ++k) {
      const int e = lane + 64 * k;
      key[k] = (k < per && e < E) ? (static_cast<unsigned long long>(total_key(row[e])) << 32) | uint32_t(~e) : 0ull;
    }
    float sel[16];
    for (int j = 0; j < top; ++j) {
      unsigned long long best = 0ull;
#pragma unroll
      for (int k = 0; k < kMaxExperts / 64; ++k) best = key[k] > best ? key[k] : best;
      best = wave_max_u64(best);
      const int e = int(~uint32_t(best & 0xFFFFFFFFu));
#pragma unroll
      for (int k = 0; k < kMaxExperts / 64; ++k)
        if (lane + 64 * k == e) key[k] = 0ull;
      if (j < 16) sel[j] = row[e];
      if (lane == 0) {
        idx[size_t(t) * top + j] = e;
        sidx[t * top + j] = e;
      }
    }
    // weights: softmax renormalised over the selection (largest logit first)
    if (lane == 0) {
      const float m = sel[0];
      float tot = 0.f;
      for (int j = 0; j < top; ++j) tot += __expf(sel[j] - m);
      for (int j = 0; j < top; ++j) weights[size_t(t) * top + j] = __expf(sel[j] - m) / tot;
    }
  }
  __syncthreads();
  const int P = T * top;
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
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(inc, off, 64);
    if (lane >= off) inc += u;
  }
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
  }
  __syncthreads();
  const int excl = scan[wave] + inc - v;
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
  }
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

// grid (tokens), 256 threads, each thread hidden/256 columns.
__global__ __launch_bounds__(256) void moe_combine_kernel(const bf16_t* __restrict__ down,
                                                          const float* __restrict__ weights,
                                                          const int32_t* __restrict__ inverse,
                                                          const float* __restrict__ logits, int ld_logits, int sg_col,
                                                          int top, int T, int H, float* __restrict__ residual) {
  const int t = blockIdx.x;
  const int P = T * top;
  const float sg = logits[size_t(t) * ld_logits + sg_col];
  const float gate = 1.f / (1.f + __expf(-sg));
  for (int d = threadIdx.x; d < H; d += blockDim.x) {
    float y = 0.f;
    for (int j = 0; j < top; ++j)
      y += weights[size_t(t) * top + j] * bf16_to_f32(down[size_t(inverse[size_t(t) * top + j]) * H + d]);
    y += bf16_to_f32(down[size_t(P + t) * H + d]) * gate;
    residual[size_t(t) * H + d] += y;
  }
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

void moe_route(const float* logits, int ld_logits, int tokens, int experts, int top, int32_t* idx, float* weights,
               int32_t* counts, int32_t* offsets, int32_t* order, int32_t* inverse, hipStream_t stream) {
  require(logits && idx && weights && counts && offsets && order && inverse, "moe_route: null pointer");
  require(experts > 0 && experts <= kMaxExperts, "moe_route: experts must be 1..1024");
  require(top > 0 && top <= experts && top <= 16, "moe_route: top must be 1..16 and <= experts");
  require(tokens > 0 && tokens * top <= kMoeMaxPairs, "moe_route: tokens * top exceeds one routing workgroup");
  require(ld_logits >= experts, "moe_route: logits row stride");
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(kRouteThreads), 0, stream, logits, ld_logits, tokens, experts,
                     top, idx, weights, counts, offsets, order, inverse);
  HB_CHECK(hipGetLastError());
}

void moe_grouped_qmm(const bf16_t* x, int K, const uint32_t* w_tiled, const bf16_t* sb_tiled, int n_rows,
                     const int32_t* counts, const int32_t* offsets, const int32_t* order, int experts, int top,
                     int tokens, int swiglu, bf16_t* y, hipStream_t stream) {
  require(x && w_tiled && sb_tiled && counts && offsets && order && y, "moe_grouped_qmm: null pointer");
  require(n_rows % 16 == 0 && K % 128 == 0 && K / 128 <= 32, "moe_grouped_qmm: needs n_rows % 16 == 0, K % 128 == 0");
  require(tokens > 0 && experts > 0 && top > 0, "moe_grouped_qmm: invalid geometry");
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
                 int sg_col, int top, int tokens, int hidden, float* residual, hipStream_t stream) {
  require(down && weights && inverse && logits && residual, "moe_combine: null pointer");
  if (tokens <= 0) return;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(tokens), dim3(256), 0, stream, down, weights, inverse, logits,
                     ld_logits, sg_col, top, tokens, hidden, residual);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
