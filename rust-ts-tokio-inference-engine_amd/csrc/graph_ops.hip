// General f32 kernels of the graph API's fused operators (rs_mlx_kernel ops 1-6).
#include "graph_ops.h"

namespace hb {
namespace {

constexpr int kBlock = 256;

__global__ void rope_kernel(const float* __restrict__ x, float* __restrict__ y, int rows, int L, int D, int dims,
                            int offset, float base) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  const int half = dims / 2, tail = D - dims;
  const size_t per_row = size_t(half) + tail;  // rotated pairs, then copied columns
  if (i >= size_t(rows) * L * per_row) return;
  const size_t rl = i / per_row;
  const int c = int(i % per_row);
  const float* xr = x + rl * D;
  float* yr = y + rl * D;
  if (c >= half) {
    const int col = dims + (c - half);
    yr[col] = xr[col];
    return;
  }
  const float pos = float(offset + int(rl % size_t(L)));
  const float freq = powf(base, -2.f * float(c) / float(dims));
  float sn, cs;
  sincosf(pos * freq, &sn, &cs);
  const float a = xr[c], b = xr[c + half];
  yr[c] = a * cs - b * sn;
  yr[c + half] = b * cs + a * sn;
}

// one workgroup per (b, query head, query): scores of every key into the row's
// scratch, then max, sum and the weighted sum of values
__global__ __launch_bounds__(kBlock) void sdpa_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                      const float* __restrict__ v, float* __restrict__ scores,
                                                      float* __restrict__ out, int Hq, int Hkv, int Tq, int Tk, int D,
                                                      int Dv, float scale, int causal) {
  const int tq = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
  const int hk = hq / (Hq / Hkv);
  const float* qr = q + ((size_t(b) * Hq + hq) * Tq + tq) * D;
  const float* kb = k + (size_t(b) * Hkv + hk) * size_t(Tk) * D;
  const float* vb = v + (size_t(b) * Hkv + hk) * size_t(Tk) * Dv;
  float* sr = scores + ((size_t(b) * Hq + hq) * Tq + tq) * size_t(Tk);
  const int last = causal ? tq + Tk - Tq : Tk - 1;  // keys 0..last are visible
  __shared__ float red[kBlock];
  float mx = -INFINITY;
  for (int j = threadIdx.x; j <= last; j += kBlock) {
    float dot = 0.f;
    for (int d = 0; d < D; ++d) dot += qr[d] * kb[size_t(j) * D + d];
    dot *= scale;
    sr[j] = dot;
    mx = fmaxf(mx, dot);
  }
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int st = kBlock / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
    __syncthreads();
  }
  mx = red[0];
  __syncthreads();
  float sum = 0.f;
  for (int j = threadIdx.x; j <= last; j += kBlock) {
    const float p = expf(sr[j] - mx);
    sr[j] = p;
    sum += p;
  }
  red[threadIdx.x] = sum;
  __syncthreads();
  for (int st = kBlock / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
    __syncthreads();
  }
  const float inv = 1.f / red[0];
  float* orow = out + ((size_t(b) * Hq + hq) * Tq + tq) * Dv;
  for (int d = threadIdx.x; d < Dv; d += kBlock) {
    float acc = 0.f;
    for (int j = 0; j <= last; ++j) acc += sr[j] * vb[size_t(j) * Dv + d];
    orow[d] = acc * inv;
  }
}

// one thread per (b, value head, value row dv): that row of the state over Dk
__global__ void gated_delta_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                   const float* __restrict__ v, const float* __restrict__ decay,
                                   const float* __restrict__ beta, const float* __restrict__ state,
                                   float* __restrict__ y, float* __restrict__ S, int B, int T, int Hk, int Hv, int Dk,
                                   int Dv) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= size_t(B) * Hv * Dv) return;
  const int dv = int(i % Dv), hv = int((i / Dv) % Hv), b = int(i / (size_t(Dv) * Hv));
  const int hk = hv / (Hv / Hk);
  float* s = S + ((size_t(b) * Hv + hv) * Dv + dv) * Dk;
  const float* s0 = state + ((size_t(b) * Hv + hv) * Dv + dv) * Dk;
  for (int c = 0; c < Dk; ++c) s[c] = s0[c];
  for (int t = 0; t < T; ++t) {
    const size_t bt = size_t(b) * T + t;
    const float* kt = k + (bt * Hk + hk) * Dk;
    const float* qt = q + (bt * Hk + hk) * Dk;
    const float g = decay[bt * Hv + hv], be = beta[bt * Hv + hv];
    float mem = 0.f;
    for (int c = 0; c < Dk; ++c) {
      const float d = s[c] * g;
      s[c] = d;
      mem += d * kt[c];
    }
    const float delta = (v[(bt * Hv + hv) * Dv + dv] - mem) * be;
    float out = 0.f;
    for (int c = 0; c < Dk; ++c) {
      const float u = s[c] + kt[c] * delta;
      s[c] = u;
      out += u * qt[c];
    }
    y[(bt * Hv + hv) * Dv + dv] = out;
  }
}

// (p, index) order: higher probability first, then the lower index
__device__ inline bool before(float pa, int ia, float pb, int ib) { return pa > pb || (pa == pb && ia < ib); }

// one 64-lane wave per row: softmax, then `top` rounds of the largest
// (p, index) strictly after the previous pick
__global__ __launch_bounds__(64) void route_kernel(const float* __restrict__ logits, uint32_t* __restrict__ idx,
                                                   float* __restrict__ scores, int E, int top) {
  const int r = blockIdx.x, lane = threadIdx.x;
  const float* lr = logits + size_t(r) * E;
  float mx = -INFINITY;
  for (int e = lane; e < E; e += 64) mx = fmaxf(mx, lr[e]);
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = 0.f;
  for (int e = lane; e < E; e += 64) sum += expf(lr[e] - mx);
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  const float inv = 1.f / sum;
  float prev_p = INFINITY, picked = 0.f;
  int prev_i = -1;
  for (int j = 0; j < top; ++j) {
    float bp = -1.f;
    int bi = E;
    for (int e = lane; e < E; e += 64) {
      const float p = expf(lr[e] - mx) * inv;
      if (before(prev_p, prev_i, p, e) && before(p, e, bp, bi)) bp = p, bi = e;
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float op = __shfl_xor(bp, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (before(op, oi, bp, bi)) bp = op, bi = oi;
    }
    if (lane == 0) {
      idx[size_t(r) * top + j] = uint32_t(bi);
      scores[size_t(r) * top + j] = bp;
    }
    picked += bp;
    prev_p = bp;
    prev_i = bi;
  }
  const float norm = 1.f / picked;
  for (int j = lane; j < top; j += 64) scores[size_t(r) * top + j] *= norm;
}

// 64 lanes per (row, slot, output n), striding over K
__global__ __launch_bounds__(64) void gather_qmm_kernel(const float* __restrict__ x, const uint32_t* __restrict__ w,
                                                        const float* __restrict__ scales,
                                                        const float* __restrict__ biases,
                                                        const uint32_t* __restrict__ idx, float* __restrict__ y,
                                                        int top, int N, int K, int group, int bits) {
  const int n = blockIdx.x, rs = blockIdx.y, lane = threadIdx.x;
  const int r = rs / top;
  const size_t e = idx[rs];
  const int words = K * bits / 32, G = K / group;
  const uint32_t* row = w + (e * N + n) * size_t(words);
  const float* sc = scales + (e * N + n) * size_t(G);
  const float* bi = biases + (e * N + n) * size_t(G);
  const float* xr = x + size_t(r) * K;
  const uint32_t mask = (1u << bits) - 1u;
  float acc = 0.f;
  for (int c = lane; c < K; c += 64) {
    const size_t bit = size_t(c) * bits;
    const size_t word = bit >> 5;
    const unsigned shift = unsigned(bit & 31);
    uint64_t val = row[word];
    if (shift + bits > 32) val |= uint64_t(row[word + 1]) << 32;
    const float qv = float(uint32_t(val >> shift) & mask);
    const int g = c / group;
    acc += xr[c] * (sc[g] * qv + bi[g]);
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) y[size_t(rs) * N + n] = acc;
}

__global__ void mix_kernel(const float* __restrict__ ex, const float* __restrict__ sc, float* __restrict__ y, int rows,
                           int top, int N) {
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= size_t(rows) * N) return;
  const int r = int(i / N), n = int(i % N);
  float acc = 0.f;
  for (int j = 0; j < top; ++j) acc += ex[(size_t(r) * top + j) * N + n] * sc[size_t(r) * top + j];
  y[i] = acc;
}

inline unsigned blocks(size_t n) { return unsigned((n + kBlock - 1) / kBlock); }

}  // namespace

void graph_rope(const float* x, float* y, int rows, int L, int D, int dims, int offset, float base, hipStream_t s) {
  const size_t n = size_t(rows) * L * (size_t(dims / 2) + (D - dims));
  if (!n) return;
  hipLaunchKernelGGL(rope_kernel, dim3(blocks(n)), dim3(kBlock), 0, s, x, y, rows, L, D, dims, offset, base);
  HB_CHECK(hipGetLastError());
}

void graph_sdpa(const float* q, const float* k, const float* v, float* scores, float* out, int B, int Hq, int Hkv,
                int Tq, int Tk, int D, int Dv, float scale, bool causal, hipStream_t s) {
  if (!B || !Hq || !Tq) return;
  hipLaunchKernelGGL(sdpa_kernel, dim3(Tq, Hq, B), dim3(kBlock), 0, s, q, k, v, scores, out, Hq, Hkv, Tq, Tk, D, Dv,
                     scale, causal ? 1 : 0);
  HB_CHECK(hipGetLastError());
}

void graph_gated_delta(const float* q, const float* k, const float* v, const float* decay, const float* beta,
                       const float* state, float* y, float* state_out, int B, int T, int Hk, int Hv, int Dk, int Dv,
                       hipStream_t s) {
  const size_t n = size_t(B) * Hv * Dv;
  if (!n) return;
  hipLaunchKernelGGL(gated_delta_kernel, dim3(blocks(n)), dim3(kBlock), 0, s, q, k, v, decay, beta, state, y,
                     state_out, B, T, Hk, Hv, Dk, Dv);
  HB_CHECK(hipGetLastError());
}

void graph_route_topk(const float* logits, uint32_t* idx, float* scores, int rows, int E, int top, hipStream_t s) {
  if (!rows) return;
  hipLaunchKernelGGL(route_kernel, dim3(rows), dim3(64), 0, s, logits, idx, scores, E, top);
  HB_CHECK(hipGetLastError());
}

void graph_gather_qmm(const float* x, const uint32_t* w, const float* scales, const float* biases,
                      const uint32_t* idx, float* y, int rows, int top, int N, int K, int group, int bits,
                      hipStream_t s) {
  if (!rows || !top || !N) return;
  hipLaunchKernelGGL(gather_qmm_kernel, dim3(N, rows * top), dim3(64), 0, s, x, w, scales, biases, idx, y, top, N, K,
                     group, bits);
  HB_CHECK(hipGetLastError());
}

void graph_mix(const float* experts, const float* scores, float* y, int rows, int top, int N, hipStream_t s) {
  const size_t n = size_t(rows) * N;
  if (!n) return;
  hipLaunchKernelGGL(mix_kernel, dim3(blocks(n)), dim3(kBlock), 0, s, experts, scores, y, rows, top, N);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
