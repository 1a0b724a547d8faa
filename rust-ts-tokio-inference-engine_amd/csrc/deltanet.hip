// Gated DeltaNet for ragged packed rows on gfx950.
//
// gdn_prep: one workgroup per (row, 512-channel chunk) walks the row's tokens:
// causal depthwise conv over the window (committed history + new rows), SiLU,
// per-head q/k normalisation (one wave per head), and (chunk 0) the decay/beta
// gates.
//
// gdn_recurrence: one workgroup of 256 threads per (row, value head); each
// value column i of the state is held by two threads, 64 key rows each (fp32,
// in registers for the whole step), so a token costs three 64-wide dot/axpy
// passes per thread plus one cross-half exchange per dot product. k and q of
// the current token are staged in LDS. The state is read once and written
// once per step, whatever the number of tokens, which is what bounds this
// kernel (2 x 64 KiB of HBM traffic per row and head).
#include "deltanet.h"

namespace hb {
namespace {

constexpr int kPrepThreads = 256;

__device__ inline float silu(float x) { return x / (1.f + __expf(-x)); }

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The prep arithmetic of one channel and one head, shared by gdn_prep_kernel
// and the fused decode kernel so both produce the same bits.
// conv over stream[j .. j + H] = roll[0..H-1], x_j, then SiLU
template <int MAXW>
__device__ inline float conv_silu(const float (&roll)[MAXW], const float (&w)[MAXW], float xv, int H) {
  float acc = 0.f;
#pragma unroll
  for (int tau = 0; tau < MAXW; ++tau) {
    if (tau > H) break;
    acc += (tau < H ? roll[tau] : xv) * w[tau];
  }
  return silu(acc);
}
// the window after x_j: roll[0..H-2] <- roll[1..H-1], roll[H-1] <- x_j
template <int MAXW>
__device__ inline void conv_roll(float (&roll)[MAXW], float xv, int H) {
#pragma unroll
  for (int tau = 0; tau < MAXW - 1; ++tau) roll[tau] = tau + 1 < H ? roll[tau + 1] : xv;
}
// q / (rms * key_dim) or k / (rms * sqrt(key_dim)) for a head held two
// channels per lane of one wave
__device__ inline float head_rms(float a0, float a1, int dk) {
  const float tot = wave_sum(a0 * a0 + a1 * a1);
  return sqrtf(tot / float(dk) + 1e-6f);
}
__device__ inline float gate_decay(float a_raw, float dt_bias, float a_log) {
  const float av = a_raw + dt_bias;
  const float sp = fmaxf(av, 0.f) + log1pf(__expf(-fabsf(av)));
  return __expf(-__expf(a_log) * sp);
}
__device__ inline float gate_beta(float b_raw) { return 1.f / (1.f + __expf(-b_raw)); }

// grid (channels / 512, rows): each wave covers 128 consecutive channels, two
// per lane (c and c + 64), so a q or k head (key_dim 128) is one wave and its
// norm is a wave reduction. Every load a step needs is issued before its first
// use: the history and conv taps up front, the next token's input one token
// ahead, so a row costs a few memory latencies rather than one per value.
// CW: the conv width when known at compile time (loads and taps unrolled to
// it), 0 for any width up to 8.
template <int CW>
__global__ __launch_bounds__(kPrepThreads) void gdn_prep_kernel(
    const bf16_t* __restrict__ qkv, int ld_qkv, const bf16_t* __restrict__ a, const bf16_t* __restrict__ b, int ld_ab,
    const float* __restrict__ conv_w, const float* __restrict__ a_log, const float* __restrict__ dt_bias,
    bf16_t* __restrict__ window, const int32_t* __restrict__ hist_off, const int32_t* __restrict__ src_slot,
    const int32_t* __restrict__ dst_slot, const int32_t* __restrict__ cu_seqlens, GdnGeom g,
    float* __restrict__ q_hat, float* __restrict__ k_hat, float* __restrict__ vout, float* __restrict__ decay,
    float* __restrict__ beta) {
  const int r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kd = g.key_heads * g.key_dim, vd = g.value_heads * g.value_dim, C = 2 * kd + vd;
  constexpr int kMaxW = CW > 0 ? CW : 8;  // conv taps held per channel
  const int conv = CW > 0 ? CW : g.conv;
  const int H = conv - 1;  // history rows
  const int cbase = blockIdx.x * (2 * kPrepThreads) + wave * 128;
  const int t0 = cu_seqlens[r], T = cu_seqlens[r + 1] - t0;
  if (T <= 0) return;
  const int off = hist_off[r];
  const size_t win_rows = size_t(H + g.max_tokens);
  const bf16_t* wsrc = window + size_t(src_slot ? src_slot[r] : r) * win_rows * C;
  bf16_t* win = window + size_t(dst_slot ? dst_slot[r] : r) * win_rows * C;
  int ch[2];
  float roll[2][kMaxW], w[2][kMaxW];  // roll: the last H stream values (history, then new rows)
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    ch[k] = cbase + 64 * k + lane;
#pragma unroll
    for (int j = 0; j < kMaxW - 1; ++j) roll[k][j] = bf16_to_f32(wsrc[size_t(off + min(j, H - 1)) * C + ch[k]]);
#pragma unroll
    for (int tau = 0; tau < kMaxW; ++tau) w[k][tau] = conv_w[size_t(ch[k]) * conv + min(tau, conv - 1)];
  }
  // Rewrite the window as [history | new rows]: each thread owns its channels.
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int j = 0; j < kMaxW - 1; ++j)
      if (j < H) win[size_t(j) * C + ch[k]] = f32_to_bf16(roll[k][j]);
  const bool is_q = cbase < kd, is_k = !is_q && cbase < 2 * kd;  // wave-uniform
  const int dk = g.key_dim;
  bf16_t xn[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) xn[k] = qkv[size_t(t0) * ld_qkv + ch[k]];
  for (int j = 0; j < T; ++j) {
    const int i = t0 + j;
    bf16_t xc[2] = {xn[0], xn[1]};
    const int nxt = t0 + min(j + 1, T - 1);
#pragma unroll
    for (int k = 0; k < 2; ++k) xn[k] = qkv[size_t(nxt) * ld_qkv + ch[k]];
    float act[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      win[size_t(H + j) * C + ch[k]] = xc[k];
      // conv taps tau = 0..conv-1 over stream[j .. j + conv - 1] = roll[0..H-1], x_j
      const float xv = bf16_to_f32(xc[k]);
      act[k] = conv_silu(roll[k], w[k], xv, H);
      conv_roll(roll[k], xv, H);
    }
    if (is_q || is_k) {
      const float rms = head_rms(act[0], act[1], dk);  // the head's 128 channels
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        if (is_q)
          q_hat[size_t(i) * kd + ch[k]] = act[k] / (rms * float(dk));
        else
          k_hat[size_t(i) * kd + (ch[k] - kd)] = act[k] / (rms * sqrtf(float(dk)));
      }
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k) vout[size_t(i) * vd + (ch[k] - 2 * kd)] = act[k];
    }
    if (blockIdx.x == 0 && tid < g.value_heads) {
      decay[size_t(i) * g.value_heads + tid] =
          gate_decay(bf16_to_f32(a[size_t(i) * ld_ab + tid]), dt_bias[tid], a_log[tid]);
      beta[size_t(i) * g.value_heads + tid] = gate_beta(bf16_to_f32(b[size_t(i) * ld_ab + tid]));
    }
  }
}

constexpr int kDim = 128;  // key_dim == value_dim handled by the recurrence kernel

constexpr int kHalf = kDim / 2;        // key rows per thread
constexpr int kRecThreads = 2 * kDim;  // two threads per value column
// LDS operands (k, q) a thread's state loops keep in flight between schedule
// barriers: 8 keeps gdn_recurrence_kernel within 116 VGPRs, spill-free at four
// waves per SIMD (16 spilled 4 VGPRs to scratch)
constexpr int kLdsRun = 8;

// The state is read and written once per step: streaming (non-temporal)
// accesses keep it out of the caches, so its dirty lines are written back
// during this kernel instead of being flushed from the Infinity Cache by the
// next large read (the attention after the MoE paid ~30 us for it).
__device__ inline float state_load(const float* p) { return __builtin_nontemporal_load(p); }
__device__ inline void state_store(float* p, float v) { __builtin_nontemporal_store(v, p); }

// grid (value_heads, rows), 256 threads: lane l of wave w owns value column
// i = 32 w + (l & 31) and key rows c in [64 (l >> 5), 64 (l >> 5) + 64), so a
// (row, head) state tile is held in registers 64 floats per thread and the
// two halves of each dot product meet with one cross-half lane exchange.
// Splitting the keys keeps the register file small enough for several waves
// per SIMD, which is what hides the HBM latency of the state stream.
__global__ __launch_bounds__(kRecThreads, 4) void gdn_recurrence_kernel(
    const float* __restrict__ q_hat, const float* __restrict__ k_hat, const float* __restrict__ v,
    const float* __restrict__ decay, const float* __restrict__ beta, const int32_t* __restrict__ cu_seqlens, GdnGeom g,
    float* __restrict__ state, const int32_t* __restrict__ src_slot, const int32_t* __restrict__ dst_slot,
    GdnLog log_in, const int32_t* __restrict__ log_count, GdnLog log_out, int log_cap, int speculative,
    float* __restrict__ o_out, const bf16_t* __restrict__ z, int ld_z, const float* __restrict__ norm_w,
    bf16_t* __restrict__ y_out) {
  const int h = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i = 32 * w + (lane & 31), c0 = kHalf * (lane >> 5);
  const bool lower = lane < 32;  // the half that stores per-column results
  const int Hv = g.value_heads, kh = h / (Hv / g.key_heads);
  const int t0 = cu_seqlens[r], T = cu_seqlens[r + 1] - t0;
  const int pending = log_count ? log_count[r] : 0;
  if (T <= 0 && pending <= 0) return;
  __shared__ float sk[kDim], sq[kDim], red[kRecThreads / 64];
  const int ss = src_slot ? src_slot[r] : r, ds = dst_slot ? dst_slot[r] : r;
  // state tile stored key-major ([key c][value i]): for each c the 32 lanes
  // of a half read 128 consecutive bytes
  const float* sin_t = state + (size_t(ss) * Hv + h) * kDim * kDim + size_t(c0) * kDim + i;
  float* st_t = state + (size_t(ds) * Hv + h) * kDim * kDim + size_t(c0) * kDim + i;
  float s[kHalf];
#pragma unroll
  for (int c = 0; c < kHalf; ++c) s[c] = state_load(sin_t + c * kDim);
  // 1. replay the committed part of the previous speculative step
  for (int t = 0; t < pending; ++t) {
    const size_t lrow = (size_t(ss) * log_cap + t) * Hv + h;
    __syncthreads();
    if (tid < kDim) sk[tid] = log_in.k[lrow * kDim + tid];
    __syncthreads();
    const float gt = log_in.g[lrow];
    const float dt = log_in.delta[lrow * kDim + i];
    // Same roundings as the token loop below (a separately rounded decay
    // multiply, then one fused multiply-add), so a replayed state is
    // bit-identical to the one the speculative step computed.
#pragma unroll
    for (int c = 0; c < kHalf; ++c) {
      s[c] = __builtin_fmaf(dt, sk[c0 + c], __fmul_rn(s[c], gt));
      if (c % kLdsRun == kLdsRun - 1) __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (speculative) {
#pragma unroll
    for (int c = 0; c < kHalf; ++c) state_store(st_t + c * kDim, s[c]);
  }
  // 2. this step's tokens
  for (int j = 0; j < T; ++j) {
    const int tok = t0 + j;
    __syncthreads();  // previous readers of sk/sq (and of the log rows rewritten below) are done
    if (tid < kDim)
      sk[tid] = k_hat[(size_t(tok) * g.key_heads + kh) * kDim + tid];
    else
      sq[tid - kDim] = q_hat[(size_t(tok) * g.key_heads + kh) * kDim + tid - kDim];
    __syncthreads();
    const float gt = decay[size_t(tok) * Hv + h], bt = beta[size_t(tok) * Hv + h];
    float mem = 0.f;
#pragma unroll
    for (int c = 0; c < kHalf; ++c) {
      s[c] = __fmul_rn(s[c], gt);
      mem = __builtin_fmaf(s[c], sk[c0 + c], mem);
      if (c % kLdsRun == kLdsRun - 1) __builtin_amdgcn_sched_barrier(0);  // bounds the LDS operands in flight
    }
    mem += __shfl_xor(mem, 32, 64);  // lower half + upper half, the same sum in both lanes
    const float delta = (v[(size_t(tok) * Hv + h) * kDim + i] - mem) * bt;
    float o = 0.f;
#pragma unroll
    for (int c = 0; c < kHalf; ++c) {
      s[c] = __builtin_fmaf(delta, sk[c0 + c], s[c]);
      o = __builtin_fmaf(s[c], sq[c0 + c], o);
      if (c % kLdsRun == kLdsRun - 1) __builtin_amdgcn_sched_barrier(0);
    }
    o += __shfl_xor(o, 32, 64);
    if (speculative && j < log_cap) {
      const size_t lrow = (size_t(ds) * log_cap + j) * Hv + h;
      if (tid < kDim) log_out.k[lrow * kDim + tid] = sk[tid];
      if (lower) log_out.delta[lrow * kDim + i] = delta;
      if (tid == 0) log_out.g[lrow] = gt;
    }
    if (o_out && lower) o_out[(size_t(tok) * Hv + h) * kDim + i] = o;
    if (y_out) {
      const float sum = wave_sum(lower ? o * o : 0.f);
      if (lane == 0) red[w] = sum;
      __syncthreads();
      float tot = 0.f;
#pragma unroll
      for (int k = 0; k < kRecThreads / 64; ++k) tot += red[k];
      const float inv = 1.f / sqrtf(tot / float(kDim) + 1e-6f);
      if (lower) {
        const float zz = bf16_to_f32(z[size_t(tok) * ld_z + h * kDim + i]);
        y_out[size_t(tok) * (Hv * kDim) + h * kDim + i] = f32_to_bf16(o * inv * norm_w[i] * silu(zz));
      }
    }
  }
  if (!speculative) {
#pragma unroll
    for (int c = 0; c < kHalf; ++c) state_store(st_t + c * kDim, s[c]);
  }
}

// Decode step with the prep fused in (conv width 4): one workgroup per (row,
// key head) holds the states of the key head's `group` value heads, 256
// threads per head laid out as in gdn_recurrence_kernel. It prepares its
// inputs with gdn_prep_kernel's arithmetic, wave for wave: wave 0 the key
// head's q channels, wave 1 its k channels, wave 2 + v the v channels of value
// head v (two channels per lane, so the q/k norms are the same wave
// reductions), and wave 2 + group the heads' decay and beta. q_hat, k_hat, v
// and the gates go to LDS instead of HBM, so outputs, state, logs and the conv
// window are bit-identical to gdn_prep followed by gdn_recurrence; every
// window channel is read and rewritten by one thread of one workgroup.
//
// The prep runs one token ahead of the update, into the other half of a
// double-buffered LDS slot: token 0's inputs are loaded before the state tile
// and prepared while the state is still in flight, and token j + 1's while
// token j updates the state, so one barrier per token separates them.
template <int GROUP>
__global__ __launch_bounds__(kRecThreads * GROUP) __attribute__((amdgpu_waves_per_eu(4, 8))) void gdn_decode_kernel(
    const bf16_t* __restrict__ qkv, int ld_qkv, const bf16_t* __restrict__ a_in, const bf16_t* __restrict__ b_in,
    int ld_ab, const float* __restrict__ conv_w, const float* __restrict__ a_log, const float* __restrict__ dt_bias,
    bf16_t* __restrict__ window, const int32_t* __restrict__ hist_off, const int32_t* __restrict__ cu_seqlens,
    GdnGeom g, float* __restrict__ state, const int32_t* __restrict__ src_slot, const int32_t* __restrict__ dst_slot,
    GdnLog log_in, const int32_t* __restrict__ log_count, GdnLog log_out, int log_cap, int speculative,
    float* __restrict__ o_out, const bf16_t* __restrict__ z, int ld_z, const float* __restrict__ norm_w,
    bf16_t* __restrict__ y_out) {
  constexpr int kW = 4, H = kW - 1;  // conv width, history rows
  const int kh = blockIdx.x, r = blockIdx.y, lane = threadIdx.x & 63, wg = threadIdx.x >> 6;
  const int hh = threadIdx.x / kRecThreads, tid = threadIdx.x % kRecThreads, w = tid >> 6;  // head within the group
  const int h = kh * GROUP + hh;
  const int i = 32 * w + (lane & 31), c0 = kHalf * (lane >> 5);
  const bool lower = lane < 32;
  const int Hv = g.value_heads;
  const int kd = g.key_heads * kDim, C = 2 * kd + Hv * kDim;
  const int t0 = cu_seqlens[r], T = cu_seqlens[r + 1] - t0;
  const int pending = log_count ? log_count[r] : 0;
  if (T <= 0 && pending <= 0) return;
  // prepared inputs, double-buffered by token parity
  // sio[parity]: q_hat, k_hat, then each value head's v
  __shared__ float sio[2][2 + GROUP][kDim], sgate[2][GROUP][2];
  __shared__ float slk[GROUP][kDim], red[GROUP][kRecThreads / 64];  // a logged k; the norm's partial sums
  // conv taps and rolling history of the conv waves' channels, per lane (kept
  // out of registers: the state tile needs them)
  __shared__ float4 staps[2 + GROUP][2][64], shist[2 + GROUP][2][64];
  const int ss = src_slot ? src_slot[r] : r, ds = dst_slot ? dst_slot[r] : r;

  // prep roles (wave-uniform): wave 0 q, 1 k, 2 .. 1 + GROUP the value heads' v, 2 + GROUP the gates
  const bool conv_wave = wg < 2 + GROUP, gate_wave = wg == 2 + GROUP;
  const int cb = wg == 0 ? kh * kDim : wg == 1 ? kd + kh * kDim : 2 * kd + (kh * GROUP + wg - 2) * kDim;
  const size_t win_rows = size_t(H + g.max_tokens);
  const bf16_t* wsrc = window + size_t(ss) * win_rows * C;
  bf16_t* win = window + size_t(ds) * win_rows * C;
  // the next token's raw inputs: a conv lane's two channels, or a gate lane's
  // a and b (one pair of registers for both roles: registers held across the
  // state loops are what the kernel runs short of)
  bf16_t xn[2] = {0, 0};
  __shared__ float sgp[GROUP][2];  // the gate lanes' dt_bias and A_log
  // where a lane's two next inputs come from: token t's are at in[k][t * ld]
  const bool gate_lane = gate_wave && lane < GROUP;
  const bf16_t* in[2] = {gate_lane ? a_in + kh * GROUP + lane : qkv + cb + lane,
                         gate_lane ? b_in + kh * GROUP + lane : qkv + cb + 64 + lane};
  const size_t ld_in = gate_lane ? ld_ab : ld_qkv;
  // token 0's inputs, issued ahead of the state tile
  if (T > 0) {
    if (conv_wave) {
      const int off = hist_off[r];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int ch = cb + 64 * k + lane;
        float hist[H];
#pragma unroll
        for (int j = 0; j < H; ++j) hist[j] = bf16_to_f32(wsrc[size_t(off + j) * C + ch]);
        staps[wg][k][lane] = *reinterpret_cast<const float4*>(conv_w + size_t(ch) * kW);
        shist[wg][k][lane] = make_float4(hist[0], hist[1], hist[2], 0.f);
        xn[k] = in[k][size_t(t0) * ld_in];
        // rewrite the window as [history | new rows]: each lane owns its channels
#pragma unroll
        for (int j = 0; j < H; ++j) win[size_t(j) * C + ch] = f32_to_bf16(hist[j]);
      }
    } else if (gate_lane) {
      xn[0] = in[0][size_t(t0) * ld_in];
      xn[1] = in[1][size_t(t0) * ld_in];
      sgp[lane][0] = dt_bias[kh * GROUP + lane];
      sgp[lane][1] = a_log[kh * GROUP + lane];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const float* sin_t = state + (size_t(ss) * Hv + h) * kDim * kDim + size_t(c0) * kDim + i;
  float* st_t = state + (size_t(ds) * Hv + h) * kDim * kDim + size_t(c0) * kDim + i;
  float s[kHalf];
#pragma unroll
  for (int c = 0; c < kHalf; ++c) s[c] = state_load(sin_t + c * kDim);
  __builtin_amdgcn_sched_barrier(0);

  // prepares token j into buffer j & 1 (the caller has made that buffer free)
  // and loads token j + 1's inputs
  auto prep = [&](int j) {
    const int bu = j & 1, nxt = t0 + min(j + 1, T - 1);
    if (conv_wave) {
      const bf16_t xc[2] = {xn[0], xn[1]};
#pragma unroll
      for (int k = 0; k < 2; ++k) xn[k] = in[k][size_t(nxt) * ld_in];
      float act[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        win[size_t(H + j) * C + cb + 64 * k + lane] = xc[k];
        const float xv = bf16_to_f32(xc[k]);
        const float4 t4 = staps[wg][k][lane], h4 = shist[wg][k][lane];
        const float wt[kW] = {t4.x, t4.y, t4.z, t4.w};
        float roll[kW] = {h4.x, h4.y, h4.z, 0.f};
        act[k] = conv_silu(roll, wt, xv, H);
        conv_roll(roll, xv, H);
        shist[wg][k][lane] = make_float4(roll[0], roll[1], roll[2], 0.f);
      }
      if (wg < 2) {
        const float rms = head_rms(act[0], act[1], kDim);
        const float den = wg == 0 ? rms * float(kDim) : rms * sqrtf(float(kDim));
#pragma unroll
        for (int k = 0; k < 2; ++k) act[k] = act[k] / den;
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) sio[bu][wg][64 * k + lane] = act[k];
    } else if (gate_lane) {
      sgate[bu][lane][0] = gate_decay(bf16_to_f32(xn[0]), sgp[lane][0], sgp[lane][1]);
      sgate[bu][lane][1] = gate_beta(bf16_to_f32(xn[1]));
      xn[0] = in[0][size_t(nxt) * ld_in];
      xn[1] = in[1][size_t(nxt) * ld_in];
    }
  };
  if (T > 0) prep(0);  // overlaps the state tile's loads

  // 1. replay the committed part of the previous speculative step
  for (int t = 0; t < pending; ++t) {
    const size_t lrow = (size_t(ss) * log_cap + t) * Hv + h;
    __syncthreads();
    if (tid < kDim) slk[hh][tid] = log_in.k[lrow * kDim + tid];  // this head's logged k
    __syncthreads();
    const float gt = log_in.g[lrow];
    const float dt = log_in.delta[lrow * kDim + i];
#pragma unroll
    for (int c = 0; c < kHalf; ++c) {
      s[c] = __builtin_fmaf(dt, slk[hh][c0 + c], __fmul_rn(s[c], gt));
      if (c % 4 == 3) __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (speculative) {
#pragma unroll
    for (int c = 0; c < kHalf; ++c) state_store(st_t + c * kDim, s[c]);
  }
  // 2. this step's tokens: token j + 1 is prepared while token j updates
  for (int j = 0; j < T; ++j) {
    const int tok = t0 + j, bu = j & 1;
    // token j's buffer is complete; the readers of the other one (token j - 1) are done
    __syncthreads();
    if (j + 1 < T) prep(j + 1);
    const float* q_s = sio[bu][0];
    const float* k_s = sio[bu][1];
    const float gt = sgate[bu][hh][0], bt = sgate[bu][hh][1];
    float mem = 0.f;
#pragma unroll
    for (int c = 0; c < kHalf; ++c) {
      s[c] = __fmul_rn(s[c], gt);
      mem = __builtin_fmaf(s[c], k_s[c0 + c], mem);
      if (c % 4 == 3) __builtin_amdgcn_sched_barrier(0);
    }
    mem += __shfl_xor(mem, 32, 64);
    const float delta = (sio[bu][2 + hh][i] - mem) * bt;
    float o = 0.f;
#pragma unroll
    for (int c = 0; c < kHalf; ++c) {
      s[c] = __builtin_fmaf(delta, k_s[c0 + c], s[c]);
      o = __builtin_fmaf(s[c], q_s[c0 + c], o);
      if (c % 4 == 3) __builtin_amdgcn_sched_barrier(0);
    }
    o += __shfl_xor(o, 32, 64);
    if (speculative && j < log_cap) {
      const size_t lrow = (size_t(ds) * log_cap + j) * Hv + h;
      if (tid < kDim) log_out.k[lrow * kDim + tid] = k_s[tid];
      if (lower) log_out.delta[lrow * kDim + i] = delta;
      if (tid == 0) log_out.g[lrow] = gt;
    }
    if (o_out && lower) o_out[(size_t(tok) * Hv + h) * kDim + i] = o;
    if (y_out) {
      const float sum = wave_sum(lower ? o * o : 0.f);
      // red is rewritten only after the next token's first barrier
      if (lane == 0) red[hh][w] = sum;
      __syncthreads();
      float tot = 0.f;
#pragma unroll
      for (int k = 0; k < kRecThreads / 64; ++k) tot += red[hh][k];
      const float inv = 1.f / sqrtf(tot / float(kDim) + 1e-6f);
      if (lower) {
        const float zz = bf16_to_f32(z[size_t(tok) * ld_z + h * kDim + i]);
        y_out[size_t(tok) * (Hv * kDim) + h * kDim + i] = f32_to_bf16(o * inv * norm_w[i] * silu(zz));
      }
    }
  }
  if (!speculative) {
#pragma unroll
    for (int c = 0; c < kHalf; ++c) state_store(st_t + c * kDim, s[c]);
  }
}

}  // namespace

void gdn_prep(const bf16_t* qkv, int ld_qkv, const bf16_t* a, const bf16_t* b, int ld_ab, const float* conv_w,
              const float* a_log, const float* dt_bias, bf16_t* window, const int32_t* hist_off,
              const GdnSlots& slots, const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* q_hat,
              float* k_hat, float* v, float* decay, float* beta, hipStream_t stream) {
  const int C = 2 * g.key_heads * g.key_dim + g.value_heads * g.value_dim;
  require(C % (2 * kPrepThreads) == 0 && g.key_dim == 128, "gdn_prep: channel geometry (key_dim 128, C % 512)");
  require(g.conv >= 2 && g.conv <= 8, "gdn_prep: conv width must be 2..8");
  require(g.value_heads <= kPrepThreads, "gdn_prep: too many value heads");
  if (rows <= 0) return;
  const auto kernel = g.conv == 4 ? gdn_prep_kernel<4> : gdn_prep_kernel<0>;
  hipLaunchKernelGGL(kernel, dim3(C / (2 * kPrepThreads), rows), dim3(kPrepThreads), 0, stream, qkv, ld_qkv, a, b,
                     ld_ab, conv_w, a_log, dt_bias, window, hist_off, slots.src, slots.dst, cu_seqlens, g, q_hat,
                     k_hat, v, decay, beta);
  HB_CHECK(hipGetLastError());
}

void gdn_recurrence(const float* q_hat, const float* k_hat, const float* v, const float* decay, const float* beta,
                    const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* state, const GdnSlots& slots,
                    const GdnLog& log_in, const int32_t* log_count, const GdnLog& log_out, int log_cap,
                    int speculative, float* o_out, const bf16_t* z, int ld_z, const float* norm_w, bf16_t* y_out,
                    hipStream_t stream) {
  require(g.key_dim == kDim && g.value_dim == kDim, "gdn_recurrence: head dims must be 128");
  require(g.value_heads % g.key_heads == 0, "gdn_recurrence: value_heads % key_heads");
  require(!y_out || (z && norm_w), "gdn_recurrence: gated norm needs z and norm weight");
  require(!speculative || (log_out.k && log_out.delta && log_out.g && log_cap > 0), "gdn_recurrence: log buffers");
  require(!log_count || (log_in.k && log_in.delta && log_in.g), "gdn_recurrence: pending log buffers");
  if (rows <= 0) return;
  launch_timed(gdn_recurrence_kernel, dim3(g.value_heads, rows), dim3(kRecThreads), 0, stream, q_hat, k_hat, v, decay,
               beta, cu_seqlens, g, state, slots.src, slots.dst, log_in, log_count, log_out, log_cap, speculative,
               o_out, z, ld_z, norm_w, y_out);
  HB_CHECK(hipGetLastError());
}

bool gdn_decode(const bf16_t* qkv, int ld_qkv, const bf16_t* a, const bf16_t* b, int ld_ab, const float* conv_w,
                const float* a_log, const float* dt_bias, bf16_t* window, const int32_t* hist_off,
                const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* state, const GdnSlots& slots,
                const GdnLog& log_in, const int32_t* log_count, const GdnLog& log_out, int log_cap, int speculative,
                float* o_out, const bf16_t* z, int ld_z, const float* norm_w, bf16_t* y_out, hipStream_t stream) {
  if (g.conv != 4 || g.key_dim != kDim || g.value_dim != kDim || g.value_heads != 2 * g.key_heads) return false;
  require(!y_out || (z && norm_w), "gdn_decode: gated norm needs z and norm weight");
  require(!speculative || (log_out.k && log_out.delta && log_out.g && log_cap > 0), "gdn_decode: log buffers");
  require(!log_count || (log_in.k && log_in.delta && log_in.g), "gdn_decode: pending log buffers");
  if (rows <= 0) return true;
  launch_timed(gdn_decode_kernel<2>, dim3(g.key_heads, rows), dim3(2 * kRecThreads), 0, stream, qkv, ld_qkv, a, b,
               ld_ab,
               conv_w, a_log, dt_bias, window, hist_off, cu_seqlens, g, state, slots.src, slots.dst, log_in,
               log_count, log_out, log_cap, speculative, o_out, z, ld_z, norm_w, y_out);
  HB_CHECK(hipGetLastError());
  return true;
}

}  // namespace hb
