// Chunked gated delta rule for prefill steps on MFMA (see deltanet.h).
//
// Per (row, value head) and chunk of up to 64 tokens, with L_t the chunk's
// prefix sum of log g (Gamma_t = exp L_t) and D_t = exp(L_last - L_t):
//   R = diag(beta) (V - diag(Gamma) K S^T)              [t][dv]
//   A = strict_lower(beta_t exp(L_t - L_i) k_t . k_i)   [t][i]
//   U = (I + A)^-1 R                                    (corrected values)
//   O = diag(Gamma) Q S^T + P U,  P = lower(exp(L_t - L_i) q_t . k_i)
//   S <- Gamma_last S + (diag(D) U)^T K                 (state, [dv][dk])
// which is the token-serial rule S <- g S; S += beta (v - S k) k^T; o = S q
// regrouped. The triangular system is solved in 16-token blocks: U_b =
// (I + A_bb)^-1 (R_b - sum_{j<b} A_bj U_j), the diagonal-block inverses by
// forward substitution.
//
// Every product runs on the bf16 MFMA with FP32 operands split into bf16
// high and low parts (a b = a_hi b_hi + a_hi b_lo + a_lo b_hi, about 16
// mantissa bits per operand), which keeps the state at FP32-class accuracy
// while the work per chunk is matrix products instead of 64 dependent token
// steps.
//
// One workgroup of 8 waves owns one (row, head), two waves per SIMD. Wave w
// keeps the state rows of keys [16 w, 16 w + 16) in registers across the
// row's chunks; in the token-parallel phases it works on token block w & 3
// and value half w >> 2; in the block substitution it owns value columns
// [16 w, 16 w + 16) for all 64 tokens, with the corrected values held in
// registers (the 16x16x16 MFMA's output layout is its B-operand layout, so
// U_j feeds the next block's product directly).
#include "deltanet.h"
#include "q4_device.h"

namespace hb {
namespace {

constexpr int kD = 128;  // key_dim == value_dim
constexpr int kC = 64;   // tokens per chunk
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
static_assert(kThreads == 512, "K staging: one 4-token x 4-key block per thread");

// LDS (uint4 units). X: S^T hi/lo as bf16 [dv][k] (2 x 2048), then the
// values R as f32 [dv][t] (2048), then U and D U hi/lo as bf16 [dv][t] (4 x
// 1024). Y: K hi/lo as bf16 [t][k] (2 x 1024), later A (f32 [t][i]) and P
// (f32 [t][i], swizzled) (1024 each). Z: K^T hi/lo as bf16 [k][t] (2 x 1024).
// Then the inverted diagonal blocks (I + A_bb)^-1 as f32 [t][16], the chunk's
// log-decay prefix L, exp(L), exp(L_last - L), betas and the two value
// halves' partial sums of squares of o.
constexpr int kX = 0, kY = 4096, kZ = kY + 2048, kSmall = kZ + 2048;
constexpr int kUhi = kX, kUlo = kX + 1024, kDUhi = kX + 2048, kDUlo = kX + 3072;
constexpr int kSmallFloats = 1024 + 4 * 64 + 128;
constexpr size_t kLds = size_t(kSmall) * 16 + kSmallFloats * 4;

// row r, 16-byte chunk c of a matrix with nc chunks per row, XOR-swizzled by
// row so that 16 lanes reading the same chunk of 16 rows hit distinct banks
__device__ inline int sw(int r, int c, int nc) { return r * nc + (c ^ (r & (nc - 1))); }
// f32 element (r, col) of a 64-column matrix stored in swizzled 4-float chunks
__device__ inline int swf(int r, int col) { return sw(r, col >> 2, 16) * 4 + (col & 3); }

typedef short s16x4 __attribute__((ext_vector_type(4)));

struct Split8 {
  bf16x8 hi, lo;
};
struct Split4 {
  s16x4 hi, lo;
};

// two floats to a bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32)
__device__ inline uint32_t pack_rne(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
}

// a float pair split into bf16 high parts and the bf16 residuals
__device__ inline void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack_rne(a, b);
  lo = pack_rne(a - __builtin_bit_cast(float, hi << 16), b - __builtin_bit_cast(float, hi & 0xFFFF0000u));
}

__device__ inline Split8 split8(const float (&f)[8]) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) split2(f[2 * q], f[2 * q + 1], h[q], l[q]);
  const u32x4 hv = {h[0], h[1], h[2], h[3]}, lv = {l[0], l[1], l[2], l[3]};
  return {__builtin_bit_cast(bf16x8, hv), __builtin_bit_cast(bf16x8, lv)};
}

// Vectors are converted whole: __builtin_bit_cast of one element of a vector
// value (v[i]) miscompiles to element 0 with this compiler.
__device__ inline Split4 split4(f32x4 v) {
  float f[4];
  __builtin_memcpy(f, &v, 16);
  uint32_t h[2], l[2];
  split2(f[0], f[1], h[0], l[0]);
  split2(f[2], f[3], h[1], l[1]);
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  const u2 hv = {h[0], h[1]}, lv = {l[0], l[1]};
  return {__builtin_bit_cast(s16x4, hv), __builtin_bit_cast(s16x4, lv)};
}

__device__ inline f32x4 mfma3(const Split8& a, const Split8& b, f32x4 acc) {
  acc = mfma16(a.lo, b.hi, acc);
  acc = mfma16(a.hi, b.lo, acc);
  return mfma16(a.hi, b.hi, acc);
}

// the same on the 16x16x16 MFMA (4 k per lane: A row l % 16, B column l % 16,
// k = 4 (l / 16) + e, which is also where that MFMA leaves output row k)
__device__ inline f32x4 mfma3k16(const Split4& a, const Split4& b, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.lo, b.hi, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.hi, b.lo, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.hi, b.hi, acc, 0, 0, 0);
}

// 8 consecutive floats from two swizzled 4-float chunks (row r, chunks c, c+1)
__device__ inline void read8f(const uint4* m, int r, int c, float (&f)[8]) {
  const f32x4 a = __builtin_bit_cast(f32x4, m[sw(r, c, 16)]), b = __builtin_bit_cast(f32x4, m[sw(r, c + 1, 16)]);
  __builtin_memcpy(f, &a, 16);
  __builtin_memcpy(f + 4, &b, 16);
}

template <int CTRL, int ROWS = 0xF>
__device__ inline float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}
// sum over the 16 lanes of a DPP row (rotations by 8, 4, 2, 1)
__device__ inline float row_sum(float v) {
  v += dpp<0x128>(v);
  v += dpp<0x124>(v);
  v += dpp<0x122>(v);
  return v + dpp<0x121>(v);
}
// inclusive prefix sum over the 64 lanes: shifts within rows, then the
// row ends broadcast to the following rows (lanes past a row's start read 0)
__device__ inline float wave_prefix_sum(float v) {
  v += dpp<0x111>(v);
  v += dpp<0x112>(v);
  v += dpp<0x114>(v);
  v += dpp<0x118>(v);
  v += dpp<0x142, 0xA>(v);
  return v + dpp<0x143, 0xC>(v);
}

// sum over the 4 lanes of a quad (DPP quad permutations)
__device__ inline float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}

// orders this wave's LDS stores before its later loads of other lanes' data
__device__ inline void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local"); }

// base[elem] with a 32-bit byte offset from a workgroup-uniform base, so the
// address is one SGPR pair plus one VGPR instead of 64-bit arithmetic per load
template <class T>
__device__ inline T& at(T* base, uint32_t elem) {
  return *reinterpret_cast<T*>(reinterpret_cast<char*>(base) + elem * uint32_t(sizeof(T)));
}
template <class T>
__device__ inline const T& at(const T* base, uint32_t elem) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + elem * uint32_t(sizeof(T)));
}

__device__ inline float silu_f(float x) { return __fdividef(x, 1.f + __expf(-x)); }

__global__ __launch_bounds__(kThreads, 1) void gdn_chunk_kernel(
    const float* __restrict__ q_hat, const float* __restrict__ k_hat, const float* __restrict__ v,
    const float* __restrict__ decay, const float* __restrict__ beta, const int32_t* __restrict__ cu_seqlens, GdnGeom g,
    float* __restrict__ state, const int32_t* __restrict__ src_slot, const int32_t* __restrict__ dst_slot,
    float* __restrict__ o_out, const bf16_t* __restrict__ z, int ld_z, const float* __restrict__ norm_w,
    bf16_t* __restrict__ y_out) {
  extern __shared__ uint4 lds[];
  float* const fD = reinterpret_cast<float*>(lds + kSmall);  // (I + A_bb)^-1 [t][16]
  float* const sL = fD + 1024;                                // log-decay prefix of the chunk
  float* const sG = sL + 64;                                  // exp(L_t)
  float* const sE = sG + 64;                                  // exp(L_last - L_t)
  float* const sB = sE + 64;                                  // betas
  float* const sN = sB + 64;                                  // [value half][t] partial sums of o^2
  float* const fA = reinterpret_cast<float*>(lds + kY);       // A [t][i]
  float* const fP = fA + 1024 * 4;                            // P [t][i] (swizzled chunks)
  const int h = blockIdx.x, r = blockIdx.y, lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tb = w & 3, hf = w >> 2;  // token block and value half of the token-parallel phases
  const int Hv = g.value_heads, Hk = g.key_heads, kh = h / (Hv / Hk);
  const int t0 = cu_seqlens[r], T = cu_seqlens[r + 1] - t0;
  if (T <= 0) return;  // uniform over the workgroup
  const int ss = src_slot ? src_slot[r] : r, ds = dst_slot ? dst_slot[r] : r;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const uint32_t ldk = Hk * kD, ldv = Hv * kD;

  // this wave's state rows: S[ct][e] = Skm[k][dv] (key-major), k = 16 w + 4 qt + e, dv = 16 ct + r16
  f32x4 S[8];
  {
    const int r16 = lane & 15, qt = lane >> 4;
    const float* src = state + (size_t(ss) * Hv + h) * kD * kD;
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[ct][e] = at(src, (16 * w + 4 * qt + e) * kD + 16 * ct + r16);
  }

  // K of a chunk, thread (token group tg, key group kg) holding K[4 tg + tt]
  // [4 kg .. 4 kg + 3], which feeds both the [t][k] and the [k][t] staging;
  // and (wave 0) the chunk's decays and betas. Loaded one chunk ahead, while
  // the previous chunk computes.
  f32x4 kpre[4];
  float gpre = 1.f, bpre = 0.f;
  auto fetch = [&](int cn, int lnx) {
    const int Tn = min(kC, T - cn);
    const size_t tokn = size_t(t0) + cn;
    const f32x4* const kbn = reinterpret_cast<const f32x4*>(k_hat + (tokn * Hk + kh) * kD);
    const int idx = 64 * w + lnx, kg = idx & 31, tg = idx >> 5;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) kpre[tt] = at(kbn, (min(4 * tg + tt, Tn - 1) * ldk) / 4 + kg);  // clamped
    if (w == 0) {
      const int tl = min(lnx, Tn - 1);
      gpre = at(decay + tokn * Hv + h, tl * Hv);
      bpre = at(beta + tokn * Hv + h, tl * Hv);
    }
  };
  fetch(0, lane);

  float nw[4];  // norm weights of this wave's output columns 16 (4 hf + c4) + r16
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) nw[c4] = y_out ? norm_w[16 * (4 * hf + c4) + (lane & 15)] : 0.f;

  for (int c0 = 0; c0 < T; c0 += kC) {
    const int Tc = min(kC, T - c0);
    // lane indices re-derived per chunk: keeps the compiler from hoisting
    // (and spilling) every lane-dependent address of the body out of the loop
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r16 = ln & 15, qt = ln >> 4, tid = 64 * w + ln;
    const size_t tok0 = size_t(t0) + c0;
    // chunk bases (uniform); token t of the chunk at t * ldk (q, k), t * ldv (v)
    const float* const qb = q_hat + (tok0 * Hk + kh) * kD;
    const float* const vb = v + (tok0 * Hv + h) * kD;
    const int tw = 16 * tb + r16;  // A-operand token row of this wave

    // 0. this wave's Q rows (A operands, keys 32 s + 8 qt .. + 7), issued
    // first; V (step 1) and z (step 3) follow in later phases, so that the
    // previous chunk's output stores and these loads stay within the
    // memory counter's range
    float qraw[4][8], vraw[4][4], zraw[4][4];
    const int tr0 = 16 * tb + 4 * qt;  // output rows tr0 + j of this wave
    {
      const uint32_t trow = min(tw, Tc - 1) * ldk;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f32x4 a = at(reinterpret_cast<const f32x4*>(qb), (trow + 32 * s + 8 * qt) / 4);
        const f32x4 b = at(reinterpret_cast<const f32x4*>(qb), (trow + 32 * s + 8 * qt) / 4 + 1);
        __builtin_memcpy(qraw[s], &a, 16);
        __builtin_memcpy(qraw[s] + 4, &b, 16);
      }
    }
    // log-decay prefix and betas (wave 0); tokens past Tc: g = 1, beta = 0
    if (w == 0) {
      const bool live = ln < Tc;
      const float gt = live ? gpre : 1.f, bl = bpre;
      const float lg = wave_prefix_sum(logf(fmaxf(gt, 1e-30f)));
      const float last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lg), 63));
      sL[ln] = lg;
      sG[ln] = expf(lg);
      sE[ln] = expf(last - lg);
      sB[ln] = live ? bl : 0.f;
    }
    // staging: S^T hi/lo [dv][k] from the state registers
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      const int dv = 16 * ct + r16, c = 2 * w + (qt >> 1);  // 8-key chunk of keys 16 w + 4 qt .. + 3
      uint2 hi, lo;
      split2(S[ct][0], S[ct][1], hi.x, lo.x);
      split2(S[ct][2], S[ct][3], hi.y, lo.y);
      uint2* xs = reinterpret_cast<uint2*>(lds + kX);
      xs[sw(dv, c, 16) * 2 + (qt & 1)] = hi;
      xs[(2048 + sw(dv, c, 16)) * 2 + (qt & 1)] = lo;
    }
    // K hi/lo [t][k] and K^T hi/lo [k][t] (rows past Tc are zeros)
    {
      const int kg = tid & 31, tg = tid >> 5;
      float kv[4][4];  // [token][key] of this thread's block, hi and lo parts below
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        float f[4];
        __builtin_memcpy(f, &kpre[tt], 16);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) kv[tt][kk] = 4 * tg + tt < Tc ? f[kk] : 0.f;
      }
      uint2* const l2 = reinterpret_cast<uint2*>(lds);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {  // [t][k]: keys 4 kg .. + 3 = half (kg & 1) of chunk kg >> 1
        uint2 hi, lo;
        split2(kv[tt][0], kv[tt][1], hi.x, lo.x);
        split2(kv[tt][2], kv[tt][3], hi.y, lo.y);
        const int o = sw(4 * tg + tt, kg >> 1, 16) * 2 + (kg & 1);
        l2[kY * 2 + o] = hi;
        l2[(kY + 1024) * 2 + o] = lo;
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {  // [k][t]: tokens 4 tg .. + 3 = half (tg & 1) of chunk tg >> 1
        uint2 hi, lo;
        split2(kv[0][kk], kv[1][kk], hi.x, lo.x);
        split2(kv[2][kk], kv[3][kk], hi.y, lo.y);
        const int o = sw(4 * kg + kk, tg >> 1, 8) * 2 + (tg & 1);
        l2[kZ * 2 + o] = hi;
        l2[(kZ + 1024) * 2 + o] = lo;
      }
    }
    if (c0 + kC < T) fetch(c0 + kC, ln);  // uniform
    lds_barrier();

#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int j = 0; j < 4; ++j) vraw[c4][j] = at(vb, min(tr0 + j, Tc - 1) * ldv + 16 * (4 * hf + c4) + r16);

    // 1. token block tb x value half hf: W = K S^T and Q S^T (4 value tiles);
    // value half 0 also K K^T, half 1 Q K^T (token blocks <= tb)
    Split8 Ka[4], Qa[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = sw(tw, 4 * s + qt, 16);
      Ka[s] = {__builtin_bit_cast(bf16x8, lds[kY + row]), __builtin_bit_cast(bf16x8, lds[kY + 1024 + row])};
      float f[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) f[m] = tw < Tc ? qraw[s][m] : 0.f;
      Qa[s] = split8(f);
    }
    f32x4 W[4], QS[4], XK[4];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      W[c4] = QS[c4] = zero;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int row = sw(16 * (4 * hf + c4) + r16, 4 * s + qt, 16);
        const Split8 b{__builtin_bit_cast(bf16x8, lds[kX + row]), __builtin_bit_cast(bf16x8, lds[kX + 2048 + row])};
        W[c4] = mfma3(Ka[s], b, W[c4]);
        QS[c4] = mfma3(Qa[s], b, QS[c4]);
      }
    }
#pragma unroll
    for (int ci = 0; ci < 4; ++ci) {
      XK[ci] = zero;
      if (ci > tb) continue;  // uniform over the wave
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int row = sw(16 * ci + r16, 4 * s + qt, 16);
        const Split8 b{__builtin_bit_cast(bf16x8, lds[kY + row]), __builtin_bit_cast(bf16x8, lds[kY + 1024 + row])};
        XK[ci] = mfma3(hf == 0 ? Ka[s] : Qa[s], b, XK[ci]);
      }
    }
    lds_barrier();  // S^T and K [t][k] are no longer read: X and Y are reused

    // 2. R -> X as [dv][t]; A (half 0) or P (half 1) -> Y as [t][i]; lane rows t = 16 tb + 4 qt + j
    float Lt[4], Gt[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Lt[j] = sL[16 * tb + 4 * qt + j];
      Gt[j] = sG[16 * tb + 4 * qt + j];
    }
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const int dv = 16 * (4 * hf + c4) + r16;
      float rv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tb + 4 * qt + j;
        const float vv = t < Tc ? vraw[c4][j] : 0.f;
        rv[j] = sB[t] * (vv - Gt[j] * W[c4][j]);
      }
      lds[kX + sw(dv, 4 * tb + qt, 16)] = make_uint4(__builtin_bit_cast(uint32_t, rv[0]), __builtin_bit_cast(uint32_t, rv[1]),
                                                   __builtin_bit_cast(uint32_t, rv[2]), __builtin_bit_cast(uint32_t, rv[3]));
    }
#pragma unroll
    for (int ci = 0; ci < 4; ++ci) {
      const int i = 16 * ci + r16;
      const float Li = sL[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tb + 4 * qt + j;
        const float e = __expf(fminf(Lt[j] - Li, 0.f));  // i <= t: L_t <= L_i
        if (hf == 0)
          fA[t * 64 + i] = i < t ? sB[t] * e * XK[ci][j] : 0.f;
        else
          fP[swf(t, i)] = i <= t ? e * XK[ci][j] : 0.f;
      }
    }
    // the diagonal block D_tb = (I + A_bb)^-1 by forward substitution, lanes
    // 4 jj .. 4 jj + 3 on column jj (keys 4 p .. 4 p + 3 each)
    if (hf == 0) {
      wave_lds_fence();
      const int jj = ln >> 2, p = ln & 3, base = 16 * tb;
      f32x4 arow[16];
#pragma unroll
      for (int m = 0; m < 16; ++m) arow[m] = *reinterpret_cast<const f32x4*>(fA + (base + m) * 64 + base + 4 * p);
      float x[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        float a[4];
        __builtin_memcpy(a, &arow[m], 16);
        const float part = quad_sum(a[0] * x[0] + a[1] * x[1] + a[2] * x[2] + a[3] * x[3]);
        const float val = (m == jj ? 1.f : 0.f) - part;
        if (p == (m >> 2)) x[m & 3] = val;
        if (p == 0) fD[(base + m) * 16 + jj] = val;
      }
    }
    lds_barrier();

    if (y_out) {  // uniform
      const bf16_t* const zb = z + tok0 * ld_z + h * kD;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          zraw[c4][j] = bf16_to_f32(at(zb, min(tr0 + j, Tc - 1) * ld_z + 16 * (4 * hf + c4) + r16));
    }

    // 3. U_b = D_b (R_b - sum_{j<b} A_bj U_j) on value columns 16 w .. 16 w + 15,
    // in registers: U[b] holds rows 16 b + 4 qt + e, column 16 w + r16
    // U and D U go out as bf16 hi/lo [dv][t] (the B operands of step 4) over
    // the R region: every wave reads its R first
    {
      const int dv = 16 * w + r16;
      f32x4 U[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) U[b] = __builtin_bit_cast(f32x4, lds[kX + sw(dv, 4 * b + qt, 16)]);
      lds_barrier();
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        f32x4 acc = U[b];
#pragma unroll
        for (int j = 0; j < b; ++j) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(fA + (16 * b + r16) * 64 + 16 * j + 4 * qt);
          acc = mfma3k16(split4(-a), split4(U[j]), acc);
        }
        const f32x4 d = *reinterpret_cast<const f32x4*>(fD + (16 * b + r16) * 16 + 4 * qt);
        U[b] = mfma3k16(split4(d), split4(acc), zero);
      }
      uint2* const xs = reinterpret_cast<uint2*>(lds);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        // rows 16 b + 4 qt .. + 3: half (qt & 1) of the 8-token chunk 2 b + (qt >> 1)
        const int o = sw(dv, 2 * b + (qt >> 1), 8) * 2 + (qt & 1);
        const f32x4 ev = *reinterpret_cast<const f32x4*>(sE + 16 * b + 4 * qt);
        const Split4 u = split4(U[b]), du = split4(U[b] * ev);
        xs[kUhi * 2 + o] = __builtin_bit_cast(uint2, u.hi);
        xs[kUlo * 2 + o] = __builtin_bit_cast(uint2, u.lo);
        xs[kDUhi * 2 + o] = __builtin_bit_cast(uint2, du.hi);
        xs[kDUlo * 2 + o] = __builtin_bit_cast(uint2, du.lo);
      }
    }
    lds_barrier();

    // 4a. O = diag(Gamma) Q S^T + P U (token block tb, value half hf)
    f32x4 O[4];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int j = 0; j < 4; ++j) O[c4][j] = Gt[j] * QS[c4][j];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (32 * s > 16 * tb + 15) continue;  // P is zero past the diagonal (uniform)
      float fp[8];
      read8f(reinterpret_cast<const uint4*>(fP), tw, 8 * s + 2 * qt, fp);
      const Split8 a = split8(fp);
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int row = sw(16 * (4 * hf + c4) + r16, 4 * s + qt, 8);
        const Split8 u{__builtin_bit_cast(bf16x8, lds[kUhi + row]), __builtin_bit_cast(bf16x8, lds[kUlo + row])};
        O[c4] = mfma3(a, u, O[c4]);
      }
    }
    // 4b. S <- Gamma_last S + K^T (D U): this wave's key rows, all values
    const float Glast = sG[63];
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[ct][e] *= Glast;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int row = sw(16 * w + r16, 4 * s + qt, 8);
      const Split8 ka{__builtin_bit_cast(bf16x8, lds[kZ + row]), __builtin_bit_cast(bf16x8, lds[kZ + 1024 + row])};
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        const int rw = sw(16 * ct + r16, 4 * s + qt, 8);
        const Split8 du{__builtin_bit_cast(bf16x8, lds[kDUhi + rw]), __builtin_bit_cast(bf16x8, lds[kDUlo + rw])};
        S[ct] = mfma3(ka, du, S[ct]);
      }
    }
    // 4c. partial sums of o^2 over this wave's value half, per token
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float ssq = 0.f;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) ssq += O[c4][j] * O[c4][j];
      ssq = row_sum(ssq);
      if (r16 == 0) sN[hf * 64 + 16 * tb + 4 * qt + j] = ssq;
    }
    lds_barrier();  // also ends every read of this chunk's X, Y, Z and small arrays

    // 5. outputs of the live tokens: o, and the gated norm y
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tb + 4 * qt + j;
      if (t >= Tc) continue;
      const float inv = 1.f / sqrtf((sN[t] + sN[64 + t]) / float(kD) + 1e-6f);
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int dv = 16 * (4 * hf + c4) + r16;
        const float o = O[c4][j];
        if (o_out) at(o_out + (tok0 * Hv + h) * kD, t * ldv + dv) = o;
        if (y_out)
          at(y_out + (tok0 * Hv + h) * kD, t * ldv + dv) = f32_to_bf16(o * inv * nw[c4] * silu_f(zraw[c4][j]));
      }
    }
  }

  float* dst = state + (size_t(ds) * Hv + h) * kD * kD;
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int r16 = ln & 15, qt = ln >> 4;
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
#pragma unroll
    for (int e = 0; e < 4; ++e) at(dst, (16 * w + 4 * qt + e) * kD + 16 * ct + r16) = S[ct][e];
}

}  // namespace

size_t gdn_chunked_lds_bytes() { return kLds; }

void gdn_chunked(const float* q_hat, const float* k_hat, const float* v, const float* decay, const float* beta,
                 const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* state, const GdnSlots& slots,
                 float* o_out, const bf16_t* z, int ld_z, const float* norm_w, bf16_t* y_out, hipStream_t stream) {
  require(g.key_dim == kD && g.value_dim == kD, "gdn_chunked: key and value dims must be 128");
  require(g.value_heads % g.key_heads == 0, "gdn_chunked: head grouping");
  require(!y_out || (z && norm_w), "gdn_chunked: gated norm needs z and norm weight");
  if (rows <= 0) return;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(gdn_chunk_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(kLds));
  HB_CHECK(attr);
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(g.value_heads, rows), dim3(kThreads), kLds, stream, q_hat, k_hat, v, decay,
                     beta, cu_seqlens, g, state, slots.src, slots.dst, o_out, z, ld_z, norm_w, y_out);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
