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
// regrouped. The triangular system is solved in 16-token blocks: each wave
// inverts one diagonal block (I + A_bb) by forward substitution, then every
// wave runs the block substitution U_b = (I + A_bb)^-1 (R_b - sum_{j<b} A_bj
// U_j) on its own 32 value columns.
//
// Every product runs on the bf16 MFMA with FP32 operands split into bf16
// high and low parts (a b = a_hi b_hi + a_hi b_lo + a_lo b_hi, about 16
// mantissa bits per operand), which keeps the state at FP32-class accuracy
// while the work per chunk is matrix products instead of 64 dependent token
// steps. The workgroup (4 waves) owns one (row, head): wave w computes the
// rows of token block w (16 tokens) and the state rows of keys [32 w, 32 w +
// 32), which stay in registers across the row's chunks.
#include "deltanet.h"
#include "q4_device.h"

namespace hb {
namespace {

constexpr int kD = 128;   // key_dim == value_dim
constexpr int kC = 64;    // tokens per chunk
constexpr int kThreads = 256;

// LDS (uint4 units). X: S^T hi/lo as bf16 [dv][k] (2 x 2048), later the
// corrected values R -> U as f32 [dv][t] (2048) and the inverted diagonal
// blocks (I + A_bb)^-1 as f32 [t][16] (256). Y: K hi/lo as bf16 [t][k]
// (2 x 1024), later A and P as f32 [t][i] (1024 each). Z: K^T hi/lo as bf16
// [k][t] (2 x 1024). Then the chunk's log-decay prefix and betas.
constexpr int kX = 0, kY = 4096, kZ = kY + 2048, kSmall = kZ + 2048;
constexpr int kSmallFloats = 64 + 64;
constexpr size_t kLds = size_t(kSmall) * 16 + kSmallFloats * 4;

// row r, 16-byte chunk c of a matrix with nc chunks per row, XOR-swizzled by
// row so that 16 lanes reading the same chunk of 16 rows hit distinct banks
__device__ inline int sw(int r, int c, int nc) { return r * nc + (c ^ (r & (nc - 1))); }
// f32 element (r, col) of a 64-column matrix stored in swizzled 4-float chunks
__device__ inline int swf(int r, int col) { return sw(r, col >> 2, 16) * 4 + (col & 3); }

struct Split8 {
  bf16x8 hi, lo;
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

__device__ inline f32x4 mfma3(const Split8& a, const Split8& b, f32x4 acc) {
  acc = mfma16(a.lo, b.hi, acc);
  acc = mfma16(a.hi, b.lo, acc);
  return mfma16(a.hi, b.hi, acc);
}

// 8 consecutive floats from two swizzled 4-float chunks (row r, chunks c, c+1).
// Vectors are converted whole: __builtin_bit_cast of one element of a vector
// value (v[i]) miscompiles to element 0 with this compiler.
__device__ inline void read8f(const uint4* m, int r, int c, float (&f)[8]) {
  const f32x4 a = __builtin_bit_cast(f32x4, m[sw(r, c, 16)]), b = __builtin_bit_cast(f32x4, m[sw(r, c + 1, 16)]);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[q] = a[q];
    f[4 + q] = b[q];
  }
}

// orders this wave's LDS stores before its later loads of other lanes' data
__device__ inline void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup"); }

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
  float* const sL = reinterpret_cast<float*>(lds + kSmall);  // log-decay prefix of the chunk
  float* const sB = sL + 64;                                  // betas
  float* const fX = reinterpret_cast<float*>(lds + kX);       // R / U [dv][t] (swizzled chunks)
  float* const fD = fX + 2048 * 4;                            // (I + A_bb)^-1 [t][16]
  float* const fA = reinterpret_cast<float*>(lds + kY);       // A [t][i]
  float* const fP = fA + 1024 * 4;                            // P [t][i] (swizzled chunks)
  const int h = blockIdx.x, r = blockIdx.y, lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Hv = g.value_heads, Hk = g.key_heads, kh = h / (Hv / Hk);
  const int t0 = cu_seqlens[r], T = cu_seqlens[r + 1] - t0;
  if (T <= 0) return;  // uniform over the workgroup
  const int ss = src_slot ? src_slot[r] : r, ds = dst_slot ? dst_slot[r] : r;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  // this wave's state rows: Skm[k][dv] (key-major), k = 32 w + 16 kt + 4 qt + j, dv = 16 ct + r16
  f32x4 S[2][8];
  {
    const int r16 = lane & 15, qt = lane >> 4;
    const float* src = state + (size_t(ss) * Hv + h) * kD * kD;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          S[kt][ct][j] = at(src, (32 * w + 16 * kt + 4 * qt + j) * kD + 16 * ct + r16);
  }

  for (int c0 = 0; c0 < T; c0 += kC) {
    const int Tc = min(kC, T - c0);
    // lane indices re-derived per chunk: keeps the compiler from hoisting
    // (and spilling) every lane-dependent address of the body out of the loop
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r16 = ln & 15, qt = ln >> 4, tid = 64 * w + ln;
    const size_t tok0 = size_t(t0) + c0;
    // chunk bases (uniform); token t of the chunk at t * ldk (q, k), t * ldv (v)
    const float* const kb = k_hat + (tok0 * Hk + kh) * kD;
    const float* const qb = q_hat + (tok0 * Hk + kh) * kD;
    const float* const vb = v + (tok0 * Hv + h) * kD;
    const uint32_t ldk = Hk * kD, ldv = Hv * kD;

    // 0. log-decay prefix and betas (wave 0); tokens past Tc: g = 1, beta = 0
    if (w == 0) {
      const bool live = ln < Tc;
      const int tl = min(ln, Tc - 1);
      const float gl = at(decay + tok0 * Hv + h, tl * Hv), bl = at(beta + tok0 * Hv + h, tl * Hv);
      const float gt = live ? gl : 1.f;
      float lg = __logf(fmaxf(gt, 1e-30f));
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_up(lg, off, 64);
        if (ln >= off) lg += o;
      }
      sL[ln] = lg;
      sB[ln] = live ? bl : 0.f;
    }
    // 1. staging: S^T hi/lo [dv][k] from the state registers
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        const int dv = 16 * ct + r16, c = 4 * w + 2 * kt + (qt >> 1);  // 8-key chunk of keys 32w+16kt+4qt..+3
        uint2 hi, lo;
        split2(S[kt][ct][0], S[kt][ct][1], hi.x, lo.x);
        split2(S[kt][ct][2], S[kt][ct][3], hi.y, lo.y);
        uint2* xs = reinterpret_cast<uint2*>(lds + kX);
        xs[sw(dv, c, 16) * 2 + (qt & 1)] = hi;
        xs[(2048 + sw(dv, c, 16)) * 2 + (qt & 1)] = lo;
      }
    // K hi/lo [t][k] and K^T hi/lo [k][t] (rows past Tc are zeros)
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = tid + it * kThreads;
      {
        const int t = idx >> 4, c = idx & 15;
        const uint32_t o = min(t, Tc - 1) * ldk + 8 * c;  // clamped: loads issue unconditionally
        float f[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) f[m] = at(kb, o + m);
#pragma unroll
        for (int m = 0; m < 8; ++m) f[m] = t < Tc ? f[m] : 0.f;
        const Split8 s = split8(f);
        lds[kY + sw(t, c, 16)] = __builtin_bit_cast(uint4, s.hi);
        lds[kY + 1024 + sw(t, c, 16)] = __builtin_bit_cast(uint4, s.lo);
      }
      {
        const int k = idx & 127, c = idx >> 7;  // tokens 8c .. 8c + 7 of key k
        float f[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) f[m] = at(kb, min(8 * c + m, Tc - 1) * ldk + k);
#pragma unroll
        for (int m = 0; m < 8; ++m) f[m] = 8 * c + m < Tc ? f[m] : 0.f;
        const Split8 s = split8(f);
        lds[kZ + sw(k, c, 8)] = __builtin_bit_cast(uint4, s.hi);
        lds[kZ + 1024 + sw(k, c, 8)] = __builtin_bit_cast(uint4, s.lo);
      }
    }
    __syncthreads();

    // 2. with A operands of token block w (keys 32 s + 8 qt .. + 7):
    // W = K S^T and K K^T (token blocks <= w), then Q S^T and Q K^T
    const int tw = 16 * w + r16;
    const uint32_t trow = min(tw, Tc - 1) * ldk;
    auto a_frags = [&](const float* base, Split8 (&fr)[4]) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float f[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) f[m] = at(base, trow + 32 * s + 8 * qt + m);
#pragma unroll
        for (int m = 0; m < 8; ++m) f[m] = tw < Tc ? f[m] : 0.f;
        fr[s] = split8(f);
      }
    };
    auto products = [&](const Split8 (&fr)[4], f32x4 (&SS)[8], f32x4 (&XK)[4]) {
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        SS[ct] = zero;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int row = sw(16 * ct + r16, 4 * s + qt, 16);
          const Split8 b{__builtin_bit_cast(bf16x8, lds[kX + row]), __builtin_bit_cast(bf16x8, lds[kX + 2048 + row])};
          SS[ct] = mfma3(fr[s], b, SS[ct]);
        }
      }
#pragma unroll
      for (int ci = 0; ci < 4; ++ci) {
        XK[ci] = zero;
        if (ci > w) continue;  // uniform over the wave
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int row = sw(16 * ci + r16, 4 * s + qt, 16);
          const Split8 b{__builtin_bit_cast(bf16x8, lds[kY + row]), __builtin_bit_cast(bf16x8, lds[kY + 1024 + row])};
          XK[ci] = mfma3(fr[s], b, XK[ci]);
        }
      }
    };
    f32x4 W[8], QS[8], KK[4], QK[4];
    {
      Split8 fr[4];
      a_frags(kb, fr);
      products(fr, W, KK);
    }
    {
      Split8 fr[4];
      a_frags(qb, fr);
      products(fr, QS, QK);
    }
    __syncthreads();  // S^T and K [t][k] are no longer read: X and Y are reused

    // 3. R -> X as [dv][t]; A and P -> Y as [t][i]; lane rows t = 16 w + 4 qt + j
    float Lt[4], Gt[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Lt[j] = sL[16 * w + 4 * qt + j];
      Gt[j] = __expf(Lt[j]);
    }
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      const int dv = 16 * ct + r16;
      float rv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * w + 4 * qt + j;
        const float vl = at(vb, min(t, Tc - 1) * ldv + dv);
        const float vv = t < Tc ? vl : 0.f;
        rv[j] = sB[t] * (vv - Gt[j] * W[ct][j]);
      }
      lds[kX + sw(dv, 4 * w + qt, 16)] = make_uint4(__builtin_bit_cast(uint32_t, rv[0]), __builtin_bit_cast(uint32_t, rv[1]),
                                                  __builtin_bit_cast(uint32_t, rv[2]), __builtin_bit_cast(uint32_t, rv[3]));
    }
#pragma unroll
    for (int ci = 0; ci < 4; ++ci) {
      const int i = 16 * ci + r16;
      const float Li = sL[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * w + 4 * qt + j;
        const float e = __expf(Lt[j] - Li);
        fA[t * 64 + i] = i < t ? sB[t] * e * KK[ci][j] : 0.f;
        fP[swf(t, i)] = i <= t ? e * QK[ci][j] : 0.f;
      }
    }
    wave_lds_fence();

    // 4a. this wave's diagonal block: D_w = (I + A_ww)^-1 by forward
    // substitution, lanes 4 jj .. 4 jj + 3 on column jj (keys 4 p .. 4 p + 3 each)
    {
      const int jj = ln >> 2, p = ln & 3, base = 16 * w;
      float x[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const float4 a = *reinterpret_cast<const float4*>(fA + (base + m) * 64 + base + 4 * p);
        float part = a.x * x[0] + a.y * x[1] + a.z * x[2] + a.w * x[3];
        part += __shfl_xor(part, 1, 64);
        part += __shfl_xor(part, 2, 64);
        const float val = (m == jj ? 1.f : 0.f) - part;
        if (p == (m >> 2)) x[m & 3] = val;
        if (p == 0) fD[(base + m) * 16 + jj] = val;
      }
    }
    __syncthreads();

    // 4b. U_b = D_b (R_b - sum_{j<b} A_bj U_j) on value columns 32 w .. 32 w + 31
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 acc[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        acc[e] = __builtin_bit_cast(f32x4, lds[kX + sw(32 * w + 16 * e + r16, 4 * b + qt, 16)]);
      }
#pragma unroll
      for (int s = 0; 32 * s < 16 * b; ++s) {
        float fa[8];
        const bool live = 32 * s + 8 * qt < 16 * b;
#pragma unroll
        for (int m = 0; m < 8; ++m) fa[m] = live ? -fA[(16 * b + r16) * 64 + 32 * s + 8 * qt + m] : 0.f;
        const Split8 a = split8(fa);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float fu[8];
          read8f(lds + kX, 32 * w + 16 * e + r16, 8 * s + 2 * qt, fu);
          acc[e] = mfma3(a, split8(fu), acc[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 2; ++e)
        lds[kX + sw(32 * w + 16 * e + r16, 4 * b + qt, 16)] = __builtin_bit_cast(uint4, acc[e]);
      wave_lds_fence();
      float fd[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) fd[m] = qt < 2 ? fD[(16 * b + r16) * 16 + 8 * qt + m] : 0.f;
      const Split8 d = split8(fd);
      f32x4 u[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        float fy[8];
        if (qt < 2) {
          read8f(lds + kX, 32 * w + 16 * e + r16, 4 * b + 2 * qt, fy);
        } else {
#pragma unroll
          for (int m = 0; m < 8; ++m) fy[m] = 0.f;
        }
        u[e] = mfma3(d, split8(fy), zero);
      }
      wave_lds_fence();
#pragma unroll
      for (int e = 0; e < 2; ++e)
        lds[kX + sw(32 * w + 16 * e + r16, 4 * b + qt, 16)] = __builtin_bit_cast(uint4, u[e]);
      wave_lds_fence();
    }
    __syncthreads();

    // 5a. O = diag(Gamma) Q S^T + P U (token block w)
    f32x4 O[8];
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
      for (int j = 0; j < 4; ++j) O[ct][j] = Gt[j] * QS[ct][j];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float fp[8];
      read8f(reinterpret_cast<const uint4*>(fP), tw, 8 * s + 2 * qt, fp);
      const Split8 a = split8(fp);
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        float fu[8];
        read8f(lds + kX, 16 * ct + r16, 8 * s + 2 * qt, fu);
        O[ct] = mfma3(a, split8(fu), O[ct]);
      }
    }
    // 5b. S <- Gamma_last S + K^T (D U): this wave's key rows
    const float Llast = sL[63];
    const float Glast = __expf(Llast);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j) S[kt][ct][j] *= Glast;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float Ds[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) Ds[m] = __expf(Llast - sL[32 * s + 8 * qt + m]);
      Split8 ka[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int row = sw(32 * w + 16 * kt + r16, 4 * s + qt, 8);
        ka[kt] = {__builtin_bit_cast(bf16x8, lds[kZ + row]), __builtin_bit_cast(bf16x8, lds[kZ + 1024 + row])};
      }
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        float fu[8];
        read8f(lds + kX, 16 * ct + r16, 8 * s + 2 * qt, fu);
#pragma unroll
        for (int m = 0; m < 8; ++m) fu[m] *= Ds[m];
        const Split8 b = split8(fu);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) S[kt][ct] = mfma3(ka[kt], b, S[kt][ct]);
      }
    }

    // 6. outputs of the live tokens: o, and the gated norm y
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * w + 4 * qt + j;
      float ssq = 0.f;
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) ssq += O[ct][j] * O[ct][j];
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) ssq += __shfl_xor(ssq, off, 64);
      if (t >= Tc) continue;
      const float inv = rsqrtf(ssq / float(kD) + 1e-6f);
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        const int dv = 16 * ct + r16;
        const float o = O[ct][j];
        if (o_out) at(o_out + (tok0 * Hv + h) * kD, t * ldv + dv) = o;
        if (y_out) {
          const float zz = bf16_to_f32(at(z + tok0 * ld_z + h * kD, t * ld_z + dv));
          at(y_out + (tok0 * Hv + h) * kD, t * ldv + dv) = f32_to_bf16(o * inv * norm_w[dv] * silu_f(zz));
        }
      }
    }
    __syncthreads();  // the next chunk rewrites every LDS region
  }

  float* dst = state + (size_t(ds) * Hv + h) * kD * kD;
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int r16 = ln & 15, qt = ln >> 4;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
      for (int j = 0; j < 4; ++j) at(dst, (32 * w + 16 * kt + 4 * qt + j) * kD + 16 * ct + r16) = S[kt][ct][j];
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
