// Gated GQA attention over a paged KV cache for ragged decode / MTP verify rows.
//
// paged_attention: one wave per (row, kv head, 16 query pairs, key split).
// A "pair" is (token, q head of the group): group = q_heads / kv_heads = 8, so a
// 16-pair row group covers two tokens of the row. Scores are computed
// transposed, S^T = K . Q^T (v_mfma_f32_16x16x32_bf16, A = 16 keys of one page,
// B = Q^T held in registers), which leaves each lane with the scores of one
// pair for 8 keys of a 32-key step -- exactly the B-operand fragment of the
// second product O^T += V^T . P^T when the k index of both operands runs over
// keys {4q..4q+3} of the first page and {4q..4q+3} of the second page for lane
// quarter q. V pages are stored transposed ([dim][16 keys]), so the V^T operand
// of that k set is two contiguous 8-byte loads. No LDS and no lane shuffles are
// needed between the two products; the online softmax needs two xor shuffles
// per step for the row max and row sum. Each wave streams its split with the
// next 32 keys' K and V fragments loaded while the current ones are used.
// attn_combine merges the splits (log-sum-exp) and applies sigmoid(gate).
#include "attention.h"

namespace hb {
namespace {

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// grid (q_heads + 2*kv_heads, tokens), one wave: q heads, then k heads, then v heads.
__global__ __launch_bounds__(64) void attn_prep_kernel(const bf16_t* __restrict__ qg, int ld_qg,
                                                       const bf16_t* __restrict__ kv, int ld_kv, int kv_off,
                                                       const float* __restrict__ q_norm,
                                                       const float* __restrict__ k_norm,
                                                       const int32_t* __restrict__ token_pos,
                                                       const int32_t* __restrict__ kv_slot, AttnGeom g,
                                                       bf16_t* __restrict__ qout, bf16_t* __restrict__ kcache,
                                                       bf16_t* __restrict__ vcache) {
  const int head = blockIdx.x, i = blockIdx.y, lane = threadIdx.x;
  const int D = g.head_dim, per = D / 64;  // elements per lane (<= 4)
  const int Hq = g.q_heads, Hkv = g.kv_heads;
  const int kind = head < Hq ? 0 : (head < Hq + Hkv ? 1 : 2);  // 0 q, 1 k, 2 v
  const int hh = kind == 0 ? head : (kind == 1 ? head - Hq : head - Hq - Hkv);
  const bf16_t* src = kind == 0 ? qg + size_t(i) * ld_qg + size_t(hh) * 2 * D
                                : kv + size_t(i) * ld_kv + (kind == 2 ? kv_off : 0) + size_t(hh) * D;
  // every load of the head is issued before the first use (clamped indices)
  float v[4], nw[4];
  const float* wn = kind == 0 ? q_norm : k_norm;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = bf16_to_f32(src[lane * per + min(e, per - 1)]);
    nw[e] = wn[lane * per + min(e, per - 1)];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = e < per ? v[e] : 0.f;
  const int pos = token_pos[i];
  const int slot = kv_slot[i];
  if (kind != 2) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += v[e] * v[e];
    const float inv = 1.f / sqrtf(wave_sum(ss) / float(D) + g.eps);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < per) v[e] = v[e] * inv * nw[e];
    // Non-traditional RoPE on the first `rotary` dims: pairs (j, j + rotary/2),
    // angle pos * theta^(-2j/rotary) in f32 as MLX's fast::rope computes it.
    const int half = g.rotary / 2, lane_off = half / per;
    const int partner = lane < lane_off ? lane + lane_off : lane - lane_off;
    const float log2_theta = log2f(g.theta);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float other = __shfl(v[e], partner, 64);
      const int idx = lane * per + e;
      if (e < per && idx < g.rotary) {
        const int j = idx < half ? idx : idx - half;
        const float ang = float(pos) * exp2f(-2.f * float(j) / float(g.rotary) * log2_theta);
        float sn, cs;
        sincosf(ang, &sn, &cs);
        v[e] = idx < half ? v[e] * cs - other * sn : other * sn + v[e] * cs;
      }
    }
  }
  const int page = slot / kPage, within = slot % kPage;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (e >= per) continue;
    const int idx = lane * per + e;
    const bf16_t out = f32_to_bf16(v[e]);
    if (kind == 0)
      qout[(size_t(i) * Hq + hh) * D + idx] = out;
    else if (kind == 1)
      kcache[((size_t(page) * Hkv + hh) * kPage + within) * D + idx] = out;
    else
      vcache[((size_t(page) * Hkv + hh) * D + idx) * kPage + within] = out;
  }
}

__device__ inline f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Two floats to a bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
}

constexpr int kD = 256;          // head_dim of the paged kernel
constexpr int kMaxPieceSteps = 8;  // 32-key steps of a piece: split_len <= 256
constexpr int kDT = kD / 16;     // 16-dim output tiles

// One 32-key step over two pages (keys 0..15 of p0, 16..31 of p1). The score
// product S^T = K . Q^T runs as two MFMAs whose rows are keys
// {0-3, 8-11, 16-19, 24-27} and {4-7, 12-15, 20-23, 28-31}: lane quarter q then
// holds the scores of keys 8q..8q+7, which is both the B fragment of
// O^T += V^T . P^T and one 16-byte row slice of a transposed V page.
struct KVFrag {
  bf16x8 k0[8], k1[8];  // K fragments of the two key sets, 8 dim steps
  u32x4 v[kDT];         // V^T fragments of the 16 dim tiles (keys 8q..8q+7)
};

// K/V pages are read once per launch where every row fits one 16-pair group:
// streaming loads keep them from displacing the caches' other contents. A
// verify row's second pair group reads the same pages right away on the same
// XCD (the piece list puts the two 8 slots apart), so launches with such rows
// load them normally and the second read hits L2.
template <bool NT, class V>
__device__ inline V kv_load(const V* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

template <bool NT>
__device__ inline void load_kv(KVFrag& f, const bf16_t* __restrict__ kcache, const bf16_t* __restrict__ vcache,
                               int p0, int p1, int Hkv, int kh, int col, int qd) {
  const int key0 = (col >> 2) * 8 + (col & 3);  // key of row `col` in the first set; +4 in the second
  const int kp = key0 < 16 ? p0 : p1;
  const bf16_t* ka0 = kcache + ((size_t(kp) * Hkv + kh) * kPage + (key0 & 15)) * kD + 8 * qd;
  const bf16_t* ka1 = ka0 + 4 * kD;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    f.k0[s] = kv_load<NT>(reinterpret_cast<const bf16x8*>(ka0 + 32 * s));
    f.k1[s] = kv_load<NT>(reinterpret_cast<const bf16x8*>(ka1 + 32 * s));
  }
  const int vp = qd < 2 ? p0 : p1;
  const bf16_t* va = vcache + ((size_t(vp) * Hkv + kh) * kD + col) * kPage + 8 * (qd & 1);
#pragma unroll
  for (int dt = 0; dt < kDT; ++dt) f.v[dt] = kv_load<NT>(reinterpret_cast<const u32x4*>(va + dt * 16 * kPage));
}

// Work list (one workgroup). A piece is (row, 16-pair row group, split,
// kv head): keys [split * split_len, min((split + 1) * split_len, context)) of
// the row, so a row's result never depends on the rest of the batch. Whole
// pieces are listed first, then the rows' shorter last pieces by decreasing
// length: waves are dispatched in list order, so the longest work starts first
// and the last waves to start are the shortest (longest-first list scheduling).
constexpr int kPlanThreads = 1024;

__device__ inline int block_exclusive_scan(int v, int* sc) {
  const int tid = threadIdx.x;
  sc[tid] = v;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int add = tid >= off ? sc[tid - off] : 0;
    __syncthreads();
    sc[tid] += add;
    __syncthreads();
  }
  const int incl = sc[tid];
  __syncthreads();
  return incl - v;
}

struct RowPieces {
  int groups, whole, tail;  // row groups, whole pieces, keys in the last short piece (0: none)
};

__device__ inline RowPieces row_pieces(const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ context,
                                       int r, int group, int row_groups, int splits, int split_len) {
  RowPieces p{0, 0, 0};
  const int ctx = context[r];
  p.groups = min((cu_seqlens[r + 1] - cu_seqlens[r]) * group + 15, 16 * row_groups) / 16;
  if (p.groups == 0 || ctx <= 0) return RowPieces{0, 0, 0};
  p.whole = min(ctx / split_len, splits);
  p.tail = p.whole < splits ? ctx % split_len : 0;
  return p;
}

constexpr int kPlanMaxRows = 2048;
constexpr int kPlanBuckets = 32 * kMaxPieceSteps;  // short-piece lengths 1..split_len-1

__global__ __launch_bounds__(kPlanThreads) void attn_plan_kernel(const int32_t* __restrict__ cu_seqlens,
                                                                 const int32_t* __restrict__ context, int rows,
                                                                 int group, int row_groups, int splits, int split_len,
                                                                 int Hkv, int32_t* __restrict__ plan) {
  __shared__ int sc[kPlanThreads];
  __shared__ int row_off[kPlanMaxRows + 1];  // first list slot of each row's whole pieces
  __shared__ short row_groups_s[kPlanMaxRows], row_tail[kPlanMaxRows];
  __shared__ int bucket[kPlanBuckets];       // short pieces per length, then their first slot
  int2* items = reinterpret_cast<int2*>(plan + 2);
  const int tid = threadIdx.x;
  for (int b = tid; b < kPlanBuckets; b += kPlanThreads) bucket[b] = 0;
  int carry = 0;
  for (int base = 0; base < rows; base += kPlanThreads) {
    const int r = base + tid;
    RowPieces p{0, 0, 0};
    if (r < rows) {
      p = row_pieces(cu_seqlens, context, r, group, row_groups, splits, split_len);
      row_groups_s[r] = short(p.groups);
      row_tail[r] = short(p.tail);
      if (p.tail > 0) atomicAdd(&bucket[p.tail], p.groups * Hkv);
    }
    const int cnt = p.groups * p.whole * Hkv;
    const int off = carry + block_exclusive_scan(cnt, sc);
    if (r < rows) row_off[r] = off;
    if (tid == kPlanThreads - 1) sc[0] = off + cnt;
    __syncthreads();
    carry = sc[0];
    __syncthreads();
  }
  const int whole_total = carry;
  if (tid == 0) row_off[rows] = whole_total;
  // short pieces: slots by decreasing length after the whole pieces
  if (tid == 0) {
    int at = whole_total;
    for (int b = kPlanBuckets - 1; b > 0; --b) {
      const int n = bucket[b];
      bucket[b] = at;
      at += n;
    }
    plan[0] = at;
  }
  __syncthreads();
  // whole pieces: list slot i belongs to the last row with row_off <= i. A
  // row's keys (split, kv head) go in blocks of 8, each block listed once per
  // row group: the row groups of one key range then sit 8 slots apart, and
  // since list slot i runs as workgroup i, on XCD i % 8, they share that XCD's
  // L2 and run together, so the second group's K/V reads hit the first's.
  for (int i = tid; i < whole_total; i += kPlanThreads) {
    int lo = 0, hi = rows;
    while (hi - lo > 1) {
      const int mid = (lo + hi) / 2;
      if (row_off[mid] <= i)
        lo = mid;
      else
        hi = mid;
    }
    const int j = i - row_off[lo];
    const int G = row_groups_s[lo];
    const int keys = (row_off[lo + 1] - row_off[lo]) / G;  // whole * Hkv
    const int b = j / (8 * G), in = j % (8 * G);
    const int m = min(8, keys - 8 * b);                     // keys in this block
    items[i] = int2{lo * row_groups + in / m, 8 * b + in % m};  // (row, group), split * Hkv + kv head
  }
  for (int r = tid; r < rows; r += kPlanThreads) {
    const int tail = row_tail[r];
    if (tail == 0) continue;
    const int n = row_groups_s[r] * Hkv;
    const int at = atomicAdd(&bucket[tail], n);
    const int whole = min(context[r] / split_len, splits);
    for (int j = 0; j < n; ++j) items[at + j] = int2{r * row_groups + j / Hkv, whole * Hkv + j % Hkv};
  }
}

// Persistent waves, one per SIMD, each walking the piece list with a stride
// of the grid. A piece's start is a chain of dependent loads (list entry, row
// tables, block table, then the first K/V step: about 10 us, measured, against
// 4.5 us for each later 32-key step), so while a wave runs a piece it already
// loads the next piece's entry, row tables and page numbers, and the piece's
// last K/V load is the next piece's first step; only the q fragments (L2
// hits) are loaded at the switch. Pieces run an even
// number of 32-key steps (a tail piece's extra step is fully masked), so that
// first step always lands in the same fragment buffer.
template <bool NT>
__global__ __launch_bounds__(64) void paged_attn_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kcache,
                                                        const bf16_t* __restrict__ vcache,
                                                        const int32_t* __restrict__ block_table, int max_pages,
                                                        const int32_t* __restrict__ cu_seqlens,
                                                        const int32_t* __restrict__ context, int Hq, int Hkv,
                                                        float scale, int row_groups, int splits, int split_len,
                                                        const int32_t* __restrict__ plan, float* __restrict__ work_o,
                                                        float* __restrict__ work_ml) {
  const int n_items = plan[0];
  const int2* items = reinterpret_cast<const int2*>(plan + 2);
  const int lane = threadIdx.x, col = lane & 15, qd = lane >> 4;
  const int group = Hq / Hkv;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  int item = blockIdx.x;
  if (item >= n_items) return;  // uniform over the wave

  // a piece's row, keys and pages (wave-uniform)
  struct Meta {
    int r, rg, split, kh, tok0, T, ctx, kbeg, kend, steps;
  };
  auto meta = [&](int i) {
    const int2 it = items[i];
    Meta mt;
    mt.r = it.x / row_groups;
    mt.rg = it.x % row_groups;
    mt.split = it.y / Hkv;
    mt.kh = it.y % Hkv;
    mt.tok0 = cu_seqlens[mt.r];
    mt.T = cu_seqlens[mt.r + 1] - mt.tok0;
    mt.ctx = context[mt.r];
    mt.kbeg = mt.split * split_len;
    mt.kend = min(mt.kbeg + split_len, mt.ctx);
    mt.steps = ((mt.kend - mt.kbeg + 31) / 32 + 1) & ~1;  // even
    return mt;
  };
  // page numbers of the piece's steps, the last page repeated past its end:
  // lane i holds page i (read out with readlane, so no scalar registers hold
  // the lists of two pieces)
  constexpr int kPg = 2 * kMaxPieceSteps + 2;
  static_assert(kPg <= 64, "one page per lane");
  auto pages = [&](const Meta& mt) {
    const int32_t* bt = block_table + size_t(mt.r) * max_pages;
    const int last_page = (mt.ctx - 1) / kPage, p0 = mt.kbeg / kPage;
    return bt[min(p0 + min(lane, kPg - 1), last_page)];
  };
  auto page = [](int pgv, int i) { return __builtin_amdgcn_readlane(pgv, i); };
  // the lane's (token, q head) pair of the piece and its q fragments
  auto load_q = [&](const Meta& mt, bf16x8 (&qf)[8]) {
    const int pair = mt.rg * 16 + col;
    const bool live = pair < mt.T * group;
    const int t = live ? pair / group : mt.T - 1;
    const int h = mt.kh * group + pair % group;
    const bf16_t* qrow = q + (size_t(mt.tok0 + t) * Hq + h) * kD + 8 * qd;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
    if (!live)
#pragma unroll
      for (int s = 0; s < 8; ++s) qf[s] = bf16x8{};
  };

  Meta cur = meta(item);
  int pg = pages(cur);
  bf16x8 qf[8];
  load_q(cur, qf);
  // A piece's f32 partial (16 KB per wave) goes to an LDS stash at its end and
  // reaches work_o during the next piece, a 4 KB chunk after each step pair's
  // loads: stored all at once, every wave's 16 stores sat in the vector memory
  // queue ahead of its next loads at the same moment, and a copy of this
  // loop's loads and products took 17 % longer with them (4.6 against 5.5 TB/s).
  __shared__ f32x4 stash[kDT * 64];  // [dt][lane]
  float* pend = nullptr;             // this lane's row of the stashed partial (null: none)
  auto flush = [&](int k) {          // dim tiles 4k .. 4k + 3 of the stashed partial
    if (pend)
#pragma unroll
      for (int d = 0; d < 4; ++d)
        *reinterpret_cast<f32x4*>(pend + (4 * k + d) * 16) = stash[(4 * k + d) * 64 + lane];
  };
  KVFrag fa, fb;
  load_kv<NT>(fa, kcache, vcache, page(pg, 0), page(pg, 1), Hkv, cur.kh, col, qd);
  for (;;) {
    // the next piece: its entry, tables, pages and q load while this one runs
    const int nitem = item + gridDim.x;
    const bool has_next = nitem < n_items;
    const Meta nxt = has_next ? meta(nitem) : cur;
    const int npg = pages(nxt);

    const int pairs = cur.T * group;
    const int pair = cur.rg * 16 + col;
    const bool live = pair < pairs;
    const int t = live ? pair / group : cur.T - 1;
    const int pos_t = cur.ctx - cur.T + t;
    const int t_min = cur.ctx - cur.T;  // keys up to here are visible to every token of the row
    const int kbeg = cur.kbeg, kend = cur.kend;
    f32x4 o[kDT];
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) o[dt] = zero;
    float m = -INFINITY, l = 0.f;
    auto step = [&](const KVFrag& f, int j0) {
      f32x4 s0 = zero, s1 = zero;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        s0 = mfma16(f.k0[s], qf[s], s0);
        s1 = mfma16(f.k1[s], qf[s], s1);
      }
      float sv[8];
      float mx = -INFINITY;
      if (j0 >= kbeg && j0 + 32 <= kend && j0 + 31 <= t_min) {  // wave-uniform: no masked key
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          sv[e] = (e < 4 ? s0[e] : s1[e - 4]) * scale;
          mx = fmaxf(mx, sv[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = j0 + 8 * qd + e;
          const float raw = e < 4 ? s0[e] : s1[e - 4];
          const bool ok = key >= kbeg && key < kend && key <= pos_t;
          sv[e] = ok ? raw * scale : -INFINITY;
          mx = fmaxf(mx, sv[e]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m, mx);
      float alpha = 1.f, psum = 0.f;
      float p[8];
      if (m_new == -INFINITY) {
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e] = 0.f;
      } else {
        alpha = __expf(m - m_new);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = __expf(sv[e] - m_new);
          psum += p[e];
        }
      }
      psum += __shfl_xor(psum, 16, 64);
      psum += __shfl_xor(psum, 32, 64);
      l = l * alpha + psum;
      m = m_new;
      // once a pair's running max settles, alpha is 1 for the rest of the piece
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) o[dt][rr] *= alpha;
      }
      const u32x4 pbits = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                           pack_bf16x2(p[6], p[7])};
      const bf16x8 pb = __builtin_bit_cast(bf16x8, pbits);
#pragma unroll
      for (int dt = 0; dt < kDT; ++dt) o[dt] = mfma16(__builtin_bit_cast(bf16x8, f.v[dt]), pb, o[dt]);
    };

    // Two fragment buffers alternate: the next 32 keys' loads are issued
    // before the current 32 keys are used, and every load is unconditional
    // (past the piece's keys its last page again, unused), so the wait before
    // a step only covers that step's own loads. The last load is the next
    // piece's first step (or this piece's last page again: unused).
    static_assert(kMaxPieceSteps == 8 && kDT == 16, "a step pair flushes a quarter of the stashed partial");
    int flushed = 0;  // chunks of the previous partial written so far
#pragma unroll
    for (int i = 0; i < kMaxPieceSteps; i += 2) {
      load_kv<NT>(fb, kcache, vcache, page(pg, 2 * i + 2), page(pg, 2 * i + 3), Hkv, cur.kh, col, qd);
      step(fa, kbeg + 32 * i);
      if (i + 2 < cur.steps)
        load_kv<NT>(fa, kcache, vcache, page(pg, 2 * i + 4), page(pg, 2 * i + 5), Hkv, cur.kh, col, qd);
      else
        load_kv<NT>(fa, kcache, vcache, page(npg, 0), page(npg, 1), Hkv, nxt.kh, col, qd);
      flush(i / 2);
      flushed = i / 2 + 1;
      step(fb, kbeg + 32 * (i + 1));
      if (i + 2 >= cur.steps) break;
    }
    for (int k = flushed; k < 4; ++k) flush(k);  // a short piece: the rest of the previous partial
    pend = nullptr;
    if (live) {
      const size_t base = ((size_t(cur.r) * Hkv + cur.kh) * row_groups + cur.rg) * splits + cur.split;
#pragma unroll
      for (int dt = 0; dt < kDT; ++dt) stash[dt * 64 + lane] = o[dt];
      pend = work_o + (base * 16 + col) * kD + 4 * qd;
      if (qd == 0) *reinterpret_cast<float2*>(work_ml + (base * 16 + col) * 2) = float2{m, l};
    }
    if (!has_next) {
      for (int k = 0; k < 4; ++k) flush(k);
      break;
    }
    item = nitem;
    cur = nxt;
    pg = npg;
    load_q(cur, qf);  // from L2: the step's q is 1 MB and read by every piece of its rows
  }
}

// grid (q_heads, tokens), head_dim threads.
constexpr int kMaxCombineSplits = 1024;

__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ work_o,
                                                           const float* __restrict__ work_ml,
                                                           const int32_t* __restrict__ token_row,
                                                           const int32_t* __restrict__ cu_seqlens,
                                                           const bf16_t* __restrict__ qg, int ld_qg, int Hq, int Hkv,
                                                           int D, int row_groups, int splits, int split_len,
                                                           const int32_t* __restrict__ context,
                                                           bf16_t* __restrict__ out) {
  const int h = blockIdx.x, i = blockIdx.y, d = threadIdx.x;
  const int r = token_row[i], t = i - cu_seqlens[r];
  const int group = Hq / Hkv, kh = h / group, pair = t * group + h % group;
  const int rg = pair / 16, col = pair % 16;
  const int ns = (context[r] + split_len - 1) / split_len;
  const size_t base = ((size_t(r) * Hkv + kh) * row_groups + rg) * splits;
  // wave 0 turns the splits' (max, sum) into weights once; then every thread
  // sums its column over the splits with independent loads. The first kPre
  // splits' values and the gate are loaded before the weights are known.
  constexpr int kPre = 8;
  __shared__ float wts[kMaxCombineSplits];
  __shared__ float2 mls[kMaxCombineSplits];  // each split's (max, sum), read once
  __shared__ float sden;
  // a row with no keys (context 0: malformed, no pieces were listed) has
  // ns = 0; its clamped loads stay on its own first split and it writes zeros
  float pre[kPre];
#pragma unroll
  for (int k = 0; k < kPre; ++k) pre[k] = work_o[((base + min(k, max(ns - 1, 0))) * 16 + col) * D + d];
  const float gate = bf16_to_f32(qg[size_t(i) * ld_qg + size_t(h) * 2 * D + D + d]);
  if (d < 64) {
    float M = -INFINITY;
    for (int s0 = 0; s0 < ns; s0 += 64)
      if (s0 + d < ns) {
        const float2 ml = *reinterpret_cast<const float2*>(work_ml + ((base + s0 + d) * 16 + col) * 2);
        mls[s0 + d] = ml;  // read back below by this lane only
        M = fmaxf(M, ml.x);
      }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    float den = 0.f;
    for (int s0 = 0; s0 < ns; s0 += 64) {
      const int s = s0 + d;
      float wgt = 0.f;
      if (s < ns) {
        const float2 ml = mls[s];
        wgt = ml.x == -INFINITY ? 0.f : __expf(ml.x - M);
        den += wgt * ml.y;
        wts[s] = wgt;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) den += __shfl_xor(den, off, 64);
    if (d == 0) sden = den;
  }
  __syncthreads();
  const float den = sden;
  float num = 0.f;
#pragma unroll
  for (int k = 0; k < kPre; ++k)
    if (k < ns) num += wts[k] * pre[k];
#pragma unroll 8
  for (int s = kPre; s < ns; ++s) num += wts[s] * work_o[((base + s) * 16 + col) * D + d];
  const float y = den > 0.f ? num / den : 0.f;
  out[(size_t(i) * Hq + h) * D + d] = f32_to_bf16(y / (1.f + __expf(-gate)));
}

}  // namespace

void attn_prep(const bf16_t* qg, int ld_qg, const bf16_t* kv, int ld_kv, int kv_off, const float* q_norm,
               const float* k_norm, const int32_t* token_pos, const int32_t* kv_slot, int tokens, const AttnGeom& g,
               bf16_t* qout, bf16_t* kcache, bf16_t* vcache, hipStream_t stream) {
  require(g.head_dim % 64 == 0 && g.head_dim <= 256, "attn_prep: head_dim must be a multiple of 64, <= 256");
  require(g.rotary > 0 && g.rotary <= g.head_dim && (g.rotary / 2) % (g.head_dim / 64) == 0,
          "attn_prep: unsupported rotary width");
  require(g.q_heads % g.kv_heads == 0, "attn_prep: q_heads % kv_heads");
  if (tokens <= 0) return;
  hipLaunchKernelGGL(attn_prep_kernel, dim3(g.q_heads + 2 * g.kv_heads, tokens), dim3(64), 0, stream, qg, ld_qg, kv,
                     ld_kv, kv_off, q_norm, k_norm, token_pos, kv_slot, g, qout, kcache, vcache);
  HB_CHECK(hipGetLastError());
}

size_t attn_work_floats_o(int rows, int kv_heads, int head_dim, int max_tokens, int group, int max_context,
                          int split_len) {
  const int rgs = (max_tokens * group + 15) / 16;
  const int splits = (max_context + split_len - 1) / split_len;
  return size_t(rows) * kv_heads * rgs * splits * 16 * head_dim;
}

size_t attn_plan_ints(int rows, int kv_heads, int row_groups, int splits) {
  return 2 + 2 * size_t(rows) * kv_heads * row_groups * splits;
}

void attn_plan(const int32_t* cu_seqlens, const int32_t* context, const AttnGeom& g, const AttnWork& w,
               hipStream_t stream) {
  require(w.rows > 0 && w.rows <= kPlanMaxRows && w.row_groups > 0 && w.row_groups < 32768 && w.splits > 0 &&
              w.split_len > 0 && w.split_len <= kPlanBuckets && w.plan,
          "attn_plan: invalid work geometry (at most 2048 rows, split_len <= 256)");
  hipLaunchKernelGGL(attn_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, cu_seqlens, context, w.rows,
                     g.q_heads / g.kv_heads, w.row_groups, w.splits, w.split_len, g.kv_heads, w.plan);
  HB_CHECK(hipGetLastError());
}

void paged_attention(const bf16_t* q, const bf16_t* kcache, const bf16_t* vcache, const int32_t* block_table,
                     int max_pages, const int32_t* cu_seqlens, const int32_t* context, const AttnGeom& g, float scale,
                     const AttnWork& w, hipStream_t stream) {
  require(g.head_dim == kD, "paged_attention: head_dim 256 only");
  require(w.split_len > 0 && w.split_len % 32 == 0 && w.split_len <= 32 * kMaxPieceSteps,
          "paged_attention: split_len must be a multiple of 32, at most 256");
  require(w.row_groups * 16 >= w.max_tokens * (g.q_heads / g.kv_heads), "paged_attention: row groups");
  // persistent: one wave per SIMD (the kernel holds one wave's registers per
  // SIMD), never more waves than pieces could need
  static int slots = 0;
  if (!slots) {
    int dev = 0, cus = 0;
    HB_CHECK(hipGetDevice(&dev));
    HB_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    slots = 4 * cus;
  }
  const size_t most = size_t(w.rows) * g.kv_heads * w.row_groups * w.splits;
  const int grid = int(std::min<size_t>(most, size_t(slots)));
  const bool one_group = w.max_tokens * (g.q_heads / g.kv_heads) <= 16;
  launch_timed(one_group ? paged_attn_kernel<true> : paged_attn_kernel<false>, dim3(grid), dim3(64), 0, stream, q,
               kcache, vcache, block_table, max_pages, cu_seqlens, context, g.q_heads, g.kv_heads, scale, w.row_groups,
               w.splits, w.split_len, w.plan, w.work_o, w.work_ml);
  HB_CHECK(hipGetLastError());
}

void attn_combine(const AttnWork& w, const int32_t* token_row, const int32_t* cu_seqlens, const int32_t* context,
                  const bf16_t* qg, int ld_qg, int tokens, const AttnGeom& g, bf16_t* out, hipStream_t stream) {
  require(w.splits <= kMaxCombineSplits && g.head_dim >= 64 && g.head_dim <= 256,
          "attn_combine: at most 1024 splits and a head_dim of 64..256");
  if (tokens <= 0) return;
  launch_timed(attn_combine_kernel, dim3(g.q_heads, tokens), dim3(g.head_dim), 0, stream, w.work_o, w.work_ml,
               token_row, cu_seqlens, qg, ld_qg, g.q_heads, g.kv_heads, g.head_dim, w.row_groups, w.splits,
               w.split_len, context, out);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
