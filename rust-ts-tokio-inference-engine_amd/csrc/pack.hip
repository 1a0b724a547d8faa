// Ragged packing tables for one continuous-batching step.
//
// The reference packer (native/qwen_batch.inc:2-50) concatenates the state of
// up to three equal-position rows; here rows carry different token counts
// (1 decode, up to 4 MTP verify, 64-token prefill chunks) and positions, so the
// step is described by tables built on the device:
//   cu_seqlens[r+1] = cu_seqlens[r] + row_tokens[r]        (exclusive prefix sum)
//   token_row[i] = r, token_pos[i] = positions[r] + j       (i = cu_seqlens[r] + j)
//   kv_slot[i]   = block_table[r][pos / page] * page + pos % page
//   context[r]   = positions[r] + row_tokens[r]
// One workgroup: each wave scans 64 row counts with DPP-free shuffles, wave
// totals are scanned in LDS, then every thread expands its rows.
#include "pack.h"

namespace hb {
namespace {

constexpr int kPackThreads = 1024;

__device__ inline int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

__global__ __launch_bounds__(kPackThreads) void pack_tables_kernel(
    const int32_t* __restrict__ row_tokens, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ block_table, int max_pages, int rows, int page, int32_t* __restrict__ cu_seqlens,
    int32_t* __restrict__ token_row, int32_t* __restrict__ token_pos, int32_t* __restrict__ kv_slot,
    int32_t* __restrict__ context, int32_t* __restrict__ status) {
  __shared__ int wave_sums[kPackThreads / 64];
  __shared__ int carry;
  __shared__ int bad;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) {
    carry = 0;
    bad = 0;
    cu_seqlens[0] = 0;
  }
  __syncthreads();
  for (int base = 0; base < rows; base += kPackThreads) {
    const int r = base + tid;
    const int t = r < rows ? row_tokens[r] : 0;
    const int pos = r < rows ? positions[r] : 0;
    if (r < rows && (t < 0 || pos < 0 || int64_t(pos) + t > int64_t(max_pages) * page)) atomicOr(&bad, 1);
    const int inc = wave_inclusive_scan(t, lane);
    if (lane == 63) wave_sums[wave] = inc;
    __syncthreads();
    if (wave == 0) {
      const int ws = lane < kPackThreads / 64 ? wave_sums[lane] : 0;
      const int ws_inc = wave_inclusive_scan(ws, lane);
      if (lane < kPackThreads / 64) wave_sums[lane] = ws_inc - ws;  // exclusive offsets of the waves
    }
    __syncthreads();
    const int start = carry + wave_sums[wave] + inc - t;
    if (r < rows) {
      cu_seqlens[r + 1] = start + t;
      context[r] = pos + t;
    }
    __syncthreads();
    if (tid == kPackThreads - 1) carry = start + t;
    __syncthreads();
    if (r < rows && !bad) {
      for (int j = 0; j < t; ++j) {
        const int i = start + j, p = pos + j;
        token_row[i] = r;
        token_pos[i] = p;
        kv_slot[i] = block_table[size_t(r) * max_pages + p / page] * page + p % page;
      }
    }
  }
  __syncthreads();
  if (tid == 0) status[0] = bad;
}

// grid (pairs, pools): one workgroup moves one page of one pool in 16-byte pieces.
__global__ __launch_bounds__(256) void page_copy_kernel(bf16_t* const* __restrict__ pools,
                                                        const int32_t* __restrict__ pairs, int n, int page_elems,
                                                        bf16_t* __restrict__ gather) {
  const int i = blockIdx.x, p = blockIdx.y;
  const uint4* src = reinterpret_cast<const uint4*>(pools[p] + size_t(pairs[2 * i]) * page_elems);
  uint4* dst = reinterpret_cast<uint4*>(gather ? gather + (size_t(p) * n + i) * page_elems
                                               : pools[p] + size_t(pairs[2 * i + 1]) * page_elems);
  for (int j = threadIdx.x; j < page_elems / 8; j += blockDim.x) dst[j] = src[j];
}

}  // namespace

void copy_pages(bf16_t* const* pools, int n_pools, const int32_t* pairs, int n, int page_elems, bf16_t* gather,
                hipStream_t stream) {
  require(pools && pairs && n_pools > 0 && page_elems > 0 && page_elems % 8 == 0, "copy_pages: invalid geometry");
  if (n == 0) return;
  hipLaunchKernelGGL(page_copy_kernel, dim3(n, n_pools), dim3(256), 0, stream, pools, pairs, n, page_elems, gather);
  HB_CHECK(hipGetLastError());
}

void pack_tables(const int32_t* row_tokens, const int32_t* positions, const int32_t* block_table, int max_pages,
                 int rows, int page, int32_t* cu_seqlens, int32_t* token_row, int32_t* token_pos, int32_t* kv_slot,
                 int32_t* context, int32_t* status, hipStream_t stream) {
  require(row_tokens && positions && block_table && cu_seqlens && token_row && token_pos && kv_slot && context &&
              status,
          "pack_tables: null pointer");
  require(rows > 0 && max_pages > 0 && page > 0, "pack_tables: invalid geometry");
  hipLaunchKernelGGL(pack_tables_kernel, dim3(1), dim3(kPackThreads), 0, stream, row_tokens, positions, block_table,
                     max_pages, rows, page, cu_seqlens, token_row, token_pos, kv_slot, context, status);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
