// Greedy selection (argmax + margin under f32 total order) and MTP acceptance.
#include <mutex>
#include <vector>

#include "select.h"
#include "select_device.h"

namespace hb {
namespace {

constexpr int kSelThreads = 256;

__global__ __launch_bounds__(kSelThreads) void argmax_margin_kernel(const float* __restrict__ logits, int ld,
                                                                    int vocab, uint32_t* __restrict__ winner,
                                                                    float* __restrict__ margin,
                                                                    int32_t* __restrict__ status) {
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* row = logits + size_t(r) * ld;
  Top2 t{0u, 0xFFFFFFFFu, 0u, false};
  int bad = 0;
  for (int i = tid; i < vocab; i += kSelThreads) {
    const float v = row[i];
    if (!isfinite(v)) bad = 1;
    const Top2 one{total_key(v), uint32_t(i), 0u, false};
    t = merge(t, one);
  }
  __shared__ Top2 part[kSelThreads];
  __shared__ int sbad[kSelThreads];
  part[tid] = t;
  sbad[tid] = bad;
  __syncthreads();
  for (int s = kSelThreads / 2; s > 0; s >>= 1) {
    if (tid < s) {
      part[tid] = merge(part[tid], part[tid + s]);
      sbad[tid] |= sbad[tid + s];
    }
    __syncthreads();
  }
  if (tid == 0) {
    const Top2 f = part[0];
    winner[r] = f.i1;
    const float best = key_value(f.k1);
    margin[r] = f.has2 ? best - key_value(f.k2) : INFINITY;
    status[r] = sbad[0];
  }
}

// Two-level variant for long rows: grid (chunks, rows), each workgroup scans
// kSelChunk columns and leaves its (best, second, non-finite) in part[row][chunk];
// one thread per row then merges the chunks in column order.
constexpr int kSelChunk = 8192;

__global__ __launch_bounds__(kSelThreads) void argmax_partial_kernel(const float* __restrict__ logits, int ld,
                                                                     int vocab, int nchunk,
                                                                     uint4* __restrict__ part) {
  const int chunk = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
  const float* row = logits + size_t(r) * ld;
  const int c0 = chunk * kSelChunk, c1 = min(vocab, c0 + kSelChunk);
  Top2 t{0u, 0xFFFFFFFFu, 0u, false};
  int bad = 0;
  for (int i = c0 + tid; i < c1; i += kSelThreads) {
    const float v = row[i];
    if (!isfinite(v)) bad = 1;
    t = merge(t, Top2{total_key(v), uint32_t(i), 0u, false});
  }
  __shared__ Top2 sp[kSelThreads];
  __shared__ int sb[kSelThreads];
  sp[tid] = t;
  sb[tid] = bad;
  __syncthreads();
  for (int s = kSelThreads / 2; s > 0; s >>= 1) {
    if (tid < s) {
      sp[tid] = merge(sp[tid], sp[tid + s]);
      sb[tid] |= sb[tid + s];
    }
    __syncthreads();
  }
  if (tid == 0) part[size_t(r) * nchunk + chunk] = make_uint4(sp[0].k1, sp[0].i1, sp[0].k2, (sp[0].has2 ? 1u : 0u) | (sb[0] ? 2u : 0u));
}

__global__ void argmax_final_kernel(const uint4* __restrict__ part, int nchunk, int rows, uint32_t* __restrict__ winner,
                                    float* __restrict__ margin, int32_t* __restrict__ status) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  Top2 t{0u, 0xFFFFFFFFu, 0u, false};
  int bad = 0;
  for (int c = 0; c < nchunk; ++c) {
    const uint4 p = part[size_t(r) * nchunk + c];
    t = merge(t, Top2{p.x, p.y, p.z, (p.w & 1u) != 0});
    bad |= (p.w & 2u) != 0;
  }
  winner[r] = t.i1;
  margin[r] = t.has2 ? key_value(t.k1) - key_value(t.k2) : INFINITY;
  status[r] = bad;
}

__global__ void mtp_plan_kernel(const uint32_t* __restrict__ draft, const int32_t* __restrict__ n_draft,
                                int max_draft, const uint32_t* __restrict__ target, const uint32_t* __restrict__ eos,
                                int n_eos, const int32_t* __restrict__ remaining, int rows, int vocab,
                                uint32_t* __restrict__ emitted, int32_t* __restrict__ n_emitted,
                                int32_t* __restrict__ accepted, int32_t* __restrict__ terminal,
                                int32_t* __restrict__ status) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int n = n_draft[r], rem = remaining[r];
  const uint32_t* d = draft + size_t(r) * max_draft;
  const uint32_t* tg = target + size_t(r) * (max_draft + 1);
  uint32_t* out = emitted + size_t(r) * (max_draft + 1);
  bool bad = n < 0 || n > 8 || n > max_draft || rem <= 0 || n > rem;
  for (int i = 0; i < n_eos; ++i) bad |= eos[i] >= uint32_t(vocab);
  if (!bad)
    for (int i = 0; i < n; ++i) bad |= d[i] >= uint32_t(vocab);
  for (int i = 0; !bad && i <= n; ++i) bad |= tg[i] >= uint32_t(vocab);
  status[r] = bad;
  if (bad) {
    n_emitted[r] = 0;
    accepted[r] = 0;
    terminal[r] = 0;
    return;
  }
  auto is_eos = [&](uint32_t t) {
    for (int i = 0; i < n_eos; ++i)
      if (eos[i] == t) return true;
    return false;
  };
  int ne = 0, acc = 0;
  bool term = false;
  for (int i = 0; i < n; ++i) {
    const uint32_t tgt = tg[i];
    out[ne++] = tgt;
    term = is_eos(tgt);
    if (d[i] != tgt || term) {
      acc += d[i] == tgt;
      n_emitted[r] = ne;
      accepted[r] = acc;
      terminal[r] = term;
      return;
    }
    acc += 1;
  }
  if (ne < rem) {
    const uint32_t bonus = tg[n];
    out[ne++] = bonus;
    term = is_eos(bonus);
  }
  n_emitted[r] = ne;
  accepted[r] = acc;
  terminal[r] = term;
}

}  // namespace

// Partial summaries of the allocation-free selection: one uint4 per (row,
// chunk). Each GPU the library runs on holds its own copy until the process
// ends. Host code never names it: its device address comes from
// hipGetSymbolAddress, once per device (select_scratch below).
static __device__ __align__(256) uint4 scratch[kSelectScratchBytes / sizeof(uint4)];

void* select_scratch() {
  static std::mutex lock;
  static std::vector<void*> address;  // per device ordinal
  int dev = 0;
  HB_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> hold(lock);
  if (size_t(dev) >= address.size()) address.resize(size_t(dev) + 1, nullptr);
  if (!address[dev]) {
    void* p = nullptr;
    HB_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    require(p != nullptr, "select scratch: no device address");
    address[dev] = p;
  }
  return address[dev];
}

size_t argmax_workspace_bytes(int rows, int vocab) {
  return size_t(rows) * ((vocab + kSelChunk - 1) / kSelChunk) * sizeof(uint4);
}

void argmax_margin(const float* logits, int ld, int rows, int vocab, uint32_t* winner, float* margin,
                   int32_t* status, hipStream_t stream, void* workspace) {
  require(logits && winner && margin && status, "argmax_margin: null pointer");
  require(vocab > 0 && ld >= vocab, "argmax_margin: invalid vocabulary");
  if (rows <= 0) return;
  const int nchunk = (vocab + kSelChunk - 1) / kSelChunk;
  if (workspace && nchunk > 1) {
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(nchunk, rows), dim3(kSelThreads), 0, stream, logits, ld, vocab,
                       nchunk, static_cast<uint4*>(workspace));
    HB_CHECK(hipGetLastError());
    hipLaunchKernelGGL(argmax_final_kernel, dim3((rows + 63) / 64), dim3(64), 0, stream,
                       static_cast<const uint4*>(workspace), nchunk, rows, winner, margin, status);
    HB_CHECK(hipGetLastError());
    return;
  }
  hipLaunchKernelGGL(argmax_margin_kernel, dim3(rows), dim3(kSelThreads), 0, stream, logits, ld, vocab, winner,
                     margin, status);
  HB_CHECK(hipGetLastError());
}

void mtp_plan(const uint32_t* draft, const int32_t* n_draft, int max_draft, const uint32_t* target,
              const uint32_t* eos, int n_eos, const int32_t* remaining, int rows, int vocab, uint32_t* emitted,
              int32_t* n_emitted, int32_t* accepted, int32_t* terminal, int32_t* status, hipStream_t stream) {
  require(draft && n_draft && target && remaining && emitted && n_emitted && accepted && terminal && status,
          "mtp_plan: null pointer");
  require(max_draft >= 1 && max_draft <= 8 && n_eos >= 0 && (n_eos == 0 || eos), "mtp_plan: invalid descriptor");
  if (rows <= 0) return;
  hipLaunchKernelGGL(mtp_plan_kernel, dim3((rows + 63) / 64), dim3(64), 0, stream, draft, n_draft, max_draft, target,
                     eos, n_eos, remaining, rows, vocab, emitted, n_emitted, accepted, terminal, status);
  HB_CHECK(hipGetLastError());
}

}  // namespace hb
