// Memory-rate probes of the device (no reference counterpart): a plain
// streaming read and a streaming copy, launched by the benchmark beside the
// kernels it measures so their rates can be read against what the device's
// memory system delivers for the same bytes and the same launch pattern.
#include "hb_common.h"

namespace hb {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;  // 16-byte loads in flight per thread and iteration

template <bool NT>
__device__ inline uint4 probe_load(const uint4* p) {
  if constexpr (NT) {
    using v4u = unsigned __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return uint4{v.x, v.y, v.z, v.w};
  } else {
    return *p;
  }
}

// Grid-stride read of n uint4; each wave XOR-folds what it read into one
// word of `sink` (blocks x waves words), so no load can be dropped.
template <bool NT>
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const uint4* __restrict__ src, size_t n,
                                                                    uint32_t* __restrict__ sink) {
  const size_t stride = size_t(gridDim.x) * kProbeThreads;
  size_t i = size_t(blockIdx.x) * kProbeThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kProbeUnroll - 1) * stride < n; i += kProbeUnroll * stride) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = probe_load<NT>(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n; i += stride) {
    const uint4 v = probe_load<NT>(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) sink[size_t(blockIdx.x) * (kProbeThreads / 64) + threadIdx.x / 64] = acc;
}

// Grid-stride copy of n uint4 with streaming loads and stores.
__global__ __launch_bounds__(kProbeThreads) void stream_copy_kernel(uint4* __restrict__ dst,
                                                                    const uint4* __restrict__ src, size_t n) {
  using v4u = unsigned __attribute__((ext_vector_type(4)));
  const size_t stride = size_t(gridDim.x) * kProbeThreads;
  size_t i = size_t(blockIdx.x) * kProbeThreads + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * stride < n; i += kProbeUnroll * stride) {
    v4u v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + i + u * stride));
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) __builtin_nontemporal_store(v[u], reinterpret_cast<v4u*>(dst + i + u * stride));
  }
  for (; i < n; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + i)),
                                reinterpret_cast<v4u*>(dst + i));
}

// Chunked forms: workgroup b reads (copies) the contiguous chunk [b per, (b + 1)
// per) of uint4, 16 loads in flight per thread (64 KiB per workgroup), as a
// kernel that owns a block of state per workgroup does. per % 4096 == 0.
constexpr int kChunkUnroll = 16;
template <bool NT>
__global__ __launch_bounds__(kProbeThreads) void chunk_read_kernel(const uint4* __restrict__ src, size_t per,
                                                                   uint32_t* __restrict__ sink) {
  const uint4* c = src + size_t(blockIdx.x) * per;
  uint32_t acc = 0;
  for (size_t j = threadIdx.x; j < per; j += kProbeThreads * kChunkUnroll) {
    uint4 v[kChunkUnroll];
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u) v[u] = probe_load<NT>(c + j + u * kProbeThreads);
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) sink[size_t(blockIdx.x) * (kProbeThreads / 64) + threadIdx.x / 64] = acc;
}

__global__ __launch_bounds__(kProbeThreads) void chunk_copy_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                                   size_t per) {
  using v4u = unsigned __attribute__((ext_vector_type(4)));
  const size_t c = size_t(blockIdx.x) * per;
  for (size_t j = threadIdx.x; j < per; j += kProbeThreads * kChunkUnroll) {
    v4u v[kChunkUnroll];
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u)
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + c + j + u * kProbeThreads));
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u)
      __builtin_nontemporal_store(v[u], reinterpret_cast<v4u*>(dst + c + j + u * kProbeThreads));
  }
}

}  // namespace
}  // namespace hb

using namespace hb;

extern "C" size_t hb_stream_read_sink_bytes(int blocks) {
  return blocks > 0 ? size_t(blocks) * (kProbeThreads / 64) * sizeof(uint32_t) : 0;
}

extern "C" int hb_stream_read(const void* src, size_t bytes, void* sink, int blocks, int nontemporal, void* stream,
                              char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(src && sink, "hb_stream_read: null pointer");
    require(bytes > 0 && bytes % 16 == 0, "hb_stream_read: bytes must be a positive multiple of 16");
    require(blocks > 0 && blocks <= 65536, "hb_stream_read: blocks must be in 1..65536");
    const auto* s = static_cast<const uint4*>(src);
    auto* k = static_cast<uint32_t*>(sink);
    if (nontemporal)
      hipLaunchKernelGGL(stream_read_kernel<true>, dim3(blocks), dim3(kProbeThreads), 0, as_stream(stream), s,
                         bytes / 16, k);
    else
      hipLaunchKernelGGL(stream_read_kernel<false>, dim3(blocks), dim3(kProbeThreads), 0, as_stream(stream), s,
                         bytes / 16, k);
    HB_CHECK(hipGetLastError());
  });
}

extern "C" int hb_stream_copy(void* dst, const void* src, size_t bytes, int blocks, void* stream, char* error,
                              size_t capacity) {
  return guarded(error, capacity, [&] {
    require(dst && src, "hb_stream_copy: null pointer");
    require(bytes > 0 && bytes % 16 == 0, "hb_stream_copy: bytes must be a positive multiple of 16");
    require(blocks > 0 && blocks <= 65536, "hb_stream_copy: blocks must be in 1..65536");
    hipLaunchKernelGGL(stream_copy_kernel, dim3(blocks), dim3(kProbeThreads), 0, as_stream(stream),
                       static_cast<uint4*>(dst), static_cast<const uint4*>(src), bytes / 16);
    HB_CHECK(hipGetLastError());
  });
}

extern "C" int hb_stream_read_chunked(const void* src, size_t bytes, size_t chunk_bytes, void* sink, int nontemporal,
                                      void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(src && sink, "hb_stream_read_chunked: null pointer");
    require(chunk_bytes > 0 && chunk_bytes % (16 * kProbeThreads * kChunkUnroll) == 0,
            "hb_stream_read_chunked: chunk_bytes must be a positive multiple of 64 KiB");
    require(bytes > 0 && bytes % chunk_bytes == 0 && bytes / chunk_bytes <= 65536,
            "hb_stream_read_chunked: bytes must be 1..65536 chunks");
    const int blocks = int(bytes / chunk_bytes);
    const auto* s = static_cast<const uint4*>(src);
    auto* k = static_cast<uint32_t*>(sink);
    if (nontemporal)
      hipLaunchKernelGGL(chunk_read_kernel<true>, dim3(blocks), dim3(kProbeThreads), 0, as_stream(stream), s,
                         chunk_bytes / 16, k);
    else
      hipLaunchKernelGGL(chunk_read_kernel<false>, dim3(blocks), dim3(kProbeThreads), 0, as_stream(stream), s,
                         chunk_bytes / 16, k);
    HB_CHECK(hipGetLastError());
  });
}

extern "C" int hb_stream_copy_chunked(void* dst, const void* src, size_t bytes, size_t chunk_bytes, void* stream,
                                      char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(dst && src, "hb_stream_copy_chunked: null pointer");
    require(chunk_bytes > 0 && chunk_bytes % (16 * kProbeThreads * kChunkUnroll) == 0,
            "hb_stream_copy_chunked: chunk_bytes must be a positive multiple of 64 KiB");
    require(bytes > 0 && bytes % chunk_bytes == 0 && bytes / chunk_bytes <= 65536,
            "hb_stream_copy_chunked: bytes must be 1..65536 chunks");
    hipLaunchKernelGGL(chunk_copy_kernel, dim3(int(bytes / chunk_bytes)), dim3(kProbeThreads), 0, as_stream(stream),
                       static_cast<uint4*>(dst), static_cast<const uint4*>(src), chunk_bytes / 16);
    HB_CHECK(hipGetLastError());
  });
}
