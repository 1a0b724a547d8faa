// Additive device-pointer entry points (hb_*). Plumbing (memory, streams,
// events) plus one entry per hot-path operator.
#include "../../include/hip_bridge.h"
#include "hb_common.h"
#include "qmm.h"

using namespace hb;

extern "C" int hb_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

extern "C" const char* hb_device_name(int device) {
  static thread_local hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return "";
  return prop.gcnArchName;
}

extern "C" void* hb_malloc(size_t bytes, char* error, size_t capacity) {
  void* p = nullptr;
  int rc = guarded(error, capacity, [&] {
    require(bytes > 0, "hb_malloc: zero bytes");
    HB_CHECK(hipMalloc(&p, bytes));
  });
  return rc ? nullptr : p;
}

extern "C" int hb_free(void* ptr) { return ptr && hipFree(ptr) != hipSuccess ? -1 : 0; }

extern "C" int hb_memcpy_h2d(void* dst, const void* src, size_t bytes, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(dst && src, "hb_memcpy_h2d: null pointer");
    HB_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  });
}

extern "C" int hb_memcpy_d2h(void* dst, const void* src, size_t bytes, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(dst && src, "hb_memcpy_d2h: null pointer");
    HB_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  });
}

extern "C" int hb_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(dst && src, "hb_memcpy_d2d: null pointer");
    HB_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
  });
}

extern "C" int hb_memset(void* ptr, int value, size_t bytes, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(ptr != nullptr, "hb_memset: null pointer");
    HB_CHECK(hipMemsetAsync(ptr, value, bytes, as_stream(stream)));
  });
}

extern "C" int hb_synchronize(void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    if (stream)
      HB_CHECK(hipStreamSynchronize(as_stream(stream)));
    else
      HB_CHECK(hipDeviceSynchronize());
  });
}

extern "C" void* hb_stream_create(char* error, size_t capacity) {
  hipStream_t s = nullptr;
  int rc = guarded(error, capacity, [&] { HB_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); });
  return rc ? nullptr : static_cast<void*>(s);
}

extern "C" void hb_stream_destroy(void* stream) {
  if (stream) (void)hipStreamDestroy(as_stream(stream));
}

extern "C" void* hb_event_create(char* error, size_t capacity) {
  hipEvent_t e = nullptr;
  int rc = guarded(error, capacity, [&] { HB_CHECK(hipEventCreate(&e)); });
  return rc ? nullptr : static_cast<void*>(e);
}

extern "C" void hb_event_destroy(void* event) {
  if (event) (void)hipEventDestroy(static_cast<hipEvent_t>(event));
}

extern "C" int hb_event_record(void* event, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(event != nullptr, "hb_event_record: null event");
    HB_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)));
  });
}

extern "C" int hb_event_elapsed(void* start, void* end, float* ms, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(start && end && ms, "hb_event_elapsed: null argument");
    HB_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(end)));
    float v = 0.f;
    HB_CHECK(hipEventElapsedTime(&v, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
    *ms = v;
  });
}

extern "C" int hb_graph_begin(void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(stream != nullptr, "hb_graph_begin: capture needs a created stream");
    HB_CHECK(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
  });
}

extern "C" void* hb_graph_end(void* stream, char* error, size_t capacity) {
  hipGraphExec_t exec = nullptr;
  int rc = guarded(error, capacity, [&] {
    require(stream != nullptr, "hb_graph_end: null stream");
    hipGraph_t graph = nullptr;
    HB_CHECK(hipStreamEndCapture(as_stream(stream), &graph));
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HB_CHECK(e);
  });
  return rc ? nullptr : static_cast<void*>(exec);
}

extern "C" int hb_graph_launch(void* graph_exec, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    require(graph_exec != nullptr, "hb_graph_launch: null graph");
    HB_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
  });
}

extern "C" void hb_graph_destroy(void* graph_exec) {
  if (graph_exec) (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec));
}

extern "C" int hb_q4_tile(const uint32_t* w, const void* scales, const void* biases, uint32_t* w_tiled,
                          void* sb_tiled, int N, int K, void* stream, char* error, size_t capacity) {
  return guarded(error, capacity, [&] {
    q4_tile(w, static_cast<const bf16_t*>(scales), static_cast<const bf16_t*>(biases), w_tiled,
            static_cast<bf16_t*>(sb_tiled), N, K, as_stream(stream));
  });
}

extern "C" int hb_qmm(const void* x, const uint32_t* w, const void* scales, const void* biases, void* y, int M, int N,
                      int K, int group, int bits, int layout, int y_f32, int ldy, void* stream, char* error,
                      size_t capacity) {
  return guarded(error, capacity, [&] {
    qmm(static_cast<const bf16_t*>(x), M, K, w, static_cast<const bf16_t*>(scales),
        static_cast<const bf16_t*>(biases), N, group, bits, layout, y, y_f32, ldy, as_stream(stream));
  });
}
