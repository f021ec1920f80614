// Library runtime: error state, version, staging casts, hipGraph
// record/replay and the bounded stream wait.
#include "q4mi_common.h"

#include <chrono>
#include <thread>

namespace q4 {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
void clear_error() { g_err[0] = 0; }

// Plan overrides (q4_tune_set): -1 = none. Plain ints: the planners read them
// on the host before each launch.
static int g_tune[Q4_TUNE_COUNT] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, -1};
int tune_value(int knob) { return knob >= 0 && knob < Q4_TUNE_COUNT ? g_tune[knob] : -1; }

// f32 -> f16 (RNE) and f16 -> f32 staging casts, 4 elements per thread.
__global__ void cast_f32_f16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst, size_t n) {
  size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n) {
    float4 v = *reinterpret_cast<const float4*>(src + i);
    ushort4 o;
    o.x = f2h(v.x); o.y = f2h(v.y); o.z = f2h(v.z); o.w = f2h(v.w);
    *reinterpret_cast<ushort4*>(dst + i) = o;
  } else {
    for (; i < n; ++i) dst[i] = f2h(src[i]);
  }
}

__global__ void cast_f16_f32_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst, size_t n) {
  size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n) {
    ushort4 v = *reinterpret_cast<const ushort4*>(src + i);
    float4 o;
    o.x = h2f(v.x); o.y = h2f(v.y); o.z = h2f(v.z); o.w = h2f(v.w);
    *reinterpret_cast<float4*>(dst + i) = o;
  } else {
    for (; i < n; ++i) dst[i] = h2f(src[i]);
  }
}

}  // namespace q4

using namespace q4;

extern "C" {

const char* q4_version(void) { return "q4mi 0.1.0 gfx950"; }

const char* q4_last_error(void) { return g_err; }

int q4_tune_set(int knob, int value) {
  clear_error();
  Q4_ARG(knob >= 0 && knob < Q4_TUNE_COUNT, "unknown tuning knob %d", knob);
  g_tune[knob] = value < 0 ? -1 : value;
  return Q4_OK;
}

int q4_tune_get(int knob) { return tune_value(knob); }

void q4_tune_reset(void) {
  for (int& v : g_tune) v = -1;
}

int q4_dev_bytes(int N, int K, size_t* wq_bytes, size_t* scale_elems) {
  clear_error();
  Q4_ARG(N > 0 && K > 0 && K % BLK == 0, "bad shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
  size_t units = (size_t)pad_rows(N) * (K / BLK);
  if (wq_bytes) *wq_bytes = units * 16;
  if (scale_elems) *scale_elems = units;
  return Q4_OK;
}

int q4_cast_f32_f16(const float* src, uint16_t* dst, size_t n, void* stream) {
  clear_error();
  Q4_ARG(src && dst, "null pointer");
  Q4_ARG(((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 7) == 0, "misaligned cast buffers");
  if (n == 0) return Q4_OK;
  size_t threads = (n + 3) / 4;
  unsigned grid = (unsigned)((threads + 255) / 256);
  hipLaunchKernelGGL(cast_f32_f16_kernel, dim3(grid), dim3(256), 0, as_stream(stream), src, dst, n);
  Q4_LAUNCHED("cast_f32_f16");
  return Q4_OK;
}

int q4_cast_f16_f32(const uint16_t* src, float* dst, size_t n, void* stream) {
  clear_error();
  Q4_ARG(src && dst, "null pointer");
  Q4_ARG(((uintptr_t)src & 7) == 0 && ((uintptr_t)dst & 15) == 0, "misaligned cast buffers");
  if (n == 0) return Q4_OK;
  size_t threads = (n + 3) / 4;
  unsigned grid = (unsigned)((threads + 255) / 256);
  hipLaunchKernelGGL(cast_f16_f32_kernel, dim3(grid), dim3(256), 0, as_stream(stream), src, dst, n);
  Q4_LAUNCHED("cast_f16_f32");
  return Q4_OK;
}

int q4_graph_begin(void* stream) {
  clear_error();
  Q4_ARG(stream != nullptr, "graph capture needs a non-null stream");
  Q4_HIP(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
  return Q4_OK;
}

int q4_graph_end(void* stream, void** graph_exec) {
  clear_error();
  Q4_ARG(stream != nullptr && graph_exec != nullptr, "null stream or output pointer");
  hipGraph_t g = nullptr;
  Q4_HIP(hipStreamEndCapture(as_stream(stream), &g));
  hipGraphExec_t ge = nullptr;
  hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    set_error("hipGraphInstantiate failed: %s", hipGetErrorString(e));
    return Q4_ERR_HIP;
  }
  *graph_exec = (void*)ge;
  return Q4_OK;
}

int q4_graph_launch(void* graph_exec, void* stream) {
  clear_error();
  Q4_ARG(graph_exec != nullptr, "null graph");
  Q4_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, as_stream(stream)));
  return Q4_OK;
}

// GPU timestamps: slot i of a device array takes the constant-rate wall
// clock (s_memrealtime) when a one-wave stamp launch runs. Stream-ordered
// like any launch, so inside a stream capture it is a node of the graph and
// every replay stamps again. The host reads the array back after the wait.
struct Timestamps {
  int n;
  unsigned long long* dev;
  double khz;
};

}  // extern "C"

namespace q4 {
__global__ void __launch_bounds__(64) stamp_kernel(unsigned long long* __restrict__ t, int i) {
  if (threadIdx.x == 0) t[i] = wall_clock64();
}
}  // namespace q4

extern "C" {

int q4_timestamps_create(int n, void** ts) {
  clear_error();
  Q4_ARG(n >= 2 && n <= (1 << 16) && ts, "timestamps: 2..65536 slots and an output pointer");
  int dev = 0, khz = 0;
  Q4_HIP(hipGetDevice(&dev));
  Q4_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  Q4_ARG(khz > 0, "no wall clock rate");
  unsigned long long* d = nullptr;
  Q4_HIP(hipMalloc(&d, (size_t)n * sizeof(unsigned long long)));
  hipError_t e = hipMemset(d, 0, (size_t)n * sizeof(unsigned long long));
  if (e != hipSuccess) {
    (void)hipFree(d);
    set_error("hipMemset failed: %s", hipGetErrorString(e));
    return Q4_ERR_HIP;
  }
  *ts = new Timestamps{n, d, (double)khz};
  return Q4_OK;
}

int q4_timestamp_record(void* ts, int i, void* stream) {
  clear_error();
  Timestamps* t = reinterpret_cast<Timestamps*>(ts);
  Q4_ARG(t && i >= 0 && i < t->n, "timestamp index %d out of range", i);
  hipLaunchKernelGGL(stamp_kernel, dim3(1), dim3(64), 0, as_stream(stream), t->dev, i);
  Q4_LAUNCHED("stamp");
  return Q4_OK;
}

int q4_timestamps_read(void* ts, double* ms) {
  clear_error();
  Timestamps* t = reinterpret_cast<Timestamps*>(ts);
  Q4_ARG(t && ms, "null pointer");
  unsigned long long* h = new unsigned long long[t->n];
  const hipError_t e = hipMemcpy(h, t->dev, (size_t)t->n * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  if (e == hipSuccess)
    for (int i = 0; i < t->n; ++i) ms[i] = (double)(long long)(h[i] - h[0]) / t->khz;
  delete[] h;
  if (e != hipSuccess) {
    set_error("hipMemcpy failed: %s", hipGetErrorString(e));
    return Q4_ERR_HIP;
  }
  return Q4_OK;
}

int q4_timestamps_destroy(void* ts) {
  clear_error();
  Timestamps* t = reinterpret_cast<Timestamps*>(ts);
  if (!t) return Q4_OK;
  const hipError_t e = hipFree(t->dev);
  delete t;
  if (e != hipSuccess) {
    set_error("hipFree failed: %s", hipGetErrorString(e));
    return Q4_ERR_HIP;
  }
  return Q4_OK;
}

int q4_graph_destroy(void* graph_exec) {
  clear_error();
  if (!graph_exec) return Q4_OK;
  Q4_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
  return Q4_OK;
}

int q4_stream_wait(void* stream, int timeout_ms) {
  clear_error();
  if (timeout_ms <= 0) {
    Q4_HIP(hipStreamSynchronize(as_stream(stream)));
    return Q4_OK;
  }
  auto t0 = std::chrono::steady_clock::now();
  for (;;) {
    hipError_t e = hipStreamQuery(as_stream(stream));
    if (e == hipSuccess) return Q4_OK;
    if (e != hipErrorNotReady) {
      set_error("hipStreamQuery failed: %s", hipGetErrorString(e));
      return Q4_ERR_HIP;
    }
    auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(std::chrono::steady_clock::now() - t0).count();
    if (ms >= timeout_ms) {
      set_error("stream wait timed out after %d ms", timeout_ms);
      return Q4_ERR_TIMEOUT;
    }
    // yield rather than sleep: a sleep rounds up to the kernel's timer slack
    // (~50 us), which a decode token (a few ms) would pay on every wait
    std::this_thread::yield();
  }
}

}  // extern "C"
