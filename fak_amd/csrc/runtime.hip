// runtime.hip — device selection, pooled device memory, copies, streams, events and the
// library-owned workspace of the fakhip C ABI (include/fakhip.h).
//
// The pool mirrors the CUDA tenant's size-bucketed free lists (internal/compute/cuda_kernels.cu:
// 42-44,108-173): fhip_free parks a block under its bucket size and the next fhip_malloc of the
// same bucket reuses it, so per-token output tensors never reach hipMalloc/hipFree in steady
// state.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace fhip {
namespace {

thread_local char g_err[512];
hipStream_t g_stream = nullptr;
int g_inited = 0;
int g_cus = 0;
int g_lds = 64 * 1024;

std::mutex g_pool_mu;
std::unordered_map<void *, size_t> g_live;  // ptr -> bucket bytes
std::multimap<size_t, void *> g_free;       // bucket bytes -> parked ptr
size_t g_free_bytes = 0;

void *g_ws = nullptr;
size_t g_ws_bytes = 0;
std::vector<void *> g_ws_retired;  // earlier, smaller workspaces (kept for captured graphs)

size_t bucket(size_t n) {
  if (n <= 4096) return 4096;
  if (n <= (1u << 20)) return (n + 4095) & ~size_t(4095);
  return (n + (2u << 20) - 1) & ~size_t((2u << 20) - 1);
}

}  // namespace

hipStream_t stream() { return g_stream; }
int cu_count() { return g_cus; }
int lds_limit() { return g_lds; }

void clear_error() { g_err[0] = 0; }

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  snprintf(g_err, sizeof g_err, "%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
  return 1000 + (int)e;
}

void *workspace(size_t bytes) {
  if (bytes <= g_ws_bytes) return g_ws;
  size_t want = bytes + bytes / 4;
  if (want < (16u << 20)) want = 16u << 20;
  // A smaller workspace is retired, not freed: graphs captured earlier may still launch
  // kernels that use it (the growth is geometric, so the retired total stays below the
  // current size).
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) { hip_fail(e, "workspace: hipMalloc"); return nullptr; }
  if (g_ws) g_ws_retired.push_back(g_ws);
  g_ws = p;
  g_ws_bytes = want;
  return g_ws;
}

}  // namespace fhip

using namespace fhip;

extern "C" {

const char *fhip_last_error(void) { return g_err; }

int fhip_init(char *name, int namelen, int *arch, size_t *total_mem) {
  clear_error();
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) return fail(FHIP_ENODEV, "no HIP device visible");
  FHIP_CHECK(hipSetDevice(0));
  hipDeviceProp_t prop;
  FHIP_CHECK(hipGetDeviceProperties(&prop, 0));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(FHIP_ENODEV, "device 0 is %s; this backend is built for gfx950 only",
                prop.gcnArchName);
  g_cus = prop.multiProcessorCount;
  g_lds = (int)prop.sharedMemPerBlock;
  if (name && namelen > 0) {
    strncpy(name, prop.name, (size_t)namelen - 1);
    name[namelen - 1] = 0;
  }
  if (arch) *arch = 950;
  if (total_mem) *total_mem = prop.totalGlobalMem;
  g_inited = 1;
  return FHIP_OK;
}

int fhip_mem_info(size_t *free_mem, size_t *total_mem) {
  clear_error();
  size_t f = 0, t = 0;
  FHIP_CHECK(hipMemGetInfo(&f, &t));
  if (free_mem) *free_mem = f;
  if (total_mem) *total_mem = t;
  return FHIP_OK;
}

void *fhip_malloc(size_t bytes) {
  clear_error();
  size_t b = bucket(bytes ? bytes : 1);
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    auto it = g_free.find(b);
    if (it != g_free.end()) {
      void *p = it->second;
      g_free.erase(it);
      g_free_bytes -= b;
      g_live[p] = b;
      return p;
    }
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, b);
  if (e != hipSuccess) {
    // Return parked blocks to the driver and try once more before giving up.
    fhip_trim_pool(0);
    e = hipMalloc(&p, b);
    if (e != hipSuccess) {
      hip_fail(e, "fhip_malloc: hipMalloc");
      return nullptr;
    }
  }
  std::lock_guard<std::mutex> lk(g_pool_mu);
  g_live[p] = b;
  return p;
}

void fhip_free(void *d) {
  if (!d) return;
  std::lock_guard<std::mutex> lk(g_pool_mu);
  auto it = g_live.find(d);
  if (it == g_live.end()) return;  // not ours: ignore rather than corrupt the pool
  g_free.emplace(it->second, d);
  g_free_bytes += it->second;
  g_live.erase(it);
}

void fhip_trim_pool(size_t max_keep_bytes) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  if (g_free_bytes <= max_keep_bytes) return;
  // Parked blocks may still be referenced by queued work: drain before releasing.
  (void)hipDeviceSynchronize();
  while (g_free_bytes > max_keep_bytes && !g_free.empty()) {
    auto it = std::prev(g_free.end());  // largest parked block first
    (void)hipFree(it->second);
    g_free_bytes -= it->first;
    g_free.erase(it);
  }
}

int fhip_h2d(void *d, const void *h, size_t bytes) {
  clear_error();
  if (bytes == 0) return FHIP_OK;
  if (!d || !h) return fail(FHIP_EINVAL, "fhip_h2d: null pointer");
  FHIP_CHECK(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice));
  return FHIP_OK;
}

int fhip_d2h(void *h, const void *d, size_t bytes) {
  clear_error();
  if (bytes == 0) return FHIP_OK;
  if (!d || !h) return fail(FHIP_EINVAL, "fhip_d2h: null pointer");
  FHIP_CHECK(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, g_stream));
  FHIP_CHECK(hipStreamSynchronize(g_stream));
  return FHIP_OK;
}

int fhip_d2d(void *dst, const void *src, size_t bytes) {
  clear_error();
  if (bytes == 0) return FHIP_OK;
  if (!dst || !src) return fail(FHIP_EINVAL, "fhip_d2d: null pointer");
  FHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  FHIP_CHECK(hipStreamSynchronize(g_stream));
  return FHIP_OK;
}

int fhip_sync(void) {
  clear_error();
  FHIP_CHECK(hipDeviceSynchronize());
  return FHIP_OK;
}

int fhip_h2d_async(void *d, const void *h, size_t bytes) {
  clear_error();
  if (bytes == 0) return FHIP_OK;
  if (!d || !h) return fail(FHIP_EINVAL, "fhip_h2d_async: null pointer");
  FHIP_CHECK(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, g_stream));
  return FHIP_OK;
}

int fhip_d2h_async(void *h, const void *d, size_t bytes) {
  clear_error();
  if (bytes == 0) return FHIP_OK;
  if (!d || !h) return fail(FHIP_EINVAL, "fhip_d2h_async: null pointer");
  FHIP_CHECK(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, g_stream));
  return FHIP_OK;
}

int fhip_memset_async(void *d, int value, size_t bytes) {
  clear_error();
  if (bytes == 0) return FHIP_OK;
  if (!d) return fail(FHIP_EINVAL, "fhip_memset_async: null pointer");
  FHIP_CHECK(hipMemsetAsync(d, value, bytes, g_stream));
  return FHIP_OK;
}

int fhip_stream_create(void **s) {
  clear_error();
  if (!s) return fail(FHIP_EINVAL, "fhip_stream_create: null out pointer");
  hipStream_t st = nullptr;
  FHIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  *s = (void *)st;
  return FHIP_OK;
}

int fhip_stream_destroy(void *s) {
  clear_error();
  if (!s) return FHIP_OK;
  if ((hipStream_t)s == g_stream) g_stream = nullptr;
  FHIP_CHECK(hipStreamDestroy((hipStream_t)s));
  return FHIP_OK;
}

int fhip_set_stream(void *s) {
  clear_error();
  g_stream = (hipStream_t)s;
  return FHIP_OK;
}

int fhip_stream_sync(void *s) {
  clear_error();
  FHIP_CHECK(hipStreamSynchronize((hipStream_t)s));
  return FHIP_OK;
}

int fhip_graph_begin(void) {
  clear_error();
  if (!g_stream)
    return fail(FHIP_EINVAL, "fhip_graph_begin: capture needs a stream from fhip_stream_create "
                             "made current with fhip_set_stream");
  FHIP_CHECK(hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed));
  return FHIP_OK;
}

int fhip_graph_end(void **graph) {
  clear_error();
  if (!graph) return fail(FHIP_EINVAL, "fhip_graph_end: null out pointer");
  *graph = nullptr;
  hipGraph_t g = nullptr;
  FHIP_CHECK(hipStreamEndCapture(g_stream, &g));
  hipGraphExec_t ex = nullptr;
  const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "fhip_graph_end: hipGraphInstantiate");
  *graph = (void *)ex;
  return FHIP_OK;
}

int fhip_graph_launch(void *graph) {
  clear_error();
  if (!graph) return fail(FHIP_EINVAL, "fhip_graph_launch: null graph");
  FHIP_CHECK(hipGraphLaunch((hipGraphExec_t)graph, g_stream));
  return FHIP_OK;
}

int fhip_graph_destroy(void *graph) {
  clear_error();
  if (!graph) return FHIP_OK;
  FHIP_CHECK(hipGraphExecDestroy((hipGraphExec_t)graph));
  return FHIP_OK;
}

int fhip_event_create(void **ev) {
  clear_error();
  if (!ev) return fail(FHIP_EINVAL, "fhip_event_create: null out pointer");
  hipEvent_t e = nullptr;
  FHIP_CHECK(hipEventCreate(&e));
  *ev = (void *)e;
  return FHIP_OK;
}

int fhip_event_destroy(void *ev) {
  clear_error();
  if (!ev) return FHIP_OK;
  FHIP_CHECK(hipEventDestroy((hipEvent_t)ev));
  return FHIP_OK;
}

int fhip_event_record(void *ev) {
  clear_error();
  if (!ev) return fail(FHIP_EINVAL, "fhip_event_record: null event");
  FHIP_CHECK(hipEventRecord((hipEvent_t)ev, g_stream));
  return FHIP_OK;
}

int fhip_event_elapsed_ms(void *start, void *end, float *ms) {
  clear_error();
  if (!start || !end || !ms) return fail(FHIP_EINVAL, "fhip_event_elapsed_ms: null argument");
  FHIP_CHECK(hipEventSynchronize((hipEvent_t)end));
  FHIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return FHIP_OK;
}

}  // extern "C"
