// runtime.hip — device selection, pooled device memory, copies, streams, events, the per-stream
// workspaces, the tuning knobs and the registry of tiled weights of the fakhip C ABI
// (include/fakhip.h).
//
// The pool mirrors the CUDA tenant's size-bucketed free lists (internal/compute/cuda_kernels.cu:
// 42-44,108-173): fhip_free parks a block under its bucket size and the next fhip_malloc of the
// same bucket reuses it, so per-token output tensors never reach hipMalloc/hipFree in steady
// state.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "common.hpp"

namespace fhip {
namespace {

thread_local char g_err[512];
hipStream_t g_stream = nullptr;
int g_inited = 0;
int g_cus = 0;
int g_lds = 64 * 1024;
Tuning g_tuning = {};

std::mutex g_pool_mu;
std::unordered_map<void *, size_t> g_live;  // ptr -> bucket bytes
std::multimap<size_t, void *> g_free;       // bucket bytes -> parked ptr
size_t g_free_bytes = 0;

// One grow-only workspace per stream. A buffer outgrown, or left by a destroyed stream, is freed
// at once (after its stream drains) when no graph was ever captured on that stream; otherwise a
// graph may still launch kernels that use it, so it is retired and freed by fhip_trim_pool once
// no graph is alive.
struct StreamWs {
  void *buf = nullptr;
  size_t bytes = 0;
};
std::unordered_map<hipStream_t, StreamWs> g_ws;
std::vector<void *> g_ws_retired;
std::unordered_set<hipStream_t> g_captured;  // streams a capture ever began on
int g_live_graphs = 0;                       // instantiated graphs not yet destroyed
bool g_capturing = false;                    // between fhip_graph_begin and fhip_graph_end

// An instantiated graph and the stream it was captured on: its kernels use that stream's
// workspace, so it replays only there.
struct GraphHandle {
  hipGraphExec_t exec;
  hipStream_t stream;
};

// Give up a workspace buffer of stream s (see StreamWs).
void release_ws(hipStream_t s, void *buf) {
  if (!buf) return;
  if (g_captured.count(s)) {
    g_ws_retired.push_back(buf);
    return;
  }
  (void)hipStreamSynchronize(s);
  (void)hipFree(buf);
}

// fhip_time_next_launch's events, pending for the next launch that takes them.
hipEvent_t g_next_start = nullptr, g_next_stop = nullptr;

// The active ScratchScope, if any.
void *g_scope_base = nullptr;
size_t g_scope_cap = 0;
bool g_scope_on = false;

struct Tag {
  uintptr_t end;
  int kind, out, in;
};
std::map<uintptr_t, Tag> g_tags;  // start -> tiled weight (guarded by g_pool_mu)

size_t bucket(size_t n) {
  if (n <= 4096) return 4096;
  if (n <= (1u << 20)) return (n + 4095) & ~size_t(4095);
  return (n + (2u << 20) - 1) & ~size_t((2u << 20) - 1);
}

int env_knob(const char *name) {
  const char *v = getenv(name);
  return v ? atoi(v) : 0;
}

const char *kind_name(int k) {
  return k == kWeightQ4K ? "Q4_K" : k == kWeightQ8_0 ? "Q8_0" : k == kWeightQ6K ? "Q6_K" : "?";
}

// Drop every record overlapping [a, b) (g_pool_mu held).
void untag_locked(uintptr_t a, uintptr_t b) {
  if (a >= b) return;
  auto it = g_tags.upper_bound(a);
  if (it != g_tags.begin()) {
    auto prev = std::prev(it);
    if (prev->second.end > a) it = prev;
  }
  while (it != g_tags.end() && it->first < b) it = g_tags.erase(it);
}

}  // namespace

hipStream_t stream() { return g_stream; }
int cu_count() { return g_cus; }
int lds_limit() { return g_lds; }
const Tuning &tuning() { return g_tuning; }

void clear_error() { g_err[0] = 0; }

void take_launch_events(hipEvent_t *start, hipEvent_t *stop) {
  if (g_capturing) {  // a captured launch takes none: the pair waits for the next eager launch
    *start = *stop = nullptr;
    return;
  }
  *start = g_next_start;
  *stop = g_next_stop;
  g_next_start = g_next_stop = nullptr;
}

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
  if (g_scope_on) {
    if (bytes <= g_scope_cap) return g_scope_base;
    fail(FHIP_EINVAL, "scratch: the call needs %zu bytes, more than the %zu-byte region it was given",
         bytes, g_scope_cap);
    return nullptr;
  }
  StreamWs &w = g_ws[g_stream];
  if (bytes <= w.bytes) return w.buf;
  size_t want = bytes + bytes / 4;
  if (want < (16u << 20)) want = 16u << 20;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) { hip_fail(e, "workspace: hipMalloc"); return nullptr; }
  release_ws(g_stream, w.buf);
  w.buf = p;
  w.bytes = want;
  return w.buf;
}

ScratchScope::ScratchScope(void *base, size_t cap)
    : prev_base_(g_scope_base), prev_cap_(g_scope_cap), prev_on_(g_scope_on) {
  g_scope_base = base;
  g_scope_cap = cap;
  g_scope_on = true;
}

ScratchScope::~ScratchScope() {
  g_scope_base = prev_base_;
  g_scope_cap = prev_cap_;
  g_scope_on = prev_on_;
}

void tag_weight(const void *p, size_t bytes, int kind, int out, int in) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  const uintptr_t a = (uintptr_t)p;
  untag_locked(a, a + bytes);
  g_tags[a] = Tag{a + bytes, kind, out, in};
}

void untag_range(const void *p, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  untag_locked((uintptr_t)p, (uintptr_t)p + bytes);
}

int check_weight(const char *who, const void *p, int kind, int out, int in) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  auto it = g_tags.find((uintptr_t)p);
  if (it == g_tags.end())
    return fail(FHIP_EINVAL,
                "%s: %p is not a tiled %s weight (upload it with fhip_*_upload or lay it out "
                "with fhip_*_repack; raw GGUF bytes are not accepted)",
                who, p, kind_name(kind));
  const Tag &t = it->second;
  if (t.kind != kind || t.out != out || t.in != in)
    return fail(FHIP_EINVAL, "%s: %p holds a tiled %s weight [%d, %d], not %s [%d, %d]", who, p,
                kind_name(t.kind), t.out, t.in, kind_name(kind), out, in);
  return FHIP_OK;
}

int check_disjoint(const char *who, const void *a, size_t na, const void *b, size_t nb) {
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  if (na && nb && a0 < b0 + nb && b0 < a0 + na)
    return fail(FHIP_EINVAL, "%s: an input buffer overlaps the scratch region of the call", who);
  return FHIP_OK;
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
  if (int rc = noalloc_setup()) return rc;
  // Tuning overrides are read here once, never per call. FAK_HIP_GEMV16_FROM only names a width
  // from which the 5..16-token kernel can take every wider call (1..5); anything else keeps the
  // rule.
  g_tuning.gemv_tw = env_knob("FAK_HIP_GEMV_TW");
  g_tuning.gemv_kw = env_knob("FAK_HIP_GEMV_KW");
  g_tuning.gemv_globalx = env_knob("FAK_HIP_GEMV_GLOBALX");
  const int from16 = env_knob("FAK_HIP_GEMV16_FROM");
  g_tuning.gemv16_from = from16 >= 1 && from16 <= 5 ? from16 : 0;
  g_tuning.gemm32_form = env_knob("FAK_HIP_GEMM32_FORM");
  g_tuning.gemm32_nt = env_knob("FAK_HIP_GEMM32_NT");
  g_tuning.gemm32_sk = env_knob("FAK_HIP_GEMM32_SK");
  g_tuning.gemm32_nwb = env_knob("FAK_HIP_GEMM32_NWB");
  g_tuning.i8r_kw = env_knob("FAK_HIP_I8R_KW");
  g_tuning.i8r_tw = env_knob("FAK_HIP_I8R_TW");
  g_tuning.q8_tw = env_knob("FAK_HIP_Q8_TW");
  g_tuning.q8_kw = env_knob("FAK_HIP_Q8_KW");
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
  untag_locked((uintptr_t)d, (uintptr_t)d + it->second);
  g_free.emplace(it->second, d);
  g_free_bytes += it->second;
  g_live.erase(it);
}

void fhip_trim_pool(size_t max_keep_bytes) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  // Retired workspaces: once no graph is alive (and none is being captured), nothing can launch
  // kernels that use them; drained, they go back to the driver.
  if (!g_ws_retired.empty() && g_live_graphs == 0 && !g_capturing) {
    (void)hipDeviceSynchronize();
    for (void *b : g_ws_retired) (void)hipFree(b);
    g_ws_retired.clear();
  }
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
  untag_range(d, bytes);
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
  Tag copy{0, 0, 0, 0};
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    auto it = g_tags.find((uintptr_t)src);
    if (it != g_tags.end() && it->second.end - it->first == bytes) copy = it->second;
    untag_locked((uintptr_t)dst, (uintptr_t)dst + bytes);
  }
  FHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  FHIP_CHECK(hipStreamSynchronize(g_stream));
  if (copy.kind) tag_weight(dst, bytes, copy.kind, copy.out, copy.in);
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
  untag_range(d, bytes);
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
  untag_range(d, bytes);
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
  // Its workspace is freed once the stream drains, or retired if a graph captured on the stream
  // may still use it.
  auto it = g_ws.find((hipStream_t)s);
  if (it != g_ws.end()) {
    release_ws((hipStream_t)s, it->second.buf);
    g_ws.erase(it);
  }
  g_captured.erase((hipStream_t)s);
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
  g_captured.insert(g_stream);
  FHIP_CHECK(hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed));
  g_capturing = true;
  return FHIP_OK;
}

int fhip_graph_end(void **graph) {
  clear_error();
  if (!graph) return fail(FHIP_EINVAL, "fhip_graph_end: null out pointer");
  *graph = nullptr;
  hipGraph_t g = nullptr;
  g_capturing = false;
  FHIP_CHECK(hipStreamEndCapture(g_stream, &g));
  hipGraphExec_t ex = nullptr;
  const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "fhip_graph_end: hipGraphInstantiate");
  *graph = new GraphHandle{ex, g_stream};
  ++g_live_graphs;
  return FHIP_OK;
}

int fhip_graph_launch(void *graph) {
  clear_error();
  if (!graph) return fail(FHIP_EINVAL, "fhip_graph_launch: null graph");
  const GraphHandle *h = static_cast<const GraphHandle *>(graph);
  // Its kernels use the scratch of the stream they were captured on; replayed on another
  // stream they would race with work queued there.
  if (h->stream != g_stream)
    return fail(FHIP_EINVAL, "fhip_graph_launch: a graph replays only on the stream it was "
                             "captured on; make that stream current with fhip_set_stream");
  FHIP_CHECK(hipGraphLaunch(h->exec, h->stream));
  return FHIP_OK;
}

int fhip_graph_destroy(void *graph) {
  clear_error();
  if (!graph) return FHIP_OK;
  GraphHandle *h = static_cast<GraphHandle *>(graph);
  const hipError_t e = hipGraphExecDestroy(h->exec);
  delete h;
  --g_live_graphs;
  if (e != hipSuccess) return hip_fail(e, "fhip_graph_destroy: hipGraphExecDestroy");
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

int fhip_time_next_launch(void *start, void *stop) {
  clear_error();
  if (!start || !stop) return fail(FHIP_EINVAL, "fhip_time_next_launch: null event");
  if (g_capturing) return fail(FHIP_EINVAL, "fhip_time_next_launch: not during graph capture");
  g_next_start = (hipEvent_t)start;
  g_next_stop = (hipEvent_t)stop;
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
