// qhip_runtime.hip - device, memory, stream, graph and event-timing services of the
// HIP layer.  One stream per process carries every launch, in program order.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "qhip.h"
#include "qhip_internal.h"

namespace {
hipStream_t g_stream = nullptr;
int g_ready = 0;
int g_ncu = 0;
thread_local char g_err[512] = "";
std::mutex g_init_mu;

struct ProfRec { int cls; hipEvent_t a, b; };
bool g_prof = false;
int g_prof_mode = 0;     // QHIP_PROF_* bits of the last qhip_profile_enable
std::vector<ProfRec> g_prof_recs;
std::vector<hipEvent_t> g_event_pool;
const char *g_class_names[QK_NUM_CLASSES] = {
    "embed", "rmsnorm_quant", "gemv_qkv", "rope_append", "attn_scores", "quant_rows",
    "gemv_o", "gemv_gate_up", "swiglu_quant", "gemv_down", "gemv_head", "argmax", "other", "attn_pv", "pf_gemm", "pf_attn", "pf_other",
    "attn_fast", "attn_layer", "flush"};

hipEvent_t take_event() {
  if (!g_event_pool.empty()) { hipEvent_t e = g_event_pool.back(); g_event_pool.pop_back(); return e; }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

namespace qh {
thread_local int g_prof_suspended = 0;
void prof_suspend(int on) { g_prof_suspended = on; }
hipStream_t stream() { return g_stream; }
int num_cus() { return g_ncu; }

int fail(const char *what, hipError_t e) {
  snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
  return 1;
}

int fail_msg(const char *msg) {
  snprintf(g_err, sizeof g_err, "%s", msg);
  return 1;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : fail(what, e);
}

bool prof_events(int cls, hipEvent_t *start, hipEvent_t *stop) {
  if (!g_prof || g_prof_suspended || cls == QK_FLUSH) return false;
  // A kernel's start stamp is taken when the packet processor picks up its
  // packet, which for back-to-back launches is before the previous kernel has
  // ended: serialized profiling drains the stream first, so the interval is the
  // kernel's own execution; cold profiling also flushes the caches first.
  if ((g_prof_mode & QHIP_PROF_COLD) && qhip_flush_caches()) return false;
  if ((g_prof_mode & (QHIP_PROF_SERIAL | QHIP_PROF_COLD)) && hipStreamSynchronize(g_stream) != hipSuccess) return false;
  hipEvent_t a = take_event(), b = take_event();
  if (!a || !b) {
    if (a) g_event_pool.push_back(a);
    if (b) g_event_pool.push_back(b);
    return false;
  }
  g_prof_recs.push_back({cls, a, b});
  *start = a;
  *stop = b;
  return true;
}
}  // namespace qh

using namespace qh;

extern "C" {

int qhip_init(void) {
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_ready) return 0;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) return fail_msg("no HIP device visible");
  if ((e = hipSetDevice(0)) != hipSuccess) return fail("hipSetDevice", e);
  if ((e = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking)) != hipSuccess)
    return fail("hipStreamCreate", e);
  if ((e = hipDeviceGetAttribute(&g_ncu, hipDeviceAttributeMultiprocessorCount, 0)) != hipSuccess || g_ncu <= 0)
    return fail("hipDeviceGetAttribute(multiprocessor count)", e);
  g_ready = 1;
  return 0;
}

int qhip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

const char *qhip_last_error(void) { return g_err; }

void *qhip_malloc(size_t bytes) {
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
  if (e != hipSuccess) {
    fail("hipMalloc", e);
    (void)hipGetLastError();     // a refused allocation must not fail the next launch's check
    return nullptr;
  }
  return p;
}

void qhip_free(void *p) { if (p) (void)hipFree(p); }

void *qhip_host_alloc(size_t bytes) {
  void *p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault);
  if (e != hipSuccess) {
    fail("hipHostMalloc", e);
    (void)hipGetLastError();
    return nullptr;
  }
  return p;
}

void qhip_host_free(void *p) { if (p) (void)hipHostFree(p); }

int qhip_h2d(void *dst, const void *src, size_t n) {
  if (!n) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  return e == hipSuccess ? 0 : fail("copy to device", e);
}

int qhip_d2h(void *dst, const void *src, size_t n) {
  if (!n) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  return e == hipSuccess ? 0 : fail("copy to host", e);
}

int qhip_h2d_async(void *dst, const void *src, size_t n) {
  if (!n) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g_stream);
  return e == hipSuccess ? 0 : fail("async copy to device", e);
}

int qhip_d2h_async(void *dst, const void *src, size_t n) {
  if (!n) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g_stream);
  return e == hipSuccess ? 0 : fail("async copy to host", e);
}

int qhip_d2d_async(void *dst, const void *src, size_t n) {
  if (!n) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, g_stream);
  return e == hipSuccess ? 0 : fail("device copy", e);
}

// Staged upload: two pinned buffers; the CPU fills one (several threads for
// large chunks: the source is often a freshly mapped file, whose page faults
// dominate) while the DMA of the other is in flight.
namespace {
struct Stager {
  void *buf[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  bool busy[2] = {false, false};
  size_t chunk = 0;
  int next = 0;
} g_up;

void par_copy(void *dst, const void *src, size_t n) {
  const size_t kMinPart = (size_t)8 << 20;
  const int parts = n >= 4 * kMinPart ? 4 : 1;
  if (parts == 1) { memcpy(dst, src, n); return; }
  std::vector<std::thread> th;
  const size_t per = (n + parts - 1) / parts;
  for (int i = 0; i < parts; i++) {
    const size_t o = per * (size_t)i, c = o >= n ? 0 : (n - o < per ? n - o : per);
    if (c) th.emplace_back([=] { memcpy((char *)dst + o, (const char *)src + o, c); });
  }
  for (auto &t : th) t.join();
}
}  // namespace

int qhip_upload_begin(size_t chunk) {
  if (qhip_init()) return 1;
  if (g_up.buf[0]) return fail_msg("upload already in progress");
  g_up.chunk = chunk;
  g_up.next = 0;
  for (int b = 0; b < 2; b++) {
    hipError_t e = hipHostMalloc(&g_up.buf[b], chunk, hipHostMallocDefault);
    if (e != hipSuccess) return fail("hipHostMalloc (upload staging)", e);
    if ((e = hipEventCreateWithFlags(&g_up.ev[b], hipEventDisableTiming)) != hipSuccess)
      return fail("hipEventCreate (upload staging)", e);
    g_up.busy[b] = false;
  }
  return 0;
}

int qhip_upload(void *dst, const void *src, size_t n) {
  if (!g_up.buf[0]) return fail_msg("upload not begun");
  for (size_t o = 0; o < n; o += g_up.chunk) {
    const size_t c = n - o < g_up.chunk ? n - o : g_up.chunk;
    const int b = g_up.next;
    hipError_t e;
    if (g_up.busy[b] && (e = hipEventSynchronize(g_up.ev[b])) != hipSuccess) return fail("upload wait", e);
    par_copy(g_up.buf[b], (const char *)src + o, c);
    if ((e = hipMemcpyAsync((char *)dst + o, g_up.buf[b], c, hipMemcpyHostToDevice, g_stream)) != hipSuccess)
      return fail("upload copy", e);
    if ((e = hipEventRecord(g_up.ev[b], g_stream)) != hipSuccess) return fail("upload record", e);
    g_up.busy[b] = true;
    g_up.next ^= 1;
  }
  return 0;
}

int qhip_upload_end(void) {
  int rc = g_up.buf[0] ? qhip_sync() : 0;
  for (int b = 0; b < 2; b++) {
    if (g_up.buf[b]) (void)hipHostFree(g_up.buf[b]);
    if (g_up.ev[b]) (void)hipEventDestroy(g_up.ev[b]);
    g_up.buf[b] = nullptr;
    g_up.ev[b] = nullptr;
    g_up.busy[b] = false;
  }
  return rc;
}

int qhip_copy2d_d2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, size_t height) {
  if (!width || !height) return 0;
  hipError_t e = hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDeviceToDevice, g_stream);
  return e == hipSuccess ? 0 : fail("2-D device copy", e);
}

int qhip_sync(void) {
  if (!g_ready) return 0;
  hipError_t e = hipStreamSynchronize(g_stream);
  return e == hipSuccess ? 0 : fail("stream synchronize", e);
}

void *qhip_stream(void) { return (void*)g_stream; }

int qhip_device_sync(void) {
  if (!g_ready) return 0;
  hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? 0 : fail("device synchronize", e);
}

int qhip_capture_begin(void) {
  hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal);
  return e == hipSuccess ? 0 : fail("begin capture", e);
}

int qhip_capture_end(void **exec) {
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &g);
  if (e != hipSuccess) return fail("end capture", e);
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return fail("graph instantiate", e);
  *exec = (void*)x;
  return 0;
}

int qhip_graph_launch(void *exec) {
  hipError_t e = hipGraphLaunch((hipGraphExec_t)exec, g_stream);
  return e == hipSuccess ? 0 : fail("graph launch", e);
}

void qhip_graph_destroy(void *exec) {
  if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}

int qhip_profile_enable(int on) {
  if (qhip_init()) return 1;
  if (!on && g_prof) qhip_sync();
  g_prof = on != 0;
  g_prof_mode = on;
  return 0;
}

// Aggregates every (start, stop) pair recorded since the last read per class.
int qhip_profile_read(char *names, int names_len, double *ms, long long *count, int max) {
  if (qhip_sync()) return -1;
  double tot[QK_NUM_CLASSES] = {0};
  long long cnt[QK_NUM_CLASSES] = {0};
  for (auto &r : g_prof_recs) {
    float t = 0.0f;
    if (hipEventElapsedTime(&t, r.a, r.b) == hipSuccess) { tot[r.cls] += t; cnt[r.cls]++; }
    g_event_pool.push_back(r.a);
    g_event_pool.push_back(r.b);
  }
  g_prof_recs.clear();
  std::string all;
  int n = 0;
  for (int c = 0; c < QK_NUM_CLASSES && n < max; c++) {
    if (!cnt[c]) continue;
    ms[n] = tot[c] / (double)cnt[c];
    count[n] = cnt[c];
    all += g_class_names[c];
    all += ",";
    n++;
  }
  if (names && names_len > 0) {
    strncpy(names, all.c_str(), (size_t)names_len - 1);
    names[names_len - 1] = '\0';
  }
  return n;
}

}  // extern "C"

// Wall time of the launches enqueued between qhip_timer_start and qhip_timer_stop
// on the library stream (HIP events); qhip_timer_stop waits for the stop event.
namespace {
hipEvent_t g_t0 = nullptr, g_t1 = nullptr;
}

extern "C" int qhip_timer_start(void) {
  if (!g_t0 && (hipEventCreate(&g_t0) != hipSuccess || hipEventCreate(&g_t1) != hipSuccess))
    return qh::fail_msg("hipEventCreate failed");
  hipError_t e = hipEventRecord(g_t0, g_stream);
  return e == hipSuccess ? 0 : qh::fail("hipEventRecord", e);
}

extern "C" int qhip_timer_stop(double *ms) {
  hipError_t e = hipEventRecord(g_t1, g_stream);
  if (e == hipSuccess) e = hipEventSynchronize(g_t1);
  float t = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&t, g_t0, g_t1);
  if (e != hipSuccess) return qh::fail("timer", e);
  *ms = t;
  return 0;
}

// 1 while per-kernel event timing is on (callers launch eagerly then).
extern "C" int qhip_profiling(void) { return g_prof ? 1 : 0; }
