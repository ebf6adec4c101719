// Device services of libomt_hip.so: per-thread error messages, the library stream, a caching device allocator,
// copies and events.
//
// The allocator replaces the reference's wgpu buffer pool (alloc_buf / free_buf, csrc/runtime.cpp:177-249). Blocks
// are rounded to size classes (512 B granules up to 1 MiB, then 2 MiB granules) and parked when freed. Reuse is stream
// ordered: a block belongs to the stream it was allocated on, and a parked block is handed out again only to an
// allocation on that same stream, whose later work is ordered after every earlier use of the block there. A block
// that other streams also used (omt_record_stream, torch's record_stream) is not parked at once when freed: an event
// is recorded on each of those streams, and the block waits in a pending list until all of them have completed.
//
// Graph pools. While a graph is being captured, the memory its kernels touch must stay theirs for every replay. Between
// omt_graph_pool_begin and omt_graph_pool_end every allocation (from any thread: autograd runs backward on its own
// thread) is served from that pool: from its own parked blocks, else a block of the allocating stream moved over from
// the general free lists, else hipMalloc. Blocks of a graph pool go back to that pool when freed (its replays run in
// capture order), never to the general one, until omt_graph_pool_release returns them all (after the graphs that use
// them are gone).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <string>
#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

#include "omt_internal.h"

namespace omt {

static thread_local std::string t_last_error;

int fail(int st, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_last_error = buf;
  return st;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return OMT_OK;
  if (e == hipErrorOutOfMemory) return fail(OMT_OOM, "%s: %s", what, hipGetErrorString(e));
  return fail(OMT_DEVICE_ERROR, "%s: %s", what, hipGetErrorString(e));
}

// ---- per-kernel launch counts and timings ----------------------------------------------------------------------
//
// Every launch site reports its kernel's name through launch_check; the counts are kept per name pointer (the
// literals of one translation unit) and merged by name when read. With timing on, each report first synchronizes the
// device and adds the wall time since the previous report to the kernel: that launch's enqueue and run, a debug
// measurement that serializes the program (the reference times each dispatch the same way, re-running it after a
// synchronization, csrc/runtime.cpp:573-610).
namespace {
struct KernelStat {
  int64_t launches = 0;
  double ms = 0;
};
std::mutex g_kstat_mu;
std::unordered_map<const char*, KernelStat> g_kstats;
std::vector<std::pair<std::string, KernelStat>> g_kstat_view;  // merged by name at omt_kernel_stat_count
std::atomic<bool> g_ktime{false};
std::chrono::steady_clock::time_point g_klast;
}  // namespace

int launch_check(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(OMT_DEVICE_ERROR, "launch of %s failed: %s", kernel, hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_kstat_mu);
  KernelStat& st = g_kstats[kernel];
  ++st.launches;
  if (g_ktime.load(std::memory_order_relaxed)) {
    e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(OMT_DEVICE_ERROR, "%s: %s", kernel, hipGetErrorString(e));
    const auto now = std::chrono::steady_clock::now();
    st.ms += std::chrono::duration<double, std::milli>(now - g_klast).count();
    g_klast = now;
  }
  return OMT_OK;
}

static std::mutex g_stream_mu;
static hipStream_t g_stream = nullptr;

hipStream_t stream_of(void* s) { return (hipStream_t)s; }

// ---- caching allocator -----------------------------------------------------------------------------------------

namespace {
struct Block {
  size_t cls = 0;
  hipStream_t stream = nullptr;      // the stream it was allocated on
  std::vector<hipStream_t> uses;     // other streams that used it (omt_record_stream)
};

using FreeKey = std::pair<hipStream_t, size_t>;  // (stream, size class)

struct GraphPool {
  std::map<FreeKey, std::vector<void*>> free_lists;  // parked blocks of this pool
  std::unordered_map<void*, size_t> owned;            // every block of this pool -> size class
};

// A freed block whose other-stream uses may still be queued: parked once every event has completed.
struct Pending {
  void* p;
  size_t cls;
  hipStream_t stream;
  std::vector<hipEvent_t> events;  // empty: a use stream was capturing; released at the next device synchronization
};

struct Pool {
  std::mutex mu;
  std::map<FreeKey, std::vector<void*>> free_lists;  // (stream, size class) -> parked blocks
  std::unordered_map<void*, Block> live;              // block -> its record
  std::vector<Pending> pending;
  std::vector<hipEvent_t> spare_events;
  std::map<int, GraphPool> graph_pools;
  std::unordered_map<void*, int> graph_owner;         // block of a graph pool -> pool id
  int active = 0;                                     // graph pool receiving allocations (0: none)
  int next_id = 1;
  size_t allocated = 0;                               // bytes handed out
  size_t reserved = 0;                                // bytes held from HIP (live + parked + pending)
  size_t limit = 0;                                   // 0 = no cap

  static size_t size_class(size_t bytes) {
    if (bytes == 0) bytes = 1;
    const size_t small = 512, big = 2u << 20;
    if (bytes <= (1u << 20)) return (bytes + small - 1) / small * small;
    return (bytes + big - 1) / big * big;
  }

  // Parks the pending blocks whose events have all completed (caller holds mu). hipEventQuery is a prohibited call
  // while a thread captures in global mode, so the calling thread switches to relaxed mode around the queries.
  void collect_pending() {
    if (pending.empty()) return;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    for (size_t i = 0; i < pending.size();) {
      Pending& q = pending[i];
      bool done = !q.events.empty();
      for (hipEvent_t e : q.events) done = done && hipEventQuery(e) == hipSuccess;
      (void)hipGetLastError();  // a not-ready query leaves hipErrorNotReady behind
      if (!done) {
        ++i;
        continue;
      }
      for (hipEvent_t e : q.events) spare_events.push_back(e);
      free_lists[{q.stream, q.cls}].push_back(q.p);
      pending[i] = pending.back();
      pending.pop_back();
    }
    (void)hipThreadExchangeStreamCaptureMode(&mode);
  }

  // After a device synchronization: every pending block is idle; park them all (caller holds mu).
  void settle_pending() {
    for (Pending& q : pending) {
      for (hipEvent_t e : q.events) spare_events.push_back(e);
      free_lists[{q.stream, q.cls}].push_back(q.p);
    }
    pending.clear();
  }

  void release_parked() {  // caller holds mu
    for (auto& kv : free_lists)
      for (void* p : kv.second) {
        (void)hipFree(p);
        reserved -= kv.first.second;
      }
    free_lists.clear();
  }

  hipEvent_t take_event() {
    if (!spare_events.empty()) {
      hipEvent_t e = spare_events.back();
      spare_events.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    return e;
  }
};
Pool& pool() {
  static Pool* p = new Pool();  // never destroyed: blocks may be freed from static destructors of other libraries
  return *p;
}

// hipMalloc is a prohibited call while any thread captures a graph in global mode; allocating is still safe (it is no
// stream operation), so the calling thread switches to relaxed capture mode around it.
hipError_t malloc_relaxed(void** p, size_t bytes) {
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  const hipError_t e = hipMalloc(p, bytes);
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  return e;
}

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}
}  // namespace

}  // namespace omt

using namespace omt;

OMT_EXPORT const char* omt_last_error(void) { return t_last_error.c_str(); }
OMT_EXPORT int omt_abi_version(void) { return 5; }
OMT_EXPORT int omt_hip_runtime_version(void) {
  int v = 0;
  (void)hipRuntimeGetVersion(&v);
  return v;
}

OMT_EXPORT int omt_malloc_on(void** ptr, size_t bytes, void* stream) {
  if (!ptr) return fail(OMT_INVALID, "omt_malloc: null out-pointer");
  Pool& P = pool();
  const size_t cls = Pool::size_class(bytes);
  const hipStream_t s = stream_of(stream);
  const FreeKey key{s, cls};
  std::lock_guard<std::mutex> lk(P.mu);
  P.collect_pending();
  GraphPool* gp = P.active ? &P.graph_pools[P.active] : nullptr;
  auto hand_out = [&](void* p) {
    Block b;
    b.cls = cls;
    b.stream = s;
    P.live[p] = std::move(b);
    P.allocated += cls;
    *ptr = p;
    return OMT_OK;
  };
  if (gp) {
    auto git = gp->free_lists.find(key);
    if (git != gp->free_lists.end() && !git->second.empty()) {
      void* p = git->second.back();
      git->second.pop_back();
      return hand_out(p);
    }
  }
  auto it = P.free_lists.find(key);
  if (it != P.free_lists.end() && !it->second.empty()) {
    void* p = it->second.back();
    it->second.pop_back();
    if (gp) {
      gp->owned[p] = cls;
      P.graph_owner[p] = P.active;
    }
    return hand_out(p);
  }
  void* p = nullptr;
  bool over = P.limit && P.reserved + cls > P.limit;
  hipError_t e = over ? hipErrorOutOfMemory : malloc_relaxed(&p, cls);
  if (e != hipSuccess && !gp) {  // empty the cache once and retry (csrc/runtime.cpp:220-225); never while capturing
    (void)hipGetLastError();
    P.release_parked();
    over = P.limit && P.reserved + cls > P.limit;
    e = over ? hipErrorOutOfMemory : malloc_relaxed(&p, cls);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      *ptr = nullptr;
      return fail(OMT_OOM, "out of device memory allocating %zu bytes (%zu reserved, limit %zu)", cls, P.reserved,
                  P.limit);
    }
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    *ptr = nullptr;
    return fail(OMT_OOM, "out of device memory allocating %zu bytes in a graph pool", cls);
  }
  P.reserved += cls;
  if (gp) {
    gp->owned[p] = cls;
    P.graph_owner[p] = P.active;
  }
  return hand_out(p);
}

OMT_EXPORT int omt_malloc(void** ptr, size_t bytes) { return omt_malloc_on(ptr, bytes, nullptr); }

OMT_EXPORT int omt_record_stream(void* ptr, void* stream) {
  if (!ptr) return OMT_OK;
  Pool& P = pool();
  const hipStream_t s = stream_of(stream);
  std::lock_guard<std::mutex> lk(P.mu);
  auto it = P.live.find(ptr);
  if (it == P.live.end()) return fail(OMT_INVALID, "omt_record_stream: %p was not allocated by omt_malloc", ptr);
  Block& b = it->second;
  if (s != b.stream && std::find(b.uses.begin(), b.uses.end(), s) == b.uses.end()) b.uses.push_back(s);
  return OMT_OK;
}

OMT_EXPORT int omt_free(void* ptr) {
  if (!ptr) return OMT_OK;
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  auto it = P.live.find(ptr);
  if (it == P.live.end()) return fail(OMT_INVALID, "omt_free: %p was not allocated by omt_malloc", ptr);
  Block b = std::move(it->second);
  P.live.erase(it);
  P.allocated -= b.cls;
  auto g = P.graph_owner.find(ptr);
  if (g != P.graph_owner.end()) {  // a graph pool's replays run in capture order: back to the pool as it is
    P.graph_pools[g->second].free_lists[{b.stream, b.cls}].push_back(ptr);
    return OMT_OK;
  }
  if (b.uses.empty()) {
    P.free_lists[{b.stream, b.cls}].push_back(ptr);
    return OMT_OK;
  }
  Pending q{ptr, b.cls, b.stream, {}};
  bool ok = true;
  for (hipStream_t u : b.uses) {
    if (capturing(u)) {  // an event recorded now would become a graph node: wait for a device synchronization
      ok = false;
      break;
    }
    hipEvent_t e = P.take_event();
    if (!e || hipEventRecord(e, u) != hipSuccess) {
      (void)hipGetLastError();
      if (e) P.spare_events.push_back(e);
      ok = false;
      break;
    }
    q.events.push_back(e);
  }
  if (!ok) {
    for (hipEvent_t e : q.events) P.spare_events.push_back(e);
    q.events.clear();
  }
  P.pending.push_back(std::move(q));
  return OMT_OK;
}

OMT_EXPORT int omt_graph_pool_create(void) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  const int id = P.next_id++;
  P.graph_pools[id];
  return id;
}

OMT_EXPORT int omt_graph_pool_begin(int id) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  if (!P.graph_pools.count(id)) return fail(OMT_INVALID, "omt_graph_pool_begin: no graph pool %d", id);
  if (P.active) return fail(OMT_INVALID, "omt_graph_pool_begin: graph pool %d is already receiving", P.active);
  P.active = id;
  return OMT_OK;
}

OMT_EXPORT int omt_graph_pool_end(void) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  P.active = 0;
  return OMT_OK;
}

OMT_EXPORT int omt_graph_pool_release(int id) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  auto it = P.graph_pools.find(id);
  if (it == P.graph_pools.end()) return fail(OMT_INVALID, "omt_graph_pool_release: no graph pool %d", id);
  if (P.active == id) return fail(OMT_INVALID, "omt_graph_pool_release: pool %d is receiving allocations", id);
  OMT_HIP(hipDeviceSynchronize());  // no replay may still use the blocks
  P.settle_pending();
  for (auto& kv : it->second.free_lists)
    for (void* b : kv.second) P.free_lists[kv.first].push_back(b);
  for (auto& kv : it->second.owned) P.graph_owner.erase(kv.first);  // live blocks return to the general pool when freed
  P.graph_pools.erase(it);
  return OMT_OK;
}

OMT_EXPORT int omt_empty_cache(void) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  OMT_HIP(hipDeviceSynchronize());  // parked and pending blocks may still be used by queued kernels
  P.settle_pending();
  P.release_parked();
  return OMT_OK;
}

OMT_EXPORT size_t omt_memory_allocated(void) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  return P.allocated;
}

OMT_EXPORT size_t omt_memory_reserved(void) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  return P.reserved;
}

OMT_EXPORT void omt_set_memory_limit(size_t bytes) {
  Pool& P = pool();
  std::lock_guard<std::mutex> lk(P.mu);
  P.limit = bytes;
}

OMT_EXPORT void* omt_default_stream(void) {
  std::lock_guard<std::mutex> lk(g_stream_mu);
  if (!g_stream && hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) g_stream = nullptr;
  return (void*)g_stream;
}

OMT_EXPORT int omt_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return OMT_OK;
  if (!dst || !src) return fail(OMT_INVALID, "omt_memcpy: null pointer");
  hipStream_t s = stream_of(stream);
  hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
  OMT_HIP(hipMemcpyAsync(dst, src, bytes, k, s));
  if (kind == 1) OMT_HIP(hipStreamSynchronize(s));
  return OMT_OK;
}

OMT_EXPORT int omt_stream_sync(void* stream) {
  OMT_HIP(hipStreamSynchronize(stream_of(stream)));
  return OMT_OK;
}

OMT_EXPORT int omt_event_create(void** ev) {
  OMT_HIP(hipEventCreate((hipEvent_t*)ev));
  return OMT_OK;
}
OMT_EXPORT int omt_event_destroy(void* ev) {
  OMT_HIP(hipEventDestroy((hipEvent_t)ev));
  return OMT_OK;
}
OMT_EXPORT int omt_event_record(void* ev, void* stream) {
  OMT_HIP(hipEventRecord((hipEvent_t)ev, stream_of(stream)));
  return OMT_OK;
}
OMT_EXPORT int omt_event_query(void* ev) {
  hipError_t e = hipEventQuery((hipEvent_t)ev);
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  hip_check(e, "hipEventQuery");
  return -1;
}
OMT_EXPORT int omt_event_sync(void* ev) {
  OMT_HIP(hipEventSynchronize((hipEvent_t)ev));
  return OMT_OK;
}
OMT_EXPORT int omt_event_elapsed_ms(void* start, void* end, float* ms) {
  OMT_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return OMT_OK;
}

OMT_EXPORT void omt_conv_geo_init(omt_conv_geo* g, int64_t n, int64_t ci, int64_t co, int64_t ih, int64_t iw,
                                  int64_t ks, int64_t stride, int64_t pad) {
  g->n = n;
  g->ci = ci;
  g->co = co;
  g->ih = ih;
  g->iw = iw;
  g->oh = (ih + 2 * pad - ks) / stride + 1;
  g->ow = (iw + 2 * pad - ks) / stride + 1;
  g->ks = ks;
  g->stride = stride;
  g->pad = pad;
}

OMT_EXPORT int omt_conv_kind(int64_t x_c, int64_t w_o, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,
                             int64_t pw, int64_t dh, int64_t dw, int transposed, int64_t groups) {
  if (transposed || dh != 1 || dw != 1 || kh != kw || sh != sw || ph != pw) return OMT_CONV_NONE;
  int64_t ks = kh, s = sh, p = ph;
  bool geo_ok = ks >= 1 && ks <= 11 && s >= 1 && s <= 4 && p >= 0 && p <= ks;
  if (groups == 1 && geo_ok) return OMT_CONV_DENSE;
  bool depthwise = groups > 1 && groups == x_c && groups == w_o;
  if (depthwise && (ks == 3 || ks == 5 || ks == 7) && s == 1 && p == ks / 2) return OMT_CONV_DW;
  if (depthwise && geo_ok) return OMT_CONV_DWG;
  return OMT_CONV_NONE;
}

OMT_EXPORT void omt_set_kernel_timing(int on) {
  std::lock_guard<std::mutex> lk(g_kstat_mu);
  if (on) {
    (void)hipDeviceSynchronize();
    g_klast = std::chrono::steady_clock::now();
  }
  g_ktime.store(on != 0);
}

OMT_EXPORT void omt_kernel_stats_reset(int what) {
  std::lock_guard<std::mutex> lk(g_kstat_mu);
  for (auto& kv : g_kstats) {
    if (what & OMT_KSTAT_LAUNCHES) kv.second.launches = 0;
    if (what & OMT_KSTAT_TIMES) kv.second.ms = 0;
  }
  g_kstat_view.clear();
  if (g_ktime.load()) g_klast = std::chrono::steady_clock::now();
}

OMT_EXPORT int omt_kernel_stat_count(void) {
  std::lock_guard<std::mutex> lk(g_kstat_mu);
  std::map<std::string, KernelStat> merged;
  for (const auto& [name, st] : g_kstats) {
    KernelStat& m = merged[name];
    m.launches += st.launches;
    m.ms += st.ms;
  }
  g_kstat_view.assign(merged.begin(), merged.end());
  return (int)g_kstat_view.size();
}

OMT_EXPORT int omt_kernel_stat_entry(int i, const char** name, int64_t* launches, double* ms) {
  std::lock_guard<std::mutex> lk(g_kstat_mu);
  if (i < 0 || i >= (int)g_kstat_view.size() || !name || !launches || !ms)
    return fail(OMT_INVALID, "omt_kernel_stat_entry: entry %d of %zu", i, g_kstat_view.size());
  *name = g_kstat_view[i].first.c_str();
  *launches = g_kstat_view[i].second.launches;
  *ms = g_kstat_view[i].second.ms;
  return OMT_OK;
}
