// Device, memory, stream and event entry points of the C ABI, plus the error,
// poisoning and failure-injection state every launcher goes through.
//
// The reference's XRT shim keeps a thread-local error string and poisons the process
// when a dispatch cannot be aborted (xdna_train/_vendor/xrt_shim/xrt_shim.cpp:57-249);
// this is the HIP counterpart.  The caching allocator plays the role of XdnaBoCache
// (torch_xdna_device.cpp:205-296): size bins, reuse counters, a byte budget.
#include "common.h"
#include "../../include/xdna_hip.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <unordered_map>

namespace xdna {

namespace {
thread_local std::string t_error;
std::atomic<bool> g_poisoned{false};
std::atomic<int64_t> g_launches{0};
std::atomic<int64_t> g_inject_at{0};     // absolute launch number that fails (0: off)
std::atomic<int> g_inject_poison{0};

// Host waits (stream, event and device synchronization) are bounded: a wait that passes
// the deadline returns a timeout status distinct from an error, names what it waited
// for, and poisons the process, since the work it waited for may still be running and
// still use its buffers.  The deadline bounds a hang, not latency: the default, 30 s, is
// several hundred times the longest healthy wait of any workload here (a sweep step of
// 18 ms).  XDNA_WAIT_TIMEOUT_MS sets it; 0 waits without a limit.  The reference bounds
// its NPU dispatch waits the same way (xrt_shim.cpp:57-90, 174-233).
std::atomic<int64_t> g_wait_limit_ms{[] {
  const char* e = std::getenv("XDNA_WAIT_TIMEOUT_MS");
  if (!e || !*e) return int64_t(30000);
  char* end = nullptr;
  const long long v = std::strtoll(e, &end, 10);
  return end && *end == '\0' && v >= 0 ? int64_t(v) : int64_t(30000);
}()};
std::atomic<int64_t> g_waits{0};
std::atomic<int64_t> g_inject_wait_at{0};  // absolute wait number that times out (0: off)
std::atomic<int64_t> g_max_wait_us{0};

using WaitClock = std::chrono::steady_clock;

void note_wait(int64_t us) {
  int64_t prev = g_max_wait_us.load(std::memory_order_relaxed);
  while (us > prev && !g_max_wait_us.compare_exchange_weak(prev, us, std::memory_order_relaxed)) {
  }
}
}  // namespace

void set_error(const std::string& msg) { t_error = msg; }
void clear_error() { t_error.clear(); }

bool admit_launch(const char* what) {
  if (g_poisoned.load(std::memory_order_acquire)) {
    set_error(std::string(what) + ": refused, the process is poisoned by an earlier failure");
    return false;
  }
  const int64_t n = g_launches.fetch_add(1, std::memory_order_relaxed) + 1;
  const int64_t at = g_inject_at.load(std::memory_order_relaxed);
  if (at != 0 && n == at) {
    g_inject_at.store(0, std::memory_order_relaxed);
    if (g_inject_poison.load(std::memory_order_relaxed)) g_poisoned.store(true);
    set_error(std::string(what) + ": injected failure");
    return false;
  }
  return true;
}

int launch_failed(const char* what, hipError_t err) {
  // Errors that can leave device work in flight poison the process: later frees
  // leak and later launches are refused (xrt_shim.cpp:139-151).
  if (err == hipErrorLaunchFailure || err == hipErrorIllegalAddress ||
      err == hipErrorLaunchTimeOut || err == hipErrorAssert) {
    g_poisoned.store(true);
  }
  set_error(std::string(what) + ": " + hipGetErrorString(err));
  return -1;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return launch_failed(what, err);
  return 0;
}

// Polls `poll` (1 done, 0 pending, -1 failed with the error set) until it reports done
// or the deadline passes.  0 done, -1 error, -2 timeout (process poisoned).  The first
// 50 ms spin with yields (what a blocking HIP wait does too), later polls sleep 50 us.
template <class Poll>
int bounded_wait(const char* what, Poll poll) {
  const int64_t n = g_waits.fetch_add(1, std::memory_order_relaxed) + 1;
  const int64_t inj = g_inject_wait_at.load(std::memory_order_relaxed);
  if (inj != 0 && n == inj) {
    g_inject_wait_at.store(0, std::memory_order_relaxed);
    g_poisoned.store(true);
    set_error(std::string("deadline: wait for ") + what + " timed out (injected); the process is poisoned");
    return -2;
  }
  const int64_t limit_ms = g_wait_limit_ms.load(std::memory_order_relaxed);
  const auto t0 = WaitClock::now();
  for (;;) {
    const int r = poll();
    const int64_t us =
        std::chrono::duration_cast<std::chrono::microseconds>(WaitClock::now() - t0).count();
    if (r != 0) {
      note_wait(us);
      return r > 0 ? 0 : -1;
    }
    if (limit_ms > 0 && us >= limit_ms * 1000) {
      g_poisoned.store(true);
      set_error(std::string("deadline: wait for ") + what + " still pending after " + std::to_string(us / 1000) +
                " ms (XDNA_WAIT_TIMEOUT_MS = " + std::to_string(limit_ms) +
                "); device work may still use its buffers, so the process is poisoned");
      return -2;
    }
    if (us < 50000)
      std::this_thread::yield();
    else
      std::this_thread::sleep_for(std::chrono::microseconds(50));
  }
}

// One event per host thread for stream waits (recorded, then polled).
hipEvent_t thread_wait_event() {
  thread_local hipEvent_t ev = nullptr;
  if (!ev && hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    ev = nullptr;
  }
  return ev;
}

int poll_event(hipEvent_t ev, const char* what) {
  const hipError_t e = hipEventQuery(ev);
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  launch_failed(what, e);
  return -1;
}

// ---- caching allocator ---------------------------------------------------------

namespace {

// Blocks belong to the shared pool (id 0) or to a private pool.  A private pool serves the
// allocations a thread makes between pool_begin and pool_end (a graph capture), and keeps
// every block it ever handed out: freed blocks return to it, never to the shared pool, so
// memory a captured graph reads or writes is not given to other work while the graph may
// be replayed.  pool_release hands the pool's blocks back to the shared pool.
struct Cache {
  std::mutex mu;
  std::multimap<size_t, void*> free_blocks;  // shared pool: rounded size -> block
  struct Live {
    size_t size;
    int64_t pool;
  };
  std::unordered_map<void*, Live> live;                                  // block -> size, pool
  std::unordered_map<int64_t, std::multimap<size_t, void*>> pool_free;   // private pools
  int64_t next_pool = 1;
  int64_t cached = 0, allocated = 0, max_allocated = 0;
  int64_t fresh = 0, reuses = 0, frees = 0;
};

Cache& cache() {
  static auto* c = new Cache();  // never destroyed: frees can run at exit
  return *c;
}

thread_local int64_t t_pool = 0;  // private pool of this thread's allocations (0: shared)

// hipMalloc with the thread's stream-capture mode relaxed, so that it is legal while this
// thread captures a graph (the allocation itself is not a stream operation).
hipError_t malloc_relaxed(void** p, size_t n) {
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  const hipError_t e = hipMalloc(p, n);
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  return e;
}

size_t round_size(size_t n) {
  if (n == 0) n = 1;
  if (n <= (size_t(1) << 20)) return (n + 511) & ~size_t(511);
  const size_t big = size_t(2) << 20;
  return (n + big - 1) / big * big;
}

}  // namespace

// out[i] = the bf16 rounding every kernel of the library applies to in[i].
__global__ __launch_bounds__(256) void round_bf16_kernel(const float* __restrict__ in,
                                                         uint16_t* __restrict__ out, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
    out[i] = f32_to_bf16(in[i]);
}

}  // namespace xdna

using namespace xdna;

extern "C" {

const char* xdna_hip_last_error(void) { return t_error.c_str(); }

int xdna_hip_poisoned(void) { return g_poisoned.load() ? 1 : 0; }

int xdna_hip_inject_failure(int64_t nth_launch, int poison) {
  if (nth_launch < 0) {
    set_error("xdna_hip_inject_failure: negative launch index");
    return -1;
  }
  g_inject_poison.store(poison ? 1 : 0);
  g_inject_at.store(nth_launch == 0 ? 0 : g_launches.load() + nth_launch);
  return 0;
}

int xdna_hip_reset_failure_state(void) {
  g_poisoned.store(false);
  g_inject_at.store(0);
  g_inject_poison.store(0);
  g_inject_wait_at.store(0);
  return 0;
}

int64_t xdna_hip_launch_count(void) { return g_launches.load(); }

int xdna_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

int xdna_hip_set_device(int device) {
  const hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return launch_failed("hipSetDevice", e);
  return 0;
}

int xdna_hip_get_device(int* device) {
  const hipError_t e = hipGetDevice(device);
  if (e != hipSuccess) return launch_failed("hipGetDevice", e);
  return 0;
}

int xdna_hip_device_properties(char* name, size_t name_len, int* cu_count, size_t* total_mem,
                               int* gcn_arch) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return launch_failed("hipGetDevice", e);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return launch_failed("hipGetDeviceProperties", e);
  if (name && name_len) {
    std::snprintf(name, name_len, "%s", prop.gcnArchName);
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (total_mem) *total_mem = prop.totalGlobalMem;
  if (gcn_arch) *gcn_arch = prop.major * 100 + prop.minor * 10;  // gfx950 -> 950
  return 0;
}

void* xdna_hip_malloc(size_t bytes) {
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
  if (e != hipSuccess) {
    launch_failed("hipMalloc", e);
    return nullptr;
  }
  return p;
}

int xdna_hip_free(void* ptr) {
  if (!ptr) return 0;
  if (g_poisoned.load()) return 0;  // device work may still use it: leak
  const hipError_t e = hipFree(ptr);
  if (e != hipSuccess) return launch_failed("hipFree", e);
  return 0;
}

void* xdna_hip_cache_alloc(size_t bytes) {
  Cache& c = cache();
  const size_t n = round_size(bytes);
  const int64_t pool = t_pool;
  {
    std::lock_guard<std::mutex> lock(c.mu);
    std::multimap<size_t, void*>* fl = &c.free_blocks;
    if (pool != 0) {
      auto pit = c.pool_free.find(pool);
      fl = pit == c.pool_free.end() ? nullptr : &pit->second;
    }
    auto it = fl ? fl->find(n) : std::multimap<size_t, void*>::iterator();
    if (fl && it != fl->end()) {
      void* p = it->second;
      fl->erase(it);
      c.cached -= int64_t(n);
      c.live.emplace(p, Cache::Live{n, pool});
      c.allocated += int64_t(n);
      if (c.allocated > c.max_allocated) c.max_allocated = c.allocated;
      ++c.reuses;
      return p;
    }
  }
  void* p = nullptr;
  hipError_t e = malloc_relaxed(&p, n);
  if (e != hipSuccess && pool == 0) {
    (void)hipGetLastError();
    // Out of memory: give the cached blocks back and retry once (not while capturing:
    // emptying synchronizes the device).
    xdna_hip_cache_empty();
    e = malloc_relaxed(&p, n);
  }
  if (e != hipSuccess) {
    launch_failed("xdna_hip_cache_alloc", e);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(c.mu);
  c.live.emplace(p, Cache::Live{n, pool});
  c.allocated += int64_t(n);
  if (c.allocated > c.max_allocated) c.max_allocated = c.allocated;
  ++c.fresh;
  return p;
}

int xdna_hip_cache_free(void* ptr) {
  if (!ptr) return 0;
  Cache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  auto it = c.live.find(ptr);
  if (it == c.live.end()) {
    set_error("xdna_hip_cache_free: pointer was not allocated by the cache");
    return -1;
  }
  const Cache::Live b = it->second;
  c.live.erase(it);
  c.allocated -= int64_t(b.size);
  ++c.frees;
  if (g_poisoned.load()) return 0;  // a stuck launch may still use it: never recycle
  auto pit = b.pool != 0 ? c.pool_free.find(b.pool) : c.pool_free.end();
  if (pit != c.pool_free.end())
    pit->second.emplace(b.size, ptr);
  else
    c.free_blocks.emplace(b.size, ptr);
  c.cached += int64_t(b.size);
  return 0;
}

int xdna_hip_cache_empty(void) {
  Cache& c = cache();
  std::multimap<size_t, void*> blocks;
  {
    std::lock_guard<std::mutex> lock(c.mu);
    blocks.swap(c.free_blocks);
    for (const auto& kv : blocks) c.cached -= int64_t(kv.first);
  }
  if (blocks.empty()) return 0;
  // Blocks may still be read by queued work on any stream.
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return launch_failed("xdna_hip_cache_empty", e);
  for (auto& kv : blocks) {
    e = hipFree(kv.second);
    if (e != hipSuccess) return launch_failed("hipFree", e);
  }
  return 0;
}

int64_t xdna_hip_cache_pool_create(void) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  const int64_t id = c.next_pool++;
  c.pool_free.emplace(id, std::multimap<size_t, void*>());
  return id;
}

int xdna_hip_cache_pool_begin(int64_t pool) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  if (c.pool_free.find(pool) == c.pool_free.end()) {
    set_error("xdna_hip_cache_pool_begin: no such pool");
    return -1;
  }
  t_pool = pool;
  return 0;
}

int xdna_hip_cache_pool_end(void) {
  t_pool = 0;
  return 0;
}

int xdna_hip_cache_pool_release(int64_t pool) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  auto pit = c.pool_free.find(pool);
  if (pit == c.pool_free.end()) {
    set_error("xdna_hip_cache_pool_release: no such pool");
    return -1;
  }
  for (const auto& kv : pit->second) c.free_blocks.emplace(kv.first, kv.second);
  c.pool_free.erase(pit);
  for (auto& kv : c.live)
    if (kv.second.pool == pool) kv.second.pool = 0;  // freed later into the shared pool
  return 0;
}

int xdna_hip_cache_stats(int64_t* stats, int n) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  const int64_t v[6] = {c.cached, c.allocated, c.max_allocated, c.fresh, c.reuses, c.frees};
  for (int i = 0; i < n && i < 6; ++i) stats[i] = v[i];
  return 0;
}

int xdna_hip_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return 0;
  hipMemcpyKind k = hipMemcpyDefault;
  switch (kind) {
    case 1: k = hipMemcpyHostToDevice; break;
    case 2: k = hipMemcpyDeviceToHost; break;
    case 3: k = hipMemcpyDeviceToDevice; break;
    default: k = hipMemcpyDefault; break;
  }
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, k, as_stream(stream));
  if (e != hipSuccess) return launch_failed("hipMemcpyAsync", e);
  return 0;
}

int xdna_hip_memset_async(void* dst, int value, size_t bytes, void* stream) {
  if (bytes == 0) return 0;
  const hipError_t e = hipMemsetAsync(dst, value, bytes, as_stream(stream));
  if (e != hipSuccess) return launch_failed("hipMemsetAsync", e);
  return 0;
}

int xdna_hip_stream_synchronize(void* stream) {
  // the injected timeout comes first: it must not touch the device
  hipEvent_t ev = nullptr;
  bool recorded = false;
  return bounded_wait("the stream", [&]() -> int {
    if (!recorded) {
      ev = thread_wait_event();
      if (!ev) {
        set_error("xdna_hip_stream_synchronize: cannot create the wait event");
        return -1;
      }
      const hipError_t e = hipEventRecord(ev, as_stream(stream));
      if (e != hipSuccess) {
        launch_failed("hipEventRecord (stream wait)", e);
        return -1;
      }
      recorded = true;
    }
    return poll_event(ev, "hipEventQuery (stream wait)");
  });
}

int xdna_hip_device_synchronize(void) {
  // hipDeviceSynchronize cannot be polled: it runs on a helper thread and the caller waits
  // for it with the deadline.  A helper stuck past the deadline is left behind (detached).
  struct Job {
    std::mutex mu;
    bool done = false;
    hipError_t err = hipSuccess;
  };
  std::shared_ptr<Job> job;
  int dev = 0;
  return bounded_wait("the device", [&]() -> int {
    if (!job) {
      job = std::make_shared<Job>();
      if (hipGetDevice(&dev) != hipSuccess) (void)hipGetLastError();
      std::thread([job, dev] {
        (void)hipSetDevice(dev);
        const hipError_t e = hipDeviceSynchronize();
        std::lock_guard<std::mutex> lock(job->mu);
        job->err = e;
        job->done = true;
      }).detach();
    }
    std::lock_guard<std::mutex> lock(job->mu);
    if (!job->done) return 0;
    if (job->err != hipSuccess) {
      launch_failed("hipDeviceSynchronize", job->err);
      return -1;
    }
    return 1;
  });
}

int xdna_hip_stream_capturing(void* stream) {
  hipStreamCaptureStatus s = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(as_stream(stream), &s);
  if (e != hipSuccess) return launch_failed("hipStreamIsCapturing", e);
  return s == hipStreamCaptureStatusActive ? 1 : 0;
}

int64_t xdna_hip_cache_pool_current(void) { return t_pool; }

int xdna_hip_set_wait_timeout_ms(int64_t ms) {
  if (ms < 0) {
    set_error("xdna_hip_set_wait_timeout_ms: negative deadline");
    return -1;
  }
  g_wait_limit_ms.store(ms);
  return 0;
}

int64_t xdna_hip_wait_timeout_ms(void) { return g_wait_limit_ms.load(); }

double xdna_hip_max_wait_ms(void) { return double(g_max_wait_us.load()) / 1000.0; }

int xdna_hip_inject_wait_timeout(int64_t nth_wait) {
  if (nth_wait < 0) {
    set_error("xdna_hip_inject_wait_timeout: negative wait index");
    return -1;
  }
  g_inject_wait_at.store(nth_wait == 0 ? 0 : g_waits.load() + nth_wait);
  return 0;
}

void* xdna_hip_event_create(int timing) {
  hipEvent_t ev = nullptr;
  const hipError_t e =
      hipEventCreateWithFlags(&ev, timing ? hipEventDefault : hipEventDisableTiming);
  if (e != hipSuccess) {
    launch_failed("hipEventCreate", e);
    return nullptr;
  }
  return ev;
}

int xdna_hip_event_destroy(void* event) {
  if (!event) return 0;
  const hipError_t e = hipEventDestroy(reinterpret_cast<hipEvent_t>(event));
  if (e != hipSuccess) return launch_failed("hipEventDestroy", e);
  return 0;
}

int xdna_hip_event_record(void* event, void* stream) {
  const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream));
  if (e != hipSuccess) return launch_failed("hipEventRecord", e);
  return 0;
}

int xdna_hip_event_synchronize(void* event) {
  hipEvent_t ev = reinterpret_cast<hipEvent_t>(event);
  return bounded_wait("an event", [&]() -> int { return poll_event(ev, "hipEventQuery"); });
}

int xdna_hip_event_query(void* event) {
  const hipError_t e = hipEventQuery(reinterpret_cast<hipEvent_t>(event));
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  return launch_failed("hipEventQuery", e);
}

int xdna_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  const hipError_t e = hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                           reinterpret_cast<hipEvent_t>(stop));
  if (e != hipSuccess) return launch_failed("hipEventElapsedTime", e);
  return 0;
}

int xdna_hip_stream_wait_event(void* stream, void* event) {
  const hipError_t e =
      hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0);
  if (e != hipSuccess) return launch_failed("hipStreamWaitEvent", e);
  return 0;
}

void* xdna_hip_stream_create(void) {
  hipStream_t s = nullptr;
  // default priority; non-blocking: ordered against other streams by events only
  const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) {
    launch_failed("hipStreamCreateWithFlags", e);
    return nullptr;
  }
  return s;
}

}  // extern "C"

extern "C" int xdna_round_bf16(const float* in, uint16_t* out, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!in || !out))) {
    set_error("xdna_round_bf16: invalid arguments");
    return -1;
  }
  if (n == 0) return 0;
  if (!admit_launch("xdna_round_bf16")) return -1;
  round_bf16_kernel<<<unsigned(std::min<int64_t>(ceil_div(n, 256), 16384)), 256, 0, as_stream(stream)>>>(in, out, n);
  return check_launch("xdna_round_bf16");
}
