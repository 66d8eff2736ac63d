// Runtime half of the C ABI: device init, a stream-aware caching allocator,
// copies, streams, events, HIP graphs, thread-local error text, and the host-side
// replica of PyTorch's CPU MT19937 generator (randn / rand).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace cv3 {

static thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

// Set once by cv3_shutdown: later frees and destroys become no-ops, so objects the
// host language releases during its own teardown never touch a torn-down runtime.
static std::atomic<bool> g_shut{false};

static std::mutex g_mu;                          // allocator, stream, event and graph registries
// A thread's own stream is tagged with the shutdown generation it was made in: after
// cv3_shutdown destroys it, a thread that still holds the handle (a daemon thread
// running past interpreter exit) must not launch onto it.
static thread_local hipStream_t g_tls_stream = nullptr;
static std::vector<hipStream_t> g_thread_streams;  // every per-thread stream, for cv3_shutdown
// Every stream and event handed out by cv3_stream_create / cv3_event_create: cv3_shutdown
// destroys whatever the host language has not released yet, so no HIP object of this
// library outlives it into the runtime's own exit handlers.
static std::unordered_map<hipStream_t, bool> g_user_streams;
static std::unordered_map<hipEvent_t, bool> g_user_events;

int decode_scratch_setup();   // decode.hip: looks up its fixed scratch on the current device

bool shut_down() { return g_shut.load(); }

hipStream_t stream_of(cv3_stream_t s) {
  // After cv3_shutdown nothing may be enqueued: every block is freed, every stream destroyed.
  if (g_shut.load()) {
    fail(CV3_EINVAL, "the library has been shut down");
    return nullptr;
  }
  if (s) return reinterpret_cast<hipStream_t>(s);
  if (!g_tls_stream) {
    // Default priority only: streams of different priorities are avoided.
    hipStream_t h = nullptr;
    if (hipStreamCreateWithFlags(&h, hipStreamNonBlocking) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    g_thread_streams.push_back(h);
    g_tls_stream = h;
  }
  return g_tls_stream;
}

static bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusActive;
}

// ---------------------------------------------------------------------------
// Caching allocator.  hipFree synchronises the whole device, so the drop-in
// per-op path (which allocates temporaries on every call) keeps freed blocks in
// size-class free lists.
//
// Stream safety: a block remembers the stream it was allocated on (its home) and
// every other stream it was used on (cv3_record_stream).  Freeing records one
// event on each of those streams and on the freeing thread's stream; a later
// allocation from a different stream waits for all of them, so a block is never
// handed out while a kernel on any of its streams may still touch it.
//
// Graph capture: a block freed while the freeing thread's stream is capturing is
// still referenced by the graph being built.  It stays allocated and belongs to
// that graph from cv3_graph_end on; cv3_graph_destroy returns it to the cache
// behind the graph's last launch.  Allocation during capture reuses only blocks
// whose pending frees were all recorded on the capturing stream itself (no
// cross-stream wait inside a capture); a captured graph is launched on its
// capture stream, or after that stream has been synchronised.
// ---------------------------------------------------------------------------
struct Block {
  size_t size;
  hipStream_t home;
  std::vector<hipStream_t> users;                          // streams besides home
  std::vector<hipEvent_t> events;                          // event pool, grows to #streams
  std::vector<std::pair<hipStream_t, hipEvent_t>> pending;  // recorded at the last free
};

static std::multimap<size_t, void*> g_free;            // size class -> ptr
static std::unordered_map<void*, Block> g_blocks;      // every live or cached block
static size_t g_in_use = 0, g_cached = 0;
static thread_local std::vector<void*> g_tls_deferred;  // freed during this thread's capture

struct GraphExec {
  hipGraphExec_t exec;
  std::vector<void*> owned;   // blocks freed while it was being captured
  hipStream_t last;           // stream of its last launch
};
static std::unordered_map<GraphExec*, bool> g_graphs;

static size_t size_class(size_t b) {
  if (b <= 256) return 256;
  if (b <= (1u << 20)) {  // next power of two up to 1 MiB
    size_t c = 512;
    while (c < b) c <<= 1;
    return c;
  }
  const size_t g = 1u << 20;  // 1 MiB granules above that
  return (b + g - 1) / g * g;
}

// Records the block's pending events on `streams` and parks it in the free list.
// Caller holds g_mu.  The block always ends up parked: if an event cannot be created or
// recorded, the device is synchronised instead (so no stream can still touch the block),
// its pending list is emptied, and the HIP error is returned.
static int release_locked(void* ptr, Block& b, const std::vector<hipStream_t>& streams) {
  b.pending.clear();
  hipError_t err = hipSuccess;
  for (size_t i = 0; i < streams.size() && err == hipSuccess; ++i) {
    if (i == b.events.size()) {
      hipEvent_t ev;
      err = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (err != hipSuccess) break;
      b.events.push_back(ev);
    }
    err = hipEventRecord(b.events[i], streams[i]);
    if (err == hipSuccess) b.pending.emplace_back(streams[i], b.events[i]);
  }
  if (err != hipSuccess) {
    (void)hipDeviceSynchronize();
    b.pending.clear();
  }
  b.users.clear();
  g_free.emplace(b.size, ptr);
  g_in_use -= b.size;
  g_cached += b.size;
  if (err != hipSuccess) return fail(CV3_EHIP, "recording a freed block's stream events failed: %s", hipGetErrorString(err));
  return CV3_OK;
}

static void add_stream(std::vector<hipStream_t>& v, hipStream_t s) {
  for (hipStream_t x : v)
    if (x == s) return;
  v.push_back(s);
}

}  // namespace cv3

using namespace cv3;

extern "C" {

const char* cv3_last_error(void) { return g_error.c_str(); }

int cv3_init(int device) {
  CV3_REQUIRE(!g_shut.load(), CV3_EINVAL, "the library has been shut down");
  int n = 0;
  CV3_HIP(hipGetDeviceCount(&n));
  CV3_REQUIRE(n > 0, CV3_EHIP, "no HIP device is visible");
  CV3_REQUIRE(device >= 0 && device < n, CV3_EINVAL, "device %d out of range (have %d)", device, n);
  CV3_HIP(hipSetDevice(device));
  CV3_HIP(hipFree(nullptr));
  return decode_scratch_setup();
}

int cv3_device_info(int* cu_count, int64_t* hbm_bytes, char* name, int name_len) {
  int dev = 0;
  CV3_HIP(hipGetDevice(&dev));
  hipDeviceProp_t p;
  CV3_HIP(hipGetDeviceProperties(&p, dev));
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = (int64_t)p.totalGlobalMem;
  if (name && name_len > 0) {
    snprintf(name, name_len, "%s", p.gcnArchName);
  }
  return CV3_OK;
}

int cv3_malloc(void** ptr, size_t bytes) {
  CV3_REQUIRE(ptr, CV3_EINVAL, "null output pointer");
  CV3_REQUIRE(!g_shut.load(), CV3_EINVAL, "the library has been shut down");
  const size_t sz = size_class(bytes ? bytes : 1);
  hipStream_t cur = stream_of(nullptr);
  CV3_REQUIRE(cur, CV3_EHIP, "could not create the calling thread's stream");
  const bool cap = capturing(cur);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto range = g_free.equal_range(sz);
    for (auto it = range.first; it != range.second; ++it) {
      void* p = it->second;
      Block& b = g_blocks[p];
      bool ok = true;
      if (cap)
        for (auto& pe : b.pending) ok = ok && pe.first == cur;
      if (!ok) continue;
      for (auto& pe : b.pending)
        if (pe.first != cur) CV3_HIP(hipStreamWaitEvent(cur, pe.second, 0));
      g_free.erase(it);
      b.pending.clear();
      b.home = cur;
      b.users.clear();
      g_cached -= sz;
      g_in_use += sz;
      *ptr = p;
      return CV3_OK;
    }
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess && !cap) {
    // Out of memory: release the cache and try once more.
    cv3_empty_cache();
    (void)hipGetLastError();
    e = hipMalloc(&p, sz);
  }
  if (e != hipSuccess) return fail(CV3_EHIP, "hipMalloc(%zu) failed: %s", sz, hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_mu);
  g_blocks[p] = Block{sz, cur, {}, {}, {}};
  g_in_use += sz;
  *ptr = p;
  return CV3_OK;
}

int cv3_record_stream(void* ptr, cv3_stream_t s) {
  if (!ptr || g_shut.load()) return CV3_OK;
  hipStream_t st = stream_of(s);
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_blocks.find(ptr);
  CV3_REQUIRE(it != g_blocks.end(), CV3_EINVAL, "cv3_record_stream of a pointer not from cv3_malloc");
  if (st != it->second.home) add_stream(it->second.users, st);
  return CV3_OK;
}

int cv3_free(void* ptr) {
  if (!ptr || g_shut.load()) return CV3_OK;
  hipStream_t cur = stream_of(nullptr);
  CV3_REQUIRE(cur, CV3_EHIP, "could not create the calling thread's stream");
  if (capturing(cur)) {   // the graph being captured may still refer to it
    std::lock_guard<std::mutex> lk(g_mu);
    CV3_REQUIRE(g_blocks.count(ptr), CV3_EINVAL, "cv3_free of a pointer not from cv3_malloc");
    g_tls_deferred.push_back(ptr);
    return CV3_OK;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_blocks.find(ptr);
  CV3_REQUIRE(it != g_blocks.end(), CV3_EINVAL, "cv3_free of a pointer not from cv3_malloc");
  Block& b = it->second;
  std::vector<hipStream_t> streams{b.home};
  for (hipStream_t u : b.users) add_stream(streams, u);
  add_stream(streams, cur);
  return release_locked(ptr, b, streams);
}

int cv3_empty_cache(void) {
  if (g_shut.load()) return CV3_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& kv : g_free) {
    auto it = g_blocks.find(kv.second);
    if (it != g_blocks.end()) {
      for (auto& pe : it->second.pending) hipEventSynchronize(pe.second);
      for (hipEvent_t ev : it->second.events) hipEventDestroy(ev);
      g_cached -= it->second.size;
      g_blocks.erase(it);
    }
    hipFree(kv.second);
  }
  g_free.clear();
  return CV3_OK;
}

int cv3_mem_stats(size_t* in_use, size_t* cached) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (in_use) *in_use = g_in_use;
  if (cached) *cached = g_cached;
  return CV3_OK;
}

int cv3_copy_h2d(void* dst, const void* src, size_t bytes, cv3_stream_t s) {
  CV3_ALIVE();
  if (!bytes) return CV3_OK;
  hipStream_t st = stream_of(s);
  CV3_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st));
  CV3_HIP(hipStreamSynchronize(st));
  return CV3_OK;
}

int cv3_copy_d2h(void* dst, const void* src, size_t bytes, cv3_stream_t s) {
  CV3_ALIVE();
  if (!bytes) return CV3_OK;
  hipStream_t st = stream_of(s);
  CV3_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st));
  CV3_HIP(hipStreamSynchronize(st));
  return CV3_OK;
}

int cv3_copy_d2d(void* dst, const void* src, size_t bytes, cv3_stream_t s) {
  CV3_ALIVE();
  if (!bytes) return CV3_OK;
  CV3_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_of(s)));
  return CV3_OK;
}

int cv3_stream_create(cv3_stream_t* s) {
  CV3_REQUIRE(s, CV3_EINVAL, "null output pointer");
  CV3_REQUIRE(!g_shut.load(), CV3_EINVAL, "the library has been shut down");
  hipStream_t h;
  CV3_HIP(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
  std::lock_guard<std::mutex> lk(g_mu);
  g_user_streams[h] = true;
  *s = reinterpret_cast<cv3_stream_t>(h);
  return CV3_OK;
}

// The stream is drained first, then forgotten by every block that recorded it (as a
// user or in the events of its last free, which are complete once the stream is
// drained), so a block freed after its stream is gone never records onto it.
int cv3_stream_destroy(cv3_stream_t s) {
  if (!s || g_shut.load()) return CV3_OK;
  hipStream_t h = reinterpret_cast<hipStream_t>(s);
  std::lock_guard<std::mutex> lk(g_mu);
  CV3_REQUIRE(g_user_streams.erase(h), CV3_EINVAL, "cv3_stream_destroy of a stream not from cv3_stream_create");
  const hipError_t se = hipStreamSynchronize(h);
  for (auto& kv : g_blocks) {
    Block& b = kv.second;
    for (size_t i = 0; i < b.users.size();)
      if (b.users[i] == h) b.users.erase(b.users.begin() + i); else ++i;
    for (size_t i = 0; i < b.pending.size();)
      if (b.pending[i].first == h) b.pending.erase(b.pending.begin() + i); else ++i;
  }
  for (auto& kv : g_graphs)
    if (kv.first->last == h) kv.first->last = nullptr;  // its launches are done
  const hipError_t de = hipStreamDestroy(h);
  if (se != hipSuccess) return fail(CV3_EHIP, "hipStreamSynchronize failed: %s", hipGetErrorString(se));
  if (de != hipSuccess) return fail(CV3_EHIP, "hipStreamDestroy failed: %s", hipGetErrorString(de));
  return CV3_OK;
}

int cv3_stream_sync(cv3_stream_t s) {
  hipStream_t st = stream_of(s);
  CV3_REQUIRE(st, CV3_EINVAL, "%s", cv3_last_error());
  CV3_HIP(hipStreamSynchronize(st));
  return CV3_OK;
}

int cv3_device_sync(void) {
  CV3_ALIVE();
  CV3_HIP(hipDeviceSynchronize());
  return CV3_OK;
}

int cv3_event_create(void** ev) {
  CV3_REQUIRE(ev, CV3_EINVAL, "null output pointer");
  CV3_REQUIRE(!g_shut.load(), CV3_EINVAL, "the library has been shut down");
  hipEvent_t e;
  CV3_HIP(hipEventCreate(&e));
  std::lock_guard<std::mutex> lk(g_mu);
  g_user_events[e] = true;
  *ev = e;
  return CV3_OK;
}

int cv3_event_destroy(void* ev) {
  if (!ev || g_shut.load()) return CV3_OK;
  hipEvent_t e = reinterpret_cast<hipEvent_t>(ev);
  std::lock_guard<std::mutex> lk(g_mu);
  CV3_REQUIRE(g_user_events.erase(e), CV3_EINVAL, "cv3_event_destroy of an event not from cv3_event_create");
  CV3_HIP(hipEventDestroy(e));
  return CV3_OK;
}

int cv3_event_record(void* ev, cv3_stream_t s) {
  CV3_REQUIRE(ev, CV3_EINVAL, "null event");
  hipStream_t st = stream_of(s);
  CV3_REQUIRE(st, CV3_EINVAL, "%s", cv3_last_error());
  CV3_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), st));
  return CV3_OK;
}

int cv3_stream_wait_event(cv3_stream_t s, void* ev) {
  CV3_REQUIRE(ev, CV3_EINVAL, "null event");
  hipStream_t st = stream_of(s);
  CV3_REQUIRE(st, CV3_EINVAL, "%s", cv3_last_error());
  CV3_HIP(hipStreamWaitEvent(st, reinterpret_cast<hipEvent_t>(ev), 0));
  return CV3_OK;
}

int cv3_event_elapsed_ms(void* ev0, void* ev1, float* ms) {
  CV3_REQUIRE(!g_shut.load(), CV3_EINVAL, "the library has been shut down");
  CV3_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev1)));
  CV3_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(ev0), reinterpret_cast<hipEvent_t>(ev1)));
  return CV3_OK;
}

int cv3_graph_begin(cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(g_tls_deferred.empty(), CV3_EINVAL, "a capture is already in progress on this thread");
  CV3_HIP(hipStreamBeginCapture(stream_of(s), hipStreamCaptureModeThreadLocal));
  return CV3_OK;
}

int cv3_graph_end(cv3_stream_t s, void** exec) {
  CV3_ALIVE();
  hipGraph_t g = nullptr;
  hipStream_t st = stream_of(s);
  std::vector<void*> owned;
  owned.swap(g_tls_deferred);
  hipError_t e = hipStreamEndCapture(st, &g);
  hipGraphExec_t x = nullptr;
  if (e == hipSuccess) {
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
  }
  if (e != hipSuccess) {
    // nothing was captured for good: the deferred blocks go back behind the stream
    std::lock_guard<std::mutex> lk(g_mu);
    for (void* p : owned) {
      auto it = g_blocks.find(p);
      if (it != g_blocks.end()) release_locked(p, it->second, {it->second.home, st});
    }
    return fail(CV3_EHIP, "graph capture failed: %s", hipGetErrorString(e));
  }
  GraphExec* w = new GraphExec{x, std::move(owned), st};
  std::lock_guard<std::mutex> lk(g_mu);
  g_graphs[w] = true;
  *exec = w;
  return CV3_OK;
}

int cv3_graph_launch(void* exec, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(exec, CV3_EINVAL, "null graph");
  GraphExec* w = reinterpret_cast<GraphExec*>(exec);
  hipStream_t st = stream_of(s);
  CV3_HIP(hipGraphLaunch(w->exec, st));
  w->last = st;
  return CV3_OK;
}

int cv3_graph_destroy(void* exec) {
  if (!exec || g_shut.load()) return CV3_OK;
  GraphExec* w = reinterpret_cast<GraphExec*>(exec);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_graphs.erase(w)) return fail(CV3_EINVAL, "cv3_graph_destroy of an unknown graph");
  for (void* p : w->owned) {   // behind the graph's last launch (none if its stream was destroyed)
    auto it = g_blocks.find(p);
    if (it != g_blocks.end()) {
      std::vector<hipStream_t> streams{it->second.home};
      for (hipStream_t u : it->second.users) add_stream(streams, u);
      if (w->last) add_stream(streams, w->last);
      release_locked(p, it->second, streams);
    }
  }
  hipError_t e = hipGraphExecDestroy(w->exec);
  delete w;
  if (e != hipSuccess) return fail(CV3_EHIP, "hipGraphExecDestroy failed: %s", hipGetErrorString(e));
  return CV3_OK;
}

int cv3_shutdown(void) {
  if (g_shut.exchange(true)) return CV3_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return CV3_OK;   // the runtime was never brought up
  hipDeviceSynchronize();
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& kv : g_graphs) {
    hipGraphExecDestroy(kv.first->exec);
    delete kv.first;
  }
  g_graphs.clear();
  for (auto& kv : g_blocks) {
    for (hipEvent_t ev : kv.second.events) hipEventDestroy(ev);
    hipFree(kv.first);
  }
  g_blocks.clear();
  g_free.clear();
  g_in_use = g_cached = 0;
  for (hipStream_t st : g_thread_streams) hipStreamDestroy(st);
  g_thread_streams.clear();
  g_tls_stream = nullptr;
  for (auto& kv : g_user_streams) hipStreamDestroy(kv.first);
  g_user_streams.clear();
  for (auto& kv : g_user_events) hipEventDestroy(kv.first);
  g_user_events.clear();
  return CV3_OK;
}

int cv3_live_handles(int64_t* streams, int64_t* events, int64_t* graphs, int64_t* blocks) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (streams) *streams = (int64_t)(g_thread_streams.size() + g_user_streams.size());
  if (events) {
    size_t n = g_user_events.size();
    for (auto& kv : g_blocks) n += kv.second.events.size();
    *events = (int64_t)n;
  }
  if (graphs) *graphs = (int64_t)g_graphs.size();
  if (blocks) *blocks = (int64_t)g_blocks.size();
  return CV3_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Graph-safe zero fill (a kernel, never hipMemsetAsync).
// ---------------------------------------------------------------------------
__global__ void k_fill_zero(uint32_t* __restrict__ p, int64_t words) {
  const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = i0; i < words; i += step) p[i] = 0u;
}

__global__ void k_fill_zero_bytes(uint8_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

extern "C" int cv3_fill_zero(void* dst, size_t bytes, cv3_stream_t s) {
  CV3_ALIVE();
  if (!bytes) return CV3_OK;
  hipStream_t st = stream_of(s);
  const int64_t words = (int64_t)(bytes / 4);
  if (words) {
    int64_t blocks = std::min<int64_t>(ceil_div(words, 256), 4096);
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)blocks), dim3(256), 0, st, (uint32_t*)dst, words);
    CV3_LAUNCHED();
  }
  const int64_t tail = (int64_t)(bytes - words * 4);
  if (tail) {
    hipLaunchKernelGGL(k_fill_zero_bytes, dim3(1), dim3(64), 0, st, (uint8_t*)dst + words * 4, tail);
    CV3_LAUNCHED();
  }
  return CV3_OK;
}

// ---------------------------------------------------------------------------
// Host replica of PyTorch's CPU generator (MT19937, init_genrand seeding),
// used for the fixed ODE noise and the NSF dither.  Host code only.
// ---------------------------------------------------------------------------
namespace {
struct TorchMT {
  uint32_t s[624];
  int pos;
  explicit TorchMT(uint64_t seed) {
    s[0] = (uint32_t)(seed & 0xFFFFFFFFu);
    for (int i = 1; i < 624; ++i) s[i] = 1812433253u * (s[i - 1] ^ (s[i - 1] >> 30)) + (uint32_t)i;
    pos = 624;
  }
  void regen() {
    for (int i = 0; i < 624; ++i) {
      const uint32_t y = (s[i] & 0x80000000u) | (s[(i + 1) % 624] & 0x7FFFFFFFu);
      s[i] = s[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
    }
    pos = 0;
  }
  uint32_t next() {
    if (pos >= 624) regen();
    uint32_t y = s[pos++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9D2C5680u;
    y ^= (y << 15) & 0xEFC60000u;
    y ^= y >> 18;
    return y;
  }
  float uniform_f32() { return (float)(next() & 0xFFFFFFu) * (1.0f / 16777216.0f); }
  double uniform_f64() {
    const uint64_t hi = next(), lo = next();
    const uint64_t v = (hi << 32) | lo;
    return (double)(v & ((1ull << 53) - 1)) * (1.0 / 9007199254740992.0);
  }
};

void box_muller16(float* d) {
  double u[16];
  for (int i = 0; i < 16; ++i) u[i] = d[i];
  for (int j = 0; j < 8; ++j) {
    const double r = std::sqrt(-2.0 * std::log(1.0 - u[j]));
    const double th = 2.0 * M_PI * u[j + 8];
    d[j] = (float)(r * std::cos(th));
    d[j + 8] = (float)(r * std::sin(th));
  }
}
}  // namespace

extern "C" {

int cv3_mt_create(uint64_t seed, void** gen) {
  *gen = new TorchMT(seed);
  return CV3_OK;
}

int cv3_mt_destroy(void* gen) {
  delete reinterpret_cast<TorchMT*>(gen);
  return CV3_OK;
}

int cv3_mt_uniform_f32(void* gen, int64_t n, float* out) {
  TorchMT* g = reinterpret_cast<TorchMT*>(gen);
  for (int64_t i = 0; i < n; ++i) out[i] = g->uniform_f32();
  return CV3_OK;
}

// torch.randn semantics on a generator: below 16 elements the scalar
// normal_distribution<double> path, else 16-wide normal_fill with the last 16
// elements recomputed from fresh uniforms when n % 16 != 0.
int cv3_mt_normal_f32(void* gen, int64_t n, float* out) {
  TorchMT* g = reinterpret_cast<TorchMT*>(gen);
  if (n <= 0) return CV3_OK;
  if (n < 16) {
    for (int64_t i = 0; i < n; i += 2) {
      const double u0 = g->uniform_f64(), u1 = g->uniform_f64();
      const double r = std::sqrt(-2.0 * std::log1p(-u1));
      const double th = 2.0 * M_PI * u0;
      out[i] = (float)(r * std::cos(th));
      if (i + 1 < n) out[i + 1] = (float)(r * std::sin(th));
    }
    return CV3_OK;
  }
  for (int64_t i = 0; i < n; ++i) out[i] = g->uniform_f32();
  const int64_t full = n / 16 * 16;
  for (int64_t i = 0; i < full; i += 16) box_muller16(out + i);
  if (n % 16) {
    float* t = out + n - 16;
    for (int i = 0; i < 16; ++i) t[i] = g->uniform_f32();
    box_muller16(t);
  }
  return CV3_OK;
}

}  // extern "C"
