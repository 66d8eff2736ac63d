// Runtime half of the C ABI: device init, a stream-aware caching allocator,
// copies, streams, events, HIP graphs, thread-local error text, and the host-side
// replica of PyTorch's CPU MT19937 generator (randn / rand).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
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

static thread_local hipStream_t g_tls_stream = nullptr;

hipStream_t stream_of(cv3_stream_t s) {
  if (s) return reinterpret_cast<hipStream_t>(s);
  if (!g_tls_stream) {
    // Default priority only: streams of different priorities are avoided.
    if (hipStreamCreateWithFlags(&g_tls_stream, hipStreamNonBlocking) != hipSuccess) g_tls_stream = nullptr;
  }
  return g_tls_stream;
}

// ---------------------------------------------------------------------------
// Caching allocator.  hipFree synchronises the whole device, so the drop-in
// per-op path (which allocates temporaries on every call) keeps freed blocks in
// size-class free lists.  A freed block remembers an event recorded on the
// freeing thread's stream; a later allocation from another stream waits on it.
// ---------------------------------------------------------------------------
struct Block {
  size_t size;
  hipEvent_t ready;
  hipStream_t stream;
};

static std::mutex g_mu;
static std::multimap<size_t, void*> g_free;            // size class -> ptr
static std::unordered_map<void*, Block> g_blocks;      // every live or cached block
static size_t g_in_use = 0, g_cached = 0;

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

}  // namespace cv3

using namespace cv3;

extern "C" {

const char* cv3_last_error(void) { return g_error.c_str(); }

int cv3_init(int device) {
  int n = 0;
  CV3_HIP(hipGetDeviceCount(&n));
  CV3_REQUIRE(n > 0, CV3_EHIP, "no HIP device is visible");
  CV3_REQUIRE(device >= 0 && device < n, CV3_EINVAL, "device %d out of range (have %d)", device, n);
  CV3_HIP(hipSetDevice(device));
  CV3_HIP(hipFree(nullptr));
  return CV3_OK;
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
  const size_t sz = size_class(bytes ? bytes : 1);
  hipStream_t cur = stream_of(nullptr);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_free.find(sz);
    if (it != g_free.end()) {
      void* p = it->second;
      g_free.erase(it);
      Block& b = g_blocks[p];
      if (b.stream != cur) hipStreamWaitEvent(cur, b.ready, 0);
      g_cached -= sz;
      g_in_use += sz;
      *ptr = p;
      return CV3_OK;
    }
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess) {
    // Out of memory: release the cache and try once more.
    cv3_empty_cache();
    (void)hipGetLastError();
    e = hipMalloc(&p, sz);
  }
  if (e != hipSuccess) return fail(CV3_EHIP, "hipMalloc(%zu) failed: %s", sz, hipGetErrorString(e));
  hipEvent_t ev;
  CV3_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  std::lock_guard<std::mutex> lk(g_mu);
  g_blocks[p] = Block{sz, ev, cur};
  g_in_use += sz;
  *ptr = p;
  return CV3_OK;
}

int cv3_free(void* ptr) {
  if (!ptr) return CV3_OK;
  hipStream_t cur = stream_of(nullptr);
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_blocks.find(ptr);
  CV3_REQUIRE(it != g_blocks.end(), CV3_EINVAL, "cv3_free of a pointer not from cv3_malloc");
  Block& b = it->second;
  b.stream = cur;
  CV3_HIP(hipEventRecord(b.ready, cur));
  g_free.emplace(b.size, ptr);
  g_in_use -= b.size;
  g_cached += b.size;
  return CV3_OK;
}

int cv3_empty_cache(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& kv : g_free) {
    auto it = g_blocks.find(kv.second);
    if (it != g_blocks.end()) {
      hipEventSynchronize(it->second.ready);
      hipEventDestroy(it->second.ready);
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
  if (!bytes) return CV3_OK;
  hipStream_t st = stream_of(s);
  CV3_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st));
  CV3_HIP(hipStreamSynchronize(st));
  return CV3_OK;
}

int cv3_copy_d2h(void* dst, const void* src, size_t bytes, cv3_stream_t s) {
  if (!bytes) return CV3_OK;
  hipStream_t st = stream_of(s);
  CV3_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st));
  CV3_HIP(hipStreamSynchronize(st));
  return CV3_OK;
}

int cv3_copy_d2d(void* dst, const void* src, size_t bytes, cv3_stream_t s) {
  if (!bytes) return CV3_OK;
  CV3_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_of(s)));
  return CV3_OK;
}

int cv3_stream_create(cv3_stream_t* s) {
  hipStream_t h;
  CV3_HIP(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
  *s = reinterpret_cast<cv3_stream_t>(h);
  return CV3_OK;
}

int cv3_stream_destroy(cv3_stream_t s) {
  if (s) CV3_HIP(hipStreamDestroy(reinterpret_cast<hipStream_t>(s)));
  return CV3_OK;
}

int cv3_stream_sync(cv3_stream_t s) {
  CV3_HIP(hipStreamSynchronize(stream_of(s)));
  return CV3_OK;
}

int cv3_device_sync(void) {
  CV3_HIP(hipDeviceSynchronize());
  return CV3_OK;
}

int cv3_event_create(void** ev) {
  hipEvent_t e;
  CV3_HIP(hipEventCreate(&e));
  *ev = e;
  return CV3_OK;
}

int cv3_event_destroy(void* ev) {
  if (ev) CV3_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
  return CV3_OK;
}

int cv3_event_record(void* ev, cv3_stream_t s) {
  CV3_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), stream_of(s)));
  return CV3_OK;
}

int cv3_stream_wait_event(cv3_stream_t s, void* ev) {
  CV3_REQUIRE(ev, CV3_EINVAL, "null event");
  CV3_HIP(hipStreamWaitEvent(stream_of(s), reinterpret_cast<hipEvent_t>(ev), 0));
  return CV3_OK;
}

int cv3_event_elapsed_ms(void* ev0, void* ev1, float* ms) {
  CV3_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev1)));
  CV3_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(ev0), reinterpret_cast<hipEvent_t>(ev1)));
  return CV3_OK;
}

int cv3_graph_begin(cv3_stream_t s) {
  CV3_HIP(hipStreamBeginCapture(stream_of(s), hipStreamCaptureModeThreadLocal));
  return CV3_OK;
}

int cv3_graph_end(cv3_stream_t s, void** exec) {
  hipGraph_t g = nullptr;
  CV3_HIP(hipStreamEndCapture(stream_of(s), &g));
  hipGraphExec_t x = nullptr;
  hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return fail(CV3_EHIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
  *exec = x;
  return CV3_OK;
}

int cv3_graph_launch(void* exec, cv3_stream_t s) {
  CV3_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), stream_of(s)));
  return CV3_OK;
}

int cv3_graph_destroy(void* exec) {
  if (exec) CV3_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec)));
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
