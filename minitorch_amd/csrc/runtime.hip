// Library-wide host plumbing: the thread-local error string, the version
// query, and the runtime the Python package (or any C caller) needs so that no
// other GPU framework is required: device selection, a caching device-memory
// allocator, host/device copies, a fill kernel, streams, events and HIP-graph
// capture/replay.
//
// The reference keeps every Tensor's data in a NumPy array it owns
// (tensor.py:50-61); these entry points give a caller the same ownership of
// device memory: mtx_malloc / mtx_free back minitorch_amd's DeviceArray.
#include "mtx_common.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace mtx {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int attn_scratch(void** out);  // attn.hip: the no-allocation backward's delta array

namespace {

// ---------------------------------------------------------------------------
// Caching allocator.
//
// Blocks are rounded (512 B granules up to 1 MiB, 2 MiB granules above) and
// never split; a freed block goes to a free list and is handed out again for a
// request of the same rounded size (or up to 1/4 larger).  Reuse follows
// stream order: the library issues all work of one process on one stream at
// a time, so memory freed after the last kernel that uses it was *issued* is
// safe to hand to the next kernel issued on that stream.  A caller that uses
// several streams synchronises before freeing memory another stream still
// reads.
//
// Graph pools.  While a stream is being captured into a HIP graph
// (mtx_graph_begin .. mtx_graph_end), every block freed goes to that graph's
// private pool (pool id = capture id) and allocations draw from that pool
// first.  Blocks a recorded graph may read or write are therefore never given
// to work issued outside the graph while the graph exists; mtx_graph_destroy
// returns the pool's free blocks to the general pool, and blocks of a
// destroyed pool that are freed later go there too.
// ---------------------------------------------------------------------------
struct Block {
  size_t size;
  int pool;
};

struct Allocator {
  std::mutex mu;
  std::unordered_map<void*, Block> live;
  std::map<int, std::multimap<size_t, void*>> free_lists;  // pool -> size -> ptr
  std::unordered_map<void*, Block> cached;                 // free blocks, by ptr
  std::vector<int> live_pools{0};
  int capture_pool = 0;  // pool of the capture in progress (0: none)
  int next_pool = 1;
  size_t bytes_live = 0, bytes_cached = 0;

  static size_t round(size_t n) {
    if (n == 0) n = 1;
    if (n <= (1u << 20)) return (n + 511) & ~(size_t)511;
    const size_t g = (size_t)2 << 20;
    return (n + g - 1) / g * g;
  }
  bool pool_alive(int p) const {
    for (int q : live_pools)
      if (q == p) return true;
    return false;
  }
  void* take(int pool, size_t n) {
    auto fl = free_lists.find(pool);
    if (fl == free_lists.end()) return nullptr;
    auto it = fl->second.lower_bound(n);
    if (it == fl->second.end() || it->first > n + n / 4) return nullptr;
    void* p = it->second;
    fl->second.erase(it);
    auto c = cached.find(p);
    bytes_cached -= c->second.size;
    live[p] = Block{c->second.size, pool};
    bytes_live += c->second.size;
    cached.erase(c);
    return p;
  }
  void put(void* p, Block b) {
    free_lists[b.pool].emplace(b.size, p);
    cached[p] = b;
    bytes_cached += b.size;
  }
  // hipFree every cached block of the general pool (caller holds mu; the
  // device is synchronised first so no issued kernel still uses them)
  hipError_t release_general() {
    hipError_t rc = hipDeviceSynchronize();
    if (rc != hipSuccess) return rc;
    auto fl = free_lists.find(0);
    if (fl == free_lists.end()) return hipSuccess;
    for (auto& kv : fl->second) {
      auto c = cached.find(kv.second);
      bytes_cached -= c->second.size;
      cached.erase(c);
      rc = hipFree(kv.second);
      if (rc != hipSuccess) return rc;
    }
    fl->second.clear();
    return hipSuccess;
  }
};

Allocator& alloc() {
  static Allocator* a = new Allocator();  // never destroyed: frees may come at interpreter exit
  return *a;
}

// ---------------------------------------------------------------------------
// fill: count elements of `width` bytes (1, 2, 4 or 8) set to the low bytes of
// `pattern`; 16-byte chunks with the pattern replicated, byte stores for the
// unaligned head and tail
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fill_kernel(uint8_t* __restrict__ dst, size_t nbytes, size_t head,
                                                   size_t nchunk, uint4 rep, uint64_t pattern, int width) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t c = i; c < nchunk; c += stride) reinterpret_cast<uint4*>(dst + head)[c] = rep;
  const size_t tail0 = head + nchunk * 16;
  for (size_t b = i; b < head + (nbytes - tail0); b += stride) {
    const size_t off = b < head ? b : tail0 + (b - head);
    dst[off] = (uint8_t)(pattern >> (8 * (off % width)));
  }
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" const char* mtx_last_error(void) { return mtx::g_err; }

extern "C" const char* mtx_version(void) { return "minitorch_amd 0.2 (gfx950)"; }

// ---------------------------------------------------------------------------
// devices
// ---------------------------------------------------------------------------
extern "C" int mtx_device_count(int* n) {
  MTX_CHECK_ARG(n != nullptr, "n: null pointer");
  *n = 0;
  int c = 0;
  const hipError_t rc = hipGetDeviceCount(&c);
  if (rc == hipErrorNoDevice) return MTX_OK;  // no GPU: zero devices, not an error
  MTX_HIP(rc);
  *n = c;
  return MTX_OK;
}

extern "C" int mtx_device_init(int device) {
  int n = 0;
  int rc = mtx_device_count(&n);
  if (rc) return rc;
  MTX_CHECK_ARG(device >= 0 && device < n, "device %d not present (%d visible)", device, n);
  MTX_HIP(hipSetDevice(device));
  void* p = nullptr;
  return attn_scratch(&p);  // per-device set-up of the no-allocation backward
}

extern "C" int mtx_device_sync(void) {
  MTX_HIP(hipDeviceSynchronize());
  return MTX_OK;
}

// ---------------------------------------------------------------------------
// memory
// ---------------------------------------------------------------------------
extern "C" int mtx_malloc(void** out, size_t bytes) {
  MTX_CHECK_ARG(out != nullptr, "out: null pointer");
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  const size_t n = Allocator::round(bytes);
  void* p = nullptr;
  if (A.capture_pool) p = A.take(A.capture_pool, n);
  if (!p) p = A.take(0, n);
  if (p) {
    if (A.capture_pool) A.live[p].pool = A.capture_pool;
    *out = p;
    return MTX_OK;
  }
  hipError_t rc = hipMalloc(&p, n);
  if (rc == hipErrorOutOfMemory && !A.capture_pool) {
    (void)hipGetLastError();
    rc = A.release_general();
    if (rc == hipSuccess) rc = hipMalloc(&p, n);
  }
  if (rc != hipSuccess) {
    (void)hipGetLastError();
    return fail(MTX_ERR_HIP, "mtx_malloc(%zu bytes): %s (in use %zu, cached %zu bytes)", bytes,
                hipGetErrorString(rc), A.bytes_live, A.bytes_cached);
  }
  A.live[p] = Block{n, A.capture_pool};
  A.bytes_live += n;
  *out = p;
  return MTX_OK;
}

extern "C" int mtx_free(void* p) {
  if (!p) return MTX_OK;
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  auto it = A.live.find(p);
  MTX_CHECK_ARG(it != A.live.end(), "mtx_free(%p): not a live mtx_malloc block", p);
  Block b = it->second;
  A.live.erase(it);
  A.bytes_live -= b.size;
  if (A.capture_pool) b.pool = A.capture_pool;
  else if (!A.pool_alive(b.pool)) b.pool = 0;
  A.put(p, b);
  return MTX_OK;
}

extern "C" int mtx_empty_cache(void) {
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  MTX_CHECK_ARG(A.capture_pool == 0, "mtx_empty_cache during graph capture");
  MTX_HIP(A.release_general());
  return MTX_OK;
}

extern "C" int mtx_memory_stats(size_t* in_use, size_t* cached) {
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  if (in_use) *in_use = A.bytes_live;
  if (cached) *cached = A.bytes_cached;
  return MTX_OK;
}

extern "C" int mtx_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (!bytes) return MTX_OK;
  MTX_CHECK_ARG(dst && src, "null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  MTX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st));
  MTX_HIP(hipStreamSynchronize(st));  // the host buffer may be reused on return
  return MTX_OK;
}

extern "C" int mtx_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
  if (!bytes) return MTX_OK;
  MTX_CHECK_ARG(dst && src, "null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  MTX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st));
  MTX_HIP(hipStreamSynchronize(st));  // the values are on the host on return
  return MTX_OK;
}

extern "C" int mtx_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (!bytes) return MTX_OK;
  MTX_CHECK_ARG(dst && src, "null pointer");
  MTX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
  return MTX_OK;
}

extern "C" int mtx_fill(void* dst, size_t count, uint64_t pattern, int width, void* stream) {
  MTX_CHECK_ARG(width == 1 || width == 2 || width == 4 || width == 8, "width %d not in {1,2,4,8}", width);
  if (!count) return MTX_OK;
  MTX_CHECK_ARG(dst != nullptr, "dst: null pointer");
  MTX_CHECK_ARG(((uintptr_t)dst % width) == 0, "dst must be aligned to the element width");
  const size_t nbytes = count * width;
  const uintptr_t a = (uintptr_t)dst;
  size_t head = (16 - (a & 15)) & 15;
  if (head > nbytes) head = nbytes;
  const size_t nchunk = (nbytes - head) / 16;
  // chunk byte j sits at element phase j % width (head is a multiple of width)
  uint8_t bytes16[16];
  for (int j = 0; j < 16; ++j) bytes16[j] = (uint8_t)(pattern >> (8 * (j % width)));
  uint4 rep;
  std::memcpy(&rep, bytes16, 16);
  const size_t work = nchunk > (nbytes - nchunk * 16) ? nchunk : (nbytes - nchunk * 16);
  size_t blocks = (work + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint8_t*>(dst), nbytes, head, nchunk, rep, pattern, width);
  MTX_LAUNCHED();
  return MTX_OK;
}

// ---------------------------------------------------------------------------
// streams and events (default priority only)
// ---------------------------------------------------------------------------
extern "C" int mtx_stream_create(void** out) {
  MTX_CHECK_ARG(out != nullptr, "out: null pointer");
  hipStream_t s = nullptr;
  MTX_HIP(hipStreamCreate(&s));
  *out = s;
  return MTX_OK;
}

extern "C" int mtx_stream_destroy(void* s) {
  if (s) MTX_HIP(hipStreamDestroy(static_cast<hipStream_t>(s)));
  return MTX_OK;
}

extern "C" int mtx_stream_sync(void* s) {
  MTX_HIP(hipStreamSynchronize(static_cast<hipStream_t>(s)));
  return MTX_OK;
}

extern "C" int mtx_event_create(void** out) {
  MTX_CHECK_ARG(out != nullptr, "out: null pointer");
  hipEvent_t e = nullptr;
  MTX_HIP(hipEventCreate(&e));
  *out = e;
  return MTX_OK;
}

extern "C" int mtx_event_destroy(void* e) {
  if (e) MTX_HIP(hipEventDestroy(static_cast<hipEvent_t>(e)));
  return MTX_OK;
}

extern "C" int mtx_event_record(void* e, void* stream) {
  MTX_CHECK_ARG(e != nullptr, "event: null pointer");
  MTX_HIP(hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(stream)));
  return MTX_OK;
}

extern "C" int mtx_event_elapsed_ms(void* start, void* end, float* ms) {
  MTX_CHECK_ARG(start && end && ms, "null pointer");
  MTX_HIP(hipEventSynchronize(static_cast<hipEvent_t>(end)));
  MTX_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
  return MTX_OK;
}

extern "C" int mtx_stream_wait_event(void* stream, void* e) {
  MTX_CHECK_ARG(e != nullptr, "event: null pointer");
  MTX_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(e), 0));
  return MTX_OK;
}

// ---------------------------------------------------------------------------
// HIP graphs.  One capture at a time per process; the captured stream must
// not be the null stream.  Replays may go to any stream (the package replays
// on the null stream, where its eager work runs).
// ---------------------------------------------------------------------------
namespace {
struct GraphRec {
  hipGraph_t graph;
  hipGraphExec_t exec;
  int pool;
};

// A graph pool ends (its graph destroyed, or its capture failed): it leaves
// the live list and its free blocks join the general pool; blocks of it still
// in use go to the general pool when freed (mtx_free checks pool_alive).
void retire_pool(Allocator& A, int pool) {
  std::lock_guard<std::mutex> lk(A.mu);
  for (size_t i = 0; i < A.live_pools.size(); ++i)
    if (A.live_pools[i] == pool) {
      A.live_pools.erase(A.live_pools.begin() + i);
      break;
    }
  auto fl = A.free_lists.find(pool);
  if (fl != A.free_lists.end()) {
    for (auto& kv : fl->second) {
      A.cached[kv.second].pool = 0;
      A.free_lists[0].emplace(kv.first, kv.second);
    }
    A.free_lists.erase(pool);
  }
}
}  // namespace

extern "C" int mtx_graph_begin(void* stream) {
  MTX_CHECK_ARG(stream != nullptr, "graph capture needs a created stream (not the null stream)");
  Allocator& A = alloc();
  {
    std::lock_guard<std::mutex> lk(A.mu);
    MTX_CHECK_ARG(A.capture_pool == 0, "a graph capture is already in progress");
    A.capture_pool = A.next_pool++;
    A.live_pools.push_back(A.capture_pool);
  }
  const hipError_t rc = hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeRelaxed);
  if (rc != hipSuccess) {
    int pool;
    {
      std::lock_guard<std::mutex> lk(A.mu);
      pool = A.capture_pool;
      A.capture_pool = 0;
    }
    retire_pool(A, pool);
    (void)hipGetLastError();
    return fail(MTX_ERR_HIP, "hipStreamBeginCapture: %s", hipGetErrorString(rc));
  }
  return MTX_OK;
}

extern "C" int mtx_graph_end(void* stream, void** out) {
  MTX_CHECK_ARG(stream != nullptr && out != nullptr, "null pointer");
  Allocator& A = alloc();
  int pool;
  {
    std::lock_guard<std::mutex> lk(A.mu);
    MTX_CHECK_ARG(A.capture_pool != 0, "no graph capture in progress");
    pool = A.capture_pool;
    A.capture_pool = 0;
  }
  // on failure (a capture invalidated by an illegal call, an instantiation
  // error) the capture's pool ends here: nothing will replay it
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g);
  if (ec != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    retire_pool(A, pool);
    (void)hipGetLastError();  // reported here, not by the next launch check
    return fail(MTX_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(ec));
  }
  hipGraphExec_t ex = nullptr;
  const hipError_t rc = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (rc != hipSuccess) {
    (void)hipGraphDestroy(g);
    retire_pool(A, pool);
    (void)hipGetLastError();
    return fail(MTX_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(rc));
  }
  *out = new GraphRec{g, ex, pool};
  return MTX_OK;
}

extern "C" int mtx_graph_launch(void* graph, void* stream) {
  MTX_CHECK_ARG(graph != nullptr, "graph: null pointer");
  MTX_HIP(hipGraphLaunch(static_cast<GraphRec*>(graph)->exec, static_cast<hipStream_t>(stream)));
  return MTX_OK;
}

extern "C" int mtx_graph_destroy(void* graph) {
  if (!graph) return MTX_OK;
  GraphRec* r = static_cast<GraphRec*>(graph);
  MTX_HIP(hipDeviceSynchronize());  // no replay of it is still running
  MTX_HIP(hipGraphExecDestroy(r->exec));
  MTX_HIP(hipGraphDestroy(r->graph));
  retire_pool(alloc(), r->pool);
  delete r;
  return MTX_OK;
}
