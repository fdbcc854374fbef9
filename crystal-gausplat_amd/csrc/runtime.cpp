// Device, stream, buffer and error state: the kept gs_* symbols of the Metal
// bridge (src/metal/bridge.mm:362-482) re-implemented over HIP.
//
// MetalBuffer (src/core/buffer.cr:14-143) wraps a shared-storage MTLBuffer;
// here a buffer handle owns an explicit device allocation and host <-> device
// traffic is an explicit copy on the library stream.
#include <hip/hip_runtime.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/gs_hip.h"
#include "internal.h"

namespace gs {
namespace {

thread_local std::string t_last_error;
std::mutex g_init_mu;
// set (release) once the device and stream are ready; read (acquire) without
// the lock on every entry point's fast path
std::atomic<bool> g_inited{false};
hipStream_t g_stream = nullptr;
int g_device = 0;
char g_name[256] = "unavailable";

struct Buffer {
  void* dev;
  int64_t size;
};

struct ProfRec {
  std::string name;
  double flops, bytes;
  hipEvent_t a, b;
};
bool g_prof = false;
bool g_prof_shape = false;
std::vector<ProfRec> g_recs;
std::vector<hipEvent_t> g_pool;
size_t g_pool_used = 0;
struct ProfAgg {
  std::string name;
  int64_t launches;
  double ms, flops, bytes;
};
std::vector<ProfAgg> g_agg;

hipEvent_t pool_event() {
  if (g_pool_used == g_pool.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    g_pool.push_back(e);
  }
  return g_pool[g_pool_used++];
}

}  // namespace

bool prof_on() { return g_prof; }
bool prof_per_shape() { return g_prof_shape; }

hipEvent_t prof_start(hipStream_t s) {
  if (!g_prof) return nullptr;
  hipEvent_t e = pool_event();
  if (e) hipEventRecord(e, s);
  return e;
}

void prof_stop(hipStream_t s, hipEvent_t start, const char* kernel, double flops, double bytes) {
  if (!g_prof || !start) return;
  hipEvent_t e = pool_event();
  if (!e) return;
  hipEventRecord(e, s);
  g_recs.push_back(ProfRec{kernel, flops, bytes, start, e});
}

void set_error(const std::string& msg) { t_last_error = msg; }
const char* last_error() { return t_last_error.c_str(); }

int ensure_device() {
  if (g_inited.load(std::memory_order_acquire)) return 0;
  return gs_init_device();
}

hipStream_t default_stream() {
  ensure_device();
  return g_stream;
}

}  // namespace gs

using namespace gs;

extern "C" {

const char* gs_hip_last_error(void) { return gs::last_error(); }

int32_t gs_init_device(void) {
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_inited.load(std::memory_order_relaxed)) return 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    set_error("gs_init_device: no HIP device");
    return -1;
  }
  if (hipSetDevice(g_device) != hipSuccess) {
    set_error("gs_init_device: hipSetDevice failed");
    return -1;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, g_device) == hipSuccess) {
    strncpy(g_name, prop.name, sizeof(g_name) - 1);
    g_name[sizeof(g_name) - 1] = 0;
  }
  // Op-level calls take their scratch from the device's default memory pool
  // (hipMallocAsync / hipFreeAsync). With the pool's default release
  // threshold of 0 every synchronisation hands the memory back to the driver,
  // so a caller that synchronises after each op would pay a fresh allocation
  // on every call; keep up to 256 MB cached in the pool instead.
  hipMemPool_t pool;
  if (hipDeviceGetDefaultMemPool(&pool, g_device) == hipSuccess) {
    uint64_t keep = (uint64_t)256 << 20;
    (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
  }
  // Default-priority, non-blocking stream.
  if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) {
    set_error("gs_init_device: stream creation failed");
    return -2;
  }
  g_inited.store(true, std::memory_order_release);
  return 0;
}

void* gs_get_device(void) {
  if (ensure_device()) return nullptr;
  return (void*)(intptr_t)(g_device + 1);
}

void* gs_get_command_queue(void) {
  if (ensure_device()) return nullptr;
  return (void*)g_stream;
}

void gs_synchronize(void) {
  if (ensure_device()) return;
  hipStreamSynchronize(g_stream);
}

const char* gs_device_name(void) {
  ensure_device();
  return g_name;
}

int32_t gs_max_threads_per_threadgroup(void) { return 1024; }

int64_t gs_recommended_working_set_size(void) {
  if (ensure_device()) return 0;
  size_t fr = 0, tot = 0;
  if (hipMemGetInfo(&fr, &tot) != hipSuccess) return 0;
  return (int64_t)tot;
}

int32_t gs_has_unified_memory(void) { return 0; }

void* gs_create_buffer(int64_t size, int32_t storage_mode) {
  (void)storage_mode;
  if (size <= 0) {
    set_error("gs_create_buffer: size must be positive");
    return nullptr;
  }
  if (ensure_device()) return nullptr;
  Buffer* b = new Buffer{nullptr, size};
  if (hipMalloc(&b->dev, (size_t)size) != hipSuccess) {
    set_error("gs_create_buffer: hipMalloc failed");
    delete b;
    return nullptr;
  }
  return b;
}

void gs_release_buffer(void* handle) {
  if (!handle) return;
  Buffer* b = (Buffer*)handle;
  hipStreamSynchronize(g_stream);
  hipFree(b->dev);
  delete b;
}

void* gs_buffer_contents(void* handle) {
  if (!handle) return nullptr;
  return ((Buffer*)handle)->dev;
}

void gs_buffer_write(void* handle, void* data, int64_t size) {
  if (!handle || !data) return;
  Buffer* b = (Buffer*)handle;
  if (size > b->size) {
    set_error("gs_buffer_write: size exceeds buffer");
    return;
  }
  hipMemcpyAsync(b->dev, data, (size_t)size, hipMemcpyHostToDevice, g_stream);
  hipStreamSynchronize(g_stream);
}

void gs_buffer_read(void* handle, void* dest, int64_t size) {
  if (!handle || !dest) return;
  Buffer* b = (Buffer*)handle;
  if (size > b->size) {
    set_error("gs_buffer_read: size exceeds buffer");
    return;
  }
  hipMemcpyAsync(dest, b->dev, (size_t)size, hipMemcpyDeviceToHost, g_stream);
  hipStreamSynchronize(g_stream);
}

void gs_buffer_sync(void* handle) { (void)handle; }

int32_t gs_hip_profile_begin(int32_t per_shape) {
  if (ensure_device()) return -2;
  g_prof_shape = per_shape != 0;
  g_recs.clear();
  g_agg.clear();
  g_pool_used = 0;
  g_prof = true;
  return 0;
}

int32_t gs_hip_profile_end(void) {
  g_prof = false;
  std::map<std::string, size_t> idx;
  g_agg.clear();
  for (auto& r : g_recs) {
    if (hipEventSynchronize(r.b) != hipSuccess) {
      set_error("profile_end: event synchronisation failed");
      return -3;
    }
    float ms = 0.f;
    hipEventElapsedTime(&ms, r.a, r.b);
    auto it = idx.find(r.name);
    if (it == idx.end()) {
      idx[r.name] = g_agg.size();
      g_agg.push_back(ProfAgg{r.name, 0, 0.0, 0.0, 0.0});
      it = idx.find(r.name);
    }
    ProfAgg& a = g_agg[it->second];
    a.launches += 1;
    a.ms += ms;
    a.flops += r.flops;
    a.bytes += r.bytes;
  }
  g_recs.clear();
  g_pool_used = 0;
  return (int32_t)g_agg.size();
}

int32_t gs_hip_profile_entry(int32_t i, char* name, int32_t cap, int64_t* launches, double* ms,
                             double* flops, double* bytes) {
  if (i < 0 || i >= (int32_t)g_agg.size()) return -1;
  const ProfAgg& a = g_agg[i];
  if (name && cap > 0) {
    strncpy(name, a.name.c_str(), cap - 1);
    name[cap - 1] = 0;
  }
  if (launches) *launches = a.launches;
  if (ms) *ms = a.ms;
  if (flops) *flops = a.flops;
  if (bytes) *bytes = a.bytes;
  return 0;
}

int32_t gs_buffer_write_async(void* handle, const void* host, int64_t size, int64_t offset,
                              void* stream) {
  GS_REQUIRE(handle && host, "gs_buffer_write_async: null argument");
  Buffer* b = (Buffer*)handle;
  GS_REQUIRE(size >= 0 && offset >= 0 && offset + size <= b->size,
             "gs_buffer_write_async: range exceeds the buffer");
  if (size == 0) return 0;
  GS_CHECK_HIP(hipMemcpyAsync((char*)b->dev + offset, host, (size_t)size, hipMemcpyHostToDevice,
                              (hipStream_t)stream));
  return 0;
}

int32_t gs_buffer_read_async(void* handle, void* host, int64_t size, int64_t offset,
                             void* stream) {
  GS_REQUIRE(handle && host, "gs_buffer_read_async: null argument");
  Buffer* b = (Buffer*)handle;
  GS_REQUIRE(size >= 0 && offset >= 0 && offset + size <= b->size,
             "gs_buffer_read_async: range exceeds the buffer");
  if (size == 0) return 0;
  GS_CHECK_HIP(hipMemcpyAsync(host, (const char*)b->dev + offset, (size_t)size,
                              hipMemcpyDeviceToHost, (hipStream_t)stream));
  return 0;
}

void* gs_host_alloc(int64_t size) {
  if (size <= 0) {
    set_error("gs_host_alloc: size must be positive");
    return nullptr;
  }
  if (ensure_device()) return nullptr;
  void* p = nullptr;
  if (hipHostMalloc(&p, (size_t)size, hipHostMallocDefault) != hipSuccess) {
    set_error("gs_host_alloc: hipHostMalloc failed");
    return nullptr;
  }
  return p;
}

void gs_host_free(void* ptr) {
  if (ptr) hipHostFree(ptr);
}

int32_t gs_stream_synchronize(void* stream) {
  if (ensure_device()) return -2;
  GS_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

void gs_buffer_copy(void* src_handle, void* dst_handle, int64_t size) {
  if (!src_handle || !dst_handle) return;
  Buffer* s = (Buffer*)src_handle;
  Buffer* d = (Buffer*)dst_handle;
  if (size > s->size || size > d->size) {
    set_error("gs_buffer_copy: size exceeds buffer");
    return;
  }
  hipMemcpyAsync(d->dev, s->dev, (size_t)size, hipMemcpyDeviceToDevice, g_stream);
}

}  // extern "C"
