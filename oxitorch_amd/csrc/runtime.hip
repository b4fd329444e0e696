// Runtime half of liboxihip: device selection, the library stream, a
// stream-ordered caching allocator for device storage and workspaces, copies,
// events and the thread-local error slot.
//
// All kernels of the library run on ONE stream per process (default priority),
// so a freed block can be handed to the next allocation without waiting: any
// later use is queued behind every earlier use on the same stream.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include <cstdlib>

#include "internal.h"

namespace oxi {
namespace {

thread_local std::string g_last_error;

// Device scratch of the allocation-free entry point (oxi_layer_norm_bwd_noalloc):
// OXI_NOALLOC_SCRATCH_BYTES on every device the library runs on, held until
// the process ends. In host code `scratch` is only a stand-in for the symbol;
// its device address comes from hipGetSymbolAddress at init (one per device,
// kept in Runtime::scratch) and is the only way host code refers to it.
static __device__ __align__(256) unsigned char scratch[OXI_NOALLOC_SCRATCH_BYTES];

struct Runtime {
  std::mutex mu;
  int device = -1;
  int cus = 0;
  hipStream_t stream = nullptr;
  hipStream_t side = nullptr;  // default priority, see side_stream()
  int* guard = nullptr;  // device int, see guard_flag()
  int64_t* readback = nullptr;  // pinned host slot, see readback_slot()
  std::mutex readback_mu;
  // caching allocator state
  std::multimap<size_t, void*> free_blocks;  // rounded size -> block
  std::unordered_map<void*, size_t> live;    // block -> rounded size
  size_t bytes_in_use = 0;
  size_t bytes_cached = 0;
  int fail_after = 0;  // debug hook
  std::vector<hipEvent_t> events;  // pooled ordering events, see take_event()
  std::unordered_map<int, void*> scratch;  // device -> device address of `scratch`
  std::mutex scratch_mu;  // held by an allocation-free call from its first launch to its last
};

Runtime& rt() {
  static Runtime* r = new Runtime();  // never destroyed: outlives static dtors
  return *r;
}

size_t round_size(size_t n) {
  if (n <= (size_t(1) << 20)) return (n + 511) & ~size_t(511);
  return (n + (size_t(2) << 20) - 1) & ~((size_t(2) << 20) - 1);
}

int init_locked(Runtime& r, int device) {
  if (r.device == device && r.stream) return OXI_OK;
  if (r.device >= 0 && r.device != device)
    return fail(OXI_INVALID_ARGUMENT,
                "liboxihip is already bound to device %d; one device per process", r.device);
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return fail(OXI_OTHER, "no HIP device available (hipGetDeviceCount: %s)",
                e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  if (device < 0 || device >= n)
    return fail(OXI_INVALID_ARGUMENT, "device index %d out of range for %d HIP device(s)", device, n);
  if ((e = hipSetDevice(device)) != hipSuccess) return fail_hip(e, "hipSetDevice");
  if (!r.scratch.count(device)) {
    void* sp = nullptr;
    if ((e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch))) != hipSuccess || !sp)
      return fail_hip(e == hipSuccess ? hipErrorInvalidSymbol : e, "hipGetSymbolAddress(scratch)");
    r.scratch[device] = sp;
  }
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
    return fail_hip(e, "hipGetDeviceProperties");
  r.cus = prop.multiProcessorCount;
  if ((e = hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking)) != hipSuccess)
    return fail_hip(e, "hipStreamCreateWithFlags");
  if ((e = hipStreamCreateWithFlags(&r.side, hipStreamNonBlocking)) != hipSuccess)
    return fail_hip(e, "hipStreamCreateWithFlags(side)");
  if ((e = hipMalloc(&r.guard, sizeof(int))) != hipSuccess) return fail_hip(e, "hipMalloc(guard)");
  if ((e = hipMemsetAsync(r.guard, 0, sizeof(int), r.stream)) != hipSuccess)
    return fail_hip(e, "hipMemsetAsync(guard)");
  // coherent: a kernel's system-scope store reaches the host while it runs
  if ((e = hipHostMalloc(reinterpret_cast<void**>(&r.readback), sizeof(int64_t), hipHostMallocCoherent)) != hipSuccess)
    return fail_hip(e, "hipHostMalloc(readback)");
  *r.readback = 0;
  if ((e = hipStreamSynchronize(r.stream)) != hipSuccess) return fail_hip(e, "hipStreamSynchronize");
  r.device = device;
  return OXI_OK;
}

void release_cache_locked(Runtime& r) {
  for (auto& kv : r.free_blocks) (void)hipFree(kv.second);
  r.free_blocks.clear();
  r.bytes_cached = 0;
}

}  // namespace

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int fail_hip(hipError_t err, const char* what) {
  return fail(OXI_OTHER, "%s failed: %s", what, hipGetErrorString(err));
}

int fail_alloc(const char* what) {
  const std::string cause = g_last_error;
  return fail(OXI_OTHER, "%s: %s", what, cause.c_str());
}

bool initialised() {
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  return r.stream != nullptr;
}

void* noalloc_scratch() {
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  auto it = r.scratch.find(r.device);
  return it == r.scratch.end() ? nullptr : it->second;
}

std::mutex& noalloc_mutex() { return rt().scratch_mu; }

// The device an implicit initialisation binds: OXI_HIP_DEVICE (a device
// index), else 0; -1 with the error set when the variable is not an index.
int env_device() {
  const char* e = std::getenv("OXI_HIP_DEVICE");
  if (!e || !*e) return 0;
  char* end = nullptr;
  const long v = std::strtol(e, &end, 10);
  if (*end != '\0' || v < 0 || v > 1 << 20) {
    fail(OXI_INVALID_ARGUMENT, "OXI_HIP_DEVICE=\"%s\" is not a device index", e);
    return -1;
  }
  return (int)v;
}

bool ensure_init() {
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  if (r.stream) return true;
  const int dev = env_device();
  return dev >= 0 && init_locked(r, dev) == OXI_OK;
}

hipStream_t stream() { return rt().stream; }
hipStream_t side_stream() { return rt().side; }

hipEvent_t take_event() {
  Runtime& r = rt();
  {
    std::lock_guard<std::mutex> lk(r.mu);
    if (!r.events.empty()) {
      hipEvent_t e = r.events.back();
      r.events.pop_back();
      return e;
    }
  }
  // device-scope release: both streams work on device memory, and a default
  // (system-scope) record writes back and invalidates the caches each time
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventReleaseToDevice) != hipSuccess) return nullptr;
  return e;
}

void give_event(hipEvent_t e) {
  if (!e) return;
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  r.events.push_back(e);
}
int* guard_flag() { return rt().guard; }
int64_t* readback_slot() { return rt().readback; }
std::mutex& readback_mutex() { return rt().readback_mu; }
int cu_count() { return rt().cus > 0 ? rt().cus : 256; }

void* ws_alloc(size_t bytes) {
  void* p = nullptr;
  if (oxi_hip_alloc(bytes, &p) != OXI_OK) return nullptr;
  return p;
}

void ws_free(void* p) { (void)oxi_hip_free(p); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, what);
  return OXI_OK;
}

}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_hip_init(int device) {
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  return init_locked(r, device);
}

int oxi_hip_device_count(int* count) {
  if (!count) return fail(OXI_INVALID_ARGUMENT, "count must not be NULL");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return OXI_OK;
}

int oxi_hip_current_device(int* device) {
  if (!device) return fail(OXI_INVALID_ARGUMENT, "device must not be NULL");
  *device = rt().device;
  return OXI_OK;
}

int oxi_hip_default_device(int* device) {
  if (!device) return fail(OXI_INVALID_ARGUMENT, "device must not be NULL");
  const int bound = rt().device;
  const int d = bound >= 0 ? bound : env_device();
  if (d < 0) return OXI_INVALID_ARGUMENT;
  *device = d;
  return OXI_OK;
}

int oxi_hip_alloc(size_t bytes, void** out) {
  if (!out) return fail(OXI_INVALID_ARGUMENT, "out must not be NULL");
  *out = nullptr;
  if (bytes == 0) return OXI_OK;
  OXI_CHECK_INIT();
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  if (r.fail_after > 0 && --r.fail_after == 0)
    return fail(OXI_OTHER, "device allocation of %zu bytes failed (injected by oxi_hip_debug_fail_alloc_after)", bytes);
  const size_t sz = round_size(bytes);
  auto it = r.free_blocks.find(sz);
  void* p = nullptr;
  if (it != r.free_blocks.end()) {
    p = it->second;
    r.free_blocks.erase(it);
    r.bytes_cached -= sz;
  } else {
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      // Give the cache back to the driver and retry once. The stream must be
      // idle before blocks are released to the driver.
      (void)hipStreamSynchronize(r.side);
      (void)hipStreamSynchronize(r.stream);
      release_cache_locked(r);
      e = hipMalloc(&p, sz);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(OXI_OTHER, "device allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
      }
    }
  }
  r.live[p] = sz;
  r.bytes_in_use += sz;
  *out = p;
  return OXI_OK;
}

int oxi_hip_free(void* ptr) {
  if (!ptr) return OXI_OK;
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  auto it = r.live.find(ptr);
  if (it == r.live.end()) return fail(OXI_INVALID_ARGUMENT, "oxi_hip_free: %p was not allocated by liboxihip", ptr);
  const size_t sz = it->second;
  r.live.erase(it);
  r.bytes_in_use -= sz;
  r.free_blocks.emplace(sz, ptr);
  r.bytes_cached += sz;
  return OXI_OK;
}

int oxi_hip_empty_cache(void) {
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  if (r.side) (void)hipStreamSynchronize(r.side);
  if (r.stream) (void)hipStreamSynchronize(r.stream);
  release_cache_locked(r);
  return OXI_OK;
}

int oxi_hip_memory_stats(size_t* in_use, size_t* cached) {
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  if (in_use) *in_use = r.bytes_in_use;
  if (cached) *cached = r.bytes_cached;
  return OXI_OK;
}

int oxi_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return OXI_OK;
  if (!dst || !src) return fail(OXI_INVALID_ARGUMENT, "memcpy_h2d: NULL pointer");
  OXI_CHECK_INIT();
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream());
  if (e != hipSuccess) return fail_hip(e, "hipMemcpyAsync(h2d)");
  // The source is pageable caller memory that may be reused right after the
  // call returns; wait so the copy has consumed it.
  e = hipStreamSynchronize(stream());
  return e == hipSuccess ? OXI_OK : fail_hip(e, "hipStreamSynchronize(h2d)");
}

int oxi_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return OXI_OK;
  if (!dst || !src) return fail(OXI_INVALID_ARGUMENT, "memcpy_d2h: NULL pointer");
  OXI_CHECK_INIT();
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream());
  if (e != hipSuccess) return fail_hip(e, "hipMemcpyAsync(d2h)");
  e = hipStreamSynchronize(stream());
  return e == hipSuccess ? OXI_OK : fail_hip(e, "hipStreamSynchronize(d2h)");
}

int oxi_hip_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return OXI_OK;
  if (!dst || !src) return fail(OXI_INVALID_ARGUMENT, "memcpy_d2d: NULL pointer");
  OXI_CHECK_INIT();
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream());
  return e == hipSuccess ? OXI_OK : fail_hip(e, "hipMemcpyAsync(d2d)");
}

int oxi_hip_sync(void) {
  OXI_CHECK_INIT();
  hipError_t e = hipStreamSynchronize(side_stream());
  if (e == hipSuccess) e = hipStreamSynchronize(stream());
  if (e != hipSuccess) return fail_hip(e, "hipStreamSynchronize");
  int flag = 0;
  e = hipMemcpy(&flag, guard_flag(), sizeof(int), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return fail_hip(e, "hipMemcpy(guard)");
  if (flag != 0) {
    const int zero = 0;
    (void)hipMemcpy(guard_flag(), &zero, sizeof(int), hipMemcpyHostToDevice);
    if (flag & 3)
      return fail(OXI_OUT_OF_BOUNDS, "a device kernel met an index outside its valid range; the affected output was written with zeros");
    return fail(OXI_OTHER, "masked_select: a tile's offset wait did not finish; that tile's picks were not written");
  }
  return OXI_OK;
}

const char* oxi_hip_last_error(void) { return g_last_error.c_str(); }

int oxi_hip_stream(void** s) {
  if (!s) return fail(OXI_INVALID_ARGUMENT, "stream must not be NULL");
  OXI_CHECK_INIT();
  *s = (void*)stream();
  return OXI_OK;
}

int oxi_hip_event_create(void** ev) {
  if (!ev) return fail(OXI_INVALID_ARGUMENT, "event must not be NULL");
  OXI_CHECK_INIT();
  // timing only: no system-scope fence, which would write back and
  // invalidate the caches at every record and perturb the kernels timed
  hipEvent_t e;
  hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
  if (err != hipSuccess) return fail_hip(err, "hipEventCreateWithFlags");
  *ev = (void*)e;
  return OXI_OK;
}

int oxi_hip_event_record(void* ev) {
  OXI_CHECK_INIT();
  hipError_t err = hipEventRecord((hipEvent_t)ev, stream());
  return err == hipSuccess ? OXI_OK : fail_hip(err, "hipEventRecord");
}

int oxi_hip_event_elapsed_ms(void* a, void* b, float* ms) {
  if (!ms) return fail(OXI_INVALID_ARGUMENT, "ms must not be NULL");
  hipError_t err = hipEventSynchronize((hipEvent_t)b);
  if (err != hipSuccess) return fail_hip(err, "hipEventSynchronize");
  err = hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b);
  return err == hipSuccess ? OXI_OK : fail_hip(err, "hipEventElapsedTime");
}

int oxi_hip_event_destroy(void* ev) {
  if (!ev) return OXI_OK;
  hipError_t err = hipEventDestroy((hipEvent_t)ev);
  return err == hipSuccess ? OXI_OK : fail_hip(err, "hipEventDestroy");
}

int oxi_hip_device_props(oxi_device_props* out) {
  if (!out) return fail(OXI_INVALID_ARGUMENT, "device_props: out must not be NULL");
  OXI_CHECK_INIT();
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, rt().device);
  if (e != hipSuccess) return fail_hip(e, "hipGetDeviceProperties");
  std::memset(out, 0, sizeof *out);
  out->compute_units = p.multiProcessorCount;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_bits = p.memoryBusWidth;
  out->l2_bytes = p.l2CacheSize;
  out->hbm_bytes = (int64_t)p.totalGlobalMem;
  std::snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
  return OXI_OK;
}

int oxi_hip_debug_fail_alloc_after(int n) {
  Runtime& r = rt();
  std::lock_guard<std::mutex> lk(r.mu);
  r.fail_after = n < 0 ? 0 : n;
  return OXI_OK;
}

}  // extern "C"
