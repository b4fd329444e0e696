// Host <-> device transfers that do not stall the library stream.
//
// Uploads go through a ring of page-locked (pinned) host memory: the caller's
// bytes are copied into the next free region on the host, the DMA from that
// region to the device is queued on the library stream, and an event recorded
// after it marks when the region may be reused. The call returns as soon as
// the caller's buffer may be reused, without waiting for the device, so an
// upload of ids or targets overlaps the kernels already queued. Large uploads
// move in chunks, so the host copy of one chunk overlaps the DMA of the
// previous one. Downloads stage through the same ring in the other direction.
//
// An upload of up to KERNEL_COPY_MAX bytes (ids, targets, small parameters)
// goes through a second, small ring and is copied out of it by a kernel on
// the library stream rather than by a DMA engine. A DMA copy on a stream with
// kernels in flight stalled the host for several milliseconds every few
// hundred uploads; a kernel launch queues like any other. The small ring is
// allocated coherent, so the kernel reads what the host wrote, and it is
// small so that its pages stay in the host's caches: the host's copy into
// pinned pages it has not touched lately ran at about 3 GB/s.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <deque>
#include <mutex>
#include <vector>

#include "internal.h"

namespace oxi {
namespace {

constexpr size_t RING_BYTES = size_t(64) << 20;   // pinned staging ring (DMA)
constexpr size_t CHUNK_BYTES = size_t(16) << 20;  // largest single region
constexpr size_t ALIGN = 256;
constexpr size_t SMALL_RING_BYTES = size_t(4) << 20;  // ring of the kernel copies
constexpr size_t KERNEL_COPY_MAX = size_t(1) << 20;   // larger uploads use DMA
constexpr int COPY_BS = 256;
static_assert(SMALL_RING_BYTES >= 2 * KERNEL_COPY_MAX, "small ring holds two largest copies");
// a download keeps two chunks in flight; with four chunks of room their
// regions never need the ring to wait
static_assert(RING_BYTES >= 4 * CHUNK_BYTES, "staging ring too small for double-buffered downloads");

struct Region {
  size_t start, end;
  hipEvent_t done;
};

struct Ring {
  const size_t bytes;
  const unsigned flags;  // hipHostMalloc flags
  std::mutex mu;
  char* buf = nullptr;
  const char* dbuf = nullptr;  // the ring's address for kernels
  size_t head = 0;  // offset after the newest region
  std::deque<Region> inflight;
  std::vector<hipEvent_t> spare;
  Ring(size_t n, unsigned f) : bytes(n), flags(f) {}
};

// never destroyed: they outlive static destructors
Ring& ring() {
  static Ring* r = new Ring(RING_BYTES, hipHostMallocDefault);
  return *r;
}
Ring& small_ring() {
  static Ring* r = new Ring(SMALL_RING_BYTES, hipHostMallocCoherent);
  return *r;
}

int ensure_ring(Ring& r) {
  if (r.buf) return OXI_OK;
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, r.bytes, r.flags);
  if (e != hipSuccess) return fail_hip(e, "hipHostMalloc(staging ring)");
  void* dp = nullptr;
  e = hipHostGetDevicePointer(&dp, p, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return fail_hip(e, "hipHostGetDevicePointer(staging ring)");
  }
  r.buf = static_cast<char*>(p);
  r.dbuf = static_cast<const char*>(dp);
  return OXI_OK;
}

// Hands back the events of regions whose copies have finished, oldest first,
// without waiting: the ring then records few events in flight.
void retire_finished(Ring& r) {
  while (!r.inflight.empty()) {
    const hipError_t q = hipEventQuery(r.inflight.front().done);
    if (q != hipSuccess) {
      (void)hipGetLastError();  // "not ready" is an answer, not a failure
      return;
    }
    r.spare.push_back(r.inflight.front().done);
    r.inflight.pop_front();
  }
  r.head = 0;
}

bool overlaps(const Region& a, size_t s, size_t e) { return a.start < e && s < a.end; }

int retire_front(Ring& r) {
  Region& f = r.inflight.front();
  hipError_t e = hipEventSynchronize(f.done);
  if (e != hipSuccess) return fail_hip(e, "hipEventSynchronize(staging)");
  r.spare.push_back(f.done);
  r.inflight.pop_front();
  if (r.inflight.empty()) r.head = 0;
  return OXI_OK;
}

// Reserves [*start, *start + len) of the ring, waiting for the oldest
// regions to drain when needed. len <= CHUNK_BYTES.
int reserve(Ring& r, size_t len, size_t* start) {
  len = (len + ALIGN - 1) / ALIGN * ALIGN;
  for (;;) {
    size_t s = r.head + len <= r.bytes ? r.head : 0;
    bool busy = false;
    for (const Region& q : r.inflight)
      if (overlaps(q, s, s + len)) {
        busy = true;
        break;
      }
    if (!busy) {
      *start = s;
      r.head = s + len;
      return OXI_OK;
    }
    int rc = retire_front(r);
    if (rc != OXI_OK) return rc;
  }
}

int record(Ring& r, size_t start, size_t len) {
  hipEvent_t ev;
  if (!r.spare.empty()) {
    ev = r.spare.back();
    r.spare.pop_back();
  } else {
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return fail_hip(e, "hipEventCreateWithFlags(staging)");
  }
  hipError_t e = hipEventRecord(ev, stream());
  if (e != hipSuccess) {
    r.spare.push_back(ev);
    return fail_hip(e, "hipEventRecord(staging)");
  }
  r.inflight.push_back({start, start + (len + ALIGN - 1) / ALIGN * ALIGN, ev});
  return OXI_OK;
}

__global__ __launch_bounds__(COPY_BS) void ring_copy_k(const unsigned char* __restrict__ src,
                                                      unsigned char* __restrict__ dst, size_t bytes, int vec) {
  const size_t stride = (size_t)gridDim.x * COPY_BS;
  const size_t tid = (size_t)blockIdx.x * COPY_BS + threadIdx.x;
  size_t done = 0;
  if (vec) {
    const size_t n16 = bytes / 16;
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    for (size_t i = tid; i < n16; i += stride) d4[i] = s4[i];
    done = n16 * 16;
  }
  for (size_t i = done + tid; i < bytes; i += stride) dst[i] = src[i];
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_hip_host_alloc(size_t bytes, void** out) {
  if (!out) return fail(OXI_INVALID_ARGUMENT, "host_alloc: out must not be NULL");
  *out = nullptr;
  if (bytes == 0) return OXI_OK;
  OXI_CHECK_INIT();
  hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    *out = nullptr;
    return fail(OXI_OTHER, "pinned host allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
  }
  return OXI_OK;
}

int oxi_hip_host_free(void* ptr) {
  if (!ptr) return OXI_OK;
  // the caller may still have DMA queued from this buffer: let it finish
  if (ensure_init()) (void)hipStreamSynchronize(stream());
  hipError_t e = hipHostFree(ptr);
  return e == hipSuccess ? OXI_OK : fail_hip(e, "hipHostFree");
}

int oxi_hip_upload(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return OXI_OK;
  if (!dst || !src) return fail(OXI_INVALID_ARGUMENT, "upload: NULL pointer");
  OXI_CHECK_INIT();
  const char* s = static_cast<const char*>(src);
  char* d = static_cast<char*>(dst);
  if (bytes <= KERNEL_COPY_MAX) {
    Ring& r = small_ring();
    std::lock_guard<std::mutex> lk(r.mu);
    int rc = ensure_ring(r);
    if (rc != OXI_OK) return rc;
    retire_finished(r);
    size_t at = 0;
    if ((rc = reserve(r, bytes, &at)) != OXI_OK) return rc;
    std::memcpy(r.buf + at, s, bytes);
    const int vec = (reinterpret_cast<uintptr_t>(dst) % 16 == 0) ? 1 : 0;
    const size_t units = vec ? std::max<size_t>(bytes / 16, 1) : bytes;
    const unsigned blocks = (unsigned)std::min<size_t>((units + COPY_BS - 1) / COPY_BS, 1024);
    ring_copy_k<<<blocks, COPY_BS, 0, stream()>>>(reinterpret_cast<const unsigned char*>(r.dbuf + at),
                                                  static_cast<unsigned char*>(dst), bytes, vec);
    if ((rc = check_launch("upload")) != OXI_OK) return rc;
    return record(r, at, bytes);
  }
  Ring& r = ring();
  std::lock_guard<std::mutex> lk(r.mu);
  int rc = ensure_ring(r);
  if (rc != OXI_OK) return rc;
  for (size_t off = 0; off < bytes; off += CHUNK_BYTES) {
    const size_t len = std::min(CHUNK_BYTES, bytes - off);
    size_t at = 0;
    if ((rc = reserve(r, len, &at)) != OXI_OK) return rc;
    std::memcpy(r.buf + at, s + off, len);
    hipError_t e = hipMemcpyAsync(d + off, r.buf + at, len, hipMemcpyHostToDevice, stream());
    if (e != hipSuccess) return fail_hip(e, "hipMemcpyAsync(upload)");
    if ((rc = record(r, at, len)) != OXI_OK) return rc;
  }
  return OXI_OK;
}

int oxi_hip_memcpy_h2d_async(void* dst, const void* pinned_src, size_t bytes) {
  if (bytes == 0) return OXI_OK;
  if (!dst || !pinned_src) return fail(OXI_INVALID_ARGUMENT, "memcpy_h2d_async: NULL pointer");
  OXI_CHECK_INIT();
  hipError_t e = hipMemcpyAsync(dst, pinned_src, bytes, hipMemcpyHostToDevice, stream());
  return e == hipSuccess ? OXI_OK : fail_hip(e, "hipMemcpyAsync(h2d_async)");
}

int oxi_hip_download(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return OXI_OK;
  if (!dst || !src) return fail(OXI_INVALID_ARGUMENT, "download: NULL pointer");
  OXI_CHECK_INIT();
  Ring& r = ring();
  std::lock_guard<std::mutex> lk(r.mu);
  int rc = ensure_ring(r);
  if (rc != OXI_OK) return rc;
  const char* s = static_cast<const char*>(src);
  char* d = static_cast<char*>(dst);
  // DMA of chunk k+1 is queued before the host copies chunk k out
  struct Pending {
    size_t off, len, at;
  };
  std::deque<Pending> pend;
  auto drain_one = [&]() -> int {
    const Pending p = pend.front();
    pend.pop_front();
    const int rc2 = retire_front(r);  // the oldest region is this chunk's
    if (rc2 != OXI_OK) return rc2;
    std::memcpy(d + p.off, r.buf + p.at, p.len);
    return OXI_OK;
  };
  // earlier uploads still in flight are retired first, so the regions of this
  // download are the oldest from here on
  while (!r.inflight.empty())
    if ((rc = retire_front(r)) != OXI_OK) return rc;
  for (size_t off = 0; off < bytes; off += CHUNK_BYTES) {
    const size_t len = std::min(CHUNK_BYTES, bytes - off);
    size_t at = 0;
    while (pend.size() >= 2)
      if ((rc = drain_one()) != OXI_OK) return rc;
    if ((rc = reserve(r, len, &at)) != OXI_OK) return rc;
    hipError_t e = hipMemcpyAsync(r.buf + at, s + off, len, hipMemcpyDeviceToHost, stream());
    if (e != hipSuccess) return fail_hip(e, "hipMemcpyAsync(download)");
    if ((rc = record(r, at, len)) != OXI_OK) return rc;
    pend.push_back({off, len, at});
  }
  while (!pend.empty())
    if ((rc = drain_one()) != OXI_OK) return rc;
  return OXI_OK;
}

}  // extern "C"
