// Internal helpers shared by the liboxihip translation units: status/error
// plumbing, the library stream, workspace allocation and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>

#include "oxihip.h"

namespace oxi {

// Sets the thread-local error message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a failing HIP call to OXI_OTHER with its name and HIP error string.
int fail_hip(hipError_t err, const char* what);
// Stream of the initialised device; initialises device 0 on first use.
// Returns nullptr and sets the error when no device can be initialised.
bool ensure_init();
// True once the library is bound to a device (no initialisation here).
bool initialised();
hipStream_t stream();
// Device address of the bound device's OXI_NOALLOC_SCRATCH_BYTES scratch
// array (from hipGetSymbolAddress at init); nullptr before init. Every call
// that uses it on one device shares it: callers hold noalloc_mutex() from
// their first launch that touches it to their last, so calls from several
// host threads do not interleave on the library stream.
void* noalloc_scratch();
std::mutex& noalloc_mutex();
// A second stream, default priority, for work that overlaps the library
// stream (e.g. the embedding VJP's id sort queued at forward time). Work on
// it first waits for an event recorded on the library stream, and the
// library stream waits for an event recorded after it, so memory from the
// stream-ordered allocator stays safe.
hipStream_t side_stream();
// Ordering events without timing, pooled: give_event() returns one for reuse
// instead of destroying it, because destroying an event the device has not
// reached yet can make the host wait for it. Re-recording a pooled event is
// safe once every wait on its previous record has been queued.
hipEvent_t take_event();
void give_event(hipEvent_t e);
// Workspace from the caching allocator (stream-ordered reuse, no sync).
void* ws_alloc(size_t bytes);
void ws_free(void* p);
// Device-side guard flag: kernels that meet an index outside its range set it;
// oxi_hip_sync() reports it. Pointer to one int in device memory.
int* guard_flag();
// A pinned host int64 that a kernel can store one result to (a data-dependent
// size, say), read by the host after the stream is synchronised: no copy call.
// Callers hold readback_mutex() from the launch until the read.
int64_t* readback_slot();
std::mutex& readback_mutex();
// Checks the launch that just happened.
int check_launch(const char* what);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Number of compute units of the current device (cached).
int cu_count();

// A small RAII workspace holder.
struct Workspace {
  void* p = nullptr;
  explicit Workspace(size_t bytes) : p(bytes ? ws_alloc(bytes) : nullptr) {}
  ~Workspace() { if (p) ws_free(p); }
  Workspace(const Workspace&) = delete;
  Workspace& operator=(const Workspace&) = delete;
  template <typename T> T* as() const { return static_cast<T*>(p); }
};

}  // namespace oxi

#define OXI_CHECK_INIT()                                   \
  do {                                                     \
    if (!oxi::ensure_init()) return OXI_OTHER;             \
  } while (0)

// ---------------------------------------------------------------------------
// Device-side reductions over a wave64 (CDNA: 64 lanes per wavefront).

#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)
namespace oxi {

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Sum across the `TPR` threads of a row group. TPR is 64 (one wave, no LDS)
// or a multiple of 64 equal to the block size (LDS combine in fixed order, so
// every thread gets the same, deterministic result). `lds` holds TPR/64 floats.
template <int TPR, typename T>
__device__ __forceinline__ T group_sum(T v, T* lds) {
  v = wave_sum(v);
  if constexpr (TPR > 64) {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    v = lds[0];
#pragma unroll
    for (int i = 1; i < TPR / 64; ++i) v += lds[i];
  }
  return v;
}

// group_sum / group_max without the leading barrier, which only keeps a
// reduction from overwriting slots that waves still read from the one
// before. Callers give consecutive reductions alternate slot sets (`lds`
// holds TPR/64 values each): every wave reads a reduction's slots before it
// reaches the next reduction's barrier, so a set is free again by the
// reduction after that. The first reduction of a kernel may take either set.
template <int TPR, typename T>
__device__ __forceinline__ T group_sum_once(T v, T* lds) {
  v = wave_sum(v);
  if constexpr (TPR > 64) {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    v = lds[0];
#pragma unroll
    for (int i = 1; i < TPR / 64; ++i) v += lds[i];
  }
  return v;
}

template <int TPR>
__device__ __forceinline__ float group_max(float v, float* lds) {
  v = wave_max(v);
  if constexpr (TPR > 64) {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    v = lds[0];
#pragma unroll
    for (int i = 1; i < TPR / 64; ++i) v = fmaxf(v, lds[i]);
  }
  return v;
}

template <int TPR>
__device__ __forceinline__ float group_max_once(float v, float* lds) {
  v = wave_max(v);
  if constexpr (TPR > 64) {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    v = lds[0];
#pragma unroll
    for (int i = 1; i < TPR / 64; ++i) v = fmaxf(v, lds[i]);
  }
  return v;
}

}  // namespace oxi
#endif
