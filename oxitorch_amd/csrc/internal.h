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
// After a failed oxi_hip_alloc / ws_alloc: OXI_OTHER with `what` (the call
// site) in front of the allocator's own message.
int fail_alloc(const char* what);
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
// A pinned, coherent host int64 that a kernel can store one result to (a
// data-dependent size, say), read by the host after the stream is
// synchronised, or polled while the kernel runs when the kernel stores it
// with system scope: no copy call. Callers hold readback_mutex() from the
// launch until the read.
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

// Float reductions over a full wave64 through DPP lane permutes, which run in
// the VALU pipeline (a __shfl_xor is an LDS-crossbar round trip, and a
// butterfly chains six of them). Within each row of 16 lanes: swap with the
// neighbour (xor 1), then within quads (xor 2), then mirror within halves of
// 8 and within the row; each step combines a lane with a partner lane that
// holds the mirrored partial, so with a commutative op (+, fmaxf) every lane
// ends with the same bits. The four row results are then combined in fixed
// order through readlane, so the result is uniform and deterministic. All
// 64 lanes must be active, as for the butterfly.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;  // quad_perm:[1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // quad_perm:[2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

template <>
__device__ __forceinline__ float wave_sum<float>(float v) {
  v += dpp_f32<DPP_QUAD_XOR1>(v);
  v += dpp_f32<DPP_QUAD_XOR2>(v);
  v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
  v += dpp_f32<DPP_ROW_MIRROR>(v);
  return (readlane_f32(v, 0) + readlane_f32(v, 16)) + (readlane_f32(v, 32) + readlane_f32(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<DPP_QUAD_XOR1>(v));
  v = fmaxf(v, dpp_f32<DPP_QUAD_XOR2>(v));
  v = fmaxf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
  return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)), fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
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

// Two maxima over the group with one barrier (the _once contract above;
// `lds` holds 2 * TPR/64 values).
template <int TPR>
__device__ __forceinline__ void group_max2_once(float& a, float& b, float* lds) {
  a = wave_max(a);
  b = wave_max(b);
  if constexpr (TPR > 64) {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    if (lane == 0) {
      lds[wid] = a;
      lds[TPR / 64 + wid] = b;
    }
    __syncthreads();
    a = lds[0];
    b = lds[TPR / 64];
#pragma unroll
    for (int i = 1; i < TPR / 64; ++i) {
      a = fmaxf(a, lds[i]);
      b = fmaxf(b, lds[TPR / 64 + i]);
    }
  }
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
