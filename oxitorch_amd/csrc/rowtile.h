// Register-resident row tiles for the row-wise kernels (norms, softmax).
//
// A row of H floats (H % 4 == 0, 16-byte aligned rows) is spread over a row
// group of TPR threads: thread t holds float4 number k*TPR + t for k < NV, so
// each load instruction of the group reads TPR*16 consecutive bytes (fully
// coalesced). Out-of-range float4s are zero-filled and never stored.
// Rows are streamed (see ld_stream / st_stream below).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace oxi {

typedef float f4 __attribute__((ext_vector_type(4)));

// Streaming accesses: each tensor byte crosses memory once per kernel.
// Loads are non-temporal (a one-pass stream should not evict what the next
// kernel reuses). Stores take a per-launch hint NT from nt_stores(): plain
// stores leave a producer's output in the 256 MB Infinity Cache for the
// kernel that consumes it next; non-temporal ones suit outputs too large to
// stay there and small ones, whose end-of-kernel L2 write-back dominates.
#ifndef OXI_NT_LOADS
#define OXI_NT_LOADS 1
#endif

template <typename T>
__device__ __forceinline__ T ld_stream(const T* p) {
  if constexpr (OXI_NT_LOADS) return __builtin_nontemporal_load(p);
  else return *p;
}

// The hint is a template parameter: with a run-time flag the compiler merges
// the two stores of `if (nt) ... else ...` into one and drops the hint.
template <bool NT, typename T>
__device__ __forceinline__ void st_stream(T v, T* p) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Row helpers shared by the softmax kernels and the norm + softmax VJP.
constexpr float NEG_INF = -__builtin_huge_valf();

__device__ __forceinline__ float max4(const f4& v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }
__device__ __forceinline__ float min4(const f4& v) { return fminf(fminf(v.x, v.y), fminf(v.z, v.w)); }
__device__ __forceinline__ float sum4(const f4& v) { return (v.x + v.y) + (v.z + v.w); }
__device__ __forceinline__ f4 exp4(const f4& v) { return f4{expf(v.x), expf(v.y), expf(v.z), expf(v.w)}; }

// Store hint for a launch writing `bytes` of output: plain between 32 MB and
// 320 MB, non-temporal otherwise. Measured on MI355X (fwd+bwd steps): plain
// stores gain 8% on a chain of 50 MB tensors and 1-3% on 268 MB ones, and
// lose 16-35% on 0.5-1 GB outputs and ~10% on 12 MB ones.
#ifndef OXI_NT_STORE_LO
#define OXI_NT_STORE_LO (32 << 20)
#endif
#ifndef OXI_NT_STORE_HI
#define OXI_NT_STORE_HI (320 << 20)
#endif
inline bool nt_stores(int64_t bytes) { return bytes < (int64_t)OXI_NT_STORE_LO || bytes > (int64_t)OXI_NT_STORE_HI; }

// Threads per block of a row kernel whose rows take TPR threads: 256 (several
// rows per block) when TPR divides 256, else one row per block of TPR.
constexpr int row_block_threads(int tpr) { return (256 % tpr == 0) ? 256 : tpr; }

// (TPR, NV) for rows of h4 float4s, encoded TPR*10 + NV; 0 when the row does
// not fit in registers. Rows keep several float4s per lane: measured on
// MI355X, one float4 per lane (192 threads per 768-float row, 1024 per
// 4096-float row) made the layer-norm forward 30% slower, the block-wide
// reductions over many waves costing more than the access pattern gains;
// 512 x 2 for a 4096-float row measured the same as 256 x 4 (layer-norm
// forward at (16384, 4096): 88.8-89.5 us against 87.7-89.3 us).
inline int pick_row_cfg(int64_t h4) {
  if (h4 <= 64) return 641;
  if (h4 <= 128) return 642;
  if (h4 <= 192) return 643;
  if (h4 <= 256) return 644;
  if (h4 <= 512) return 2562;
  if (h4 <= 1024) return 2564;
  if (h4 <= 2048) return 2568;
  return 0;
}

template <int TPR, int NV>
struct RowTile {
  f4 v[NV];

  __device__ __forceinline__ void load(const float* __restrict__ row, int h4, int t) {
    const f4* p = reinterpret_cast<const f4*>(row);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * TPR + t;
      v[k] = (c < h4) ? ld_stream(p + c) : f4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // Every lane loads: lanes past the row (c >= h4) re-read its last float4,
  // so the loads issue unconditionally; the caller zeroes those lanes at use.
  // NT = false: plain loads, for rows the caller reads again soon.
  template <bool NT = true>
  __device__ __forceinline__ void load_clamped(const float* __restrict__ row, int h4, int t) {
    const f4* p = reinterpret_cast<const f4*>(row);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const f4* q = p + min(k * TPR + t, h4 - 1);
      if constexpr (NT) v[k] = ld_stream(q);
      else v[k] = *q;
    }
  }
  template <bool NT>
  __device__ __forceinline__ void store(float* __restrict__ row, int h4, int t) const {
    f4* p = reinterpret_cast<f4*>(row);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * TPR + t;
      if (c < h4) st_stream<NT>(v[k], p + c);
    }
  }
};

}  // namespace oxi
