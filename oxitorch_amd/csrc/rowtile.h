// Register-resident row tiles for the row-wise kernels (norms, softmax).
//
// A row of H floats (H % 4 == 0, 16-byte aligned rows) is spread over a row
// group of TPR threads: thread t holds float4 number k*TPR + t for k < NV, so
// each load instruction of the group reads TPR*16 consecutive bytes (fully
// coalesced). Out-of-range float4s are zero-filled and never stored.
// Rows are streamed: loads and stores are non-temporal (each row byte crosses
// HBM once per kernel, so caching it would only evict reusable data; measured
// +8% copy bandwidth on MI355X).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace oxi {

typedef float f4 __attribute__((ext_vector_type(4)));

template <int TPR, int NV>
struct RowTile {
  f4 v[NV];

  __device__ __forceinline__ void load(const float* __restrict__ row, int h4, int t) {
    const f4* p = reinterpret_cast<const f4*>(row);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * TPR + t;
      v[k] = (c < h4) ? __builtin_nontemporal_load(p + c) : f4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ row, int h4, int t) const {
    f4* p = reinterpret_cast<f4*>(row);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c = k * TPR + t;
      if (c < h4) __builtin_nontemporal_store(v[k], p + c);
    }
  }
};

}  // namespace oxi
