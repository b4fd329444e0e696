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
// exp(z) for z <= 0 (and NaN), as the softmax family needs it (z = x - max,
// or a log-probability): the steps of ROCm's expf -- a two-part product with
// log2(e), exp2 of the reduced argument, an exponent scale, 0 below the log of
// the smallest subnormal -- without its overflow select, which only acts for
// z > 88.7. Two of its thirteen instructions fewer per element.
__device__ __forceinline__ float exp_le0(float z) {
  const float ph = z * 0x1.715476p+0f;                                      // z * log2(e), rounded
  const float pl = fmaf(z, 0x1.4ae0bep-26f, fmaf(z, 0x1.715476p+0f, -ph));  // its residual + log2(e)'s low part
  const float n = __builtin_rintf(ph);
  const float r = __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), (int)n);
  return z < -0x1.9d1da0p+6f ? 0.0f : r;
}
__device__ __forceinline__ f4 exp4(const f4& v) { return f4{exp_le0(v.x), exp_le0(v.y), exp_le0(v.z), exp_le0(v.w)}; }

// v[k] / s for the NV float4s of a row that share the sum s (the softmax's
// exponentials, all >= 0), rounded to nearest like the division operator:
// q = e * (1/s), then twice q + (e - q*s) * (1/s) with the remainder exact by
// FMA, which lands on the rounded quotient whenever it is a normal number
// (Markstein's correction; the first step brings q within an ulp). The
// operator's own sequence recomputes the divisor's scaling and reciprocal for
// every element: 11 instructions against these 5. A wave whose row could give
// a subnormal quotient (an exponential in (0, 2^-100)) or whose sum is outside
// [2^-20, 2^20] (NaN and inf included) divides with the operator.
template <int NV>
__device__ __forceinline__ void div_by_sum(f4 (&v)[NV], float s) {
  // bits(e) - 1 >= bits(2^-100) - 1  <=>  e == 0 or e >= 2^-100 (for e >= 0)
  unsigned lo = 0xffffffffu;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    lo = min(lo, __float_as_uint(v[k].x) - 1u);
    lo = min(lo, __float_as_uint(v[k].y) - 1u);
    lo = min(lo, __float_as_uint(v[k].z) - 1u);
    lo = min(lo, __float_as_uint(v[k].w) - 1u);
  }
  const bool ok = lo >= __float_as_uint(0x1p-100f) - 1u && s >= 0x1p-20f && s <= 0x1p20f;
  if (__all(ok)) {
    const float rs = 1.0f / s;
    auto q1 = [&](float e) {
      float q = e * rs;
      q = fmaf(fmaf(-q, s, e), rs, q);
      return fmaf(fmaf(-q, s, e), rs, q);
    };
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = f4{q1(v[k].x), q1(v[k].y), q1(v[k].z), q1(v[k].w)};
  } else {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = v[k] / s;
  }
}

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
