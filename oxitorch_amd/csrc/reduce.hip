// Dim reductions (sum, mean, max, min, argmax, argmin, norm) over strided
// tensors, with the semantics of ReduceKind::reduce_strip
// (crates/oxi-tensor/src/ops.rs:246-285) and Tensor::reduce
// (crates/oxi-tensor/src/lib.rs:519-576).
//
// Two kernels:
//   strip-contiguous (reduced dim has stride 1): one wave64 per strip, lanes
//     stride the strip, shuffle-tree combine;
//   strided (any other stride): one thread per output element walking its
//     strip in order; for sum/mean/norm this is the reference's own
//     sequential f32 fold, so the result is bit-identical to it. Adjacent
//     threads own adjacent output elements, so a column reduction of a
//     row-major tensor reads coalesced rows.
// max/min fold with fmaxf/fminf (NaN ignored, as f32::max/min); argmax/argmin
// keep the first strict winner starting from index 0, so a NaN at index 0
// sticks and later NaNs are ignored. Indices are written as floats.
#include <algorithm>

#include "internal.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;
constexpr int MAXD = OXI_MAX_DIMS;

struct RPlan {
  int nd;              // dims other than the reduced one
  int64_t size[MAXD];  // row-major order of the remaining dims
  int64_t st[MAXD];
  int64_t len;         // reduced dim size
  int64_t rst;         // reduced dim stride
};

__device__ __forceinline__ int64_t base_of(const RPlan& p, int64_t e) {
  int64_t off = 0;
  for (int d = p.nd - 1; d >= 0; --d) {
    const int64_t c = e % p.size[d];
    e /= p.size[d];
    off += c * p.st[d];
  }
  return off;
}

// Accumulator state per kind.
template <int K>
struct Acc {
  float v;
  int64_t i;
  __device__ __forceinline__ void init(float first) {
    if constexpr (K == OXI_REDUCE_MAX) v = -__builtin_huge_valf();
    else if constexpr (K == OXI_REDUCE_MIN) v = __builtin_huge_valf();
    else if constexpr (K == OXI_REDUCE_ARGMAX || K == OXI_REDUCE_ARGMIN) v = first;
    else v = 0.f;
    i = 0;
  }
  __device__ __forceinline__ void add(float a, int64_t k) {
    if constexpr (K == OXI_REDUCE_SUM || K == OXI_REDUCE_MEAN) v += a;
    else if constexpr (K == OXI_REDUCE_NORM) v += a * a;
    else if constexpr (K == OXI_REDUCE_MAX) v = fmaxf(v, a);
    else if constexpr (K == OXI_REDUCE_MIN) v = fminf(v, a);
    else if constexpr (K == OXI_REDUCE_ARGMAX) { if (a > v) { v = a; i = k; } }
    else { if (a < v) { v = a; i = k; } }
  }
  __device__ __forceinline__ float result(int64_t len) const {
    if constexpr (K == OXI_REDUCE_MEAN) return v / (float)len;
    else if constexpr (K == OXI_REDUCE_NORM) return sqrtf(v);
    else if constexpr (K == OXI_REDUCE_ARGMAX || K == OXI_REDUCE_ARGMIN) return (float)i;
    else return v;
  }
};

template <int K>
__global__ __launch_bounds__(BS) void reduce_strided_k(const float* __restrict__ x, RPlan p, int64_t nout,
                                                       float* __restrict__ out) {
  for (int64_t e = (int64_t)blockIdx.x * BS + threadIdx.x; e < nout; e += (int64_t)gridDim.x * BS) {
    const float* s = x + base_of(p, e);
    Acc<K> a;
    a.init(p.len ? s[0] : 0.f);
    for (int64_t k = 0; k < p.len; ++k) a.add(s[k * p.rst], k);
    out[e] = a.result(p.len);
  }
}

// Four adjacent outputs per thread when they are adjacent in memory (the
// last remaining dim has stride 1): 16-byte loads walk the strip. Same
// sequential fold per output as reduce_strided_k. Not used for arg* kinds.
template <int K>
__global__ __launch_bounds__(BS) void reduce_strided_vec_k(const float* __restrict__ x, RPlan p, int64_t nout4,
                                                           float* __restrict__ out) {
  for (int64_t e4 = (int64_t)blockIdx.x * BS + threadIdx.x; e4 < nout4; e4 += (int64_t)gridDim.x * BS) {
    const float* s = x + base_of(p, e4 * 4);
    f4 a;
    if constexpr (K == OXI_REDUCE_MAX) a = f4{-__builtin_huge_valf(), -__builtin_huge_valf(), -__builtin_huge_valf(), -__builtin_huge_valf()};
    else if constexpr (K == OXI_REDUCE_MIN) a = f4{__builtin_huge_valf(), __builtin_huge_valf(), __builtin_huge_valf(), __builtin_huge_valf()};
    else a = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int64_t k = 0; k < p.len; ++k) {
      const f4 v = ld_stream(reinterpret_cast<const f4*>(s + k * p.rst));
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if constexpr (K == OXI_REDUCE_SUM || K == OXI_REDUCE_MEAN) a[c] += v[c];
        else if constexpr (K == OXI_REDUCE_NORM) a[c] += v[c] * v[c];
        else if constexpr (K == OXI_REDUCE_MAX) a[c] = fmaxf(a[c], v[c]);
        else a[c] = fminf(a[c], v[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if constexpr (K == OXI_REDUCE_MEAN) a[c] = a[c] / (float)p.len;
      else if constexpr (K == OXI_REDUCE_NORM) a[c] = sqrtf(a[c]);
    }
    *reinterpret_cast<f4*>(out + e4 * 4) = a;
  }
}

// Combine two partial states of a strip; (vb, ib) comes from later positions
// only when ib > ia, so ties go to the smaller index as in the sequential scan.
template <int K>
__device__ __forceinline__ void combine(float& va, int64_t& ia, bool& has_a, float vb, int64_t ib, bool has_b) {
  if constexpr (K == OXI_REDUCE_SUM || K == OXI_REDUCE_MEAN || K == OXI_REDUCE_NORM) va += vb;
  else if constexpr (K == OXI_REDUCE_MAX) va = fmaxf(va, vb);
  else if constexpr (K == OXI_REDUCE_MIN) va = fminf(va, vb);
  else {
    if (!has_b) return;
    if (!has_a) { va = vb; ia = ib; has_a = true; return; }
    const bool better = (K == OXI_REDUCE_ARGMAX) ? (vb > va) : (vb < va);
    if (better || (vb == va && ib < ia)) { va = vb; ia = ib; }
  }
}

// One wave per strip (reduced dim contiguous). For argmax/argmin each lane
// tracks the first winner of its own positions among non-NaN values; a NaN
// at position 0 forces index 0, matching the sequential scan.
template <int K>
__global__ __launch_bounds__(BS) void reduce_contig_k(const float* __restrict__ x, RPlan p, int64_t nout,
                                                      float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t e = ((int64_t)blockIdx.x * BS + threadIdx.x) >> 6;
  if (e >= nout) return;
  const float* s = x + base_of(p, e);
  const int64_t len = p.len;
  float v;
  int64_t idx = 0;
  bool has = false;
  if constexpr (K == OXI_REDUCE_MAX) v = -__builtin_huge_valf();
  else if constexpr (K == OXI_REDUCE_MIN) v = __builtin_huge_valf();
  else v = 0.f;
  for (int64_t k = lane; k < len; k += 64) {
    const float a = s[k];
    if constexpr (K == OXI_REDUCE_SUM || K == OXI_REDUCE_MEAN) v += a;
    else if constexpr (K == OXI_REDUCE_NORM) v += a * a;
    else if constexpr (K == OXI_REDUCE_MAX) v = fmaxf(v, a);
    else if constexpr (K == OXI_REDUCE_MIN) v = fminf(v, a);
    else {
      if (a == a) {
        const bool better = (K == OXI_REDUCE_ARGMAX) ? (a > v) : (a < v);
        if (!has || better) { v = a; idx = k; has = true; }
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float vo = __shfl_xor(v, m, 64);
    const int64_t io = __shfl_xor(idx, m, 64);
    const bool ho = __shfl_xor((int)has, m, 64) != 0;
    combine<K>(v, idx, has, vo, io, ho);
  }
  if (lane == 0) {
    float r;
    if constexpr (K == OXI_REDUCE_MEAN) r = v / (float)len;
    else if constexpr (K == OXI_REDUCE_NORM) r = sqrtf(v);
    else if constexpr (K == OXI_REDUCE_ARGMAX || K == OXI_REDUCE_ARGMIN) r = (s[0] != s[0] || !has) ? 0.f : (float)idx;
    else r = v;
    out[e] = r;
  }
}

template <int K>
int launch(const float* x, const RPlan& p, int64_t nout, float* out) {
  hipStream_t s = stream();
  if (p.rst == 1 && p.len >= 32) {
    const int64_t blocks = ceil_div(nout * 64, BS);
    if (blocks < ((int64_t)1 << 31)) {
      reduce_contig_k<K><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(x, p, nout, out);
      return check_launch("reduce");
    }
  }
  if constexpr (K != OXI_REDUCE_ARGMAX && K != OXI_REDUCE_ARGMIN) {
    // vector path: innermost remaining dim contiguous, every row start 16-byte aligned
    bool vec = p.nd > 0 && p.st[p.nd - 1] == 1 && p.size[p.nd - 1] % 4 == 0 && p.rst % 4 == 0 &&
               (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
    for (int d = 0; d + 1 < p.nd && vec; ++d)
      if (p.st[d] % 4) vec = false;
    if (vec) {
      const int64_t nout4 = nout / 4;
      const int64_t blocks = std::min<int64_t>(ceil_div(nout4, BS), (int64_t)cu_count() * 64);
      reduce_strided_vec_k<K><<<dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(BS), 0, s>>>(x, p, nout4, out);
      return check_launch("reduce");
    }
  }
  const int64_t blocks = std::min<int64_t>(ceil_div(nout, BS), (int64_t)cu_count() * 64);
  reduce_strided_k<K><<<dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(BS), 0, s>>>(x, p, nout, out);
  return check_launch("reduce");
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_reduce(int kind, const float* x, const int64_t* xs, const int64_t* shape, int ndim, int dim, float* out) {
  if (kind < OXI_REDUCE_SUM || kind > OXI_REDUCE_NORM) return fail(OXI_INVALID_ARGUMENT, "unknown reduction kind %d", kind);
  if (ndim < 1 || ndim > MAXD) return fail(OXI_INVALID_ARGUMENT, "reduce: rank %d outside [1, %d]", ndim, MAXD);
  if (dim < 0 || dim >= ndim) return fail(OXI_INVALID_ARGUMENT, "reduce: dim %d out of range for rank %d", dim, ndim);
  if (!shape || !xs) return fail(OXI_INVALID_ARGUMENT, "reduce: NULL shape/strides");
  RPlan p;
  p.nd = 0;
  int64_t nout = 1;
  int64_t total = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return fail(OXI_INVALID_ARGUMENT, "reduce: negative dim size");
    if (shape[d] && total > (((int64_t)1 << 60) / shape[d]))
      return fail(OXI_INVALID_ARGUMENT, "reduce: element count exceeds the kernel limits");
    total *= shape[d];
    if (d == dim) continue;
    p.size[p.nd] = shape[d];
    p.st[p.nd] = xs[d];
    ++p.nd;
    nout *= shape[d];
  }
  p.len = shape[dim];
  p.rst = xs[dim];
  if (p.len == 0) {
    if (kind == OXI_REDUCE_ARGMAX || kind == OXI_REDUCE_ARGMIN)
      return fail(OXI_INVALID_ARGUMENT, "cannot compute argmax/argmin over a zero-length dim");
    if (kind == OXI_REDUCE_MAX || kind == OXI_REDUCE_MIN)
      return fail(OXI_INVALID_ARGUMENT, "cannot compute max/min over a zero-length dim");
  }
  if (nout == 0) return OXI_OK;
  if (!out || (!x && p.len)) return fail(OXI_INVALID_ARGUMENT, "reduce: NULL tensor pointer");
  OXI_CHECK_INIT();
  if (p.len == 0) return oxi_fill(out, nout, 0.f);
  switch (kind) {
    case OXI_REDUCE_SUM: return launch<OXI_REDUCE_SUM>(x, p, nout, out);
    case OXI_REDUCE_MEAN: return launch<OXI_REDUCE_MEAN>(x, p, nout, out);
    case OXI_REDUCE_MAX: return launch<OXI_REDUCE_MAX>(x, p, nout, out);
    case OXI_REDUCE_MIN: return launch<OXI_REDUCE_MIN>(x, p, nout, out);
    case OXI_REDUCE_ARGMAX: return launch<OXI_REDUCE_ARGMAX>(x, p, nout, out);
    case OXI_REDUCE_ARGMIN: return launch<OXI_REDUCE_ARGMIN>(x, p, nout, out);
    default: return launch<OXI_REDUCE_NORM>(x, p, nout, out);
  }
}

}  // extern "C"
