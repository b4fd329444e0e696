// Strided/broadcast elementwise engine for gfx950: the device replacement of
// iterate::map_n (crates/oxi-tensor/src/iterate.rs:21-75) for the unary and
// binary registries and the fused activations.
//
// The host side of each call builds a Plan: size-1 dims dropped, dims ordered
// by the output's strides, mergeable neighbours coalesced. The plan then
// selects one of four kernels:
//   flat    every operand is contiguous over the whole plan or a broadcast
//           scalar: float4 loads/stores, 4 vectors in flight per thread;
//   rows    the innermost dim is contiguous or broadcast for every operand:
//           one block walks a chunk of one row, offsets computed once per row;
//   tiled   an input is transposed relative to the output (its unit-stride
//           dim is not the output's innermost dim). With float4-aligned
//           operands one wave owns a 32x32 tile and each lane a 4x4 block,
//           read as float4 rows along the input's unit-stride dim and
//           written as float4 columns along the output's innermost dim, so
//           both coalesce with no LDS; otherwise 64x64 tiles go through LDS;
//   generic anything else: per-element index arithmetic.
#include <algorithm>
#include <cstring>

#include "internal.h"
#include "ops.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;
constexpr int MAXD = OXI_MAX_DIMS;

template <int N>
struct Plan {
  int ndim;
  int64_t shape[MAXD];
  int64_t st[N + 1][MAXD];  // [0] = output, [1..N] = inputs
  float* y;
  const float* x[N];
};

template <class F, int N>
__device__ __forceinline__ float apply(const F& f, const float* v) {
  if constexpr (N == 1) return f(v[0]);
  else return f(v[0], v[1]);
}

// ---------------------------------------------------------------------------
// flat: y[i] = f(x0[i or 0], x1[i or 0]) for i < n.

#ifndef OXI_FLAT_U
#define OXI_FLAT_U 1
#endif
constexpr int FLAT_U = OXI_FLAT_U;  // float4s per thread in the flat kernels

template <class F, int N, bool NTS>
__global__ __launch_bounds__(BS) void map_flat_vec_k(F f, Plan<N> p, int64_t n, unsigned bcast_mask) {
  const int64_t n4 = n >> 2;
  const int64_t base = ((int64_t)blockIdx.x * BS * FLAT_U) + threadIdx.x;
  f4 in[N][FLAT_U];
  float sc[N];
#pragma unroll
  for (int k = 0; k < N; ++k) sc[k] = (bcast_mask >> k & 1u) ? p.x[k][0] : 0.f;
#pragma unroll
  for (int u = 0; u < FLAT_U; ++u) {
    const int64_t i = base + (int64_t)u * BS;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      if (bcast_mask >> k & 1u) in[k][u] = f4{sc[k], sc[k], sc[k], sc[k]};
      else if (i < n4) in[k][u] = ld_stream(reinterpret_cast<const f4*>(p.x[k]) + i);
    }
  }
#pragma unroll
  for (int u = 0; u < FLAT_U; ++u) {
    const int64_t i = base + (int64_t)u * BS;
    if (i < n4) {
      f4 r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v[N];
#pragma unroll
        for (int k = 0; k < N; ++k) v[k] = in[k][u][j];
        r[j] = apply<F, N>(f, v);
      }
      st_stream<NTS>(r, reinterpret_cast<f4*>(p.y) + i);
    }
  }
  // scalar tail (n % 4 elements) handled by the first block
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
    const int64_t i = n4 * 4 + threadIdx.x;
    float v[N];
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = (bcast_mask >> k & 1u) ? sc[k] : p.x[k][i];
    p.y[i] = apply<F, N>(f, v);
  }
}

template <class F, int N>
__global__ __launch_bounds__(BS) void map_flat_k(F f, Plan<N> p, int64_t n, unsigned bcast_mask) {
  for (int64_t i = (int64_t)blockIdx.x * BS + threadIdx.x; i < n; i += (int64_t)gridDim.x * BS) {
    float v[N];
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = p.x[k][(bcast_mask >> k & 1u) ? 0 : i];
    p.y[i] = apply<F, N>(f, v);
  }
}

// ---------------------------------------------------------------------------
// rows: innermost dim has stride 0 or 1 for every operand.

template <int N>
__device__ __forceinline__ void row_offsets(const Plan<N>& p, int64_t row, int64_t* off) {
#pragma unroll
  for (int k = 0; k <= N; ++k) off[k] = 0;
  for (int d = p.ndim - 2; d >= 0; --d) {
    const int64_t c = row % p.shape[d];
    row /= p.shape[d];
#pragma unroll
    for (int k = 0; k <= N; ++k) off[k] += c * p.st[k][d];
  }
}

template <class F, int N, bool VEC>
__global__ __launch_bounds__(BS) void map_rows_k(F f, Plan<N> p, int64_t chunks_per_row, int64_t chunk) {
  const int64_t row = blockIdx.x / chunks_per_row;
  const int64_t c0 = (blockIdx.x % chunks_per_row) * chunk;
  const int64_t inner = p.shape[p.ndim - 1];
  int64_t off[N + 1];
  row_offsets<N>(p, row, off);
  const int64_t c1 = min(c0 + chunk, inner);
  if constexpr (VEC) {
    for (int64_t c = c0 + threadIdx.x * 4; c < c1; c += BS * 4) {
      f4 in[N];
#pragma unroll
      for (int k = 0; k < N; ++k) {
        const float* q = p.x[k] + off[k + 1];
        if (p.st[k + 1][p.ndim - 1] == 0) in[k] = f4{q[0], q[0], q[0], q[0]};
        else in[k] = *reinterpret_cast<const f4*>(q + c);
      }
      f4 r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v[N];
#pragma unroll
        for (int k = 0; k < N; ++k) v[k] = in[k][j];
        r[j] = apply<F, N>(f, v);
      }
      *reinterpret_cast<f4*>(p.y + off[0] + c) = r;
    }
  } else {
    for (int64_t c = c0 + threadIdx.x; c < c1; c += BS) {
      float v[N];
#pragma unroll
      for (int k = 0; k < N; ++k) v[k] = p.x[k][off[k + 1] + c * p.st[k + 1][p.ndim - 1]];
      p.y[off[0] + c * p.st[0][p.ndim - 1]] = apply<F, N>(f, v);
    }
  }
}

// ---------------------------------------------------------------------------
// tiled: 64 (dim jd) x 64 (innermost dim) tiles; inputs flagged in tmask are
// read along jd (their unit-stride dim) and transposed through LDS.

constexpr int T = 64;

template <class F, int N>
__global__ __launch_bounds__(BS) void map_tiled_k(F f, Plan<N> p, int jd, unsigned tmask, int64_t tiles_d,
                                                  int64_t tiles_j) {
  __shared__ float tile[N][T][T + 1];
  const int d = p.ndim - 1;
  int64_t b = blockIdx.x;
  const int64_t td = b % tiles_d;
  b /= tiles_d;
  const int64_t tj = b % tiles_j;
  b /= tiles_j;
  // batch offsets over the remaining dims
  int64_t off[N + 1];
#pragma unroll
  for (int k = 0; k <= N; ++k) off[k] = 0;
  for (int q = p.ndim - 2; q >= 0; --q) {
    if (q == jd) continue;
    const int64_t c = b % p.shape[q];
    b /= p.shape[q];
#pragma unroll
    for (int k = 0; k <= N; ++k) off[k] += c * p.st[k][q];
  }
  const int64_t j0 = tj * T, d0 = td * T;
  const int64_t nj = p.shape[jd], nd = p.shape[d];
  // load transposed inputs: consecutive threads walk jd
#pragma unroll
  for (int k = 0; k < N; ++k) {
    if (!(tmask >> k & 1u)) continue;
    const float* q = p.x[k] + off[k + 1];
    for (int l = threadIdx.x; l < T * T; l += BS) {
      const int jj = l % T, dd = l / T;
      const int64_t gj = j0 + jj, gd = d0 + dd;
      tile[k][dd][jj] = (gj < nj && gd < nd) ? q[gj * p.st[k + 1][jd] + gd * p.st[k + 1][d]] : 0.f;
    }
  }
  __syncthreads();
  // compute + store: consecutive threads walk the innermost dim
  for (int l = threadIdx.x; l < T * T; l += BS) {
    const int dd = l % T, jj = l / T;
    const int64_t gj = j0 + jj, gd = d0 + dd;
    if (gj >= nj || gd >= nd) continue;
    float v[N];
#pragma unroll
    for (int k = 0; k < N; ++k)
      v[k] = (tmask >> k & 1u) ? tile[k][dd][jj] : p.x[k][off[k + 1] + gj * p.st[k + 1][jd] + gd * p.st[k + 1][d]];
    p.y[off[0] + gj * p.st[0][jd] + gd * p.st[0][d]] = apply<F, N>(f, v);
  }
}

// tiled in registers: one wave per 32 x 32 tile, lanes on an 8 x 8 grid, each
// lane a 4 (jd) x 4 (innermost) block. A transposed input is read as 4
// float4 rows along its unit-stride dim; the output is written as 4 float4
// columns along its innermost dim; the transpose between them is only which
// register goes where. Each load or store instruction of a wave covers 8
// runs of 128 contiguous bytes; no LDS, no barriers.
constexpr int RT = 32;  // tile extent per wave in both dims

template <class F, int N, unsigned TM, bool NTS>
__global__ __launch_bounds__(BS) void map_regt_k(F f, Plan<N> p, int jd, unsigned tiles_d, unsigned tiles_j,
                                                 unsigned tiles) {
  unsigned b = blockIdx.x * (BS / 64) + (threadIdx.x >> 6);  // this wave's tile
  if (b >= tiles) return;
  const int d = p.ndim - 1;
  const unsigned td = b % tiles_d;
  b /= tiles_d;
  const unsigned tj = b % tiles_j;
  b /= tiles_j;
  int64_t off[N + 1];
#pragma unroll
  for (int k = 0; k <= N; ++k) off[k] = 0;
  for (int q = p.ndim - 2; q >= 0; --q) {
    if (q == jd) continue;
    const unsigned sz = (unsigned)p.shape[q];
    const unsigned c = b % sz;
    b /= sz;
#pragma unroll
    for (int k = 0; k <= N; ++k) off[k] += (int64_t)c * p.st[k][q];
  }
  const int lane = threadIdx.x & 63;
  const int gj = (int)tj * RT + 4 * (lane & 7), gd = (int)td * RT + 4 * (lane >> 3);
  // both dims are multiples of 4: a block is wholly inside or wholly outside
  if (gj >= (int)p.shape[jd] || gd >= (int)p.shape[d]) return;
  float v[N][4][4];  // [input][jd offset c][innermost offset r]
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const float* q = p.x[k] + off[k + 1];
    if ((TM >> k) & 1u) {
      const int64_t sd = p.st[k + 1][d];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const f4 t = ld_stream(reinterpret_cast<const f4*>(q + gj + (int64_t)(gd + r) * sd));
#pragma unroll
        for (int c = 0; c < 4; ++c) v[k][c][r] = t[c];
      }
    } else {
      const int64_t sj = p.st[k + 1][jd];
      const bool bc = p.st[k + 1][d] == 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float* row = q + (int64_t)(gj + c) * sj;
        const f4 t = bc ? f4{row[0], row[0], row[0], row[0]} : *reinterpret_cast<const f4*>(row + gd);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[k][c][r] = t[r];
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    f4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float a[N];
#pragma unroll
      for (int k = 0; k < N; ++k) a[k] = v[k][c][r];
      o[r] = apply<F, N>(f, a);
    }
    st_stream<NTS>(o, reinterpret_cast<f4*>(p.y + off[0] + (int64_t)(gj + c) * p.st[0][jd] + gd));
  }
}

template <class F, int N, unsigned TM>
void launch_regt(F f, const Plan<N>& p, int jd, unsigned tiles_d, unsigned tiles_j, unsigned tiles, bool nts,
                 hipStream_t s) {
  const unsigned blocks = (tiles + BS / 64 - 1) / (BS / 64);
  if (nts) map_regt_k<F, N, TM, true><<<dim3(blocks), dim3(BS), 0, s>>>(f, p, jd, tiles_d, tiles_j, tiles);
  else map_regt_k<F, N, TM, false><<<dim3(blocks), dim3(BS), 0, s>>>(f, p, jd, tiles_d, tiles_j, tiles);
}

// ---------------------------------------------------------------------------
// generic: one element per thread, full index arithmetic.

template <class F, int N>
__global__ __launch_bounds__(BS) void map_generic_k(F f, Plan<N> p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * BS + threadIdx.x; i < n; i += (int64_t)gridDim.x * BS) {
    int64_t r = i;
    int64_t off[N + 1];
#pragma unroll
    for (int k = 0; k <= N; ++k) off[k] = 0;
    for (int d = p.ndim - 1; d >= 0; --d) {
      const int64_t c = r % p.shape[d];
      r /= p.shape[d];
#pragma unroll
      for (int k = 0; k <= N; ++k) off[k] += c * p.st[k][d];
    }
    float v[N];
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = p.x[k][off[k + 1]];
    p.y[off[0]] = apply<F, N>(f, v);
  }
}

// ---------------------------------------------------------------------------
// Host-side planning.

template <int N>
int build_plan(Plan<N>& p, float* y, const int64_t* ys, const float* const* xs, const int64_t* const* xst,
               const int64_t* shape, int ndim, int64_t* numel) {
  if (ndim < 0 || ndim > MAXD) return fail(OXI_INVALID_ARGUMENT, "rank %d exceeds the supported %d dims", ndim, MAXD);
  if (ndim > 0 && !shape) return fail(OXI_INVALID_ARGUMENT, "NULL shape");
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return fail(OXI_INVALID_ARGUMENT, "negative dim size %lld", (long long)shape[d]);
    if (shape[d] && n > (((int64_t)1 << 60) / shape[d])) return fail(OXI_INVALID_ARGUMENT, "element count exceeds the kernel limits");
    n *= shape[d];
  }
  *numel = n;
  p.y = y;
  for (int k = 0; k < N; ++k) p.x[k] = xs[k];
  if (n == 0) {
    p.ndim = 0;
    return OXI_OK;
  }
  if (!y) return fail(OXI_INVALID_ARGUMENT, "NULL output pointer");
  for (int k = 0; k < N; ++k)
    if (!xs[k]) return fail(OXI_INVALID_ARGUMENT, "NULL input pointer");
  // a 0-d operand has no strides: its stride arrays may be NULL
  if (ndim > 0) {
    if (!ys) return fail(OXI_INVALID_ARGUMENT, "NULL output strides");
    for (int k = 0; k < N; ++k)
      if (!xst[k]) return fail(OXI_INVALID_ARGUMENT, "NULL input strides");
  }
  // collect non-trivial dims
  struct Dim { int64_t size; int64_t st[N + 1]; };
  Dim dims[MAXD];
  int m = 0;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] == 1) continue;
    dims[m].size = shape[d];
    dims[m].st[0] = ys[d];
    for (int k = 0; k < N; ++k) dims[m].st[k + 1] = xst[k][d];
    ++m;
  }
  // order dims by decreasing |output stride| (stable): iteration follows the
  // output's memory order, so a row-major output is walked row-major.
  std::stable_sort(dims, dims + m, [](const Dim& a, const Dim& b) {
    const int64_t sa = a.st[0] < 0 ? -a.st[0] : a.st[0];
    const int64_t sb = b.st[0] < 0 ? -b.st[0] : b.st[0];
    return sa > sb;
  });
  // coalesce neighbours d, d+1 when every operand has st[d] == st[d+1]*size[d+1]
  Dim out[MAXD];
  int q = 0;
  for (int d = 0; d < m; ++d) {
    if (q > 0) {
      Dim& prev = out[q - 1];
      bool ok = true;
      for (int k = 0; k <= N; ++k)
        if (prev.st[k] != dims[d].st[k] * dims[d].size) { ok = false; break; }
      if (ok) {
        prev.size *= dims[d].size;
        for (int k = 0; k <= N; ++k) prev.st[k] = dims[d].st[k];
        continue;
      }
    }
    out[q++] = dims[d];
  }
  if (q == 0) {  // every dim has size 1: a single element
    out[0].size = 1;
    for (int k = 0; k <= N; ++k) out[0].st[k] = 0;
    q = 1;
  }
  p.ndim = q;
  for (int d = 0; d < q; ++d) {
    p.shape[d] = out[d].size;
    for (int k = 0; k <= N; ++k) p.st[k][d] = out[d].st[k];
  }
  return OXI_OK;
}

inline bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

template <class F, int N>
int launch_map(F f, const char* what, float* y, const int64_t* ys, const float* const* xs,
               const int64_t* const* xst, const int64_t* shape, int ndim) {
  Plan<N> p;
  int64_t n = 0;
  if (int rc = build_plan<N>(p, y, ys, xs, xst, shape, ndim, &n)) return rc;
  if (n == 0) return OXI_OK;
  const bool nts = nt_stores(n * 4);
  OXI_CHECK_INIT();
  hipStream_t s = stream();
  const int d = p.ndim - 1;
  // flat?
  bool flat = (p.ndim == 1 && p.st[0][0] == 1);
  unsigned bmask = 0;
  for (int k = 0; k < N && flat; ++k) {
    if (p.st[k + 1][0] == 0) bmask |= 1u << k;
    else if (p.st[k + 1][0] != 1) flat = false;
  }
  if (p.ndim == 1 && n == 1) {  // single element: strides irrelevant
    flat = true;
    bmask = (1u << N) - 1;
  }
  if (flat) {
    bool vec = al16(p.y);
    for (int k = 0; k < N; ++k)
      if (!(bmask >> k & 1u) && !al16(p.x[k])) vec = false;
    if (vec && n >= 4) {
      const int64_t n4 = n >> 2;
      const int64_t blocks = std::max<int64_t>(1, ceil_div(n4, (int64_t)BS * FLAT_U));
      if (nts) map_flat_vec_k<F, N, true><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(f, p, n, bmask);
      else map_flat_vec_k<F, N, false><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(f, p, n, bmask);
    } else {
      const int64_t blocks = std::min<int64_t>(ceil_div(n, BS), (int64_t)cu_count() * 32);
      map_flat_k<F, N><<<dim3((unsigned)std::max<int64_t>(1, blocks)), dim3(BS), 0, s>>>(f, p, n, bmask);
    }
    return check_launch(what);
  }
  // rows? innermost stride in {0,1} for every operand (output must be 1)
  bool rows_ok = p.st[0][d] == 1;
  for (int k = 0; k < N && rows_ok; ++k) rows_ok = (p.st[k + 1][d] == 0 || p.st[k + 1][d] == 1);
  const int64_t inner = p.shape[d];
  if (rows_ok && inner >= 64) {
    bool vec = (inner % 4 == 0) && al16(p.y);
    for (int q = 0; q < d && vec; ++q)
      if (p.st[0][q] % 4) vec = false;
    for (int k = 0; k < N && vec; ++k) {
      if (p.st[k + 1][d] == 0) continue;
      if (!al16(p.x[k])) vec = false;
      for (int q = 0; q < d && vec; ++q)
        if (p.st[k + 1][q] % 4) vec = false;
    }
    const int64_t chunk = vec ? (int64_t)BS * 4 * 4 : (int64_t)BS * 4;
    const int64_t cpr = ceil_div(inner, chunk);
    const int64_t rows = n / inner;
    if (rows * cpr < ((int64_t)1 << 31)) {
      if (vec) map_rows_k<F, N, true><<<dim3((unsigned)(rows * cpr)), dim3(BS), 0, s>>>(f, p, cpr, chunk);
      else map_rows_k<F, N, false><<<dim3((unsigned)(rows * cpr)), dim3(BS), 0, s>>>(f, p, cpr, chunk);
      return check_launch(what);
    }
  }
  // tiled? output innermost stride 1, some inputs transposed with a shared unit-stride dim
  if (p.st[0][d] == 1 && p.ndim >= 2) {
    unsigned tmask = 0;
    bool other_ok = true;
    for (int k = 0; k < N; ++k) {
      const int64_t sd = p.st[k + 1][d];
      if (sd == 0 || sd == 1) continue;
      tmask |= 1u << k;
    }
    int jd = -1;
    if (tmask) {
      for (int q = 0; q < d && jd < 0; ++q) {
        bool all = true;
        for (int k = 0; k < N; ++k)
          if ((tmask >> k & 1u) && p.st[k + 1][q] != 1) all = false;
        if (all) jd = q;
      }
      (void)other_ok;
    }
    if (jd >= 0) {
      const int64_t tiles_d = ceil_div(p.shape[d], T), tiles_j = ceil_div(p.shape[jd], T);
      const int64_t batch = n / (p.shape[d] * p.shape[jd]);
      const int64_t blocks = tiles_d * tiles_j * batch;
      if (blocks < ((int64_t)1 << 31)) {
        // 16-byte accesses need 4-element alignment of every row start touched
        bool vec = p.shape[d] % 4 == 0 && p.shape[jd] % 4 == 0 && al16(p.y);
        for (int q = 0; q < p.ndim && vec; ++q)
          if (q != d && p.st[0][q] % 4) vec = false;
        for (int k = 0; k < N && vec; ++k) {
          const bool tr = tmask >> k & 1u;
          if (p.st[k + 1][d] == 0 && !tr) continue;  // broadcast along d: scalar reads
          if (!al16(p.x[k])) vec = false;
          for (int q = 0; q < p.ndim && vec; ++q) {
            if (tr && q == jd) continue;   // the unit-stride dim of a transposed input
            if (!tr && q == d) continue;   // the unit-stride dim of a direct input
            if (p.st[k + 1][q] % 4) vec = false;
          }
        }
        // 32-bit block decode: every dim and the block count stay below 2^31
        for (int q = 0; q < p.ndim && vec; ++q)
          if (p.shape[q] >= ((int64_t)1 << 31)) vec = false;
        const int64_t rtiles = ceil_div(p.shape[d], RT) * ceil_div(p.shape[jd], RT) * batch;
        if (vec && rtiles < ((int64_t)1 << 31)) {
          const unsigned ntd = (unsigned)ceil_div(p.shape[d], RT), ntj = (unsigned)ceil_div(p.shape[jd], RT);
          const unsigned nt = (unsigned)rtiles;
          if (tmask == 1u) launch_regt<F, N, 1u>(f, p, jd, ntd, ntj, nt, nts, s);
          else if constexpr (N == 2) {
            if (tmask == 2u) launch_regt<F, N, 2u>(f, p, jd, ntd, ntj, nt, nts, s);
            else launch_regt<F, N, 3u>(f, p, jd, ntd, ntj, nt, nts, s);
          }
        } else
          map_tiled_k<F, N><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(f, p, jd, tmask, tiles_d, tiles_j);
        return check_launch(what);
      }
    }
  }
  const int64_t blocks = std::min<int64_t>(ceil_div(n, BS), (int64_t)cu_count() * 64);
  map_generic_k<F, N><<<dim3((unsigned)std::max<int64_t>(1, blocks)), dim3(BS), 0, s>>>(f, p, n);
  return check_launch(what);
}

template <int OP>
int run_unary(const float* x, const int64_t* xs, float* y, const int64_t* ys, const int64_t* shape, int ndim) {
  const float* in[1] = {x};
  const int64_t* st[1] = {xs};
  return launch_map<Unary<OP>, 1>(Unary<OP>{}, "unary", y, ys, in, st, shape, ndim);
}

template <int OP>
int run_binary(const float* a, const int64_t* as, const float* b, const int64_t* bs, float* y, const int64_t* ys,
               const int64_t* shape, int ndim) {
  const float* in[2] = {a, b};
  const int64_t* st[2] = {as, bs};
  return launch_map<Binary<OP>, 2>(Binary<OP>{}, "binary", y, ys, in, st, shape, ndim);
}

__global__ __launch_bounds__(BS) void fill_k(float* __restrict__ y, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * BS + threadIdx.x; i < n; i += (int64_t)gridDim.x * BS) y[i] = v;
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_fill(float* y, int64_t n, float value) {
  if (n < 0) return fail(OXI_INVALID_ARGUMENT, "fill: negative size");
  if (n == 0) return OXI_OK;
  if (!y) return fail(OXI_INVALID_ARGUMENT, "fill: NULL output pointer");
  OXI_CHECK_INIT();
  const int64_t blocks = std::min<int64_t>(ceil_div(n, BS), (int64_t)cu_count() * 16);
  fill_k<<<dim3((unsigned)blocks), dim3(BS), 0, stream()>>>(y, n, value);
  return check_launch("fill");
}

int oxi_unary(int op, const float* x, const int64_t* xs, float* y, const int64_t* ys, const int64_t* shape, int ndim) {
  switch (op) {
#define OXI_U(ID) case ID: return run_unary<ID>(x, xs, y, ys, shape, ndim);
    OXI_U(OXI_UNARY_NEG) OXI_U(OXI_UNARY_ABS) OXI_U(OXI_UNARY_SQRT) OXI_U(OXI_UNARY_RSQRT)
    OXI_U(OXI_UNARY_EXP) OXI_U(OXI_UNARY_LOG) OXI_U(OXI_UNARY_LOG2) OXI_U(OXI_UNARY_LOG10)
    OXI_U(OXI_UNARY_SIN) OXI_U(OXI_UNARY_COS) OXI_U(OXI_UNARY_TANH) OXI_U(OXI_UNARY_RELU)
    OXI_U(OXI_UNARY_SIGMOID) OXI_U(OXI_UNARY_FLOOR) OXI_U(OXI_UNARY_CEIL) OXI_U(OXI_UNARY_ROUND)
    OXI_U(OXI_UNARY_SIGN) OXI_U(OXI_UNARY_SQUARE) OXI_U(OXI_UNARY_RECIPROCAL) OXI_U(OXI_UNARY_IDENTITY)
#undef OXI_U
    default:
      return fail(OXI_INVALID_ARGUMENT, "unknown unary op id %d", op);
  }
}

int oxi_binary(int op, const float* a, const int64_t* as, const float* b, const int64_t* bs, float* y,
               const int64_t* ys, const int64_t* shape, int ndim) {
  switch (op) {
#define OXI_B(ID) case ID: return run_binary<ID>(a, as, b, bs, y, ys, shape, ndim);
    OXI_B(OXI_BINARY_ADD) OXI_B(OXI_BINARY_SUB) OXI_B(OXI_BINARY_MUL) OXI_B(OXI_BINARY_DIV)
    OXI_B(OXI_BINARY_POW) OXI_B(OXI_BINARY_MIN) OXI_B(OXI_BINARY_MAX) OXI_B(OXI_CMP_EQ)
    OXI_B(OXI_CMP_NE) OXI_B(OXI_CMP_LT) OXI_B(OXI_CMP_LE) OXI_B(OXI_CMP_GT) OXI_B(OXI_CMP_GE)
#undef OXI_B
    default:
      return fail(OXI_INVALID_ARGUMENT, "unknown binary op id %d", op);
  }
}

int oxi_gelu_fwd(const float* x, const int64_t* xs, float* y, const int64_t* ys, const int64_t* shape, int ndim,
                 int approximate) {
  const float* in[1] = {x};
  const int64_t* st[1] = {xs};
  if (approximate == OXI_GELU_TANH) return launch_map<GeluTanhFwd, 1>(GeluTanhFwd{}, "gelu_fwd", y, ys, in, st, shape, ndim);
  if (approximate == OXI_GELU_ERF) return launch_map<GeluErfFwd, 1>(GeluErfFwd{}, "gelu_fwd", y, ys, in, st, shape, ndim);
  return fail(OXI_INVALID_ARGUMENT, "gelu: unknown approximation %d", approximate);
}

int oxi_gelu_bwd(const float* x, const int64_t* xs, const float* g, const int64_t* gs, float* dx, const int64_t* dxs,
                 const int64_t* shape, int ndim, int approximate) {
  const float* in[2] = {x, g};
  const int64_t* st[2] = {xs, gs};
  if (approximate == OXI_GELU_TANH) return launch_map<GeluTanhBwd, 2>(GeluTanhBwd{}, "gelu_bwd", dx, dxs, in, st, shape, ndim);
  if (approximate == OXI_GELU_ERF) return launch_map<GeluErfBwd, 2>(GeluErfBwd{}, "gelu_bwd", dx, dxs, in, st, shape, ndim);
  return fail(OXI_INVALID_ARGUMENT, "gelu: unknown approximation %d", approximate);
}

int oxi_silu_fwd(const float* x, const int64_t* xs, float* y, const int64_t* ys, const int64_t* shape, int ndim) {
  const float* in[1] = {x};
  const int64_t* st[1] = {xs};
  return launch_map<SiluFwd, 1>(SiluFwd{}, "silu_fwd", y, ys, in, st, shape, ndim);
}

int oxi_silu_bwd(const float* x, const int64_t* xs, const float* g, const int64_t* gs, float* dx, const int64_t* dxs,
                 const int64_t* shape, int ndim) {
  const float* in[2] = {x, g};
  const int64_t* st[2] = {xs, gs};
  return launch_map<SiluBwd, 2>(SiluBwd{}, "silu_bwd", dx, dxs, in, st, shape, ndim);
}

}  // extern "C"
