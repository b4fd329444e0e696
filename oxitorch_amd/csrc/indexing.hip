// Row scatter with last-write-wins and boolean-mask selection, forward and
// VJP (Tensor::scatter_dim0 / masked_select, crates/oxi-tensor/src/lib.rs:
// 895-961; aops::scatter_dim0 / masked_select, crates/oxi-autograd/src/ops.rs:
// 531-667).
//
// Scatter: the last writer of each row is an integer max over positions
// (order-independent, so deterministic); every output row is then one copy
// from either the base or the winning values row.
//
// Mask selection: the broadcast grid is cut into tiles of TILE elements in
// row-major order. The first launch reads x and the mask once, records one
// pick bit per element and counts each tile's picks; one block scans the
// counts into tile offsets; the last launch reads the bits and x and writes
// each tile's picks at its offset, ranked within the tile by block scans.
// Offsets and bits form the selection's record, which the VJP reads instead
// of x and the mask: each picked grid point takes the gradient of its rank.
#include <cmath>

#include <cstdlib>
#include <cstring>

#include "internal.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;

// ---- scatter_dim0 -----------------------------------------------------------

__global__ __launch_bounds__(BS) void winner_clear_k(int* __restrict__ w, int64_t rows) {
  const int64_t i = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (i < rows) w[i] = 0;
}

// w[r] = 1 + the largest position p with idx[p] == r (0: never written).
__global__ __launch_bounds__(BS) void winner_max_k(const int64_t* __restrict__ idx, int64_t n, int64_t rows,
                                                   int* __restrict__ w, int* guard) {
  const int64_t p = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (p >= n) return;
  int64_t r = idx[p];
  if (r < 0) r += rows;
  if (r < 0 || r >= rows) {
    atomicOr(guard, 1);
    return;
  }
  atomicMax(w + r, (int)(p + 1));
}

// out row r = values row w[r]-1 when written, else base row r. `iu` units per
// row: float4s when VEC, floats otherwise.
// Row and column of unit u: 32-bit division when every unit index fits.
template <bool NARROW>
__device__ __forceinline__ void row_col(int64_t u, int64_t iu, int64_t* r, int64_t* c) {
  if constexpr (NARROW) {
    const uint32_t q = (uint32_t)u / (uint32_t)iu;
    *r = q;
    *c = (int64_t)((uint32_t)u - q * (uint32_t)iu);
  } else {
    *r = u / iu;
    *c = u - *r * iu;
  }
}

template <bool VEC, bool NTS, bool NARROW>
__global__ __launch_bounds__(BS) void scatter_rows_k(const float* __restrict__ base, const float* __restrict__ values,
                                                     const int* __restrict__ w, float* __restrict__ out, int64_t iu,
                                                     int64_t units) {
  const int64_t u = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (u >= units) return;
  int64_t r, c;
  row_col<NARROW>(u, iu, &r, &c);
  const int win = w[r];
  if constexpr (VEC) {
    const f4* src = win ? reinterpret_cast<const f4*>(values) + (int64_t)(win - 1) * iu
                        : reinterpret_cast<const f4*>(base) + r * iu;
    st_stream<NTS>(ld_stream(src + c), reinterpret_cast<f4*>(out) + u);
  } else {
    const float* src = win ? values + (int64_t)(win - 1) * iu : base + r * iu;
    out[u] = src[c];
  }
}

// VJP in one launch: units [0, gb_units) give gbase = g * (written ? 0 : 1);
// the rest give gvalues slot p = g row idx[p] when p won that row, else 0.
// FUSED (both outputs wanted): a base unit whose row was written also stores
// its g value into the winning slot of gvalues, so each row of g is read
// once, and the gvalues units only write the zeros of the slots that lost.
template <bool VEC, bool NARROW, bool FUSED>
__global__ __launch_bounds__(BS) void scatter_rows_bwd_k(const float* __restrict__ g, const int64_t* __restrict__ idx,
                                                         const int* __restrict__ w, float* __restrict__ gbase,
                                                         float* __restrict__ gvalues, int64_t rows, int64_t iu,
                                                         int64_t gb_units, int64_t units) {
  const int64_t u = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (u >= units) return;
  if (u < gb_units) {
    int64_t r, c0;
    row_col<NARROW>(u, iu, &r, &c0);
    const int win = w[r];  // winning position + 1, 0 when the row keeps its base value
    const float m = win ? 0.0f : 1.0f;
    if constexpr (VEC) {
      f4 v = ld_stream(reinterpret_cast<const f4*>(g) + u);
      if (FUSED && win) reinterpret_cast<f4*>(gvalues)[(int64_t)(win - 1) * iu + c0] = v;
      v.x = v.x * m;
      v.y = v.y * m;
      v.z = v.z * m;
      v.w = v.w * m;
      reinterpret_cast<f4*>(gbase)[u] = v;
    } else {
      const float v = g[u];
      if (FUSED && win) gvalues[(int64_t)(win - 1) * iu + c0] = v;
      gbase[u] = v * m;
    }
    return;
  }
  const int64_t q = u - gb_units;
  int64_t p, c;
  row_col<NARROW>(q, iu, &p, &c);
  int64_t r = idx[p];
  if (r < 0) r += rows;
  const bool won = r >= 0 && r < rows && w[r] == (int)(p + 1);
  if (FUSED && won) return;  // stored by the base unit of row r
  if constexpr (VEC) {
    reinterpret_cast<f4*>(gvalues)[q] = won ? reinterpret_cast<const f4*>(g)[r * iu + c] : f4{0.f, 0.f, 0.f, 0.f};
  } else {
    gvalues[q] = won ? g[r * iu + c] : 0.0f;
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Computes the winner table into `w` (rows ints) on the library stream.
int winners(const int64_t* idx, int64_t n, int64_t rows, int* w) {
  hipStream_t s = stream();
  winner_clear_k<<<(unsigned)ceil_div(rows, BS), BS, 0, s>>>(w, rows);
  if (n > 0) winner_max_k<<<(unsigned)ceil_div(n, BS), BS, 0, s>>>(idx, n, rows, w, guard_flag());
  return OXI_OK;
}

// ---- masked_select ------------------------------------------------------------

constexpr int MAXD = OXI_MAX_DIMS;
constexpr int MB = 256;                 // threads per block of the selection kernels
constexpr int STEPS = 4;                // float4 groups per thread per tile
constexpr int TILE = MB * 4 * STEPS;    // grid elements per tile
constexpr int WAVES = MB / 64;
// Pick record of a tile: STEPS x WAVES x 4 words of 64 bits. Word k of
// (step j, wave w) holds at bit `lane` the pick of grid element
// tile0 + j*MB*4 + (w*64 + lane)*4 + k (one ballot per k).
constexpr int REC_WORDS = STEPS * WAVES * 4;
static_assert(STEPS * 16 <= 64 && MB * 4 < 65536, "packed step counts must fit 16-bit fields");

// The grid after dropping size-1 dims and merging dims that are contiguous
// for every stride set (row-major order is preserved).
template <int NS>
struct Grid {
  int ndim;
  int64_t shape[MAXD];
  int64_t st[NS][MAXD];
};

template <int NS>
Grid<NS> make_grid(const int64_t* shape, int ndim, const int64_t* const* st) {
  Grid<NS> g{};
  int m = 0;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] == 1) continue;
    if (m > 0) {
      bool merge = true;
      for (int k = 0; k < NS; ++k) merge = merge && g.st[k][m - 1] == st[k][d] * shape[d];
      if (merge) {
        g.shape[m - 1] *= shape[d];
        for (int k = 0; k < NS; ++k) g.st[k][m - 1] = st[k][d];
        continue;
      }
    }
    g.shape[m] = shape[d];
    for (int k = 0; k < NS; ++k) g.st[k][m] = st[k][d];
    ++m;
  }
  if (m == 0) {  // a single element
    g.shape[0] = 1;
    for (int k = 0; k < NS; ++k) g.st[k][0] = 0;
    m = 1;
  }
  g.ndim = m;
  return g;
}

// True when stride set k walks the grid contiguously (one dim, stride 1).
template <int NS>
bool contiguous(const Grid<NS>& g, int k) { return g.ndim == 1 && g.st[k][0] == 1; }

// Decodes grid element e into coordinates and the offsets of every stride set.
template <int NS>
__device__ __forceinline__ void grid_decode(const Grid<NS>& g, int64_t e, int64_t* idx, int64_t* off) {
#pragma unroll
  for (int k = 0; k < NS; ++k) off[k] = 0;
  for (int d = g.ndim - 1; d >= 0; --d) {
    idx[d] = e % g.shape[d];
    e /= g.shape[d];
#pragma unroll
    for (int k = 0; k < NS; ++k) off[k] += idx[d] * g.st[k][d];
  }
}

// Steps the coordinates and offsets to the next grid element.
template <int NS>
__device__ __forceinline__ void grid_step(const Grid<NS>& g, int64_t* idx, int64_t* off) {
  for (int d = g.ndim - 1; d >= 0; --d) {
    if (++idx[d] < g.shape[d]) {
#pragma unroll
      for (int k = 0; k < NS; ++k) off[k] += g.st[k][d];
      return;
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) off[k] -= (g.shape[d] - 1) * g.st[k][d];
    idx[d] = 0;
  }
}

// A pick: the mask value is not zero and x is not NaN (the reference marks
// unpicked elements NaN and drops every NaN, lib.rs:955-958).
__device__ __forceinline__ bool picked(float x, float m) { return m != 0.0f && !isnan(x); }

// Pick bits (bit k: element e0+k) of one thread's 4 grid elements. FAST: x
// and mask are contiguous over the grid with 16-byte aligned bases.
template <bool FAST>
__device__ __forceinline__ unsigned pick_bits(const Grid<2>& g, const float* x, const float* m, int64_t e0,
                                              int64_t E) {
  unsigned bits = 0;
  if (e0 >= E) return 0;
  if constexpr (FAST) {
    if (e0 + 4 <= E) {
      const f4 xv = ld_stream(reinterpret_cast<const f4*>(x + e0));
      const f4 mv = ld_stream(reinterpret_cast<const f4*>(m + e0));
#pragma unroll
      for (int k = 0; k < 4; ++k) bits |= (unsigned)picked(xv[k], mv[k]) << k;
      return bits;
    }
    for (int k = 0; k < 4 && e0 + k < E; ++k) bits |= (unsigned)picked(x[e0 + k], m[e0 + k]) << k;
    return bits;
  } else {
    int64_t idx[MAXD], off[2];
    grid_decode(g, e0, idx, off);
    for (int k = 0; k < 4 && e0 + k < E; ++k) {
      if (k) grid_step(g, idx, off);
      bits |= (unsigned)picked(x[off[0]], m[off[1]]) << k;
    }
    return bits;
  }
}

// Exclusive scan over the block of STEPS pick counts at once: field j (16
// bits) of `v` is this thread's count at step j (at most 4, so a field's
// block total, at most 4*MB, never carries into the next). Returns the
// exclusive prefix; `tot` gets the block totals, packed the same way.
__device__ __forceinline__ uint64_t block_excl_scan_packed(uint64_t v, uint64_t* lds, uint64_t* tot) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  uint64_t inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) lds[wid] = inc;
  __syncthreads();
  uint64_t before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < WAVES; ++i) {
    const uint64_t t = lds[i];
    before += i < wid ? t : 0;
    all += t;
  }
  *tot = all;
  return before + inc - v;
}

// Ranks within the tile of this thread's first pick at each step, from the
// packed per-step counts; returns the tile's pick total.
__device__ __forceinline__ int step_ranks(const unsigned* bits, uint64_t* lds, int* rank) {
  uint64_t packed = 0;
#pragma unroll
  for (int j = 0; j < STEPS; ++j) packed |= (uint64_t)__builtin_popcount(bits[j]) << (16 * j);
  uint64_t tot;
  const uint64_t ex = block_excl_scan_packed(packed, lds, &tot);
  int pos = 0;
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    rank[j] = pos + (int)((ex >> (16 * j)) & 0xFFFFu);
    pos += (int)((tot >> (16 * j)) & 0xFFFFu);
  }
  return pos;
}

// This thread's 4 pick bits at step j of tile `tile`, from the record.
__device__ __forceinline__ unsigned record_bits(const uint64_t* rec, int64_t tile, int j) {
  // the wave index is uniform: the compiler then reads the words with scalar loads
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint64_t* w = rec + tile * REC_WORDS + (j * WAVES + wid) * 4;
  const int lane = threadIdx.x & 63;
  unsigned bits = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) bits |= (unsigned)((w[k] >> lane) & 1u) << k;
  return bits;
}

// Pass 1: pick bits into the record, and each tile's pick count.
template <bool FAST>
__global__ __launch_bounds__(MB) void msel_count_k(Grid<2> g, const float* __restrict__ x,
                                                   const float* __restrict__ m, int64_t E, int* __restrict__ counts,
                                                   uint64_t* __restrict__ rec) {
  __shared__ int lds[WAVES];
  const int64_t tile0 = (int64_t)blockIdx.x * TILE;
  const int lane = threadIdx.x & 63;
  int c = 0;
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    const int64_t e0 = tile0 + (int64_t)j * MB * 4 + threadIdx.x * 4;
    const unsigned bits = pick_bits<FAST>(g, x, m, e0, E);
    c += __builtin_popcount(bits);
    uint64_t b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) b[k] = __ballot((bits >> k) & 1u);
    if (lane < 4) {
      uint64_t v = b[0];
#pragma unroll
      for (int k = 1; k < 4; ++k) v = lane == k ? b[k] : v;
      rec[(int64_t)blockIdx.x * REC_WORDS + (j * WAVES + (threadIdx.x >> 6)) * 4 + lane] = v;
    }
  }
  c = wave_sum(c);
  if (lane == 0) lds[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) t += lds[i];
    counts[blockIdx.x] = t;
  }
}

// One block: offs[t] = counts[0] + ... + counts[t-1], offs[T] = the total.
// Chunks of SCAN_CH counts are staged in LDS with coalesced loads (padded by
// one word per SCAN_PER so each thread's run is conflict-free), scanned, and
// written back coalesced, with a running carry between chunks.
constexpr int SCAN_BS = 1024;
constexpr int SCAN_PER = 8;
constexpr int SCAN_CH = SCAN_BS * SCAN_PER;
__device__ __forceinline__ int scan_pad(int i) { return i + i / SCAN_PER; }

__global__ __launch_bounds__(SCAN_BS) void msel_scan_k(const int* __restrict__ counts, int64_t T,
                                                        int64_t* __restrict__ offs, int64_t* host_total) {
  __shared__ int cnt[SCAN_CH + SCAN_CH / SCAN_PER];
  __shared__ int wsum[SCAN_BS / 64];
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  int64_t carry = 0;
  for (int64_t c0 = 0; c0 < T; c0 += SCAN_CH) {
    const int n = (int)min((int64_t)SCAN_CH, T - c0);
    for (int i = threadIdx.x; i < n; i += SCAN_BS) cnt[scan_pad(i)] = counts[c0 + i];
    __syncthreads();
    int v[SCAN_PER];
    int s = 0;
#pragma unroll
    for (int k = 0; k < SCAN_PER; ++k) {
      const int i = threadIdx.x * SCAN_PER + k;
      v[k] = i < n ? cnt[scan_pad(i)] : 0;
      s += v[k];
    }
    int inc = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(inc, o, 64);
      if (lane >= o) inc += t;
    }
    if (lane == 63) wsum[wid] = inc;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < SCAN_BS / 64; ++i) {
      before += i < wid ? wsum[i] : 0;
      all += wsum[i];
    }
    int run = before + inc - s;
#pragma unroll
    for (int k = 0; k < SCAN_PER; ++k) {
      const int i = threadIdx.x * SCAN_PER + k;
      if (i < n) cnt[scan_pad(i)] = run;
      run += v[k];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += SCAN_BS) offs[c0 + i] = carry + cnt[scan_pad(i)];
    carry += all;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    offs[T] = carry;
    if (host_total) *host_total = carry;
  }
}

// Pass 2: each tile's picks at its offset, in grid order; reads x only where
// the record has a pick. All steps' loads are issued before the one scan.
template <bool FAST>
__global__ __launch_bounds__(MB) void msel_write_k(Grid<1> g, const float* __restrict__ x, int64_t E,
                                                   const int64_t* __restrict__ offs,
                                                   const uint64_t* __restrict__ rec, float* __restrict__ out) {
  __shared__ uint64_t lds[WAVES];
  __shared__ float stage[TILE];
  const int64_t tile0 = (int64_t)blockIdx.x * TILE;
  unsigned bits[STEPS];
#pragma unroll
  for (int j = 0; j < STEPS; ++j) bits[j] = record_bits(rec, blockIdx.x, j);
  float v[STEPS][4];
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    const int64_t e0 = tile0 + (int64_t)j * MB * 4 + threadIdx.x * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[j][k] = 0.0f;
    if (!bits[j]) continue;
    if constexpr (FAST) {
      if (e0 + 4 <= E) {
        const f4 xv = ld_stream(reinterpret_cast<const f4*>(x + e0));
#pragma unroll
        for (int k = 0; k < 4; ++k) v[j][k] = xv[k];
      } else {
        for (int k = 0; k < 4; ++k)
          if (bits[j] >> k & 1u) v[j][k] = x[e0 + k];
      }
    } else {
      int64_t idx[MAXD], off[1];
      grid_decode(g, e0, idx, off);
      for (int k = 0; k < 4 && e0 + k < E; ++k) {
        if (k) grid_step(g, idx, off);
        if (bits[j] >> k & 1u) v[j][k] = x[off[0]];
      }
    }
  }
  // picks go to LDS at their rank in the tile, then out in coalesced runs
  int rank[STEPS];
  const int n = step_ranks(bits, lds, rank);
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    int r = rank[j];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (bits[j] >> k & 1u) stage[r++] = v[j][k];
  }
  __syncthreads();
  float* o = out + offs[blockIdx.x];
#pragma unroll
  for (int c = 0; c < TILE / MB; ++c) {
    const int i = c * MB + threadIdx.x;
    if (i < n) o[i] = stage[i];
  }
}

// One pass over x and the mask: the record and the picks written at their
// final offsets, so x crosses HBM once (the two passes above read it twice).
// A block owns a chunk of MSEL_CHUNK consecutive tiles, taken from an atomic
// ticket in the order blocks start, so a chunk only ever waits for chunks
// whose blocks already run. It loads all its tiles, ranks each tile's picks,
// publishes the chunk's pick count in status[chunk] (flag LB_AGG), then adds
// the counts, or the inclusive prefix (flag LB_PRE), of the chunks before it,
// walking back until it meets a prefix (a decoupled look-back; the first
// wave reads 64 status words per poll), publishes its own inclusive prefix,
// and stores each tile's picks through LDS as coalesced runs. The record and
// the tile offsets keep the two-pass layout, so the VJP reads either.
// Measured at (16384, 4096): one tile per block took 244 us against 178 us
// for the two passes; without the ticket (block order) and without the walk
// it took 87 us, with the ticket alone 213 us: 16384 device-scope adds on one
// address serialise at about 8 ns each, and each walk holds its block's
// registers while it waits. Chunks of 2, 4, 6 and 8 tiles: 198, 183, 212 and
// 306 us (4 tiles: 84 VGPRs; 8: 160). Wider windows (the whole block's 256
// words per poll) were slower. The status words carry the values, so relaxed
// device-scope atomics order everything the walk needs. Every wait is
// bounded: a walk that polls `spin_limit` times without progress (a negative
// limit: at once) raises the guard flag (bit 4) and its chunk stores no
// picks; the call reports a failed last chunk, oxi_hip_sync any other. The
// output holds room for every grid point (the host moves picks that fill at
// most a third of it into an exact-size buffer).
constexpr uint64_t LB_AGG = 1ull << 62, LB_PRE = 2ull << 62, LB_VAL = (1ull << 62) - 1;
#ifndef OXI_MSEL_CHUNK
#define OXI_MSEL_CHUNK 4
#endif
constexpr int MSEL_CHUNK = OXI_MSEL_CHUNK;  // tiles per block of the one pass

__device__ __forceinline__ uint64_t lb_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lb_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// x values and pick bits of one thread's 4 grid elements (as pick_bits).
template <bool FAST>
__device__ __forceinline__ unsigned load_picks(const Grid<2>& g, const float* x, const float* m, int64_t e0,
                                               int64_t E, float (&v)[4]) {
  unsigned bits = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = 0.0f;
  if (e0 >= E) return 0;
  if constexpr (FAST) {
    if (e0 + 4 <= E) {
      const f4 xv = ld_stream(reinterpret_cast<const f4*>(x + e0));
      const f4 mv = ld_stream(reinterpret_cast<const f4*>(m + e0));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k] = xv[k];
        bits |= (unsigned)picked(xv[k], mv[k]) << k;
      }
      return bits;
    }
    for (int k = 0; k < 4 && e0 + k < E; ++k) {
      v[k] = x[e0 + k];
      bits |= (unsigned)picked(v[k], m[e0 + k]) << k;
    }
    return bits;
  } else {
    int64_t idx[MAXD], off[2];
    grid_decode(g, e0, idx, off);
    for (int k = 0; k < 4 && e0 + k < E; ++k) {
      if (k) grid_step(g, idx, off);
      v[k] = x[off[0]];
      bits |= (unsigned)picked(v[k], m[off[1]]) << k;
    }
    return bits;
  }
}

template <bool FAST, int CH>
__global__ __launch_bounds__(MB) void msel_onepass_k(Grid<2> g, const float* __restrict__ x,
                                                     const float* __restrict__ m, int64_t E, int64_t T,
                                                     uint64_t* __restrict__ status, int* __restrict__ ticket,
                                                     int64_t* __restrict__ offs, uint64_t* __restrict__ rec,
                                                     float* __restrict__ out, int64_t* host_total, int* guard,
                                                     int spin_limit) {
  __shared__ uint64_t lds[CH][WAVES];
  __shared__ float stage[TILE];
  __shared__ int64_t s_chunk, s_pre;
  if (threadIdx.x == 0) s_chunk = atomicAdd(ticket, 1);
  __syncthreads();
  const int64_t chunk = s_chunk;
  const int64_t tile0 = chunk * CH;  // first tile of the chunk
  const int lane = threadIdx.x & 63;
  unsigned bits[CH][STEPS];
  float v[CH][STEPS][4];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int j = 0; j < STEPS; ++j)
      bits[c][j] = load_picks<FAST>(g, x, m, (tile0 + c) * TILE + (int64_t)j * MB * 4 + threadIdx.x * 4, E, v[c][j]);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (tile0 + c >= T) break;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
      uint64_t b[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) b[k] = __ballot((bits[c][j] >> k) & 1u);
      if (lane < 4) {
        uint64_t w = b[0];
#pragma unroll
        for (int k = 1; k < 4; ++k) w = lane == k ? b[k] : w;
        rec[(tile0 + c) * REC_WORDS + (j * WAVES + (threadIdx.x >> 6)) * 4 + lane] = w;
      }
    }
  }
  int rank[CH][STEPS], n[CH];
  int N = 0;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    n[c] = step_ranks(bits[c], lds[c], rank[c]);  // the first barrier orders the ticket read
    N += n[c];
  }
  if (threadIdx.x < 64) {  // the first wave walks back, 64 status words per poll
    int64_t pre = 0;
    bool ok = true;
    if (chunk == 0) {
      if (lane == 0) lb_store(status, LB_PRE | (uint64_t)N);
    } else {
      if (lane == 0) lb_store(status + chunk, LB_AGG | (uint64_t)N);
      // Lane l reads status[hi - l]; chunks below 0 count as a prefix of 0.
      // Chunk 0 publishes a prefix, so the walk ends by the window holding it.
      for (int64_t hi = chunk - 1;; hi -= 64) {
        const int64_t j = hi - lane;
        uint64_t st = j >= 0 ? lb_load(status + j) : LB_PRE;
        uint64_t need, pm;
        for (int spins = 0;; ++spins) {
          if (spin_limit < 0) {  // the host's switch that fails every wait
            ok = false;
            break;
          }
          // lanes up to the nearest prefix must have published
          pm = __ballot((st >> 62) == 2);
          need = pm ? (pm & (~pm + 1)) | ((pm & (~pm + 1)) - 1) : ~0ull;
          if ((__ballot((st >> 62) == 0) & need) == 0) break;
          if (spins >= spin_limit) {
            ok = false;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          if ((st >> 62) == 0) st = lb_load(status + j);
        }
        if (!ok) break;
        int64_t add = (need >> lane & 1) ? (int64_t)(st & LB_VAL) : 0;
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) add += __shfl_xor(add, s, 64);
        pre += add;
        if (pm) break;  // a prefix was in the window
      }
      if (ok && lane == 0) lb_store(status + chunk, LB_PRE | (uint64_t)(pre + N));
    }
    if (lane == 0) {
      if (!ok) atomicOr(guard, 4);
      s_pre = ok ? pre : -1;
      int64_t o = pre;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (tile0 + c >= T) break;
        offs[tile0 + c] = o;
        o += n[c];
        if (ok && tile0 + c == T - 1) {
          offs[T] = o;
          // system scope: the host polls it while the other blocks finish
          __hip_atomic_store(host_total, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
      }
    }
  }
  int64_t base = -1;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (c) __syncthreads();  // the previous tile's stage is read
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
      int r = rank[c][j];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (bits[c][j] >> k & 1u) stage[r++] = v[c][j][k];
    }
    __syncthreads();
    if (c == 0) base = s_pre;
    if (base < 0) return;
    float* o = out + base;
#pragma unroll
    for (int q = 0; q < TILE / MB; ++q) {
      const int i = q * MB + threadIdx.x;
      if (i < n[c]) o[i] = stage[i];
    }
    base += n[c];
  }
}

// VJP: the grid point of pick rank r gets 0 + up[r] (the reference adds the
// upstream gradient to a zero), every other point 0, stored at the point's
// offset in `g` (stride set 0). A record whose total differs from `count`
// raises the guard flag and reads no gradient beyond `count`.
template <bool FAST, bool NTS>
__global__ __launch_bounds__(MB) void msel_grad_k(Grid<1> g, int64_t E, const int64_t* __restrict__ offs,
                                                  const uint64_t* __restrict__ rec, const float* __restrict__ up,
                                                  int64_t count, float* __restrict__ dst, int64_t T, int* guard) {
  __shared__ uint64_t lds[WAVES];
  __shared__ float stage[TILE];
  if (blockIdx.x == 0 && threadIdx.x == 0 && offs[T] != count) atomicOr(guard, 1);
  const int64_t tile0 = (int64_t)blockIdx.x * TILE;
  unsigned bits[STEPS];
#pragma unroll
  for (int j = 0; j < STEPS; ++j) bits[j] = record_bits(rec, blockIdx.x, j);
  int rank[STEPS];
  const int n = step_ranks(bits, lds, rank);
  // the tile's upstream gradients, one coalesced run, into LDS
  const int64_t pos = offs[blockIdx.x];
  if (pos + n <= count) {
#pragma unroll
    for (int c = 0; c < TILE / MB; ++c) {
      const int i = c * MB + threadIdx.x;
      if (i < n) stage[i] = up[pos + i];
    }
  } else {
    for (int i = threadIdx.x; i < n; i += MB) {
      float u = 0.0f;
      if (pos + i < count) u = up[pos + i];
      else atomicOr(guard, 1);
      stage[i] = u;
    }
  }
  __syncthreads();
  float v[STEPS][4];
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    int r = rank[j];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[j][k] = 0.0f;
      if (bits[j] >> k & 1u) v[j][k] = 0.0f + stage[r++];
    }
  }
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    const int64_t e0 = tile0 + (int64_t)j * MB * 4 + threadIdx.x * 4;
    if (e0 >= E) continue;
    if constexpr (FAST) {
      if (e0 + 4 <= E) {
        st_stream<NTS>(f4{v[j][0], v[j][1], v[j][2], v[j][3]}, reinterpret_cast<f4*>(dst + e0));
      } else {
        for (int k = 0; k < 4 && e0 + k < E; ++k) dst[e0 + k] = v[j][k];
      }
    } else {
      int64_t idx[MAXD], off[1];
      grid_decode(g, e0, idx, off);
      for (int k = 0; k < 4 && e0 + k < E; ++k) {
        if (k) grid_step(g, idx, off);
        dst[off[0]] = v[j][k];
      }
    }
  }
}

// Broadcast x: grad_x[i] = 0 + the contributions of x element i's grid points
// in grid order. Kept dims (x's own) locate the element; broadcast dims are
// walked row-major. `contrib` is dense in grid order.
struct AccPlan {
  int nk, nb;
  int64_t ksize[MAXD], kstride[MAXD];  // x's own dims, grid row-major strides
  int64_t bsize[MAXD], bstride[MAXD];  // broadcast dims
  int64_t npts;                        // points per x element
};

__global__ __launch_bounds__(BS) void msel_accum_k(AccPlan a, const float* __restrict__ contrib, int64_t xn,
                                                   float* __restrict__ gx) {
  const int64_t i = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (i >= xn) return;
  int64_t base = 0, r = i;
  for (int d = a.nk - 1; d >= 0; --d) {
    base += (r % a.ksize[d]) * a.kstride[d];
    r /= a.ksize[d];
  }
  int64_t c[MAXD];
  for (int d = 0; d < a.nb; ++d) c[d] = 0;
  int64_t off = base;
  float acc = 0.0f;
  for (int64_t p = 0; p < a.npts; ++p) {
    acc += contrib[off];
    for (int d = a.nb - 1; d >= 0; --d) {
      if (++c[d] < a.bsize[d]) {
        off += a.bstride[d];
        break;
      }
      off -= (a.bsize[d] - 1) * a.bstride[d];
      c[d] = 0;
    }
  }
  gx[i] = acc;
}

// Grid size and tile count of a selection over `shape`.
int grid_size(const int64_t* shape, int ndim, int64_t* E, int64_t* T, const char* what) {
  if (ndim < 0 || ndim > MAXD) return fail(OXI_INVALID_ARGUMENT, "%s: rank %d exceeds %d dims", what, ndim, MAXD);
  if (ndim > 0 && !shape) return fail(OXI_INVALID_ARGUMENT, "%s: NULL shape", what);
  int64_t e = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return fail(OXI_INVALID_ARGUMENT, "%s: negative dim size", what);
    if (shape[d] && e > (((int64_t)1 << 60) / shape[d])) return fail(OXI_INVALID_ARGUMENT, "%s: grid too large", what);
    e *= shape[d];
  }
  *E = e;
  *T = ceil_div(e, TILE);
  if (*T >= ((int64_t)1 << 31)) return fail(OXI_INVALID_ARGUMENT, "%s: grid too large", what);
  return OXI_OK;
}

int64_t record_bytes(int64_t T) { return 8 * (T + 1) + 8 * (int64_t)REC_WORDS * T; }

// The one pass's pick total: the block of the last tile stores it to the
// slot (system scope) before its own stores, and other blocks may still be
// storing picks, so the host polls the slot instead of waiting for the
// stream and returns while the kernel drains (the caller's next launches
// queue behind it). The poll ends when the value arrives or the stream's
// work has ended (then the slot holds the total, or -1 after a failed walk);
// a failed stream returns its error.
int poll_total(int64_t* slot, hipStream_t st, int64_t* total) {
  for (unsigned i = 1;; ++i) {
    const int64_t v = __atomic_load_n(slot, __ATOMIC_ACQUIRE);
    if (v >= 0) {
      *total = v;
      return OXI_OK;
    }
    if ((i & 63) == 0) {  // a driver call now and then
      const hipError_t e = hipStreamQuery(st);
      if (e == hipSuccess) {
        *total = __atomic_load_n(slot, __ATOMIC_ACQUIRE);
        return OXI_OK;
      }
      if (e != hipErrorNotReady) return fail_hip(e, "hipStreamQuery(masked_select)");
    }
    __builtin_ia32_pause();
  }
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_scatter_rows(const float* base, int64_t rows, int64_t inner, const int64_t* idx, int64_t n,
                     const float* values, float* out) {
  if (rows < 0 || inner < 0 || n < 0) return fail(OXI_INVALID_ARGUMENT, "scatter_rows: negative size");
  if (n >= INT32_MAX) return fail(OXI_INVALID_ARGUMENT, "scatter_rows: too many positions (%lld)", (long long)n);
  if (inner && (rows + n) > (((int64_t)1 << 60) / inner))
    return fail(OXI_INVALID_ARGUMENT, "scatter_rows: size exceeds the kernel limits");
  if (rows == 0 && n > 0) return fail(OXI_INVALID_ARGUMENT, "scatter_rows: positions into an empty tensor");
  if (rows == 0 || inner == 0) return OXI_OK;
  if (!base || !out || (n > 0 && (!idx || !values)))
    return fail(OXI_INVALID_ARGUMENT, "scatter_rows: NULL pointer");
  OXI_CHECK_INIT();
  Workspace ws(sizeof(int) * (size_t)rows);
  if (!ws.p) return fail_alloc("scatter_rows: workspace");
  int* w = ws.as<int>();
  winners(idx, n, rows, w);
  const bool vec = inner % 4 == 0 && al16(base) && al16(out) && (n == 0 || al16(values));
  const int64_t iu = vec ? inner / 4 : inner;
  const int64_t units = rows * iu;
  const bool nts = nt_stores(rows * inner * 4);
  hipStream_t s = stream();
  const unsigned blocks = (unsigned)ceil_div(units, BS);
  const bool narrow = blocks * (int64_t)BS <= (int64_t)UINT32_MAX;
  if (vec && nts && narrow) scatter_rows_k<true, true, true><<<blocks, BS, 0, s>>>(base, values, w, out, iu, units);
  else if (vec && nts) scatter_rows_k<true, true, false><<<blocks, BS, 0, s>>>(base, values, w, out, iu, units);
  else if (vec && narrow) scatter_rows_k<true, false, true><<<blocks, BS, 0, s>>>(base, values, w, out, iu, units);
  else if (vec) scatter_rows_k<true, false, false><<<blocks, BS, 0, s>>>(base, values, w, out, iu, units);
  else scatter_rows_k<false, false, false><<<blocks, BS, 0, s>>>(base, values, w, out, iu, units);
  return check_launch("scatter_rows");
}

int oxi_scatter_rows_bwd(const float* g, int64_t rows, int64_t inner, const int64_t* idx, int64_t n, float* gbase,
                         float* gvalues) {
  if (rows < 0 || inner < 0 || n < 0) return fail(OXI_INVALID_ARGUMENT, "scatter_rows_bwd: negative size");
  if (n >= INT32_MAX) return fail(OXI_INVALID_ARGUMENT, "scatter_rows_bwd: too many positions (%lld)", (long long)n);
  if (inner && (rows + n) > (((int64_t)1 << 60) / inner))
    return fail(OXI_INVALID_ARGUMENT, "scatter_rows_bwd: size exceeds the kernel limits");
  if (inner == 0 || (rows == 0 && n == 0)) return OXI_OK;
  if (rows == 0) return fail(OXI_INVALID_ARGUMENT, "scatter_rows_bwd: positions into an empty tensor");
  if (!g || (n > 0 && !idx)) return fail(OXI_INVALID_ARGUMENT, "scatter_rows_bwd: NULL pointer");
  if (!gbase && !gvalues) return OXI_OK;
  OXI_CHECK_INIT();
  Workspace ws(sizeof(int) * (size_t)rows);
  if (!ws.p) return fail_alloc("scatter_rows_bwd: workspace");
  int* w = ws.as<int>();
  winners(idx, n, rows, w);
  const bool vec = inner % 4 == 0 && al16(g) && (!gbase || al16(gbase)) && (!gvalues || al16(gvalues));
  const int64_t iu = vec ? inner / 4 : inner;
  const int64_t gb_units = gbase ? rows * iu : 0;
  // without gbase, shift gvalues' units to start at 0
  const int64_t units = gb_units + (gvalues ? n * iu : 0);
  if (units == 0) return OXI_OK;
  hipStream_t s = stream();
  const unsigned blocks = (unsigned)ceil_div(units, BS);
  const bool narrow = blocks * (int64_t)BS <= (int64_t)UINT32_MAX;
  const bool fused = gbase && gvalues;
#define OXI_SRB(V, NW, FU) \
  scatter_rows_bwd_k<V, NW, FU><<<blocks, BS, 0, s>>>(g, idx, w, gbase, gvalues, rows, iu, gb_units, units)
  if (vec && narrow) {
    if (fused) OXI_SRB(true, true, true);
    else OXI_SRB(true, true, false);
  } else if (vec) {
    if (fused) OXI_SRB(true, false, true);
    else OXI_SRB(true, false, false);
  } else {
    if (fused) OXI_SRB(false, false, true);
    else OXI_SRB(false, false, false);
  }
#undef OXI_SRB
  return check_launch("scatter_rows_bwd");
}

int oxi_masked_select_record_bytes(const int64_t* shape, int ndim, int64_t* bytes) {
  if (!bytes) return fail(OXI_INVALID_ARGUMENT, "masked_select_record_bytes: NULL bytes");
  int64_t E = 0, T = 0;
  int rc = grid_size(shape, ndim, &E, &T, "masked_select_record_bytes");
  if (rc != OXI_OK) return rc;
  *bytes = record_bytes(T);
  return OXI_OK;
}

int oxi_masked_select(const float* x, const int64_t* x_strides, const float* mask, const int64_t* m_strides,
                      const int64_t* shape, int ndim, float** out, int64_t* count, void* record) {
  if (!out || !count) return fail(OXI_INVALID_ARGUMENT, "masked_select: NULL out or count");
  *out = nullptr;
  *count = 0;
  int64_t E = 0, T = 0;
  int rc = grid_size(shape, ndim, &E, &T, "masked_select");
  if (rc != OXI_OK || E == 0) return rc;
  if (ndim > 0 && (!x_strides || !m_strides)) return fail(OXI_INVALID_ARGUMENT, "masked_select: NULL strides");
  if (!x || !mask) return fail(OXI_INVALID_ARGUMENT, "masked_select: NULL tensor pointer");
  OXI_CHECK_INIT();
  const int64_t* st2[2] = {x_strides, m_strides};
  const Grid<2> g2 = make_grid<2>(shape, ndim, st2);
  const Grid<1> g1 = make_grid<1>(shape, ndim, st2);
  const bool fast2 = contiguous(g2, 0) && contiguous(g2, 1) && al16(x) && al16(mask);
  const bool fast1 = contiguous(g1, 0) && al16(x);
  Workspace wr(record ? 0 : (size_t)record_bytes(T));
  if (!record && !wr.p) return fail_alloc("masked_select: workspace");
  int64_t* offs = static_cast<int64_t*>(record ? record : wr.p);
  uint64_t* rec = reinterpret_cast<uint64_t*>(offs + T + 1);
  hipStream_t st = stream();
  // One pass when the output can hold every grid point (its tensor uses the
  // first `count`), else the count pass, the scan and the write pass, which
  // read x twice but allocate the output at its exact size: always with
  // OXI_MASKED_SELECT_EXACT=1, for callers short of device memory.
  const char* exact_env = std::getenv("OXI_MASKED_SELECT_EXACT");
  const bool exact = exact_env && std::strcmp(exact_env, "1") == 0;
  void* big = nullptr;
  if (!exact && oxi_hip_alloc(sizeof(float) * (size_t)E, &big) == OXI_OK && big) {
    const int64_t C = ceil_div(T, MSEL_CHUNK);
    Workspace wl(sizeof(uint64_t) * (size_t)C + 16);  // chunk status words, then the ticket
    if (!wl.p) {
      oxi_hip_free(big);
      return fail_alloc("masked_select: look-back workspace");
    }
    uint64_t* status = wl.as<uint64_t>();
    int* ticket = reinterpret_cast<int*>(status + C);
    // all-zero bits: no chunk published, ticket 0 (a fill kernel, not a memset)
    if ((rc = oxi_fill(wl.as<float>(), 2 * C + 4, 0.0f)) != OXI_OK) {
      oxi_hip_free(big);
      return rc;
    }
    int64_t total = -1;
    {
      std::lock_guard<std::mutex> lk(readback_mutex());
      int64_t* slot = readback_slot();
      *static_cast<volatile int64_t*>(slot) = -1;
      // polls of about 1 us: a wait past a second is a failure (never seen);
      // OXI_MSEL_SPIN_LIMIT=-1 fails every wait, to test that path
      const char* sl = std::getenv("OXI_MSEL_SPIN_LIMIT");
      const int SPIN_LIMIT = sl && std::strcmp(sl, "-1") == 0 ? -1 : 1 << 20;
      if (fast2)
        msel_onepass_k<true, MSEL_CHUNK><<<(unsigned)C, MB, 0, st>>>(
            g2, x, mask, E, T, status, ticket, offs, rec, static_cast<float*>(big), slot, guard_flag(), SPIN_LIMIT);
      else
        msel_onepass_k<false, MSEL_CHUNK><<<(unsigned)C, MB, 0, st>>>(
            g2, x, mask, E, T, status, ticket, offs, rec, static_cast<float*>(big), slot, guard_flag(), SPIN_LIMIT);
      if ((rc = check_launch("masked_select")) == OXI_OK) rc = poll_total(slot, st, &total);
      if (rc != OXI_OK) {
        oxi_hip_free(big);
        return rc;
      }
    }
    if (total < 0) {
      oxi_hip_free(big);
      return fail(OXI_OTHER, "masked_select: a tile's offset wait did not finish (look-back)");
    }
    if (total == 0) {
      oxi_hip_free(big);
      return OXI_OK;
    }
    // Picks that fill at most a third of the grid-sized buffer move into an
    // exact-size one (the copy queued after the kernel), so a sparse mask's
    // result holds at most three times its picks' memory; if that allocation
    // fails, the grid-sized buffer is kept.
    if (total * 3 <= E) {
      void* exact = nullptr;
      if (oxi_hip_alloc(sizeof(float) * (size_t)total, &exact) == OXI_OK && exact) {
        const hipError_t e = hipMemcpyAsync(exact, big, sizeof(float) * (size_t)total, hipMemcpyDeviceToDevice, st);
        oxi_hip_free(e == hipSuccess ? big : exact);
        if (e != hipSuccess) {
          oxi_hip_free(big);
          return fail_hip(e, "hipMemcpyAsync(masked_select)");
        }
        big = exact;
      }
    }
    *out = static_cast<float*>(big);
    *count = total;
    return OXI_OK;
  }
  Workspace wc(sizeof(int) * (size_t)T);
  if (!wc.p) return fail_alloc("masked_select: workspace");
  if (fast2) msel_count_k<true><<<(unsigned)T, MB, 0, st>>>(g2, x, mask, E, wc.as<int>(), rec);
  else msel_count_k<false><<<(unsigned)T, MB, 0, st>>>(g2, x, mask, E, wc.as<int>(), rec);
  int64_t total = 0;
  {
    // the scan stores the total straight to pinned host memory
    std::lock_guard<std::mutex> lk(readback_mutex());
    int64_t* slot = readback_slot();
    msel_scan_k<<<1, SCAN_BS, 0, st>>>(wc.as<int>(), T, offs, slot);
    if ((rc = check_launch("masked_select(count)")) != OXI_OK) return rc;
    const hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return fail_hip(e, "hipStreamSynchronize(masked_select)");
    total = *static_cast<volatile int64_t*>(slot);
  }
  if (total == 0) return OXI_OK;
  void* buf = nullptr;
  if (oxi_hip_alloc(sizeof(float) * (size_t)total, &buf) != OXI_OK) return fail_alloc("masked_select: output");
  float* o = static_cast<float*>(buf);
  if (fast1) msel_write_k<true><<<(unsigned)T, MB, 0, st>>>(g1, x, E, offs, rec, o);
  else msel_write_k<false><<<(unsigned)T, MB, 0, st>>>(g1, x, E, offs, rec, o);
  if ((rc = check_launch("masked_select")) != OXI_OK) {
    oxi_hip_free(buf);
    return rc;
  }
  *out = o;
  *count = total;
  return OXI_OK;
}

int oxi_masked_select_bwd(const void* record, const int64_t* shape, int ndim, const float* g, int64_t count,
                          float* grad_x, const int64_t* gx_strides, int64_t x_numel) {
  if (count < 0 || x_numel < 0) return fail(OXI_INVALID_ARGUMENT, "masked_select_bwd: negative size");
  int64_t E = 0, T = 0;
  int rc = grid_size(shape, ndim, &E, &T, "masked_select_bwd");
  if (rc != OXI_OK) return rc;
  if (ndim > 0 && !gx_strides) return fail(OXI_INVALID_ARGUMENT, "masked_select_bwd: NULL gradient strides");
  if (E == 0) {
    if (count != 0)
      return fail(OXI_SHAPE_MISMATCH, "masked_select_bwd: %lld upstream gradients for 0 picks", (long long)count);
    if (x_numel == 0) return OXI_OK;
    if (!grad_x) return fail(OXI_INVALID_ARGUMENT, "masked_select_bwd: NULL grad_x");
    return oxi_fill(grad_x, x_numel, 0.0f);
  }
  // x's own elements are the grid dims where its gradient layout has a
  // stride; every gradient offset must land inside x_numel
  int64_t xn = 1, last = 0;
  bool bcast = false;
  for (int d = 0; d < ndim; ++d) {
    if (gx_strides[d] < 0) return fail(OXI_INVALID_ARGUMENT, "masked_select_bwd: negative gradient stride");
    if (gx_strides[d] != 0) xn *= shape[d];
    else if (shape[d] > 1) bcast = true;
    last += (shape[d] - 1) * gx_strides[d];
  }
  if (xn != x_numel || last >= x_numel)
    return fail(OXI_INVALID_ARGUMENT, "masked_select_bwd: gradient strides do not describe %lld elements",
                (long long)x_numel);
  if (!record || !grad_x || (count > 0 && !g)) return fail(OXI_INVALID_ARGUMENT, "masked_select_bwd: NULL pointer");
  OXI_CHECK_INIT();
  const int64_t* offs = static_cast<const int64_t*>(record);
  const uint64_t* rec = reinterpret_cast<const uint64_t*>(offs + T + 1);
  Workspace wt(bcast ? sizeof(float) * (size_t)E : 0);
  if (bcast && !wt.p) return fail_alloc("masked_select_bwd: workspace");
  // the gradient layout: x's own (no broadcast) or a dense grid-order buffer
  int64_t rms[MAXD];
  int64_t acc = 1;
  for (int d = ndim - 1; d >= 0; --d) {
    rms[d] = acc;
    acc *= shape[d];
  }
  const int64_t* st1[1] = {bcast ? rms : gx_strides};
  const Grid<1> go = make_grid<1>(shape, ndim, st1);
  float* dst = bcast ? wt.as<float>() : grad_x;
  const bool fast = contiguous(go, 0) && al16(dst);
  hipStream_t st = stream();
  const bool nts = nt_stores(E * 4);
  if (fast && nts) msel_grad_k<true, true><<<(unsigned)T, MB, 0, st>>>(go, E, offs, rec, g, count, dst, T, guard_flag());
  else if (fast) msel_grad_k<true, false><<<(unsigned)T, MB, 0, st>>>(go, E, offs, rec, g, count, dst, T, guard_flag());
  else msel_grad_k<false, false><<<(unsigned)T, MB, 0, st>>>(go, E, offs, rec, g, count, dst, T, guard_flag());
  if (bcast) {
    AccPlan a{};
    a.npts = 1;
    for (int d = 0; d < ndim; ++d) {
      if (shape[d] == 1) continue;
      if (gx_strides[d] != 0) {
        a.ksize[a.nk] = shape[d];
        a.kstride[a.nk++] = rms[d];
      } else {
        a.bsize[a.nb] = shape[d];
        a.bstride[a.nb++] = rms[d];
        a.npts *= shape[d];
      }
    }
    msel_accum_k<<<(unsigned)ceil_div(x_numel, BS), BS, 0, st>>>(a, wt.as<float>(), x_numel, grad_x);
  }
  return check_launch("masked_select_bwd");
}

}  // extern "C"
