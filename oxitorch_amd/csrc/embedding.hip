// index_select gather and its deterministic duplicate-accumulating VJP
// (F.embedding: python/oxitorch/nn/functional.py:245-247; Tensor::index_select:
// crates/oxi-tensor/src/lib.rs:665-703; scatter_index_select:
// crates/oxi-autograd/src/ops.rs:741-769).
//
// Gather: out[o, k, :] = src[o, idx[k], :]. Each block copies GRPB (2) rows
// with float4 accesses, the rows' loads issued together; threads per block
// are the row's float4 count rounded up to whole waves.
//
// VJP without float atomics (6 launches for 16-bit keys):
//   1. stable LSD radix sort of (key, position) by 8-bit digits, a histogram
//      and a scatter kernel per pass; keys are the ids wrapped to [0, len),
//      out-of-range ids get the sentinel key `len` (never summed) and raise
//      the guard flag; the first scatter flags every key that occurs;
//   2. segmented reduction over the sorted positions: one wave per (tile of
//      <= 64 positions, 64-vector column chunk) sums every run of equal keys
//      in position order in f32 -- the reference's own order, so a run of at
//      most one tile's length gives a bit-identical row -- writing it straight
//      to the output (a run into the next tile too: its wave reads on); a
//      longer run leaves per-tile partial sums formed in float64; the same
//      launch writes the zero rows of keys that never occur;
//   3. fix-up: each key of a longer run adds its partial sums in tile order in
//      float64, so its row is its float64 sum rounded once to f32 (the
//      reference's sequential f32 sum drifts from that by up to a few hundred
//      ulp over a 41k-position run; the parity bar for such rows is the
//      float64 sum).
// Every wave of step 2 does the same amount of work whatever the id
// distribution (a key owning a third of all positions is spread over many
// tiles).
#include <algorithm>
#include <type_traits>

#include "internal.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;
// Rows per gather block. Measured in the cold step (the table's rows first
// come from HBM): C4's gather 130.7 us at 2 rows, 123.8 at 4, 124.0 at 8;
// C5's 24.3-24.6, 22.6-23.0 and 21.6 us. With the table in the Infinity
// Cache (warm) 2 rows measured best (C4 90.2 against 92.7 us at 4).
#ifndef OXI_GRPB
#define OXI_GRPB 4
#endif
constexpr int GRPB = OXI_GRPB;

__device__ __forceinline__ int64_t wrap_id(int64_t id, int64_t len, bool& ok) {
  if (id < 0) id += len;
  ok = (id >= 0 && id < len);
  return ok ? id : 0;
}

// ---------------------------------------------------------------------------
// Gather.

template <bool VEC, bool NTS>
__global__ __launch_bounds__(BS) void gather_k(const float* __restrict__ src, int64_t outer, int64_t len,
                                               int64_t inner, const int64_t* __restrict__ idx, int64_t n,
                                               float* __restrict__ out, int* __restrict__ guard) {
  const int64_t rows = outer * n;
  const int64_t r0 = (int64_t)blockIdx.x * GRPB;
  const int64_t units = VEC ? inner / 4 : inner;
  int64_t srow[GRPB];
  bool okr[GRPB];
#pragma unroll
  for (int r = 0; r < GRPB; ++r) {
    const int64_t row = r0 + r;
    okr[r] = false;
    srow[r] = 0;
    if (row < rows) {
      const int64_t o = row / n, k = row % n;
      bool ok;
      const int64_t id = wrap_id(idx[k], len, ok);
      okr[r] = ok;
      srow[r] = (o * len + id) * inner;
      if (!ok && threadIdx.x == 0) atomicOr(guard, 1);
    }
  }
  for (int64_t c = threadIdx.x; c < units; c += blockDim.x) {
    if constexpr (VEC) {
      f4 v[GRPB];
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        v[r] = (r0 + r < rows && okr[r]) ? reinterpret_cast<const f4*>(src + srow[r])[c] : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        if (r0 + r < rows) st_stream<NTS>(v[r], reinterpret_cast<f4*>(out + (r0 + r) * inner) + c);
    } else {
      float v[GRPB];
#pragma unroll
      for (int r = 0; r < GRPB; ++r) v[r] = (r0 + r < rows && okr[r]) ? src[srow[r] + c] : 0.f;
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        if (r0 + r < rows) out[(r0 + r) * inner + c] = v[r];
    }
  }
}

// Gather when rows are short (inner < 64): one element per thread.
__global__ __launch_bounds__(BS) void gather_elem_k(const float* __restrict__ src, int64_t outer, int64_t len,
                                                    int64_t inner, const int64_t* __restrict__ idx, int64_t n,
                                                    float* __restrict__ out, int* __restrict__ guard) {
  const int64_t total = outer * n * inner;
  for (int64_t e = (int64_t)blockIdx.x * BS + threadIdx.x; e < total; e += (int64_t)gridDim.x * BS) {
    const int64_t i = e % inner;
    const int64_t row = e / inner;
    const int64_t o = row / n, k = row % n;
    bool ok;
    const int64_t id = wrap_id(idx[k], len, ok);
    if (!ok) atomicOr(guard, 1);
    out[e] = ok ? src[(o * len + id) * inner + i] : 0.f;
  }
}

// ---------------------------------------------------------------------------
// Batch gather: the rows `idx` of up to BG_MAX columns sharing dim 0, one
// launch. A block belongs to one column: GRPB rows of it (rows of 64 or more
// floats, float4 when aligned) or BS elements (shorter rows).

constexpr int BG_MAX = 8;
enum BgMode : int { BG_ROWS = 0, BG_ROWS4 = 1, BG_ELEMS = 2 };

struct BatchArgs {
  const float* src[BG_MAX];
  float* dst[BG_MAX];
  int64_t inner[BG_MAX];
  unsigned block_end[BG_MAX];  // exclusive end of each column's blocks
  int mode[BG_MAX];
  int count;
};

template <bool NTS>
__global__ __launch_bounds__(BS) void batch_gather_k(BatchArgs a, int64_t len, const int64_t* __restrict__ idx,
                                                     int64_t n, int* __restrict__ guard) {
  int c = 0;
  while (c + 1 < a.count && blockIdx.x >= a.block_end[c]) ++c;
  const int64_t b = (int64_t)blockIdx.x - (c ? a.block_end[c - 1] : 0u);
  const float* __restrict__ src = a.src[c];
  float* __restrict__ dst = a.dst[c];
  const int64_t inner = a.inner[c];
  const int mode = a.mode[c];
  if (mode == BG_ELEMS) {
    const int64_t e = b * BS + threadIdx.x;
    if (e < n * inner) {
      const int64_t k = e / inner, i = e % inner;
      bool ok;
      const int64_t id = wrap_id(idx[k], len, ok);
      if (!ok) atomicOr(guard, 1);
      dst[e] = ok ? src[id * inner + i] : 0.f;
    }
    return;
  }
  const int64_t r0 = b * GRPB;
  int64_t srow[GRPB];
  bool okr[GRPB];
#pragma unroll
  for (int r = 0; r < GRPB; ++r) {
    okr[r] = false;
    srow[r] = 0;
    if (r0 + r < n) {
      bool ok;
      const int64_t id = wrap_id(idx[r0 + r], len, ok);
      okr[r] = ok;
      srow[r] = id * inner;
      if (!ok && threadIdx.x == 0) atomicOr(guard, 1);
    }
  }
  if (mode == BG_ROWS4) {
    const int64_t units = inner / 4;
    for (int64_t u = threadIdx.x; u < units; u += BS) {
      f4 v[GRPB];
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        v[r] = (r0 + r < n && okr[r]) ? reinterpret_cast<const f4*>(src + srow[r])[u] : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        if (r0 + r < n) st_stream<NTS>(v[r], reinterpret_cast<f4*>(dst + (r0 + r) * inner) + u);
    }
  } else {
    for (int64_t u = threadIdx.x; u < inner; u += BS) {
      float v[GRPB];
#pragma unroll
      for (int r = 0; r < GRPB; ++r) v[r] = (r0 + r < n && okr[r]) ? src[srow[r] + u] : 0.f;
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        if (r0 + r < n) dst[(r0 + r) * inner + u] = v[r];
    }
  }
}

// ---------------------------------------------------------------------------
// VJP, sort: stable LSD radix sort of (key, position) pairs, 8-bit digits.
// Keys are the ids wrapped to [0, len); an out-of-range id gets the sentinel
// key `len` (sorted last, never summed) and raises the guard flag. A block owns
// a tile of SBS * IPT consecutive elements. Per pass:
//   sort_hist_k    per-tile digit counts (LDS integer atomics: exact) into a
//                  tile-major table cnt[tile * 256 + digit];
//   sort_scatter_k each block first derives its tile's 256 output offsets
//                  from the whole table (digit-major exclusive prefix: the
//                  stable order), then sends each element to its digit's
//                  offset plus the number of earlier elements of the tile with
//                  that digit (wave ballots + per-wave LDS counts).
// Tables of more than 256 tiles are scanned once by sort_offsets_k instead.
// The first pass reads the int64 ids directly and flags every key present.

constexpr int SBS = 256;
constexpr int SCAN_REG = 64;     // table rows one thread holds at a time
constexpr int SELF_SCAN_MAX = 256;  // tiles up to which each scatter block scans the table itself
constexpr int SEEN = 1024;       // LDS filter of recently flagged keys

// Key of a raw id (no memory access: callers load a batch of ids first, so
// that the loads are in flight together, then convert and report once).
__device__ __forceinline__ int key_from(int64_t raw, int64_t len, bool& bad) {
  bool ok;
  const int64_t id = wrap_id(raw, len, ok);
  bad |= !ok;
  return ok ? (int)id : (int)len;
}

// Exclusive scan of the 256 per-digit values `v` of the block (thread t
// holds digit t's value); returns thread t's exclusive prefix. `ws` holds 4 ints.
__device__ __forceinline__ int block_excl_scan256(int v, int* ws) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) ws[w] = inc;
  __syncthreads();
  int pre = 0;
#pragma unroll
  for (int q = 0; q < SBS / 64; ++q) pre += (q < w) ? ws[q] : 0;
  return pre + inc - v;
}

// Digit t's counts (thread t) summed over all `ntiles` tiles of the table,
// and over the tiles before `upto`.
__device__ __forceinline__ void column_sums(const int* __restrict__ tab, int ntiles, int upto, int& total,
                                            int& before) {
  total = 0;
  before = 0;
  for (int jb = 0; jb < ntiles; jb += SCAN_REG) {
    int v[SCAN_REG];
#pragma unroll
    for (int q = 0; q < SCAN_REG; ++q) {
      const int j = min(jb + q, ntiles - 1);  // always in range: loads issue together
      v[q] = tab[(int64_t)j * 256 + threadIdx.x];
    }
#pragma unroll
    for (int q = 0; q < SCAN_REG; ++q) {
      total += (jb + q < ntiles) ? v[q] : 0;
      before += (jb + q < upto) ? v[q] : 0;
    }
  }
}

template <int IPT, bool FROM_IDX>
__global__ __launch_bounds__(SBS) void sort_hist_k(const int64_t* __restrict__ idx, const int* __restrict__ keys,
                                                   int64_t n, int64_t len, int shift, int* __restrict__ tab,
                                                   int* __restrict__ present, int* __restrict__ owner_count,
                                                   int* guard) {
  __shared__ int cnt[256];
  const int t = threadIdx.x;
  cnt[t] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * (SBS * IPT);
  int k[IPT];
  if constexpr (FROM_IDX) {
    int64_t raw[IPT];
#pragma unroll
    for (int i = 0; i < IPT; ++i) raw[i] = idx[min<int64_t>(base + i * SBS + t, n - 1)];
    bool bad = false;
#pragma unroll
    for (int i = 0; i < IPT; ++i) k[i] = (base + i * SBS + t < n) ? key_from(raw[i], len, bad) : -1;
    if (bad) atomicOr(guard, 1);
  } else {
#pragma unroll
    for (int i = 0; i < IPT; ++i) k[i] = keys[min<int64_t>(base + i * SBS + t, n - 1)];
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if (base + i * SBS + t >= n) k[i] = -1;
  }
#pragma unroll
  for (int i = 0; i < IPT; ++i)
    if (k[i] >= 0) atomicAdd(&cnt[(k[i] >> shift) & 255], 1);  // LDS integer atomics: exact counts
  if (present)  // first pass: clear this call's present-key flags and owner count
    for (int64_t v = (int64_t)blockIdx.x * SBS + t; v < len; v += (int64_t)gridDim.x * SBS) present[v] = 0;
  if (owner_count && blockIdx.x == 0 && t == 0) *owner_count = 0;
  __syncthreads();
  tab[(int64_t)blockIdx.x * 256 + t] = cnt[t];
}

// One block: the count table becomes the offset table, in place.
__global__ __launch_bounds__(SBS) void sort_offsets_k(int* tab, int ntiles) {
  __shared__ int ws[SBS / 64];
  const int t = threadIdx.x;
  int total, unused;
  column_sums(tab, ntiles, 0, total, unused);
  int run = block_excl_scan256(total, ws);
  for (int j = 0; j < ntiles; ++j) {
    const int x = tab[(int64_t)j * 256 + t];
    tab[(int64_t)j * 256 + t] = run;
    run += x;
  }
}

// How a scatter block finds its 256 output offsets.
enum { OFFS_TABLE = 0, OFFS_SCAN_COUNTS = 1 };

template <int IPT, bool FROM_IDX, int OFFS>
__global__ __launch_bounds__(SBS) void sort_scatter_k(const int64_t* __restrict__ idx, const int* __restrict__ keys,
                                                      const int* __restrict__ vals, int64_t n, int64_t len, int shift,
                                                      int ntiles, const int* __restrict__ tab,
                                                      int* __restrict__ keys_out, int* __restrict__ vals_out,
                                                      int* __restrict__ present, int* guard) {
  __shared__ int base[256];
  __shared__ int cnt[SBS / 64][256];
  __shared__ int ws[SBS / 64];
  __shared__ int seen[SEEN];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t tile0 = (int64_t)blockIdx.x * (SBS * IPT);
  // all of this thread's elements up front: one load latency for the tile
  int kk[IPT], vv[IPT];
  if constexpr (FROM_IDX) {
    int64_t raw[IPT];
#pragma unroll
    for (int r = 0; r < IPT; ++r) raw[r] = idx[min<int64_t>(tile0 + r * SBS + t, n - 1)];
    bool bad = false;
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
      const int64_t p = tile0 + r * SBS + t;
      kk[r] = p < n ? key_from(raw[r], len, bad) : 0;
      vv[r] = (int)p;
    }
    if (bad) atomicOr(guard, 1);
  } else {
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
      const int64_t pc = min<int64_t>(tile0 + r * SBS + t, n - 1);
      kk[r] = keys[pc];
      vv[r] = vals[pc];
    }
  }
  if constexpr (OFFS == OFFS_SCAN_COUNTS) {
    int total, before;
    column_sums(tab, ntiles, (int)blockIdx.x, total, before);
    base[t] = block_excl_scan256(total, ws) + before;
  } else {
    base[t] = tab[(int64_t)blockIdx.x * 256 + t];
  }
  if constexpr (FROM_IDX) {
    // flag every key present; the LDS filter drops repeats of hot keys
    for (int q = t; q < SEEN; q += SBS) seen[q] = -1;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < IPT; ++r) {
      const int k = kk[r];
      if (tile0 + r * SBS + t < n && (uint64_t)k < (uint64_t)len && seen[k & (SEEN - 1)] != k) {
        seen[k & (SEEN - 1)] = k;  // racing writers store the same flag: harmless
        present[k] = 1;
      }
    }
  }
  const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int r = 0; r < IPT; ++r) {
    const int64_t p = tile0 + r * SBS + t;
    const bool valid = p < n;
    const int k = kk[r], v = vv[r];
    const int d = (k >> shift) & 255;
    unsigned long long peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1;
      const unsigned long long m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
#pragma unroll
    for (int q = 0; q < SBS / 64; ++q) cnt[q][t] = 0;
    __syncthreads();
    if (valid && (__ffsll((long long)peers) - 1) == lane) cnt[w][d] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pre = base[d];
      for (int q = 0; q < w; ++q) pre += cnt[q][d];
      const int dst = pre + __popcll(peers & lt);
      if ((uint64_t)dst < (uint64_t)n) {
        keys_out[dst] = k;
        vals_out[dst] = v;
      } else {
        atomicOr(guard, 2);  // inconsistent offsets: reported, never written out of range
      }
    }
    __syncthreads();
    int add = 0;
#pragma unroll
    for (int q = 0; q < SBS / 64; ++q) add += cnt[q][t];
    base[t] += add;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// VJP, segmented reduction. The sorted positions are cut into tiles of `st`
// (<= 64) positions; one wave owns a (tile, 64-column-vector chunk) pair and
// holds the tile's keys and positions one per lane. Every run of equal keys is
// summed in position order in f32 -- the reference's own order, so such a run
// gives a bit-identical row:
//  * a run inside the tile is written to its output row;
//  * a run that starts in the tile and ends in the next one is finished by
//    this wave, which reads on into the next tile's positions (the next tile's
//    wave skips it);
//  * a longer run (a "long key") is summed per tile in float64 into partial
//    slots -- 2*tile+1 where it continues into the next tile, 2*tile where it
//    ends --
//    and the tile where it starts joins the owner list while the tile where it
//    ends records itself in end_tile[key]; seg_fixup_k adds the slots.
// Zero rows for keys that never occur (ZR rows per block) are written by
// blocks past the segment work, so those writes overlap the gathers, or, from
// DB_MIN_IDS ids on, by blocks past the fix-up work (see the launch).

// Rows in flight per lane, and the longest segment tile (below). Measured on
// C4 (131072 Zipf ids, 1024-float rows), C4 step: 8 and 64 take 252 us;
// 4 rows 264 us, 32-position tiles 259 us, 16 or 32 rows (the accumulation
// loop no longer unrolls) 440-463 us.
#ifndef OXI_SEG_U
#define OXI_SEG_U 8
#endif
constexpr int SEG_U = OXI_SEG_U;
#ifndef OXI_SEG_ZR
#define OXI_SEG_ZR 4
#endif
constexpr int ZR = OXI_SEG_ZR;  // zero rows per block
// Waves per SIMD the segment kernel is held to: at 5 it fits 84 VGPRs with no
// spill (unbounded, the compiler takes 120: 4 waves). Measured: C5's
// embedding VJP 35.8-36.1 us against 38.5-38.8; C4's unchanged (145-148 us).
// At 6 and 8 it spills 4 and 24 VGPRs. Segment blocks spread evenly among the
// zero-row blocks (instead of first) measured 42-46 us on C5, 147-149 on C4.
#ifndef OXI_SEG_WPE
#define OXI_SEG_WPE 5
#endif
// DB: the loads of the next SEG_U positions issue before the current ones
// are added (two register sets, 141 VGPRs: 3 waves per SIMD). Measured in
// the cold step: C4's embedding VJP 158.6 us against 164.9 single-buffered;
// C5's 48.5 against 38.3 us (a small grid needs the occupancy), so it is
// taken from DB_MIN_IDS ids on. At 4 waves per SIMD it spills (173 us);
// 6 rows at 4 waves took 161.9 us, 4 rows at 5 waves 167.4.
constexpr int64_t DB_MIN_IDS = 65536;

// The dW rows of keys that never occur, ZR per block (block zb of the
// zero-row blocks), written with zeros.
template <bool VEC, bool NTS>
__device__ __forceinline__ void zero_rows(int64_t zb, const int* __restrict__ present, float* __restrict__ grad,
                                          int64_t outer, int64_t len, int64_t inner) {
  const int64_t units = VEC ? inner / 4 : inner;
  const int64_t v0 = zb * ZR;
  for (int r = 0; r < ZR; ++r) {
    const int64_t v = v0 + r;
    if (v >= len || present[v]) continue;
    for (int64_t o = 0; o < outer; ++o) {
      float* dst = grad + (o * len + v) * inner;
      for (int64_t c = threadIdx.x; c < units; c += 256) {
        if constexpr (VEC) st_stream<NTS>(f4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<f4*>(dst) + c);
        else st_stream<NTS>(0.f, dst + c);
      }
    }
  }
}

template <bool VEC, bool NTS, bool DB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DB ? 3 : OXI_SEG_WPE))) void seg_wave_k(
    const float* __restrict__ g, int64_t outer, int64_t n, int64_t inner, int64_t len,
    const int* __restrict__ skeys, const int* __restrict__ perm, float* __restrict__ grad,
    double* __restrict__ part, const int* __restrict__ present, int* __restrict__ owners,
    int* __restrict__ owner_count, int* __restrict__ end_tile, int st, int64_t stiles, int chunks,
    int64_t seg_blocks) {
  using V = typename std::conditional<VEC, f4, float>::type;
  const int64_t units = VEC ? inner / 4 : inner;
  if ((int64_t)blockIdx.x >= seg_blocks) {
    zero_rows<VEC, NTS>((int64_t)blockIdx.x - seg_blocks, present, grad, outer, len, inner);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t tile = item / chunks;
  const int chunk = (int)(item - tile * chunks);
  if (tile >= stiles) return;  // uniform per wave
  const int64_t p0 = tile * st;
  const int cnt = (int)min<int64_t>(st, n - p0);
  const int64_t p1 = p0 + cnt;                       // first position of the next tile
  const int cnt2 = (int)min<int64_t>(st, n - p1);    // its size (<= 0 if none)
  // this tile and, speculatively, the next one (for a run reaching into it)
  const int my_key = lane < cnt ? skeys[p0 + lane] : -2;
  const int my_pos = lane < cnt ? perm[p0 + lane] : 0;
  const int nx_key = lane < cnt2 ? skeys[p1 + lane] : -2;
  const int nx_pos = lane < cnt2 ? perm[p1 + lane] : 0;
  const int key_before = p0 > 0 ? skeys[p0 - 1] : -1;
  const int key_after2 = p1 + cnt2 < n ? skeys[p1 + max(cnt2, 0)] : -1;  // first key after the next tile
  const int key_prev2 = p0 - st - 1 >= 0 ? skeys[p0 - st - 1] : -1;      // key before the previous tile
  const int key_after = __builtin_amdgcn_readfirstlane(nx_key) ;          // -2 when there is no next tile
  const int nxt0 = __shfl_down(my_key, 1, 64);
  const int nxt = (lane == cnt - 1) ? key_after : nxt0;
  // run ends inside the tile: key changes, or the tile's last position
  const unsigned long long ends = __ballot(lane < cnt && (nxt != my_key || lane == cnt - 1));
  const int key0 = __builtin_amdgcn_readfirstlane(my_key);
  const int keyl = __builtin_amdgcn_readlane(my_key, cnt - 1);
  const bool head_inc = key_before == key0;   // first run continues from the previous tile
  const bool tail_inc = key_after == keyl;    // last run continues into the next tile
  const bool single = key0 == keyl;           // the tile holds one key
  // tail run that starts here and continues: ends in the next tile (extend)
  // or runs past it (long key, this tile owns it)
  const bool tail_here = tail_inc && !(head_inc && single);
  const unsigned long long nx_diff = __ballot(lane < cnt2 && nx_key != keyl);
  const bool tail_long = tail_here && nx_diff == 0 && key_after2 == keyl;
  const bool tail_ext = tail_here && !tail_long;
  const int ext_len = tail_ext ? (nx_diff ? (__ffsll((long long)nx_diff) - 1) : cnt2) : 0;
  // head run that continues from the previous tile and ends here: skipped if
  // it started in the previous tile (that wave finished it), else a long key
  const bool head_end = head_inc && !(tail_inc && single);
  const bool head_skip = head_end && key_prev2 != key0;
  if (chunk == 0 && lane == 0) {
    if (tail_long && (uint64_t)keyl < (uint64_t)len) {
      const int oi = atomicAdd(owner_count, 1);
      owners[2 * oi] = (int)tile;  // with its key: one dependent load less in the fix-up
      owners[2 * oi + 1] = keyl;
    }
    if (head_end && !head_skip && (uint64_t)key0 < (uint64_t)len) end_tile[key0] = (int)tile;
  }
  const int first = head_skip ? __ffsll((long long)ends) : 0;  // one past the head run's end
  const int64_t u = (int64_t)chunk * 64 + lane;
  const bool active = u < units;
  const int64_t slot_head = 2 * tile, slot_tail = slot_head + 1;
  constexpr int NC = VEC ? 4 : 1;
  for (int64_t o = 0; o < outer; ++o) {
    const float* gb = g + o * n * inner;
    V acc = V{};
    // the same run summed in float64: what a partial slot of a long key
    // (a run over more than two tiles) receives
    double accd[NC];
#pragma unroll
    for (int q = 0; q < NC; ++q) accd[q] = 0.0;
    int start = first;
    auto consume = [&](V (&vals)[SEG_U], int i) {
#pragma unroll
      for (int j = 0; j < SEG_U; ++j) {
        const int q = i + j;
        if (q >= cnt) break;
        acc = acc + vals[j];
        if constexpr (VEC) {
          accd[0] += (double)vals[j].x;
          accd[1] += (double)vals[j].y;
          accd[2] += (double)vals[j].z;
          accd[3] += (double)vals[j].w;
        } else {
          accd[0] += (double)vals[j];
        }
        if (((ends >> q) & 1ull) && !(tail_ext && q == cnt - 1)) {  // run [start, q] ends here
          const int key = __builtin_amdgcn_readlane(my_key, q);
          if ((uint64_t)key < (uint64_t)len && active) {
            const bool to_tail = tail_inc && q == cnt - 1;
            const bool to_head = !to_tail && head_inc && start == 0;
            if (to_tail || to_head) {  // float64 partial slots, re-read by the fix-up: plain stores
              double* dst = part + (((to_tail ? slot_tail : slot_head) * outer + o) * inner + u * NC);
#pragma unroll
              for (int c = 0; c < NC; ++c) dst[c] = accd[c];
            } else {
              float* dst = grad + (o * len + key) * inner;
              if constexpr (VEC) st_stream<NTS>(acc, reinterpret_cast<f4*>(dst) + u);
              else st_stream<NTS>(acc, dst + u);
            }
          }
          acc = V{};
#pragma unroll
          for (int c = 0; c < NC; ++c) accd[c] = 0.0;
          start = q + 1;
        }
      }
    };
    if constexpr (DB) {
      // Every load issues (its position clamped into the tile, an invalid
      // one read as row 0 and zeroed), so each wait counts exactly the
      // younger loads.
      auto load_batch = [&](V (&v)[SEG_U], int i) {
#pragma unroll
        for (int j = 0; j < SEG_U; ++j) {
          const int pj = __builtin_amdgcn_readlane(my_pos, min(i + j, cnt - 1));
          const bool okp = (uint64_t)pj < (uint64_t)n;
          const float* row = gb + (int64_t)(okp ? pj : 0) * inner;
          V t = V{};
          if (active) {
            if constexpr (VEC) t = ld_stream(reinterpret_cast<const f4*>(row) + u);
            else t = ld_stream(row + u);
          }
          v[j] = okp ? t : V{};
        }
      };
      V va[SEG_U], vb[SEG_U];
      if (first < cnt) load_batch(va, first);
      for (int i = first; i < cnt;) {
        load_batch(vb, i + SEG_U);
        __builtin_amdgcn_sched_barrier(0);
        consume(va, i);
        i += SEG_U;
        if (i >= cnt) break;
        load_batch(va, i + SEG_U);
        __builtin_amdgcn_sched_barrier(0);
        consume(vb, i);
        i += SEG_U;
      }
    } else {
      for (int i = first; i < cnt; i += SEG_U) {
        V vals[SEG_U];
#pragma unroll
        for (int j = 0; j < SEG_U; ++j) {
          vals[j] = V{};
          const int pj = __builtin_amdgcn_readlane(my_pos, (i + j) & 63);  // uniform; used only if i + j < cnt
          if (i + j < cnt && active && (uint64_t)pj < (uint64_t)n) {
            const float* row = gb + (int64_t)pj * inner;
            if constexpr (VEC) vals[j] = ld_stream(reinterpret_cast<const f4*>(row) + u);
            else vals[j] = ld_stream(row + u);
          }
        }
        consume(vals, i);
      }
    }
    if (tail_ext) {  // the last run goes on into the next tile's first ext_len positions
      for (int i = 0; i < ext_len; i += SEG_U) {
        V vals[SEG_U];
#pragma unroll
        for (int j = 0; j < SEG_U; ++j) {
          vals[j] = V{};
          const int pj = __builtin_amdgcn_readlane(nx_pos, (i + j) & 63);
          if (i + j < ext_len && active && (uint64_t)pj < (uint64_t)n) {
            const float* row = gb + (int64_t)pj * inner;
            if constexpr (VEC) vals[j] = ld_stream(reinterpret_cast<const f4*>(row) + u);
            else vals[j] = ld_stream(row + u);
          }
        }
#pragma unroll
        for (int j = 0; j < SEG_U; ++j)
          if (i + j < ext_len) acc = acc + vals[j];
      }
      if ((uint64_t)keyl < (uint64_t)len && active) {
        float* dst = grad + (o * len + keyl) * inner;
        if constexpr (VEC) st_stream<NTS>(acc, reinterpret_cast<f4*>(dst) + u);
        else st_stream<NTS>(acc, dst + u);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// VJP, fix-up of long keys. Work unit = (owner, 16-vector column chunk);
// blocks walk the units grid-stride, bounded by the owner count. In a unit,
// thread (s, c) adds column c of slots s, s+16, s+32, ... in order in float64
// (FXU slots in flight); the 16 slot sums are then combined in a fixed tree
// (wave shuffles over the 4 slot lanes a wave holds, then the 4 waves in
// order). Slots: tail slots of tiles ta..tb-1, head slot of tb.

// Measured on C4 (85 long keys; the spike key has 649 slots, so each of its
// 16 units walks 41 slots per thread): 15.8 us. 8 slots in flight (4 waves
// per SIMD instead of 3): 15.4 us; units of 4 columns x 64 slices (64 units
// for the spike key, 4x the units in all): 39 us, each unit paying its chain
// of dependent loads (owner, end tile, slots) in turn.
constexpr int FXU = 16;

template <bool VEC, bool NTS>
__global__ __launch_bounds__(256) void seg_fixup_k(int64_t outer, int64_t inner, int64_t len,
                                                   int64_t stiles, const int* __restrict__ owners,
                                                   const int* __restrict__ owner_count,
                                                   const int* __restrict__ end_tile, const double* __restrict__ part,
                                                   float* __restrict__ grad, int c16, int* guard,
                                                   const int* __restrict__ present, int64_t fb) {
  if ((int64_t)blockIdx.x >= fb) {  // the zero rows, behind the long keys' latency-bound sums
    zero_rows<VEC, NTS>((int64_t)blockIdx.x - fb, present, grad, outer, len, inner);
    return;
  }
  constexpr int NC = VEC ? 4 : 1;
  __shared__ double red[4][16][NC];
  const int64_t units = VEC ? inner / 4 : inner;
  const int sl = threadIdx.x >> 4, c = threadIdx.x & 15, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t nunits = (int64_t)(*owner_count) * c16;
  for (int64_t wk = blockIdx.x; wk < nunits; wk += fb) {
    const int64_t oi = wk / c16;
    const int chunk = (int)(wk - oi * c16);
    const int2 ow = reinterpret_cast<const int2*>(owners)[oi];
    const int64_t ta = ow.x;
    const int key = ow.y;
    const int64_t tb = ((uint64_t)key < (uint64_t)len) ? end_tile[key] : -1;
    if (tb <= ta + 1 || tb >= stiles) {  // inconsistent: reported, nothing written
      if (threadIdx.x == 0) atomicOr(guard, 2);
      continue;
    }
    const int64_t m = tb - ta + 1;  // partial slots
    const int64_t u = (int64_t)chunk * 16 + c;
    const bool active = u < units;
    for (int64_t o = 0; o < outer; ++o) {
      double a[NC];
#pragma unroll
      for (int q = 0; q < NC; ++q) a[q] = 0.0;
      for (int64_t j0 = sl; j0 < m; j0 += 16 * FXU) {
        double v[FXU][NC];
#pragma unroll
        for (int q = 0; q < FXU; ++q) {
          const int64_t j = min<int64_t>(j0 + 16 * q, m - 1);  // in range: loads issue together
          const int64_t slot = (j < m - 1) ? 2 * (ta + j) + 1 : 2 * tb;
          const double* src = part + ((slot * outer + o) * inner + u * NC);
#pragma unroll
          for (int c = 0; c < NC; ++c) v[q][c] = active ? src[c] : 0.0;
        }
#pragma unroll
        for (int q = 0; q < FXU; ++q)
          if (j0 + 16 * q < m)
#pragma unroll
            for (int c = 0; c < NC; ++c) a[c] += v[q][c];
      }
      // lanes c, c+16, c+32, c+48 of a wave hold 4 slot lanes of column c
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        a[q] += __shfl_xor(a[q], 16, 64);
        a[q] += __shfl_xor(a[q], 32, 64);
      }
      if (lane < 16)
#pragma unroll
        for (int q = 0; q < NC; ++q) red[w][c][q] = a[q];
      __syncthreads();
      if (threadIdx.x < 16 && active) {
        double r[NC];
#pragma unroll
        for (int q = 0; q < NC; ++q) r[q] = (red[0][c][q] + red[1][c][q]) + (red[2][c][q] + red[3][c][q]);
        float* dst = grad + (o * len + key) * inner;
        if constexpr (VEC) reinterpret_cast<f4*>(dst)[u] = f4{(float)r[0], (float)r[1], (float)r[2], (float)r[3]};
        else dst[u] = (float)r[0];
      }
      __syncthreads();
    }
  }
}

template <int IPT>
void sort_pass(hipStream_t s, int ps, int64_t n, int64_t len, int ntiles, const int64_t* idx, const int* ka,
               const int* va, int* kb, int* vb, int* tab, int* present, int* owner_count) {
  const int shift = 8 * ps;
  const unsigned nb = (unsigned)ntiles;
  int* gd = guard_flag();
  const bool self = ntiles <= SELF_SCAN_MAX;
  if (ps == 0) sort_hist_k<IPT, true><<<nb, SBS, 0, s>>>(idx, nullptr, n, len, shift, tab, present, owner_count, gd);
  else sort_hist_k<IPT, false><<<nb, SBS, 0, s>>>(nullptr, ka, n, len, shift, tab, nullptr, nullptr, gd);
  if (!self) sort_offsets_k<<<1, SBS, 0, s>>>(tab, ntiles);
  if (ps == 0) {
    if (self) sort_scatter_k<IPT, true, OFFS_SCAN_COUNTS><<<nb, SBS, 0, s>>>(idx, nullptr, nullptr, n, len, shift, ntiles, tab, kb, vb, present, gd);
    else sort_scatter_k<IPT, true, OFFS_TABLE><<<nb, SBS, 0, s>>>(idx, nullptr, nullptr, n, len, shift, ntiles, tab, kb, vb, present, gd);
  } else {
    if (self) sort_scatter_k<IPT, false, OFFS_SCAN_COUNTS><<<nb, SBS, 0, s>>>(nullptr, ka, va, n, len, shift, ntiles, tab, kb, vb, nullptr, gd);
    else sort_scatter_k<IPT, false, OFFS_TABLE><<<nb, SBS, 0, s>>>(nullptr, ka, va, n, len, shift, ntiles, tab, kb, vb, nullptr, gd);
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_sizes(const char* what, int64_t outer, int64_t len, int64_t inner, int64_t n) {
  if (outer < 0 || len < 0 || inner < 0 || n < 0) return fail(OXI_INVALID_ARGUMENT, "%s: negative size", what);
  if (len >= ((int64_t)1 << 31) - 1 || n >= ((int64_t)1 << 31) - 1)
    return fail(OXI_INVALID_ARGUMENT, "%s: index space exceeds the kernel limits", what);
  // element counts (outer * max(len, n) * inner) must stay well inside int64
  const int64_t rows = std::max(len, n);
  const int64_t limit = (int64_t)1 << 60;
  if (outer && rows && inner && (outer > limit / rows || outer * rows > limit / inner))
    return fail(OXI_INVALID_ARGUMENT, "%s: size (%lld, %lld, %lld) exceeds the kernel limits", what,
                (long long)outer, (long long)rows, (long long)inner);
  return OXI_OK;
}

// The id-dependent half of the VJP: the stable sort of (key, position)
// pairs and each key's presence flag. Built on any stream; `ready` is set
// when it was built on the side stream.
struct SortPlan {
  int64_t n = 0, len = 0;
  void* ws = nullptr;  // keys, pos, keys2, pos2, count table, present, owner count
  const int* ka = nullptr;  // sorted keys and their positions
  const int* va = nullptr;
  int* present = nullptr;
  int* owner_count = nullptr;  // zeroed by the sort; counts long-key owners in an apply
  hipEvent_t queued = nullptr;  // the library stream's position when the plan was queued
  hipEvent_t ready = nullptr;   // recorded on the side stream after the sort
  mutable int applies = 0;  // a second apply (retain_graph) re-zeroes the owner count
  bool recorded = false;    // `ready` holds the sort's completion
  // the library stream is already ordered after the sort (an apply waited
  // for `ready`, or saw it complete): freeing the plan needs no wait
  mutable bool ordered = false;
};

int build_plan(const int64_t* idx, int64_t n, int64_t len, hipStream_t s, SortPlan* p) {
  p->n = n;
  p->len = len;
  if (n == 0) return OXI_OK;
  if (len + 1 >= ((int64_t)1 << 31)) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: dim too large");
  // sort tiles: 2, 8 or 32 elements per thread, so that tables stay within
  // SELF_SCAN_MAX tiles up to 2M indices
  const int ipt = n <= 65536 ? 2 : (n <= 524288 ? 8 : 32);
  const int64_t rtiles = ceil_div(n, (int64_t)SBS * ipt);
  if (rtiles * 256 >= ((int64_t)1 << 31)) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: too many indices");
  int passes = 0;
  for (int64_t m = len; m > 0; m >>= 8) ++passes;  // keys are in [0, len]
  if (passes == 0) passes = 1;
  const size_t ints = 4 * (size_t)n + 256 * (size_t)rtiles + (size_t)len + 1;
  p->ws = ws_alloc(ints * sizeof(int));
  if (!p->ws) return fail_alloc("index_select_bwd: sort workspace");
  int* keys = static_cast<int*>(p->ws);
  int* pos = keys + n;
  int* keys2 = pos + n;
  int* pos2 = keys2 + n;
  int* tab = pos2 + n;
  p->present = tab + 256 * rtiles;
  p->owner_count = p->present + len;
  // pass p reads (ka, va) and writes (kb, vb); pass 0 reads the ids
  const int* ka = nullptr;
  const int* va = nullptr;
  int* bufk[2] = {keys, keys2};
  int* bufv[2] = {pos, pos2};
  for (int ps = 0; ps < passes; ++ps) {
    int* kb = bufk[ps & 1];
    int* vb = bufv[ps & 1];
    if (ipt == 2) sort_pass<2>(s, ps, n, len, (int)rtiles, idx, ka, va, kb, vb, tab, p->present, p->owner_count);
    else if (ipt == 8) sort_pass<8>(s, ps, n, len, (int)rtiles, idx, ka, va, kb, vb, tab, p->present, p->owner_count);
    else sort_pass<32>(s, ps, n, len, (int)rtiles, idx, ka, va, kb, vb, tab, p->present, p->owner_count);
    ka = kb;
    va = vb;
  }
  p->ka = ka;
  p->va = va;
  return check_launch("index_select_bwd/sort");
}

// The gradient half, on the library stream: segment sums of g's rows in the
// plan's order, zero rows for absent keys, the fix-up of long keys.
int apply_plan(const SortPlan& p, const float* g, int64_t outer, int64_t inner, float* grad) {
  const int64_t n = p.n, len = p.len;
  const int64_t total_out = outer * len * inner;
  if (total_out == 0) return OXI_OK;
  if (!grad) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: NULL output pointer");
  if (n == 0) return oxi_fill(grad, total_out, 0.f);
  if (!g) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: NULL tensor pointer");
  hipStream_t s = stream();
  // segment tiles: as long as possible (fewer cut runs) while still giving
  // every CU several waves
  const bool vec = inner % 4 == 0 && al16(g) && al16(grad);
  const int64_t units = vec ? inner / 4 : inner;
  const int64_t chunks = ceil_div(units, 64);
  const int64_t c16 = ceil_div(units, 16);
  if (c16 >= (1 << 24)) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: rows too wide");
#ifndef OXI_SEG_ST
#define OXI_SEG_ST 64
#endif
  int st = OXI_SEG_ST;
  while (st > 16 && ceil_div(n, st) * chunks < 8 * (int64_t)cu_count()) st >>= 1;
  const int64_t stiles = ceil_div(n, st);
  // end tile per key and the owner list of long keys; partial rows
  Workspace wsi(((size_t)len + 1 + 2 * (size_t)stiles) * sizeof(int));
  Workspace wsp((size_t)2 * (size_t)stiles * (size_t)outer * (size_t)inner * sizeof(double));
  if (!wsi.p || !wsp.p) return fail_alloc("index_select_bwd: apply workspace");
  int* end_tile = wsi.as<int>();
  int* owners = end_tile + len + (len & 1);  // (tile, key) pairs, 8-byte aligned
  const int* ka = p.ka;
  const int* va = p.va;
  int* present = p.present;
  int* owner_count = p.owner_count;
  if (p.applies++ > 0) {
    if (int rc = oxi_fill(reinterpret_cast<float*>(owner_count), 1, 0.0f)) return rc;  // 0.0f is all-zero bits
  }
  double* part = wsp.as<double>();
  const int64_t seg_blocks = ceil_div(stiles * chunks, 4);
  // the rows of g stream through the cache while dW is written: decide on
  // the launch's whole traffic, not on dW alone
  const bool nts = nt_stores((total_out + outer * n * inner) * 4);
  // From DB_MIN_IDS ids on the zero rows are written by the fix-up launch,
  // behind its latency-bound sums: C4's VJP 160.8-161.0 us against
  // 163.2-163.6 with them in the segment launch. Below, the segment launch
  // writes them, where they hide behind its gathers: there C5's VJP took
  // 46.6-46.9 us with them in the fix-up against 38.3-38.7.
  const bool db = n >= DB_MIN_IDS;
  const int64_t zblocks = ceil_div(len, ZR);
  const int64_t fb = std::max<int64_t>(1, std::min<int64_t>(stiles * c16, 4 * (int64_t)cu_count()));
  const int64_t blocks = seg_blocks + (db ? 0 : zblocks);
  const int64_t fblocks = fb + (db ? zblocks : 0);
  if (blocks >= ((int64_t)1 << 31) || fblocks >= ((int64_t)1 << 31))
    return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: too many rows");
  const dim3 sg((unsigned)blocks), st256(256);
#define OXI_SEG(VEC, NTS, DB)                                                                                     \
  seg_wave_k<VEC, NTS, DB><<<sg, st256, 0, s>>>(g, outer, n, inner, len, ka, va, grad, part, present, owners,     \
                                                owner_count, end_tile, st, stiles, (int)chunks, seg_blocks)
  if (vec && nts) {
    if (db) OXI_SEG(true, true, true);
    else OXI_SEG(true, true, false);
  } else if (vec) {
    if (db) OXI_SEG(true, false, true);
    else OXI_SEG(true, false, false);
  } else {
    OXI_SEG(false, false, false);
  }
#undef OXI_SEG
  if (int rc = check_launch("index_select_bwd/segments")) return rc;
#define OXI_FIX(VEC, NTS)                                                                                        \
  seg_fixup_k<VEC, NTS><<<dim3((unsigned)fblocks), st256, 0, s>>>(outer, inner, len, stiles, owners,              \
                                                                 owner_count, end_tile, part, grad, (int)c16,    \
                                                                 guard_flag(), present, fb)
  if (vec && nts) OXI_FIX(true, true);
  else if (vec) OXI_FIX(true, false);
  else OXI_FIX(false, false);
#undef OXI_FIX
  return check_launch("index_select_bwd/fixup");
}

}  // namespace
}  // namespace oxi

using namespace oxi;

extern "C" {

int oxi_index_select(const float* src, int64_t outer, int64_t len, int64_t inner, const int64_t* idx, int64_t n,
                     float* out) {
  if (int rc = check_sizes("index_select", outer, len, inner, n)) return rc;
  const int64_t rows = outer * n;
  if (rows == 0 || inner == 0) return OXI_OK;
  if (len == 0) return fail(OXI_OUT_OF_BOUNDS, "index_select: indices into an empty dim");
  if (!src || !idx || !out) return fail(OXI_INVALID_ARGUMENT, "index_select: NULL tensor pointer");
  OXI_CHECK_INIT();
  hipStream_t s = stream();
  if (inner >= 64) {
    const bool vec = inner % 4 == 0 && al16(src) && al16(out);
    const int64_t blocks = ceil_div(rows, GRPB);
    if (blocks >= ((int64_t)1 << 31)) return fail(OXI_INVALID_ARGUMENT, "index_select: too many rows");
    // threads per block: the row's vector count rounded up to whole waves
    // (192 for a 768-float row), at most BS
    const int64_t units = vec ? inner / 4 : inner;
    const unsigned bt = (unsigned)std::min<int64_t>(BS, ceil_div(units, 64) * 64);
    const bool nts = nt_stores(rows * inner * 4);
    const dim3 gb((unsigned)blocks), tb(bt);
    if (vec && nts) gather_k<true, true><<<gb, tb, 0, s>>>(src, outer, len, inner, idx, n, out, guard_flag());
    else if (vec) gather_k<true, false><<<gb, tb, 0, s>>>(src, outer, len, inner, idx, n, out, guard_flag());
    else gather_k<false, false><<<gb, tb, 0, s>>>(src, outer, len, inner, idx, n, out, guard_flag());
  } else {
    const int64_t blocks = std::min<int64_t>(ceil_div(rows * inner, BS), (int64_t)cu_count() * 32);
    gather_elem_k<<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(src, outer, len, inner, idx, n, out, guard_flag());
  }
  return check_launch("index_select");
}

int oxi_batch_gather(const oxi_batch_column* cols, int ncols, int64_t len, const int64_t* idx, int64_t n) {
  if (ncols < 0 || n < 0 || len < 0) return fail(OXI_INVALID_ARGUMENT, "batch_gather: negative size");
  if (ncols > 0 && !cols) return fail(OXI_INVALID_ARGUMENT, "batch_gather: NULL column list");
  int64_t out_bytes = 0;
  for (int c = 0; c < ncols; ++c) {
    const oxi_batch_column& col = cols[c];
    if (col.inner < 0) return fail(OXI_INVALID_ARGUMENT, "batch_gather: column %d has a negative row size", c);
    if (int rc = check_sizes("batch_gather", 1, len, col.inner, n)) return rc;
    if (n > 0 && col.inner > 0 && (!col.src || !col.dst))
      return fail(OXI_INVALID_ARGUMENT, "batch_gather: column %d has a NULL pointer", c);
    out_bytes += n * col.inner * 4;
  }
  if (out_bytes == 0) return OXI_OK;
  if (len == 0) return fail(OXI_OUT_OF_BOUNDS, "batch_gather: indices into an empty dataset");
  if (!idx) return fail(OXI_INVALID_ARGUMENT, "batch_gather: NULL indices");
  OXI_CHECK_INIT();
  hipStream_t s = stream();
  const bool nts = nt_stores(out_bytes);
  BatchArgs a{};
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (a.count == 0) return OXI_OK;
    if (nts) batch_gather_k<true><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(a, len, idx, n, guard_flag());
    else batch_gather_k<false><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(a, len, idx, n, guard_flag());
    a = BatchArgs{};
    blocks = 0;
    return check_launch("batch_gather");
  };
  for (int c = 0; c < ncols; ++c) {
    const oxi_batch_column& col = cols[c];
    if (col.inner == 0) continue;
    int mode = BG_ELEMS;
    int64_t nb = ceil_div(n * col.inner, BS);
    if (col.inner >= 64) {
      mode = (col.inner % 4 == 0 && al16(col.src) && al16(col.dst)) ? BG_ROWS4 : BG_ROWS;
      nb = ceil_div(n, GRPB);
    }
    if (a.count == BG_MAX || blocks + nb >= ((int64_t)1 << 31)) {
      if (int rc = flush()) return rc;
    }
    if (nb >= ((int64_t)1 << 31)) return fail(OXI_INVALID_ARGUMENT, "batch_gather: column %d is too large", c);
    a.src[a.count] = col.src;
    a.dst[a.count] = col.dst;
    a.inner[a.count] = col.inner;
    a.mode[a.count] = mode;
    blocks += nb;
    a.block_end[a.count] = (unsigned)blocks;
    ++a.count;
  }
  return flush();
}

int oxi_index_select_bwd_plan(const int64_t* idx, int64_t n, int64_t len, void** plan) {
  if (!plan) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd_plan: NULL plan");
  *plan = nullptr;
  if (int rc = check_sizes("index_select_bwd_plan", 1, len, 1, n)) return rc;
  if (n > 0 && !idx) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd_plan: NULL ids");
  OXI_CHECK_INIT();
  SortPlan* p = new SortPlan();
  // the side stream starts after everything already queued on the library
  // stream: the ids' upload, and every earlier user of the plan's memory
  p->queued = take_event();
  p->ready = take_event();
  if (!p->queued || !p->ready) {
    (void)oxi_index_select_bwd_plan_free(p);
    return fail(OXI_OTHER, "index_select_bwd_plan: no event available");
  }
  hipError_t e = hipEventRecord(p->queued, stream());
  if (e == hipSuccess) e = hipStreamWaitEvent(side_stream(), p->queued, 0);
  if (e != hipSuccess) {
    (void)oxi_index_select_bwd_plan_free(p);
    return fail_hip(e, "index_select_bwd_plan: ordering the side stream");
  }
  int rc = build_plan(idx, n, len, side_stream(), p);
  if (rc == OXI_OK) {
    e = hipEventRecord(p->ready, side_stream());
    if (e != hipSuccess) rc = fail_hip(e, "index_select_bwd_plan: recording the plan");
    else p->recorded = true;
  }
  if (rc != OXI_OK) {
    (void)oxi_index_select_bwd_plan_free(p);
    return rc;
  }
  *plan = p;
  return OXI_OK;
}

int oxi_index_select_bwd_apply(const void* plan, const float* g, int64_t outer, int64_t inner, float* grad) {
  if (!plan) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd_apply: NULL plan");
  const SortPlan& p = *static_cast<const SortPlan*>(plan);
  if (int rc = check_sizes("index_select_bwd_apply", outer, p.len, inner, p.n)) return rc;
  OXI_CHECK_INIT();
  // a cross-stream wait costs a barrier packet on the library stream: skip it
  // when the sort has already finished
  if (p.recorded && !p.ordered) {
    if (hipEventQuery(p.ready) != hipSuccess) {
      hipError_t e = hipStreamWaitEvent(stream(), p.ready, 0);
      if (e != hipSuccess) return fail_hip(e, "index_select_bwd_apply: waiting for the plan");
    }
    p.ordered = true;
  }
  return apply_plan(p, g, outer, inner, grad);
}

int oxi_index_select_bwd_plan_free(void* plan) {
  if (!plan) return OXI_OK;
  SortPlan* p = static_cast<SortPlan*>(plan);
  // the library stream passes the plan's sort before its memory can be
  // reused, and before its events go back to the pool (already so after an
  // apply; the next plan's sort waits for the library stream's work queued
  // before it, this plan's apply included, so it cannot reuse the memory early)
  if (p->recorded && !p->ordered && ensure_init() && hipEventQuery(p->ready) != hipSuccess)
    (void)hipStreamWaitEvent(stream(), p->ready, 0);
  // a plan whose build failed part-way has no completion event: kernels it
  // queued may still run on the side stream, so drain it (error path only)
  if (!p->recorded && p->ws) (void)hipStreamSynchronize(side_stream());
  if (p->ws) ws_free(p->ws);
  give_event(p->queued);
  give_event(p->ready);
  delete p;
  return OXI_OK;
}

int oxi_index_select_bwd(const float* g, int64_t outer, int64_t len, int64_t inner, const int64_t* idx, int64_t n,
                         float* grad) {
  if (int rc = check_sizes("index_select_bwd", outer, len, inner, n)) return rc;
  const int64_t total_out = outer * len * inner;
  if (total_out == 0) return OXI_OK;
  if (!grad) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: NULL output pointer");
  OXI_CHECK_INIT();
  if (n == 0) return oxi_fill(grad, total_out, 0.f);
  if (!g || !idx) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: NULL tensor pointer");
  // the whole VJP on the library stream
  SortPlan p;
  int rc = build_plan(idx, n, len, stream(), &p);
  if (rc == OXI_OK) rc = apply_plan(p, g, outer, inner, grad);
  if (p.ws) ws_free(p.ws);
  return rc;
}

int oxi_embedding_fwd(const float* W, const int64_t* ids, int64_t n, int64_t V, int64_t D, float* out) {
  return oxi_index_select(W, 1, V, D, ids, n, out);
}

int oxi_embedding_bwd(const float* g, const int64_t* ids, int64_t n, int64_t V, int64_t D, float* dW) {
  return oxi_index_select_bwd(g, 1, V, D, ids, n, dW);
}

}  // extern "C"
