// index_select gather and its deterministic duplicate-accumulating VJP
// (F.embedding: python/oxitorch/nn/functional.py:245-247; Tensor::index_select:
// crates/oxi-tensor/src/lib.rs:665-703; scatter_index_select:
// crates/oxi-autograd/src/ops.rs:741-769).
//
// Gather: out[o, k, :] = src[o, idx[k], :]. Each block copies 8 rows per step
// with float4 accesses (8 independent loads in flight per thread).
//
// VJP without float atomics:
//   1. keys: ids wrapped to [0, len); out-of-range ids get the sentinel key
//      `len` (never summed) and raise the guard flag;
//   2. stable LSD radix sort of positions by key, 8-bit digits: per-tile digit
//      histograms (LDS integer atomics), a one-block LDS scan, and a scatter
//      whose ranks come from wave ballots plus per-wave counts, so equal keys
//      keep position order;
//   3. tile-segmented reduction over the sorted positions: each block owns
//      ST positions and sums every run of equal keys in position order in
//      f32 -- the reference's own order, so a run inside one tile gives a
//      bit-identical row -- writing complete runs straight to the output and
//      runs cut by a tile edge to per-tile partial slots;
//   4. fix-up: a key spanning several tiles adds its partial slots in tile
//      order in float64 (16 waves split the slots, so a key that owns a third
//      of all positions is not serialised on one wave);
//   5. rows of absent keys are zero-filled.
// Every block does the same amount of work whatever the id distribution.
#include <algorithm>
#include <type_traits>

#include "internal.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;
constexpr int GRPB = 8;       // rows per gather step

__device__ __forceinline__ int64_t wrap_id(int64_t id, int64_t len, bool& ok) {
  if (id < 0) id += len;
  ok = (id >= 0 && id < len);
  return ok ? id : 0;
}

// ---------------------------------------------------------------------------
// Gather.

template <bool VEC>
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
  for (int64_t c = threadIdx.x; c < units; c += BS) {
    if constexpr (VEC) {
      f4 v[GRPB];
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        v[r] = (r0 + r < rows && okr[r]) ? reinterpret_cast<const f4*>(src + srow[r])[c] : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < GRPB; ++r)
        if (r0 + r < rows) __builtin_nontemporal_store(v[r], reinterpret_cast<f4*>(out + (r0 + r) * inner) + c);
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
// VJP step 1: keys. Out-of-range ids become the sentinel key `len` (never
// summed) and raise the guard flag.

__global__ __launch_bounds__(BS) void keys_k(const int64_t* __restrict__ idx, int64_t n, int64_t len,
                                             int* __restrict__ keys, int* __restrict__ pos, int* __restrict__ guard) {
  for (int64_t p = (int64_t)blockIdx.x * BS + threadIdx.x; p < n; p += (int64_t)gridDim.x * BS) {
    bool ok;
    const int64_t id = wrap_id(idx[p], len, ok);
    if (!ok) atomicOr(guard, 1);
    keys[p] = ok ? (int)id : (int)len;
    pos[p] = (int)p;
  }
}

// ---------------------------------------------------------------------------
// VJP step 2: stable LSD radix sort of (key, position), 8-bit digits.
// A block owns a tile of RT consecutive elements (256 threads x 8 items).

constexpr int RT = 2048;

// hist[d * ntiles + tile] = number of elements of `tile` whose digit is d.
__global__ __launch_bounds__(BS) void radix_hist_k(const int* __restrict__ keys, int64_t n, int shift, int ntiles,
                                                   int* __restrict__ hist) {
  __shared__ int cnt[256];
  const int t = threadIdx.x;
  cnt[t] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * RT;
#pragma unroll
  for (int i = 0; i < RT / BS; ++i) {
    const int64_t p = base + i * BS + t;
    if (p < n) atomicAdd(&cnt[(keys[p] >> shift) & 255], 1);  // LDS integer atomics: exact counts
  }
  __syncthreads();
  hist[(int64_t)t * ntiles + blockIdx.x] = cnt[t];
}

// In-place exclusive scan of m ints by one block of 1024 threads, in LDS
// chunks of 8192 (coalesced loads/stores; padded LDS rows avoid bank conflicts).
constexpr int SCAN_T = 1024;
constexpr int SCAN_CHUNK = 8 * SCAN_T;

__device__ __forceinline__ int pad_idx(int e) { return e + (e >> 3); }

__global__ __launch_bounds__(SCAN_T) void scan_k(int* a, int64_t m) {
  __shared__ int buf[SCAN_CHUNK + SCAN_CHUNK / 8];
  __shared__ int wsum[SCAN_T / 64];
  __shared__ int carry_s;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (t == 0) carry_s = 0;
  for (int64_t base = 0; base < m; base += SCAN_CHUNK) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = i * SCAN_T + t;
      buf[pad_idx(e)] = (base + e < m) ? a[base + e] : 0;
    }
    __syncthreads();
    int v[8], sum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      v[k] = buf[pad_idx(t * 8 + k)];
      sum += v[k];
    }
    // inclusive wave scan of per-thread sums
    int inc = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(inc, d, 64);
      if (lane >= d) inc += o;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    if (t == 0) {
      int run = 0;
      for (int q = 0; q < SCAN_T / 64; ++q) {
        const int x = wsum[q];
        wsum[q] = run;
        run += x;
      }
    }
    __syncthreads();
    int run = carry_s + wsum[w] + inc - sum;  // exclusive prefix of this thread
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      buf[pad_idx(t * 8 + k)] = run;
      run += v[k];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = i * SCAN_T + t;
      if (base + e < m) a[base + e] = buf[pad_idx(e)];
    }
    if (t == SCAN_T - 1) carry_s = run;
    __syncthreads();
  }
}

// Stable scatter: element r*256 + t of a tile goes after every earlier element
// with the same digit. Ranks within a wave come from ballots; counts of the
// earlier waves of the same round from LDS.
__global__ __launch_bounds__(BS) void radix_scatter_k(const int* __restrict__ keys, const int* __restrict__ vals,
                                                      int64_t n, int shift, int ntiles, const int* __restrict__ offs,
                                                      int* __restrict__ keys_out, int* __restrict__ vals_out) {
  __shared__ int base[256];
  __shared__ int cnt[BS / 64][256];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  base[t] = offs[(int64_t)t * ntiles + blockIdx.x];
  const unsigned long long lt = (1ull << lane) - 1ull;
  const int64_t tile0 = (int64_t)blockIdx.x * RT;
  for (int r = 0; r < RT / BS; ++r) {
    const int64_t p = tile0 + r * BS + t;
    const bool valid = p < n;
    const int k = valid ? keys[p] : 0;
    const int v = valid ? vals[p] : 0;
    const int d = (k >> shift) & 255;
    unsigned long long peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1;
      const unsigned long long m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
#pragma unroll
    for (int q = 0; q < BS / 64; ++q) cnt[q][t] = 0;
    __syncthreads();
    if (valid && (__ffsll((long long)peers) - 1) == lane) cnt[w][d] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pre = base[d];
      for (int q = 0; q < w; ++q) pre += cnt[q][d];
      const int dst = pre + __popcll(peers & lt);
      keys_out[dst] = k;
      vals_out[dst] = v;
    }
    __syncthreads();
    int add = 0;
#pragma unroll
    for (int q = 0; q < BS / 64; ++q) add += cnt[q][t];
    base[t] += add;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// VJP step 3: tile-segmented reduction. A block owns ST consecutive sorted
// positions; every run of equal keys inside the tile is summed in position
// order. A run that neither continues from the previous tile nor into the
// next one is complete: its sum is the output row. Otherwise the sum goes to
// a partial slot of the tile: slot 2*tile+1 for the run that continues into
// the next tile, slot 2*tile for the first run continuing from the previous.

constexpr int ST = 128;
constexpr int SU = 8;  // rows in flight per thread

template <bool VEC>
__global__ __launch_bounds__(BS) void seg_tile_k(const float* __restrict__ g, int64_t outer, int64_t n, int64_t inner,
                                                 int64_t len, const int* __restrict__ skeys,
                                                 const int* __restrict__ perm, float* __restrict__ grad,
                                                 float* __restrict__ part, int* __restrict__ present) {
  __shared__ int key_s[ST + 2];  // [0] = key before the tile (-1 if none), [cnt+1] = key after
  __shared__ int pos_s[ST];
  const int t = threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.x * ST;
  const int cnt = (int)min<int64_t>(ST, n - p0);
  if (t < cnt) {
    key_s[t + 1] = skeys[p0 + t];
    pos_s[t] = perm[p0 + t];
  }
  if (t == 0) key_s[0] = p0 > 0 ? skeys[p0 - 1] : -1;
  if (t == 1) key_s[cnt + 1] = p0 + cnt < n ? skeys[p0 + cnt] : -1;
  __syncthreads();
  if (t == 0) {  // mark present keys (plain stores of 1: order-free)
    for (int i = 0; i < cnt; ++i)
      if (key_s[i + 1] != key_s[i] && key_s[i + 1] < len) present[key_s[i + 1]] = 1;
  }
  const int64_t units = VEC ? inner / 4 : inner;
  const int64_t slot_head = 2 * (int64_t)blockIdx.x, slot_tail = slot_head + 1;
  for (int64_t o = 0; o < outer; ++o) {
    const float* gb = g + o * n * inner;
    for (int64_t u = t; u < units; u += BS) {
      using V = typename std::conditional<VEC, f4, float>::type;
      V acc = V{};
      int start = 0;
      for (int i = 0; i < cnt; i += SU) {
        V vals[SU];
#pragma unroll
        for (int j = 0; j < SU; ++j) {
          if (i + j < cnt) {
            const float* row = gb + (int64_t)pos_s[i + j] * inner;
            if constexpr (VEC) vals[j] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(row) + u);
            else vals[j] = row[u];
          }
        }
#pragma unroll
        for (int j = 0; j < SU; ++j) {
          const int q = i + j;
          if (q >= cnt) break;
          acc = acc + vals[j];
          const int key = key_s[q + 1];
          if (key_s[q + 2] != key || q == cnt - 1) {  // run [start, q] ends here
            if (key < len) {
              const bool head_inc = (start == 0) && (key_s[0] == key);
              const bool tail_inc = (q == cnt - 1) && (key_s[cnt + 1] == key);
              float* dst;
              if (!head_inc && !tail_inc) dst = grad + (o * len + key) * inner;
              else dst = part + ((tail_inc ? slot_tail : slot_head) * outer + o) * inner;
              if constexpr (VEC) reinterpret_cast<f4*>(dst)[u] = acc;
              else dst[u] = acc;
            }
            acc = V{};
            start = q + 1;
          }
        }
      }
    }
  }
}

// VJP step 4: a segment spanning tiles ta..tb is owned by ta; its partials
// are the tail slots of ta..tb-1 and the head slot of tb, added in tile order
// in float64. Block: 16 waves x 64 lanes, blockIdx.y = column chunk.
constexpr int FX_W = 16;

template <bool VEC>
__global__ __launch_bounds__(64 * FX_W) void seg_fixup_k(int64_t outer, int64_t n, int64_t inner, int64_t len,
                                                         const int* __restrict__ skeys,
                                                         const float* __restrict__ part, float* __restrict__ grad) {
  const int64_t tile = blockIdx.x;
  const int64_t p0 = tile * ST;
  const int64_t p1 = min<int64_t>(p0 + ST, n);
  if (p1 >= n) return;  // nothing continues past the last tile
  const int klast = skeys[p1 - 1];
  if (skeys[p1] != klast || klast >= len) return;                       // tail run ends in this tile
  if (p0 > 0 && skeys[p0] == klast && skeys[p0 - 1] == klast) return;  // run started in an earlier tile
  // last position of the segment: upper_bound over [p1, n) - 1
  int64_t lo = p1, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (skeys[mid] <= klast) lo = mid + 1;
    else hi = mid;
  }
  const int64_t tb = (lo - 1) / ST;
  const int64_t m = tb - tile + 1;  // partial slots
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t u = (int64_t)blockIdx.y * 64 + lane;
  const int64_t units = VEC ? inner / 4 : inner;
  __shared__ double red[FX_W][64][VEC ? 4 : 1];
  for (int64_t o = 0; o < outer; ++o) {
    double a[4] = {0.0, 0.0, 0.0, 0.0};
    if (u < units) {
      for (int64_t j = wv; j < m; j += FX_W) {
        const int64_t slot = (j < m - 1) ? 2 * (tile + j) + 1 : 2 * tb;
        const float* src = part + (slot * outer + o) * inner;
        if constexpr (VEC) {
          const f4 v = reinterpret_cast<const f4*>(src)[u];
          a[0] += v.x; a[1] += v.y; a[2] += v.z; a[3] += v.w;
        } else {
          a[0] += src[u];
        }
      }
    }
#pragma unroll
    for (int c = 0; c < (VEC ? 4 : 1); ++c) red[wv][lane][c] = a[c];
    __syncthreads();
    if (wv == 0 && u < units) {
      double r[4] = {0.0, 0.0, 0.0, 0.0};
      for (int q = 0; q < FX_W; ++q)
#pragma unroll
        for (int c = 0; c < (VEC ? 4 : 1); ++c) r[c] += red[q][lane][c];
      float* dst = grad + (o * len + klast) * inner;
      if constexpr (VEC) reinterpret_cast<f4*>(dst)[u] = f4{(float)r[0], (float)r[1], (float)r[2], (float)r[3]};
      else dst[u] = (float)r[0];
    }
    __syncthreads();
  }
}

// VJP step 5: rows of keys that never occur are zero.
constexpr int ZR = 4;  // rows per block

template <bool VEC>
__global__ __launch_bounds__(BS) void zero_absent_k(int64_t outer, int64_t len, int64_t inner,
                                                    const int* __restrict__ present, float* __restrict__ grad) {
  const int64_t units = VEC ? inner / 4 : inner;
  for (int r = 0; r < ZR; ++r) {
    const int64_t v = (int64_t)blockIdx.x * ZR + r;
    if (v >= len || present[v]) continue;
    for (int64_t o = 0; o < outer; ++o) {
      float* dst = grad + (o * len + v) * inner;
      for (int64_t u = threadIdx.x; u < units; u += BS) {
        if constexpr (VEC) __builtin_nontemporal_store(f4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<f4*>(dst) + u);
        else dst[u] = 0.f;
      }
    }
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_sizes(const char* what, int64_t outer, int64_t len, int64_t inner, int64_t n) {
  if (outer < 0 || len < 0 || inner < 0 || n < 0) return fail(OXI_INVALID_ARGUMENT, "%s: negative size", what);
  if (len >= ((int64_t)1 << 31) - 1 || n >= ((int64_t)1 << 31) - 1)
    return fail(OXI_INVALID_ARGUMENT, "%s: index space exceeds the kernel limits", what);
  return OXI_OK;
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
    if (vec) gather_k<true><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(src, outer, len, inner, idx, n, out, guard_flag());
    else gather_k<false><<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(src, outer, len, inner, idx, n, out, guard_flag());
  } else {
    const int64_t blocks = std::min<int64_t>(ceil_div(rows * inner, BS), (int64_t)cu_count() * 32);
    gather_elem_k<<<dim3((unsigned)blocks), dim3(BS), 0, s>>>(src, outer, len, inner, idx, n, out, guard_flag());
  }
  return check_launch("index_select");
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
  hipStream_t s = stream();
  const int64_t rtiles = ceil_div(n, RT);
  const int64_t stiles = ceil_div(n, ST);
  if (rtiles * 256 > ((int64_t)1 << 31) || len + 1 >= ((int64_t)1 << 31))
    return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: too many indices");
  int passes = 0;
  for (int64_t m = len; m > 0; m >>= 8) ++passes;  // keys are in [0, len]
  if (passes == 0) passes = 1;
  // workspace (ints): keys, pos, keys2, pos2 (n each), hist (256 * rtiles), present (len)
  const size_t ints = 4 * (size_t)n + 256 * (size_t)rtiles + (size_t)len;
  Workspace wsi(ints * sizeof(int));
  Workspace wsp((size_t)2 * (size_t)stiles * (size_t)outer * (size_t)inner * sizeof(float));
  if (!wsi.p || !wsp.p) return OXI_OTHER;
  int* keys = wsi.as<int>();
  int* pos = keys + n;
  int* keys2 = pos + n;
  int* pos2 = keys2 + n;
  int* hist = pos2 + n;
  int* present = hist + 256 * rtiles;
  if (int rc = oxi_fill(reinterpret_cast<float*>(present), len, 0.f)) return rc;  // +0.0f is all-zero bits
  const unsigned gb = (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, BS), (int64_t)cu_count() * 8));
  keys_k<<<gb, BS, 0, s>>>(idx, n, len, keys, pos, guard_flag());
  if (int rc = check_launch("index_select_bwd/keys")) return rc;
  int *ka = keys, *va = pos, *kb = keys2, *vb = pos2;
  for (int ps = 0; ps < passes; ++ps) {
    const int shift = 8 * ps;
    radix_hist_k<<<(unsigned)rtiles, BS, 0, s>>>(ka, n, shift, (int)rtiles, hist);
    scan_k<<<1, SCAN_T, 0, s>>>(hist, 256 * rtiles);
    radix_scatter_k<<<(unsigned)rtiles, BS, 0, s>>>(ka, va, n, shift, (int)rtiles, hist, kb, vb);
    std::swap(ka, kb);
    std::swap(va, vb);
  }
  if (int rc = check_launch("index_select_bwd/sort")) return rc;
  const bool vec = inner % 4 == 0 && al16(g) && al16(grad);
  float* part = wsp.as<float>();
  if (vec) seg_tile_k<true><<<(unsigned)stiles, BS, 0, s>>>(g, outer, n, inner, len, ka, va, grad, part, present);
  else seg_tile_k<false><<<(unsigned)stiles, BS, 0, s>>>(g, outer, n, inner, len, ka, va, grad, part, present);
  if (int rc = check_launch("index_select_bwd/segments")) return rc;
  const int64_t units = vec ? inner / 4 : inner;
  const dim3 fg((unsigned)stiles, (unsigned)ceil_div(units, 64));
  if (fg.y > 65535) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: rows too wide");
  if (vec) seg_fixup_k<true><<<fg, 64 * FX_W, 0, s>>>(outer, n, inner, len, ka, part, grad);
  else seg_fixup_k<false><<<fg, 64 * FX_W, 0, s>>>(outer, n, inner, len, ka, part, grad);
  if (int rc = check_launch("index_select_bwd/fixup")) return rc;
  const unsigned gz = (unsigned)ceil_div(len, ZR);
  if (vec) zero_absent_k<true><<<gz, BS, 0, s>>>(outer, len, inner, present, grad);
  else zero_absent_k<false><<<gz, BS, 0, s>>>(outer, len, inner, present, grad);
  return check_launch("index_select_bwd/zero");
}

int oxi_embedding_fwd(const float* W, const int64_t* ids, int64_t n, int64_t V, int64_t D, float* out) {
  return oxi_index_select(W, 1, V, D, ids, n, out);
}

int oxi_embedding_bwd(const float* g, const int64_t* ids, int64_t n, int64_t V, int64_t D, float* dW) {
  return oxi_index_select_bwd(g, 1, V, D, ids, n, dW);
}

}  // extern "C"
