// index_select gather and its deterministic duplicate-accumulating VJP
// (F.embedding: python/oxitorch/nn/functional.py:245-247; Tensor::index_select:
// crates/oxi-tensor/src/lib.rs:665-703; scatter_index_select:
// crates/oxi-autograd/src/ops.rs:741-769).
//
// Gather: out[o, k, :] = src[o, idx[k], :]. Each block copies 8 rows per step
// with float4 accesses (8 independent loads in flight per thread).
//
// VJP without float atomics:
//   1. keys: ids wrapped to [0, len) (out-of-range -> sentinel key `len`,
//      guard flag raised), per-key counts via integer atomics (order-free);
//   2. one-block scans: key offsets, chunks per key (ceil(count / CH)), and
//      partial-slot offsets for keys that span several chunks;
//   3. stable LSD radix sort of positions by key, 8-bit digits: per-tile digit
//      histograms, a scan, then a wave-synchronous scatter whose ranks come
//      from ballots, so equal keys keep position order;
//   4. chunk sums: each chunk of <= CH positions of one key is summed in
//      position order in f32 (the reference's own order, so keys with
//      <= CH occurrences are bit-identical to it) and written straight to the
//      output row, or to a partial slot when the key spans several chunks;
//   5. finalize: rows of absent keys are zero-filled and multi-chunk keys add
//      their partial rows in chunk order in float64.
// Heavy keys (a clipped-Zipf id can own a third of all positions) are split
// across many chunks, so no single block serialises on them.
#include <algorithm>

#include "internal.h"
#include "rowtile.h"

namespace oxi {
namespace {

constexpr int BS = 256;
constexpr int CH = 64;        // positions per chunk
constexpr int TILE = 1024;    // positions per radix tile (one wave per tile)
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
// VJP step 1: keys + per-key counts.

__global__ __launch_bounds__(BS) void keys_k(const int64_t* __restrict__ idx, int64_t n, int64_t len,
                                             int* __restrict__ keys, int* __restrict__ pos,
                                             int* __restrict__ counts, int* __restrict__ guard) {
  for (int64_t p = (int64_t)blockIdx.x * BS + threadIdx.x; p < n; p += (int64_t)gridDim.x * BS) {
    bool ok;
    const int64_t id = wrap_id(idx[p], len, ok);
    const int key = ok ? (int)id : (int)len;
    if (!ok) atomicOr(guard, 1);
    keys[p] = key;
    pos[p] = (int)p;
    atomicAdd(&counts[key], 1);
  }
}

// Exclusive scan of m ints (one block of 1024 threads); `total` gets the sum.
// `in` may equal `out`: each thread reads and rewrites only its own range.
__global__ __launch_bounds__(1024) void scan_k(const int* in, int* out, int64_t m, int* total) {
  __shared__ int s[1024];
  const int t = threadIdx.x;
  const int64_t per = (m + 1023) / 1024;
  const int64_t b = t * per, e = min(b + per, m);
  int sum = 0;
  for (int64_t i = b; i < e; ++i) sum += in[i];
  s[t] = sum;
  __syncthreads();
  for (int w = 1; w < 1024; w <<= 1) {
    const int v = (t >= w) ? s[t - w] : 0;
    __syncthreads();
    s[t] += v;
    __syncthreads();
  }
  int run = s[t] - sum;
  for (int64_t i = b; i < e; ++i) {
    const int v = in[i];
    out[i] = run;
    run += v;
  }
  if (t == 1023 && total) *total = s[1023];
}

// chunks per key and partial slots per multi-chunk key
__global__ __launch_bounds__(BS) void chunk_counts_k(const int* __restrict__ counts, int64_t len,
                                                     int* __restrict__ nch, int* __restrict__ npart) {
  for (int64_t v = (int64_t)blockIdx.x * BS + threadIdx.x; v < len; v += (int64_t)gridDim.x * BS) {
    const int c = counts[v];
    const int k = (c + CH - 1) / CH;
    nch[v] = k;
    npart[v] = k > 1 ? k : 0;
  }
}

// ---------------------------------------------------------------------------
// VJP step 3: stable LSD radix sort (8-bit digits), one wave per tile.

__global__ __launch_bounds__(BS) void radix_hist_k(const int* __restrict__ keys, int64_t n, int shift, int ntiles,
                                                   int* __restrict__ hist) {
  __shared__ int cnt[BS / 64][256];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tile = blockIdx.x * (BS / 64) + w;
  for (int d = lane; d < 256; d += 64) cnt[w][d] = 0;
  __syncthreads();
  if (tile < ntiles) {
    for (int i = lane; i < TILE; i += 64) {
      const int64_t p = (int64_t)tile * TILE + i;
      if (p < n) atomicAdd(&cnt[w][(keys[p] >> shift) & 255], 1);
    }
  }
  __syncthreads();
  if (tile < ntiles)
    for (int d = lane; d < 256; d += 64) hist[(int64_t)d * ntiles + tile] = cnt[w][d];
}

__global__ __launch_bounds__(BS) void radix_scatter_k(const int* __restrict__ keys, const int* __restrict__ vals,
                                                      int64_t n, int shift, int ntiles, const int* __restrict__ base_in,
                                                      int* __restrict__ keys_out, int* __restrict__ vals_out) {
  __shared__ int base[BS / 64][256];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tile = blockIdx.x * (BS / 64) + w;
  if (tile < ntiles)
    for (int d = lane; d < 256; d += 64) base[w][d] = base_in[(int64_t)d * ntiles + tile];
  __syncthreads();
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int r = 0; r < TILE / 64; ++r) {
    const int64_t p = (int64_t)tile * TILE + r * 64 + lane;
    const bool valid = tile < ntiles && p < n;
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
    if (valid) {
      const int dst = base[w][d] + __popcll(peers & lt);
      keys_out[dst] = k;
      vals_out[dst] = v;
    }
    __syncthreads();  // every lane has read base[] for this round
    if (valid && (__ffsll((long long)peers) - 1) == lane) base[w][d] += __popcll(peers);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// VJP step 4: chunk sums. Persistent grid; chunk c belongs to the last key v
// with choff[v] <= c.

template <bool VEC>
__global__ __launch_bounds__(BS) void chunk_sum_k(const float* __restrict__ g, int64_t outer, int64_t n,
                                                  int64_t inner, int64_t len, const int* __restrict__ perm,
                                                  const int* __restrict__ offs, const int* __restrict__ counts,
                                                  const int* __restrict__ nch, const int* __restrict__ choff,
                                                  const int* __restrict__ poff, const int* __restrict__ total_chunks,
                                                  float* __restrict__ grad, float* __restrict__ part) {
  __shared__ int sh[4];
  const int total = *total_chunks;
  const int64_t units = VEC ? inner / 4 : inner;
  for (int c = blockIdx.x; c < total; c += gridDim.x) {
    if (threadIdx.x == 0) {
      int lo = 0, hi = (int)len;  // search over keys [0, len) only: the sentinel key is never summed
      while (lo < hi) {          // first v with choff[v] > c
        const int mid = (lo + hi) >> 1;
        if (choff[mid] <= c) lo = mid + 1;
        else hi = mid;
      }
      const int v = lo - 1;
      const int j = c - choff[v];
      sh[0] = v;
      sh[1] = offs[v] + j * CH;
      sh[2] = min(CH, counts[v] - j * CH);
      sh[3] = nch[v] == 1 ? -1 : poff[v] + j;
    }
    __syncthreads();
    const int v = sh[0], start = sh[1], cnt = sh[2], slot = sh[3];
    __syncthreads();
    for (int64_t o = 0; o < outer; ++o) {
      const float* gb = g + o * n * inner;
      float* dst = slot < 0 ? grad + (o * len + v) * inner : part + ((int64_t)slot * outer + o) * inner;
      for (int64_t u = threadIdx.x; u < units; u += BS) {
        if constexpr (VEC) {
          f4 acc = {0.f, 0.f, 0.f, 0.f};
          int r = 0;
          for (; r + 8 <= cnt; r += 8) {
            f4 t[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) t[q] = reinterpret_cast<const f4*>(gb + (int64_t)perm[start + r + q] * inner)[u];
#pragma unroll
            for (int q = 0; q < 8; ++q) acc = acc + t[q];
          }
          for (; r < cnt; ++r) acc = acc + reinterpret_cast<const f4*>(gb + (int64_t)perm[start + r] * inner)[u];
          __builtin_nontemporal_store(acc, reinterpret_cast<f4*>(dst) + u);
        } else {
          float acc = 0.f;
          for (int r = 0; r < cnt; ++r) acc += gb[(int64_t)perm[start + r] * inner + u];
          dst[u] = acc;
        }
      }
    }
  }
}

// VJP step 5: every row (o, v) of grad not written by a single-chunk key.
template <bool VEC>
__global__ __launch_bounds__(BS) void finalize_k(int64_t outer, int64_t len, int64_t inner,
                                                 const int* __restrict__ nch, const int* __restrict__ poff,
                                                 const float* __restrict__ part, float* __restrict__ grad) {
  const int64_t row = blockIdx.x;  // o * len + v
  const int64_t v = row % len, o = row / len;
  const int k = nch[v];
  if (k == 1) return;
  float* dst = grad + row * inner;
  const int64_t units = VEC ? inner / 4 : inner;
  if (k == 0) {
    for (int64_t u = threadIdx.x; u < units; u += BS) {
      if constexpr (VEC) __builtin_nontemporal_store(f4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<f4*>(dst) + u);
      else dst[u] = 0.f;
    }
    return;
  }
  const int p0 = poff[v];
  for (int64_t u = threadIdx.x; u < units; u += BS) {
    if constexpr (VEC) {
      double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
      for (int j = 0; j < k; ++j) {
        const f4 t = reinterpret_cast<const f4*>(part + ((int64_t)(p0 + j) * outer + o) * inner)[u];
        a0 += t.x; a1 += t.y; a2 += t.z; a3 += t.w;
      }
      reinterpret_cast<f4*>(dst)[u] = f4{(float)a0, (float)a1, (float)a2, (float)a3};
    } else {
      double a = 0;
      for (int j = 0; j < k; ++j) a += part[((int64_t)(p0 + j) * outer + o) * inner + u];
      dst[u] = (float)a;
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
  const int64_t nk = len + 1;  // + sentinel key for invalid ids
  const int ntiles = (int)ceil_div(n, TILE);
  int passes = 0;
  for (int64_t m = len; m > 0; m >>= 8) ++passes;
  if (passes == 0) passes = 1;
  const int64_t max_parts = 2 * ceil_div(n, CH) + 1;
  // workspace layout (ints): keys, pos, keys2, pos2 (n each); counts, offs, nch, choff, npart, poff (nk each);
  // hist (256 * ntiles); scalars (4)
  const size_t ints = 4 * (size_t)n + 6 * (size_t)nk + 256 * (size_t)ntiles + 4;
  Workspace wsi(ints * sizeof(int));
  Workspace wsp((size_t)max_parts * (size_t)outer * (size_t)inner * sizeof(float));
  if (!wsi.p || !wsp.p) return OXI_OTHER;
  int* keys = wsi.as<int>();
  int* pos = keys + n;
  int* keys2 = pos + n;
  int* pos2 = keys2 + n;
  int* counts = pos2 + n;
  int* offs = counts + nk;
  int* nch = offs + nk;
  int* choff = nch + nk;
  int* npart = choff + nk;
  int* poff = npart + nk;
  int* hist = poff + nk;
  int* scal = hist + 256 * (int64_t)ntiles;  // [0] total chunks, [1] total partial slots, [2] n keys
  if (int rc = oxi_fill(reinterpret_cast<float*>(counts), nk, 0.f)) return rc;  // +0.0f is all-zero bits
  const unsigned gb = (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, BS), (int64_t)cu_count() * 8));
  keys_k<<<gb, BS, 0, s>>>(idx, n, len, keys, pos, counts, guard_flag());
  if (int rc = check_launch("index_select_bwd/keys")) return rc;
  scan_k<<<1, 1024, 0, s>>>(counts, offs, nk, scal + 2);
  const unsigned gk = (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(len, BS), (int64_t)cu_count() * 8));
  chunk_counts_k<<<gk, BS, 0, s>>>(counts, len, nch, npart);
  // the sentinel key contributes no chunks
  if (int rc = oxi_fill(reinterpret_cast<float*>(nch + len), 1, 0.f)) return rc;
  if (int rc = oxi_fill(reinterpret_cast<float*>(npart + len), 1, 0.f)) return rc;
  scan_k<<<1, 1024, 0, s>>>(nch, choff, nk, scal + 0);
  scan_k<<<1, 1024, 0, s>>>(npart, poff, nk, scal + 1);
  if (int rc = check_launch("index_select_bwd/scans")) return rc;
  // radix sort (keys, pos) -> sorted positions
  int *ka = keys, *va = pos, *kb = keys2, *vb = pos2;
  const unsigned gt = (unsigned)ceil_div(ntiles, BS / 64);
  for (int ps = 0; ps < passes; ++ps) {
    const int shift = 8 * ps;
    radix_hist_k<<<gt, BS, 0, s>>>(ka, n, shift, ntiles, hist);
    scan_k<<<1, 1024, 0, s>>>(hist, hist, 256 * (int64_t)ntiles, nullptr);
    radix_scatter_k<<<gt, BS, 0, s>>>(ka, va, n, shift, ntiles, hist, kb, vb);
    std::swap(ka, kb);
    std::swap(va, vb);
  }
  if (int rc = check_launch("index_select_bwd/sort")) return rc;
  const bool vec = inner % 4 == 0 && al16(g) && al16(grad) && inner >= 4;
  const unsigned gc = (unsigned)std::max<int64_t>(
      1, std::min<int64_t>(ceil_div(n, CH) + std::min<int64_t>(len, n), (int64_t)cu_count() * 8));
  float* part = wsp.as<float>();
  if (vec)
    chunk_sum_k<true><<<gc, BS, 0, s>>>(g, outer, n, inner, len, va, offs, counts, nch, choff, poff, scal, grad, part);
  else
    chunk_sum_k<false><<<gc, BS, 0, s>>>(g, outer, n, inner, len, va, offs, counts, nch, choff, poff, scal, grad, part);
  if (int rc = check_launch("index_select_bwd/chunks")) return rc;
  const int64_t frows = outer * len;
  if (frows >= ((int64_t)1 << 31)) return fail(OXI_INVALID_ARGUMENT, "index_select_bwd: too many output rows");
  if (vec) finalize_k<true><<<(unsigned)frows, BS, 0, s>>>(outer, len, inner, nch, poff, part, grad);
  else finalize_k<false><<<(unsigned)frows, BS, 0, s>>>(outer, len, inner, nch, poff, part, grad);
  return check_launch("index_select_bwd/finalize");
}

int oxi_embedding_fwd(const float* W, const int64_t* ids, int64_t n, int64_t V, int64_t D, float* out) {
  return oxi_index_select(W, 1, V, D, ids, n, out);
}

int oxi_embedding_bwd(const float* g, const int64_t* ids, int64_t n, int64_t V, int64_t D, float* dW) {
  return oxi_index_select_bwd(g, 1, V, D, ids, n, dW);
}

}  // extern "C"
