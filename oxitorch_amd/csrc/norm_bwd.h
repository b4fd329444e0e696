// Norm VJP launches shared by norm.hip (the entry points) and the
// translation units that instantiate the backward kernels, one per folded
// activation (norm_bwd_none.hip, norm_bwd_gelu.hip, norm_bwd_silu.hip,
// norm_bwd_softmax.hip), so that the build compiles them side by side.
#pragma once

#include <initializer_list>

#include "internal.h"
#include "ops.h"
#include "rowtile.h"

namespace oxi {

// One norm VJP launch: x (rows, H), the weight w, bias b (layer_norm with a
// folded activation), the forward's row statistics, the upstream gradient g;
// outputs dyo (the activation input's gradient, optional), dx, dw, db; the
// column partials in `fixed` (fixed_bytes) when set, else from the caching
// allocator; lsum (rows / lead, H), when set, the sum of dx over the leading
// dim of a (lead, rows / lead) row grid.
struct NormBwdArgs {
  const float* x;
  const float* w;
  const float* b;
  const float* mean;
  const float* rstd;
  const float* g;
  float* dyo;
  float* dx;
  float* dw;
  float* db;
  int64_t rows;
  int64_t H;
  void* fixed = nullptr;
  float* lsum = nullptr;
  int64_t lead = 0;
  size_t fixed_bytes = 0;
};

// The VJP of a layer_norm (ln) or rms_norm in VJP mode `mode` with the VJP of
// activation `act` on its output folded in: none, tanh or erf GELU, SiLU,
// softmax or log_softmax over the row.
int norm_bwd_none(bool ln, int mode, const NormBwdArgs& a);
int norm_bwd_gelu(int act, bool ln, int mode, const NormBwdArgs& a);
int norm_bwd_silu(bool ln, int mode, const NormBwdArgs& a);
int norm_bwd_softmax(int act, bool ln, int mode, const NormBwdArgs& a);

constexpr bool is_softmax_act(int act) { return act == OXI_ACT_SOFTMAX || act == OXI_ACT_LOG_SOFTMAX; }

// Rows of the leading-sum walk in flight per wave; lead must be a multiple.
#ifndef OXI_LSUM_DEPTH
#define OXI_LSUM_DEPTH 4
#endif
constexpr int LSUM_DEPTH = OXI_LSUM_DEPTH;

inline bool vec_ok(int64_t H, std::initializer_list<const void*> ptrs) {
  if (H % 4 != 0) return false;
  for (const void* p : ptrs)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15u)) return false;
  return true;
}

// (TPR, NV) of the backward for a vectorized row of h4 float4s; 0 when it
// does not fit. The backward keeps its rows multi-float4 per lane: it walks
// rows grid-strided with column partials, and one-wave groups let 16 rows
// share a block. Rows past 2048 floats spread over 512 threads: the norm +
// activation VJP needs 218 VGPRs at 256 x 4 float4s (2 waves per SIMD) and
// 128 at 512 x 2 (4 waves per SIMD), and the plain VJP runs as fast at either
// width, so both use the same configuration and their row sums agree bit
// for bit.
inline int pick_bwd_cfg(int64_t h4) {
  if (h4 <= 64) return 641;
  if (h4 <= 128) return 642;
  if (h4 <= 192) return 643;
  if (h4 <= 256) return 644;
  if (h4 <= 512) return 2562;
  if (h4 <= 1024) return 5122;
  if (h4 <= 2048) return 5124;
  return 0;
}

// 1024-thread (one-wave row) blocks per CU: 2 made C5's layer_norm + silu
// VJP 43 us against 35 us at 1 (C1's rms_norm VJP unchanged)
#ifndef OXI_BWD_BPC1024
#define OXI_BWD_BPC1024 1
#endif
// Blocks per CU of the 512- and 256-thread backward blocks: 1 took C2's
// layer_norm + erf-GELU VJP from 156.7 to 138.3 us in the warm step (half
// the column partials, and their finish, at the same bandwidth); 2 was the
// earlier setting, 3 measured 156.0. bwd_blocks_per_cu() sizes both the
// launch and its column-partial buffer (the softmax positional-sum split
// aside, which sizes its own).
#ifndef OXI_BWD_BPC_OTHER
#define OXI_BWD_BPC_OTHER 1
#endif
constexpr int bwd_blocks_per_cu(int nt) { return nt == 1024 ? OXI_BWD_BPC1024 : OXI_BWD_BPC_OTHER; }

// Bytes of column partials the backward needs for (rows, H): 2 x blocks x H
// floats, or 0 when neither dw nor db is wanted.
inline size_t bwd_part_bytes(bool need_part, int64_t rows, int64_t H, int cfg) {
  if (!need_part) return 0;
  const int tpr = cfg ? cfg / 10 : 256;  // the loop kernel: 256-thread blocks
  const int nt = tpr == 64 ? (cfg % 10 <= 3 ? 1024 : 512) : tpr;  // bwd_threads<TPR, NV>()
  int64_t nblk = ceil_div(rows, nt / tpr);
  const int64_t cap = (int64_t)cu_count() * bwd_blocks_per_cu(nt);
  if (nblk > cap) nblk = cap;
  if (nblk < 1) nblk = 1;
  return sizeof(float) * 2 * (size_t)nblk * (size_t)H;
}

}  // namespace oxi
