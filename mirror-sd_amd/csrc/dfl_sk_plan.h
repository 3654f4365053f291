// Host-side partition plans of the stream-K GEMM (dfl_stream.hip).  Pure host code, so a
// host test can check every plan the library would launch without a GPU.
#pragma once

#include <algorithm>

#include "dfl_kernels.h"

namespace dfl {

inline SKPlan streamk_plan(int N, int KB, int n_cu) {
  // One workgroup per CU.  When there are fewer wave-tiles than CUs the worker count is
  // the largest multiple of the tile count that fits, so every tile is split into the
  // same number of equal k-ranges (no worker straddles two tiles).  With at least one
  // tile per CU, each workgroup also gets dp = tiles / CUs whole tiles, streamed after its
  // share of the remaining tiles' split units (hybrid plan; the M-split kernel keeps the
  // contiguous partition, whose slot count is seg_cap).
  SKPlan p;
  const long long nt = N / 64;
  const long long U = nt * KB;
  long long W = n_cu;
  if (nt < n_cu) W = std::max(1LL, (long long)n_cu / nt) * nt;
  p.workers = (int)std::max(1LL, std::min(W, U));
  const long long per = std::max(1LL, U / p.workers);
  p.seg_cap = (int)((KB + per - 1) / per + 1);
  if (nt >= n_cu) {
    p.dp = (int)(nt / n_cu);
    const long long S = (nt - (long long)p.dp * n_cu) * KB;
    const long long sper = std::max(1LL, S / n_cu);
    p.sk_seg_cap = S > 0 ? (int)((KB + sper - 1) / sper + 1) : 1;
  }
  return p;
}

inline SKPlan streamk_plan_balanced(int N, int KB, int n_cu) {
  SKPlan p = streamk_plan(N, KB, n_cu);
  p.dp = 0;
  p.sk_seg_cap = 0;
  const long long nt = N / 64;
  if (nt < 2LL * n_cu || (KB & 1)) return p;
  p.workers = n_cu;
  // whole rounds of tiles statically, the remainder (less than one tile per workgroup) as
  // balanced half tiles: with one argmax atomic per row and workgroup the XCDs stream at
  // the same rate (242 us at 27B against 251 with 86 % static and 254 with 72 %; the
  // spread of up to a quarter between XCDs measured earlier came with an atomicMax per
  // tile on the same 32 keys)
  p.dyn_static = (int)(nt / n_cu);
  p.seg_cap = std::max(p.seg_cap, 2);
  return p;
}

// Whole tiles per workgroup that one launch of plan p uses.  The hybrid plan (dp > 0) needs
// the single-tile kernel; the M-split kernel and the fused qkv kernel (EPI_QKROPE: a Q/K
// head's two tiles complete together, worker counts taken from the contiguous partition)
// keep the contiguous partition.
inline int streamk_launch_dp(const SKPlan& p, int epi, bool m_split) {
  return (!m_split && epi != EPI_QKROPE) ? p.dp : 0;
}

}  // namespace dfl
