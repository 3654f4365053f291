// Host-side consistency checks of the kernel launch argument structs.  Each returns nullptr
// when the struct is consistent with what its kernel assumes, else a short reason; the
// launchers refuse (launch nothing) on a reason, and the C ABI reports it as DFL_EINVAL.
// Pure host code: a host test can exercise every rule without a GPU.
#pragma once

#include "dfl_kernels.h"
#include "dfl_tile_plan.h"

namespace dfl {

constexpr int CHECK_WG_WAVES = 4;   // streaming waves of a stream-K workgroup (unit walk stride)
constexpr int CHECK_MAX_CHUNKS = 64;

inline const char* check_stream_args(int wt, int epi, bool norm, const StreamArgs& a,
                                     const SKPlan& p, bool m_split) {
  if (wt != WT_INT8 && wt != WT_F16) return "unknown weight type";
  if (!a.W) return "null weight matrix";
  if (a.N <= 0 || a.N % 64) return "N must be a positive multiple of 64";
  if (a.KB < CHECK_WG_WAVES) return "fewer k-blocks than streaming waves";
  if (a.xr_n < 0 || a.xr_n > MAX_FEATS) return "row-major activations: feature count out of range";
  if (a.xr_n > 0) {
    if (wt != WT_F16 || epi != EPI_RESID || norm || m_split)
      return "row-major activations are read by the one-tile fp16 RESID kernel only";
    if (a.xr_h < 64 || a.xr_h % 16 || (long long)a.xr_n * a.xr_h != (long long)a.KB * 16)
      return "row-major activations: features do not tile the K axis in 16-column blocks";
    if (a.xr_ld < a.xr_h || a.xr_ld % 8)
      return "row-major activations: row stride below the feature width or not a multiple of 8";
    for (int j = 0; j < a.xr_n; ++j)
      if (!a.xr_p[j] || (reinterpret_cast<uintptr_t>(a.xr_p[j]) & 15))
        return "row-major activations: feature rows null or not 16-byte aligned";
  } else if (!a.X) {
    return "null activations";
  }
  if (a.M < 1) return "no activation rows";
  if (m_split ? (a.MT < 2 || a.MT > 8 || a.M > 32 * a.MT) : (a.M > 32))
    return "activation rows exceed the kernel's m-tiles";
  if (p.workers < 1 || a.seg_cap < 1 || !a.ws || !a.tile_cnt)
    return "missing split-tile workspace";
  if (wt == WT_INT8 && !a.scale) return "int8 weights without per-row scales";
  if (norm) {
    const int K = a.KB * (wt == WT_INT8 ? 32 : 16);
    if (!a.gnorm || K > 8192) return "norm-on-load needs a gain of at most 8192 entries";
    if (!a.ss_in && !a.rnorm) return "norm-on-load needs row sums or 1/rms rows";
    if (a.ss_in && (a.ss_tiles < 1 || a.ss_tiles > 128 || a.ss_n < 1))
      return "row-sum tiles outside [1, 128]";
  }
  switch (epi) {
    case EPI_STORE:
      if (!a.out || a.ldo < a.N) return "STORE without an output of N columns";
      break;
    case EPI_RESID:
      if (!a.x || !a.ss_part) return "RESID without residual rows and row sums";
      break;
    case EPI_SWIGLU:
      if (!a.out || wt != WT_INT8) return "SWIGLU needs int8 weights and an output";
      break;
    case EPI_ARGMAX:
      if (wt != WT_F16 || (!a.keys && !a.logits)) return "ARGMAX needs fp16 weights and keys or logits";
      break;
    case EPI_QKROPE: {
      const RopeEpi& r = a.rope;
      if (m_split || a.M > 32 || !norm) return "QKROPE is the single-tile normed qkv kernel";
      if (a.N != (r.NH + 2 * r.NKV) * 128 || r.NH < 1 || r.NKV < 1)
        return "QKROPE rows are not the q|k|v heads";
      if (a.N > QK_N_MAX) return "QKROPE: more q|k|v rows than the scales' LDS copy holds";
      if (!a.scale || (reinterpret_cast<uintptr_t>(a.scale) & 15) ||
          (reinterpret_cast<uintptr_t>(r.cs) & 15) || (reinterpret_cast<uintptr_t>(r.q_norm) & 15) ||
          (reinterpret_cast<uintptr_t>(r.k_norm) & 15))
        return "QKROPE tables must be 16-byte aligned";
      if (!r.Q || !r.cs || !r.q_norm || !r.k_norm || !r.sq.Kc || !r.sq.Vt || r.cap < 1)
        return "QKROPE outputs or tables missing";
      break;
    }
    default:
      return "unknown epilogue";
  }
  if (a.x_zero && epi != EPI_RESID) return "a zero residual (x_zero) is a RESID option";
  if (p.dyn_static > 0 && (!a.dyn_next || !a.err || (a.KB & 1) || epi != EPI_ARGMAX))
    return "balanced plan needs work counters, an error word and an even k-block count";
  if (a.dp > 0 && ((long long)a.dp * p.workers > a.N / 64 || m_split))
    return "hybrid plan with more whole tiles than the matrix has";
  // the fused qkv kernel completes a Q/K head's two tiles together over the contiguous
  // stream-K partition only (its whole-tile loop runs the V-head epilogue)
  if (a.dp > 0 && epi == EPI_QKROPE) return "QKROPE takes the contiguous partition (dp = 0)";
  return nullptr;
}

inline const char* check_qk_rope_args(const QKRopeArgs& a) {
  if ((a.qkv16 == nullptr) == (a.qkv32 == nullptr)) return "pass exactly one of qkv16 / qkv32";
  if (a.qkv32 && !a.oscale) return "fp32 rows without per-column scales";
  if (a.M < 1 || a.n_seq < 1 || a.n_seq > SEQ_MAX) return "rows or sequences out of range";
  if (a.NH < 1 || a.NKV < 1 || a.n_slots < 1 || a.slot0 < a.col_slot0 ||
      a.slot0 + a.n_slots > a.NH + 2 * a.NKV)
    return "head slots outside the q|k|v heads";
  if (a.layer_cols) {
    if (a.slot0 < a.NH) return "layer mode takes K|V rows only";
    if ((long long)(a.slot0 + a.n_slots - a.col_slot0) * 128 > a.layer_cols ||
        (long long)a.n_seq * a.layer_cols > a.N)
      return "slots past the row width";
    for (int s = 0; s < a.n_seq; ++s)
      if (!a.k_norm_s[s]) return "layer mode without a per-layer k_norm";
  } else if ((long long)(a.slot0 + a.n_slots - a.col_slot0) * 128 > a.N) {
    return "slots past the row width";
  }
  if (a.slot0 < a.NH && !a.Q) return "Q slots without a Q output";
  if (a.cs && !a.layer_cols)
    for (int s = 1; s < a.n_seq; ++s)
      if (a.sq[s].pos0 != a.sq[0].pos0) return "one angle table for sequences at other positions";
  if (!a.q_norm || !a.k_norm || a.cap < 1) return "missing norms or cache capacity";
  // 4-element vector loads and stores: rows, scales, gains, angles and outputs aligned
  auto mis = [](const void* q, uintptr_t m) { return (reinterpret_cast<uintptr_t>(q) & m) != 0; };
  if (a.N % 4 || mis(a.qkv32, 15) || mis(a.oscale, 7) || mis(a.qkv16, 7) || mis(a.q_norm, 7) ||
      mis(a.k_norm, 7) || mis(a.cs, 15) || mis(a.Q, 7))
    return "QK rope rows, scales, gains, angle table or Q not aligned for 4-element access";
  for (int s = 0; s < a.n_seq; ++s)
    if (mis(a.k_norm_s[s], 7) || mis(a.sq[s].Kc, 7)) return "k_norm or K cache not 8-byte aligned";
  if (a.slot0 + a.n_slots > a.NH)
    for (int s = 0; s < a.n_seq; ++s)
      if (!a.sq[s].Kc || !a.sq[s].Vt) return "K/V slots without cache pointers";
  return nullptr;
}

inline const char* check_attn_args(const AttnArgs& a) {
  if (!a.Q || !a.Op || !a.Ml || !a.O) return "missing attention buffers";
  if (a.B < 1 || a.NH < 1 || a.NKV < 1 || a.NH % a.NKV) return "bad head counts or block rows";
  if (a.n_seq < 1 || a.n_seq > SEQ_MAX) return "sequences out of range";
  if (a.max_chunks < 1 || a.max_chunks > CHECK_MAX_CHUNKS) return "chunk count out of range";
  if (a.chunk0[0] != 0) return "chunk table does not start at 0";
  for (int s = 0; s < a.n_seq; ++s) {
    const AttnSeq& q = a.sq[s];
    if (!q.Kc || !q.Vt || q.L < 1 || q.L > a.cap) return "sequence keys out of range";
    if (q.chunk < 32 || q.chunk % 32 || q.n_chunks < 1 || q.n_chunks > a.max_chunks ||
        (long long)q.chunk * q.n_chunks < q.L || (long long)q.chunk * (q.n_chunks - 1) >= q.L)
      return "key chunks do not tile the keys";
    if (a.chunk0[s + 1] != a.chunk0[s] + q.n_chunks) return "chunk table inconsistent";
  }
  return nullptr;
}

inline const char* check_tile_args(int wt, int epi, const TileArgs& a, const TilePlan& p) {
  if (wt != WT_INT8 && wt != WT_F16) return "unknown weight type";
  if (!a.W || !a.X) return "null weights or activations";
  switch (epi) {
    case TG_F32:
      if (!a.Y) return "F32 epilogue without an output";
      break;
    case TG_RESID:
      if (wt != WT_INT8 || !a.scale || !a.x || !a.ss) return "RESID needs int8 weights, scales, x and row sums";
      break;
    case TG_SWIGLU:
      if (wt != WT_INT8 || !a.scale || !a.out || p.rbw % 2)
        return "SWIGLU needs int8 weights, scales, an output and gate|up pairs in each wave";
      break;
    case TG_ARGMAX:
      if (wt != WT_F16 || !a.keys) return "ARGMAX needs fp16 weights and keys";
      break;
    default:
      return "unknown epilogue";
  }
  if (p.mtw < 1 || p.mtw > 2 || (p.rbw != 1 && p.rbw != 2 && p.rbw != 4) || p.wn < 1 ||
      p.wn > 2 || (p.kc != 32 && p.kc != 64))
    return "unknown tile shape";
  if (a.M < 1 || a.N < 1 || a.K < 64 || a.K % 64 || a.K % p.kc)
    return "M, N >= 1 and K a positive multiple of 64 and of the stage's k";
  if (a.N % (32 * p.rbw * p.wn)) return "N is not a multiple of the tile's columns";
  if (a.Y && a.ldy < a.N) return "output row shorter than N";
  if (p.tiles_n != a.N / (32 * p.rbw * p.wn) || (long long)p.tiles_m * 128 * p.mtw < a.M ||
      (long long)p.tiles_m * 128 * p.mtw >= (long long)a.M + 128 * p.mtw)
    return "tile counts do not cover the product";
  if (p.splits < 1 || p.splits > a.K / 64) return "split-K factor outside [1, K/64]";
  if (p.splits > 1 && epi != TG_F32) return "split-K writes F32 planes only";
  if (p.tail_shape >= 0) {
    if (p.tail_shape >= kNumTileShapes || p.splits != 1) return "re-tiled tail: unknown shape";
    const TileShape& u = kTileShapes[p.tail_shape];
    if (u.wt != wt || a.K % u.kc || (128 * p.mtw) % (128 * u.mtw) ||
        (32 * p.rbw * p.wn) % (32 * u.rbw * u.wn) || (epi == TG_SWIGLU && u.rbw % 2) ||
        tile_nacc(u.mtw, u.rbw) != tile_nacc(p.mtw, p.rbw))
      return "re-tiled tail: the shape does not divide the plan's tiles";
    if (p.head_tiles < 1 || p.head_tiles >= p.tiles_m * p.tiles_n)
      return "re-tiled tail: needs head tiles and a tail";
  }
  if ((long long)p.tiles_m * p.tiles_n * p.splits > 0x7fffffffLL) return "too many tiles";
  return nullptr;
}

inline const char* check_tile_reduce_args(int epi, const TileArgs& a, const float* parts,
                                          int splits) {
  if (!parts || splits < 1) return "no split-K planes";
  if (a.M < 1 || a.N < 64 || a.N % 64) return "N must be a positive multiple of 64";
  if (epi == TG_F32) {
    if (!a.Y || a.ldy < a.N) return "F32 reduction without an output of N columns";
  } else if (epi == TG_RESID) {
    if (!a.x || !a.ss || !a.scale) return "RESID reduction needs x, row sums and scales";
  } else {
    return "the reduction has F32 and RESID epilogues only";
  }
  return nullptr;
}

}  // namespace dfl
