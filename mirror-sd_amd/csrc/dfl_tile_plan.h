// Host-side planning of the tile GEMM (dfl_tile.hip): the workgroup tile shape of an
// M x N x K product and its LDS size.  Pure host code, so a host test can check plans
// without a GPU.
#pragma once

#include <algorithm>
#include <cstddef>

#include "dfl_kernels.h"

namespace dfl {

constexpr int TG_WM = 4;                   // wave rows of a workgroup (m direction)
constexpr int TG_LDS_BUDGET = 160 * 1024;  // one workgroup per CU

// The tile shapes the library instantiates: mtw m-tiles (32 rows) and rbw weight
// row-blocks (32 columns) per wave, wn wave columns (4 * wn waves), kc k per LDS stage.
// tail: used only to re-tile the partial last round of a larger shape's plan.
struct TileShape {
  int wt, mtw, rbw, wn, kc;
  bool tail;
};
constexpr TileShape kTileShapes[] = {
    {WT_INT8, 1, 1, 1, 64, false},   // 128 x 32
    {WT_INT8, 1, 2, 1, 64, false},   // 128 x 64
    {WT_INT8, 2, 4, 1, 64, false},   // 256 x 128
    {WT_INT8, 2, 4, 2, 32, false},   // 256 x 256
    {WT_F16, 2, 2, 1, 64, false},    // 256 x 64
    {WT_F16, 2, 4, 1, 32, false},    // 256 x 128
    {WT_F16, 2, 4, 2, 32, false},    // 256 x 256
    {WT_F16, 1, 4, 1, 64, true},     // 128 x 128
};
constexpr int kNumTileShapes = (int)(sizeof(kTileShapes) / sizeof(kTileShapes[0]));
// Independent MFMA accumulation chains of a shape's waves (TgShape::NACC): with two, the
// k-blocks alternate between them and the chains are added at the end, so the sums are
// rounded differently from a shape with one.
constexpr int tile_nacc(int mtw, int rbw) { return mtw * rbw >= 4 ? 1 : 2; }

constexpr int tile_waves(int wn) { return TG_WM * wn; }
// The 4-wave shapes (wn == 1) add four loader waves that issue every global -> LDS copy
// (the compute waves never stall on a full memory queue, and four issuing waves copy
// 20-28 % faster than one: the copy rate is bounded by how fast copies are issued); the
// 8-wave shapes have no room for more waves' registers, so their compute waves issue the
// copies themselves.
constexpr int tile_loaders(int wn) { return wn == 1 ? 4 : 0; }
constexpr bool tile_loader(int wn) { return tile_loaders(wn) > 0; }
// Bytes of one stage: the X records of the workgroup's m-tiles (2 KiB per tile and k-block
// of 32) and its weight blocks (1 KiB per row-block and 32 (int8) or 16 (fp16) k).
constexpr int tile_stage_bytes(int wt, int mtw, int rbw, int wn, int kc) {
  return TG_WM * mtw * (kc / 32) * 2048 + rbw * wn * (kc / (wt == WT_INT8 ? 32 : 16)) * 1024;
}
// Stage buffers: as many as fit the LDS budget, at most 8, at most 3 more than a wave's
// vmcnt field (6 bits) counts in stages of its share of the copies, at least 3.  All but
// three of them are in flight while the compute waves read one and multiply another.
constexpr int tile_stages(int wt, int mtw, int rbw, int wn, int kc) {
  const int sb = tile_stage_bytes(wt, mtw, rbw, wn, kc);
  const int per_wave =
      tile_loader(wn) ? (sb / 1024 + tile_loaders(wn) - 1) / tile_loaders(wn)
                      : (sb / 1024 + tile_waves(wn) - 1) / tile_waves(wn);
  const int by_lds = TG_LDS_BUDGET / sb;
  const int by_cnt = 3 + 63 / (per_wave > 0 ? per_wave : 1);
  const int s = by_lds < by_cnt ? by_lds : by_cnt;
  return s < 3 ? 3 : (s > 8 ? 8 : s);
}

// Estimated cycles of one k-block (32 k) of a workgroup: the larger of the MFMA time of a
// SIMD (32 cycles per 32x32x16 MFMA, wn waves per SIMD) and the copy time of the block's X
// and weight bytes at the global -> LDS rate measured for the shape at M = 128-4096 (B per
// cycle and CU: 20.5 with loader waves and 64-k stages, 18.5 with 32-k stages (one barrier
// per k-block), 12.5 when the 8 compute waves issue the copies).
inline double tile_kblock_cycles(const TileShape& s) {
  const double mfma = 32.0 * 2 * s.mtw * s.rbw * s.wn;
  const double bytes = TG_WM * s.mtw * 2048.0 + s.rbw * s.wn * 1024.0 * (s.wt == WT_INT8 ? 1 : 2);
  const double rate = tile_loader(s.wn) ? (s.kc == 64 ? 20.5 : 18.5) : 12.5;
  return std::max(mfma, bytes / rate);
}

// The instantiated shape (and split-K factor) with the least estimated time, in cycles of
// 2.4 GHz: rounds of one workgroup per CU x k-blocks x cycles per k-block, where a last
// partial round after full ones counts 0.75-1 of a round (its few workgroups copy faster:
// 0.75 measured at 16 of 256).  A split-K (allowed with split) runs fewer k-blocks per
// workgroup on larger tiles, so less X per flop, but each workgroup writes its fp32 tile
// (about 21 B per cycle) and a reduction launch reads every plane (about 1.3 KB per cycle
// over the chip, plus 12000 cycles of launch and tail).  Fitted to the measured times of
// the 8B- and 27B-class stacked products, the prompt-sized K|V ingest and the fp16
// lm_head (each picks its measured-fastest plan).
// Re-tiling (allowed with retile, no split-K): a plan of more tiles than CUs whose last
// round is partial may run that round's tiles on a smaller shape whose tiles divide them,
// several workgroups per tile over the whole K (the same sums), so that the last round
// finishes sooner; it costs one more launch (about 12000 cycles).
// Only the sub-shapes with the parent's accumulation chains qualify, so a tile's sums do
// not depend on which round it ran in.
// pairs: each wave must hold gate|up row-block pairs (SWIGLU), i.e. an even rbw.
// like (optional): only that shape (mtw, rbw, wn, kc), so that a product runs with the
// accumulation of another plan's (e.g. one layer's product stacked over several layers).
inline TilePlan tile_plan(int M, int N, int K, int wt, int n_cu, bool pairs = false,
                          bool split = false, bool retile = false,
                          const TilePlan* like = nullptr) {
  TilePlan best{};
  double best_t = 1e300;
  for (const TileShape& s : kTileShapes) {
    if (s.tail || s.wt != wt || K % s.kc || (pairs && s.rbw % 2)) continue;
    if (like && (s.mtw != like->mtw || s.rbw != like->rbw || s.wn != like->wn || s.kc != like->kc))
      continue;
    const int bm = 32 * TG_WM * s.mtw, bn = 32 * s.rbw * s.wn;
    if (N % bn) continue;
    const long long tiles = (long long)((M + bm - 1) / bm) * (N / bn);
    for (int sp = 1; sp <= (split ? 16 : 1) && sp <= K / 64; sp *= 2) {
      if (sp > 1 && tiles * sp > n_cu) break;
      const long long full = tiles * sp / n_cu, part = tiles * sp % n_cu;
      const double rounds =
          (double)full + (part == 0 ? 0.0 : full > 0 ? 0.75 + 0.25 * part / n_cu : 1.0);
      double t = rounds * ((double)K / 32 / sp) * tile_kblock_cycles(s);
      if (sp > 1)
        t += (double)bm * bn * 4 / 21.0 + (double)(sp + 1) * M * N * 4 / 1300.0 + 12000.0;
      if (t < best_t * 0.999) {
        best_t = t;
        best.mtw = s.mtw;
        best.rbw = s.rbw;
        best.wn = s.wn;
        best.kc = s.kc;
        best.tiles_m = (M + bm - 1) / bm;
        best.tiles_n = N / bn;
        best.splits = sp;
        best.head_tiles = 0;
        best.tail_shape = -1;
      }
    }
    const long long full = tiles / n_cu, part = tiles % n_cu;
    if (!retile || full < 1 || part == 0) continue;
    for (int i = 0; i < kNumTileShapes; ++i) {
      const TileShape& u = kTileShapes[i];
      const int um = 32 * TG_WM * u.mtw, un = 32 * u.rbw * u.wn;
      if (u.wt != wt || K % u.kc || (pairs && u.rbw % 2) || bm % um || bn % un ||
          (um == bm && un == bn) || tile_nacc(u.mtw, u.rbw) != tile_nacc(s.mtw, s.rbw))
        continue;
      const long long sub = (long long)(bm / um) * (bn / un);
      const long long ur = (part * sub + n_cu - 1) / n_cu;   // rounds of the sub-tiles
      const double t = ((double)full * tile_kblock_cycles(s) + ur * tile_kblock_cycles(u)) *
                           ((double)K / 32) + 12000.0;
      if (t < best_t * 0.999) {
        best_t = t;
        best.mtw = s.mtw;
        best.rbw = s.rbw;
        best.wn = s.wn;
        best.kc = s.kc;
        best.tiles_m = (M + bm - 1) / bm;
        best.tiles_n = N / bn;
        best.splits = 1;
        best.head_tiles = (int)(full * n_cu);
        best.tail_shape = i;
      }
    }
  }
  return best;
}

inline size_t tile_lds_bytes(int wt, const TilePlan& p) {
  return (size_t)tile_stages(wt, p.mtw, p.rbw, p.wn, p.kc) *
         tile_stage_bytes(wt, p.mtw, p.rbw, p.wn, p.kc);
}

}  // namespace dfl
