// Tile GEMM for stacked activation rows (M > 64): the compute-bound projection shapes.
//
//   Y[M][N] (fp32, row-major) = X[M][K] . W[N][K]^T
//
// X is in the activation fragment layout (32-row tiles of 1 KiB records, afl_offset) and
// W in the packed 1 KiB blocks of the stream-K kernel (int8 [32 rows][32 k], or fp16
// [32 rows][16 k]), so the same weight bytes serve both kernels and no fp16 copy of an
// int8 matrix exists.  For int8 weights Y holds the exact-integer-weight sums; the per-row
// scale and the fp16 rounding of the Linear are applied by the consumer (the same
// epilogue arithmetic as the stream-K kernel).
//
// At M = 256 an int8 weight byte feeds 512 flop, above the MI355X ridge (~312 flop/B), so
// these shapes are MFMA-bound rather than HBM-bound; what bounds them in practice is the
// global -> LDS copy rate (12.5-20.5 B per cycle and CU, 8-13 TB/s over the chip, set by
// how fast the issuing waves issue copies), so the larger the workgroup tile, the fewer
// bytes per flop.  A workgroup of 4 * WN compute waves (WN = 1 or 2 wave columns; plus
// four loader waves that issue every copy when WN = 1) computes a BM x BN output tile:
// BM = 128 * MTW rows (wave row wm owns m-tiles
// [wm*MTW, (wm+1)*MTW)), BN = 32 * RBW * WN columns (wave column wn owns row-blocks
// [wn*RBW, (wn+1)*RBW)).  K is walked in stages of KC (32 or 64): each stage's X records
// (BM/32 tiles x KC/16 KiB, contiguous per tile) and weight blocks (contiguous per
// row-block) are copied global -> LDS with global_load_lds (1 KiB per wave instruction,
// no VGPR staging), the copies spread over the issuing waves, into a ring of 3 to 8 stage
// buffers (as many as 160 KiB holds), all but three in flight.  The compute waves work per k-block
// of 32: the next block's fragments are read from LDS (lane-linear 16-byte reads,
// conflict-free) while the current block is multiplied; int8 blocks are dequantised
// exactly in registers (dequant_i8x16).
//
// Output lane layout of v_mfma_f32_32x32x16_f16 with A = X (rows m) and B = W (columns
// n): accumulator r of lane l is Y[8*(r/4) + 4*(l/32) + r%4][l%32], so each store
// instruction writes 128 contiguous bytes of two rows.
#include <hip/hip_ext.h>

#include <algorithm>

#include "dfl_check.h"
#include "dfl_common.h"
#include "dfl_kernels.h"
#include "dfl_tile_plan.h"

namespace dfl {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;
constexpr int TG_GROUP_M = 4;   // m-tile rows per group of the tile order

// Tile `tile` of the group order (see tile_gemm_kernel) -> its m-tile row tm and column tn.
DFL_DEV void tile_coords(const TileArgs& a, int tile, int& tm, int& tn) {
  const int gsz = TG_GROUP_M * a.tiles_n;
  const int grp = tile / gsz, first_m = grp * TG_GROUP_M;
  const int gm = min(a.tiles_m - first_m, TG_GROUP_M);
  const int tig = tile - grp * gsz;
  tm = first_m + tig % gm;
  tn = tig / gm;
}

template <int WT, int MTW, int RBW, int WN, int KC>
struct TgShape {
  static constexpr int NW = TG_WM * WN;                      // compute waves
  static constexpr bool LOADER = tile_loader(WN);            // + loader waves
  static constexpr int NLOAD = tile_loaders(WN);
  static constexpr int MT = TG_WM * MTW;                     // m-tiles per workgroup
  static constexpr int RB = RBW * WN;                        // row-blocks per workgroup
  static constexpr int KBS = KC / 32;                        // k-blocks of 32 per stage
  static constexpr int XREC = 2 * KBS;                       // X records per tile and stage
  static constexpr int X_BYTES = MT * XREC * 1024;
  static constexpr int WBLK = WT == WT_INT8 ? KBS : 2 * KBS;  // weight blocks per row-block
  static constexpr int W_BLOCKS = RB * WBLK;
  static constexpr int STAGE = X_BYTES + W_BLOCKS * 1024;
  static constexpr int IPS = STAGE / 1024;                   // copies per stage
  // copies per issuing wave (at least)
  static constexpr int PER_WAVE_MIN = LOADER ? IPS / NLOAD : IPS / NW;
  static constexpr int STAGES = tile_stages(WT, MTW, RBW, WN, KC);
  static constexpr int LDS = STAGES * STAGE;
  static_assert(STAGE == tile_stage_bytes(WT, MTW, RBW, WN, KC), "stage size");
  static_assert((STAGES - 3) * (LOADER ? (IPS + NLOAD - 1) / NLOAD : (IPS + NW - 1) / NW) < 64 &&
                    STAGES >= 3,
                "vmcnt range");
  static_assert(LDS <= TG_LDS_BUDGET, "LDS budget");
  static constexpr int NACC = tile_nacc(MTW, RBW);           // independent MFMA chains
};

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt
// left at "no wait").
template <int N>
DFL_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

DFL_DEV void tg_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

DFL_DEV u32x4 lds_read16(const unsigned char* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Fragments of one k-block (32 k) for one wave: its X fragments and raw weight blocks.
template <int WT, int MTW, int RBW>
struct TgFrag {
  static constexpr int NQ = WT == WT_INT8 ? 1 : 2;   // weight blocks per row-block and k-block
  half8_t x[NQ][MTW][WT == WT_INT8 ? 2 : 1];
  u32x4 w[NQ][RBW];
};

// Reads k-block kbl of the stage at xs for the wave at (wm, wn).
template <class S, int WT, int MTW, int RBW>
DFL_DEV void tg_read_frags(TgFrag<WT, MTW, RBW>& f, const unsigned char* xs, int kbl, int wm,
                           int wn, int lane) {
  const unsigned char* ws = xs + S::X_BYTES;
  if constexpr (WT == WT_INT8) {
    static_for<0, RBW>([&](auto r) {
      const int rb = wn * RBW + r;
      f.w[0][r] = lds_read16(ws + (rb * S::WBLK + kbl) * 1024 + lane * 16);
    });
    static_for<0, MTW>([&](auto t) {
      const int mtl = wm * MTW + t;
      f.x[0][t][0] = as_half8(lds_read16(xs + (mtl * S::XREC + 2 * kbl + 0) * 1024 + lane * 16));
      f.x[0][t][1] = as_half8(lds_read16(xs + (mtl * S::XREC + 2 * kbl + 1) * 1024 + lane * 16));
    });
  } else {
    // fp16 block q = 2*kbl + qq holds, for lane l, k = 16*q + 8*(l/32) + 0..7; the matching
    // activation halves sit in record (kbl, h = l/32) at lane position l%32 + 32*qq
    const int g = lane >> 5;
    static_for<0, 2>([&](auto qq) {
      static_for<0, RBW>([&](auto r) {
        const int rb = wn * RBW + r;
        f.w[qq][r] = lds_read16(ws + (rb * S::WBLK + 2 * kbl + qq) * 1024 + lane * 16);
      });
      static_for<0, MTW>([&](auto t) {
        const int mtl = wm * MTW + t;
        f.x[qq][t][0] = as_half8(lds_read16(xs + (mtl * S::XREC + 2 * kbl + g) * 1024 +
                                            ((lane & 31) + 32 * qq) * 16));
      });
    });
  }
}

// int8 weights with two m-tiles per wave, dequantised one row-block ahead: the 2 * MTW
// MFMAs of row-block r issue between the 16 VALU instructions that dequantise row-block
// r + 1 (row-block 0 of the next k-block, w_next, after the last), so the matrix unit runs
// while the wave's VALU work issues (one compute wave per SIMD: nothing else hides it).
// d holds row-block 0 of this k-block on entry and that of the next k-block on exit.
template <int MTW, int RBW, int NACC>
DFL_DEV void tg_mfma_i8(const TgFrag<WT_INT8, MTW, RBW>& f, half8_t (&d)[2], const u32x4& w_next,
                        floatx16 (&acc)[RBW][MTW][NACC]) {
  __builtin_amdgcn_sched_barrier(0);
  half8_t lo = d[0], hi = d[1];
  static_for<0, RBW>([&](auto r) {
    half8_t nlo, nhi;
    if constexpr (r + 1 < RBW) dequant_i8x16(f.w[0][r + 1], nlo, nhi);
    else dequant_i8x16(w_next, nlo, nhi);
    static_for<0, MTW>([&](auto t) {
      acc[r][t][0] = mfma32x32x16(f.x[0][t][0], lo, acc[r][t][0]);
      acc[r][t][NACC - 1] = mfma32x32x16(f.x[0][t][1], hi, acc[r][t][NACC - 1]);
    });
    lo = nlo;
    hi = nhi;
  });
  // keeps the next k-block's dequantisation here rather than sunk to its first use
  asm volatile("" : "+v"(lo), "+v"(hi));
  d[0] = lo;
  d[1] = hi;
  constexpr int PER = (16 + 2 * MTW - 1) / (2 * MTW);
  static_for<0, RBW * 2 * MTW>([&](auto) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, PER, 0);  // PER VALU
  });
  __builtin_amdgcn_sched_barrier(0);
}

template <int WT, int MTW, int RBW, int NACC>
DFL_DEV void tg_mfma(const TgFrag<WT, MTW, RBW>& f, floatx16 (&acc)[RBW][MTW][NACC]) {
  if constexpr (WT == WT_INT8) {
    static_for<0, RBW>([&](auto r) {
      half8_t lo, hi;
      dequant_i8x16(f.w[0][r], lo, hi);
      static_for<0, MTW>([&](auto t) {
        acc[r][t][0] = mfma32x32x16(f.x[0][t][0], lo, acc[r][t][0]);
        acc[r][t][NACC - 1] = mfma32x32x16(f.x[0][t][1], hi, acc[r][t][NACC - 1]);
      });
    });
  } else {
    static_for<0, 2>([&](auto qq) {
      static_for<0, RBW>([&](auto r) {
        static_for<0, MTW>([&](auto t) {
          constexpr int c = NACC == 1 ? 0 : (int)qq;
          acc[r][t][c] = mfma32x32x16(f.x[qq][t][0], as_half8(f.w[qq][r]), acc[r][t][c]);
        });
      });
    });
  }
}

// Barriers: before B(t) every issuing wave waits for its own copies of stage t + 1, so
// after B(t) stage t + 1 is in LDS; B(t) also orders every read of stage t - 1 (consumed by
// MFMAs before B(t)) before the copies of stage t + STAGES - 1 that refill its buffer,
// issued right after B(t).  B(-1) precedes the first read.  Every wave passes B(-1) ..
// B(nst - 2).
template <int WT, int EPI, int MTW, int RBW, int WN, int KC>
__global__ __launch_bounds__(64 * (TG_WM * WN + tile_loaders(WN))) void tile_gemm_kernel(
    TileArgs a) {
  using S = TgShape<WT, MTW, RBW, WN, KC>;
  extern __shared__ __attribute__((aligned(1024))) unsigned char tg_lds[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int wm = wv % TG_WM, wn = wv / TG_WM;

  // XCD-aware tile order: consecutive workgroups go to different XCDs, so tile t is run by
  // workgroup b with t = (b % 8) * (G / 8) + b / 8; neighbouring tiles (sharing X or W)
  // then run on one XCD and share its L2.
  const int G = gridDim.x;
  const int b = blockIdx.x;
  const int gt = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  // split-K (a.splits > 1): workgroup gt takes k-split gt / tiles of tile gt % tiles (the
  // workgroups of one split, which read the same X k-slice, neighbour each other) and writes
  // its fp32 sums into plane split of Y (reduced by tile_reduce_kernel)
  // re-tiling (a.pmt > 0): workgroup gt covers sub-tile gt % nsub of parent tile
  // tile0 + gt / nsub, whose m-tiles and row-blocks it splits in this shape's units
  const int sub_n = a.pmt ? a.prb / S::RB : 1;
  const int nsub = a.pmt ? (a.pmt / S::MT) * sub_n : 1;
  const int tiles = a.ntiles ? a.ntiles * nsub : a.tiles_m * a.tiles_n;   // of this launch
  const int sp = gt / tiles;
  const int job = gt - sp * tiles;
  // tile order in groups of TG_GROUP_M m-tile rows: consecutive tiles walk down a group's
  // rows, then across its columns, so the 32 tiles an XCD runs at once cover a 4 x 8
  // block (X of 4 row tiles, W of 8 column tiles) instead of 1 x 32 (W of 32): at large M
  // (the prompt-sized fc: 16 x 40 tiles, X 210 MB, W 262 MB) each XCD re-reads a quarter
  // of the weights per round instead of most of them.  One row tile: plain order.
  int tm, tn, mt0, nb0;   // first m-tile and weight row-block of this workgroup
  if (a.pmt) {
    const int su = job % nsub;
    tile_coords(a, a.tile0 + job / nsub, tm, tn);
    mt0 = tm * a.pmt + (su / sub_n) * S::MT;
    nb0 = tn * a.prb + (su % sub_n) * S::RB;
  } else {
    tile_coords(a, a.tile0 + job, tm, tn);
    mt0 = tm * S::MT;
    nb0 = tn * S::RB;
  }
  const int K = a.K;
  // this split's stages [st0, st0 + nst), in whole 64-k steps (an even number of k-blocks)
  const int npair = K / 64;
  const int st0 = (int)((long long)sp * npair / a.splits) * (64 / KC);
  const int nst = (int)((long long)(sp + 1) * npair / a.splits) * (64 / KC) - st0;
  const int MTt = (a.M + 31) >> 5;             // m-tiles present in X
  const int KBW = WT == WT_INT8 ? K / 32 : K / 16;   // weight blocks per row-block

  // copy i of a stage (X records first, then weight blocks) is issued by loader wave
  // i % NLOAD, or by compute wave i % NW
  constexpr int ISSUERS = S::LOADER ? S::NLOAD : S::NW;
  // iw: the issuing wave's index among the ISSUERS (a constant in each loader branch)
  auto issue_stage = [&](int ls, int iw) __attribute__((always_inline)) {
    unsigned char* buf = tg_lds + (ls % S::STAGES) * S::STAGE;
    const int s = st0 + ls;   // stage of K
#pragma unroll
    for (int j = 0; j < (S::IPS + ISSUERS - 1) / ISSUERS; ++j) {
      const int i = iw + ISSUERS * j;
      if (i < S::MT * S::XREC) {
        const int mtl = i / S::XREC, rec = i % S::XREC;
        const int mg = min(mt0 + mtl, MTt - 1);   // rows past M: any valid tile (never stored)
        const half_t* src =
            a.X + (size_t)mg * 32 * K + ((size_t)(S::XREC * s + rec) * 64 + lane) * 8;
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(buf + i * 1024), 16, 0, 0);
      } else if (i < S::IPS) {
        const int wi = i - S::MT * S::XREC;
        const int r = wi / S::WBLK, q = wi % S::WBLK;
        const uint4* src = a.W + ((size_t)(nb0 + r) * KBW + (size_t)S::WBLK * s + q) * 64 + lane;
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(buf + i * 1024), 16, 0, 0);
      }
    }
  };
  // before B(t): this wave's copies of stage t + 1 have landed; stages up to t + STAGES - 2
  // were issued, so STAGES - 3 of them may stay in flight (all landed near the end)
  auto wait_stage = [&](int t) __attribute__((always_inline)) {
    if (t + S::STAGES - 2 <= nst - 1) wait_vmcnt<(S::STAGES - 3) * S::PER_WAVE_MIN>();
    else wait_vmcnt<0>();
  };

  floatx16 acc[RBW][MTW][S::NACC];
  static_for<0, RBW>([&](auto r) {
    static_for<0, MTW>([&](auto t) {
      static_for<0, S::NACC>([&](auto c) { acc[r][t][c] = (floatx16){}; });
    });
  });

  if constexpr (S::LOADER) {
    if (wv >= S::NW) {
      // ---- loader waves: the copies and the waits; the compute waves only pass barriers ----
      auto load = [&](int iw) __attribute__((always_inline)) {
        for (int t = 0; t < S::STAGES - 2 && t < nst; ++t) issue_stage(t, iw);
        for (int t = -1; t <= nst - 2; ++t) {
          wait_stage(t);
          tg_barrier();   // B(t)
          if (t + S::STAGES - 1 < nst) issue_stage(t + S::STAGES - 1, iw);
        }
      };
      // one branch per loader, so each one's copy indexes are constants
      static_for<0, S::NLOAD>([&](auto j) {
        if (wv == S::NW + (int)j) load(j);
      });
      return;
    }
    tg_barrier();   // B(-1)
  } else {
    for (int t = 0; t < S::STAGES - 2 && t < nst; ++t) issue_stage(t, wv);
    wait_stage(-1);
    tg_barrier();   // B(-1)
    if (S::STAGES - 2 < nst) issue_stage(S::STAGES - 2, wv);
  }

  // k-blocks u = 0 .. nkb-1 of this split (local stage u / KBS); f0 / f1 alternate
  const int nkb = nst * S::KBS;
  TgFrag<WT, MTW, RBW> f0, f1;
  tg_read_frags<S>(f0, tg_lds, 0, wm, wn, lane);
  // before reading k-block u + 1: a new stage needs B(stage - 1) and refills
  auto next = [&](int u, TgFrag<WT, MTW, RBW>& f) __attribute__((always_inline)) {
    const int v = u + 1;
    const int sv = v / S::KBS;
    if (v % S::KBS == 0) {
      if constexpr (!S::LOADER) wait_stage(sv - 1);
      tg_barrier();   // B(sv - 1)
      if constexpr (!S::LOADER)
        if (sv - 1 + S::STAGES - 1 < nst) issue_stage(sv - 1 + S::STAGES - 1, wv);
    }
    tg_read_frags<S>(f, tg_lds + (sv % S::STAGES) * S::STAGE, v % S::KBS, wm, wn, lane);
  };
  if constexpr (WT == WT_INT8 && MTW >= 2) {
    // (with one m-tile the dequantisation outweighs the MFMAs; nothing to hide it under)
    half8_t d[2];
    dequant_i8x16(f0.w[0][0], d[0], d[1]);
    for (int u = 0; u < nkb; u += 2) {   // nkb is even (whole 64-k steps)
      next(u, f1);
      tg_mfma_i8<MTW, RBW, S::NACC>(f0, d, f1.w[0][0], acc);
      if (u + 2 < nkb) next(u + 1, f0);
      // after the last k-block this dequantises stale registers, never used
      tg_mfma_i8<MTW, RBW, S::NACC>(f1, d, f0.w[0][0], acc);
    }
  } else {
    for (int u = 0; u < nkb; u += 2) {   // nkb is even (whole 64-k steps)
      next(u, f1);
      tg_mfma<WT, MTW, RBW, S::NACC>(f0, acc);
      if (u + 2 < nkb) next(u + 1, f0);
      tg_mfma<WT, MTW, RBW, S::NACC>(f1, acc);
    }
  }

  // epilogue, rows m < M only.  Lane l holds, in register i of block (r, t), row
  // mbase(t) + 8*(i/4) + (i%4) and column n_lane + 32*r.
  const int g = lane >> 5;
  const int n_lane = (nb0 + wn * RBW) * 32 + (lane & 31);
  floatx16 v[RBW][MTW];
  static_for<0, RBW>([&](auto r) {
    static_for<0, MTW>([&](auto t) {
      v[r][t] = acc[r][t][0];
      if constexpr (S::NACC == 2) v[r][t] += acc[r][t][1];
    });
  });
  auto row_of = [&](int t, int i) __attribute__((always_inline)) {
    return (mt0 + wm * MTW + t) * 32 + 4 * g + 8 * (i >> 2) + (i & 3);
  };
  if constexpr (EPI == TG_F32 || EPI == TG_ARGMAX) {
    if (a.Y) {
      float* yplane = a.Y + (size_t)sp * a.M * a.ldy;
      static_for<0, MTW>([&](auto t) {
        static_for<0, RBW>([&](auto r) {
          float* yc = yplane + n_lane + 32 * r;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int m = row_of(t, i);
            if (m < a.M) yc[(size_t)m * a.ldy] = v[r][t][i];
          }
        });
      });
    }
  }
  if constexpr (EPI == TG_RESID) {
    // x += fp16(y * s) in place; row sums of squares of the new x per 32-column tile
    const int ncol = a.N >> 5;
    static_for<0, MTW>([&](auto t) {
      static_for<0, RBW>([&](auto r) {
        const int n = n_lane + 32 * r;
        const float s = h2f(a.scale[n]);
        float sq[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int m = row_of(t, i);
          sq[i] = 0.f;
          if (m < a.M) {
            half_t* xp = a.x + afl_index(m, n, a.N);
            const half_t xn = f2h(h2f(*xp) + h2f(f2h(v[r][t][i] * s)));
            *xp = xn;
            sq[i] = h2f(xn) * h2f(xn);
          }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
          for (int o = 16; o > 0; o >>= 1) sq[i] += __shfl_xor(sq[i], o, 64);
        if ((lane & 31) == 0) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int m = row_of(t, i);
            if (m < a.M) a.ss[((size_t)(m >> 5) * ncol + (n >> 5)) * 32 + (m & 31)] = sq[i];
          }
        }
      });
    });
  }
  if constexpr (EPI == TG_SWIGLU) {
    // packed gate|up: row-block 2j holds gate rows [32j, 32j+32), 2j+1 the matching up rows
    const int F = a.N >> 1;
    static_for<0, MTW>([&](auto t) {
      static_for<0, RBW / 2>([&](auto j) {
        const int ng = n_lane + 64 * j;
        const int f = (ng >> 6) * 32 + (lane & 31);
        const float sg = h2f(a.scale[ng]), su = h2f(a.scale[ng + 32]);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int m = row_of(t, i);
          if (m < a.M) {
            const float gv = h2f(f2h(v[2 * j][t][i] * sg));
            const float uv = h2f(f2h(v[2 * j + 1][t][i] * su));
            const float sig = h2f(f2h(1.0f / (1.0f + expf(-gv))));
            const float sil = h2f(f2h(gv * sig));
            a.out[afl_index(m, f, F)] = f2h(sil * uv);
          }
        }
      });
    });
  }
  if constexpr (EPI == TG_ARGMAX) {
    // per row: the wave's best column (increasing n, strict '>': lowest index on ties; NaN
    // never chosen), then the best of the 32 lanes as (order-preserving value << 32 |
    // ~index), stored in the wave column's own slot (no atomics: each row key would
    // otherwise take one atomic from every column tile)
    // (a sampling call ranks l / T + Gumbel noise instead of l)
    unsigned long long* part = a.keys + (size_t)(nb0 / RBW + wn) * a.M;
    const bool samp = a.samp_invT > 0.f;
    static_for<0, MTW>([&](auto t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float best = -INFINITY;
        int bn = -1;
        const uint32_t salt = samp ? gumbel_row_salt(a.samp_seed, row_of(t, i)) : 0u;
        static_for<0, RBW>([&](auto r) {
          const int n = n_lane + 32 * r;
          const float val = samp ? v[r][t][i] * a.samp_invT + gumbel_noise(salt, n) : v[r][t][i];
          if (val > best) {
            best = val;
            bn = n;
          }
        });
        unsigned long long key =
            bn < 0 ? 0ull
                   : ((unsigned long long)float_order_key(best) << 32) | (0xFFFFFFFFu - (uint32_t)bn);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
          const unsigned long long k2 = __shfl_xor(key, o, 64);
          key = k2 > key ? k2 : key;
        }
        const int m = row_of(t, i);
        if ((lane & 31) == 0 && m < a.M) part[m] = key;
      }
    });
  }
}

template <int WT, int EPI, int MTW, int RBW, int WN, int KC>
void launch_tile(const TileArgs& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  using S = TgShape<WT, MTW, RBW, WN, KC>;
  const int nsub = a.pmt ? (a.pmt / S::MT) * (a.prb / S::RB) : 1;
  const dim3 grid((a.ntiles ? a.ntiles * nsub : a.tiles_m * a.tiles_n) * a.splits),
      block(64 * (S::NW + S::NLOAD));
  if (e0 || e1)
    hipExtLaunchKernelGGL((tile_gemm_kernel<WT, EPI, MTW, RBW, WN, KC>), grid, block, S::LDS, st,
                          e0, e1, 0, a);
  else
    hipLaunchKernelGGL((tile_gemm_kernel<WT, EPI, MTW, RBW, WN, KC>), grid, block, S::LDS, st, a);
}

// The epilogues each weight type has: int8 F32 / RESID / SWIGLU (gate|up pairs), fp16 F32 /
// ARGMAX.  Shape I runs when `shape` is I, or (shape < 0) when it is the plan's.
template <int I>
bool launch_shape_i(int wt, int epi, const TileArgs& a, const TilePlan& p, hipStream_t st,
                    hipEvent_t e0, hipEvent_t e1, int shape = -1) {
  if constexpr (I < kNumTileShapes) {
    constexpr TileShape s = kTileShapes[I];
    if (wt == s.wt && (shape >= 0 ? shape == I
                                  : (!s.tail && p.mtw == s.mtw && p.rbw == s.rbw &&
                                     p.wn == s.wn && p.kc == s.kc))) {
      if (epi == TG_F32) {
        launch_tile<s.wt, TG_F32, s.mtw, s.rbw, s.wn, s.kc>(a, st, e0, e1);
        return true;
      }
      if constexpr (s.wt == WT_INT8) {
        if (epi == TG_RESID) {
          launch_tile<s.wt, TG_RESID, s.mtw, s.rbw, s.wn, s.kc>(a, st, e0, e1);
          return true;
        }
        if constexpr (s.rbw % 2 == 0)
          if (epi == TG_SWIGLU) {
            launch_tile<s.wt, TG_SWIGLU, s.mtw, s.rbw, s.wn, s.kc>(a, st, e0, e1);
            return true;
          }
      } else {
        if (epi == TG_ARGMAX) {
          launch_tile<s.wt, TG_ARGMAX, s.mtw, s.rbw, s.wn, s.kc>(a, st, e0, e1);
          return true;
        }
      }
      return false;
    }
    return launch_shape_i<I + 1>(wt, epi, a, p, st, e0, e1, shape);
  }
  return false;
}

}  // namespace

namespace {

// Sum of the split-K planes y[s][M][N] (s < S, fixed order) with the epilogue: TG_F32 into
// out_y [M][N], or TG_RESID (x += fp16(sum * scale), row sums of squares per 32 columns).
// One thread per column of a row; a wave covers 64 columns (two 32-column tiles).
__global__ __launch_bounds__(256) void tile_reduce_kernel(TileArgs a, const float* __restrict__ y,
                                                          int S, int epi) {
  const int lane = threadIdx.x & 63;
  const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int wpr = a.N >> 6;   // waves per row
  if (w >= (long long)a.M * wpr) return;
  const int m = (int)(w / wpr);
  const int n = (int)(w - (long long)m * wpr) * 64 + lane;
  const size_t plane = (size_t)a.M * a.N;
  const float* src = y + (size_t)m * a.N + n;
  float v = src[0];
  for (int s = 1; s < S; ++s) v += src[s * plane];
  if (epi == TG_F32) {
    a.Y[(size_t)m * a.ldy + n] = v;
    return;
  }
  half_t* xp = a.x + afl_index(m, n, a.N);
  const half_t xn = f2h(h2f(*xp) + h2f(f2h(v * h2f(a.scale[n]))));
  *xp = xn;
  float sq = h2f(xn) * h2f(xn);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
  if ((lane & 31) == 0) a.ss[((size_t)(m >> 5) * (a.N >> 5) + (n >> 5)) * 32 + (m & 31)] = sq;
}

}  // namespace

bool launch_tile_reduce(int epi, const TileArgs& a, const float* parts, int splits,
                        hipStream_t st, hipEvent_t ev_stop) {
  if (check_tile_reduce_args(epi, a, parts, splits)) return false;
  const long long waves = (long long)a.M * (a.N / 64);
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  if (ev_stop)
    hipExtLaunchKernelGGL(tile_reduce_kernel, grid, block, 0, st, nullptr, ev_stop, 0, a, parts,
                          splits, epi);
  else
    hipLaunchKernelGGL(tile_reduce_kernel, grid, block, 0, st, a, parts, splits, epi);
  return true;
}

bool launch_tile_gemm(int wt, int epi, const TileArgs& a0, const TilePlan& p, hipStream_t st,
                      hipEvent_t ev_start, hipEvent_t ev_stop) {
  if (check_tile_args(wt, epi, a0, p)) return false;
  TileArgs a = a0;
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  a.splits = p.splits;
  a.tile0 = a.ntiles = a.pmt = a.prb = 0;
  if (p.tail_shape < 0) return launch_shape_i<0>(wt, epi, a, p, st, ev_start, ev_stop);
  // the head tiles in whole rounds, then the tail tiles re-tiled on the smaller shape
  a.ntiles = p.head_tiles;
  if (!launch_shape_i<0>(wt, epi, a, p, st, ev_start, nullptr)) return false;
  a.tile0 = p.head_tiles;
  a.ntiles = p.tiles_m * p.tiles_n - p.head_tiles;
  a.pmt = TG_WM * p.mtw;
  a.prb = p.rbw * p.wn;
  return launch_shape_i<0>(wt, epi, a, p, st, nullptr, ev_stop, p.tail_shape);
}

}  // namespace dfl
