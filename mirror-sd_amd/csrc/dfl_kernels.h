// Internal kernel launch interface shared by the .hip translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dfl_common.h"

namespace dfl {

enum { WT_INT8 = 0, WT_F16 = 1 };
// EPI_QKROPE: the fused q|k|v projection of one sequence (M <= 32 rows) with the per-head
// Q/K RMSNorm, RoPE and cache scatter of qk_rope_kernel done in the epilogue (RopeEpi).
enum { EPI_SWIGLU = 1, EPI_ARGMAX = 2, EPI_STORE = 3, EPI_RESID = 4, EPI_QKROPE = 5 };

struct RopeSeq {
  long long pos0;
  half_t* Kc;
  half_t* Vt;
  int cache_row0, sink_fill, ring_j0, ring_S, ring_W;
};

// EPI_QKROPE outputs: Q [NH][M][128], the K cache rows and the Vt cache columns of the
// sequence's rows (positions sq.pos0 + m, cache rows through cache_slot).
constexpr int QK_N_MAX = 16384;   // QKROPE: most q|k|v rows (the scales' LDS copy)
struct RopeEpi {
  half_t* Q;
  const float* cs;          // [M][64] (cos, sin) of position pos0 + m, frequency j (embed_norm)
  const half_t* q_norm;
  const half_t* k_norm;
  float eps;
  double log2_theta;
  int NH, NKV, cap;
  RopeSeq sq;
};


// ---- stream-K weight-streaming GEMM for M <= 32 rows (dfl_stream.hip) ----
constexpr int MAX_FEATS = 16;   // tapped target layers (FeatPtrs, StreamArgs::xr_p)

struct StreamArgs {
  const uint4* W;           // packed weight blocks, N rows (multiple of 64)
  const half_t* scale;      // [N] per packed row (int8) or nullptr
  int N, KB;                // KB = K/32 (int8) or K/16 (fp16)
  const half_t* X;          // activations: one 32-row tile in the fragment layout (afl_offset)
  int ldx, M;
  // Row-major activations instead of X (xr_n > 0: the per-step ingest fc, fp16 weights,
  // one m-tile): element (m, k) is xr_p[k / xr_h][m * xr_ld + k % xr_h], i.e. feature j of
  // the tapped layers gives columns [j * xr_h, (j + 1) * xr_h), read in place; rows >= M
  // are zero.  Every xr_p[j] 16-byte aligned, xr_ld % 8 == 0, xr_h % 16 == 0, xr_h >= 64.
  const half_t* xr_p[MAX_FEATS];
  long long xr_ld;
  int xr_n, xr_h;
  int MT;                   // M-split kernel: 32-row m-tiles of X (M <= 32 * MT)
  const float* rnorm;       // NORM: per-row 1/rms of X (used when ss_in is null)
  const float* ss_in;       // NORM: [ss_tiles][32] row sums of squares of X (RESID output)
  int ss_tiles, ss_n;       //       tiles of ss_in, and the row length they sum over
  int ss_mstride;           // floats from one m-tile's ss_in / ss_part block to the next
  const half_t* gnorm;      // NORM: [K] gain (K <= 8192)
  float* ws;                // [N/64][seg_cap][2048] partials of tiles split across workgroups
  int seg_cap;
  int* tile_cnt;            // [N/64] arrival counters (zero-initialised, self-resetting)
  half_t* out;              // STORE: row-major [M][ldo] fp16; SWIGLU: fragment-layout tile [32][N/2]
  int ldo;
  half_t* x;                // RESID: residual stream, fragment-layout tile [32][N], updated in place
  int x_zero;               // RESID: x is taken as zero and not read (x = fp16(y * s): a Linear
                            // output in fragment layout with its per-tile row sums of squares)
  float* ss_part;           // RESID: [N/64][32] per-tile row sums of squares of the updated x
  float eps;
  float* logits;            // ARGMAX: optional [M][ldl] fp32
  int ldl;
  unsigned long long* keys; // ARGMAX: optional [M] packed (order(value) << 32 | ~index)
  // balanced mode (SKPlan::dyn_static > 0): workgroup b first takes the whole tiles
  // [b * dyn_static, (b + 1) * dyn_static), then half tiles of the remaining tiles from the
  // work counter dyn_next[0]; dyn_next[1] counts finished workgroups (both zero between
  // launches: the last workgroup resets them)
  int dyn_static;
  int* dyn_next;
  int* err;                 // device error word (bit 2: a work-queue wait gave up)
  int32_t* ids;             // balanced ARGMAX: the last workgroup turns keys [M] into ids [M]
                            // (-1 for a row without a number) and re-arms keys to zero
  int dp;                   // hybrid plan (SKPlan::dp): whole tiles per workgroup
  int dyn_test_timeout;     // balanced mode: force the work-queue wait to give up (test hook)
  RopeEpi rope;             // EPI_QKROPE
  // ARGMAX as a categorical sample (Gumbel-max, gumbel_noise): samp_invT = 1 / temperature
  // (0: plain argmax), samp_seed the call's seed, samp_row0 the first row's index for the noise
  float samp_invT;
  uint32_t samp_seed;
  int samp_row0;
};
struct SKPlan {
  int workers = 1;          // workgroups (one per CU)
  int seg_cap = 1;          // workspace slots per tile (contiguous partition)
  int dyn_static = 0;       // > 0: balanced mode with this many whole tiles per workgroup
  int dp = 0;               // > 0: hybrid plan, whole tiles per workgroup after the split
                            // units of the first N/64 - dp * workers tiles
  int sk_seg_cap = 0;       // hybrid plan: workspace slots per split tile
};
// streamk_plan / streamk_plan_balanced (the partition of a matrix over the CUs) are in
// dfl_sk_plan.h.
// M-split variant for 2 <= MT <= 8 m-tiles (M <= 256 rows): every weight block is read
// once for all m-tiles.  X, out, x, ss_*, rnorm, logits, keys point at m-tile 0; m-tile mt
// is 32*mt rows further (ss blocks ss_mstride floats further).  ws holds
// [N/64][seg_cap][MT][2048] floats.
// Both launchers return false (and launch nothing) for a weight type / epilogue pair
// they have no kernel for.
bool launch_streamk_gemm_m(int wt, int epi, bool norm, const StreamArgs& a, const SKPlan& p,
                           hipStream_t st, hipEvent_t ev_start = nullptr,
                           hipEvent_t ev_stop = nullptr);
// ev_start / ev_stop (optional) receive the kernel's own start and end timestamps.
bool launch_streamk_gemm(int wt, int epi, bool norm, const StreamArgs& a, const SKPlan& p,
                         hipStream_t st, hipEvent_t ev_start = nullptr,
                         hipEvent_t ev_stop = nullptr);

// ---- tile GEMM for stacked rows, M > 64 (dfl_tile.hip) ----
// Y[M][ldy] (fp32, columns [0, N)) = X . W^T with X in the activation fragment layout
// (ceil(M/32) tiles of 32 x K) and W packed blocks (int8: unscaled integer-weight sums).
// Tile GEMM epilogues: TG_F32 stores Y; TG_RESID, TG_SWIGLU and TG_ARGMAX do what the
// stream-K RESID / SWIGLU / ARGMAX epilogues do (same arithmetic and rounding points), with
// RESID's row sums of squares per 32-column tile.
enum { TG_F32 = 0, TG_RESID = 1, TG_SWIGLU = 2, TG_ARGMAX = 3 };
struct TileArgs {
  const uint4* W;           // packed weight blocks, N rows
  int N, K;                 // N % (32 * rb) == 0, K % 64 == 0
  const half_t* X;          // fragment-layout tiles, ceil(M/32) of them
  int M;
  float* Y;                 // TG_F32 (and optionally TG_ARGMAX): row-major fp32 [M][ldy]
  int ldy;
  const half_t* scale;      // RESID / SWIGLU: [N] per-row scales of the int8 weights
  half_t* x;                // RESID: fragment-layout residual [M][N], updated in place
  float* ss;                // RESID: [ceil(M/32)][N/32][32] row sums of squares of the new x
  half_t* out;              // SWIGLU: fragment-layout act [M][N/2] (N in packed gate|up order)
  unsigned long long* keys; // ARGMAX: [N/32/rbw][M] per-wave-column best keys (packed
                            // order(value) << 32 | ~index, 0 = none), reduced by
                            // launch_argmax_parts
  int tiles_m, tiles_n;     // set by the launcher from the plan
  int splits;               // split-K: F32 sums of split s into plane s of Y ([splits][M][ldy])
  // Tile range of the launch: tiles [tile0, tile0 + ntiles) of the plan's order (ntiles ==
  // 0: every tile).  With pmt > 0 the launch re-tiles them: each of those (parent) tiles of
  // pmt m-tiles x prb row-blocks is covered by workgroups of the launch's smaller shape.
  int tile0, ntiles;
  int pmt, prb;
  float samp_invT;          // ARGMAX: categorical sample at temperature 1 / samp_invT (0: argmax)
  uint32_t samp_seed;
};
struct TilePlan {
  int mtw = 0;              // m-tiles per wave: 1 (128-row workgroup tile) or 2 (256 rows)
  int rbw = 0;              // weight row-blocks (32 columns) per wave: 1, 2 or 4
  int wn = 0;               // wave columns: 1 (4 waves) or 2 (8 waves)
  int kc = 0;               // k per LDS stage: 32 or 64
  int tiles_m = 0, tiles_n = 0;
  int splits = 1;           // split-K factor (F32 planes, then launch_tile_reduce)
  // tail re-tiling: the first head_tiles tiles run in full rounds of the CUs; the rest (a
  // partial last round) run on the smaller shape tail_shape (an index of kTileShapes),
  // several workgroups per tile, each over the whole K, so the sums are unchanged
  int head_tiles = 0;
  int tail_shape = -1;
};
// (tile_plan / tile_lds_bytes: dfl_tile_plan.h)
// The split-K planes parts [splits][M][N] summed in plane order, with epilogue TG_F32 (into
// a.Y, row stride a.ldy) or TG_RESID (a.x, a.ss, a.scale as the RESID epilogue).  Returns
// false (and launches nothing) when the arguments fail check_tile_reduce_args.
bool launch_tile_reduce(int epi, const TileArgs& a, const float* parts, int splits,
                        hipStream_t st, hipEvent_t ev_stop = nullptr);
// Returns false (and launches nothing) when the arguments fail check_tile_args.
// ev_start / ev_stop (optional) receive the kernel's own start and end timestamps.
bool launch_tile_gemm(int wt, int epi, const TileArgs& a, const TilePlan& p, hipStream_t st,
                      hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);

// ---- pack / quantise (dfl_pack.hip) ----
// Symmetric per-row int8 quantisation of w [oc][ic] fp32.
void launch_quantize_w8(const float* w, int64_t oc, int64_t ic, int8_t* q, half_t* s,
                        hipStream_t st);
// int8 [rows][K] row-major (+ fp16 scales) -> packed blocks. Source row-block i goes to
// destination row-block rb0 + i*rb_step of a matrix with KB = K/32 k-blocks.
void launch_pack_i8(const int8_t* q, const half_t* s, int rows, int K, uint4* dst,
                    half_t* dst_scale, int rb0, int rb_step, hipStream_t st);
// fp16 [rows][K] row-major -> packed blocks (KB = K/16).
void launch_pack_f16(const half_t* w, int rows, int K, uint4* dst, hipStream_t st);

// ---- row kernels (dfl_rows.hip) ----
// x[b] = ids ? embed[ids[b]] : noise[b] (x in the activation fragment layout, K = H);
// rnorm[b] = 1/rms(x[b]); optionally
// h[b] = RMSNorm(x[b]) * g.  An id outside [0, V) yields a zero row and sets *err |= 1.
// Block embedding rows (generate.py:594-597) with an optional soft anchor in row 0
// (generate.py:1419-1437); logits_dtype 0 fp32, 1 fp16, 2 bf16; cand holds
// SA_BLOCKS * SA_TOPK_MAX keys.  err bit 0: token id out of range; bit 1: logits all NaN.
constexpr int SA_TOPK_MAX = 8, SA_BLOCKS = 64;
void launch_embed_block(const int32_t* ids, int B, const half_t* embed, int Vemb, int H,
                        const void* logits, int logits_dtype, int V, int top_k,
                        unsigned long long* cand, half_t* out, int* err, hipStream_t st);
// Feature tensors of the tapped target layers: p[j] -> [rows][ld] fp16 (first H columns
// used), 16-byte aligned, ld % 8 == 0.
struct FeatPtrs {
  const half_t* p[MAX_FEATS];
  int n;
  long long ld;
};
void launch_concat_feats(const FeatPtrs& f, int rows, int H, half_t* out, hipStream_t st);
// hidden_norm of the fp32 fc rows (rounded to fp16 first) into fragment-layout tiles xn.
void launch_fc_norm_rows(const float* fc32, int rows, int H, const half_t* g, float eps,
                         half_t* xn, hipStream_t st);
// Stream-K ingest inputs: concat_j(f_j) rows (f.n features of H columns, H % 8 == 0) into
// activation fragment layout tiles [ceil(rows/32)][32][f.n*H], padding rows zero.
void launch_feats_to_afl(const FeatPtrs& f, int rows, int H, half_t* afl, hipStream_t st);
void launch_embed_norm(const int32_t* ids, const half_t* embed, const half_t* noise, int B,
                       int H, int V, const half_t* g, float eps, half_t* x, half_t* h,
                       float* rnorm, int* err, hipStream_t st,
                       float* rope_cs = nullptr, long long pos0 = 0, double log2_theta = 0.0,
                       const double* inv_freq = nullptr);
// A layer's cache set to L rows in the reference's row order: k and v are [NKV][L][128] fp16
// (DFlashKVCache.keys / .values of one sequence, [1, NKV, L, D]); row r of the source goes to
// cache row dst_row(r) = r for r < keep_head, else r - (L - keep_tail) + keep_head for the
// last keep_tail rows (the rows between are dropped: a sink + window cache keeps its first
// keep_head = sink rows and its newest keep_tail = window rows); k -> Kc rows, v -> Vt
// columns.  Either of k / v may be null.
void launch_cache_assign(const half_t* k, const half_t* v, int NKV, int L, int keep_head,
                         int keep_tail, half_t* Kc, half_t* Vt, int cap, hipStream_t st);
// x in the activation fragment layout (afl_index) [M][N] -> h [M][N], row-major or (h_afl)
// fragment layout: h = fp16(fp16(x * r[m]) * g[n])  (apply_norm), or a plain row-major copy
// (afl_to_rows).  r[m] = 1/rms of row m from ss [M/32 m-tiles][ss_tiles][32] (row sums of
// squares per column tile), or rnorm[m].
void launch_apply_norm(const half_t* x, const float* ss, int ss_tiles, float eps, const half_t* g,
                       int M, int N, half_t* h, hipStream_t st, const float* rnorm = nullptr,
                       bool h_afl = false);
void launch_afl_to_rows(const half_t* x, int M, int N, half_t* h, hipStream_t st);
// Up to SEQ_MAX sequences (batched drafting) share one rope / attention launch.
constexpr int SEQ_MAX = 8;

// Where one sequence's rows go: absolute position of its first row and its K/V cache
// (K [NKV][cap][128], Vt [NKV][128][cap]).  Without a window (ring_W == 0) row m goes to
// cache row cache_row0 + m.  With a sink + window cache (ring_W > 0) the first sink_fill
// rows go to cache_row0 + m (filling the sink) and later ones to ring row
// ring_S + ((ring_j0 + m - sink_fill) mod ring_W).

// Per-head RMSNorm + neox RoPE + scatter of projections: fp16 qkv16 (scaled and rounded by
// the GEMM epilogue) or fp32 qkv32 (scaled and rounded here), rows [n_seq * M][N], sequence
// s owning rows s*M .. s*M + M - 1, its row m at position sq[s].pos0 + m.  Head slots
// [0, NH) -> Q[s][h][m][d] ([n_seq][NH][M][128]); slots [NH, NH+NKV) -> K cache rows;
// [NH+NKV, NH+2NKV) -> Vt cache columns.  Column 0 is head slot col_slot0 (so the ingest
// path can project only K and V).
struct QKRopeArgs {
  const half_t* qkv16;                       // projection rows, fp16 (scaled), or
  const float* qkv32; const half_t* oscale;  // fp32 GEMM rows + fp16 scale per column
  int M; int N;                              // rows per sequence, columns
  int n_seq;
  int col_slot0;                             // head slot of column 0
  int slot0, n_slots;                        // head slots handled (q,k,v numbering)
  int NH, NKV;
  const half_t* q_norm; const half_t* k_norm; float eps;
  double log2_theta;
  const double* inv_freq;                    // [64] scaled RoPE frequencies, or nullptr:
                                             // theta^(-j/64) from log2_theta
  const float* cs;                           // [M][64] (cos, sin) of row m's position, made by
                                             // launch_rope_table (entries sharing positions),
                                             // or nullptr: computed per row and head
  half_t* Q;
  int cap;
  RopeSeq sq[SEQ_MAX];
  // layer mode (layer_cols > 0): the entries are layers of one sequence sharing the rows;
  // entry s reads columns [s * layer_cols, ...) of each row (N is the row stride) and uses
  // the k_norm gain k_norm_s[s]
  int layer_cols;
  const half_t* k_norm_s[SEQ_MAX];
};
// -1: a ring row that a later row of the same launch overwrites (more than ring_W ring
// rows appended at once keep only the newest ring_W), so it is not written at all
DFL_DEV int cache_slot(const RopeSeq& q, int M, int m) {
  if (q.ring_W == 0 || m < q.sink_fill) return q.cache_row0 + m;
  if (m - q.sink_fill < M - q.sink_fill - q.ring_W) return -1;
  return q.ring_S + (q.ring_j0 + (m - q.sink_fill)) % q.ring_W;
}
// Returns false (and launches nothing) when the struct fails check_qk_rope_args.
bool launch_qk_rope(const QKRopeArgs& a, hipStream_t st);
// cs[m][j] = (cos, sin) of (pos0 + m) * inv_freq[j] (fp64 angle, as qk_rope_kernel computes
// it), for m < M, j < 64; inv_freq nullptr: theta^(-j/64) from log2_theta.
void launch_rope_table(int M, long long pos0, double log2_theta, const double* inv_freq,
                       float* cs, hipStream_t st);
// ids[m] = ~low32(keys[m]); keys[m] = 0.
void launch_argmax_finalize(unsigned long long* keys, int M, int32_t* ids, hipStream_t st);
// ids[m] from the largest of parts[p][m], p < P (the tile GEMM's ARGMAX keys); -1 if none.
void launch_argmax_parts(const unsigned long long* parts, int P, int M, int32_t* ids,
                         hipStream_t st);

// ---- attention (dfl_attn.hip) ----
// One sequence of an attention launch: its cache, key range and output rows.
// Sink + window cache (ring_W > 0): keys [0, ring_S) valid below sink_len; key ring_S + p
// valid when (ring_j - 1 - p) mod ring_W < ring_len (the ring_len newest ring rows).
struct AttnSeq {
  const half_t* Kc;       // [NKV][cap][128]
  const half_t* Vt;       // [NKV][128][cap]
  int L;                  // number of valid keys
  int chunk;              // keys per split (multiple of 32)
  int n_chunks;
  int o_row0;             // first output row in O
  int ring_S, ring_W, ring_j, ring_len, sink_len;
};
struct AttnArgs {
  const half_t* Q;        // [n_seq][NH][B][128]
  int B, NH, NKV, cap;
  int n_seq, max_chunks;  // max_chunks = max over the sequences of n_chunks
  // grid x enumerates the chunks of all sequences: sequence s owns [chunk0[s], chunk0[s+1])
  int chunk0[SEQ_MAX + 1];
  int q_per_group, kw;    // set by the launcher: query tiles per workgroup, waves per tile
  int n_cu;
  int lds_max;            // the device's LDS bytes per workgroup (two stage buffers need 160 KiB)
  float scale_log2;       // head_dim^-0.5 * log2(e)
  float* Op;              // [max_chunks][n_seq*NH*B][128] unnormalised partial outputs
  float* Ml;              // [max_chunks][n_seq*NH*B][2] running (max, sum) in log2 domain
  half_t* O;              // output rows of an activation fragment layout tile set with
                          // NH*128 columns
  AttnSeq sq[SEQ_MAX];
};
// Returns false (and launches nothing) when the struct fails check_attn_args.
bool launch_block_attention(const AttnArgs& a, hipStream_t st);

}  // namespace dfl
