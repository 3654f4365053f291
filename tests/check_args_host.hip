// Host test of the launch-argument checks (dfl_check.h): one valid struct per launcher,
// then one rule broken at a time; prints "ok" or the failing case.  Built and run by
// tests/test_host.py::test_launch_argument_checks (no GPU needed).
#include <cstdio>
#include <cstring>

#include "dfl_check.h"
#include "dfl_sk_plan.h"
#include "dfl_tile_plan.h"

using namespace dfl;

static int fails = 0;
static void expect(const char* got, const char* needle, const char* what) {
  const bool ok = needle ? (got && std::strstr(got, needle)) : !got;
  if (!ok) {
    std::printf("FAIL %s: got '%s', want '%s'\n", what, got ? got : "(accepted)",
                needle ? needle : "(accepted)");
    ++fails;
  }
}

int main() {
  alignas(16) static char dummy[64];
  void* P = dummy;
  StreamArgs a{};
  a.W = (const uint4*)P; a.scale = (const half_t*)P; a.N = 5120; a.KB = 160;
  a.X = (const half_t*)P; a.ldx = 5120; a.M = 32; a.MT = 1; a.ws = (float*)P; a.seg_cap = 3;
  a.tile_cnt = (int*)P; a.x = (half_t*)P; a.ss_part = (float*)P; a.out = (half_t*)P; a.ldo = 5120;
  SKPlan p{};
  p.workers = 240;
  a.gnorm = (const half_t*)P; a.ss_in = (const float*)P; a.ss_tiles = 80; a.ss_n = 5120;
  expect(check_stream_args(WT_INT8, EPI_RESID, false, a, p, false), nullptr, "valid RESID");
  expect(check_stream_args(WT_INT8, EPI_STORE, true, a, p, false), nullptr, "valid STORE+norm");
  { StreamArgs b = a; b.M = 33; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, false), "m-tiles", "M > 32"); }
  { StreamArgs b = a; b.M = 65; b.MT = 2; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, true), "m-tiles", "M > 32 MT"); }
  { StreamArgs b = a; b.N = 5000; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, false), "multiple of 64", "N"); }
  { StreamArgs b = a; b.KB = 2; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, false), "k-blocks", "KB"); }
  { StreamArgs b = a; b.scale = nullptr; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, false), "scales", "scale"); }
  { StreamArgs b = a; b.x = nullptr; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, false), "RESID", "x"); }
  { StreamArgs b = a; b.out = nullptr; expect(check_stream_args(WT_INT8, EPI_STORE, false, b, p, false), "STORE", "out"); }
  { StreamArgs b = a; b.ldo = 100; expect(check_stream_args(WT_INT8, EPI_STORE, false, b, p, false), "STORE", "ldo"); }
  { StreamArgs b = a; b.gnorm = nullptr; expect(check_stream_args(WT_INT8, EPI_SWIGLU, true, b, p, false), "gain", "gain"); }
  { StreamArgs b = a; b.ss_in = nullptr; b.rnorm = nullptr; expect(check_stream_args(WT_INT8, EPI_SWIGLU, true, b, p, false), "row sums", "rows"); }
  { StreamArgs b = a; b.ss_tiles = 200; expect(check_stream_args(WT_INT8, EPI_SWIGLU, true, b, p, false), "tiles", "ss tiles"); }
  { StreamArgs b = a; expect(check_stream_args(WT_INT8, EPI_ARGMAX, false, b, p, false), "ARGMAX", "argmax int8"); }
  { StreamArgs b = a; b.keys = nullptr; b.logits = nullptr; expect(check_stream_args(WT_F16, EPI_ARGMAX, false, b, p, false), "ARGMAX", "argmax outputs"); }
  { StreamArgs b = a; expect(check_stream_args(WT_INT8, EPI_QKROPE, true, b, p, false), "QKROPE", "qkrope rows"); }
  { StreamArgs b = a; b.dp = 2; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, false), "hybrid", "dp"); }
  { StreamArgs b = a; SKPlan q = p; q.dyn_static = 2; expect(check_stream_args(WT_F16, EPI_STORE, false, b, q, false), "balanced", "dyn"); }
  { StreamArgs b = a; b.ws = nullptr; expect(check_stream_args(WT_INT8, EPI_RESID, false, b, p, false), "workspace", "ws"); }
  { StreamArgs b = a; b.x_zero = 1; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), nullptr, "x_zero RESID"); }
  { StreamArgs b = a; b.x_zero = 1; expect(check_stream_args(WT_INT8, EPI_STORE, false, b, p, false), "x_zero", "x_zero STORE"); }
  {   // the per-step ingest fc reading row-major feature rows in place (5 features x 5120
      // columns = KB 1600 of 16 columns)
    StreamArgs r = a;
    r.X = nullptr; r.KB = 1600; r.x_zero = 1; r.xr_n = 5; r.xr_h = 5120; r.xr_ld = 5120;
    for (int j = 0; j < 5; ++j) r.xr_p[j] = (const half_t*)P;
    expect(check_stream_args(WT_F16, EPI_RESID, false, r, p, false), nullptr, "row-major fc");
    { StreamArgs b = r; b.xr_n = 0; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), "null activations", "row-major off, no X"); }
    { StreamArgs b = r; b.xr_n = MAX_FEATS + 1; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), "count", "xr_n range"); }
    { StreamArgs b = r; expect(check_stream_args(WT_F16, EPI_STORE, false, b, p, false), "one-tile fp16 RESID", "row-major STORE"); }
    { StreamArgs b = r; expect(check_stream_args(WT_F16, EPI_RESID, true, b, p, false), "one-tile fp16 RESID", "row-major norm"); }
    { StreamArgs b = r; b.M = 64; b.MT = 2; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, true), "one-tile fp16 RESID", "row-major m-split"); }
    { StreamArgs b = r; b.xr_h = 5112; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), "tile the K axis", "xr_h % 16"); }
    { StreamArgs b = r; b.xr_n = 4; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), "tile the K axis", "features short of K"); }
    { StreamArgs b = r; b.xr_ld = 5116; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), "row stride", "xr_ld"); }
    { StreamArgs b = r; b.xr_p[3] = (const half_t*)(dummy + 2); expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), "aligned", "xr_p alignment"); }
    { StreamArgs b = r; b.xr_p[4] = nullptr; expect(check_stream_args(WT_F16, EPI_RESID, false, b, p, false), "aligned", "xr_p null"); }
  }
  { StreamArgs b = a; expect(check_stream_args(7, EPI_RESID, false, b, p, false), "weight type", "wt"); }
  { StreamArgs b = a; expect(check_stream_args(WT_INT8, 42, false, b, p, false), "epilogue", "epi"); }

  {   // the fused qkv launch (QKROPE) keeps the contiguous partition at every CU count,
      // also where the plan has whole tiles per workgroup (dp > 0): 27B qkv (112 tiles) on
      // <= 112 CUs, or 128 q|k|v heads (256 tiles) on 256 CUs
    StreamArgs r = a;
    r.N = 7168; r.KB = 160; r.scale = (const half_t*)P;
    r.rope.NH = 40; r.rope.NKV = 8; r.rope.Q = (half_t*)P; r.rope.cs = (const float*)P;
    r.rope.q_norm = (const half_t*)P; r.rope.k_norm = (const half_t*)P;
    r.rope.sq.Kc = (half_t*)P; r.rope.sq.Vt = (half_t*)P; r.rope.cap = 4128;
    const int heads[][2] = {{40, 8}, {32, 8}, {96, 16}};
    const int cus[] = {32, 64, 80, 104, 112, 200, 256, 304};
    for (const auto& hk : heads)
      for (int ncu : cus) {
        StreamArgs b = r;
        b.rope.NH = hk[0]; b.rope.NKV = hk[1]; b.N = (hk[0] + 2 * hk[1]) * 128;
        const SKPlan sp = streamk_plan(b.N, b.KB, ncu);
        b.dp = streamk_launch_dp(sp, EPI_QKROPE, false);
        b.seg_cap = b.dp > 0 ? sp.sk_seg_cap : sp.seg_cap;
        char what[96];
        std::snprintf(what, sizeof what, "QKROPE launch %d/%d heads on %d CUs", hk[0], hk[1], ncu);
        if (b.dp != 0) expect("dp > 0", nullptr, what);
        expect(check_stream_args(WT_INT8, EPI_QKROPE, true, b, sp, false), nullptr, what);
        // the other epilogues take the hybrid plan whenever it has whole tiles
        if (streamk_launch_dp(sp, EPI_STORE, false) != sp.dp) expect("store dp", nullptr, what);
        if (streamk_launch_dp(sp, EPI_STORE, true) != 0) expect("m-split dp", nullptr, what);
      }
    { StreamArgs b = r; b.dp = 1; SKPlan sp = streamk_plan(7168, 160, 64); b.seg_cap = sp.sk_seg_cap;
      expect(check_stream_args(WT_INT8, EPI_QKROPE, true, b, sp, false), "QKROPE", "QKROPE with dp > 0"); }
  }

  QKRopeArgs q{};
  q.qkv16 = (const half_t*)P; q.M = 32; q.N = 7168; q.n_seq = 1; q.col_slot0 = 0; q.slot0 = 0;
  q.n_slots = 56; q.NH = 40; q.NKV = 8; q.q_norm = (const half_t*)P; q.k_norm = (const half_t*)P;
  q.Q = (half_t*)P; q.cap = 4128; q.sq[0].Kc = (half_t*)P; q.sq[0].Vt = (half_t*)P;
  expect(check_qk_rope_args(q), nullptr, "valid rope");
  { QKRopeArgs b = q; b.qkv32 = (const float*)P; expect(check_qk_rope_args(b), "exactly one", "both inputs"); }
  { QKRopeArgs b = q; b.qkv16 = nullptr; expect(check_qk_rope_args(b), "exactly one", "no input"); }
  { QKRopeArgs b = q; b.qkv16 = nullptr; b.qkv32 = (const float*)P; expect(check_qk_rope_args(b), "scales", "fp32 no scale"); }
  { QKRopeArgs b = q; b.Q = nullptr; expect(check_qk_rope_args(b), "Q output", "no Q"); }
  { QKRopeArgs b = q; b.n_slots = 57; expect(check_qk_rope_args(b), "slots", "slots"); }
  { QKRopeArgs b = q; b.N = 2048; expect(check_qk_rope_args(b), "row width", "width"); }
  { QKRopeArgs b = q; b.n_seq = 9; expect(check_qk_rope_args(b), "range", "n_seq"); }
  { QKRopeArgs b = q; b.sq[0].Kc = nullptr; expect(check_qk_rope_args(b), "cache", "cache"); }
  { QKRopeArgs b = q; b.Q = nullptr; b.col_slot0 = 40; b.slot0 = 40; b.n_slots = 16; b.N = 2048; expect(check_qk_rope_args(b), nullptr, "valid K|V only"); }
  {   // layer mode: 5 layers' K|V rows side by side
    QKRopeArgs b = q; b.Q = nullptr; b.col_slot0 = 40; b.slot0 = 40; b.n_slots = 16; b.N = 5 * 2048;
    b.n_seq = 5; b.layer_cols = 2048;
    for (int i = 0; i < 5; ++i) { b.k_norm_s[i] = (const half_t*)P; b.sq[i].Kc = (half_t*)P; b.sq[i].Vt = (half_t*)P; }
    expect(check_qk_rope_args(b), nullptr, "valid layer mode");
    { QKRopeArgs c = b; c.N = 4 * 2048; expect(check_qk_rope_args(c), "row width", "layer mode width"); }
    { QKRopeArgs c = b; c.k_norm_s[3] = nullptr; expect(check_qk_rope_args(c), "k_norm", "layer mode norm"); }
    { QKRopeArgs c = b; c.slot0 = 0; c.col_slot0 = 0; c.n_slots = 56; c.Q = (half_t*)P;
      expect(check_qk_rope_args(c), "K|V rows only", "layer mode Q"); }
    { QKRopeArgs c = b; c.cs = (const float*)P; c.sq[2].pos0 = 99;   // layers share the rows
      expect(check_qk_rope_args(c), nullptr, "layer mode angle table"); }
  }
  {   // one angle table only for sequences at the same positions
    QKRopeArgs b = q; b.n_seq = 2; b.sq[1] = b.sq[0]; b.cs = (const float*)P;
    expect(check_qk_rope_args(b), nullptr, "angle table, same positions");
    b.sq[1].pos0 += 32;
    expect(check_qk_rope_args(b), "angle table", "angle table, other positions");
  }

  AttnArgs t{};
  t.Q = (const half_t*)P; t.B = 32; t.NH = 40; t.NKV = 8; t.cap = 4128; t.n_seq = 1;
  t.max_chunks = 26; t.chunk0[0] = 0; t.chunk0[1] = 26; t.Op = (float*)P; t.Ml = (float*)P;
  t.O = (half_t*)P; t.sq[0].Kc = (const half_t*)P; t.sq[0].Vt = (const half_t*)P; t.sq[0].L = 4128;
  t.sq[0].chunk = 160; t.sq[0].n_chunks = 26;
  expect(check_attn_args(t), nullptr, "valid attention");
  { AttnArgs b = t; b.sq[0].chunk = 150; expect(check_attn_args(b), "chunks", "chunk not 32x"); }
  { AttnArgs b = t; b.sq[0].n_chunks = 25; b.chunk0[1] = 25; b.max_chunks = 25; expect(check_attn_args(b), "chunks", "chunks short"); }
  { AttnArgs b = t; b.chunk0[1] = 20; expect(check_attn_args(b), "table", "chunk table"); }
  { AttnArgs b = t; b.sq[0].L = 5000; expect(check_attn_args(b), "keys", "L > cap"); }
  { AttnArgs b = t; b.NH = 41; expect(check_attn_args(b), "head counts", "ratio"); }
  { AttnArgs b = t; b.O = nullptr; expect(check_attn_args(b), "buffers", "no output"); }
  { AttnArgs b = t; b.max_chunks = 65; expect(check_attn_args(b), "chunk count", "max chunks"); }
  // tile GEMM: every plan of the shapes the library multiplies covers its product, passes
  // the checks and fits 160 KiB of LDS; then one rule broken at a time
  const int shapes[][3] = {{256, 6144, 4096}, {256, 4096, 4096}, {256, 28672, 4096},
                           {256, 4096, 14336}, {256, 128256, 4096}, {4096, 2048, 5120},
                           {4096, 2048, 4096}, {65, 7168, 5120}, {96, 34816, 5120},
                           {200, 5120, 17408}, {100, 1024, 256}, {128, 512, 256}};
  for (const auto& sh : shapes)
    for (int wt = 0; wt < 2; ++wt)
      for (int epi = 0; epi < 4; ++epi) {
        if ((epi == TG_RESID || epi == TG_SWIGLU) && wt != WT_INT8) continue;
        if (epi == TG_ARGMAX && wt != WT_F16) continue;
        const TilePlan tp = tile_plan(sh[0], sh[1], sh[2], wt, 256, epi == TG_SWIGLU);
        TileArgs ta{};
        ta.W = (const uint4*)P; ta.X = (const half_t*)P; ta.Y = (float*)P;
        ta.M = sh[0]; ta.N = sh[1]; ta.K = sh[2]; ta.ldy = sh[1];
        ta.scale = (const half_t*)P; ta.x = (half_t*)P; ta.ss = (float*)P; ta.out = (half_t*)P;
        ta.keys = (unsigned long long*)P;
        char what[96];
        std::snprintf(what, sizeof what, "tile plan %dx%dx%d wt %d epi %d", sh[0], sh[1], sh[2], wt, epi);
        expect(check_tile_args(wt, epi, ta, tp), nullptr, what);
        if (tile_lds_bytes(wt, tp) > 160 * 1024) expect("LDS", nullptr, what);
      }
  {
    TileArgs ta{};
    ta.W = (const uint4*)P; ta.X = (const half_t*)P; ta.Y = (float*)P;
    ta.M = 256; ta.N = 4096; ta.K = 4096; ta.ldy = 4096;
    const TilePlan tp = tile_plan(256, 4096, 4096, WT_INT8, 256);
    { TileArgs b = ta; b.K = 4000; expect(check_tile_args(WT_INT8, TG_F32, b, tp), "multiple of 64", "tile K"); }
    { TileArgs b = ta; b.ldy = 100; expect(check_tile_args(WT_INT8, TG_F32, b, tp), "output row", "tile ldy"); }
    { TileArgs b = ta; b.Y = nullptr; expect(check_tile_args(WT_INT8, TG_F32, b, tp), "output", "tile Y"); }
    { TileArgs b = ta; b.M = 1000; expect(check_tile_args(WT_INT8, TG_F32, b, tp), "cover", "tile M"); }
    { TilePlan q = tp; q.rbw = 3; expect(check_tile_args(WT_INT8, TG_F32, ta, q), "shape", "tile rbw"); }
    { TilePlan q = tp; q.tiles_n += 1; expect(check_tile_args(WT_INT8, TG_F32, ta, q), "cover", "tile n"); }
    { TileArgs b = ta; b.N = 4010; expect(check_tile_args(WT_INT8, TG_F32, b, tp), "multiple", "tile N"); }
    { expect(check_tile_args(WT_INT8, TG_RESID, ta, tp), "RESID", "tile resid args"); }
    { expect(check_tile_args(WT_F16, TG_ARGMAX, ta, tp), "ARGMAX", "tile argmax keys"); }
    { TileArgs b = ta; b.scale = (const half_t*)P; b.out = (half_t*)P;
      TilePlan q = tp; q.rbw = 1;   // no gate|up pairs in a wave
      expect(check_tile_args(WT_INT8, TG_SWIGLU, b, q), "pairs", "tile swiglu pairs"); }
    { expect(check_tile_args(WT_INT8, 9, ta, tp), "epilogue", "tile epi"); }
    // split-K: the small-N stacked products split; the planes go through the F32 epilogue
    // only; the reduction's own rules
    const TilePlan sp = tile_plan(256, 4096, 14336, WT_INT8, 256, false, true);
    { TileArgs b = ta; b.K = 14336;
      if (sp.splits < 2) expect("no split", nullptr, "down 256 rows splits");
      if (sp.tiles_m * sp.tiles_n * sp.splits > 256) expect("over-subscribed", nullptr, "split grid");
      expect(check_tile_args(WT_INT8, TG_F32, b, sp), nullptr, "split plan F32");
      b.scale = (const half_t*)P; b.x = (half_t*)P; b.ss = (float*)P;
      expect(check_tile_args(WT_INT8, TG_RESID, b, sp), "split-K", "split plan RESID"); }
    { TilePlan q = tp; q.splits = 65; expect(check_tile_args(WT_INT8, TG_F32, ta, q), "split-K", "splits > K/64"); }
    { TileArgs b = ta; expect(check_tile_reduce_args(TG_F32, b, (const float*)P, 4), nullptr, "reduce F32"); }
    { TileArgs b = ta; b.scale = (const half_t*)P; b.x = (half_t*)P; b.ss = (float*)P;
      expect(check_tile_reduce_args(TG_RESID, b, (const float*)P, 4), nullptr, "reduce RESID"); }
    { TileArgs b = ta; expect(check_tile_reduce_args(TG_RESID, b, (const float*)P, 4), "RESID", "reduce RESID args"); }
    { TileArgs b = ta; b.N = 4000; expect(check_tile_reduce_args(TG_F32, b, (const float*)P, 4), "multiple of 64", "reduce N"); }
    { TileArgs b = ta; expect(check_tile_reduce_args(TG_SWIGLU, b, (const float*)P, 4), "F32 and RESID", "reduce epi"); }
    // re-tiled tail: the prompt-sized fc (4096 rows, 5120 x 25600 fp16) has a partial last
    // round on 256 CUs; the plan runs the full rounds whole and the rest on a smaller shape
    // whose tiles divide the plan's
    const TilePlan rt = tile_plan(4096, 5120, 25600, WT_F16, 256, false, false, true);
    const long long rt_tiles = (long long)rt.tiles_m * rt.tiles_n;
    if (rt.tail_shape < 0) expect("no re-tiled tail", nullptr, "fc re-tiled tail");
    if (rt.head_tiles % 256 || rt.head_tiles < 256 || rt.head_tiles >= rt_tiles)
      expect("head not whole rounds", nullptr, "fc head tiles");
    { TileArgs b = ta; b.M = 4096; b.N = 5120; b.K = 25600; b.ldy = 5120;
      expect(check_tile_args(WT_F16, TG_F32, b, rt), nullptr, "re-tiled plan");
      TilePlan q = rt; q.tail_shape = 0;   // an int8 shape
      expect(check_tile_args(WT_F16, TG_F32, b, q), "divide", "re-tiled wrong type");
      q = rt; q.head_tiles = 0;
      expect(check_tile_args(WT_F16, TG_F32, b, q), "head", "re-tiled no head");
      q = rt; q.tail_shape = kNumTileShapes;
      expect(check_tile_args(WT_F16, TG_F32, b, q), "unknown", "re-tiled shape index"); }
    // none without permission, nor when the tiles fill whole rounds (K|V ingest: 16 x 16
    // tiles of 256 x 128), nor in the plain plan's shape list
    if (tile_plan(4096, 5120, 25600, WT_F16, 256).tail_shape != -1) expect("tail", nullptr, "fc no re-tile");
    if (tile_plan(4096, 2048, 5120, WT_INT8, 256, false, false, true).tail_shape != -1)
      expect("tail", nullptr, "K|V whole rounds");
    for (int M : {256, 1024, 4096})
      for (int N : {5120, 28672, 128256}) {
        const TilePlan q = tile_plan(M, N, 5120, WT_F16, 256);
        for (const TileShape& u : kTileShapes)
          if (u.tail && u.wt == WT_F16 && q.mtw == u.mtw && q.rbw == u.rbw && q.wn == u.wn &&
              q.kc == u.kc)
            expect("tail-only shape planned", nullptr, "plain plan shapes");
      }
  }
  if (fails == 0) std::printf("ok\n");
  return fails ? 1 : 0;
}
