// C ABI of libdflash_hip.so: context management, weight loading, context ingest and the
// draft-block sequence.  See include/dflash_hip.h for the contract of each entry point.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>


#include "dflash_hip.h"
#include "dfl_kernels.h"
#include "dfl_check.h"
#include "dfl_sk_plan.h"
#include "dfl_tile_plan.h"

using namespace dfl;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define DFL_HIP(x)                                                                   \
  do {                                                                               \
    hipError_t e_ = (x);                                                             \
    if (e_ != hipSuccess) return fail(DFL_EHIP, std::string(#x) + ": " + hipGetErrorString(e_)); \
  } while (0)

constexpr int ING_MAX = 4096;      // context rows per ingest pass (at most)
// Ingest calls of at most SMALL_ING rows (the per-step context of a decode loop: acceptance
// + 1 rows) run on the stream-K kernels, which stream each weight once at HBM rate; larger
// (prompt) ingests are compute-bound: their K|V rows run on the tile GEMM (MFMA) over the
// packed int8 qkv matrix, the fc on the tile GEMM over the packed fp16 fc weight, reading
// the context rows (or the tapped layers' rows) where they lie.
constexpr int SMALL_ING = 64;
constexpr int MAX_CHUNKS = 64;     // attention key splits
constexpr int MT_MAX = 8;          // 32-row m-tiles per M-split GEMM launch
// Stacked blocks of more than STACK_MIN_ROWS rows (batched drafting) are compute-bound: their
// projections and the lm_head run on the tile GEMM (MFMA, LDS-staged) over the packed weights,
// with the epilogues in row kernels.
constexpr int STACK_MIN_ROWS = 64;

enum ProfCat {
  P_GEMM_W8 = 0, P_LM_HEAD, P_ATTN, P_QK_ROPE, P_ROWS, P_INGEST_FC, P_INGEST_KV, P_GEMM_TILE, P_N
};
const char* const kProfNames[P_N] = {"gemm_w8a16",   "lm_head_argmax", "attention",
                                     "qk_norm_rope", "row_reduce_norm", "ingest_fc",
                                     "ingest_kv",    "gemm_tile_rows"};

struct ProfRec {
  int cat;
  hipEvent_t a, b;
  long long bytes;
};

// Cache bookkeeping of one sequence (DFlashKVCache.offset and its row count).
//
// With a window (DFlashKVCache(sink_size, window_size), dflash.py:160-193) the cache keeps
// the first `sink` rows and the newest `window` rows.  Rows past the sink live in a ring of
// `window` cache rows: an append overwrites the oldest ring row once the ring is full, and
// a trim steps the ring back over its newest rows.  Attention is indifferent to key order,
// so the set of rows it sees is exactly the reference's concatenated sink + window.
struct SeqState {
  int len = 0;             // cached rows (the reference cache's key count)
  long long offset = 0;    // absolute position of the next row
  int last_block = 0;      // rows of the last drafted block (committable)
  int sink = 0, window = 0;
  long long ring_j = 0;    // rows appended to the ring (less trimmed ones)

  // cache rows of the next n appended rows: sink rows from row0, then the ring
  void slots(int n, int& row0, int& sink_fill, int& j0) const {
    row0 = len;
    sink_fill = window ? std::max(0, std::min(sink - len, n)) : 0;
    j0 = window ? (int)(ring_j % window) : 0;
  }
  void append(int n) {
    if (!window) {
      len += n;
      return;
    }
    const int sf = std::max(0, std::min(sink - len, n));
    ring_j += n - sf;
    len = std::min(len + n, sink + window);
  }
  void trim(int n) {
    if (window) ring_j -= std::min(n, std::max(0, len - sink));
    len = std::max(0, len - n);
  }
  // key index range attention scans (ring rows never written stay masked)
  int key_range() const {
    if (!window || len <= sink) return len;
    return sink + (int)std::min<long long>(window, ring_j);
  }
};

struct Layer {
  uint4 *w_qkv = nullptr, *w_o = nullptr, *w_gu = nullptr, *w_down = nullptr;
  half_t *s_qkv = nullptr, *s_o = nullptr, *s_gu = nullptr, *s_down = nullptr;
  half_t *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  half_t *Kc = nullptr, *Vt = nullptr;   // [max_seqs][NKV][cap][128], [max_seqs][NKV][128][cap]
  bool loaded = false;
};

}  // namespace

struct dfl_ctx {
  dfl_config cfg;
  int H, NH, NKV, F, NL, NQKV, Bmax, cap, V, NF;
  int S = 1;                 // sequences (independent KV caches)
  int RM = 0;                // activation rows: S * Bmax
  int cur = 0;               // sequence addressed by the single-sequence calls
  size_t kv_seq = 0;         // elements of one sequence's K (or Vt) cache per layer
  std::vector<SeqState> seqs;
  SeqState& sq() { return seqs[cur]; }
  half_t* kc(const Layer& L, int seq) const { return L.Kc + (size_t)seq * kv_seq; }
  half_t* vt(const Layer& L, int seq) const { return L.Vt + (size_t)seq * kv_seq; }
  std::vector<Layer> layers;
  half_t* hidden_norm = nullptr;
  bool fc_loaded = false;
  half_t* final_norm = nullptr;
  uint4* w_lm = nullptr;
  float* y32 = nullptr;      // [RM][max(NQKV, H, 2F)] fp32 rows of the stacked-block GEMMs
  float* tile_ws = nullptr;  // split-K planes of the stacked-block tile GEMMs
  size_t tile_ws_floats = 0;
  unsigned long long* lm_parts = nullptr;   // [V/32][RM] stacked lm_head argmax partial keys
  const half_t* embed = nullptr;
  bool head_loaded = false;
  int active = 0;   // layers run per call (num_draft_layers)
  // x, attn, act and h (the normed rows of stacked blocks) in the activation fragment layout
  half_t *x = nullptr, *h = nullptr, *Q = nullptr, *attn = nullptr, *act = nullptr;
  float *Op = nullptr, *Ml = nullptr;
  unsigned long long* keys = nullptr;
  unsigned long long* sa_cand = nullptr;   // soft-anchor top-k candidates per scan workgroup
  int* err = nullptr;
  // stream-K GEMM state (block step)
  int n_cu = 256;
  int lds_max = 0;               // LDS bytes per workgroup of the device
  half_t* qkvbuf = nullptr;      // [RM][NQKV] fp16 projections
  float* rnorm = nullptr;        // [RM] 1/rms of the residual rows
  float* rope_cs = nullptr;      // [32][64][2] RoPE cos, sin of a block's rows (one sequence)
  // scaled RoPE (dfl_set_rope_scaling): the 64 frequencies, fp64; unscaled RoPE computes
  // theta^(-j/64) in the kernels
  double* rope_inv = nullptr;
  bool rope_scaled = false;
  const double* rope_freqs() const { return rope_scaled ? rope_inv : nullptr; }
  float* sk_ws = nullptr;        // split-tile partials
  int* sk_tile_cnt = nullptr;    // [max tiles]
  int* dyn_next = nullptr;       // [2] work counters of the balanced lm_head (self-resetting)
  float* sk_ss = nullptr;        // [m-tiles][H/64 or H/32][32] row sums of squares of x (RESID)
  SKPlan sk_qkv, sk_o, sk_gu, sk_down, sk_lm;
  // context ingest: `ing` rows per pass (compute-bound: fc and K|V on the tile GEMM)
  int ing = 0;
  float* fc32 = nullptr;      // [ing][H] fc GEMM rows (fp32)
  float* ing_cs = nullptr;    // [ing][64][2] RoPE (cos, sin) of a prompt-sized pass's rows
  half_t* xf = nullptr;       // [ing][n_target_feat * H] fc input rows, fragment layout
  half_t* xn = nullptr;       // [ing/32][32][H] hidden_norm(fc) (or fused) rows, fragment layout
  float* kv32 = nullptr;      // [ing][NL*2*NKV*128] K|V GEMM rows of every layer (fp32)
  // per-step ingest of up to SMALL_ING rows on the stream-K kernels (no library GEMM): the
  // fc weight packed in fp16 blocks, input / normed rows in activation fragment layout,
  // fp16 fc and K|V rows
  uint4* w_fc_pk = nullptr;   // packed fc [H][NF*H] (KB = NF*H/16)
  half_t* si_in = nullptr;    // [SMALL_ING/32][32][max(NF,1)*H] fragment-layout input rows
  half_t* si_xn = nullptr;    // [SMALL_ING/32][32][H] fragment-layout fc rows (fp16)
  half_t* si_kv = nullptr;    // [SMALL_ING][NL*2*NKV*128] K|V rows of every layer (fp16, scaled)
  // the K|V rows of every layer side by side ([NL*2*NKV*128][H] packed int8 + scales), so
  // that one launch projects a per-step ingest's rows for all layers (a copy of 2*NKV*128
  // of each layer's NQKV qkv rows)
  uint4* w_kv_all = nullptr;
  half_t* s_kv_all = nullptr;
  SKPlan sk_fc;
  std::vector<void*> allocs;
  int prof = 0;   // 0 off, 1 every kernel group, 2 stream-K GEMM launches only
  int test_queue_timeout = 0;   // dfl_test_queue_timeout: balanced lm_head waits give up
  // dfl_set_sampling: draft ids as categorical samples at temperature 1 / samp_invT (0:
  // argmax); each sampling call draws its noise from seed + its call count
  float samp_invT = 0.f;
  unsigned long long samp_seed = 0, samp_calls = 0;
  float call_invT = 0.f;        // the current call's (set by draft_rows before its lm_head)
  uint32_t call_seed = 0;
  std::vector<ProfRec> recs;

  ~dfl_ctx() {
    for (auto& r : recs) {
      (void)hipEventDestroy(r.a);
      (void)hipEventDestroy(r.b);
    }
    for (void* p : allocs) (void)hipFree(p);
  }
  template <class T>
  int alloc(T** p, size_t n, bool zero = false) {
    void* v = nullptr;
    hipError_t e = hipMalloc(&v, std::max<size_t>(n, 1) * sizeof(T));
    if (e != hipSuccess)
      return fail(DFL_EHIP, std::string("hipMalloc(") + std::to_string(n * sizeof(T)) +
                                " bytes): " + hipGetErrorString(e));
    allocs.push_back(v);
    *p = static_cast<T*>(v);
    if (zero) {
      e = hipMemset(v, 0, std::max<size_t>(n, 1) * sizeof(T));
      if (e != hipSuccess) return fail(DFL_EHIP, std::string("hipMemset: ") + hipGetErrorString(e));
    }
    return DFL_OK;
  }
};

// Times the kernels launched in its scope when profiling is on.  A marker scope records
// events on the stream before and after the group (this adds marker packets, so it is
// used only in mode 1).  An attached scope (one stream-K GEMM launch) hands its events
// to the launch, which stores the kernel's own start and end timestamps in them: no
// extra packets, so mode 2 leaves the stream's timing unchanged.
struct ProfScope {
  dfl_ctx* c;
  int cat;
  long long bytes;
  hipStream_t st;
  bool attached;
  hipEvent_t a = nullptr, b = nullptr;
  ProfScope(dfl_ctx* c_, int cat_, long long bytes_, hipStream_t st_, bool attached_ = false)
      : c(c_), cat(cat_), bytes(bytes_), st(st_), attached(attached_) {
    const bool on = c->prof == 1 || (c->prof == 2 && attached);
    if (!on) return;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
      if (a) (void)hipEventDestroy(a);
      a = b = nullptr;
      return;
    }
    if (!attached) (void)hipEventRecord(a, st);
  }
  hipEvent_t start() const { return attached ? a : nullptr; }
  hipEvent_t stop() const { return attached ? b : nullptr; }
  ~ProfScope() {
    if (a && b) {
      if (!attached) (void)hipEventRecord(b, st);
      c->recs.push_back({cat, a, b, bytes});
    }
  }
};

#define DFL_TRY(x)              \
  do {                          \
    int r_ = (x);               \
    if (r_ != DFL_OK) return r_; \
  } while (0)

static int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DFL_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  return DFL_OK;
}

// Ingest buffers, allocated here so that no later call allocates device memory.
static int setup_ingest(dfl_ctx* x) {
  const int H = x->H, Nkv = 2 * x->NKV * 128;
  x->ing = std::max(32, std::min(ING_MAX, ((x->cfg.max_ctx + 31) / 32) * 32));
  int r = DFL_OK;
  if ((r = x->alloc(&x->kv32, (size_t)x->ing * x->NL * Nkv))) return r;
  if ((r = x->alloc(&x->si_in, (size_t)SMALL_ING * std::max(x->NF, 1) * H, true)) ||
      (r = x->alloc(&x->si_xn, (size_t)SMALL_ING * H, true)) ||
      (r = x->alloc(&x->si_kv, (size_t)SMALL_ING * x->NL * Nkv)) ||
      (r = x->alloc(&x->w_kv_all, (size_t)x->NL * Nkv * H / 16)) ||
      (r = x->alloc(&x->s_kv_all, (size_t)x->NL * Nkv)))
    return r;
  if ((r = x->alloc(&x->xn, (size_t)x->ing * H)) ||
      (r = x->alloc(&x->ing_cs, (size_t)x->ing * 128)))
    return r;
  if (x->NF > 0 && ((r = x->alloc(&x->fc32, (size_t)x->ing * H)) ||
                    (r = x->alloc(&x->xf, (size_t)x->ing * x->NF * H))))
    return r;
  return DFL_OK;
}

extern "C" {

const char* dfl_last_error(void) { return g_err.c_str(); }

int dfl_create(const dfl_config* cfg, dfl_ctx** out) {
  if (!cfg || !out) return fail(DFL_EINVAL, "dfl_create: null argument");
  *out = nullptr;
  const dfl_config& c = *cfg;
  if (c.head_dim != 128) return fail(DFL_EINVAL, "dfl_create: head_dim must be 128");
  if (c.hidden <= 0 || c.hidden % 128 || c.hidden > 8192)
    return fail(DFL_EINVAL, "dfl_create: hidden must be a positive multiple of 128, <= 8192");
  if (c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads)
    return fail(DFL_EINVAL, "dfl_create: n_heads must be a positive multiple of n_kv_heads");
  if (c.intermediate <= 0 || c.intermediate % 128 || c.intermediate > 8192 * 8)
    return fail(DFL_EINVAL, "dfl_create: intermediate must be a positive multiple of 128");
  if (c.n_layers <= 0) return fail(DFL_EINVAL, "dfl_create: n_layers must be positive");
  if (c.vocab < 0 || c.vocab % 64) return fail(DFL_EINVAL, "dfl_create: vocab must be a multiple of 64");
  if (c.max_block <= 0 || c.max_block > 256)
    return fail(DFL_EINVAL, "dfl_create: max_block must be in [1, 256]");
  if (c.max_ctx < 0) return fail(DFL_EINVAL, "dfl_create: max_ctx must be >= 0");
  if (c.n_target_feat < 0) return fail(DFL_EINVAL, "dfl_create: n_target_feat must be >= 0");
  if (!(c.rms_eps > 0.f) || !(c.rope_theta > 0.0))
    return fail(DFL_EINVAL, "dfl_create: rms_eps and rope_theta must be positive");
  if (c.max_seqs < 0 || c.max_seqs > 64)
    return fail(DFL_EINVAL, "dfl_create: max_seqs must be in [0, 64] (0 means 1)");

  dfl_ctx* x = new dfl_ctx();
  x->cfg = c;
  x->H = c.hidden;
  x->NH = c.n_heads;
  x->NKV = c.n_kv_heads;
  x->F = c.intermediate;
  x->NL = c.n_layers;
  x->NQKV = (c.n_heads + 2 * c.n_kv_heads) * 128;
  x->Bmax = c.max_block;
  x->V = c.vocab;
  x->NF = c.n_target_feat;
  x->cap = ((c.max_ctx + c.max_block + 63) / 64) * 64;
  x->S = std::max(1, c.max_seqs);
  x->RM = x->S * x->Bmax;
  x->kv_seq = (size_t)x->NKV * x->cap * 128;
  x->seqs.resize(x->S);
  x->layers.resize(c.n_layers);
  x->active = c.n_layers;

  const size_t Bm = x->RM;   // activation rows of a (batched) block step
  int r = DFL_OK;
  // x / attn / act are 32-row tiles in the activation fragment layout (zero padded rows)
  const size_t Bt = ((Bm + 31) / 32) * 32;
  if ((r = x->alloc(&x->x, Bt * x->H, true)) || (r = x->alloc(&x->h, Bt * x->H, true)) ||
      (r = x->alloc(&x->Q, (size_t)x->NH * Bm * 128)) ||
      (r = x->alloc(&x->attn, Bt * x->NH * 128, true)) || (r = x->alloc(&x->act, Bt * x->F, true)) ||
      (r = x->alloc(&x->Op, (size_t)MAX_CHUNKS * x->NH * Bm * 128)) ||
      (r = x->alloc(&x->Ml, (size_t)MAX_CHUNKS * x->NH * Bm * 2)) ||
      (r = x->alloc(&x->keys, Bm, true)) || (r = x->alloc(&x->err, 1, true)) ||
      (r = x->alloc(&x->sa_cand, (size_t)SA_BLOCKS * SA_TOPK_MAX))) {
    delete x;
    return r;
  }
  {
    int dev = 0, ncu = 0, lds = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        ncu > 0)
      x->n_cu = ncu;
    // the attention's LDS stage needs 80 KiB per workgroup (160 KiB for two stage buffers)
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        lds < 80 * 1024) {
      delete x;
      return fail(DFL_EINVAL, "dfl_create: the device offers " + std::to_string(lds) +
                                  " bytes of LDS per workgroup; the attention kernel needs 81920");
    }
    x->lds_max = lds;
    auto plan = [&](int N, int KB) { return streamk_plan(N, KB, x->n_cu); };
    x->sk_qkv = plan(x->NQKV, x->H / 32);
    x->sk_o = plan(x->H, x->NH * 128 / 32);
    x->sk_gu = plan(2 * x->F, x->H / 32);
    x->sk_down = plan(x->H, x->F / 32);
    x->sk_lm = streamk_plan_balanced(std::max(x->V, 64), x->H / 16, x->n_cu);
    x->sk_fc = streamk_plan(x->H, std::max(x->NF, 1) * x->H / 16, x->n_cu);
    std::vector<std::pair<SKPlan, int>> plans = {
        {x->sk_qkv, x->NQKV}, {x->sk_o, x->H}, {x->sk_gu, 2 * x->F}, {x->sk_down, x->H},
        {x->sk_lm, std::max(x->V, 64)}, {x->sk_fc, x->H}};
    // the per-step ingest's K|V rows of the first `active` layers, any active count
    for (int nl = 1; nl <= x->NL; ++nl) {
      const int n = nl * 2 * x->NKV * 128;
      plans.push_back({plan(n, x->H / 32), n});
    }
    size_t wsn = 0, tiles = 0;
    for (const auto& pr : plans) {
      wsn = std::max(wsn, (size_t)(pr.second / 64) *
                              std::max(pr.first.seg_cap, pr.first.sk_seg_cap) * 2048);
      tiles = std::max(tiles, (size_t)(pr.second / 64));
    }
    const size_t bm32 = ((Bm + 31) / 32) * 32;
    // split-tile partials hold one 32x64 slot per m-tile of a launch (the per-step ingest's
    // fc and K|V launches take up to SMALL_ING / 32 m-tiles)
    wsn *= (size_t)std::min<size_t>(MT_MAX, std::max<size_t>(bm32 / 32, SMALL_ING / 32));
    if ((r = x->alloc(&x->qkvbuf, Bm * x->NQKV)) || (r = x->alloc(&x->rnorm, bm32)) ||
        (r = x->alloc(&x->sk_ws, wsn)) || (r = x->alloc(&x->sk_tile_cnt, tiles, true)) ||
        (r = x->alloc(&x->dyn_next, 2, true)) || (r = x->alloc(&x->rope_cs, 32 * 64 * 2)) ||
        (r = x->alloc(&x->rope_inv, 64)) ||
        (r = x->alloc(&x->sk_ss, (bm32 / 32) * (size_t)(x->H / 32) * 32))) {
      delete x;
      return r;
    }
  }
  for (auto& L : x->layers) {
    const size_t kv = x->kv_seq * x->S;
    if ((r = x->alloc(&L.Kc, kv, true)) || (r = x->alloc(&L.Vt, kv, true))) {
      delete x;
      return r;
    }
  }
  if ((r = setup_ingest(x))) {
    delete x;
    return r;
  }
  if (x->RM > STACK_MIN_ROWS) {
    // split-K planes: the largest plan of the stacked qkv / o / down products over every
    // row count up to RM
    for (int M = 32; M <= ((x->RM + 31) / 32) * 32; M += 32)
      for (auto nk : {std::make_pair(x->NQKV, x->H), std::make_pair(x->H, x->NH * 128),
                      std::make_pair(x->H, x->F)}) {
        const TilePlan p = tile_plan(std::min(M, x->RM), nk.first, nk.second, WT_INT8, x->n_cu,
                                     false, true);
        x->tile_ws_floats =
            std::max(x->tile_ws_floats, (size_t)p.splits * std::min(M, x->RM) * nk.first);
      }
    if ((r = x->alloc(&x->y32, (size_t)x->RM * std::max({x->NQKV, x->H, 2 * x->F}))) ||
        (r = x->alloc(&x->tile_ws, x->tile_ws_floats))) {
      delete x;
      return r;
    }
  }
  *out = x;
  return DFL_OK;
}

int dfl_destroy(dfl_ctx* ctx) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_destroy: null context");
  (void)hipDeviceSynchronize();
  delete ctx;
  return DFL_OK;
}

int dfl_quantize_w8(const float* w, int64_t oc, int64_t ic, int8_t* q, uint16_t* scale,
                    void* stream) {
  if (!w || !q || !scale) return fail(DFL_EINVAL, "dfl_quantize_w8: null pointer");
  if (oc <= 0 || ic <= 0 || oc > (1ll << 31) - 1)
    return fail(DFL_EINVAL, "dfl_quantize_w8: bad shape");
  launch_quantize_w8(w, oc, ic, q, reinterpret_cast<half_t*>(scale), (hipStream_t)stream);
  return check_launch("quantize_w8");
}

int dfl_load_layer_w8(dfl_ctx* ctx, int layer, const int8_t* const q[7],
                      const uint16_t* const scale[7], const uint16_t* in_norm,
                      const uint16_t* post_norm, const uint16_t* q_norm, const uint16_t* k_norm,
                      void* stream) {
  if (!ctx || !q || !scale) return fail(DFL_EINVAL, "dfl_load_layer_w8: null argument");
  if (layer < 0 || layer >= ctx->NL)
    return fail(DFL_ERANGE, "dfl_load_layer_w8: layer index out of range");
  for (int i = 0; i < 7; ++i)
    if (!q[i] || !scale[i]) return fail(DFL_EINVAL, "dfl_load_layer_w8: null weight pointer");
  if (!in_norm || !post_norm || !q_norm || !k_norm)
    return fail(DFL_EINVAL, "dfl_load_layer_w8: null norm pointer");
  hipStream_t st = (hipStream_t)stream;
  Layer& L = ctx->layers[layer];
  const int H = ctx->H, NH = ctx->NH, NKV = ctx->NKV, F = ctx->F, NQ = NH * 128;
  if (!L.w_qkv) {
    DFL_TRY(ctx->alloc(&L.w_qkv, (size_t)ctx->NQKV * H / 16));
    DFL_TRY(ctx->alloc(&L.s_qkv, (size_t)ctx->NQKV));
    DFL_TRY(ctx->alloc(&L.w_o, (size_t)H * NQ / 16));
    DFL_TRY(ctx->alloc(&L.s_o, (size_t)H));
    DFL_TRY(ctx->alloc(&L.w_gu, (size_t)2 * F * H / 16));
    DFL_TRY(ctx->alloc(&L.s_gu, (size_t)2 * F));
    DFL_TRY(ctx->alloc(&L.w_down, (size_t)H * F / 16));
    DFL_TRY(ctx->alloc(&L.s_down, (size_t)H));
    DFL_TRY(ctx->alloc(&L.in_norm, (size_t)H));
    DFL_TRY(ctx->alloc(&L.post_norm, (size_t)H));
    DFL_TRY(ctx->alloc(&L.q_norm, (size_t)128));
    DFL_TRY(ctx->alloc(&L.k_norm, (size_t)128));
  }
  auto S = [&](int i) { return reinterpret_cast<const half_t*>(scale[i]); };
  // fused QKV: row-blocks [0, NH*4) = q_proj, then k_proj, then v_proj
  launch_pack_i8(q[0], S(0), NQ, H, L.w_qkv, L.s_qkv, 0, 1, st);
  launch_pack_i8(q[1], S(1), NKV * 128, H, L.w_qkv, L.s_qkv, NH * 4, 1, st);
  launch_pack_i8(q[2], S(2), NKV * 128, H, L.w_qkv, L.s_qkv, (NH + NKV) * 4, 1, st);
  launch_pack_i8(q[3], S(3), H, NQ, L.w_o, L.s_o, 0, 1, st);
  // gate|up interleaved by row-block: 2j = gate rows [32j, 32j+32), 2j+1 = up rows
  launch_pack_i8(q[4], S(4), F, H, L.w_gu, L.s_gu, 0, 2, st);
  launch_pack_i8(q[5], S(5), F, H, L.w_gu, L.s_gu, 1, 2, st);
  launch_pack_i8(q[6], S(6), H, F, L.w_down, L.s_down, 0, 1, st);
  // the k|v rows again in the all-layer matrix (row-blocks of layer l at l * 2*NKV*4)
  launch_pack_i8(q[1], S(1), NKV * 128, H, ctx->w_kv_all, ctx->s_kv_all, layer * 2 * NKV * 4, 1,
                 st);
  launch_pack_i8(q[2], S(2), NKV * 128, H, ctx->w_kv_all, ctx->s_kv_all,
                 layer * 2 * NKV * 4 + NKV * 4, 1, st);
  DFL_HIP(hipMemcpyAsync(L.in_norm, in_norm, H * 2, hipMemcpyDeviceToDevice, st));
  DFL_HIP(hipMemcpyAsync(L.post_norm, post_norm, H * 2, hipMemcpyDeviceToDevice, st));
  DFL_HIP(hipMemcpyAsync(L.q_norm, q_norm, 256, hipMemcpyDeviceToDevice, st));
  DFL_HIP(hipMemcpyAsync(L.k_norm, k_norm, 256, hipMemcpyDeviceToDevice, st));
  DFL_TRY(check_launch("pack layer weights"));
  L.loaded = true;
  return DFL_OK;
}

int dfl_load_fc(dfl_ctx* ctx, const uint16_t* fc_weight, const uint16_t* hidden_norm,
                void* stream) {
  if (!ctx || !fc_weight || !hidden_norm) return fail(DFL_EINVAL, "dfl_load_fc: null argument");
  if (ctx->NF <= 0) return fail(DFL_ESTATE, "dfl_load_fc: context created with n_target_feat = 0");
  hipStream_t st = (hipStream_t)stream;
  const int K = ctx->NF * ctx->H;
  if (!ctx->w_fc_pk) {
    DFL_TRY(ctx->alloc(&ctx->hidden_norm, (size_t)ctx->H));
    DFL_TRY(ctx->alloc(&ctx->w_fc_pk, (size_t)ctx->H * K / 8));
  }
  DFL_HIP(hipMemcpyAsync(ctx->hidden_norm, hidden_norm, ctx->H * 2, hipMemcpyDeviceToDevice, st));
  // the fc weight in the packed fp16 block layout, read by the stream-K (per-step) and
  // tile (prompt-sized) GEMMs
  launch_pack_f16(reinterpret_cast<const half_t*>(fc_weight), ctx->H, K, ctx->w_fc_pk, st);
  DFL_TRY(check_launch("pack fc"));
  ctx->fc_loaded = true;
  return DFL_OK;
}

int dfl_load_head(dfl_ctx* ctx, const uint16_t* final_norm, const uint16_t* embed,
                  const uint16_t* lm_head, void* stream) {
  if (!ctx || !final_norm) return fail(DFL_EINVAL, "dfl_load_head: null argument");
  if ((embed || lm_head) && ctx->V <= 0)
    return fail(DFL_ESTATE, "dfl_load_head: context created with vocab = 0");
  hipStream_t st = (hipStream_t)stream;
  if (!ctx->final_norm) DFL_TRY(ctx->alloc(&ctx->final_norm, (size_t)ctx->H));
  DFL_HIP(hipMemcpyAsync(ctx->final_norm, final_norm, ctx->H * 2, hipMemcpyDeviceToDevice, st));
  ctx->embed = reinterpret_cast<const half_t*>(embed);
  if (lm_head) {
    if (!ctx->w_lm) DFL_TRY(ctx->alloc(&ctx->w_lm, (size_t)ctx->V * ctx->H / 8));
    launch_pack_f16(reinterpret_cast<const half_t*>(lm_head), ctx->V, ctx->H, ctx->w_lm, st);
    DFL_TRY(check_launch("pack lm_head"));
    if (ctx->RM > STACK_MIN_ROWS && !ctx->lm_parts)
      DFL_TRY(ctx->alloc(&ctx->lm_parts, (size_t)(ctx->V / 32) * ctx->RM));
  }
  ctx->head_loaded = true;
  return DFL_OK;
}

// Stream-K GEMM over the M rows of a block: one 32-row m-tile per launch of the
// single-tile kernel, or up to 8 m-tiles per launch of the M-split kernel (each weight
// block read once for all of them).  A normed input (gnorm set) takes its 1/rms rows from
// the embedding kernel (rn_from_ss false) or from the row sums of squares that the
// previous RESID GEMM left in sk_ss (rn_from_ss true).
static int skgemm(dfl_ctx* ctx, int cat, int wt, int epi, const SKPlan& p,
                   const uint4* W, const half_t* scale, int N, int KB, const half_t* X, int ldx,
                   int M, const half_t* gnorm, bool rn_from_ss, half_t* out, int ldo,
                   half_t* xres, float* logits, unsigned long long* keys, hipStream_t st,
                   int32_t* ids = nullptr, bool* ids_done = nullptr,
                   const RopeEpi* rope = nullptr, bool x_zero = false,
                   const FeatPtrs* xr = nullptr, int xr_h = 0) {
  const long long wbytes = (wt == WT_INT8) ? (long long)N * KB * 32 + 2LL * N
                                           : (long long)N * KB * 16 * 2;
  const int ss_stride = (ctx->H / 64) * 32;
  const int n_mt = (M + 31) / 32;
  for (int g0 = 0; g0 < n_mt; g0 += MT_MAX) {
    const int mt_n = std::min(MT_MAX, n_mt - g0);
    const int m0 = g0 * 32;
    ProfScope ps(ctx, cat, wbytes, st, /*attached=*/true);
    StreamArgs a{};
    a.W = W;
    a.scale = scale;
    a.N = N;
    a.KB = KB;
    a.X = X ? X + (size_t)m0 * ldx : nullptr;
    a.ldx = ldx;
    if (xr) {   // row-major feature rows read in place (one m-tile)
      a.xr_n = xr->n;
      a.xr_ld = xr->ld;
      a.xr_h = xr_h;
      for (int j = 0; j < xr->n; ++j) a.xr_p[j] = xr->p[j];
    }
    a.M = std::min(32 * mt_n, M - m0);
    a.MT = mt_n;
    a.rnorm = ctx->rnorm + m0;
    a.ss_in = rn_from_ss ? ctx->sk_ss + (size_t)g0 * ss_stride : nullptr;
    a.ss_tiles = ctx->H / 64;
    a.ss_n = ctx->H;
    a.ss_mstride = ss_stride;
    a.gnorm = gnorm;
    a.ws = ctx->sk_ws;
    // one m-tile: the hybrid plan when it has whole tiles per workgroup; the M-split kernel
    // and the fused qkv kernel (a Q/K head's two tiles complete together) keep the
    // contiguous partition
    a.dp = streamk_launch_dp(p, epi, mt_n > 1);
    // test hook of the balanced kernel's bounded work-queue wait (its give-up path), set
    // only through dfl_test_queue_timeout
    a.dyn_test_timeout = p.dyn_static > 0 && ctx->test_queue_timeout;
    a.seg_cap = a.dp > 0 ? p.sk_seg_cap : p.seg_cap;
    a.tile_cnt = ctx->sk_tile_cnt;
    a.out = out ? out + (size_t)m0 * ldo : nullptr;
    a.ldo = ldo;
    a.x = xres ? xres + (size_t)m0 * ldo : nullptr;
    a.x_zero = x_zero;
    a.ss_part = ctx->sk_ss + (size_t)g0 * ss_stride;
    a.eps = ctx->cfg.rms_eps;
    a.logits = logits ? logits + (size_t)m0 * N : nullptr;
    a.ldl = N;
    a.keys = keys ? keys + m0 : nullptr;
    a.dyn_static = p.dyn_static;
    a.dyn_next = ctx->dyn_next;
    a.err = ctx->err;
    if (epi == EPI_ARGMAX) {
      a.samp_invT = ctx->call_invT;
      a.samp_seed = ctx->call_seed;
      a.samp_row0 = m0;
    }
    // the balanced kernel (one m-tile) finalises the argmax ids itself
    const bool fin = ids && keys && p.dyn_static > 0 && n_mt == 1;
    a.ids = fin ? ids : nullptr;
    if (ids_done) *ids_done = fin;
    if (rope) a.rope = *rope;
    if (const char* why = check_stream_args(wt, epi, gnorm != nullptr, a, p, mt_n > 1))
      return fail(DFL_EINVAL, std::string("stream-K GEMM launch refused: ") + why);
    const bool ok =
        mt_n == 1 ? launch_streamk_gemm(wt, epi, gnorm != nullptr, a, p, st, ps.start(), ps.stop())
                  : launch_streamk_gemm_m(wt, epi, gnorm != nullptr, a, p, st, ps.start(), ps.stop());
    if (!ok) return fail(DFL_EINVAL, "no GEMM kernel for this weight type / epilogue");
  }
  return DFL_OK;
}

// The rope / attention launchers with their argument checks reported as DFL_EINVAL.
static int qk_rope(const QKRopeArgs& q, hipStream_t st) {
  if (const char* why = check_qk_rope_args(q))
    return fail(DFL_EINVAL, std::string("Q/K norm + RoPE launch refused: ") + why);
  launch_qk_rope(q, st);
  return DFL_OK;
}

static int block_attention(const AttnArgs& at, hipStream_t st) {
  if (const char* why = check_attn_args(at))
    return fail(DFL_EINVAL, std::string("attention launch refused: ") + why);
  if (!launch_block_attention(at, st))
    return fail(DFL_EINVAL, "attention launch refused: more than 8 waves per workgroup");
  return DFL_OK;
}

// Tile GEMM of more than STACK_MIN_ROWS rows (X in the fragment layout) with epilogue epi
// (the TileArgs outputs e), its argument checks reported as DFL_EINVAL.
// Split-K (F32 and RESID epilogues of stacked blocks, when the plan finds it faster): the
// GEMM writes fp32 planes into tile_ws and launch_tile_reduce applies the epilogue.
// n_parts (ARGMAX): receives the number of partial key rows written (one per wave column).
// like_n (optional): plan with the tile shape the product of like_n columns would have, so
// that a product stacked over several such (the all-layer K|V ingest) sums every element
// exactly as the single one does.
static int tgemm(dfl_ctx* ctx, int cat, int wt, int epi, const uint4* W, int N, int K,
                 const half_t* X, int M, const TileArgs& e, hipStream_t st,
                 int* n_parts = nullptr, int like_n = 0) {
  const bool split_ok = (epi == TG_F32 || epi == TG_RESID) && ctx->tile_ws && M <= ctx->RM &&
                        !like_n;
  // re-tiled last rounds for the epilogues whose outputs do not depend on the tile shape
  // (the ARGMAX keys are per wave column)
  const bool retile = epi != TG_ARGMAX;
  TilePlan like{};
  if (like_n) like = tile_plan(M, like_n, K, wt, ctx->n_cu, epi == TG_SWIGLU);
  TilePlan p = tile_plan(M, N, K, wt, ctx->n_cu, epi == TG_SWIGLU, split_ok, retile,
                         like_n ? &like : nullptr);
  if (p.splits > 1 && (size_t)p.splits * M * N > ctx->tile_ws_floats)   // planes do not fit
    p = tile_plan(M, N, K, wt, ctx->n_cu, epi == TG_SWIGLU, false, retile);
  if (n_parts) *n_parts = N / (32 * p.rbw);
  TileArgs a = e;
  a.W = W;
  a.N = N;
  a.K = K;
  a.X = X;
  a.M = M;
  if (epi == TG_ARGMAX) {
    a.samp_invT = ctx->call_invT;
    a.samp_seed = ctx->call_seed;
  }
  TileArgs g = a;   // the GEMM's own arguments: F32 planes when split
  if (p.splits > 1) {
    g = TileArgs{};
    g.W = W;
    g.N = N;
    g.K = K;
    g.X = X;
    g.M = M;
    g.Y = ctx->tile_ws;
    g.ldy = N;
  }
  const int gepi = p.splits > 1 ? TG_F32 : epi;
  if (const char* why = check_tile_args(wt, gepi, g, p))
    return fail(DFL_EINVAL, std::string("tile GEMM launch refused: ") + why);
  if (p.splits > 1)
    if (const char* why = check_tile_reduce_args(epi, a, ctx->tile_ws, p.splits))
      return fail(DFL_EINVAL, std::string("tile GEMM reduction refused: ") + why);
  if (tile_lds_bytes(wt, p) > (size_t)ctx->lds_max)
    return fail(DFL_EINVAL, "tile GEMM: the device's LDS per workgroup is too small");
  const long long wbytes = (long long)N * K * (wt == WT_INT8 ? 1 : 2);
  // the attached events span the GEMM and, when split, its reduction
  ProfScope ps(ctx, cat, wbytes, st, /*attached=*/true);
  if (!launch_tile_gemm(wt, gepi, g, p, st, ps.start(), p.splits > 1 ? nullptr : ps.stop()))
    return fail(DFL_EINVAL, "no tile GEMM kernel for this shape and epilogue");
  if (p.splits > 1 && !launch_tile_reduce(epi, a, ctx->tile_ws, p.splits, st, ps.stop()))
    return fail(DFL_EINVAL, "tile GEMM reduction refused");
  return DFL_OK;
}
static TileArgs tile_f32(float* Y, int ldy) {
  TileArgs e{};
  e.Y = Y;
  e.ldy = ldy;
  return e;
}
static TileArgs tile_resid(const half_t* scale, half_t* x, float* ss) {
  TileArgs e{};
  e.scale = scale;
  e.x = x;
  e.ss = ss;
  return e;
}

static int layers_ready(dfl_ctx* ctx, const char* who) {
  for (int l = 0; l < ctx->active; ++l)
    if (!ctx->layers[l].loaded)
      return fail(DFL_ESTATE, std::string(who) + ": layer " + std::to_string(l) + " not loaded");
  return DFL_OK;
}

// Cache placement of the next n rows of sequence seq (its current state) at absolute
// position pos0.
static void rope_seq(dfl_ctx* ctx, int seq, const Layer& L, long long pos0, int n, RopeSeq& r) {
  const SeqState& q = ctx->seqs[seq];
  r.pos0 = pos0;
  r.Kc = ctx->kc(L, seq);
  r.Vt = ctx->vt(L, seq);
  q.slots(n, r.cache_row0, r.sink_fill, r.ring_j0);
  r.ring_S = q.sink;
  r.ring_W = q.window;
}

// K/V of `rows` fused context rows (fragment-layout tiles xa) for every active layer: the
// all-layer packed K|V matrix on the tile GEMM (one product: fp32 integer-weight sums, the
// same sums per element as a product per layer), then per-row scale + fp16 rounding,
// k_norm + RoPE on K (angles from one table for all layers), appended at cache row
// len + r0 with absolute position offset + r0, for up to SEQ_MAX layers per qk_rope launch.
static int ingest_kv_rows(dfl_ctx* ctx, const half_t* xa, int rows, int r0, hipStream_t st) {
  const int H = ctx->H, NH = ctx->NH, NKV = ctx->NKV;
  const int Nkv = 2 * NKV * 128, Nall = ctx->active * Nkv;
  {   // the rows' RoPE angles, once for every layer
    ProfScope ps(ctx, P_INGEST_KV, 0, st);
    launch_rope_table(rows, ctx->sq().offset + r0, std::log2(ctx->cfg.rope_theta),
                      ctx->rope_freqs(), ctx->ing_cs, st);
  }
  DFL_TRY(tgemm(ctx, P_INGEST_KV, WT_INT8, TG_F32, ctx->w_kv_all, Nall, H, xa, rows,
                tile_f32(ctx->kv32, Nall), st, nullptr, /*like_n=*/Nkv));
  for (int l0 = 0; l0 < ctx->active; l0 += SEQ_MAX) {
    const int nl = std::min(SEQ_MAX, ctx->active - l0);
    QKRopeArgs q{};
    q.qkv32 = ctx->kv32 + (size_t)l0 * Nkv;
    q.oscale = ctx->s_kv_all + (size_t)l0 * Nkv;   // scales of the k|v rows, in row order
    q.M = rows;
    q.N = Nall;
    q.n_seq = nl;
    q.layer_cols = Nkv;
    q.col_slot0 = NH;
    q.slot0 = NH;
    q.n_slots = 2 * NKV;
    q.NH = NH;
    q.NKV = NKV;
    q.q_norm = ctx->layers[l0].q_norm;
    q.k_norm = ctx->layers[l0].k_norm;
    q.eps = ctx->cfg.rms_eps;
    q.log2_theta = std::log2(ctx->cfg.rope_theta);
    q.inv_freq = ctx->rope_freqs();
    q.cs = ctx->ing_cs;
    q.Q = nullptr;
    q.cap = ctx->cap;
    for (int i = 0; i < nl; ++i) {
      const Layer& L = ctx->layers[l0 + i];
      q.k_norm_s[i] = L.k_norm;
      rope_seq(ctx, ctx->cur, L, ctx->sq().offset + r0, rows, q.sq[i]);
    }
    ProfScope ps(ctx, P_INGEST_KV, 0, st);
    DFL_TRY(qk_rope(q, st));
  }
  return DFL_OK;
}

// Per-step ingest of C <= SMALL_ING context rows on the stream-K kernels: the rows (or the
// tapped layers' features) into fragment layout; unless already fused, fc as an fp16 GEMM
// (each fc weight byte read once) whose RESID epilogue, with the residual taken as zero,
// writes the fp16 Linear output in fragment layout and its per-tile row sums of squares;
// then the K|V rows of every active layer as one int8 STORE GEMM that applies hidden_norm
// as it loads those rows (norm-on-load, 1/rms from the fc's row sums; the Linear's scale
// and fp16 rounding in its epilogue) and k_norm + RoPE into the cache.  The arithmetic of
// the prompt-sized path (fp32 accumulation, the same rounding points).
static int ingest_small(dfl_ctx* ctx, const half_t* in, int C, bool fused, const FeatPtrs* feats,
                        hipStream_t st) {
  const int H = ctx->H, NH = ctx->NH, NKV = ctx->NKV, Nkv = 2 * NKV * 128;
  FeatPtrs f{};
  if (feats) {
    f = *feats;
  } else {   // one row-major buffer: feature j is columns [j*H, (j+1)*H) of each row
    f.n = fused ? 1 : ctx->NF;
    f.ld = (long long)f.n * H;
    for (int j = 0; j < f.n; ++j) f.p[j] = in + (size_t)j * H;
  }
  const half_t* xsrc = ctx->si_in;   // fused rows: already the attention's context rows
  // Up to 16 rows the fc reads 16-byte aligned rows in place, row-major, instead of after a
  // gather into fragment layout: one launch less per step (4-12 rows: ingest 71-73 vs 76.5-77
  // us).  A row-major activation load touches one cache line per row against 8 for a
  // fragment record, which costs more than the launch from about 20 rows on (32 rows: 90 vs
  // 78.5 us).
  bool in_place = !fused && C <= 16 && H % 16 == 0 && H >= 64 && f.ld % 8 == 0;
  for (int j = 0; j < f.n && in_place; ++j)
    in_place = !(reinterpret_cast<uintptr_t>(f.p[j]) & 15);
  if (!in_place) {
    ProfScope ps(ctx, P_INGEST_FC, 0, st);
    launch_feats_to_afl(f, C, H, ctx->si_in, st);
  }
  if (!fused) {   // fc rows (fp16, fragment layout) and their per-tile sums of squares
    const int K = ctx->NF * H;
    DFL_TRY(skgemm(ctx, P_INGEST_FC, WT_F16, EPI_RESID, ctx->sk_fc, ctx->w_fc_pk, nullptr, H,
                   K / 16, in_place ? nullptr : ctx->si_in, K, C, nullptr, false, nullptr, H,
                   ctx->si_xn, nullptr, nullptr, st, nullptr, nullptr, nullptr, /*x_zero=*/true,
                   in_place ? &f : nullptr, H));
    xsrc = ctx->si_xn;
  }
  // the K|V rows of all active layers in one GEMM (the all-layer matrix; hidden_norm on
  // load unless the rows came fused), then k_norm + RoPE and the cache writes for up to
  // SEQ_MAX layers per launch
  const int KB = H / 32;
  const int Nall = ctx->active * Nkv;
  DFL_TRY(skgemm(ctx, P_INGEST_KV, WT_INT8, EPI_STORE, streamk_plan(Nall, KB, ctx->n_cu),
                 ctx->w_kv_all, ctx->s_kv_all, Nall, KB, xsrc, H, C,
                 fused ? nullptr : ctx->hidden_norm, !fused, ctx->si_kv, Nall, nullptr, nullptr,
                 nullptr, st));
  for (int l0 = 0; l0 < ctx->active; l0 += SEQ_MAX) {
    const int nl = std::min(SEQ_MAX, ctx->active - l0);
    QKRopeArgs q{};
    q.qkv16 = ctx->si_kv + (size_t)l0 * Nkv;
    q.M = C;
    q.N = Nall;
    q.n_seq = nl;
    q.layer_cols = Nkv;
    q.col_slot0 = NH;
    q.slot0 = NH;
    q.n_slots = 2 * NKV;
    q.NH = NH;
    q.NKV = NKV;
    q.q_norm = ctx->layers[l0].q_norm;
    q.k_norm = ctx->layers[l0].k_norm;
    q.eps = ctx->cfg.rms_eps;
    q.log2_theta = std::log2(ctx->cfg.rope_theta);
    q.inv_freq = ctx->rope_freqs();
    q.Q = nullptr;   // (a per-step call's few rows compute their angles in place: an angle
    q.cap = ctx->cap;   // table would cost one more launch than it saves)
    for (int i = 0; i < nl; ++i) {
      const Layer& L = ctx->layers[l0 + i];
      q.k_norm_s[i] = L.k_norm;
      rope_seq(ctx, ctx->cur, L, ctx->sq().offset, C, q.sq[i]);
    }
    ProfScope ps(ctx, P_INGEST_KV, 0, st);
    DFL_TRY(qk_rope(q, st));
  }
  ctx->sq().append(C);
  return DFL_OK;
}

// Context rows from one row-major buffer (src: [C][n_target_feat * H], or [C][H] already
// fused), or with feats set from the tapped layers' own tensors (src unused).
static int ingest(dfl_ctx* ctx, const uint16_t* src, int C, bool fused, void* stream,
                  const FeatPtrs* feats = nullptr) {
  if (!ctx || (!src && !feats && C > 0)) return fail(DFL_EINVAL, "dfl_ingest: null argument");
  if (C < 0) return fail(DFL_EINVAL, "dfl_ingest: negative row count");
  if (!ctx->sq().window && (long long)ctx->sq().len + C > ctx->cfg.max_ctx)
    return fail(DFL_ERANGE, "dfl_ingest: context rows " + std::to_string(ctx->sq().len + C) +
                                " exceed max_ctx " + std::to_string(ctx->cfg.max_ctx));
  DFL_TRY(layers_ready(ctx, "dfl_ingest"));
  if (!fused && !ctx->fc_loaded) return fail(DFL_ESTATE, "dfl_ingest_context: fc not loaded");
  hipStream_t st = (hipStream_t)stream;
  const int H = ctx->H;
  const int K = ctx->NF * H;
  const half_t* in = reinterpret_cast<const half_t*>(src);
  ctx->sq().last_block = 0;
  // per-step context rows: stream-K kernels (any alignment: the rows are gathered into
  // fragment layout first)
  if (C > 0 && C <= SMALL_ING && (fused || ctx->w_fc_pk)) {
    DFL_TRY(ingest_small(ctx, in, C, fused, feats, st));
    DFL_TRY(check_launch("ingest"));
    ctx->sq().offset += C;
    return DFL_OK;
  }
  for (int r0 = 0; r0 < C; r0 += ctx->ing) {
    const int rows = std::min(ctx->ing, C - r0);
    if (fused) {
      FeatPtrs f{};
      f.n = 1;
      f.ld = H;
      f.p[0] = in + (size_t)r0 * H;
      {
        ProfScope ps(ctx, P_INGEST_KV, 0, st);
        launch_feats_to_afl(f, rows, H, ctx->xn, st);
      }
      DFL_TRY(ingest_kv_rows(ctx, ctx->xn, rows, r0, st));
    } else {
      // hidden_norm(fc(target_hidden)): fc output rounded to fp16 (Linear), then RMSNorm.
      // The rows (or the tapped layers' rows: feature j gives columns [jH, (j+1)H)) are
      // gathered into fragment layout (any alignment), then the tile GEMM over the packed
      // fp16 fc weight.
      FeatPtrs f{};
      if (feats) {
        f = *feats;
        for (int j = 0; j < f.n; ++j) f.p[j] += (size_t)r0 * f.ld;
      } else {
        f.n = ctx->NF;
        f.ld = K;
        for (int j = 0; j < f.n; ++j) f.p[j] = in + (size_t)r0 * K + (size_t)j * H;
      }
      {
        ProfScope ps(ctx, P_INGEST_FC, 0, st);
        launch_feats_to_afl(f, rows, H, ctx->xf, st);
      }
      DFL_TRY(tgemm(ctx, P_INGEST_FC, WT_F16, TG_F32, ctx->w_fc_pk, H, K, ctx->xf, rows,
                    tile_f32(ctx->fc32, H), st));
      {
        ProfScope ps(ctx, P_INGEST_FC, 0, st);
        launch_fc_norm_rows(ctx->fc32, rows, H, ctx->hidden_norm, ctx->cfg.rms_eps, ctx->xn, st);
      }
      DFL_TRY(ingest_kv_rows(ctx, ctx->xn, rows, r0, st));
    }
    ctx->sq().append(rows);
  }
  DFL_TRY(check_launch("ingest"));
  ctx->sq().offset += C;
  return DFL_OK;
}

int dfl_ingest_context(dfl_ctx* ctx, const uint16_t* target_hidden, int32_t C, void* stream) {
  return ingest(ctx, target_hidden, C, false, stream);
}

int dfl_ingest_fused(dfl_ctx* ctx, const uint16_t* ctx_hidden, int32_t C, void* stream) {
  return ingest(ctx, ctx_hidden, C, true, stream);
}

static int feat_ptrs(const uint16_t* const* feats, int32_t n_feats, int64_t ld, int H,
                     const char* who, FeatPtrs& f) {
  const std::string w(who);
  if (!feats) return fail(DFL_EINVAL, w + ": null feature array");
  if (n_feats < 1 || n_feats > MAX_FEATS)
    return fail(DFL_EINVAL, w + ": n_feats must be in [1, " + std::to_string(MAX_FEATS) + "]");
  if (ld < H || ld % 8)
    return fail(DFL_EINVAL, w + ": row stride must be >= hidden and a multiple of 8");
  f.n = n_feats;
  f.ld = ld;
  for (int j = 0; j < n_feats; ++j) {
    if (!feats[j]) return fail(DFL_EINVAL, w + ": null feature pointer " + std::to_string(j));
    if (reinterpret_cast<uintptr_t>(feats[j]) & 15)
      return fail(DFL_EINVAL, w + ": feature " + std::to_string(j) + " not 16-byte aligned");
    f.p[j] = reinterpret_cast<const half_t*>(feats[j]);
  }
  return DFL_OK;
}

int dfl_ingest_features(dfl_ctx* ctx, const uint16_t* const* feats, int32_t n_feats,
                        int64_t ld, int32_t C, void* stream) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_ingest_features: null argument");
  FeatPtrs f{};
  DFL_TRY(feat_ptrs(feats, n_feats, ld, ctx->H, "dfl_ingest_features", f));
  if (n_feats != ctx->NF)
    return fail(DFL_EINVAL, "dfl_ingest_features: " + std::to_string(n_feats) +
                                " features, the fc expects " + std::to_string(ctx->NF));
  return ingest(ctx, nullptr, C, false, stream, &f);
}

int dfl_concat_features(const uint16_t* const* feats, int32_t n_feats, int64_t ld, int32_t C,
                        int32_t H, uint16_t* out, void* stream) {
  if (!out || C < 0 || H <= 0 || H % 8)
    return fail(DFL_EINVAL, "dfl_concat_features: bad output, rows or hidden (H % 8 == 0)");
  FeatPtrs f{};
  DFL_TRY(feat_ptrs(feats, n_feats, ld, H, "dfl_concat_features", f));
  if (reinterpret_cast<uintptr_t>(out) & 15)
    return fail(DFL_EINVAL, "dfl_concat_features: output not 16-byte aligned");
  if (C == 0) return DFL_OK;
  launch_concat_feats(f, C, H, reinterpret_cast<half_t*>(out), (hipStream_t)stream);
  return check_launch("dfl_concat_features");
}

// One draft block for sequences seq0 .. seq0 + n_seq - 1 together: B rows each, stacked
// sequence-major (row = i * B + b).  The projections run once over all n_seq * B rows;
// Q/K norm + RoPE and attention run per sequence against its own cache.
static int draft_rows(dfl_ctx* ctx, const char* who, int seq0, int n_seq,
                      const uint16_t* noise_emb, const int32_t* ids, int32_t B,
                      uint16_t* out_hidden, uint16_t* out_prenorm, float* out_logits,
                      int32_t* out_ids, void* stream) {
  const std::string w(who);
  if (B <= 0 || B > ctx->Bmax)
    return fail(DFL_ERANGE, w + ": block size " + std::to_string(B) + " outside [1, max_block=" +
                                std::to_string(ctx->Bmax) + "]");
  if ((noise_emb == nullptr) == (ids == nullptr))
    return fail(DFL_EINVAL, w + ": pass exactly one of noise_emb / ids");
  if (ids && !ctx->embed) return fail(DFL_ESTATE, w + ": embedding not loaded");
  if (!ctx->head_loaded) return fail(DFL_ESTATE, w + ": final norm not loaded");
  if ((out_logits || out_ids) && !ctx->w_lm) return fail(DFL_ESTATE, w + ": lm_head not loaded");
  for (int i = 0; i < n_seq; ++i)
    if (ctx->seqs[seq0 + i].window ? B > ctx->seqs[seq0 + i].window
                                   : ctx->seqs[seq0 + i].len + B > ctx->cap)
      return fail(DFL_ERANGE, w + ": cache capacity exceeded, or block larger than the cache "
                                  "window (sequence " + std::to_string(seq0 + i) + ")");
  DFL_TRY(layers_ready(ctx, who));

  hipStream_t st = (hipStream_t)stream;
  const int H = ctx->H, NH = ctx->NH, NKV = ctx->NKV, F = ctx->F, NQ = NH * 128;
  const int M = n_seq * B;
  const bool stacked = M > STACK_MIN_ROWS;   // compute-bound: tile GEMMs + row epilogues
  const bool fuse_rope = !stacked && n_seq == 1 && M <= 32;   // rope in the qkv epilogue
  const float eps = ctx->cfg.rms_eps;
  // x = embedding rows (residual stream); rnorm = 1/rms(x).  Every projection whose input
  // is an RMSNorm output applies the norm on its activation load.
  {
    ProfScope ps(ctx, P_ROWS, 0, st);
    launch_embed_norm(ids, ctx->embed, reinterpret_cast<const half_t*>(noise_emb), M, H, ctx->V,
                      ctx->layers[0].in_norm, eps, ctx->x, nullptr, ctx->rnorm, ctx->err, st,
                      fuse_rope ? ctx->rope_cs : nullptr, ctx->seqs[seq0].offset,
                      std::log2(ctx->cfg.rope_theta), ctx->rope_freqs());
  }

  // Attention key split.  One sequence: about one workgroup per CU ((chunks x KV heads) ~
  // CUs).  Several sequences in one launch: two per CU.  A long chunk spans several LDS
  // stages, which keeps the per-chunk partials (the merge's input) few.  The launch's grid
  // enumerates only the chunks that exist (AttnArgs::chunk0).
  // Several sequences: one chunk length for all, the shortest (a multiple of 32 keys) that
  // needs at most 2 * ceil(n_cu / NKV) chunks in all, so the chunk workgroups fill two per
  // CU in a single round and none of them is longer than the others.
  auto attn_splits = [&](const int* L, int n, int* n_split) {
    if (n == 1) {
      // one workgroup per CU: at long contexts a chunk spans several LDS stages, which
      // beats twice the chunks (and partials) at two workgroups per CU (32K keys: 1154 vs
      // 1220 us per block)
      n_split[0] = (ctx->n_cu + NKV - 1) / NKV;
    } else {
      const long long target = std::max(n, 2 * ((ctx->n_cu + NKV - 1) / NKV));
      long long total = 0;
      for (int i = 0; i < n; ++i) total += L[i];
      long long kb = std::max(1LL, (total + 32 * target - 1) / (32 * target));
      for (;; ++kb) {
        long long need = 0;
        for (int i = 0; i < n; ++i) need += (L[i] + 32 * kb - 1) / (32 * kb);
        if (need <= target) break;
      }
      for (int i = 0; i < n; ++i) n_split[i] = (int)((L[i] + 32 * kb - 1) / (32 * kb));
    }
    for (int i = 0; i < n; ++i)
      n_split[i] = std::max(1, std::min(std::min(MAX_CHUNKS, (L[i] + 31) / 32), n_split[i]));
  };


  for (int l = 0; l < ctx->active; ++l) {
    Layer& Ly = ctx->layers[l];
    // q|k|v = input_layernorm(x) @ [Wq; Wk; Wv]^T  (fp16 out, or fp32 rows for stacked blocks)
    if (stacked) {
      {
        ProfScope ps(ctx, P_ROWS, 0, st);
        launch_apply_norm(ctx->x, l > 0 ? ctx->sk_ss : nullptr, H / 32, eps, Ly.in_norm, M, H,
                          ctx->h, st, l > 0 ? nullptr : ctx->rnorm, /*h_afl=*/true);
      }
      DFL_TRY(tgemm(ctx, P_GEMM_TILE, WT_INT8, TG_F32, Ly.w_qkv, ctx->NQKV, H, ctx->h, M,
                    tile_f32(ctx->y32, ctx->NQKV), st));
    } else if (fuse_rope) {
      // one sequence: the per-head Q/K norm, RoPE and cache scatter run in the epilogue
      RopeEpi re{};
      re.Q = ctx->Q;
      re.cs = ctx->rope_cs;
      re.q_norm = Ly.q_norm;
      re.k_norm = Ly.k_norm;
      re.eps = eps;
      re.log2_theta = std::log2(ctx->cfg.rope_theta);
      re.NH = NH;
      re.NKV = NKV;
      re.cap = ctx->cap;
      rope_seq(ctx, seq0, Ly, ctx->seqs[seq0].offset, B, re.sq);
      DFL_TRY(skgemm(ctx, P_GEMM_W8, WT_INT8, EPI_QKROPE, ctx->sk_qkv, Ly.w_qkv, Ly.s_qkv,
                     ctx->NQKV, H / 32, ctx->x, H, M, Ly.in_norm, /*rn_from_ss=*/l > 0, nullptr,
                     0, nullptr, nullptr, nullptr, st, nullptr, nullptr, &re));
    } else {
      DFL_TRY(skgemm(ctx, P_GEMM_W8, WT_INT8, EPI_STORE, ctx->sk_qkv, Ly.w_qkv, Ly.s_qkv, ctx->NQKV,
                     H / 32, ctx->x, H, M, Ly.in_norm, /*rn_from_ss=*/l > 0, ctx->qkvbuf,
                     ctx->NQKV, nullptr, nullptr, nullptr, st));
    }
    // Q/K norm + RoPE and attention, up to SEQ_MAX sequences per launch
    for (int g0 = 0; g0 < n_seq; g0 += SEQ_MAX) {
      const int gn = std::min(SEQ_MAX, n_seq - g0);
      QKRopeArgs q{};
      if (stacked) {
        q.qkv32 = ctx->y32 + (size_t)g0 * B * ctx->NQKV;
        q.oscale = Ly.s_qkv;
      } else {
        q.qkv16 = ctx->qkvbuf + (size_t)g0 * B * ctx->NQKV;
      }
      q.M = B;
      q.N = ctx->NQKV;
      q.n_seq = gn;
      q.col_slot0 = 0;
      q.slot0 = 0;
      q.n_slots = NH + 2 * NKV;
      q.NH = NH;
      q.NKV = NKV;
      q.q_norm = Ly.q_norm;
      q.k_norm = Ly.k_norm;
      q.eps = eps;
      q.log2_theta = std::log2(ctx->cfg.rope_theta);
      q.inv_freq = ctx->rope_freqs();
      q.Q = ctx->Q + (size_t)g0 * NH * B * 128;
      q.cap = ctx->cap;
      AttnArgs at{};
      at.Q = q.Q;
      at.B = B;
      at.NH = NH;
      at.NKV = NKV;
      at.cap = ctx->cap;
      at.n_seq = gn;
      at.scale_log2 = (float)(1.4426950408889634 / std::sqrt(128.0));
      at.Op = ctx->Op;
      at.Ml = ctx->Ml;
      at.O = ctx->attn;
      at.n_cu = ctx->n_cu;
      at.lds_max = ctx->lds_max;
      long long kv_bytes = 0;
      int Ls[SEQ_MAX], n_split[SEQ_MAX];
      for (int i = 0; i < gn; ++i) {
        SeqState after = ctx->seqs[seq0 + g0 + i];
        after.append(B);
        Ls[i] = after.key_range();
      }
      attn_splits(Ls, gn, n_split);
      at.chunk0[0] = 0;
      for (int i = 0; i < gn; ++i) {
        const int sidx = seq0 + g0 + i;
        rope_seq(ctx, sidx, Ly, ctx->seqs[sidx].offset, B, q.sq[i]);
        SeqState after = ctx->seqs[sidx];   // the block's rows appended (evicting as the
        after.append(B);                     // window requires)
        AttnSeq& as = at.sq[i];
        as.Kc = q.sq[i].Kc;
        as.Vt = q.sq[i].Vt;
        as.L = after.key_range();
        as.ring_S = after.sink;
        as.ring_W = after.window;
        as.ring_j = after.window ? (int)(after.ring_j % after.window) : 0;
        as.ring_len = std::max(0, after.len - after.sink);
        as.sink_len = std::min(after.len, after.sink);
        as.o_row0 = (g0 + i) * B;
        const int kblocks = (as.L + 31) / 32;
        as.chunk = ((kblocks + n_split[i] - 1) / n_split[i]) * 32;
        as.n_chunks = (as.L + as.chunk - 1) / as.chunk;
        at.max_chunks = std::max(at.max_chunks, as.n_chunks);
        at.chunk0[i + 1] = at.chunk0[i] + as.n_chunks;
        kv_bytes += 2LL * NKV * as.L * 128 * 2;
      }
      if (!fuse_rope) {
        ProfScope ps(ctx, P_QK_ROPE, 0, st);
        DFL_TRY(qk_rope(q, st));
      }
      ProfScope ps(ctx, P_ATTN, kv_bytes, st);
      DFL_TRY(block_attention(at, st));
    }
    if (stacked) {
      // the same steps as tile GEMMs with the RESID / SWIGLU epilogues fused; the RMSNorm
      // of a GEMM's input is a row kernel (row sums of squares per 32-column tile)
      DFL_TRY(tgemm(ctx, P_GEMM_TILE, WT_INT8, TG_RESID, Ly.w_o, H, NQ, ctx->attn, M,
                    tile_resid(Ly.s_o, ctx->x, ctx->sk_ss), st));
      {
        ProfScope ps(ctx, P_ROWS, 0, st);
        launch_apply_norm(ctx->x, ctx->sk_ss, H / 32, eps, Ly.post_norm, M, H, ctx->h, st,
                          nullptr, /*h_afl=*/true);
      }
      TileArgs sw{};
      sw.scale = Ly.s_gu;
      sw.out = ctx->act;
      DFL_TRY(tgemm(ctx, P_GEMM_TILE, WT_INT8, TG_SWIGLU, Ly.w_gu, 2 * F, H, ctx->h, M, sw, st));
      DFL_TRY(tgemm(ctx, P_GEMM_TILE, WT_INT8, TG_RESID, Ly.w_down, H, F, ctx->act, M,
                    tile_resid(Ly.s_down, ctx->x, ctx->sk_ss), st));
    } else {
      // x += attn @ Wo^T ; per-tile row sums of squares of x -> sk_ss
      DFL_TRY(skgemm(ctx, P_GEMM_W8, WT_INT8, EPI_RESID, ctx->sk_o, Ly.w_o, Ly.s_o, H, NQ / 32,
                     ctx->attn, NQ, M, nullptr, false, nullptr, H, ctx->x, nullptr, nullptr, st));
      // act = silu(gate(post_norm(x))) * up(post_norm(x))
      DFL_TRY(skgemm(ctx, P_GEMM_W8, WT_INT8, EPI_SWIGLU, ctx->sk_gu, Ly.w_gu, Ly.s_gu, 2 * F,
                     H / 32, ctx->x, H, M, Ly.post_norm, true, ctx->act, F, nullptr, nullptr,
                     nullptr, st));
      // x += act @ Wdown^T ; per-tile row sums of squares of x -> sk_ss
      DFL_TRY(skgemm(ctx, P_GEMM_W8, WT_INT8, EPI_RESID, ctx->sk_down, Ly.w_down, Ly.s_down, H,
                     F / 32, ctx->act, F, M, nullptr, false, nullptr, H, ctx->x, nullptr, nullptr,
                     st));
    }
  }
  // row sums of squares of x: per 64 columns (stream-K RESID) or 32 (tile RESID)
  const int ss_tiles = stacked ? H / 32 : H / 64;
  // a sampling call: its own noise seed (splitmix64 of the seed and the call count)
  ctx->call_invT = out_ids ? ctx->samp_invT : 0.f;
  if (ctx->call_invT > 0.f) {
    unsigned long long z = ctx->samp_seed + 0x9E3779B97F4A7C15ull * (++ctx->samp_calls);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    ctx->call_seed = (uint32_t)(z ^ (z >> 31));
  }
  if ((out_logits || out_ids) && stacked) {
    // stacked blocks: final norm into fragment-layout rows, then the lm_head tile GEMM with
    // the argmax keys (and the fp32 logits if asked for)
    {
      ProfScope ps(ctx, P_ROWS, 0, st);
      launch_apply_norm(ctx->x, ctx->sk_ss, ss_tiles, ctx->cfg.rms_eps, ctx->final_norm, M, H,
                        ctx->h, st, nullptr, /*h_afl=*/true);
    }
    TileArgs lm = tile_f32(out_logits, ctx->V);
    lm.keys = out_ids ? ctx->lm_parts : nullptr;
    int parts = 0;
    DFL_TRY(tgemm(ctx, P_LM_HEAD, WT_F16, out_ids ? TG_ARGMAX : TG_F32, ctx->w_lm, ctx->V, H,
                  ctx->h, M, lm, st, &parts));
    if (out_ids) {
      ProfScope ps(ctx, P_ROWS, 0, st);
      launch_argmax_parts(ctx->lm_parts, parts, M, out_ids, st);
    }
  } else if (out_logits || out_ids) {
    bool ids_done = false;
    DFL_TRY(skgemm(ctx, P_LM_HEAD, WT_F16, EPI_ARGMAX, ctx->sk_lm, ctx->w_lm, nullptr, ctx->V, H / 16,
           ctx->x, H, M, ctx->final_norm, true, nullptr, 0, nullptr, out_logits,
           out_ids ? ctx->keys : nullptr, st, out_ids, &ids_done));
    if (out_ids && !ids_done) {
      ProfScope ps(ctx, P_ROWS, 0, st);
      launch_argmax_finalize(ctx->keys, M, out_ids, st);
    }
  }
  if (out_hidden) {
    ProfScope ps(ctx, P_ROWS, 0, st);
    launch_apply_norm(ctx->x, ctx->sk_ss, ss_tiles, ctx->cfg.rms_eps, ctx->final_norm, M, H,
                      reinterpret_cast<half_t*>(out_hidden), st);
  }
  if (out_prenorm) {
    ProfScope ps(ctx, P_ROWS, 0, st);
    launch_afl_to_rows(ctx->x, M, H, reinterpret_cast<half_t*>(out_prenorm), st);
  }
  DFL_TRY(check_launch(who));
  // the block's rows stay written but uncommitted: append + trim (a window keeps the
  // rows the block evicted evicted, as the reference's trim after update_and_fetch does)
  for (int i = 0; i < n_seq; ++i) {
    SeqState& q = ctx->seqs[seq0 + i];
    q.append(B);
    q.trim(B);
    q.last_block = B;
  }
  return DFL_OK;
}

int dfl_draft_block(dfl_ctx* ctx, const uint16_t* noise_emb, const int32_t* ids, int32_t B,
                    uint16_t* out_hidden, uint16_t* out_prenorm, float* out_logits,
                    int32_t* out_ids, void* stream) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_draft_block: null context");
  return draft_rows(ctx, "dfl_draft_block", ctx->cur, 1, noise_emb, ids, B, out_hidden,
                    out_prenorm, out_logits, out_ids, stream);
}

int dfl_draft_batch(dfl_ctx* ctx, int32_t n_seq, const uint16_t* noise_emb, const int32_t* ids,
                    int32_t B, uint16_t* out_hidden, uint16_t* out_prenorm, float* out_logits,
                    int32_t* out_ids, void* stream) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_draft_batch: null context");
  if (n_seq < 1 || n_seq > ctx->S)
    return fail(DFL_ERANGE, "dfl_draft_batch: n_seq must be in [1, max_seqs=" +
                                std::to_string(ctx->S) + "]");
  return draft_rows(ctx, "dfl_draft_batch", 0, n_seq, noise_emb, ids, B, out_hidden, out_prenorm,
                    out_logits, out_ids, stream);
}

int dfl_select_seq(dfl_ctx* ctx, int32_t seq) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_select_seq: null context");
  if (seq < 0 || seq >= ctx->S)
    return fail(DFL_ERANGE, "dfl_select_seq: sequence " + std::to_string(seq) + " outside [0, " +
                                std::to_string(ctx->S) + ")");
  ctx->cur = seq;
  return DFL_OK;
}

int dfl_set_num_layers(dfl_ctx* ctx, int32_t n) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_set_num_layers: null context");
  if (n < 1 || n > ctx->NL)
    return fail(DFL_ERANGE, "dfl_set_num_layers: n must be in [1, " + std::to_string(ctx->NL) + "]");
  ctx->active = n;
  return DFL_OK;
}

int dfl_cache_trim(dfl_ctx* ctx, int32_t n) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_trim: null context");
  if (n < 0) return fail(DFL_EINVAL, "dfl_cache_trim: negative count");
  SeqState& q = ctx->sq();
  q.trim(n);   // DFlashKVCache.trim clamps the length at 0
  q.offset -= n;
  q.last_block = 0;
  return DFL_OK;
}

int dfl_cache_commit(dfl_ctx* ctx, int32_t n) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_commit: null context");
  SeqState& q = ctx->sq();
  if (n < 0 || n > q.last_block)
    return fail(DFL_EINVAL, "dfl_cache_commit: n must be in [0, rows of the last block]");
  if (!q.window && q.len + n > ctx->cfg.max_ctx)
    return fail(DFL_ERANGE, "dfl_cache_commit: max_ctx exceeded");
  q.append(n);   // the block's rows are still in their cache rows
  q.offset += n;
  q.last_block = 0;
  return DFL_OK;
}

int dfl_cache_reset(dfl_ctx* ctx) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_reset: null context");
  const int sink = ctx->sq().sink, window = ctx->sq().window;
  ctx->sq() = SeqState{};
  ctx->sq().sink = sink;
  ctx->sq().window = window;
  return DFL_OK;
}

int dfl_cache_set_window(dfl_ctx* ctx, int32_t sink, int32_t window) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_set_window: null context");
  if (sink < 0 || window < 0) return fail(DFL_EINVAL, "dfl_cache_set_window: negative size");
  if ((long long)sink + window > ctx->cap)
    return fail(DFL_ERANGE, "dfl_cache_set_window: sink + window exceed the cache capacity");
  ctx->sq() = SeqState{};
  if (sink > 0 && window > 0) {   // the reference evicts only when both are set
    ctx->sq().sink = sink;
    ctx->sq().window = window;
  }
  return DFL_OK;
}

int dfl_cache_set_offset(dfl_ctx* ctx, int64_t offset) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_set_offset: null context");
  if (offset < 0) return fail(DFL_EINVAL, "dfl_cache_set_offset: negative offset");
  ctx->sq().offset = offset;
  ctx->sq().last_block = 0;
  return DFL_OK;
}

int dfl_cache_state(const dfl_ctx* ctx, int32_t* len, int64_t* offset) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_state: null context");
  const SeqState& q = ctx->seqs[ctx->cur];
  if (len) *len = q.len;
  if (offset) *offset = q.offset;
  return DFL_OK;
}

int dfl_cache_rows(const dfl_ctx* ctx, int32_t* rows, int32_t max_rows, int32_t* n) {
  if (!ctx || !n) return fail(DFL_EINVAL, "dfl_cache_rows: null argument");
  const SeqState& q = ctx->seqs[ctx->cur];
  *n = q.len;
  if (!rows) return DFL_OK;
  if (max_rows < q.len) return fail(DFL_ERANGE, "dfl_cache_rows: buffer too small");
  const int ns = q.window ? std::min(q.len, q.sink) : q.len;
  for (int i = 0; i < ns; ++i) rows[i] = i;
  const int rl = q.len - ns;   // ring rows, oldest first
  for (int i = 0; i < rl; ++i) {
    const long long j = q.ring_j - rl + i;
    rows[ns + i] = q.sink + (int)(((j % q.window) + q.window) % q.window);
  }
  return DFL_OK;
}

int dfl_cache_kv(const dfl_ctx* ctx, int32_t layer, uint16_t** k, uint16_t** vt, int32_t* cap) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_kv: null context");
  if (layer < 0 || layer >= ctx->NL) return fail(DFL_ERANGE, "dfl_cache_kv: layer out of range");
  if (k) *k = reinterpret_cast<uint16_t*>(ctx->kc(ctx->layers[layer], ctx->cur));
  if (vt) *vt = reinterpret_cast<uint16_t*>(ctx->vt(ctx->layers[layer], ctx->cur));
  if (cap) *cap = ctx->cap;
  return DFL_OK;
}

int dfl_profile_enable(dfl_ctx* ctx, int32_t on) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_profile_enable: null context");
  if (on < 0 || on > 2) return fail(DFL_EINVAL, "dfl_profile_enable: mode must be 0, 1 or 2");
  ctx->prof = on;
  return DFL_OK;
}

int dfl_profile_read(dfl_ctx* ctx, int32_t max_cat, char* names, double* total_ms,
                     int64_t* launches, int64_t* bytes, int32_t* n_cat) {
  if (!ctx || !n_cat) return fail(DFL_EINVAL, "dfl_profile_read: null argument");
  const int nc = std::min<int>(max_cat, P_N);
  std::vector<double> ms(P_N, 0.0);
  std::vector<long long> cnt(P_N, 0), by(P_N, 0);
  int rc = DFL_OK;
  for (auto& r : ctx->recs) {
    float t = 0.f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&t, r.a, r.b) != hipSuccess)
      rc = fail(DFL_EHIP, "dfl_profile_read: event timing failed");
    ms[r.cat] += t;
    cnt[r.cat] += 1;
    by[r.cat] += r.bytes;
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  ctx->recs.clear();
  for (int i = 0; i < nc; ++i) {
    if (names) {
      std::strncpy(names + 32 * i, kProfNames[i], 31);
      names[32 * i + 31] = 0;
    }
    if (total_ms) total_ms[i] = ms[i];
    if (launches) launches[i] = cnt[i];
    if (bytes) bytes[i] = by[i];
  }
  *n_cat = nc;
  return rc;
}

int dfl_embed_block(dfl_ctx* ctx, const int32_t* ids, int32_t B, const void* correction_logits,
                    int32_t logits_dtype, int32_t V, int32_t top_k, uint16_t* out_noise,
                    void* stream) {
  const std::string w = "dfl_embed_block";
  if (!ctx || !ids || !out_noise) return fail(DFL_EINVAL, w + ": null argument");
  if (!ctx->embed) return fail(DFL_ESTATE, w + ": embedding not loaded");
  if (B < 1 || B > 65535) return fail(DFL_EINVAL, w + ": block rows must be in [1, 65535]");
  if (correction_logits) {
    if (logits_dtype < 0 || logits_dtype > 2)
      return fail(DFL_EINVAL, w + ": logits_dtype must be 0 (fp32), 1 (fp16) or 2 (bf16)");
    if (top_k < 1 || top_k > SA_TOPK_MAX)
      return fail(DFL_EINVAL, w + ": top_k must be in [1, " + std::to_string(SA_TOPK_MAX) + "]");
    if (V < top_k || V > ctx->V)
      return fail(DFL_EINVAL, w + ": logits length must be in [top_k, vocab]");
  }
  launch_embed_block(ids, B, ctx->embed, ctx->V, ctx->H, correction_logits, logits_dtype, V,
                     top_k, ctx->sa_cand, reinterpret_cast<half_t*>(out_noise), ctx->err,
                     (hipStream_t)stream);
  return check_launch(w.c_str());
}

}  // extern "C"

// Candidate keys of the allocation-free soft anchor: one fixed array per GPU (the topk scan
// writes every entry before the embedding kernel reads it, so nothing needs clearing).
// Host code uses the per-device address from hipGetSymbolAddress, never the array's name.
namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
static __device__ __align__(256) unsigned long long scratch[SA_BLOCKS * SA_TOPK_MAX];
std::mutex g_scratch_mu;
unsigned long long* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// This device's copy of `scratch`, resolved once per device (with that device current).
int noalloc_scratch(unsigned long long** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DFL_EHIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return fail(DFL_EINVAL, "dfl_embed_block_noalloc: device index outside [0, 64)");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(DFL_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<unsigned long long*>(p);
  }
  *out = g_scratch_ptr[dev];
  return DFL_OK;
}
}  // namespace

extern "C" {

int dfl_embed_block_noalloc(const int32_t* ids, int32_t B, const uint16_t* embed, int32_t Vemb,
                            int32_t H, const void* correction_logits, int32_t logits_dtype,
                            int32_t V, int32_t top_k, uint16_t* out_noise, int32_t* err_flags,
                            void* stream) {
  if (!ids || !embed || !out_noise || !err_flags)
    return fail(DFL_EINVAL, "dfl_embed_block_noalloc: null argument");
  if (Vemb < 1 || H < 8 || H % 8 || (reinterpret_cast<uintptr_t>(embed) & 15))
    return fail(DFL_EINVAL, "dfl_embed_block_noalloc: embedding must have >= 1 row, H a "
                            "multiple of 8 and 16-byte alignment");
  if (B < 1 || B > 65535)
    return fail(DFL_EINVAL, "dfl_embed_block_noalloc: block rows must be in [1, 65535]");
  if (correction_logits) {
    if (logits_dtype < 0 || logits_dtype > 2)
      return fail(DFL_EINVAL, "dfl_embed_block_noalloc: logits_dtype must be 0 (fp32), 1 (fp16) "
                              "or 2 (bf16)");
    if (top_k < 1 || top_k > SA_TOPK_MAX)
      return fail(DFL_EINVAL, "dfl_embed_block_noalloc: top_k must be in [1, " +
                                  std::to_string(SA_TOPK_MAX) + "] (the fixed candidate array "
                                  "holds 64 x 8 keys)");
    if (V < top_k || V > Vemb)
      return fail(DFL_EINVAL, "dfl_embed_block_noalloc: logits length must be in [top_k, Vemb]");
  }
  unsigned long long* cand = nullptr;
  DFL_TRY(noalloc_scratch(&cand));
  launch_embed_block(ids, B, reinterpret_cast<const half_t*>(embed), Vemb, H, correction_logits,
                     logits_dtype, V, top_k, cand, reinterpret_cast<half_t*>(out_noise),
                     reinterpret_cast<int*>(err_flags), (hipStream_t)stream);
  return check_launch("dfl_embed_block_noalloc");
}

int dfl_set_rope_scaling(dfl_ctx* ctx, int32_t type, double factor, double low_freq_factor,
                         double high_freq_factor, int32_t original_max_position_embeddings) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_set_rope_scaling: null context");
  if (type == DFL_ROPE_DEFAULT) {
    ctx->rope_scaled = false;
    return DFL_OK;
  }
  if (type != DFL_ROPE_LINEAR && type != DFL_ROPE_LLAMA3)
    return fail(DFL_EINVAL, "dfl_set_rope_scaling: unknown RoPE type " + std::to_string(type));
  if (!(factor > 0.0)) return fail(DFL_EINVAL, "dfl_set_rope_scaling: factor must be positive");
  if (type == DFL_ROPE_LLAMA3 &&
      (!(high_freq_factor > low_freq_factor) || !(low_freq_factor > 0.0) ||
       original_max_position_embeddings <= 0))
    return fail(DFL_EINVAL, "dfl_set_rope_scaling: llama3 needs 0 < low_freq_factor < "
                            "high_freq_factor and a positive original context length");
  const double theta = ctx->cfg.rope_theta;
  const double pi = 3.14159265358979323846;
  double f[64];
  for (int j = 0; j < 64; ++j) {
    // the unscaled frequency of pair j, theta^(-2j/128), as the kernels compute it
    const double base = std::exp2(-(double)j * (1.0 / 64.0) * std::log2(theta));
    if (type == DFL_ROPE_LINEAR) {   // positions scaled by 1 / factor
      f[j] = base / factor;
      continue;
    }
    // llama3 (Llama 3.1): wavelengths above original / low_freq_factor are stretched by
    // factor, those below original / high_freq_factor kept, and the band between
    // interpolated smoothly in the frequency
    const double old_len = (double)original_max_position_embeddings;
    const double low_wavelen = old_len / low_freq_factor, high_wavelen = old_len / high_freq_factor;
    const double wavelen = 2.0 * pi / base;
    if (wavelen > low_wavelen) {
      f[j] = base / factor;
    } else if (wavelen > high_wavelen && wavelen < low_wavelen) {
      const double s = (old_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
      f[j] = base * ((1.0 - s) / factor + s);
    } else {
      f[j] = base;
    }
  }
  DFL_HIP(hipMemcpy(ctx->rope_inv, f, sizeof f, hipMemcpyHostToDevice));
  ctx->rope_scaled = true;
  return DFL_OK;
}

int dfl_cache_assign(dfl_ctx* ctx, int32_t layer, const uint16_t* keys, const uint16_t* values,
                     int32_t L, void* stream) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_cache_assign: null context");
  if (layer < 0 || layer >= ctx->NL) return fail(DFL_ERANGE, "dfl_cache_assign: layer out of range");
  if (L < 0) return fail(DFL_EINVAL, "dfl_cache_assign: negative row count");
  if (L > 0 && !keys && !values) return fail(DFL_EINVAL, "dfl_cache_assign: no keys or values");
  SeqState& q = ctx->sq();
  // a sink + window cache keeps its first sink rows and newest window rows (the reference's
  // next update_and_fetch applies the same window before any attention reads the rows)
  int keep_head = L, keep_tail = 0;
  if (q.window && L > q.sink + q.window) {
    keep_head = q.sink;
    keep_tail = q.window;
  }
  const int kept = keep_head + keep_tail;
  if (kept > ctx->cfg.max_ctx)
    return fail(DFL_ERANGE, "dfl_cache_assign: " + std::to_string(kept) +
                                " rows exceed the cache capacity max_ctx " +
                                std::to_string(ctx->cfg.max_ctx));
  const Layer& Ly = ctx->layers[layer];
  launch_cache_assign(reinterpret_cast<const half_t*>(keys), reinterpret_cast<const half_t*>(values),
                      ctx->NKV, L, keep_head, keep_tail, ctx->kc(Ly, ctx->cur), ctx->vt(Ly, ctx->cur),
                      ctx->cap, (hipStream_t)stream);
  DFL_TRY(check_launch("dfl_cache_assign"));
  // rows in order: the sink rows, then the window rows from ring slot 0
  q.len = kept;
  q.ring_j = q.window ? std::max(0, kept - q.sink) : 0;
  q.last_block = 0;
  return DFL_OK;
}

int dfl_set_sampling(dfl_ctx* ctx, float temperature, uint64_t seed) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_set_sampling: null context");
  if (!(temperature >= 0.f) || std::isinf(temperature))
    return fail(DFL_EINVAL, "dfl_set_sampling: temperature must be a finite value >= 0");
  // greedy below 1e-5, as sample() does (dflash.py:133-136)
  ctx->samp_invT = temperature < 1e-5f ? 0.f : 1.0f / temperature;
  ctx->samp_seed = seed;
  ctx->samp_calls = 0;
  return DFL_OK;
}

int dfl_test_queue_timeout(dfl_ctx* ctx, int32_t on) {
  if (!ctx) return fail(DFL_EINVAL, "dfl_test_queue_timeout: null context");
  ctx->test_queue_timeout = on != 0;
  return DFL_OK;
}

int dfl_device_errors(dfl_ctx* ctx, int32_t* flags, void* stream) {
  if (!ctx || !flags) return fail(DFL_EINVAL, "dfl_device_errors: null argument");
  hipStream_t st = (hipStream_t)stream;
  int v = 0;
  DFL_HIP(hipMemcpyAsync(&v, ctx->err, sizeof(int), hipMemcpyDeviceToHost, st));
  DFL_HIP(hipStreamSynchronize(st));
  DFL_HIP(hipMemsetAsync(ctx->err, 0, sizeof(int), st));
  *flags = v;
  return DFL_OK;
}

}  // extern "C"
