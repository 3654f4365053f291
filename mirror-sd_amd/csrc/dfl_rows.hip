// Row-wise kernels of the draft block: embedding + RMSNorm, split-K reduction with
// residual add and the following RMSNorm, per-head Q/K RMSNorm + neox RoPE with the
// KV-cache scatter, and the argmax finaliser.
//
// fp16 rounding points follow the MLX graph of mirror_sd/dflash.py: every Linear,
// RMSNorm, RoPE and residual add produces an fp16 tensor; internal math is fp32.
#include "dfl_common.h"
#include "dfl_kernels.h"
#include "dfl_check.h"

namespace dfl {

constexpr int ROW_THREADS = 512;
constexpr int ROW_MAXV = 16;   // hidden sizes up to 8192

__global__ __launch_bounds__(ROW_THREADS) void embed_norm_kernel(
    const int32_t* __restrict__ ids, const half_t* __restrict__ embed,
    const half_t* __restrict__ noise, int H, int V, const half_t* __restrict__ g, float eps,
    half_t* __restrict__ x, half_t* __restrict__ h, float* __restrict__ rnorm,
    int* __restrict__ err, float* __restrict__ rope_cs, long long pos0, double log2_theta,
    const double* __restrict__ inv_freq_tab) {
  __shared__ float sm[16];
  __shared__ __attribute__((aligned(16))) half_t row_s[ROW_MAXV * ROW_THREADS];
  const int b = blockIdx.x;
  const half_t* src = noise + (size_t)b * H;
  bool bad = false;
  if (ids) {
    const int id = ids[b];
    bad = id < 0 || id >= V;   // out-of-range token id: flag it, use a zero row
    src = embed + (size_t)(bad ? 0 : id) * H;
    if (bad && threadIdx.x == 0) atomicOr(err, 1);
  }
  half_t e[ROW_MAXV];
#pragma unroll
  for (int i = 0; i < ROW_MAXV; ++i) {
    const int k = threadIdx.x + i * ROW_THREADS;
    e[i] = (k < H && !bad) ? src[k] : (half_t)0.0f;
  }
  if (rope_cs && threadIdx.x < 64) {
    // RoPE angles of row b for the fused qkv epilogue (while the row's loads are in
    // flight), in fp64 as qk_rope_kernel computes them: position pos0 + b times
    // theta^(-j/64), or the scaled frequency table
    const int j = threadIdx.x;
    const double inv_freq =
        inv_freq_tab ? inv_freq_tab[j] : exp2(-(double)j * (1.0 / 64.0) * log2_theta);
    double sd, cd;
    sincos((double)(pos0 + b) * inv_freq, &sd, &cd);
    rope_cs[2 * (b * 64 + j)] = (float)cd;
    rope_cs[2 * (b * 64 + j) + 1] = (float)sd;
  }
  float v[ROW_MAXV];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < ROW_MAXV; ++i) {
    const int k = threadIdx.x + i * ROW_THREADS;
    v[i] = 0.f;
    if (k < H) {
      row_s[k] = e[i];
      v[i] = h2f(e[i]);
      ss += v[i] * v[i];
    }
  }
  ss = block_sum(ss, sm);   // (its barriers also complete row_s)
  // residual stream in the activation fragment layout, 16-byte entries of 8 columns
  for (int c = threadIdx.x; c < H / 8; c += ROW_THREADS)
    *reinterpret_cast<u32x4*>(x + afl_index(b, 8 * c, H)) =
        *reinterpret_cast<const u32x4*>(row_s + 8 * c);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  if (rnorm && threadIdx.x == 0) rnorm[b] = r;
  if (!h) return;
#pragma unroll
  for (int i = 0; i < ROW_MAXV; ++i) {
    const int k = threadIdx.x + i * ROW_THREADS;
    if (k < H) h[(size_t)b * H + k] = rms_out(v[i], r, g[k]);
  }
}

void launch_embed_norm(const int32_t* ids, const half_t* embed, const half_t* noise, int B,
                       int H, int V, const half_t* g, float eps, half_t* x, half_t* h,
                       float* rnorm, int* err, hipStream_t st, float* rope_cs, long long pos0,
                       double log2_theta, const double* inv_freq) {
  hipLaunchKernelGGL(embed_norm_kernel, dim3(B), dim3(ROW_THREADS), 0, st, ids, embed, noise, H,
                     V, g, eps, x, h, rnorm, err, B <= 32 ? rope_cs : nullptr, pos0, log2_theta,
                     inv_freq);
}

// One wave per (KV head, source row): the row's 128 K values to its cache row, the 128 V
// values down its Vt column.
__global__ __launch_bounds__(256) void cache_assign_kernel(const half_t* __restrict__ k,
                                                           const half_t* __restrict__ v, int NKV,
                                                           int L, int keep_head, int keep_tail,
                                                           half_t* __restrict__ Kc,
                                                           half_t* __restrict__ Vt, int cap) {
  const long long wid = ((long long)blockIdx.x * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wid >= (long long)NKV * L) return;
  const int g = (int)(wid / L), r = (int)(wid - (long long)g * L);
  int dst;
  if (r < keep_head) dst = r;
  else if (r >= L - keep_tail) dst = r - (L - keep_tail) + keep_head;
  else return;   // an evicted middle row
  const size_t src = ((size_t)g * L + r) * 128;
  if (k) {
    half_t* kd = Kc + ((size_t)g * cap + dst) * 128;
    kd[lane] = k[src + lane];
    kd[lane + 64] = k[src + lane + 64];
  }
  if (v) {
    half_t* vd = Vt + (size_t)g * 128 * cap + dst;
    vd[(size_t)lane * cap] = v[src + lane];
    vd[(size_t)(lane + 64) * cap] = v[src + lane + 64];
  }
}

void launch_cache_assign(const half_t* k, const half_t* v, int NKV, int L, int keep_head,
                         int keep_tail, half_t* Kc, half_t* Vt, int cap, hipStream_t st) {
  const long long waves = (long long)NKV * L;
  if (waves == 0) return;
  hipLaunchKernelGGL(cache_assign_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, k, v,
                     NKV, L, keep_head, keep_tail, Kc, Vt, cap);
}

// x (activation fragment layout, [M][N]) -> h, row-major or (h_afl) in the fragment layout;
// with g set, h = RMSNorm(x) * g where 1/rms of row m is rnorm[m], or comes from ss
// [M/32][ss_tiles][32] (per-column-tile sums of squares).
__global__ __launch_bounds__(256) void afl_rows_kernel(const half_t* __restrict__ x,
                                                       const float* __restrict__ ss, int ss_tiles,
                                                       const float* __restrict__ rnorm,
                                                       float eps, const half_t* __restrict__ g,
                                                       int N, half_t* __restrict__ h, bool h_afl) {
  __shared__ float rr_s;
  const int m = blockIdx.y;
  if (rnorm) {
    if (threadIdx.x == 0) rr_s = rnorm[m];
    __syncthreads();
  } else if (ss) {
    if (threadIdx.x < 64) {
      const float* sp = ss + (size_t)(m >> 5) * ss_tiles * 32 + (m & 31);
      float tot = 0.f;
      for (int t = threadIdx.x; t < ss_tiles; t += 64) tot += sp[(size_t)t * 32];
      tot = wave_sum(tot);
      if (threadIdx.x == 0) rr_s = 1.0f / sqrtf(tot / (float)N + eps);
    }
    __syncthreads();
  }
  const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= N) return;
  // 4 consecutive columns (n % 4 == 0) are 4 consecutive halves of one record
  const half4_t xv = *reinterpret_cast<const half4_t*>(x + afl_index(m, n, N));
  half4_t o = xv;
  if (g) {
    const float rr = rr_s;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = rms_out(h2f(xv[j]), rr, g[n + j]);
  }
  *reinterpret_cast<half4_t*>(h + (h_afl ? afl_index(m, n, N) : (size_t)m * N + n)) = o;
}

void launch_apply_norm(const half_t* x, const float* ss, int ss_tiles, float eps, const half_t* g,
                       int M, int N, half_t* h, hipStream_t st, const float* rnorm, bool h_afl) {
  hipLaunchKernelGGL(afl_rows_kernel, dim3((N / 4 + 255) / 256, M), dim3(256), 0, st, x, ss,
                     ss_tiles, rnorm, eps, g, N, h, h_afl);
}

// Row-major concatenation [rows][nf * H] of the feature tensors (the materialised
// extract_context_feature).
__global__ __launch_bounds__(256) void concat_feats_kernel(FeatPtrs f, int H,
                                                           half_t* __restrict__ out) {
  const int r = blockIdx.y;
  const int K = f.n * H;
  const int k = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (k >= K) return;
  const int j = k / H;
  *reinterpret_cast<u32x4*>(out + (size_t)r * K + k) =
      *reinterpret_cast<const u32x4*>(f.p[j] + (size_t)r * f.ld + (k - j * H));
}

void launch_concat_feats(const FeatPtrs& f, int rows, int H, half_t* out, hipStream_t st) {
  hipLaunchKernelGGL(concat_feats_kernel, dim3((f.n * H / 8 + 255) / 256, rows), dim3(256), 0, st,
                     f, H, out);
}

// Context rows into activation fragment layout tiles for the stream-K ingest GEMMs: row r,
// column k of concat_j(f_j) (feature j gives columns [j*H, (j+1)*H), read through its row
// stride) goes to afl_index(r, k, K), K = f.n * H; rows in [rows, 32 * tiles) are zero.
// One workgroup per 32-row tile and 64-column slab, through LDS so that both sides are
// contiguous: each row's 128 bytes are read by 8 lanes, and the slab's 4 fragment records
// (4 KiB, consecutive in the layout) are written by one 16-byte store per lane.
constexpr int AFL_SLAB = 64;
__global__ __launch_bounds__(256) void feats_to_afl_kernel(FeatPtrs f, int H, int rows,
                                                           half_t* __restrict__ afl) {
  __shared__ __attribute__((aligned(16))) half_t tile[32][AFL_SLAB + 8];
  const int K = f.n * H;
  const int t = blockIdx.y, k0 = blockIdx.x * AFL_SLAB, p = threadIdx.x;
  {   // read: lane p takes row p / 8, columns k0 + 8 * (p % 8) .. + 7
    const int m = p >> 3, c = 8 * (p & 7), k = k0 + c, r = t * 32 + m;
    if (k < K) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (r < rows) {
        const int j = k / H;
        const half_t* src = f.p[j] + (size_t)r * f.ld + (k - j * H);
        if (!(reinterpret_cast<uintptr_t>(src) & 15)) {
          v = *reinterpret_cast<const u32x4*>(src);
        } else {   // a caller's buffer without 16-byte alignment: 2-byte loads
          half8_t h;
#pragma unroll
          for (int i = 0; i < 8; ++i) h[i] = src[i];
          v = __builtin_bit_cast(u32x4, h);
        }
      }
      *reinterpret_cast<u32x4*>(&tile[m][c]) = v;
    }
  }
  __syncthreads();
  {   // write: lane p stores record p / 64 of the slab, lane slot p % 64
    const int R = p >> 6, l = p & 63, m = l & 31;
    const int c = 32 * (R >> 1) + 16 * (l >> 5) + 8 * (R & 1), k = k0 + c;
    if (k < K)
      *reinterpret_cast<u32x4*>(afl + afl_index(t * 32 + m, k, K)) =
          *reinterpret_cast<const u32x4*>(&tile[m][c]);
  }
}

void launch_feats_to_afl(const FeatPtrs& f, int rows, int H, half_t* afl, hipStream_t st) {
  const int tiles = (rows + 31) / 32;
  if (tiles == 0) return;
  hipLaunchKernelGGL(feats_to_afl_kernel, dim3((f.n * H + AFL_SLAB - 1) / AFL_SLAB, tiles),
                     dim3(256), 0, st, f, H, rows, afl);
}

// hidden_norm(fc(.)) for the ingest: fc32 [rows][H] fp32 GEMM rows, rounded to fp16 (the
// Linear output), then RMSNorm (fp16(fp16(x * r) * g)) into fragment-layout tiles xn
// [ceil(rows/32)][32][H] (the K|V tile GEMM's input).
__global__ __launch_bounds__(ROW_THREADS) void fc_norm_rows_kernel(const float* __restrict__ fc32,
                                                                   int H, const half_t* __restrict__ g,
                                                                   float eps,
                                                                   half_t* __restrict__ xn) {
  __shared__ float red[16];
  const int r = blockIdx.x;
  const float* src = fc32 + (size_t)r * H;
  float v[ROW_MAXV];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < ROW_MAXV; ++i) {
    const int k = threadIdx.x + i * ROW_THREADS;
    v[i] = 0.f;
    if (k < H) {
      v[i] = h2f(f2h(src[k]));
      ss += v[i] * v[i];
    }
  }
  ss = block_sum(ss, red);
  const float rr = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
  for (int i = 0; i < ROW_MAXV; ++i) {
    const int k = threadIdx.x + i * ROW_THREADS;
    if (k < H) xn[afl_index(r, k, H)] = rms_out(v[i], rr, g[k]);
  }
}

void launch_fc_norm_rows(const float* fc32, int rows, int H, const half_t* g, float eps,
                         half_t* xn, hipStream_t st) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(fc_norm_rows_kernel, dim3(rows), dim3(ROW_THREADS), 0, st, fc32, H, g, eps,
                     xn);
}

void launch_afl_to_rows(const half_t* x, int M, int N, half_t* h, hipStream_t st) {
  hipLaunchKernelGGL(afl_rows_kernel, dim3((N / 4 + 255) / 256, M), dim3(256), 0, st, x, nullptr,
                     0, nullptr, 0.f, nullptr, N, h, false);
}


// Head slots [slot0, slot0 + n_slots) in q|k|v numbering: Q heads, then K heads, then V
// heads (slot >= NH + NKV).  The launch's blocks come in two parts: the first handles the
// Q/K slots, one item (sequence, row m, slot) per quarter wave (16 items per block); the
// rest the V slots, one workgroup per (sequence, V slot, 64 rows).  Below QKR_V_TILE_MIN rows
// (a decode step's few context rows) the 64-row V workgroups would mostly idle: there the
// Q/K part takes the V slots too, with one item per wave (4 per block), so that a small
// launch still spreads over the CUs and each lane computes one angle.
constexpr int QKR_V_TILE_MIN = 64;
struct QkRopeGrid {
  int qk0, nqk, v0, nv;      // first Q/K slot and count, first V slot and count
  int items;                 // Q/K items per block: 16 (quarter waves) or 4 (waves)
  long long qk_blocks;       // blocks of the Q/K part
  int v_tiles;               // 64-row tiles per sequence
};
__host__ __device__ inline QkRopeGrid qk_rope_grid(const QKRopeArgs& a) {
  QkRopeGrid gr;
  const int kvs = a.NH + a.NKV, end = a.slot0 + a.n_slots;
  gr.qk0 = a.slot0;
  if (a.M < QKR_V_TILE_MIN) {   // few rows: the V slots by the per-row waves too
    gr.nqk = a.n_slots;
    gr.v0 = end;
    gr.nv = 0;
  } else {
    gr.nqk = (end < kvs ? end : kvs) - a.slot0;
    if (gr.nqk < 0) gr.nqk = 0;
    gr.v0 = a.slot0 > kvs ? a.slot0 : kvs;
    gr.nv = end - gr.v0;
    if (gr.nv < 0) gr.nv = 0;
  }
  gr.items = a.M < QKR_V_TILE_MIN ? 4 : 16;
  gr.qk_blocks = ((long long)a.M * gr.nqk * a.n_seq + gr.items - 1) / gr.items;
  gr.v_tiles = (a.M + 63) / 64;
  return gr;
}

// Column of slot `slot`, element 0, and the row index of row m in the projection rows.
DFL_DEV void qk_rope_src(const QKRopeArgs& a, int sidx, int m, int slot, size_t& row, int& c0) {
  row = a.layer_cols ? (size_t)m : (size_t)sidx * a.M + m;
  c0 = (a.layer_cols ? sidx * a.layer_cols : 0) + (slot - a.col_slot0) * 128;
}

// Projection values (fp16 Linear output, as float) of row `row`, columns c .. c+E-1 (c % E ==
// 0, E = 1 or 4): rounded by the GEMM epilogue (qkv16), or here from the fp32 GEMM rows and
// the per-column scales (qkv32); for E = 4 one 8- or 16-byte load (and an 8-byte scale load).
template <int E>
DFL_DEV void qk_rope_values(const QKRopeArgs& a, size_t row, int c, float v[E]) {
  if constexpr (E == 4) {
    if (a.qkv32) {
      const floatx4 x = *reinterpret_cast<const floatx4*>(a.qkv32 + row * a.N + c);
      const half4_t sc = *reinterpret_cast<const half4_t*>(a.oscale + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = h2f(mul_f16_once(x[i], sc[i]));
    } else {
      const half4_t h = *reinterpret_cast<const half4_t*>(a.qkv16 + row * a.N + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = h2f(h[i]);
    }
  } else {
    v[0] = a.qkv32 ? h2f(mul_f16_once(a.qkv32[row * a.N + c], a.oscale[c])) : h2f(a.qkv16[row * a.N + c]);
  }
}

// Q/K item (sequence sidx, row m, slot) on a group of 64/E lanes, lane L holding head
// elements E*L .. E*L+E-1 and 64+E*L .. 64+E*L+E-1: exactly the neox RoPE pairs (d, d + 64)
// (dflash.py:263-275, split-half rotation), so the rotation is lane-local.  The row's sum
// of squares is the sum tree of a 64-lane butterfly over one pair per lane (lane d:
// v_d^2 + v_(d+64)^2, pairs combined across lane bits 5, 4, ..., 0) for either E: with E = 4
// bits 5..2 of d are the group's lane bits (xor 8, 4, 2, 1), bits 1..0 the lane's four pairs.
// Angles are computed in fp64 (pos * theta^(-j/64), or the scaled frequency table) or taken
// from the angle table.
template <int E>
DFL_DEV void qk_rope_item(const QKRopeArgs& a, int sidx, int m, int slot, int L) {
  const RopeSeq& sq = a.sq[sidx];
  const int crow = slot >= a.NH ? cache_slot(sq, a.M, m) : 0;
  if (crow < 0) return;   // the whole group: one (row, head slot) per group
  size_t row;
  int c0;
  qk_rope_src(a, sidx, m, slot, row, c0);
  const int j0 = E * L;
  float v0[E], v1[E];
  qk_rope_values<E>(a, row, c0 + j0, v0);
  qk_rope_values<E>(a, row, c0 + j0 + 64, v1);
  if (slot >= a.NH + a.NKV) {   // V head (few rows): down its Vt column, no norm or rotation
    half_t* vt = sq.Vt + (size_t)(slot - a.NH - a.NKV) * 128 * a.cap + crow;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      vt[(size_t)(j0 + i) * a.cap] = f2h(v0[i]);
      vt[(size_t)(j0 + i + 64) * a.cap] = f2h(v1[i]);
    }
    return;
  }
  const bool is_q = slot < a.NH;
  const half_t* gn = is_q ? a.q_norm : (a.layer_cols ? a.k_norm_s[sidx] : a.k_norm);
  float t[E];
#pragma unroll
  for (int i = 0; i < E; ++i) t[i] = __builtin_fmaf(v0[i], v0[i], v1[i] * v1[i]);
#pragma unroll
  for (int o = 32 / E; o > 0; o >>= 1)
#pragma unroll
    for (int i = 0; i < E; ++i) t[i] += __shfl_xor(t[i], o, 64);
  float ss = t[0];
  if constexpr (E == 4) ss = (t[0] + t[2]) + (t[1] + t[3]);
  const float r = 1.0f / sqrtf(ss * (1.0f / 128.0f) + a.eps);
  float c[E], sn[E];
  if (a.cs) {   // (cos, sin) pairs of j0 .. j0 + E - 1: 8 E contiguous bytes
    const float* csp = a.cs + 2 * (m * 64 + j0);
    float w[2 * E];
    if constexpr (E == 4) {
      const floatx4 q0 = reinterpret_cast<const floatx4*>(csp)[0];
      const floatx4 q1 = reinterpret_cast<const floatx4*>(csp)[1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i] = q0[i];
        w[4 + i] = q1[i];
      }
    } else {
      w[0] = csp[0];
      w[1] = csp[1];
    }
#pragma unroll
    for (int i = 0; i < E; ++i) {
      c[i] = w[2 * i];
      sn[i] = w[2 * i + 1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const double inv_freq =
          a.inv_freq ? a.inv_freq[j0 + i] : exp2(-(double)(j0 + i) * (1.0 / 64.0) * a.log2_theta);
      const double ang = (double)(sq.pos0 + m) * inv_freq;
      double sd, cd;
      sincos(ang, &sd, &cd);
      c[i] = (float)cd;
      sn[i] = (float)sd;
    }
  }
  half_t* dst;
  if (is_q) {
    dst = a.Q + (((size_t)sidx * a.NH + slot) * a.M + m) * 128;
  } else {
    const int gk = slot - a.NH;
    dst = sq.Kc + ((size_t)gk * a.cap + crow) * 128;
  }
  half_t g0[E], g1[E], o0[E], o1[E];
  if constexpr (E == 4) {
    const half4_t h0 = *reinterpret_cast<const half4_t*>(gn + j0);
    const half4_t h1 = *reinterpret_cast<const half4_t*>(gn + j0 + 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g0[i] = h0[i];
      g1[i] = h1[i];
    }
  } else {
    g0[0] = gn[j0];
    g1[0] = gn[j0 + 64];
  }
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float y0 = h2f(rms_out_once(v0[i], r, g0[i]));
    const float y1 = h2f(rms_out_once(v1[i], r, g1[i]));
    // the rotation written out (the y * c products fused and rounded once to fp16 with the
    // rounded y * sn products), so that the result does not depend on the compiler's choices
    o0[i] = fma_f16_once(y0, c[i], -(y1 * sn[i]));
    o1[i] = fma_f16_once(y1, c[i], y0 * sn[i]);
  }
  if constexpr (E == 4) {
    *reinterpret_cast<half4_t*>(dst + j0) = (half4_t){o0[0], o0[1], o0[2], o0[3]};
    *reinterpret_cast<half4_t*>(dst + j0 + 64) = (half4_t){o1[0], o1[1], o1[2], o1[3]};
  } else {
    dst[j0] = o0[0];
    dst[j0 + 64] = o1[0];
  }
}

// Q/K part: qk_rope_item per (sequence, row, slot).
// V part: the workgroup reads its 64 rows x 128 values row by row (coalesced), transposes
// them through LDS and writes each Vt row d as 64 consecutive cache columns, so the
// transposed cache layout costs no scattered 2-byte stores.
__global__ __launch_bounds__(256) void qk_rope_kernel(QKRopeArgs a) {
  __shared__ half_t vt_s[128][66];   // [d][row], rows padded against bank conflicts
  const QkRopeGrid gr = qk_rope_grid(a);
  if ((long long)blockIdx.x >= gr.qk_blocks) {
    const long long vb = (long long)blockIdx.x - gr.qk_blocks;
    const int tile = (int)(vb % gr.v_tiles);
    const long long sv = vb / gr.v_tiles;
    const int sidx = (int)(sv / gr.nv), slot = gr.v0 + (int)(sv % gr.nv);
    const RopeSeq& sq = a.sq[sidx];
    const int m0 = tile * 64;
    for (int i = threadIdx.x; i < 64 * 32; i += 256) {
      const int r = i >> 5, d = (i & 31) * 4;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (m0 + r < a.M) {
        size_t row;
        int c0;
        qk_rope_src(a, sidx, m0 + r, slot, row, c0);
        qk_rope_values<4>(a, row, c0 + d, v);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) vt_s[d + k][r] = f2h(v[k]);
    }
    __syncthreads();
    const int gk = slot - (a.NH + a.NKV);
    half_t* vt = sq.Vt + (size_t)gk * 128 * a.cap;
    for (int i = threadIdx.x; i < 64 * 128; i += 256) {
      const int d = i >> 6, r = i & 63;
      if (m0 + r >= a.M) continue;
      const int crow = cache_slot(sq, a.M, m0 + r);
      if (crow >= 0) vt[(size_t)d * a.cap + crow] = vt_s[d][r];
    }
    return;
  }
  const long long per_seq = (long long)a.M * gr.nqk;
  long long p;
  int L;
  if (gr.items == 16) {   // prompt-sized: a quarter wave per item
    p = (long long)blockIdx.x * 16 + (threadIdx.x >> 4);
    L = threadIdx.x & 15;
  } else {                // few rows: a wave per item
    p = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    L = threadIdx.x & 63;
  }
  if (p >= per_seq * a.n_seq) return;   // a whole group (its shuffles stay inside it)
  const int sidx = (int)(p / per_seq);
  const long long pr = p - (long long)sidx * per_seq;
  const int m = (int)(pr / gr.nqk);
  const int slot = gr.qk0 + (int)(pr - (long long)m * gr.nqk);
  if (gr.items == 16) qk_rope_item<4>(a, sidx, m, slot, L);
  else qk_rope_item<1>(a, sidx, m, slot, L);
}

__global__ __launch_bounds__(256) void rope_table_kernel(int M, long long pos0, double log2_theta,
                                                         const double* __restrict__ inv_freq,
                                                         float* __restrict__ cs) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= M * 64) return;
  const int m = i >> 6, j = i & 63;
  const double f = inv_freq ? inv_freq[j] : exp2(-(double)j * (1.0 / 64.0) * log2_theta);
  double sd, cd;
  sincos((double)(pos0 + m) * f, &sd, &cd);
  cs[2 * i] = (float)cd;
  cs[2 * i + 1] = (float)sd;
}

void launch_rope_table(int M, long long pos0, double log2_theta, const double* inv_freq,
                       float* cs, hipStream_t st) {
  if (M <= 0) return;
  hipLaunchKernelGGL(rope_table_kernel, dim3((M * 64 + 255) / 256), dim3(256), 0, st, M, pos0,
                     log2_theta, inv_freq, cs);
}

bool launch_qk_rope(const QKRopeArgs& a, hipStream_t st) {
  if (check_qk_rope_args(a)) return false;
  const QkRopeGrid gr = qk_rope_grid(a);
  const long long blocks = gr.qk_blocks + (long long)a.n_seq * gr.nv * gr.v_tiles;
  hipLaunchKernelGGL(qk_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
  return true;
}

__global__ void argmax_finalize_kernel(unsigned long long* keys, int M, int32_t* ids) {
  const int m = threadIdx.x;
  if (m < M) {
    const unsigned long long k = keys[m];
    ids[m] = k ? (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull)) : -1;
    keys[m] = 0ull;
  }
}

// One wave per row: the largest of the P partial keys (fixed tree order), as an id.
__global__ __launch_bounds__(256) void argmax_parts_kernel(const unsigned long long* parts, int P,
                                                           int M, int32_t* ids) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  unsigned long long k = 0ull;
  for (int p = lane; p < P; p += 64) {
    const unsigned long long v = parts[(size_t)p * M + m];
    k = v > k ? v : k;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long k2 = __shfl_xor(k, o, 64);
    k = k2 > k ? k2 : k;
  }
  if (lane == 0) ids[m] = k ? (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull)) : -1;
}

void launch_argmax_parts(const unsigned long long* parts, int P, int M, int32_t* ids,
                         hipStream_t st) {
  if (M <= 0) return;
  hipLaunchKernelGGL(argmax_parts_kernel, dim3((M + 3) / 4), dim3(256), 0, st, parts, P, M, ids);
}

void launch_argmax_finalize(unsigned long long* keys, int M, int32_t* ids, hipStream_t st) {
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(64 * ((M + 63) / 64)), 0, st, keys,
                     M, ids);
}

// ---- block embedding with the soft anchor (generate.py:1419-1437) ----
// noise rows = embed[ids[b]]; with correction logits, row 0 is instead
//   sum_r softmax(top logits)_r * embed[top id_r]   (top_k largest logits, fp32 softmax and
// fp32 sum, cast to fp16).  The top-k runs in two launches: SA_BLOCKS workgroups each keep
// the top_k of a contiguous slice of the vocabulary, then workgroup 0 of the embedding
// launch merges the SA_BLOCKS * SA_TOPK_MAX candidates.  Ranking: larger logit first,
// lower index on ties, NaN after every number.

template <int DT>
DFL_DEV float logit_value(const void* p, size_t i) {
  if constexpr (DT == 0) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (DT == 1) return h2f(reinterpret_cast<const half_t*>(p)[i]);
  else return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);   // bf16
}

DFL_DEV unsigned long long rank_key(float v, uint32_t i) {
  if (v != v) return 0ull;   // NaN: never selected ahead of a number; 0 also marks "empty"
  return ((unsigned long long)float_order_key(v) << 32) | (0xFFFFFFFFu - i);
}
DFL_DEV uint32_t rank_index(unsigned long long key) {
  return 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull);
}

// t: descending list; insert x if it beats the last entry (one bubble pass keeps the order)
DFL_DEV void topk_push(unsigned long long (&t)[SA_TOPK_MAX], unsigned long long x) {
  if (x <= t[SA_TOPK_MAX - 1]) return;
  t[SA_TOPK_MAX - 1] = x;
#pragma unroll
  for (int i = SA_TOPK_MAX - 1; i > 0; --i) {
    const unsigned long long a = t[i - 1], b = t[i];
    t[i - 1] = a > b ? a : b;
    t[i] = a > b ? b : a;
  }
}

DFL_DEV unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

// The k largest keys held in the block's per-thread lists -> out[0 .. k) (shared memory),
// 0 where fewer exist.  Keys are unique (they carry the index), so one thread pops.
DFL_DEV void block_topk(unsigned long long (&t)[SA_TOPK_MAX], int k, unsigned long long* sm,
                        unsigned long long* out) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, nw = blockDim.x >> 6;
  for (int r = 0; r < k; ++r) {
    const unsigned long long c = wave_max_u64(t[0]);
    if (l == 0) sm[w] = c;
    __syncthreads();
    unsigned long long best = sm[0];
    for (int i = 1; i < nw; ++i) best = sm[i] > best ? sm[i] : best;
    if (best != 0ull && t[0] == best) {
#pragma unroll
      for (int i = 0; i < SA_TOPK_MAX - 1; ++i) t[i] = t[i + 1];
      t[SA_TOPK_MAX - 1] = 0ull;
    }
    if (threadIdx.x == 0) out[r] = best;
    __syncthreads();   // sm is rewritten by the next round
  }
}

template <int DT>
__global__ __launch_bounds__(256) void topk_scan_kernel(const void* __restrict__ logits, int V,
                                                        int k, unsigned long long* __restrict__ cand) {
  __shared__ unsigned long long sm[16], top[SA_TOPK_MAX];
  unsigned long long t[SA_TOPK_MAX];
#pragma unroll
  for (int i = 0; i < SA_TOPK_MAX; ++i) t[i] = 0ull;
  const int chunk = (V + gridDim.x - 1) / gridDim.x;
  const int lo = blockIdx.x * chunk, hi = min(V, lo + chunk);
  for (int i = lo + (int)threadIdx.x; i < hi; i += blockDim.x)
    topk_push(t, rank_key(logit_value<DT>(logits, i), (uint32_t)i));
  block_topk(t, k, sm, top);
  if (threadIdx.x < SA_TOPK_MAX)
    cand[blockIdx.x * SA_TOPK_MAX + threadIdx.x] = (int)threadIdx.x < k ? top[threadIdx.x] : 0ull;
}

template <int DT>
__global__ __launch_bounds__(256) void embed_block_kernel(
    const int32_t* __restrict__ ids, const half_t* __restrict__ embed, int Vemb, int H,
    const void* __restrict__ logits, int k, const unsigned long long* __restrict__ cand,
    half_t* __restrict__ out, int* __restrict__ err) {
  const int b = blockIdx.x;
  half_t* dst = out + (size_t)b * H;
  if (b == 0 && logits) {
    __shared__ unsigned long long sm[16], top[SA_TOPK_MAX];
    __shared__ float wgt[SA_TOPK_MAX];
    __shared__ int row[SA_TOPK_MAX];
    unsigned long long t[SA_TOPK_MAX];
#pragma unroll
    for (int i = 0; i < SA_TOPK_MAX; ++i) t[i] = 0ull;
    for (int i = threadIdx.x; i < SA_BLOCKS * SA_TOPK_MAX; i += blockDim.x) topk_push(t, cand[i]);
    block_topk(t, k, sm, top);
    if (threadIdx.x == 0) {
      // softmax over the selected logits in fp32; top[0] holds the largest
      float v[SA_TOPK_MAX], s = 0.f;
      const float mx = top[0] ? logit_value<DT>(logits, rank_index(top[0])) : 0.f;
      for (int r = 0; r < k; ++r) {
        row[r] = top[r] ? (int)rank_index(top[r]) : -1;
        v[r] = row[r] >= 0 ? expf(logit_value<DT>(logits, row[r]) - mx) : 0.f;
        s += v[r];
      }
      if (!top[0]) atomicOr(err, 2);   // no number among the logits: zero anchor row
      for (int r = 0; r < k; ++r) wgt[r] = top[0] ? v[r] / s : 0.f;
    }
    __syncthreads();
    for (int c = threadIdx.x; c < H; c += blockDim.x) {
      float acc = 0.f;
      for (int r = 0; r < k; ++r)
        if (row[r] >= 0) acc += wgt[r] * h2f(embed[(size_t)row[r] * H + c]);
      dst[c] = f2h(acc);
    }
    return;
  }
  const int id = ids[b];
  const bool bad = id < 0 || id >= Vemb;   // out-of-range token id: flag it, zero row
  if (bad && threadIdx.x == 0) atomicOr(err, 1);
  const half_t* src = embed + (size_t)(bad ? 0 : id) * H;
  for (int c = threadIdx.x; c < H; c += blockDim.x) dst[c] = bad ? (half_t)0.0f : src[c];
}

template <int DT>
static void launch_embed_block_t(const int32_t* ids, int B, const half_t* embed, int Vemb, int H,
                                 const void* logits, int V, int top_k, unsigned long long* cand,
                                 half_t* out, int* err, hipStream_t st) {
  if (logits)
    hipLaunchKernelGGL(topk_scan_kernel<DT>, dim3(SA_BLOCKS), dim3(256), 0, st, logits, V, top_k,
                       cand);
  hipLaunchKernelGGL(embed_block_kernel<DT>, dim3(B), dim3(256), 0, st, ids, embed, Vemb, H,
                     logits, top_k, cand, out, err);
}

void launch_embed_block(const int32_t* ids, int B, const half_t* embed, int Vemb, int H,
                        const void* logits, int logits_dtype, int V, int top_k,
                        unsigned long long* cand, half_t* out, int* err, hipStream_t st) {
  if (logits_dtype == 0)
    launch_embed_block_t<0>(ids, B, embed, Vemb, H, logits, V, top_k, cand, out, err, st);
  else if (logits_dtype == 1)
    launch_embed_block_t<1>(ids, B, embed, Vemb, H, logits, V, top_k, cand, out, err, st);
  else
    launch_embed_block_t<2>(ids, B, embed, Vemb, H, logits, V, top_k, cand, out, err, st);
}

}  // namespace dfl
