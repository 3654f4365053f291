// Weight-streaming GEMMs for the draft block: Y[M, N] = X[M, K] * W[N, K]^T with
// M <= 32 rows of fp16 activations per m-tile and W either int8 with per-row fp16
// scales (W8A16 projections) or fp16 (fc, lm_head).
//
// Why MFMA for a skinny GEMM: at M = 32 every int8 weight byte feeds 64 flops, so
// streaming weights at 8 TB/s needs ~512 TFLOP/s -- above what the fp32/dot2 VALU
// path can issue (~157 TFLOP/s).  v_mfma_f32_32x32x16_f16 has ample headroom, and
// the int8 -> fp16 dequant (exact, 1.25 VALU ops per byte) hides under the loads.
//
// Weight layout in HBM (written once at load by the pack kernels): blocks of
// 32 rows x KBK k-values (KBK = 32 for int8, 16 for fp16), 1 KiB each, ordered
// [row-block][k-block]; inside a block lane l's 16 bytes are
//   int8: W[rb*32 + l%32][kb*32 + 16*(l/32) + 0..15]
//   fp16: W[rb*32 + l%32][kb*16 +  8*(l/32) + 0..7]
// so one wave-wide 128-bit load reads 1 KiB contiguous and hands every lane its
// MFMA A-fragment directly (int8: two MFMAs per load).  The per-row scale factors
// out of the k-sum and is applied once in the epilogue.
//
// Work decomposition: a wave owns a "wave-tile" of 64 rows (two row-blocks) and
// one k-slice; a 256-thread workgroup holds TN = 4/SK wave-tiles x SK k-slices
// and sums the SK slices through LDS in a fixed order; S_x workgroups split K
// further and write fp32 partials that a follow-up kernel reduces in a fixed
// order (deterministic, no atomics on the data).
#include "dfl_common.h"
#include "dfl_kernels.h"

namespace dfl {

template <int WT>
struct WTraits;
template <>
struct WTraits<WT_INT8> {
  static constexpr int KBK = 32;  // k-values per 1 KiB block
  static constexpr int NX = 2;    // activation fragments (uint4) per block
};
template <>
struct WTraits<WT_F16> {
  static constexpr int KBK = 16;
  static constexpr int NX = 1;
};

template <int WT, int EPI, int SK, int P>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void skinny_gemm_kernel(SkinnyArgs a) {
  constexpr int TN = 4 / SK;
  constexpr int KBK = WTraits<WT>::KBK;
  constexpr int NX = WTraits<WT>::NX;
  __shared__ float red[(SK > 1) ? 4 * 2 * 16 * 64 : 1];

  const int lane = threadIdx.x & 63;
  // wave-uniform values (readfirstlane lets the compiler use scalar branches)
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = blockIdx.x / a.S_x;
  const int split = blockIdx.x - group * a.S_x;
  const int wt = group * TN + w / SK;          // wave-tile (64 packed rows)
  const int sk = w % SK;
  const int mt = blockIdx.y;                    // 32-row m-tile
  const int n_wt = a.N >> 6;
  const bool active = wt < n_wt;

  const int n_slices = a.S_x * SK;
  const int si = split * SK + sk;
  const int kb0 = (int)(((long long)si * a.KB) / n_slices);
  const int kb1 = (int)(((long long)(si + 1) * a.KB) / n_slices);
  const int nkb = active ? (kb1 - kb0) : 0;

  const int m = lane & 31;
  const int g = lane >> 5;
  const int row = mt * 32 + m;
  const bool row_ok = row < a.M;

  // Rows past M read row 0: an activation row only feeds its own output column
  // (D[n][m] = sum_k W[n][k] X[m][k]), which is never stored, so no masking is needed
  // and every load stays unconditional.
  const uint4* w0 = a.W + ((size_t)(2 * wt) * a.KB + kb0) * 64 + lane;
  const uint4* w1 = w0 + (size_t)a.KB * 64;
  const half_t* xrow = a.X + (size_t)(row_ok ? row : 0) * a.ldx + (size_t)kb0 * KBK +
                       (WT == WT_INT8 ? 16 * g : 8 * g);

  floatx16 acc0 = {}, acc1 = {};

  // One pipeline stage holds P consecutive k-blocks: two 1 KiB weight fragments per
  // k-block and NX activation fragments.
  struct Stage {
    u32x4 w0[P], w1[P], x[P][NX];
  };
  // Loads are unconditional: block indices past the wave's range are clamped to its
  // last block (a cache hit) and contribute nothing (zero activation at use).
  auto issue = [&](Stage& st, int base, int last) {
    static_for<0, P>([&](auto s) {
      const int i = min(base + (int)s, last);
      st.w0[s] = load_stream(w0 + (size_t)i * 64);
      st.w1[s] = load_stream(w1 + (size_t)i * 64);
      const half_t* xp = xrow + (size_t)i * KBK;
      static_for<0, NX>([&](auto x) { st.x[s][x] = load_vec(xp + 8 * x); });
    });
  };
  auto consume = [&](const Stage& st, int base, int nkb_) {
    static_for<0, P>([&](auto s) {
      const bool valid = base + (int)s < nkb_;
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 xa = valid ? st.x[s][0] : z;
      const u32x4 xb = valid ? st.x[s][NX - 1] : z;
      if constexpr (WT == WT_INT8) {
        half8_t lo0, hi0, lo1, hi1;
        dequant_i8x16(st.w0[s], lo0, hi0);
        dequant_i8x16(st.w1[s], lo1, hi1);
        const half8_t xl = as_half8(xa), xh = as_half8(xb);
        acc0 = mfma32x32x16(lo0, xl, acc0);
        acc1 = mfma32x32x16(lo1, xl, acc1);
        acc0 = mfma32x32x16(hi0, xh, acc0);
        acc1 = mfma32x32x16(hi1, xh, acc1);
      } else {
        const half8_t xv = as_half8(xa);
        acc0 = mfma32x32x16(as_half8(st.w0[s]), xv, acc0);
        acc1 = mfma32x32x16(as_half8(st.w1[s]), xv, acc1);
      }
    });
  };

  // Ping-pong between two register stages: the loads of one stage stay in flight
  // while the other is consumed (no register copies, so no forced waits).
  // sched_barrier keeps the scheduler from sinking a stage's loads down to their uses.
  if (nkb > 0) {
    const int last = nkb - 1;
    Stage A, B;
    issue(A, 0, last);
    for (int base = 0; base < nkb; base += 2 * P) {
      issue(B, base + P, last);
      __builtin_amdgcn_sched_barrier(0);
      consume(A, base, nkb);
      if (base + P >= nkb) break;
      issue(A, base + 2 * P, last);
      __builtin_amdgcn_sched_barrier(0);
      consume(B, base + P, nkb);
    }
  }

  if constexpr (SK > 1) {
    if (sk != 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        red[((w * 2 + 0) * 16 + r) * 64 + lane] = acc0[r];
        red[((w * 2 + 1) * 16 + r) * 64 + lane] = acc1[r];
      }
    }
    __syncthreads();
    if (sk != 0) return;
#pragma unroll
    for (int j = 1; j < SK; ++j) {
      const int ww = w + j;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc0[r] += red[((ww * 2 + 0) * 16 + r) * 64 + lane];
        acc1[r] += red[((ww * 2 + 1) * 16 + r) * 64 + lane];
      }
    }
  }
  if (!active || !row_ok) return;

  // Row n of the packed matrix held in accumulator r of tile t:
  //   n = (2*wt + t)*32 + 8*(r/4) + 4*g + (r%4)
  if constexpr (EPI == EPI_PARTIAL) {
    float* dst = a.ws + ((size_t)split * a.M + row) * a.N + (size_t)(2 * wt) * 32 + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      *reinterpret_cast<floatx4*>(dst + 8 * q) =
          (floatx4){acc0[4 * q], acc0[4 * q + 1], acc0[4 * q + 2], acc0[4 * q + 3]};
      *reinterpret_cast<floatx4*>(dst + 32 + 8 * q) =
          (floatx4){acc1[4 * q], acc1[4 * q + 1], acc1[4 * q + 2], acc1[4 * q + 3]};
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    // Tile 0 holds gate rows f = wt*32 + j, tile 1 the up rows of the same f.
    const half_t* sg = a.scale + (size_t)(2 * wt) * 32 + 4 * g;
    const half_t* su = sg + 32;
    half_t* dst = a.out + (size_t)row * a.ldo + (size_t)wt * 32 + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      half4_t o;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int r = 4 * q + b;
        const float gv = h2f(f2h(acc0[r] * h2f(sg[8 * q + b])));
        const float uv = h2f(f2h(acc1[r] * h2f(su[8 * q + b])));
        const float sig = h2f(f2h(1.0f / (1.0f + expf(-gv))));
        const float si_ = h2f(f2h(gv * sig));
        o[b] = f2h(si_ * uv);
      }
      *reinterpret_cast<half4_t*>(dst + 8 * q) = o;
    }
  } else {  // EPI_ARGMAX (fp16 weights, no scale)
    const int nbase = (2 * wt) * 32 + 4 * g;
    if (a.logits) {
      float* dst = a.logits + (size_t)row * a.ldl + nbase;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        *reinterpret_cast<floatx4*>(dst + 8 * q) =
            (floatx4){acc0[4 * q], acc0[4 * q + 1], acc0[4 * q + 2], acc0[4 * q + 3]};
        *reinterpret_cast<floatx4*>(dst + 32 + 8 * q) =
            (floatx4){acc1[4 * q], acc1[4 * q + 1], acc1[4 * q + 2], acc1[4 * q + 3]};
      }
    }
    if (a.keys) {
      // Scan in increasing n so that strict '>' keeps the lowest index on ties.
      float best = -INFINITY;
      int bn = 0x7fffffff;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = nbase + 8 * (r >> 2) + (r & 3);
        if (acc0[r] > best) { best = acc0[r]; bn = n; }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = nbase + 32 + 8 * (r >> 2) + (r & 3);
        if (acc1[r] > best) { best = acc1[r]; bn = n; }
      }
      const float ob = __shfl_xor(best, 32, 64);
      const int on = __shfl_xor(bn, 32, 64);
      if (ob > best || (ob == best && on < bn)) { best = ob; bn = on; }
      if (g == 0 && bn != 0x7fffffff) {
        const unsigned long long key =
            ((unsigned long long)float_order_key(best) << 32) | (0xFFFFFFFFu - (uint32_t)bn);
        atomicMax(a.keys + row, key);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side launcher
// ---------------------------------------------------------------------------

template <int WT, int EPI, int SK>
static void launch_sk(const SkinnyArgs& a, int n_mtiles, hipStream_t st) {
  constexpr int TN = 4 / SK;
  const int n_wt = a.N / 64;
  const int n_groups = (n_wt + TN - 1) / TN;
  dim3 grid(n_groups * a.S_x, n_mtiles);
  hipLaunchKernelGGL((skinny_gemm_kernel<WT, EPI, SK, 4>), grid, dim3(256), 0, st, a);
}

template <int WT, int EPI>
static void launch_w(const SkinnyArgs& a, int SK, int n_mtiles, hipStream_t st) {
  switch (SK) {
    case 1: launch_sk<WT, EPI, 1>(a, n_mtiles, st); break;
    case 2: launch_sk<WT, EPI, 2>(a, n_mtiles, st); break;
    default: launch_sk<WT, EPI, 4>(a, n_mtiles, st); break;
  }
}

void launch_skinny_gemm(int wt, int epi, const SkinnyArgs& a, int SK, int n_mtiles,
                        hipStream_t st) {
  if (wt == WT_INT8) {
    if (epi == EPI_PARTIAL) launch_w<WT_INT8, EPI_PARTIAL>(a, SK, n_mtiles, st);
    else launch_w<WT_INT8, EPI_SWIGLU>(a, SK, n_mtiles, st);
  } else {
    if (epi == EPI_PARTIAL) launch_w<WT_F16, EPI_PARTIAL>(a, SK, n_mtiles, st);
    else launch_w<WT_F16, EPI_ARGMAX>(a, SK, n_mtiles, st);
  }
}

}  // namespace dfl
