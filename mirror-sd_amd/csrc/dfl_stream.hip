// Stream-K weight-streaming GEMM for the draft block (M <= 32 activation rows):
//   Y[m, n] = sum_k Xn[m, k] * W[n, k]  (* scale[n] for int8 weights)
// with an optional RMSNorm applied to X on load (Xn = fp16(fp16(X * r[m]) * g[k])).
//
// Partition.  The packed weight matrix (see dfl_gemm.hip for the block layout) is a
// sequence of U = (N/64) * KB work units (64-row wave-tile x one 1 KiB k-block pair),
// tile-major.  The grid is exactly one 512-thread workgroup per CU; workgroup b takes
// the contiguous unit range [b*U/G, (b+1)*U/G), so every CU streams the same number of
// bytes and there is no second-round tail.  A range is cut into segments at tile
// boundaries; the 8 waves split each segment's k-blocks, stream them with a two-stage
// register pipeline, and reduce through LDS in a fixed order.
//
// Completion.  A segment that covers a whole tile runs the epilogue directly.  A tile
// split across workgroups is finished by whichever of them arrives last: each writes its
// fp32 partial to a workspace slot, fences (device scope), and bumps the tile's counter;
// the last one sums the slots in segment order (deterministic) and runs the epilogue,
// then re-arms the counter.  No workgroup ever waits for another.
//
// Epilogues: STORE (fp16 y with the per-row scale), RESID (x += fp16(y), per-row sums of
// squares; the last tile of the launch turns them into r = rsqrt(mean(x^2) + eps) for
// the next GEMM's norm-on-load), SWIGLU (gate/up row-blocks interleaved), ARGMAX (fp32
// logits + packed (value, index) atomicMax per row).
#include "dfl_common.h"
#include "dfl_kernels.h"

namespace dfl {

namespace {

constexpr int SK_WAVES = 8;
constexpr int SK_THREADS = 64 * SK_WAVES;

template <int WT>
struct KTraits;
template <>
struct KTraits<WT_INT8> {
  static constexpr int KBK = 32;
  static constexpr int NX = 2;
};
template <>
struct KTraits<WT_F16> {
  static constexpr int KBK = 16;
  static constexpr int NX = 1;
};

// First workgroup whose unit range contains unit u: max b with floor(b*U/G) <= u.
DFL_DEV int wg_of(long long u, long long U, int G) { return (int)(((u + 1) * G - 1) / U); }

// fp16(fp16(x * r) * g) for 8 packed halves (RMSNorm output expression).
DFL_DEV u32x4 norm8(u32x4 xv, float r, u32x4 gv) {
  const half8_t x = as_half8(xv), gg = as_half8(gv);
  half8_t y;
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = f2h(h2f(f2h(h2f(x[j]) * r)) * h2f(gg[j]));
  return __builtin_bit_cast(u32x4, y);
}

}  // namespace

template <int WT, int EPI, bool NORM, int P>
__global__ __launch_bounds__(SK_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void streamk_gemm_kernel(StreamArgs a) {
  constexpr int KBK = KTraits<WT>::KBK;
  constexpr int NX = KTraits<WT>::NX;
  __shared__ float red[(SK_WAVES - 1) * 2 * 16 * 64];
  __shared__ half_t gsh[NORM ? 8192 : 8];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = lane & 31, g = lane >> 5;
  const bool row_ok = m < a.M;
  const int xr = row_ok ? m : 0;   // rows >= M read row 0: they only feed unstored columns
  const int n_wt = a.N >> 6;
  const long long U = (long long)n_wt * a.KB;
  const int G = gridDim.x;
  const int b = blockIdx.x;
  const long long u0 = (long long)b * U / G, u1 = (long long)(b + 1) * U / G;

  float rn = 1.0f;
  if constexpr (NORM) {
    rn = a.rnorm[xr];
    const int K = a.KB * KBK;
    for (int k = threadIdx.x; k < K; k += SK_THREADS) gsh[k] = a.gnorm[k];
    __syncthreads();
  }

  const half_t* xrow = a.X + (size_t)xr * a.ldx + (WT == WT_INT8 ? 16 * g : 8 * g);
  const int goff = (WT == WT_INT8 ? 16 * g : 8 * g);

  struct Stage {
    u32x4 w0[P], w1[P], x[P][NX];
  };

  for (long long u = u0; u < u1;) {
    const int t = (int)(u / a.KB);
    const int kbs = (int)(u - (long long)t * a.KB);
    const int kbe = (int)min((long long)a.KB, (long long)kbs + (u1 - u));
    const int L = kbe - kbs;
    // this wave's share of the segment
    const int v0 = kbs + (w * L) / SK_WAVES, v1 = kbs + ((w + 1) * L) / SK_WAVES;
    const int nkb = v1 - v0;

    const uint4* w0p = a.W + ((size_t)(2 * t) * a.KB + v0) * 64 + lane;
    const uint4* w1p = w0p + (size_t)a.KB * 64;
    const half_t* xp0 = xrow + (size_t)v0 * KBK;

    floatx16 acc0 = {}, acc1 = {};
    auto issue = [&](Stage& st, int base, int last) {
      static_for<0, P>([&](auto s) {
        const int i = min(base + (int)s, last);
        st.w0[s] = load_stream(w0p + (size_t)i * 64);
        st.w1[s] = load_stream(w1p + (size_t)i * 64);
        const half_t* xp = xp0 + (size_t)i * KBK;
        static_for<0, NX>([&](auto x) { st.x[s][x] = load_vec(xp + 8 * x); });
      });
    };
    auto consume = [&](const Stage& st, int base) {
      static_for<0, P>([&](auto s) {
        const int i = base + (int)s;
        const bool valid = i < nkb;
        const u32x4 z = {0u, 0u, 0u, 0u};
        u32x4 xa = st.x[s][0], xb = st.x[s][NX - 1];
        if constexpr (NORM) {
          const int kk = (v0 + min(i, nkb - 1)) * KBK + goff;
          xa = norm8(xa, rn, *reinterpret_cast<const u32x4*>(gsh + kk));
          if constexpr (NX > 1) xb = norm8(xb, rn, *reinterpret_cast<const u32x4*>(gsh + kk + 8));
          else xb = xa;
        }
        xa = valid ? xa : z;
        xb = valid ? xb : z;
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
    if (nkb > 0) {
      const int last = nkb - 1;
      Stage A, B;
      issue(A, 0, last);
      for (int base = 0; base < nkb; base += 2 * P) {
        issue(B, base + P, last);
        __builtin_amdgcn_sched_barrier(0);
        consume(A, base);
        if (base + P >= nkb) break;
        issue(A, base + 2 * P, last);
        __builtin_amdgcn_sched_barrier(0);
        consume(B, base + P);
      }
    }

    // ---- reduce the 8 waves' partials into wave 0 (fixed order) ----
    if (w != 0) {
      float* dst = red + (size_t)(w - 1) * 2048;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dst[r * 64 + lane] = acc0[r];
        dst[1024 + r * 64 + lane] = acc1[r];
      }
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int j = 0; j < SK_WAVES - 1; ++j) {
        const float* src = red + (size_t)j * 2048;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc0[r] += src[r * 64 + lane];
          acc1[r] += src[1024 + r * 64 + lane];
        }
      }
      bool complete = (kbs == 0 && kbe == a.KB);
      if (!complete) {
        // cross-workgroup split of tile t: slot j among the workgroups covering it
        const long long tu0 = (long long)t * a.KB;
        const int first = wg_of(tu0, U, G);
        const int count = wg_of(tu0 + a.KB - 1, U, G) - first + 1;
        const int j = b - first;
        float* slot = a.ws + ((size_t)t * a.seg_cap + j) * 2048;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          slot[r * 64 + lane] = acc0[r];
          slot[1024 + r * 64 + lane] = acc1[r];
        }
        __threadfence();
        int prev = 0;
        if (lane == 0) prev = atomicAdd(a.tile_cnt + t, 1);
        prev = __shfl(prev, 0, 64);
        if (prev == count - 1) {
          __threadfence();
          acc0 = (floatx16){};
          acc1 = (floatx16){};
          for (int jj = 0; jj < count; ++jj) {
            const float* src = a.ws + ((size_t)t * a.seg_cap + jj) * 2048;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              acc0[r] += __builtin_nontemporal_load(src + r * 64 + lane);
              acc1[r] += __builtin_nontemporal_load(src + 1024 + r * 64 + lane);
            }
          }
          if (lane == 0) a.tile_cnt[t] = 0;
          complete = true;
        }
      }
      if (complete) {
        // ---- epilogue for tile t: n = (2t + tt)*32 + 8*q + 4*g + (0..3) ----
        const int nb = (2 * t) * 32 + 4 * g;
        if constexpr (EPI == EPI_STORE) {
          if (row_ok) {
            half_t* dst = a.out + (size_t)m * a.ldo + nb;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              half4_t o0, o1;
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                o0[c] = f2h(acc0[4 * q + c] * h2f(a.scale[nb + 8 * q + c]));
                o1[c] = f2h(acc1[4 * q + c] * h2f(a.scale[nb + 32 + 8 * q + c]));
              }
              *reinterpret_cast<half4_t*>(dst + 8 * q) = o0;
              *reinterpret_cast<half4_t*>(dst + 32 + 8 * q) = o1;
            }
          }
        } else if constexpr (EPI == EPI_RESID) {
          float ss = 0.f;
          if (row_ok) {
            half_t* xr_ = a.x + (size_t)m * a.ldo + nb;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
              for (int tt = 0; tt < 2; ++tt) {
                half4_t xv = *reinterpret_cast<const half4_t*>(xr_ + 32 * tt + 8 * q);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                  const float acc = tt ? acc1[4 * q + c] : acc0[4 * q + c];
                  const float y = h2f(f2h(acc * h2f(a.scale[nb + 32 * tt + 8 * q + c])));
                  const half_t xn = f2h(h2f(xv[c]) + y);
                  xv[c] = xn;
                  ss += h2f(xn) * h2f(xn);
                }
                *reinterpret_cast<half4_t*>(xr_ + 32 * tt + 8 * q) = xv;
              }
            }
          }
          ss += __shfl_xor(ss, 32, 64);
          if (g == 0 && row_ok) a.ss_part[(size_t)t * 32 + m] = ss;
          __threadfence();
          int prev = 0;
          if (lane == 0) prev = atomicAdd(a.done_cnt, 1);
          prev = __shfl(prev, 0, 64);
          if (prev == n_wt - 1) {   // last tile of the launch: per-row rsqrt for the next norm
            __threadfence();
            if (g == 0 && row_ok) {
              float tot = 0.f;
              for (int tt = 0; tt < n_wt; ++tt)
                tot += __builtin_nontemporal_load(a.ss_part + (size_t)tt * 32 + m);
              a.rnorm_out[m] = 1.0f / sqrtf(tot / (float)a.N + a.eps);
            }
            if (lane == 0) *a.done_cnt = 0;
          }
        } else if constexpr (EPI == EPI_SWIGLU) {
          if (row_ok) {
            const half_t* sg = a.scale + nb;
            half_t* dst = a.out + (size_t)m * a.ldo + (size_t)t * 32 + 4 * g;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              half4_t o;
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                const int r = 4 * q + c;
                const float gv = h2f(f2h(acc0[r] * h2f(sg[8 * q + c])));
                const float uv = h2f(f2h(acc1[r] * h2f(sg[32 + 8 * q + c])));
                const float sig = h2f(f2h(1.0f / (1.0f + expf(-gv))));
                const float sil = h2f(f2h(gv * sig));
                o[c] = f2h(sil * uv);
              }
              *reinterpret_cast<half4_t*>(dst + 8 * q) = o;
            }
          }
        } else {  // EPI_ARGMAX: fp16 weights, no scale
          if (row_ok && a.logits) {
            float* dst = a.logits + (size_t)m * a.ldl + nb;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              *reinterpret_cast<floatx4*>(dst + 8 * q) =
                  (floatx4){acc0[4 * q], acc0[4 * q + 1], acc0[4 * q + 2], acc0[4 * q + 3]};
              *reinterpret_cast<floatx4*>(dst + 32 + 8 * q) =
                  (floatx4){acc1[4 * q], acc1[4 * q + 1], acc1[4 * q + 2], acc1[4 * q + 3]};
            }
          }
          if (a.keys) {
            float best = -INFINITY;
            int bn = 0x7fffffff;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int n = nb + 8 * (r >> 2) + (r & 3);
              if (acc0[r] > best) { best = acc0[r]; bn = n; }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int n = nb + 32 + 8 * (r >> 2) + (r & 3);
              if (acc1[r] > best) { best = acc1[r]; bn = n; }
            }
            const float ob = __shfl_xor(best, 32, 64);
            const int on = __shfl_xor(bn, 32, 64);
            if (ob > best || (ob == best && on < bn)) { best = ob; bn = on; }
            if (g == 0 && row_ok && bn != 0x7fffffff) {
              const unsigned long long key =
                  ((unsigned long long)float_order_key(best) << 32) | (0xFFFFFFFFu - (uint32_t)bn);
              atomicMax(a.keys + m, key);
            }
          }
        }
      }
    }
    u += L;
    __syncthreads();   // red[] is reused by the next segment
  }
}

// Workgroups: one per CU, never more than the number of units.
int streamk_grid(int N, int KB, int n_cu) {
  const long long U = (long long)(N / 64) * KB;
  return (int)std::max(1LL, std::min<long long>(n_cu, U));
}

// Workspace slots per tile for a given grid: ceil(KB / floor(U/G)) + 1.
int streamk_seg_cap(int N, int KB, int G) {
  const long long U = (long long)(N / 64) * KB;
  const long long per = std::max(1LL, U / G);
  return (int)((KB + per - 1) / per + 1);
}

template <int WT, int EPI, bool NORM>
static void launch_t(const StreamArgs& a, int G, hipStream_t st) {
  hipLaunchKernelGGL((streamk_gemm_kernel<WT, EPI, NORM, 4>), dim3(G), dim3(SK_THREADS), 0, st, a);
}

void launch_streamk_gemm(int wt, int epi, bool norm, const StreamArgs& a, int G, hipStream_t st) {
#define DFL_SK_CASE(W_, E_)                                        \
  if (wt == W_ && epi == E_) {                                     \
    if (norm) launch_t<W_, E_, true>(a, G, st);                    \
    else launch_t<W_, E_, false>(a, G, st);                        \
    return;                                                        \
  }
  DFL_SK_CASE(WT_INT8, EPI_STORE)
  DFL_SK_CASE(WT_INT8, EPI_RESID)
  DFL_SK_CASE(WT_INT8, EPI_SWIGLU)
  DFL_SK_CASE(WT_F16, EPI_ARGMAX)
#undef DFL_SK_CASE
}

}  // namespace dfl
