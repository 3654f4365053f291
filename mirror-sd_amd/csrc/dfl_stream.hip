// Stream-K weight-streaming GEMM for the draft block (M <= 32 activation rows):
//   Y[m, n] = sum_k Xn[m, k] * W[n, k]  (* scale[n] for int8 weights)
// with an optional RMSNorm applied to X on load (Xn = fp16(fp16(X * r[m]) * g[k])).
// X is a 32-row tile in the activation fragment layout (afl_offset in dfl_common.h), so
// activation fragments, like weight fragments, arrive as contiguous 1 KiB wave loads; the
// residual and SwiGLU epilogues write their outputs in the same layout.
//
// Partition.  The packed weight matrix (block layout: see dfl_pack.hip) is a sequence of
// U = (N/64) * KB work units (one 64-row wave-tile x one k-block), tile-major.  One
// workgroup per CU takes an equal contiguous unit range, so every CU streams the same
// number of bytes; the range crosses tile boundaries, which cut it into segments.
//
// Workgroup = 4 streaming waves + 1 reducer wave.  The streaming waves split each
// segment's k-blocks, write their fp32 partial to an LDS slot (two slot sets, used by
// alternate segments) and go straight on to the next segment.  The reducer wave stages
// the RMSNorm gain and 1/rms rows in LDS at the start (its copies are issued before any
// weight load), then for each segment in turn sums the 4 partials in a fixed order and
// completes the tile, so the cross-workgroup fix-up and the epilogue overlap the next
// segment's weight stream instead of stalling it.
//
// Completion.  A segment covering a whole tile runs the epilogue directly.  A tile split
// across workgroups is finished by whichever arrives last: each stores its fp32 partial
// with agent-scope atomic stores, waits for them to complete (s_waitcnt), then bumps the
// tile's agent-scope counter; the last one reads the slots back with agent-scope atomic
// loads in slot order (deterministic sum), runs the epilogue and re-arms the counter.
// Only agent-scope atomics touch the shared slots, so no L2 write-back / invalidate is
// needed, and no workgroup ever waits for another.
//
// Epilogues: STORE (fp16 y with the per-row scale), RESID (x += fp16(y), per-tile row sums
// of squares for the next GEMM's 1/rms), SWIGLU (gate/up row-blocks interleaved), ARGMAX
// (fp32 logits + packed (value, index) atomicMax per row), QKROPE (the fused q|k|v rows
// of one sequence: per-head Q/K RMSNorm + RoPE and the K/V cache writes; a head's two
// tiles complete together).
#include "dfl_common.h"
#include "dfl_kernels.h"
#include "dfl_check.h"

#include <hip/hip_ext.h>

#include <climits>

namespace dfl {

namespace {

// Streaming waves per workgroup: one per SIMD.  (A second streaming wave on a SIMD loses
// the issue arbitration to the older one and finishes its equal share ~40 % later.)
// The reducer wave shares SIMD 0.
constexpr int WG_WAVES = 4;

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

// Largest worker index w with floor(w*U/NW) <= u (the worker holding unit u).
DFL_DEV int worker_of(long long u, long long U, int NW) { return (int)(((u + 1) * NW - 1) / U); }

// fp32(x * r) for the low / high fp16 half of a dword, in one v_fma_mix_f32 (fma with a
// -0.0 addend is the exactly rounded product, signed zeros included) instead of a
// convert and a multiply.
DFL_DEV float mul_f16lo_f32(uint32_t xv, float r) {
  float d;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(xv), "v"(r), "v"(-0.0f));
  return d;
}
DFL_DEV float mul_f16hi_f32(uint32_t xv, float r) {
  float d;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=v"(d) : "v"(xv), "v"(r), "v"(-0.0f));
  return d;
}

// fp16(fp16(x * r) * g) for 8 packed halves (RMSNorm output expression).  The second
// product is a packed fp16 multiply: the product of two fp16 values is exact in fp32, so
// rounding it to fp16 once is the same as the fp32 multiply followed by the conversion.
DFL_DEV u32x4 norm8(u32x4 xv, float r, u32x4 gv) {
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    half2_t p = (half2_t){f2h(mul_f16lo_f32(xv[j], r)), f2h(mul_f16hi_f32(xv[j], r))};
    p = p * __builtin_bit_cast(half2_t, gv[j]);
    o[j] = __builtin_bit_cast(uint32_t, p);
  }
  return o;
}

DFL_DEV void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DFL_DEV float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Norm prologue hand-off through the LDS word `ready`: the reducer wave issues the
// prologue's loads and sets it to PRO_ISSUED, then stores the gain and 1/rms to LDS and
// sets PRO_DONE.  The streaming waves of a NORM kernel issue no weight load before
// PRO_ISSUED: a CU serves its vector memory requests in order, so prologue loads queued
// behind the streaming waves' 64-128 KiB of weight loads would wait several microseconds.
constexpr int PRO_ISSUED = 1, PRO_DONE = 2;
DFL_DEV void mark_issued(int* ready) {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __hip_atomic_store(ready, PRO_ISSUED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
DFL_DEV void wait_ready(int* ready, int state) {
  while (__hip_atomic_load(ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < state)
    __builtin_amdgcn_s_sleep(1);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Norm prologue copies, global -> LDS with global_load_lds (16 B per lane, 1 KiB per
// wave instruction, `bytes` a multiple of 16): the loads write LDS directly, so none of
// them waits for another and no VGPR holds the data; the copy costs one memory latency
// and a few instructions.  The caller waits with s_waitcnt vmcnt before reading.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
DFL_DEV void copy_to_lds(const void* src, void* lds_dst, int bytes, int lane) {
  for (int off = 0; off < bytes; off += 1024) {
    const int o = off + lane * 16;
    if (o < bytes)
      __builtin_amdgcn_global_load_lds(static_cast<const char*>(src) + o,
                                       (lds_ptr_t)(static_cast<char*>(lds_dst) + off), 16, 0, 0);
  }
}

// 1/rms of activation row m (lane & 31) from the per-tile sums of squares of the RESID
// epilogue that produced X (global memory or an LDS copy): lane (m, g) adds tiles g, g+2,
// ... with eight loads in flight.
DFL_DEV float rn_from_ss(const float* ss, int tiles, int n, float eps, int lane) {
  const int m = lane & 31, g = lane >> 5;
  const float* sp = ss + m;
  float tot = 0.f;
  int tt = g;
  for (; tt + 14 < tiles; tt += 16) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = sp[(size_t)(tt + 2 * j) * 32];
    tot += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  }
  for (; tt < tiles; tt += 2) tot += sp[(size_t)tt * 32];
  tot += __shfl_xor(tot, 32, 64);
  return 1.0f / sqrtf(tot / (float)n + eps);
}

// ---------------------------------------------------------------------------------------
// Streaming wave w walks the workgroup's work list -- units [u0, u1), then [v0, v1) (unit
// = 64-row wave-tile t x k-block kb, u = t * KB + kb) -- taking every WG_WAVES-th unit of
// the concatenation (w, w + WG_WAVES, ...) in one continuous load pipeline.  Two register
// stages of P units alternate (sched_barrier keeps each stage's loads issued ahead of use);
// loads past the wave's last unit repeat its address and are not consumed.  Every tile a
// range touches is one segment, numbered in list order; when the wave leaves a segment it
// hands its fp32 partial (two 32x32 accumulators, zero if it had no unit there) to the
// reducer wave through LDS slot set (segment & 1), while the next units' loads are already
// in flight.
// ---------------------------------------------------------------------------------------
// XRM (fp16 only): the activations are row-major feature rows (StreamArgs::xr_p) instead of
// the fragment-layout tile X; lane (m, g) of k-block kb loads X[m][16 kb + 8 g .. + 7], the
// same eight values its fragment-layout record entry holds.
template <int WT, bool NORM, int P, bool XRM = false>
DFL_DEV void stream_range(const StreamArgs& a, const half_t* gsh, const float* rn_lds,
                          int* ready, float (*red)[WG_WAVES][2048], int* arrived, int* reduced,
                          long long u0, long long u1, long long v0, long long v1, int w,
                          int lane, int& si, const int* abort = nullptr) {
  constexpr int KBK = KTraits<WT>::KBK;
  constexpr int NX = KTraits<WT>::NX;
  const int m = lane & 31, g = lane >> 5;
  const int goff = (WT == WT_INT8 ? 16 * g : 8 * g);
  const int KB = a.KB;
  // activation records: int8 k-block kb = 32 k -> records (kb, 0), (kb, 1), this lane's
  // entry; fp16 k-block kb = 16 k -> record (kb/2, g) at entry m + 32*(kb & 1)
  const u32x4* xf = reinterpret_cast<const u32x4*>(a.X);

  floatx16 acc0 = (floatx16){}, acc1 = (floatx16){};
  // si: segments flushed so far by this wave (continues across calls)
  auto flush = [&]() {
    // slot set si & 1 was last used by segment si - 2: wait until it has been reduced (or
    // the workgroup aborted: its results are invalid, every wave just runs to its end)
    while (__hip_atomic_load(reduced, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < si - 1 &&
           !(abort && __hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)))
      __builtin_amdgcn_s_sleep(1);
    float* dst = red[si & 1][w];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dst[r * 64 + lane] = acc0[r];
      dst[1024 + r * 64 + lane] = acc1[r];
    }
    if (lane == 0)
      __hip_atomic_fetch_add(&arrived[si & 1], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    acc0 = (floatx16){};
    acc1 = (floatx16){};
    ++si;
  };

  const int len1 = (int)(u1 - u0), len = len1 + (int)(v1 - v0);
  const int nseg1 = len1 > 0 ? (int)((u1 - 1) / KB - u0 / KB + 1) : 0;
  const int nseg = nseg1 + (v1 > v0 ? (int)((v1 - 1) / KB - v0 / KB + 1) : 0);
  const int J = w < len ? (len - w + WG_WAVES - 1) / WG_WAVES : 0;
  // units of this wave in the first range; its first unit of the second range is list
  // position w + WG_WAVES * J1
  const int J1 = w < len1 ? (len1 - w + WG_WAVES - 1) / WG_WAVES : 0;
  int cs = 0;   // consume cursor: segment of the next unit (segments before it are flushed)
  if (J > 0) {
    // issue cursor: tile it, k-block ikb, segment isg of the next unit (KB >= WG_WAVES);
    // the second range starts at (it2, ikb2, isg2)
    int it, ikb, isg, it2 = 0, ikb2 = 0, isg2 = 0;
    {
      const long long ua = w < len1 ? u0 + w : v0 + (w - len1);
      it = (int)(ua / KB);
      ikb = (int)(ua - (long long)it * KB);
      isg = w < len1 ? it - (int)(u0 / KB) : nseg1 + it - (int)(v0 / KB);
      if (J1 > 0 && J1 < J) {
        const long long ub = v0 + (w + WG_WAVES * J1 - len1);
        it2 = (int)(ub / KB);
        ikb2 = (int)(ub - (long long)it2 * KB);
        isg2 = nseg1 + it2 - (int)(v0 / KB);
      }
    }
    int issued = 0;
    // XRM: feature xr_j covers k-blocks from xr_k0 / 16; xr_row is this lane's row in it
    // (offset 8 g), moved only when the walk enters another feature (a tile change, the
    // second range, or every xr_h / 64 of the wave's units)
    [[maybe_unused]] int xr_j = 0, xr_k0 = INT_MIN / 2;
    [[maybe_unused]] const half_t* xr_row = nullptr;
    [[maybe_unused]] const size_t xr_lane = XRM ? (size_t)m * a.xr_ld + 8 * g : 0;
    auto xr_track = [&](int kb) {
      if constexpr (XRM) {
        const int k = 16 * kb;
        if (k < xr_k0 || k >= xr_k0 + a.xr_h) {
          xr_j = k / a.xr_h;
          xr_k0 = xr_j * a.xr_h;
          xr_row = a.xr_p[xr_j] + xr_lane;
        }
      }
    };
    xr_track(ikb);
    struct Stage {
      u32x4 w0[P], w1[P], x[P][NX];
      int kb[P], sg[P];
    };
    auto issue = [&](Stage& st) {
      static_for<0, P>([&](auto s) {
        const uint4* wp = a.W + ((size_t)(2 * it) * KB + ikb) * 64 + lane;
        st.w0[s] = load_stream(wp);
        st.w1[s] = load_stream(wp + (size_t)KB * 64);
        st.kb[s] = ikb;
        st.sg[s] = isg;
        if constexpr (WT == WT_INT8) {
          st.x[s][0] = xf[(size_t)(2 * ikb) * 64 + lane];
          st.x[s][NX - 1] = xf[(size_t)(2 * ikb + 1) * 64 + lane];
        } else if constexpr (XRM) {
          u32x4 v = {0u, 0u, 0u, 0u};
          if (m < a.M) v = *reinterpret_cast<const u32x4*>(xr_row + (16 * ikb - xr_k0));
          st.x[s][0] = v;
        } else {
          st.x[s][0] = xf[(size_t)((ikb >> 1) * 2 + g) * 64 + m + 32 * (ikb & 1)];
        }
        if (++issued < J) {
          if (issued == J1) {   // into the second range
            it = it2;
            ikb = ikb2;
            isg = isg2;
          } else {
            ikb += WG_WAVES;
            if (ikb >= KB) {
              ikb -= KB;
              ++it;
              ++isg;
            }
          }
          xr_track(ikb);
        }
      });
    };
    float rn = 1.0f;
    auto consume = [&](const Stage& st, int base) {
      static_for<0, P>([&](auto s) {
        if (base + (int)s < J) {
          while (cs < st.sg[s]) {   // left a segment (or segments): hand over its partial
            flush();
            ++cs;
          }
          u32x4 xa = st.x[s][0], xb = st.x[s][NX - 1];
          if constexpr (NORM) {
            const int kk = st.kb[s] * KBK + goff;
            xa = norm8(xa, rn, *reinterpret_cast<const u32x4*>(gsh + kk));
            if constexpr (NX > 1) xb = norm8(xb, rn, *reinterpret_cast<const u32x4*>(gsh + kk + 8));
            else xb = xa;
          }
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
        }
      });
    };

    Stage A, B;
    if constexpr (NORM) {
      wait_ready(ready, PRO_ISSUED);
      issue(A);
      issue(B);   // both stages in flight while the reducer's prologue completes
      wait_ready(ready, PRO_DONE);   // gain and 1/rms from the reducer wave's prologue
      rn = rn_lds[m];
    } else {
      issue(A);
    }
    for (int base = 0; base < J; base += 2 * P) {
      if (!NORM || base > 0) issue(B);
      __builtin_amdgcn_sched_barrier(0);
      consume(A, base);
      if (base + P >= J) break;
      issue(A);
      __builtin_amdgcn_sched_barrier(0);
      consume(B, base + P);
    }
  }
  // the segment of the last unit, then trailing segments without a unit of this wave
  for (; cs < nseg; ++cs) flush();
}

// Split-tile slot (t, slot) of the workspace: a worker's fp32 partial of tile t.
DFL_DEV float* ws_slot(const StreamArgs& a, int t, int slot) {
  return a.ws + ((size_t)t * a.seg_cap + slot) * 2048;
}

// Publishes this worker's partial in slot (t, slot) and bumps counter `cnt` once the
// stores have completed (agent-coherent); returns the counter's previous value.
DFL_DEV int publish_partial(const StreamArgs& a, int lane, int t, int slot, int* cnt,
                            const floatx16& acc0, const floatx16& acc1) {
  float* mine = ws_slot(a, t, slot);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    store_agent(mine + r * 64 + lane, acc0[r]);
    store_agent(mine + 1024 + r * 64 + lane, acc1[r]);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  int prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0, 64);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return prev;
}

// acc += slots 0 .. count-1 of tile t, in slot order (deterministic sums).  The loads of up to
// three slots are issued together: a device-coherent round trip costs 1-2 us at a launch's
// end (several under a full weight stream), and the last worker of a split tile would
// otherwise wait one per slot.
// Slot j at slot0 + j * stride floats.
DFL_DEV void add_slots_at(const float* slot0, size_t stride, int lane, int count,
                          floatx16& acc0, floatx16& acc1) {
  constexpr int C = 3;
  for (int j0 = 0; j0 < count; j0 += C) {
    float v0[C][16], v1[C][16];
#pragma unroll
    for (int jj = 0; jj < C; ++jj) {
      const float* src = slot0 + (size_t)min(j0 + jj, count - 1) * stride;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        v0[jj][r] = load_agent(src + r * 64 + lane);
        v1[jj][r] = load_agent(src + 1024 + r * 64 + lane);
      }
    }
#pragma unroll
    for (int jj = 0; jj < C; ++jj)
      if (j0 + jj < count)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc0[r] += v0[jj][r];
          acc1[r] += v1[jj][r];
        }
  }
}
DFL_DEV void add_slots(const StreamArgs& a, int lane, int t, int count, floatx16& acc0,
                       floatx16& acc1) {
  add_slots_at(ws_slot(a, t, 0), 2048, lane, count, acc0, acc1);
}

// Cross-worker completion of tile t.  `slot` is this worker's index among the `count`
// workers covering the tile.  Returns true (with the full sums in acc0/acc1) for the last
// worker to arrive; the others return false after publishing their partial.
DFL_DEV bool finish_split_tile(const StreamArgs& a, int lane, int t, int slot, int count,
                               floatx16& acc0, floatx16& acc1) {
  if (publish_partial(a, lane, t, slot, a.tile_cnt + t, acc0, acc1) != count - 1) return false;
  acc0 = (floatx16){};
  acc1 = (floatx16){};
  add_slots(a, lane, t, count, acc0, acc1);
  if (lane == 0) a.tile_cnt[t] = 0;   // next use is a later launch
  return true;
}

// 64 fp16 ones: the "scales" of a tile's epilogue over fp16 weights.
__device__ __attribute__((aligned(16))) const half_t kOnes64[64] = {
    1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1,
    1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1};

// Global inputs of a tile's epilogue, loaded ahead of it (before the reducer waits for
// the streaming waves' partials) so that completing the launch's last tiles costs no load
// latency: the per-row scales of the lane's 32 rows and, for RESID, its residual values.
struct EpiIn {
  half4_t s0[4], s1[4];   // scale[nb + 8q + 0..3], scale[nb + 32 + 8q + 0..3]
  half4_t xv[2][4];       // RESID: x row m, columns nb + 32 tt + 8 q + 0..3
};

template <int EPI>
DFL_DEV EpiIn epi_prefetch(const StreamArgs& a, int lane, int t) {
  EpiIn in;
  const int m = lane & 31, g = lane >> 5;
  const int nb = (2 * t) * 32 + 4 * g;
  // the scales, or ones for fp16 weights: one pointer, no branch (a branch here made the
  // compiler keep the values in a scratch array on the tile's completion path)
  const half_t* sp = a.scale ? a.scale + nb : kOnes64 + 4 * g;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    in.s0[q] = *reinterpret_cast<const half4_t*>(sp + 8 * q);
    in.s1[q] = *reinterpret_cast<const half4_t*>(sp + 32 + 8 * q);
  }
  if constexpr (EPI == EPI_RESID) {
    // x is an AFL tile [32][N] (32 rows always allocated)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        in.xv[tt][q] = a.x_zero ? (half4_t){0, 0, 0, 0}
                                : *reinterpret_cast<const half4_t*>(a.x + afl_offset(m, nb + 32 * tt + 8 * q));
  }
  return in;
}

// Epilogue of a completed tile t for the 32 activation rows held by this wave, with its
// global inputs from epi_prefetch (EPI_STORE, EPI_RESID, EPI_SWIGLU).
// Row n of the packed matrix in accumulator r of block tt: n = (2t+tt)*32 + 8*(r/4)
// + 4*g + (r%4), activation row m = lane % 32.
// ARGMAX with key_acc: the row's best key so far is kept in *key_acc (lanes 0..31, one row
// each) instead of an atomicMax per tile; the caller publishes it once at its end.
template <int EPI>
DFL_DEV void tile_epilogue(const StreamArgs& a, int lane, int t, const floatx16& acc0,
                           const floatx16& acc1, const EpiIn& in,
                           unsigned long long* key_acc = nullptr) {
  const int m = lane & 31, g = lane >> 5;
  const bool row_ok = m < a.M;
  const int nb = (2 * t) * 32 + 4 * g;
  if constexpr (EPI == EPI_STORE) {
    if (!row_ok) return;
    half_t* dst = a.out + (size_t)m * a.ldo + nb;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      half4_t o0, o1;
#pragma unroll
      for (int c = 0; c < 4; ++c) {   // fp16 weights carry no scale (in.s = 1)
        o0[c] = f2h(acc0[4 * q + c] * h2f(in.s0[q][c]));
        o1[c] = f2h(acc1[4 * q + c] * h2f(in.s1[q][c]));
      }
      *reinterpret_cast<half4_t*>(dst + 8 * q) = o0;
      *reinterpret_cast<half4_t*>(dst + 32 + 8 * q) = o1;
    }
  } else if constexpr (EPI == EPI_RESID) {
    // x is an AFL tile [32][N]; columns nb + 32*tt + 8*q + (0..3) of row m are 4
    // consecutive halves of record (2t + tt, q & 1), entry m + 32*(q >> 1), offset 4g.
    float ss = 0.f;
    if (row_ok) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          half_t* xp = a.x + afl_offset(m, nb + 32 * tt + 8 * q);
          half4_t xv = in.xv[tt][q];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float acc = tt ? acc1[4 * q + c] : acc0[4 * q + c];
            const float y = h2f(f2h(acc * h2f(tt ? in.s1[q][c] : in.s0[q][c])));
            const half_t xn = f2h(h2f(xv[c]) + y);
            xv[c] = xn;
            ss += h2f(xn) * h2f(xn);
          }
          *reinterpret_cast<half4_t*>(xp) = xv;
        }
      }
    }
    ss += __shfl_xor(ss, 32, 64);
    if (g == 0 && row_ok) store_agent(a.ss_part + (size_t)t * 32 + m, ss);
  } else if constexpr (EPI == EPI_SWIGLU) {
    if (!row_ok) return;
    // out is an AFL tile [32][N/2]: columns 32t + 8q + 4g + (0..3) of row m
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      half_t* dst = a.out + afl_offset(m, t * 32 + 8 * q + 4 * g);
      half4_t o;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int r = 4 * q + c;
        const float gv = h2f(f2h(acc0[r] * h2f(in.s0[q][c])));
        const float uv = h2f(f2h(acc1[r] * h2f(in.s1[q][c])));
        const float sig = h2f(f2h(1.0f / (1.0f + expf(-gv))));
        const float sil = h2f(f2h(gv * sig));
        o[c] = f2h(sil * uv);
      }
      *reinterpret_cast<half4_t*>(dst) = o;
    }
  } else if constexpr (EPI == EPI_QKROPE) {
    // a V head's tile (Q and K heads complete in qk_head_epilogue): the fp16 Linear output
    // of row m goes to its transposed cache column, Vt[gk][d][crow], as in qk_rope_kernel
    const RopeEpi& r = a.rope;
    if (!row_ok) return;
    const int crow = cache_slot(r.sq, a.M, m);
    if (crow < 0) return;
    half_t* vt = r.sq.Vt + (size_t)((t >> 1) - r.NH - r.NKV) * 128 * r.cap + crow;
    const int d0 = 64 * (t & 1) + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = d0 + 8 * q + c;
        vt[(size_t)d * r.cap] = f2h(acc0[4 * q + c] * h2f(in.s0[q][c]));
        vt[(size_t)(d + 32) * r.cap] = f2h(acc1[4 * q + c] * h2f(in.s1[q][c]));
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
      // scan in increasing n so that strict '>' keeps the lowest index on ties; a sampling
      // call ranks l / T + Gumbel noise instead of l
      const bool samp = a.samp_invT > 0.f;
      const uint32_t salt = samp ? gumbel_row_salt(a.samp_seed, a.samp_row0 + m) : 0u;
      auto rank = [&](float l, int n) { return samp ? l * a.samp_invT + gumbel_noise(salt, n) : l; };
      float best = -INFINITY;
      int bn = 0x7fffffff;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = nb + 8 * (r >> 2) + (r & 3);
        const float v = rank(acc0[r], n);
        if (v > best) { best = v; bn = n; }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = nb + 32 + 8 * (r >> 2) + (r & 3);
        const float v = rank(acc1[r], n);
        if (v > best) { best = v; bn = n; }
      }
      const float ob = __shfl_xor(best, 32, 64);
      const int on = __shfl_xor(bn, 32, 64);
      if (ob > best || (ob == best && on < bn)) { best = ob; bn = on; }
      if (g == 0 && row_ok && bn != 0x7fffffff) {
        const unsigned long long key =
            ((unsigned long long)float_order_key(best) << 32) | (0xFFFFFFFFu - (uint32_t)bn);
        if (key_acc) *key_acc = key > *key_acc ? key : *key_acc;
        else atomicMax(a.keys + m, key);
      }
    }
  }
}

// The epilogue with its inputs loaded on the spot.
template <int EPI>
DFL_DEV void tile_epilogue(const StreamArgs& a, int lane, int t, const floatx16& acc0,
                           const floatx16& acc1) {
  tile_epilogue<EPI>(a, lane, t, acc0, acc1, epi_prefetch<EPI>(a, lane, t));
}

// Norm prologue of the reducer wave: the gain and ss_in are copied to LDS (issued before
// any streaming wave's weight load), then 1/rms of each activation row goes to rn_s.
template <int WT>
DFL_DEV void reducer_norm_prologue(const StreamArgs& a, int lane, half_t* gsh, float* ss_s,
                                   float* rn_s, int* ready) {
  const int K = a.KB * KTraits<WT>::KBK;
  copy_to_lds(a.gnorm, gsh, K * 2, lane);
  float rn = 1.0f;
  if (a.ss_in) copy_to_lds(a.ss_in, ss_s, a.ss_tiles * 32 * 4, lane);
  else rn = a.rnorm[lane & 31];
  if (lane == 0) mark_issued(ready);
  __builtin_amdgcn_s_waitcnt(0);   // both copies have landed in LDS
  if (a.ss_in) rn = rn_from_ss(ss_s, a.ss_tiles, a.ss_n, a.eps, lane);
  if (lane < 32) rn_s[lane] = rn;
  __builtin_amdgcn_s_waitcnt(0);
  if (lane == 0) __hip_atomic_store(ready, PRO_DONE, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Reducer wave, segment si (tile t): waits for the 4 streaming waves' partials, sums them
// in a fixed order, hands the slot set back and completes the tile -- directly when the
// segment covers it (count == 1), else as worker `slot` of the `count` sharing it.
DFL_DEV void sum_wave_partials(int lane, float (*red)[WG_WAVES][2048], int* arrived,
                               int* reduced, int si, floatx16& acc0, floatx16& acc1,
                               const int* abort = nullptr) {
  while (__hip_atomic_load(&arrived[si & 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
             WG_WAVES * ((si >> 1) + 1) &&
         !(abort && __hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)))
    __builtin_amdgcn_s_sleep(1);
  acc0 = (floatx16){};
  acc1 = (floatx16){};
#pragma unroll 1
  for (int j = 0; j < WG_WAVES; ++j) {
    const float* src = red[si & 1][j];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc0[r] += src[r * 64 + lane];
      acc1[r] += src[1024 + r * 64 + lane];
    }
  }
  __builtin_amdgcn_s_waitcnt(0);   // slot reads done before the set is handed back
  if (lane == 0) __hip_atomic_store(reduced, si + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int EPI>
DFL_DEV void reduce_segment(const StreamArgs& a, int lane, float (*red)[WG_WAVES][2048],
                            int* arrived, int* reduced, int si, int t, int slot, int count,
                            const int* abort = nullptr, unsigned long long* key_acc = nullptr) {
  const EpiIn in = epi_prefetch<EPI>(a, lane, t);   // in flight while the partials arrive
  floatx16 acc0, acc1;
  sum_wave_partials(lane, red, arrived, reduced, si, acc0, acc1, abort);
  const bool complete = count == 1 || finish_split_tile(a, lane, t, slot, count, acc0, acc1);
  if (complete) tile_epilogue<EPI>(a, lane, t, acc0, acc1, in, key_acc);
}

// Q or K head h of the fused qkv projection, complete: lo = d 0..63 (tile 2h), hi = d
// 64..127 (tile 2h+1), in the accumulator layout of tile_epilogue, so lane (m, g) holds the
// neox pair (d, d + 64) at the same register.  Per head and row: fp16 Linear output, RMSNorm
// over the 128 d (q_norm / k_norm), split-half RoPE with the block's angle table ([m][j]
// cos, sin, j = d mod 64), then Q[h][m] or the K cache row (qk_rope_kernel's arithmetic;
// dflash.py:251-252, 263-275).  Its tables are LDS copies made by the reducer wave at the
// start of the launch (QkTables), so none of its reads waits on global memory.
struct QkTables {
  const half_t* scale;   // [N] per-row scales of the q|k|v matrix
  const float* cs;       // [M][64] (cos, sin) of the block's positions
  const half_t* gn;      // [2][128] q_norm, k_norm
};
DFL_DEV void qk_head_epilogue(const StreamArgs& a, int lane, int h, const floatx16& lo0,
                              const floatx16& lo1, const floatx16& hi0, const floatx16& hi1,
                              const QkTables& tb) {
  const RopeEpi& r = a.rope;
  const int m = lane & 31, g = lane >> 5;
  __builtin_amdgcn_s_waitcnt(0);   // the reducer's table copies (issued at its start) landed
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const int nlo = 128 * h + 4 * g;   // packed row of d = 4g (+ 32 tt + 8 q + c)
  float vl[32], vh[32];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {   // i = 16 tt + 4 q + c: d = 32 tt + 8 q + 4 g + c
    const int f = 32 * (i >> 4) + 8 * ((i >> 2) & 3) + (i & 3);
    const float al = i < 16 ? lo0[i] : lo1[i - 16], ah = i < 16 ? hi0[i] : hi1[i - 16];
    vl[i] = h2f(f2h(al * h2f(tb.scale[nlo + f])));
    vh[i] = h2f(f2h(ah * h2f(tb.scale[nlo + 64 + f])));
    ss += vl[i] * vl[i] + vh[i] * vh[i];
  }
  ss += __shfl_xor(ss, 32, 64);
  if (m >= a.M) return;
  const bool is_q = h < r.NH;
  half_t* dst;
  if (is_q) {
    dst = r.Q + ((size_t)h * a.M + m) * 128;
  } else {
    const int crow = cache_slot(r.sq, a.M, m);
    if (crow < 0) return;
    dst = r.sq.Kc + ((size_t)(h - r.NH) * r.cap + crow) * 128;
  }
  const half_t* gn = tb.gn + (is_q ? 0 : 128);
  const float rr = 1.0f / sqrtf(ss * (1.0f / 128.0f) + r.eps);
#pragma unroll
  for (int q8 = 0; q8 < 8; ++q8) {   // 4 consecutive d per (tt, q)
    const int f0 = 32 * (q8 >> 2) + 8 * (q8 & 3) + 4 * g;
    const floatx4* csp = reinterpret_cast<const floatx4*>(tb.cs + 2 * (m * 64 + f0));
    const floatx4 cs01 = csp[0], cs23 = csp[1];   // (cos, sin) of f0 .. f0 + 3
    half4_t ol, oh;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = 4 * q8 + c, f = f0 + c;
      const float y0 = h2f(rms_out(vl[i], rr, gn[f]));
      const float y1 = h2f(rms_out(vh[i], rr, gn[f + 64]));
      const floatx4& cp = c < 2 ? cs01 : cs23;
      const float cc = cp[2 * (c & 1)], sn = cp[2 * (c & 1) + 1];
      // the contraction written out (the y0 products fused, the y1 products rounded), so
      // that the result does not depend on the compiler's choice of fma
      ol[c] = f2h(__builtin_fmaf(cc, y0, -(sn * y1)));
      oh[c] = f2h(__builtin_fmaf(sn, y0, cc * y1));
    }
    *reinterpret_cast<half4_t*>(dst + f0) = ol;
    *reinterpret_cast<half4_t*>(dst + 64 + f0) = oh;
  }
}

// Reducer wave, segment si of tile t of a Q/K head of the fused qkv projection: the head's
// two tiles complete together, through the split-tile protocol with one counter (tile
// 2h's) over the c_lo + c_hi workers of both tiles.  Every worker publishes its partial in
// its tile's slot `slot`; the last one sums each tile's slots in slot order (the same sums
// as a per-tile completion) and runs qk_head_epilogue.
DFL_DEV void reduce_head(const StreamArgs& a, int lane, float (*red)[WG_WAVES][2048],
                         int* arrived, int* reduced, int si, int t, int slot, int c_lo,
                         int c_hi, const QkTables& tb) {
  floatx16 acc0, acc1;
  sum_wave_partials(lane, red, arrived, reduced, si, acc0, acc1);
  const int t0 = t & ~1;
  if (publish_partial(a, lane, t, slot, a.tile_cnt + t0, acc0, acc1) != c_lo + c_hi - 1) return;
  floatx16 lo0 = (floatx16){}, lo1 = (floatx16){}, hi0 = (floatx16){}, hi1 = (floatx16){};
  if (c_lo <= 2 && c_hi <= 2) {   // both tiles' slots in one round trip
    float v[4][32];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int tt = jj >> 1, j = jj & 1, c = tt ? c_hi : c_lo;
      const float* src = ws_slot(a, t0 + tt, min(j, c - 1));
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        v[jj][r] = load_agent(src + r * 64 + lane);
        v[jj][16 + r] = load_agent(src + 1024 + r * 64 + lane);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (j < c_lo) {
          lo0[r] += v[j][r];
          lo1[r] += v[j][16 + r];
        }
        if (j < c_hi) {
          hi0[r] += v[2 + j][r];
          hi1[r] += v[2 + j][16 + r];
        }
      }
  } else {
    add_slots(a, lane, t0, c_lo, lo0, lo1);
    add_slots(a, lane, t0 + 1, c_hi, hi0, hi1);
  }
  if (lane == 0) a.tile_cnt[t0] = 0;   // next use is a later launch
  qk_head_epilogue(a, lane, t0 >> 1, lo0, lo1, hi0, hi1, tb);
}

// ---------------------------------------------------------------------------------------
// M-split mode (2 <= MT <= 8 activation m-tiles): streaming wave w owns m-tiles
// w*MTW .. w*MTW + MTW - 1 and walks every unit of the workgroup range in order, so each
// weight block is read from HBM once (the other waves hit the cache) and dequantised in
// registers once per wave for MTW m-tiles.  At each tile end the wave hands its MTW
// partials to the reducer through LDS slot set (segment & 1).
// ---------------------------------------------------------------------------------------
template <int WT, bool NORM, int P, int MTW>
DFL_DEV void stream_range_m(const StreamArgs& a, const half_t* gsh, const float* rn_lds,
                            int* ready, float (*red)[WG_WAVES][MTW][2048], int* arrived,
                            int* reduced, long long u0, long long u1, int w, int lane) {
  constexpr int KBK = KTraits<WT>::KBK;
  constexpr int NX = KTraits<WT>::NX;
  const int m = lane & 31, g = lane >> 5;
  const int goff = (WT == WT_INT8 ? 16 * g : 8 * g);
  const int KB = a.KB;
  const int mt0 = w * MTW;
  const int nmt = max(0, min(MTW, a.MT - mt0));   // m-tiles of this wave
  const size_t xstride = (size_t)32 * a.ldx;      // halves from one AFL m-tile to the next

  floatx16 acc[MTW][2];
#pragma unroll
  for (int j = 0; j < MTW; ++j) acc[j][0] = acc[j][1] = (floatx16){};
  int si = 0;
  auto flush = [&]() {
    while (__hip_atomic_load(reduced, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < si - 1)
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < MTW; ++j) {
      float* dst = red[si & 1][w][j];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dst[r * 64 + lane] = acc[j][0][r];
        dst[1024 + r * 64 + lane] = acc[j][1][r];
      }
      acc[j][0] = acc[j][1] = (floatx16){};
    }
    if (lane == 0)
      __hip_atomic_fetch_add(&arrived[si & 1], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    ++si;
  };
  const int t_first = (int)(u0 / KB);
  const int t_last = (int)((u1 - 1) / KB);
  if (nmt == 0) {   // no m-tile here: hand over zero partials, in step with the others
    for (int t = t_first; t <= t_last; ++t) flush();
    return;
  }
  const u32x4* xf[MTW];
#pragma unroll
  for (int j = 0; j < MTW; ++j)
    xf[j] = reinterpret_cast<const u32x4*>(a.X + (size_t)(mt0 + min(j, nmt - 1)) * xstride);

  const int J = (int)(u1 - u0);
  int ct = t_first;
  int it = t_first, ikb = (int)(u0 - (long long)t_first * KB), issued = 0;
  struct Stage {
    u32x4 w0[P], w1[P], x[P][MTW][NX];
    int kb[P], t[P];
  };
  auto issue = [&](Stage& st) {
    static_for<0, P>([&](auto s) {
      const uint4* wp = a.W + ((size_t)(2 * it) * KB + ikb) * 64 + lane;
      st.w0[s] = load_stream(wp);
      st.w1[s] = load_stream(wp + (size_t)KB * 64);
      st.kb[s] = ikb;
      st.t[s] = it;
#pragma unroll
      for (int j = 0; j < MTW; ++j) {
        if constexpr (WT == WT_INT8) {
          st.x[s][j][0] = xf[j][(size_t)(2 * ikb) * 64 + lane];
          st.x[s][j][NX - 1] = xf[j][(size_t)(2 * ikb + 1) * 64 + lane];
        } else {
          st.x[s][j][0] = xf[j][(size_t)((ikb >> 1) * 2 + g) * 64 + m + 32 * (ikb & 1)];
        }
      }
      if (++issued < J) {
        if (++ikb == KB) {
          ikb = 0;
          ++it;
        }
      }
    });
  };
  float rn[MTW];
#pragma unroll
  for (int j = 0; j < MTW; ++j) rn[j] = 1.0f;
  auto consume = [&](const Stage& st, int base) {
    static_for<0, P>([&](auto s) {
      if (base + (int)s < J) {
        while (ct < st.t[s]) {
          flush();
          ++ct;
        }
        half8_t lo0, hi0, lo1, hi1;
        if constexpr (WT == WT_INT8) {
          dequant_i8x16(st.w0[s], lo0, hi0);
          dequant_i8x16(st.w1[s], lo1, hi1);
        }
#pragma unroll
        for (int j = 0; j < MTW; ++j) {
          if (j < nmt) {
            u32x4 xa = st.x[s][j][0], xb = st.x[s][j][NX - 1];
            if constexpr (NORM) {
              const int kk = st.kb[s] * KBK + goff;
              xa = norm8(xa, rn[j], *reinterpret_cast<const u32x4*>(gsh + kk));
              if constexpr (NX > 1)
                xb = norm8(xb, rn[j], *reinterpret_cast<const u32x4*>(gsh + kk + 8));
              else xb = xa;
            }
            if constexpr (WT == WT_INT8) {
              const half8_t xl = as_half8(xa), xh = as_half8(xb);
              acc[j][0] = mfma32x32x16(lo0, xl, acc[j][0]);
              acc[j][1] = mfma32x32x16(lo1, xl, acc[j][1]);
              acc[j][0] = mfma32x32x16(hi0, xh, acc[j][0]);
              acc[j][1] = mfma32x32x16(hi1, xh, acc[j][1]);
            } else {
              const half8_t xv = as_half8(xa);
              acc[j][0] = mfma32x32x16(as_half8(st.w0[s]), xv, acc[j][0]);
              acc[j][1] = mfma32x32x16(as_half8(st.w1[s]), xv, acc[j][1]);
            }
          }
        }
      }
    });
  };

  Stage A, B;
  if constexpr (NORM) {
    wait_ready(ready, PRO_ISSUED);
    issue(A);
    issue(B);   // both stages in flight while the reducer's prologue completes
    wait_ready(ready, PRO_DONE);
#pragma unroll
    for (int j = 0; j < MTW; ++j) rn[j] = rn_lds[(mt0 + min(j, nmt - 1)) * 32 + m];
  } else {
    issue(A);
  }
  for (int base = 0; base < J; base += 2 * P) {
    if (!NORM || base > 0) issue(B);
    __builtin_amdgcn_sched_barrier(0);
    consume(A, base);
    if (base + P >= J) break;
    issue(A);
    __builtin_amdgcn_sched_barrier(0);
    consume(B, base + P);
  }
  for (int t = ct; t <= t_last; ++t) flush();
}

// The arguments of m-tile mt as seen by tile_epilogue (a 32-row view).
DFL_DEV StreamArgs mtile_view(const StreamArgs& a, int mt) {
  StreamArgs v = a;
  v.M = min(32, a.M - 32 * mt);
  const size_t rows = (size_t)32 * mt;
  if (a.out) v.out = a.out + rows * a.ldo;   // STORE rows / SWIGLU AFL tiles (ldo = N/2)
  if (a.x) v.x = a.x + rows * a.N;           // RESID AFL tiles
  if (a.ss_part) v.ss_part = a.ss_part + (size_t)mt * a.ss_mstride;
  if (a.logits) v.logits = a.logits + rows * a.ldl;
  if (a.keys) v.keys = a.keys + rows;
  v.samp_row0 = a.samp_row0 + (int)rows;
  return v;
}

}  // namespace

// ---------------------------------------------------------------------------------------
// The stream-K kernel: one workgroup per CU, 4 streaming waves + 1 reducer wave.
// ---------------------------------------------------------------------------------------
template <int WT, int EPI, bool NORM, int P, bool XRM = false>
__global__ __launch_bounds__(64 * (WG_WAVES + 1)) void gsk_gemm_kernel(StreamArgs a) {
  __shared__ float red[2][WG_WAVES][2048];     // partial slots, two sets
  __shared__ half_t gsh[NORM ? 8192 : 8];
  __shared__ float ss_s[NORM ? 128 * 32 : 1];  // LDS copy of ss_in (<= 128 tiles)
  __shared__ float rn_s[32];
  // arrived[p]: partials written for segments of parity p (monotonic: a set is rewritten
  // only after its previous segment was reduced); reduced: segments summed so far;
  // ready: norm prologue state (PRO_ISSUED, PRO_DONE)
  __shared__ int arrived[2], reduced, ready;
  // QKROPE: the head epilogue's tables (scales, angles, Q/K norm gains), copied to LDS
  __shared__ __attribute__((aligned(16))) half_t qk_sc[EPI == EPI_QKROPE ? QK_N_MAX : 8];
  __shared__ __attribute__((aligned(16))) float qk_cs[EPI == EPI_QKROPE ? 32 * 128 : 4];
  __shared__ __attribute__((aligned(16))) half_t qk_gn[EPI == EPI_QKROPE ? 256 : 8];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x;
  const int b = blockIdx.x;
  // Work list: the split (stream-K) units of tiles [0, T - dp*G), an equal contiguous range
  // per workgroup, first; then dp whole tiles of its own.  Split tiles are completed by
  // cross-workgroup fix-ups while the whole tiles stream, so the launch ends on local
  // epilogues only.  dp == 0: one stream-K range over the whole matrix.
  const int T = a.N >> 6, dp = a.dp;
  const long long U = (long long)(T - dp * G) * a.KB;   // split units
  const long long u0 = (long long)b * U / G, u1 = (long long)(b + 1) * U / G;
  const long long v0 = (long long)(T - dp * G + dp * b) * a.KB, v1 = v0 + (long long)dp * a.KB;
  if (u0 >= u1 && v0 >= v1) return;   // (the plan never makes more workgroups than units)
  if (threadIdx.x == 0) {
    arrived[0] = arrived[1] = 0;
    reduced = 0;
    ready = 0;
  }
  __syncthreads();

  if (w < WG_WAVES) {
    int si = 0;
    stream_range<WT, NORM, P, XRM>(a, gsh, rn_s, &ready, red, arrived, &reduced, u0, u1, v0, v1,
                                   w, lane, si);
    return;
  }

  // ---- reducer wave ----
  if constexpr (NORM) reducer_norm_prologue<WT>(a, lane, gsh, ss_s, rn_s, &ready);
  [[maybe_unused]] const QkTables qkt{qk_sc, qk_cs, qk_gn};
  if constexpr (EPI == EPI_QKROPE) {   // needed by the first head's epilogue, not before
    copy_to_lds(a.scale, qk_sc, a.N * 2, lane);
    copy_to_lds(a.rope.cs, qk_cs, a.M * 64 * 8, lane);
    copy_to_lds(a.rope.q_norm, qk_gn, 256, lane);
    copy_to_lds(a.rope.k_norm, qk_gn + 128, 256, lane);
  }
  // ARGMAX: each row's best key over the tiles this wave completes, one atomicMax at the end
  unsigned long long kacc = 0;
  unsigned long long* ka = EPI == EPI_ARGMAX ? &kacc : nullptr;
  int si = 0;
  for (long long u = u0; u < u1; ++si) {
    const int t = (int)(u / a.KB);
    const int kbs = (int)(u - (long long)t * a.KB);
    const int kbe = (int)min((long long)a.KB, (long long)kbs + (u1 - u));
    if constexpr (EPI == EPI_QKROPE) {
      if ((t >> 1) < a.rope.NH + a.rope.NKV) {   // Q or K head: both tiles complete together
        const long long h0 = (long long)(t & ~1) * a.KB;
        const int f_lo = worker_of(h0, U, G), f_hi = worker_of(h0 + a.KB, U, G);
        const int c_lo = worker_of(h0 + a.KB - 1, U, G) - f_lo + 1;
        const int c_hi = worker_of(h0 + 2 * a.KB - 1, U, G) - f_hi + 1;
        reduce_head(a, lane, red, arrived, &reduced, si, t, b - ((t & 1) ? f_hi : f_lo), c_lo,
                    c_hi, qkt);
        u += kbe - kbs;
        continue;
      }
    }
    int first = b, count = 1;
    if (!(kbs == 0 && kbe == a.KB)) {
      const long long tu0 = (long long)t * a.KB;
      first = worker_of(tu0, U, G);
      count = worker_of(tu0 + a.KB - 1, U, G) - first + 1;
    }
    reduce_segment<EPI>(a, lane, red, arrived, &reduced, si, t, b - first, count, nullptr, ka);
    u += kbe - kbs;
  }
  for (long long u = v0; u < v1; u += a.KB, ++si)   // whole tiles: local epilogues
    reduce_segment<EPI>(a, lane, red, arrived, &reduced, si, (int)(u / a.KB), 0, 1, nullptr,
                        ka);
  if constexpr (EPI == EPI_ARGMAX)
    if (a.keys && lane < 32 && lane < a.M && kacc) atomicMax(a.keys + lane, kacc);
}

// ---------------------------------------------------------------------------------------
// Balanced stream-K kernel (long matrices: the lm_head).  Streaming waves, reducer and
// completion as in gsk_gemm_kernel, but the work is not cut into equal ranges: workgroup
// b first streams the whole tiles [b*S, (b+1)*S) (S = dyn_static; no split, no fix-up),
// then half tiles of tiles [G*S, N/64) taken from a device-wide counter, so CUs that get
// more bandwidth (the XCDs differ) take more of them.  Half tile c is tile G*S + c/2,
// k-blocks [(c&1)*KB/2, (c&1+1)*KB/2); its two halves complete through the split-tile
// protocol as slots 0 and 1 (summed in slot order: results do not depend on which
// workgroup took which half).
//
// Queue: the reducer wave takes the next chunk id before it waits for the partials of
// the segment in flight and publishes it in an LDS ring of 4 (entry k in q_chunk[k & 3],
// q_pub = entries published, -1 = no more), so the streaming waves find entry k + 1 there
// when they finish chunk k.  The reducer publishes entry k + 2 only after reducing chunk
// k, which every streaming wave has flushed, so a slot is never overwritten before all
// have read it.  Each workgroup takes chunk ids until one is past the end, so the counter
// has stopped moving once every workgroup has bumped dyn_next[1]; the last one resets
// both counters to zero for the next launch.
// ---------------------------------------------------------------------------------------
constexpr int DYN_SPIN_LIMIT = 1 << 24;   // s_sleep rounds before a queue wait gives up
constexpr int DYN_ERR = 4;                // device error bit: a queue wait gave up
// With StreamArgs::dyn_test_timeout set, the queue wait's condition is never met and it gives
// up after this many rounds: the host forces the give-up path (its test), every wave still
// ends normally.
constexpr int DYN_TEST_SPIN_LIMIT = 256;

template <int WT, int EPI, bool NORM, int P>
__global__ __launch_bounds__(64 * (WG_WAVES + 1)) void gsk_dyn_kernel(StreamArgs a) {
  __shared__ float red[2][WG_WAVES][2048];
  __shared__ half_t gsh[NORM ? 8192 : 8];
  __shared__ float ss_s[NORM ? 128 * 32 : 1];
  __shared__ float rn_s[32];
  __shared__ int arrived[2], reduced, ready;
  __shared__ int q_chunk[4], q_pub;
  // abort: set by a streaming wave whose queue wait gave up; every other wait of the
  // workgroup then stops waiting, so all waves run to their end (results invalid, DYN_ERR set)
  __shared__ int abort;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x, b = blockIdx.x;
  const int KB = a.KB, S = a.dyn_static, half = KB >> 1;
  const int T0 = G * S;                          // first tile handed out at run time
  const int n_chunks = 2 * ((a.N >> 6) - T0);
  if (threadIdx.x == 0) {
    arrived[0] = arrived[1] = 0;
    reduced = 0;
    ready = 0;
    q_pub = 0;
    abort = 0;
  }
  __syncthreads();

  if (w < WG_WAVES) {
    int si = 0;
    if (S > 0)
      stream_range<WT, NORM, P>(a, gsh, rn_s, &ready, red, arrived, &reduced,
                                (long long)b * S * KB, (long long)(b + 1) * S * KB, 0, 0, w,
                                lane, si, &abort);
    const int limit = a.dyn_test_timeout ? DYN_TEST_SPIN_LIMIT : DYN_SPIN_LIMIT;
    for (int k = 0;; ++k) {
      int spins = 0;
      while (__hip_atomic_load(&q_pub, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <= k ||
             a.dyn_test_timeout) {
        if (++spins > limit ||
            __hip_atomic_load(&abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) {
          if (lane == 0) {
            atomicOr(a.err, DYN_ERR);
            __hip_atomic_store(&abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          }
          return;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      const int c = q_chunk[k & 3];
      if (c < 0) break;
      const long long c0 = (long long)(T0 + (c >> 1)) * KB + (long long)(c & 1) * half;
      stream_range<WT, NORM, P>(a, gsh, rn_s, &ready, red, arrived, &reduced, c0, c0 + half, 0,
                                0, w, lane, si, &abort);
    }
    return;
  }

  // ---- reducer wave ----
  if constexpr (NORM) reducer_norm_prologue<WT>(a, lane, gsh, ss_s, rn_s, &ready);
  int n_pub = 0;
  bool exhausted = false;
  auto publish_next = [&]() {
    if (exhausted) return;
    int c = 0;
    if (lane == 0) c = __hip_atomic_fetch_add(a.dyn_next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    c = __shfl(c, 0, 64);
    if (c >= n_chunks) {
      c = -1;
      exhausted = true;
    }
    if (lane == 0) {
      q_chunk[n_pub & 3] = c;
      __hip_atomic_store(&q_pub, n_pub + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    ++n_pub;
  };
  int si = 0;
  // ARGMAX: the best key of each row over this workgroup's tiles, one atomicMax per row at
  // the end (one per row and tile contended on the same 32 keys: 8.5 us of the lm_head)
  unsigned long long kacc = 0;
  unsigned long long* ka = EPI == EPI_ARGMAX ? &kacc : nullptr;
  for (int i = 0; i < S; ++i, ++si) {
    if (i == S - 1) publish_next();   // entry 0 before the last static segment's wait
    reduce_segment<EPI>(a, lane, red, arrived, &reduced, si, b * S + i, 0, 1, &abort, ka);
  }
  if (S == 0) publish_next();
  for (int k = 0;; ++k, ++si) {
    const int c = __shfl(q_chunk[k & 3], 0, 64);   // entry k, published by this wave
    if (c < 0) break;
    publish_next();                   // entry k + 1 before waiting for chunk k
    reduce_segment<EPI>(a, lane, red, arrived, &reduced, si, T0 + (c >> 1), c & 1, 2, &abort,
                        ka);
  }
  if constexpr (EPI == EPI_ARGMAX)
    if (a.keys && lane < 32 && lane < a.M && kacc) atomicMax(a.keys + lane, kacc);
  // this workgroup's epilogue atomics and stores are performed before it counts itself
  // finished, so the last one to finish sees every tile's argmax key
  __builtin_amdgcn_s_waitcnt(0);
  int prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(a.dyn_next + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0, 64);
  if (prev == G - 1) {
    if (EPI == EPI_ARGMAX && a.ids && a.keys && lane < a.M) {
      unsigned long long* kp = a.keys + lane;
      const unsigned long long k =
          __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      a.ids[lane] = k ? (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull)) : -1;
      __hip_atomic_store(kp, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) {
      __hip_atomic_store(a.dyn_next, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.dyn_next + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------------------
// The M-split stream-K kernel (2 <= MT <= 8): same partition, reducer and completion as
// gsk_gemm_kernel, with the m-tiles (not the k-blocks) divided among the streaming waves.
// ---------------------------------------------------------------------------------------
template <int WT, int EPI, bool NORM, int P, int MTW>
__global__ __launch_bounds__(64 * (WG_WAVES + 1)) void gsk_gemm_m_kernel(StreamArgs a) {
  constexpr int KBK = KTraits<WT>::KBK;
  __shared__ float red[2][WG_WAVES][MTW][2048];
  __shared__ half_t gsh[NORM ? 8192 : 8];
  __shared__ float rn_s[32 * WG_WAVES * MTW];
  __shared__ int arrived[2], reduced, ready;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x;
  const int b = blockIdx.x;
  const long long U = (long long)(a.N >> 6) * a.KB;
  const long long u0 = (long long)b * U / G, u1 = (long long)(b + 1) * U / G;
  if (u0 >= u1) return;
  if (threadIdx.x == 0) {
    arrived[0] = arrived[1] = 0;
    reduced = 0;
    ready = 0;
  }
  __syncthreads();

  if (w < WG_WAVES) {
    stream_range_m<WT, NORM, P, MTW>(a, gsh, rn_s, &ready, red, arrived, &reduced, u0, u1, w,
                                     lane);
    return;
  }

  // ---- reducer wave ----
  if constexpr (NORM) {
    const int K = a.KB * KBK;
    copy_to_lds(a.gnorm, gsh, K * 2, lane);
    if (lane == 0) mark_issued(&ready);
    for (int mt = 0; mt < a.MT; ++mt) {
      const float rn = a.ss_in ? rn_from_ss(a.ss_in + (size_t)mt * a.ss_mstride, a.ss_tiles,
                                            a.ss_n, a.eps, lane)
                               : a.rnorm[mt * 32 + (lane & 31)];
      if (lane < 32) rn_s[mt * 32 + lane] = rn;
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) __hip_atomic_store(&ready, PRO_DONE, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  int si = 0;
  for (long long u = u0; u < u1; ++si) {
    const int t = (int)(u / a.KB);
    const int kbs = (int)(u - (long long)t * a.KB);
    const int kbe = (int)min((long long)a.KB, (long long)kbs + (u1 - u));
    while (__hip_atomic_load(&arrived[si & 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
           WG_WAVES * ((si >> 1) + 1))
      __builtin_amdgcn_s_sleep(1);
    const bool whole = (kbs == 0 && kbe == a.KB);
    int slot = 0, count = 1;
    if (!whole) {
      const long long tu0 = (long long)t * a.KB;
      const int first = worker_of(tu0, U, G);
      count = worker_of(tu0 + a.KB - 1, U, G) - first + 1;
      slot = b - first;
    }
    // whole tile: epilogue straight from LDS; split tile: publish all m-tile partials,
    // then the last workgroup to arrive sums them slot by slot
    for (int mt = 0; mt < a.MT; ++mt) {
      const float* src = red[si & 1][mt / MTW][mt % MTW];
      floatx16 acc0, acc1;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc0[r] = src[r * 64 + lane];
        acc1[r] = src[1024 + r * 64 + lane];
      }
      if (whole) {
        tile_epilogue<EPI>(mtile_view(a, mt), lane, t, acc0, acc1);
      } else {
        float* mine = a.ws + (((size_t)t * a.seg_cap + slot) * a.MT + mt) * 2048;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          store_agent(mine + r * 64 + lane, acc0[r]);
          store_agent(mine + 1024 + r * 64 + lane, acc1[r]);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);   // slot reads (and partial stores) done
    if (lane == 0) __hip_atomic_store(&reduced, si + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (!whole) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      int prev = 0;
      if (lane == 0)
        prev = __hip_atomic_fetch_add(a.tile_cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      prev = __shfl(prev, 0, 64);
      if (prev == count - 1) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        for (int mt = 0; mt < a.MT; ++mt) {
          floatx16 acc0 = (floatx16){}, acc1 = (floatx16){};
          add_slots_at(a.ws + ((size_t)t * a.seg_cap * a.MT + mt) * 2048, (size_t)a.MT * 2048,
                       lane, count, acc0, acc1);
          tile_epilogue<EPI>(mtile_view(a, mt), lane, t, acc0, acc1);
        }
        if (lane == 0) a.tile_cnt[t] = 0;   // next use is a later launch
      }
    }
    u += kbe - kbs;
  }
}

// ---------------------------------------------------------------------------------------
// Host-side planning and launch
// ---------------------------------------------------------------------------------------

template <int WT, int EPI, bool NORM>
static void launch_dyn_t(const StreamArgs& a, const SKPlan& p, hipStream_t st, hipEvent_t e0,
                         hipEvent_t e1) {
  const dim3 grid(p.workers), block(64 * (WG_WAVES + 1));
  if (e0 || e1)
    hipExtLaunchKernelGGL((gsk_dyn_kernel<WT, EPI, NORM, 4>), grid, block, 0, st, e0, e1, 0, a);
  else
    hipLaunchKernelGGL((gsk_dyn_kernel<WT, EPI, NORM, 4>), grid, block, 0, st, a);
}

// With events, the dispatch itself records its start / end time into them (the same
// timestamps a kernel trace reports); no marker packets are added to the stream.
template <int WT, int EPI, bool NORM, bool XRM = false>
static void launch_t(const StreamArgs& a, const SKPlan& p, hipStream_t st, hipEvent_t e0,
                     hipEvent_t e1) {
  const dim3 grid(p.workers), block(64 * (WG_WAVES + 1));
  if (e0 || e1)
    hipExtLaunchKernelGGL((gsk_gemm_kernel<WT, EPI, NORM, 4, XRM>), grid, block, 0, st, e0, e1, 0,
                          a);
  else
    hipLaunchKernelGGL((gsk_gemm_kernel<WT, EPI, NORM, 4, XRM>), grid, block, 0, st, a);
}

template <int WT, int EPI, bool NORM, int MTW>
static void launch_m_w(const StreamArgs& a, const SKPlan& p, hipStream_t st, hipEvent_t e0,
                       hipEvent_t e1) {
  constexpr int P = (WT == WT_INT8) ? 3 : 4;
  const dim3 grid(p.workers), block(64 * (WG_WAVES + 1));
  if (e0 || e1)
    hipExtLaunchKernelGGL((gsk_gemm_m_kernel<WT, EPI, NORM, P, MTW>), grid, block, 0, st, e0, e1,
                          0, a);
  else
    hipLaunchKernelGGL((gsk_gemm_m_kernel<WT, EPI, NORM, P, MTW>), grid, block, 0, st, a);
}

// One m-tile per streaming wave up to 4 m-tiles, two up to 8.
template <int WT, int EPI, bool NORM>
static void launch_m_t(const StreamArgs& a, const SKPlan& p, hipStream_t st, hipEvent_t e0,
                       hipEvent_t e1) {
  if (a.MT <= WG_WAVES) launch_m_w<WT, EPI, NORM, 1>(a, p, st, e0, e1);
  else launch_m_w<WT, EPI, NORM, 2>(a, p, st, e0, e1);
}

bool launch_streamk_gemm_m(int wt, int epi, bool norm, const StreamArgs& a, const SKPlan& p,
                           hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
  if (check_stream_args(wt, epi, norm, a, p, true)) return false;
#define DFL_SKM_CASE(W_, E_)                                         \
  if (wt == W_ && epi == E_) {                                       \
    if (norm) launch_m_t<W_, E_, true>(a, p, st, ev_start, ev_stop); \
    else launch_m_t<W_, E_, false>(a, p, st, ev_start, ev_stop);     \
    return true;                                                     \
  }
  DFL_SKM_CASE(WT_INT8, EPI_STORE)
  DFL_SKM_CASE(WT_INT8, EPI_RESID)
  DFL_SKM_CASE(WT_INT8, EPI_SWIGLU)
  DFL_SKM_CASE(WT_F16, EPI_ARGMAX)
  DFL_SKM_CASE(WT_F16, EPI_STORE)
#undef DFL_SKM_CASE
  if (wt == WT_F16 && epi == EPI_RESID && !norm) {   // the per-step ingest's fc (x_zero)
    launch_m_t<WT_F16, EPI_RESID, false>(a, p, st, ev_start, ev_stop);
    return true;
  }
  return false;
}

bool launch_streamk_gemm(int wt, int epi, bool norm, const StreamArgs& a, const SKPlan& p,
                         hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
  if (check_stream_args(wt, epi, norm, a, p, false)) return false;
  if (p.dyn_static > 0) {   // balanced mode: the fp16 ARGMAX lm_head only
    if (wt != WT_F16 || epi != EPI_ARGMAX || !a.dyn_next || !a.err) return false;
    if (norm) launch_dyn_t<WT_F16, EPI_ARGMAX, true>(a, p, st, ev_start, ev_stop);
    else launch_dyn_t<WT_F16, EPI_ARGMAX, false>(a, p, st, ev_start, ev_stop);
    return true;
  }
#define DFL_SK_CASE(W_, E_)                                        \
  if (wt == W_ && epi == E_) {                                     \
    if (norm) launch_t<W_, E_, true>(a, p, st, ev_start, ev_stop); \
    else launch_t<W_, E_, false>(a, p, st, ev_start, ev_stop);     \
    return true;                                                   \
  }
  DFL_SK_CASE(WT_INT8, EPI_STORE)
  DFL_SK_CASE(WT_INT8, EPI_RESID)
  DFL_SK_CASE(WT_INT8, EPI_SWIGLU)
  DFL_SK_CASE(WT_F16, EPI_ARGMAX)
  DFL_SK_CASE(WT_F16, EPI_STORE)
  if (wt == WT_F16 && epi == EPI_RESID && !norm) {   // the per-step ingest's fc (x_zero)
    if (a.xr_n > 0) launch_t<WT_F16, EPI_RESID, false, true>(a, p, st, ev_start, ev_stop);
    else launch_t<WT_F16, EPI_RESID, false>(a, p, st, ev_start, ev_stop);
    return true;
  }
  if (wt == WT_INT8 && epi == EPI_QKROPE && norm && a.M <= 32) {   // one sequence, one m-tile
    launch_t<WT_INT8, EPI_QKROPE, true>(a, p, st, ev_start, ev_stop);
    return true;
  }
#undef DFL_SK_CASE
  return false;
}

}  // namespace dfl
