// Non-causal block-diffusion attention for one draft block (dflash.py:277-319 with
// make_draft_mask -> None, dflash.py:215-233): every block query attends to every key
// of [context ; block], GQA with query head h reading KV head h / (NH/NKV).
//
// Data layout: Q [NH][B][128] (the ratio*B query rows of one KV head are contiguous),
// K cache [NKV][cap][128], V cache transposed Vt [NKV][128][cap].
//
// Work split.  The keys are cut into chunks so that (splits x KV heads) workgroups cover
// the CUs in one round (one per CU for one sequence, two for several); a chunk longer than
// 160 keys spans several LDS stages.  One workgroup handles (chunk, KV head,
// group of query tiles): its K and V are read from HBM once, through LDS, and shared by
// every query head of the KV head.  Each 32-row query tile gets KW waves that take the
// chunk's 32-key blocks round-robin; their (max, sum, O) states are merged in LDS at the
// end, so one fp32 partial per (chunk, row) goes to the merge kernel.
//
// LDS stage (up to 5 key blocks): per block, K rows [32 keys][256 B] and Vt rows
// [128 d][64 B], filled with direct global->LDS loads (global_load_lds_dwordx4, one wave
// instruction = 1 KiB).  The 16-byte chunks of each row are XOR-swizzled so the MFMA
// fragment reads below hit distinct banks (for 32- and 64-bank LDS alike).
//
// Per wave and 32-key block:
//   S^T = K * Q^T   with v_mfma_f32_32x32x16_f16, keys on the MFMA M-axis;
//   softmax per query column (16 keys per lane + 16 in lane^32), fp32, log2 domain, with
//   a lazily updated reference max (rescale only when a block's max exceeds it by > 8,
//   so p <= 2^8, exact in the merge algebra);
//   O^T += Vt * P   with P fed straight from the S^T accumulators converted to fp16.
// K rows are read in a permuted order so that accumulator r of lane (q, g) holds key
// 8g + r (r < 8) or 16 + 8g + (r - 8); those are exactly the 8-key groups the PV MFMA
// needs as its B fragment, so P never goes through LDS.
#include "dfl_common.h"
#include "dfl_kernels.h"
#include "dfl_check.h"

#include <algorithm>

namespace dfl {

namespace {

constexpr int AT_STAGE_BLOCKS = 5;              // 32-key blocks per LDS stage
constexpr int AT_KBLK = 32 * 256;               // K rows of one key block (bytes)
constexpr int AT_VBLK = 128 * 64;               // Vt rows of one key block (bytes)
constexpr int AT_STAGE_BYTES = AT_STAGE_BLOCKS * (AT_KBLK + AT_VBLK);
constexpr int AT_PART_BYTES = (64 * 64 + 2 * 64) * 4;   // one wave's O accumulators + (m, l)
constexpr float AT_RESCALE = 8.f;               // log2 slack of the lazy reference max

// chunk slot of 16-byte chunk c in K row r (16 chunks per 256-byte row)
DFL_DEV int kswz(int r) { return (r & 3) | (((r >> 3) & 1) << 2) | (((r >> 2) & 1) << 3); }
// chunk slot of chunk c (8 keys) in Vt row d of a key block (4 chunks per 64-byte row)
DFL_DEV int vswz(int d) { return ((d >> 1) & 3) ^ ((d >> 3) & 1); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

}  // namespace

// PIPE (one sequence, chunks of several stages, one workgroup of <= 5 waves per CU): two
// stage buffers (160 KiB), the next stage's loads in flight while this one computes.
// MAXW: the most waves a launch of the instantiation has.  The kernel needs about 190
// VGPRs, so a CU holds 8 of its waves (2 per SIMD): MAXW <= 8 gives every instantiation
// that budget (a 12-wave bound held it to 168 and spilled 21 VGPRs), and the launcher keeps
// a workgroup's waves within 8, or 4 where two workgroups share a CU.  The two-buffer kernel
// with 5 query tiles runs on 8 waves (SPLIT below: 32K keys 1034 vs 1050-1056 us per
// block).
template <bool PIPE, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void block_attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  const int g = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // SPLIT: the two-buffer kernel with 5 query tiles on 8 waves -- waves 0-3 take tiles 0-3
  // whole, waves 4-7 the key blocks of tile 4 round-robin (at most 7 of a stage's 25
  // tile-blocks per SIMD instead of 10); tile 4's four states merge in LDS at the end
  constexpr bool SPLIT = PIPE && MAXW == 8;
  const int KW = SPLIT ? (wv < 4 ? 1 : 4) : a.kw;
  const int qtl = SPLIT ? (wv < 4 ? wv : 4) : wv / KW;   // query tile in group
  const int kwi = SPLIT ? (wv < 4 ? 0 : wv - 4) : wv - qtl * KW;   // key lane
  const int ratio = a.NH / a.NKV;
  const int R = ratio * a.B;
  int sidx = 0;                                          // sequence of chunk blockIdx.x
  while (sidx + 1 < a.n_seq && (int)blockIdx.x >= a.chunk0[sidx + 1]) ++sidx;
  const int c = blockIdx.x - a.chunk0[sidx];             // chunk within the sequence
  const AttnSeq& sq = a.sq[sidx];
  const int qt = blockIdx.z * a.q_per_group + qtl;
  const int q = lane & 31, gg = lane >> 5;
  const int rq = qt * 32 + q;
  const bool row_ok = rq < R;

  // Q fragments (step st covers d = 64*gg + 8*st + 0..7), loaded after the first
  // stage's K/V loads are issued so the two latencies overlap.
  half8_t qf[8];
  const uint4* qp = reinterpret_cast<const uint4*>(
      a.Q + ((size_t)sidx * a.NH * a.B + (size_t)g * R + (row_ok ? rq : 0)) * 128 +
      64 * gg);   // rows >= R: never stored

  const int k_begin = c * sq.chunk;
  const int k_end = min(sq.L, k_begin + sq.chunk);

  // Permuted key row supplied by this lane as MFMA A row i = lane % 32.
  const int i = lane & 31;
  const int koff = 16 * (i >> 4) + 8 * ((i >> 2) & 1) + 4 * ((i >> 3) & 1) + (i & 3);
  const int kxor = kswz(koff);
  const int vrow = lane & 31;

  float mrun = -INFINITY, lrun = 0.f;
  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = (floatx16){};

  const half_t* kg = sq.Kc + (size_t)g * a.cap * 128;
  const half_t* vg = sq.Vt + (size_t)g * 128 * a.cap;
  const int vlast = (sq.L - 1) & ~7;   // last 8-key group holding a valid key

  // 16 segments per key block: 8 for K (4 key rows each), 8 for Vt (16 d rows each).
  // Keys past L are clamped to valid addresses; they are masked (K) or meet p = 0 (V).
  auto issue_stage = [&](int k0, unsigned char* buf) {
    const int nblk = min(AT_STAGE_BLOCKS, (k_end - k0 + 31) >> 5);
    for (int sgi = wv; sgi < 16 * nblk; sgi += nw) {
      const int j = sgi >> 4, s = sgi & 15;
      const half_t* src;
      unsigned char* dst;
      if (s < 8) {
        const int r = 4 * s + (lane >> 4);                        // key row in the block
        const int cc = (lane & 15) ^ kswz(r);
        const int key = min(k0 + 32 * j + r, sq.L - 1);
        src = kg + (size_t)key * 128 + cc * 8;
        dst = buf + j * AT_KBLK + s * 1024;
      } else {
        const int d = 16 * (s - 8) + (lane >> 2);
        const int cc = (lane & 3) ^ vswz(d);
        src = vg + (size_t)d * a.cap + min(k0 + 32 * j + 8 * cc, vlast);
        dst = buf + AT_STAGE_BLOCKS * AT_KBLK + j * AT_VBLK + (s - 8) * 1024;
      }
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)dst, 16, 0, 0);
    }
  };
  // One buffer: issue a stage, wait, compute, repeat.  PIPE: the buffers alternate, and the
  // next stage is issued into the other one before this one computes.
  int k0 = k_begin, p = 0;
  issue_stage(k0, lds);
#pragma unroll
  for (int st = 0; st < 8; ++st) qf[st] = as_half8(qp[st]);   // overlaps the first stage
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (;;) {
    const int nblk = min(AT_STAGE_BLOCKS, (k_end - k0 + 31) >> 5);
    const int kn = k0 + 32 * AT_STAGE_BLOCKS;
    const unsigned char* buf = lds + (PIPE ? p * AT_STAGE_BYTES : 0);
    if (PIPE && kn < k_end) issue_stage(kn, lds + (p ^ 1) * AT_STAGE_BYTES);

    for (int j = kwi; j < nblk; j += KW) {
      const unsigned char* kb_lds = buf + j * AT_KBLK + koff * 256;
      const unsigned char* vb_lds = buf + AT_STAGE_BLOCKS * AT_KBLK + j * AT_VBLK;
      floatx16 s = {};
      u32x4 vf[4][2];
      if constexpr (PIPE) {
        // all eight K fragment reads in flight before the first product, and the V
        // fragments read while the softmax runs (the two-buffer kernel has the registers)
        u32x4 kf[8];
        static_for<0, 8>([&](auto st) {
          kf[st] = *reinterpret_cast<const u32x4*>(kb_lds + (((8 * gg + st) ^ kxor) << 4));
        });
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, 8>([&](auto st) { s = mfma32x32x16(as_half8(kf[st]), qf[st], s); });
        static_for<0, 4>([&](auto dt) {
          const unsigned char* vr = vb_lds + (dt * 32 + vrow) * 64;
          const int vx = vswz(dt * 32 + vrow);
          vf[dt][0] = *reinterpret_cast<const u32x4*>(vr + ((gg ^ vx) << 4));
          vf[dt][1] = *reinterpret_cast<const u32x4*>(vr + (((gg + 2) ^ vx) << 4));
        });
        __builtin_amdgcn_sched_barrier(0);
      } else {
        static_for<0, 8>([&](auto st) {
          const u32x4 kf =
              *reinterpret_cast<const u32x4*>(kb_lds + (((8 * gg + st) ^ kxor) << 4));
          s = mfma32x32x16(as_half8(kf), qf[st], s);
        });
      }
      // Accumulator r holds key kbase + (r < 8 ? 8*gg + r : 16 + 8*gg + r - 8).
      const int kbase = k0 + 32 * j;
      float psum = 0.f;
      half8_t p1, p2;
      // rescale o and lrun when the block's max exceeds the lazy reference by > AT_RESCALE
      auto update_ref = [&](float bmax) {
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        if (!__all(bmax <= mrun + AT_RESCALE)) {
          const float mnew = bmax > mrun + AT_RESCALE ? bmax : mrun;
          const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
          lrun *= alpha;
          static_for<0, 4>([&](auto dt) { o[dt] *= alpha; });
          mrun = mnew;
        }
      };
      if (sq.ring_W == 0 && kbase + 32 <= k_end) {
        // every key valid: max(s * c) = max(s) * c (c > 0, rounding is monotonic), and mrun
        // is finite after update_ref, so p = 2^(s * c - mrun) needs no mask; p in fp16 two
        // per v_cvt_pk, the row sum of the fp16 p two per v_dot2 (half the VALU work of the
        // masked path, which bounds the compute of long chunks: 32K keys 1053 vs 1085 us
        // per block)
        float smax = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) smax = fmaxf(smax, s[r]);
        update_ref(smax * a.scale_log2);
        const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const half2_t ph = __builtin_convertvector(
              ((floatx2){__builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.scale_log2, -mrun)),
                         __builtin_amdgcn_exp2f(__builtin_fmaf(s[r + 1], a.scale_log2, -mrun))}),
              half2_t);
          psum = __builtin_amdgcn_fdot2(ph, one2, psum, false);
          if (r < 8) { p1[r] = ph.x; p1[r + 1] = ph.y; } else { p2[r - 8] = ph.x; p2[r - 7] = ph.y; }
        }
      } else {
        float v[16];
        if (sq.ring_W > 0) {   // sink + window cache: only the valid ring rows count
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kr = kbase + (r < 8 ? 8 * gg + r : 16 + 8 * gg + (r - 8));
            bool ok = kr < k_end;
            if (kr < sq.ring_S) {
              ok = ok && kr < sq.sink_len;
            } else {
              const int back = (sq.ring_j - 1 - (kr - sq.ring_S)) % sq.ring_W;
              ok = ok && (back < 0 ? back + sq.ring_W : back) < sq.ring_len;
            }
            v[r] = ok ? s[r] * a.scale_log2 : -INFINITY;
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kr = kbase + (r < 8 ? 8 * gg + r : 16 + 8 * gg + (r - 8));
            v[r] = kr < k_end ? s[r] * a.scale_log2 : -INFINITY;
          }
        }
        float bmax = v[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) bmax = fmaxf(bmax, v[r]);
        update_ref(bmax);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          // masked keys contribute 0 (also when every key so far was masked, mrun = -inf)
          const half_t ph = v[r] == -INFINITY ? (half_t)0.0f : f2h(__builtin_amdgcn_exp2f(v[r] - mrun));
          psum += h2f(ph);
          if (r < 8) p1[r] = ph; else p2[r - 8] = ph;
        }
      }
      lrun += psum + __shfl_xor(psum, 32, 64);
      static_for<0, 4>([&](auto dt) {
        u32x4 v1, v2;
        if constexpr (PIPE) {
          v1 = vf[dt][0];
          v2 = vf[dt][1];
        } else {
          const unsigned char* vr = vb_lds + (dt * 32 + vrow) * 64;
          const int vx = vswz(dt * 32 + vrow);
          v1 = *reinterpret_cast<const u32x4*>(vr + ((gg ^ vx) << 4));
          v2 = *reinterpret_cast<const u32x4*>(vr + (((gg + 2) ^ vx) << 4));
        }
        o[dt] = mfma32x32x16(as_half8(v1), p1, o[dt]);
        o[dt] = mfma32x32x16(as_half8(v2), p2, o[dt]);
      });
    }
    if (kn >= k_end) break;
    if (!PIPE) {
      __syncthreads();   // every wave is done with the single buffer
      issue_stage(kn, lds);
    }
    __builtin_amdgcn_s_waitcnt(0);   // this wave's loads of the next stage have landed
    __syncthreads();                 // everyone's, and no wave reads the buffer they reuse
    k0 = kn;
    p ^= 1;
  }
  __syncthreads();   // the stage buffers are reused by the merge

  // Merge the KW key lanes of each query tile (fixed order), then store the partial.
  if (SPLIT || a.kw > 1) {   // (uniform over the workgroup: every wave reaches the barrier)
    float* part = reinterpret_cast<float*>(lds) +
                  (SPLIT ? 0 : (size_t)(qtl * (KW - 1)) * (AT_PART_BYTES / 4));
    if (kwi > 0) {
      float* my = part + (size_t)(kwi - 1) * (AT_PART_BYTES / 4);
      static_for<0, 4>([&](auto dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) my[(dt * 16 + r) * 64 + lane] = o[dt][r];
      });
      my[64 * 64 + lane] = mrun;
      my[64 * 64 + 64 + lane] = lrun;
    }
    __syncthreads();
    if (kwi > 0) return;
    for (int w = 0; w < KW - 1; ++w) {
      const float* ot = part + (size_t)w * (AT_PART_BYTES / 4);
      const float m2 = ot[64 * 64 + lane], l2 = ot[64 * 64 + 64 + lane];
      const float mn = fmaxf(mrun, m2);
      if (mn == -INFINITY) continue;
      const float a1 = __builtin_amdgcn_exp2f(mrun - mn), a2 = __builtin_amdgcn_exp2f(m2 - mn);
      static_for<0, 4>([&](auto dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] * a1 + ot[(dt * 16 + r) * 64 + lane] * a2;
      });
      lrun = lrun * a1 + l2 * a2;
      mrun = mn;
    }
  }

  if (!row_ok) return;
  // partial row of all sequences: s * NH * B + h * B + b  (g * R + rq = h * B + b)
  const size_t rowg = (size_t)sidx * a.NH * a.B + (size_t)g * R + rq;
  const size_t NB = (size_t)a.n_seq * a.NH * a.B;
  float* op = a.Op + ((size_t)c * NB + rowg) * 128 + 4 * gg;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      *reinterpret_cast<floatx4*>(op + dt * 32 + 8 * qq) =
          (floatx4){o[dt][4 * qq], o[dt][4 * qq + 1], o[dt][4 * qq + 2], o[dt][4 * qq + 3]};
  if (gg == 0) {
    a.Ml[((size_t)c * NB + rowg) * 2] = mrun;
    a.Ml[((size_t)c * NB + rowg) * 2 + 1] = lrun;
  }
}

// out[b][h*128 + d] = sum_c Op_c * 2^(m_c - M) / sum_c l_c * 2^(m_c - M), fp16.
// The per-chunk (max, sum) pairs are staged in LDS first so the Op loads of all chunks
// are independent of each other.
__global__ __launch_bounds__(128) void attn_merge_kernel(AttnArgs a) {
  __shared__ float wts[64];
  __shared__ float den_s;
  const int rowg = blockIdx.x;   // s * NH * B + h * B + b
  const int d = threadIdx.x;
  const int per_seq = a.NH * a.B;
  const int sidx = rowg / per_seq;
  const size_t NB = (size_t)a.n_seq * per_seq;
  const int nc = a.sq[sidx].n_chunks;
  float mc = -INFINITY, lc = 0.f;
  if (d < nc) {
    mc = a.Ml[((size_t)d * NB + rowg) * 2];
    lc = a.Ml[((size_t)d * NB + rowg) * 2 + 1];
  }
  float M = mc;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  if (d < 64) {
    const float w = (d < nc) ? exp2f(mc - M) : 0.f;
    wts[d] = w;
    float dl = w * lc;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) dl += __shfl_xor(dl, o, 64);
    if (d == 0) den_s = dl;
  }
  // every chunk's load is issued before the first product (nc <= MAX_CHUNKS = 64), in
  // groups of 32 so that one group costs a single memory latency
  const float* op = a.Op + (size_t)rowg * 128 + d;
  float num = 0.f;
  for (int c0 = 0; c0 < nc; c0 += 32) {
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = c0 + j < nc ? op[(size_t)(c0 + j) * NB * 128] : 0.f;
    if (c0 == 0) __syncthreads();   // wts complete
#pragma unroll
    for (int j = 0; j < 32; ++j)
      if (c0 + j < nc) num += v[j] * wts[c0 + j];
  }
  const int hb = rowg - sidx * per_seq;
  const int h = hb / a.B, b = hb - h * a.B;
  const int orow = a.sq[sidx].o_row0 + b;
  a.O[afl_index(orow, h * 128 + d, a.NH * 128)] = f2h(num / den_s);
}

bool launch_block_attention(const AttnArgs& a_in, hipStream_t st) {
  if (check_attn_args(a_in)) return false;
  AttnArgs a = a_in;
  const int R = (a.NH / a.NKV) * a.B;
  const int n_qt = (R + 31) / 32;
  a.q_per_group = std::min(n_qt, 8);
  // Extra waves per query tile only where the tiles alone leave the CU short of waves;
  // each takes at least one key block of the chunk.  At most 8 waves per CU (the kernel's
  // registers allow 2 per SIMD): 8 per workgroup for one sequence (one workgroup per CU),
  // 4 for several (two per CU).
  int cblocks = 1 << 30;
  for (int i = 0; i < a.n_seq; ++i) cblocks = std::min(cblocks, a.sq[i].chunk / 32);
  const int wg_waves = a.n_seq == 1 ? 8 : 4;
  a.kw = a.q_per_group >= 3 ? 1
                            : std::max(1, std::min(std::min(4, cblocks), wg_waves / a.q_per_group));
  if (a.q_per_group * a.kw > 8) return false;   // beyond every instantiation's bound
  const int groups = (n_qt + a.q_per_group - 1) / a.q_per_group;
  const int merge_bytes = a.q_per_group * (a.kw - 1) * AT_PART_BYTES;
  const int lds_bytes = std::max(AT_STAGE_BYTES, merge_bytes);
  // two stage buffers: one sequence whose chunks span several stages, one wave per query
  // tile and at most 5 tiles, and at most one workgroup per CU (the LDS of two buffers)
  const bool pipe = a.n_seq == 1 && a.sq[0].chunk > 32 * AT_STAGE_BLOCKS && a.kw == 1 &&
                    a.q_per_group <= 5 && (long long)a.chunk0[1] * a.NKV * groups <= a.n_cu &&
                    a.lds_max >= 2 * AT_STAGE_BYTES;
  const dim3 grid(a.chunk0[a.n_seq], a.NKV, groups), block(64 * a.q_per_group * a.kw);
  if (pipe && a.q_per_group == 5)
    hipLaunchKernelGGL((block_attn_kernel<true, 8>), grid, dim3(512), 2 * AT_STAGE_BYTES, st, a);
  else if (pipe)
    hipLaunchKernelGGL((block_attn_kernel<true, 5>), grid, block, 2 * AT_STAGE_BYTES, st, a);
  else if (a.q_per_group * a.kw <= 5)
    hipLaunchKernelGGL((block_attn_kernel<false, 5>), grid, block, lds_bytes, st, a);
  else
    hipLaunchKernelGGL((block_attn_kernel<false, 8>), grid, block, lds_bytes, st, a);
  hipLaunchKernelGGL(attn_merge_kernel, dim3(a.n_seq * a.NH * a.B), dim3(128), 0, st, a);
  return true;
}

}  // namespace dfl
