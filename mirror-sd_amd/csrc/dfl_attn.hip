// Non-causal block-diffusion attention for one draft block (dflash.py:277-319 with
// make_draft_mask -> None, dflash.py:215-233): every block query attends to every key
// of [context ; block], GQA with query head h reading KV head h / (NH/NKV).
//
// Data layout: Q [NH][B][128] (the ratio*B query rows of one KV head are contiguous),
// K cache [NKV][cap][128], V cache transposed Vt [NKV][128][cap].
//
// One wave handles (key chunk, KV head, 32-row query tile):
//   S^T = K * Q^T   with v_mfma_f32_32x32x16_f16, keys on the MFMA M-axis;
//   online softmax per query column (16 keys per lane + 16 in lane^32), fp32, log2 domain;
//   O^T += Vt * P   with P fed straight from the S^T accumulators converted to fp16.
// K rows are loaded in a permuted order so that accumulator r of lane (q, g) holds key
// 8g + r (r < 8) or 16 + 8g + (r - 8); those are exactly the 8-key groups the PV MFMA
// needs as its B fragment, so P never goes through LDS.  A merge kernel combines the
// chunk partials with their (max, sum) statistics.
#include "dfl_common.h"
#include "dfl_kernels.h"

namespace dfl {

__global__ __launch_bounds__(64) void block_attn_kernel(AttnArgs a) {
  const int c = blockIdx.x, g = blockIdx.y, qt = blockIdx.z;
  const int lane = threadIdx.x;
  const int q = lane & 31, gg = lane >> 5;
  const int ratio = a.NH / a.NKV;
  const int R = ratio * a.B;
  const int rq = qt * 32 + q;
  const bool row_ok = rq < R;

  // Q fragments: step st covers d = 64*gg + 8*st + 0..7.
  half8_t qf[8];
  {
    const uint4* qp = reinterpret_cast<const uint4*>(a.Q + ((size_t)g * R + (row_ok ? rq : 0)) * 128 +
                                                     64 * gg);
#pragma unroll
    for (int st = 0; st < 8; ++st) qf[st] = as_half8(qp[st]);   // rows >= R: never stored
  }

  const int k_begin = c * a.chunk;
  const int k_end = min(a.L, k_begin + a.chunk);

  // Permuted key row supplied by this lane as MFMA A row i = lane % 32.
  const int i = lane & 31;
  const int koff = 16 * (i >> 4) + 8 * ((i >> 2) & 1) + 4 * ((i >> 3) & 1) + (i & 3);

  float mrun = -INFINITY, lrun = 0.f;
  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = (floatx16){};

  const half_t* kbase = a.Kc + (size_t)g * a.cap * 128 + 64 * gg;
  const half_t* vbase = a.Vt + (size_t)g * 128 * a.cap + 8 * gg + (size_t)(lane & 31) * a.cap;

  // K fragment of a 32-key block: this lane's key row (clamped into the chunk so the
  // address is valid; out-of-chunk keys are masked to -inf after the MFMA).
  auto load_k = [&](u32x4 (&kf)[8], int kb) {
    const int key = min(kb + koff, k_end - 1);
    const half_t* kp = kbase + (size_t)key * 128;
    static_for<0, 8>([&](auto st) { kf[st] = load_vec(kp + 8 * st); });
  };
  // V fragments (transposed cache): rows d = dt*32 + lane%32, keys kb + 8*gg + 0..7 and
  // kb + 16 + 8*gg + 0..7.  Keys past L hold finite data (zero-initialised cache) and
  // meet p = 0.
  auto load_v = [&](u32x4 (&vf)[8], int kb) {
    static_for<0, 4>([&](auto dt) {
      const half_t* vp = vbase + (size_t)dt * 32 * a.cap + kb;
      vf[2 * dt] = load_vec(vp);
      vf[2 * dt + 1] = load_vec(vp + 16);
    });
  };

  u32x4 kcur[8], knext[8], vcur[8];
  load_k(kcur, k_begin);
  for (int kb = k_begin; kb < k_end; kb += 32) {
    load_v(vcur, kb);
    const bool more = kb + 32 < k_end;
    load_k(knext, more ? kb + 32 : kb);
    __builtin_amdgcn_sched_barrier(0);
    floatx16 s = {};
    static_for<0, 8>([&](auto st) { s = mfma32x32x16(as_half8(kcur[st]), qf[st], s); });
    // Accumulator r holds key kb + (r < 8 ? 8*gg + r : 16 + 8*gg + r - 8).
    float v[16];
    float bmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb + (r < 8 ? 8 * gg + r : 16 + 8 * gg + (r - 8));
      v[r] = kr < k_end ? s[r] * a.scale_log2 : -INFINITY;
      bmax = fmaxf(bmax, v[r]);
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(mrun, bmax);
    const float alpha = exp2f(mrun - mnew);
    float psum = 0.f;
    half8_t p1, p2;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = exp2f(v[r] - mnew);
      const half_t ph = f2h(p);
      psum += h2f(ph);
      if (r < 8) p1[r] = ph; else p2[r - 8] = ph;
    }
    psum += __shfl_xor(psum, 32, 64);
    lrun = lrun * alpha + psum;
    mrun = mnew;
    static_for<0, 4>([&](auto dt) {
      o[dt] *= alpha;
      o[dt] = mfma32x32x16(as_half8(vcur[2 * dt]), p1, o[dt]);
      o[dt] = mfma32x32x16(as_half8(vcur[2 * dt + 1]), p2, o[dt]);
    });
    static_for<0, 8>([&](auto st) { kcur[st] = knext[st]; });
  }

  if (!row_ok) return;
  const int rowg = g * R + rq;   // = h * B + b
  const size_t NB = (size_t)a.NH * a.B;
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
  const int rowg = blockIdx.x;   // h * B + b
  const int d = threadIdx.x;
  const size_t NB = (size_t)a.NH * a.B;
  const int nc = a.n_chunks;
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
  __syncthreads();
  float num = 0.f;
  const float* op = a.Op + (size_t)rowg * 128 + d;
#pragma unroll 8
  for (int c = 0; c < nc; ++c) num += op[(size_t)c * NB * 128] * wts[c];
  const int h = rowg / a.B, b = rowg - h * a.B;
  a.O[afl_index(b, h * 128 + d, a.NH * 128)] = f2h(num / den_s);
}

void launch_block_attention(const AttnArgs& a, hipStream_t st) {
  const int R = (a.NH / a.NKV) * a.B;
  dim3 grid(a.n_chunks, a.NKV, (R + 31) / 32);
  hipLaunchKernelGGL(block_attn_kernel, grid, dim3(64), 0, st, a);
  hipLaunchKernelGGL(attn_merge_kernel, dim3(a.NH * a.B), dim3(128), 0, st, a);
}

}  // namespace dfl
