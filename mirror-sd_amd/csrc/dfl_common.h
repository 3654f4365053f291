// Shared device helpers for the DFlash draft kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this library:
//  * fp16 tensors are passed as uint16_t* at the C ABI and used as _Float16 here.
//  * A "row-block" is 32 consecutive output rows of a projection; MFMA tiles are
//    v_mfma_f32_32x32x16_f16 (wave64).  For that instruction lane l supplies
//    A[i = l%32][k = 8*(l/32) + 0..7] and B[k = 8*(l/32) + 0..7][j = l%32], and
//    receives D[i = 8*(r/4) + 4*(l/32) + (r%4)][j = l%32] in accumulator r.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define DFL_DEV __device__ __forceinline__

// Compile-time loop: calls f(std::integral_constant<int, I>) for I in [B, E), so array
// indices derived from I are constants and register arrays are never demoted to scratch.
template <int B, int E, class F>
DFL_DEV void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// D += A(32x16) * B(16x32), fp16 inputs, fp32 accumulate.
DFL_DEV floatx16 mfma32x32x16(half8_t a, half8_t b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

DFL_DEV half8_t as_half8(uint4 v) { return __builtin_bit_cast(half8_t, v); }
DFL_DEV uint4 as_uint4(half8_t v) { return __builtin_bit_cast(uint4, v); }

// 128-bit loads into native vector registers (u32x4 is a first-class vector, so selects
// and copies stay in VGPRs).  load_stream adds the nontemporal hint for data read once.
DFL_DEV u32x4 load_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
DFL_DEV u32x4 load_vec(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
DFL_DEV half8_t as_half8(u32x4 v) { return __builtin_bit_cast(half8_t, v); }

// Exact int8 -> fp16 conversion of 16 packed bytes (bytes 0..7 -> lo, 8..15 -> hi).  The
// packers store each weight q in [-127, 127] biased, as the byte u = q ^ 0x80 = q + 128 in
// [1, 255]; the fp16 bit pattern 0x6400 | u encodes 1024 + u exactly, so
// (0x6400 | u) - 1152 = q exactly: 16 VALU instructions per 16 weights.
DFL_DEV void dequant_i8x16(u32x4 w, half8_t& lo, half8_t& hi) {
  const uint32_t k64 = 0x64646464u;
  uint32_t d[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __builtin_amdgcn_perm(k64, d[i], 0x04010400u);      // [b0, 64, b1, 64]
    o[2 * i + 1] = __builtin_amdgcn_perm(k64, d[i], 0x04030402u);  // [b2, 64, b3, 64]
  }
  const half2_t bias = {(half_t)1152.0f, (half_t)1152.0f};
  half2_t h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = __builtin_bit_cast(half2_t, o[i]) - bias;
  lo = (half8_t){h[0].x, h[0].y, h[1].x, h[1].y, h[2].x, h[2].y, h[3].x, h[3].y};
  hi = (half8_t){h[4].x, h[4].y, h[5].x, h[5].y, h[6].x, h[6].y, h[7].x, h[7].y};
}

// Activation fragment layout ("AFL") of a 32-row activation tile X[32][K], K % 32 == 0,
// the operand order of the W8A16 MFMA loop: 1 KiB records, record (kb, h) holding for lane
// l the 8 halves X[l % 32][32*kb + 16*(l/32) + 8*h + 0..7].  One wave-wide 128-bit load of a
// record is a contiguous 1 KiB read (a row-major fragment load touches 32 cache lines).
// Offset in halves of element (m, k), m in [0, 32):
DFL_DEV size_t afl_offset(int m, int k) {
  return ((size_t)((k >> 5) * 2 + ((k >> 3) & 1)) * 64 + m + 32 * ((k >> 4) & 1)) * 8 + (k & 7);
}
// Element (row, k) of a multi-tile AFL buffer (tiles of 32 rows, each 32*K halves).
DFL_DEV size_t afl_index(int row, int k, int K) {
  return (size_t)(row >> 5) * 32 * K + afl_offset(row & 31, k);
}

DFL_DEV float h2f(half_t h) { return (float)h; }
DFL_DEV half_t f2h(float f) { return (half_t)f; }   // round-to-nearest-even
// RMSNorm output expression: fp16(fp16(x * r) * g)  (nn.RMSNorm, dflash.py:338-339).
DFL_DEV half_t rms_out(float x, float r, half_t g) { return f2h(h2f(f2h(x * r)) * h2f(g)); }
// rms_out with fp16(x * r) rounded once from the exact product (v_fma_mix with a +0 addend,
// so a zero product comes out +0).  The compiler turns f2h(x * r) into either that or an fp32
// product and a conversion (two roundings, now and then a different fp16) depending on the
// surrounding code; a kernel whose results must not depend on that choice uses this form.
DFL_DEV half_t rms_out_once(float x, float r, half_t g) {
  uint32_t d = 0;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "+v"(d) : "v"(x), "v"(r));
  return f2h(h2f(__builtin_bit_cast(half_t, (uint16_t)d)) * h2f(g));
}
// fp16(a * b + c) rounded once from the exact fma (the same choice for fp16(fmaf(a, b, c))).
DFL_DEV half_t fma_f16_once(float a, float b, float c) {
  uint32_t d = 0;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3" : "+v"(d) : "v"(a), "v"(b), "v"(c));
  return __builtin_bit_cast(half_t, (uint16_t)d);
}
// fp16(x * s) for an fp16 scale s, rounded once from the exact product (the same choice).
DFL_DEV half_t mul_f16_once(float x, half_t s) {
  uint32_t d = 0;
  const uint32_t sv = __builtin_bit_cast(uint16_t, s);
  asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "+v"(d) : "v"(x), "v"(sv));
  return __builtin_bit_cast(half_t, (uint16_t)d);
}

// Wave64 reductions via cross-lane shuffles.
DFL_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
DFL_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Block-wide sum over all threads (blockDim.x a multiple of 64, <= 1024).
DFL_DEV float block_sum(float v, float* smem /* >= 16 floats */) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) smem[w] = v;
  __syncthreads();
  float t = 0.f;
  const int nw = blockDim.x >> 6;
  for (int i = 0; i < nw; ++i) t += smem[i];   // fixed order: deterministic
  return t;
}

// Gumbel-max sampling: argmax_n (l_n / T + G_n) over independent standard Gumbel G_n is a
// draw from softmax(l / T) (the categorical of dflash.py:133-136).  The noise of (row,
// column) comes from a 32-bit integer hash (C. Wellons' "lowbias32" finaliser) of the column
// mixed with the row's salt, itself a hash of the call's seed and the row; U = (24 hash bits
// + 1/2) 2^-24 lies in (0, 1) and G = -ln(-ln U), so G never exceeds 17.3.
DFL_DEV uint32_t hash32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
DFL_DEV uint32_t gumbel_row_salt(uint32_t seed, int row) {
  return hash32(seed ^ hash32((uint32_t)row * 0x9E3779B9u + 0x85ebca6bu));
}
DFL_DEV float gumbel_noise(uint32_t salt, int col) {
  const uint32_t h = hash32(salt ^ ((uint32_t)col * 0xc2b2ae35u));
  const float u = ((float)(h >> 8) + 0.5f) * (1.0f / 16777216.0f);
  return -__logf(-__logf(u));
}

// Monotone map of a float onto uint32 so that unsigned comparison orders floats.
DFL_DEV uint32_t float_order_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
