// Weight preparation kernels: the W8A16 quantiser and the HBM block packers.
//
// Weight layout in HBM (written once at load by the pack kernels): blocks of 32 rows x
// KBK k-values (KBK = 32 for int8, 16 for fp16), 1 KiB each, ordered [row-block][k-block];
// inside a block lane l's 16 bytes are
//   int8: W[rb*32 + l%32][kb*32 + 16*(l/32) + 0..15], each stored as q ^ 0x80 (= q + 128)
//   fp16: W[rb*32 + l%32][kb*16 +  8*(l/32) + 0..7]
// so one wave-wide 128-bit load reads 1 KiB contiguous and hands every lane its
// v_mfma_f32_32x32x16_f16 A-fragment directly (int8: two MFMAs per load, after the exact
// int8 -> fp16 conversion).  Per-row fp16 scales are kept apart and applied in the GEMM
// epilogue: y = s * sum x*q is exact reassociation (each fp16*int8 product is exact in fp32).
#include "dfl_common.h"
#include "dfl_kernels.h"

namespace dfl {

// Symmetric per-output-channel int8 quantisation (ane_model.py:265-279):
//   max = max_k |w[n][k]| (0 -> 1),  scale = max / 127 (fp32, correctly rounded),
//   q = clamp(rint(w / scale), -127, 127),  stored scale = fp16(scale).
// Same fp32 operation sequence as the numpy reference, so results are bit-identical.
__global__ __launch_bounds__(256) void quantize_w8_kernel(const float* __restrict__ w, int64_t ic,
                                                          int8_t* __restrict__ q,
                                                          half_t* __restrict__ s) {
  __shared__ float smax[4];
  const int64_t rowi = blockIdx.x;
  const float* wr = w + rowi * ic;
  float mx = 0.f;
  for (int64_t k = threadIdx.x; k < ic; k += blockDim.x) mx = fmaxf(mx, fabsf(wr[k]));
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) smax[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
  if (mx == 0.f) mx = 1.0f;
  const float scale = __fdiv_rn(mx, 127.0f);
  int8_t* qr = q + rowi * ic;
  for (int64_t k = threadIdx.x; k < ic; k += blockDim.x) {
    float v = rintf(__fdiv_rn(wr[k], scale));
    v = fminf(fmaxf(v, -127.f), 127.f);
    qr[k] = (int8_t)(int)v;
  }
  if (threadIdx.x == 0) s[rowi] = f2h(scale);
}

void launch_quantize_w8(const float* w, int64_t oc, int64_t ic, int8_t* q, half_t* s,
                        hipStream_t st) {
  hipLaunchKernelGGL(quantize_w8_kernel, dim3((unsigned)oc), dim3(256), 0, st, w, ic, q, s);
}

__global__ __launch_bounds__(64) void pack_i8_kernel(const int8_t* __restrict__ q,
                                                     const half_t* __restrict__ s, int K,
                                                     uint4* __restrict__ dst,
                                                     half_t* __restrict__ dscale, int rb0,
                                                     int rb_step) {
  const int kb = blockIdx.x, rb = blockIdx.y, l = threadIdx.x;
  const int KB = K / 32;
  const int drb = rb0 + rb * rb_step;
  const int8_t* src = q + (size_t)(rb * 32 + (l & 31)) * K + (size_t)kb * 32 + 16 * (l >> 5);
  uint4 v = *reinterpret_cast<const uint4*>(src);
  v.x ^= 0x80808080u;   // biased bytes q + 128 (dequant_i8x16)
  v.y ^= 0x80808080u;
  v.z ^= 0x80808080u;
  v.w ^= 0x80808080u;
  dst[((size_t)drb * KB + kb) * 64 + l] = v;
  if (kb == 0 && l < 32) dscale[(size_t)drb * 32 + l] = s[(size_t)rb * 32 + l];
}

void launch_pack_i8(const int8_t* q, const half_t* s, int rows, int K, uint4* dst,
                    half_t* dst_scale, int rb0, int rb_step, hipStream_t st) {
  hipLaunchKernelGGL(pack_i8_kernel, dim3(K / 32, rows / 32), dim3(64), 0, st, q, s, K, dst,
                     dst_scale, rb0, rb_step);
}

__global__ __launch_bounds__(64) void pack_f16_kernel(const half_t* __restrict__ w, int K,
                                                      uint4* __restrict__ dst) {
  const int kb = blockIdx.x, rb = blockIdx.y, l = threadIdx.x;
  const int KB = K / 16;
  const half_t* src = w + (size_t)(rb * 32 + (l & 31)) * K + (size_t)kb * 16 + 8 * (l >> 5);
  dst[((size_t)rb * KB + kb) * 64 + l] = *reinterpret_cast<const uint4*>(src);
}

void launch_pack_f16(const half_t* w, int rows, int K, uint4* dst, hipStream_t st) {
  hipLaunchKernelGGL(pack_f16_kernel, dim3(K / 16, rows / 32), dim3(64), 0, st, w, K, dst);
}

}  // namespace dfl
