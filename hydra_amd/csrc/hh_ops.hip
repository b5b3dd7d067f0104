// hh_ops.hip — operator-level kernels behind the parity entry points.
#include "hh_common.hpp"

namespace hh {

// MXFP4 → fp32 through the same scaled convert the expert products use (then exact widening).
// One thread per 16-byte block (mxfp4_dequantize, mxfp4.metal:25). Scale byte 255 encodes NaN
// in the OCP MX format; for it this op reproduces the reference's value × +inf
// (MXFP4.swift:38-41) instead of the convert's result.
__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint8_t *blocks,
                                                            const uint8_t *scales, int64_t n,
                                                            float *out) {
  const int64_t b = blockIdx.x * 256ll + threadIdx.x;
  if (b >= n) return;
  const u32x4 w = *(const u32x4 *)(blocks + b * 16);
  const float sc = e8m0_to_f32(scales[b]);
  f32x4 *o = (f32x4 *)(out + b * 32);
  if (scales[b] == 255) {
    for (int k = 0; k < 32; ++k) {
      const uint32_t nib = (w[k >> 3] >> (4 * (k & 7))) & 0xF;
      out[b * 32 + k] = (nib & 7) ? __uint_as_float(((nib & 8) << 28) | 0x7F800000u)
                                  : __uint_as_float(0x7FC00000u);
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4 v = __builtin_bit_cast(u32x4, mxfp4_to_bf16(w[k], sc));
    o[2 * k] = f32x4{__uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xFFFF0000u),
                     __uint_as_float(v[1] << 16), __uint_as_float(v[1] & 0xFFFF0000u)};
    o[2 * k + 1] = f32x4{__uint_as_float(v[2] << 16), __uint_as_float(v[2] & 0xFFFF0000u),
                         __uint_as_float(v[3] << 16), __uint_as_float(v[3] & 0xFFFF0000u)};
  }
}

// MLX affine → fp32: fma(q, scale, bias) per value (MLXAffine.dequantize,
// Gemma4ReferenceOps.swift:210-221). One thread per output value.
__global__ __launch_bounds__(256) void mlx_dequant_kernel(const uint32_t *words,
                                                          const uint16_t *scales,
                                                          const uint16_t *biases, int rows,
                                                          int cols, int bits, int group,
                                                          float *out) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)rows * cols) return;
  const int64_t r = i / cols, c = i - r * cols;
  const int per = 32 / bits;
  const uint32_t w = words[r * (cols / per) + c / per];
  const uint32_t q = (w >> ((c % per) * bits)) & ((1u << bits) - 1u);
  const int64_t gi = r * (cols / group) + c / group;
  out[i] = __builtin_fmaf((float)q, bf16_bits_to_f32(scales[gi]), bf16_bits_to_f32(biases[gi]));
}

__global__ __launch_bounds__(256) void activation_kernel(int act, float alpha, float limit,
                                                         const float *gate, const float *up,
                                                         int64_t n, float *out) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i < n) out[i] = activate(act, gate[i], up[i], alpha, limit);
}

}  // namespace hh

namespace hh {
hipError_t launch_mxfp4_dequant(const uint8_t *blocks, const uint8_t *scales, int64_t n,
                                float *out, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     blocks, scales, n, out);
  return hipGetLastError();
}
hipError_t launch_mlx_dequant(const uint32_t *words, const uint16_t *scales,
                              const uint16_t *biases, int rows, int cols, int bits, int group,
                              float *out, hipStream_t s) {
  const int64_t n = (int64_t)rows * cols;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(mlx_dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     words, scales, biases, rows, cols, bits, group, out);
  return hipGetLastError();
}
hipError_t launch_activation(int act, float alpha, float limit, const float *gate,
                             const float *up, int64_t n, float *out, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(activation_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, act,
                     alpha, limit, gate, up, n, out);
  return hipGetLastError();
}
}  // namespace hh
