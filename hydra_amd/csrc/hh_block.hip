// hh_block.hip — the normalisation and residual kernels around the MoE layer (the whole FFN
// block): the pre-norm that turns the fp32 residual stream into the layer's bf16 input, and
// Gemma's branch post-norms, branch sum, final norm, residual add and layer scalar.
//
// Reference: ReferenceLayer.decode (ReferenceLayer.swift:189-202: rmsNorm(hidden, postNorm) →
// router/experts → hidden += mixture) with ReferenceOps.rmsNorm (ReferenceOps.swift:20-25);
// QwenLayerRunner (QwenLayerRunner.swift:11-14: hidden += mixture(post_attention_layernorm(
// hidden))); Gemma4ReferenceLayer.forward (Gemma4ReferenceLayer.swift:175-214) with
// Gemma4ReferenceOps.rmsNorm (Gemma4ReferenceOps.swift:25-31), as the GPU encodes it in
// Gemma4LayerRunner.encodeCombineBranches (Gemma4LayerRunner.swift:683-723).
//
// Arithmetic: every reduction and product is fp64 (squares of fp32 values are exact in fp64), as
// in the fp64 reference; the bf16 layer input is the fp64 value rounded once to bf16.
#include "hh_common.hpp"
#include "hh_norm.hpp"

namespace hh {

constexpr int kBlockThreads = 256;

__device__ __forceinline__ double block_sum_f64(double v, double *s_red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[w] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < kBlockThreads / 64; ++i) t += s_red[i];
  __syncthreads();
  return t;
}

// One wave per token: xn[t] = bf16(hidden[t]·f·w) (the layer's expert and router input), and,
// when xr is given, xr[t] = bf16(hidden[t]) (the residual the GEMMA router reads). The same
// arithmetic as the small-batch router kernel's own rows (norm_row_bf16).
__global__ __launch_bounds__(64) void block_norm_kernel(const float *hidden, const uint16_t *weight,
                                                        int H, float eps, int pow_form, uint16_t *xn,
                                                        uint16_t *xr) {
  const size_t t = blockIdx.x;
  norm_row_bf16(hidden + t * H, weight, H, eps, pow_form, xn + t * H, xr ? xr + t * H : nullptr);
}

// One workgroup per token, Gemma's parallel branches:
//   b1 = rms(dense, n1), b2 = rms(mix, n2), c = rms(b1 + b2, n),
//   hidden = (hidden + c) · scalar.
// s_row holds b1 + b2 in fp64 (H ≤ kMaxBlockHidden).
constexpr int kMaxBlockHidden = 8192;
__global__ __launch_bounds__(kBlockThreads) void block_gemma_finish_kernel(
    float *hidden, const float *mix, const float *dense, const uint16_t *n1, const uint16_t *n2,
    const uint16_t *n, const uint16_t *scalar, int H, float eps) {
  __shared__ double s_red[kBlockThreads / 64];
  __shared__ double s_row[kMaxBlockHidden];
  const size_t t = blockIdx.x;
  const float *d = dense + t * H, *m = mix + t * H;
  double sd = 0.0, sm = 0.0;
  for (int h = threadIdx.x; h < H; h += kBlockThreads) {
    const double a = d[h], b = m[h];
    sd += a * a;
    sm += b * b;
  }
  const double fd = norm_factor(block_sum_f64(sd, s_red), H, (double)eps, 1);
  const double fm = norm_factor(block_sum_f64(sm, s_red), H, (double)eps, 1);
  double sc = 0.0;
  for (int h = threadIdx.x; h < H; h += kBlockThreads) {
    const double b1 = (double)d[h] * fd * (double)bf16_bits_to_f32(n1[h]);
    const double b2 = (double)m[h] * fm * (double)bf16_bits_to_f32(n2[h]);
    const double s = b1 + b2;
    s_row[h] = s;
    sc += s * s;
  }
  const double fc = norm_factor(block_sum_f64(sc, s_red), H, (double)eps, 1);
  const double ls = scalar ? (double)bf16_bits_to_f32(scalar[0]) : 1.0;
  float *y = hidden + t * H;
  for (int h = threadIdx.x; h < H; h += kBlockThreads) {
    const double c = s_row[h] * fc * (double)bf16_bits_to_f32(n[h]);
    y[h] = (float)(((double)y[h] + c) * ls);
  }
}

hipError_t launch_block_norm(const float *hidden, const uint16_t *weight, int H, float eps,
                             int pow_form, int T, uint16_t *xn, uint16_t *xr, hipStream_t s) {
  hipLaunchKernelGGL(block_norm_kernel, dim3(T), dim3(64), 0, s, hidden, weight, H, eps,
                     pow_form, xn, xr);
  return hipGetLastError();
}

hipError_t launch_block_gemma_finish(float *hidden, const float *mix, const float *dense,
                                     const uint16_t *n1, const uint16_t *n2, const uint16_t *n,
                                     const uint16_t *scalar, int H, float eps, int T,
                                     hipStream_t s) {
  if (H > kMaxBlockHidden) return hipErrorInvalidValue;
  hipLaunchKernelGGL(block_gemma_finish_kernel, dim3(T), dim3(kBlockThreads), 0, s, hidden, mix,
                     dense, n1, n2, n, scalar, H, eps);
  return hipGetLastError();
}

}  // namespace hh
