// hh_norm.hpp — the FFN block's RMSNorm of one token row into the layer's bf16 input, by one
// wave, in one fixed arithmetic shared by the block's stand-alone norm kernel and the small-batch
// router kernel (which forms the row itself): a T-token block therefore sees exactly the input of
// T one-token blocks.
//
// Reference: ReferenceOps.rmsNorm (ReferenceOps.swift:20-25), Gemma4ReferenceOps.rmsNorm
// (Gemma4ReferenceOps.swift:25-31). fp64 throughout (squares of fp32 values are exact in fp64);
// each value x·f·w is rounded once to bf16.
#pragma once
#include "hh_common.hpp"

namespace hh {

// fp64 → bf16 bits, round to nearest even, one rounding: the value is first narrowed to fp32
// with round-to-odd (truncate, then set the last bit when inexact), which keeps the information
// a later rounding to 8 significant bits needs, then rounded to bf16 by RNE.
__device__ __forceinline__ uint32_t f64_to_bf16_bits(double v) {
  float f = (float)v;
  if (f != f) return f32_to_bf16_bits(f);
  const double back = (double)f;
  if (back != v) {
    uint32_t b = __float_as_uint(f);
    if (fabs(back) > fabs(v)) b -= 1;   // the truncation: one step toward zero
    f = __uint_as_float(b | 1u);
  }
  return f32_to_bf16_bits(f);
}

// The norm's factor (mean(x²) + eps)^-½ in the family's form: 1/√(·) (ReferenceOps.rmsNorm) or
// pow(·, -½) (Gemma4ReferenceOps.rmsNorm).
__device__ __forceinline__ double norm_factor(double sumsq, int H, double eps, int pow_form) {
  const double m = sumsq / (double)H + eps;
  return pow_form ? pow(m, -0.5) : 1.0 / sqrt(m);
}

// Σ x² of row x[0..H) by one wave in the canonical lane layout of a row (that of exact_logit):
// lane l holds columns 2048i + 512u + 8l .. +7 (u = 0..3) of each 2048-column step i, and adds
// their squares in (i, u, column) order; then the lanes by a fixed butterfly. Every lane returns
// the sum. H is a multiple of 8, x 16-byte aligned. Two steps' loads go out together (columns
// past H read as zero, whose squares add nothing).
__device__ __forceinline__ double row_sumsq(const float *x, int H) {
  const int lane = threadIdx.x & 63;
  double s = 0.0;
  for (int base = 0; base < H; base += 4096) {
    f32x4 v[2][4][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int h = base + 2048 * i + 512 * u + 8 * lane;
        const int hc = min(h, H - 8);
        v[i][u][0] = *(const f32x4 *)(x + hc);
        v[i][u][1] = *(const f32x4 *)(x + hc + 4);
        if (h >= H) v[i][u][0] = v[i][u][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const double d = v[i][u][k >> 2][k & 3];
          s += d * d;
        }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  return s;
}

// One wave: dst[h] = bf16(x[h]·f·w[h]) for the row (dst may be global memory or LDS) and, when
// dst_raw is given, dst_raw[h] = bf16(x[h]) (the residual the GEMMA router reads). H is a
// multiple of 4, x 16-byte aligned, w and dst 8-byte aligned.
__device__ __forceinline__ void norm_row_bf16(const float *x, const uint16_t *w, int H, float eps,
                                              int pow_form, uint16_t *dst, uint16_t *dst_raw) {
  const int lane = threadIdx.x & 63, n4 = H / 4;
  const double f = norm_factor(row_sumsq(x, H), H, (double)eps, pow_form);
  const f32x4 *x4 = (const f32x4 *)x;
  const u32x2 *w4 = (const u32x2 *)w;
  for (int base = 0; base < n4; base += 512) {
    f32x4 v[8];
    u32x2 wv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = min(base + 64 * k + lane, n4 - 1);
      v[k] = x4[i];
      wv[k] = w4[i];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = base + 64 * k + lane;
      if (i < n4) {
        uint32_t o[4], r[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t wb = (wv[k][c >> 1] >> (16 * (c & 1))) & 0xFFFFu;
          o[c] = f64_to_bf16_bits((double)v[k][c] * f * (double)bf16_bits_to_f32(wb));
          r[c] = f32_to_bf16_bits(v[k][c]);
        }
        *(u32x2 *)(dst + 4 * i) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
        if (dst_raw) *(u32x2 *)(dst_raw + 4 * i) = u32x2{r[0] | (r[1] << 16), r[2] | (r[3] << 16)};
      }
    }
  }
}

}  // namespace hh
