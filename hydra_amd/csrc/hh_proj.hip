// hh_proj.hip — operator-level expert projections and the weighted combine, on the layer's own
// device code.
//
// A projection y[t] = W·x[t] (+ bias) with W in one of the expert formats is run as the down
// product of a one-expert layer whose "down" tensors are W: the fp32 input rows become the
// down product's activation operand exactly as the gate-up epilogue writes it (MXFP4: three fp8
// terms per 32-column block, quant_block; BF16 / MLX: a bf16 hi + lo pair), each token routes
// to expert 0 with weight 1, and the layer's down kernels compute the product: down_small for
// up to 16 tokens, the prefill kernels (one work list of 32-token items) above. The canonical
// accumulation order makes every token's result independent of the batch, so hh_expert_gemm of
// T tokens equals T calls of hh_expert_gemv bit for bit.
//
// Reference: ForwardEncoder.expertProjection (ForwardEncoder.swift:947-972, MXFP4 + bias),
// mlxAffineProjection (:328-365), encodeProjection(.bf16) (:300-313) and their batched forms
// (BatchEncoder.expertProjection, BatchEncoder.swift:147-173); write_expert_scaled +
// sum_expert_slices (dense.metal:131-158) via LayerRunner.encodeCombineSlices
// (LayerRunner.swift:279-301).
#include "hh_common.hpp"

#include <algorithm>

namespace hh {

// One workgroup per token: the activation operand of row t (slot t) from fp32 x [T][cols], the
// token's routing (expert 0, weight 1) and, from workgroup 0, the work list of 16·nt-token
// items over all T tokens (order = identity).
template <bool MX>
__global__ __launch_bounds__(256) void proj_prepare_kernel(GemmArgs a, const float *x, int T,
                                                           int cols, int32_t *topk,
                                                           int32_t *order, int tile_tokens) {
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *xr = x + (size_t)t * cols;
  if constexpr (MX) {
    // Wave w takes the 16-block groups w, w + 4, ...; lane (g, l16) block 16·k + l16, columns
    // 8g .. 8g+7 (quant_block's layout, as the gate-up epilogue's store_hq).
    const int wave = tid >> 6, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
    const int nb = cols / 32;
    for (int k = wave; 16 * k < nb; k += 4) {
      const int b = 16 * k + l16, bc = min(b, nb - 1);
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = xr[32 * bc + 8 * g + i];
      uint32_t q[NTH][2], sb[NTH];
      quant_block<NTH>(v, q, sb);
      if (b < nb) {
#pragma unroll
        for (int j = 0; j < NTH; ++j) {
          uint8_t *row = a.hq + ((size_t)t * NTH + j) * a.hld;
          *(u32x2 *)(row + 32 * b + 8 * g) = u32x2{q[j][0], q[j][1]};
          if (g == 0) a.hs[((size_t)t * NTH + j) * (a.hld / 32) + b] = (uint8_t)sb[j];
        }
      }
    }
  } else {
    for (int i = tid; i < cols; i += 256) {
      const float v = xr[i];
      const uint32_t hi = f32_to_bf16_bits(v);
      a.h_hi[(size_t)t * a.ldh + i] = (uint16_t)hi;
      a.h_lo[(size_t)t * a.ldh + i] = (uint16_t)f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
    }
  }
  if (tid == 0) {
    topk[t] = 0;
    ((float *)a.slot_w)[t] = 1.0f;
    order[t] = t;
  }
  if (t == 0 && order) {
    const int items = (T + tile_tokens - 1) / tile_tokens;
    for (int j = tid; j < items; j += 256)
      ((int4 *)a.work)[j] = make_int4(0, j * tile_tokens, min(tile_tokens, T - j * tile_tokens), 0);
    if (tid == 0) *(int32_t *)a.n_work = items;
  }
}

hipError_t launch_proj_prepare(const GemmArgs &a, const float *x, int T, int cols, int32_t *topk,
                               int32_t *order, int tile_tokens, hipStream_t s) {
  if (a.quant == Q_MXFP4)
    hipLaunchKernelGGL(proj_prepare_kernel<true>, dim3(T), dim3(256), 0, s, a, x, T, cols, topk, order, tile_tokens);
  else
    hipLaunchKernelGGL(proj_prepare_kernel<false>, dim3(T), dim3(256), 0, s, a, x, T, cols, topk, order, tile_tokens);
  return hipGetLastError();
}

// y[t][j] = Σ_r w[t][r] · slots[t][r][j] in rank order: each slot scaled on its own, then the
// slots added from rank 0 (write_expert_scaled then sum_expert_slices, dense.metal:131-158).
// With no weights the slots are summed as they are.
__global__ __launch_bounds__(256) void combine_weighted_kernel(const float *slots, const float *w,
                                                               int T, int count, int size, float *y) {
  const size_t n = (size_t)T * size;
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const size_t t = i / size, j = i - t * size;
    const float *src = slots + t * (size_t)count * size + j;
    float total = 0.0f;
    for (int r = 0; r < count; ++r) {
      const float v = src[(size_t)r * size];
      total += w ? w[t * count + r] * v : v;
    }
    y[i] = total;
  }
}

hipError_t launch_combine_weighted(const float *slots, const float *w, int T, int count, int size,
                                   float *y, hipStream_t s) {
  const size_t n = (size_t)T * size;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_weighted_kernel, dim3(blocks), dim3(256), 0, s, slots, w, T, count, size, y);
  return hipGetLastError();
}

}  // namespace hh
