// hh_logit.hpp — exact fp64 router logits of single (token, expert) pairs, one wave each: the
// small-batch router kernel and the fused decode kernel both compute them this way.
//
// Reference: router_topk (attention.metal:249-300), gemma_router_topk (gemma.metal:158),
// ReferenceOps.router (ReferenceOps.swift:173-183), QwenReferenceOps.router (:159-179),
// Gemma4ReferenceOps.router (:131-156).
#pragma once
#include "hh_common.hpp"
#include "hh_norm.hpp"

namespace hh {

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// The wave sums of N values at once (N a power of two ≤ 64) as a reduce-scatter over the same
// butterfly as wave_sum_f64 (partners l ^ 32, l ^ 16, ..., l ^ 1; every node adds the same two
// operands, in one order or the other), so each total has wave_sum_f64's bits. While more than
// one value is left, a level halves them: the lanes with the level's bit clear keep the first
// half, the others the second (levels 32 and 16 on the row swaps, the rest on shuffles).
// Returns the total of v[lane >> (6 − log2 N)]. Every lane must be active.
__device__ __forceinline__ void swap32_f64(double &a, double &b, int m) {
  const uint64_t ua = (uint64_t)__double_as_longlong(a), ub = (uint64_t)__double_as_longlong(b);
  uint32_t alo = (uint32_t)ua, ahi = (uint32_t)(ua >> 32), blo = (uint32_t)ub, bhi = (uint32_t)(ub >> 32);
  if (m == 32) {
    const auto l = __builtin_amdgcn_permlane32_swap(alo, blo, false, false);
    const auto h = __builtin_amdgcn_permlane32_swap(ahi, bhi, false, false);
    alo = l[0]; blo = l[1]; ahi = h[0]; bhi = h[1];
  } else {
    const auto l = __builtin_amdgcn_permlane16_swap(alo, blo, false, false);
    const auto h = __builtin_amdgcn_permlane16_swap(ahi, bhi, false, false);
    alo = l[0]; blo = l[1]; ahi = h[0]; bhi = h[1];
  }
  a = __longlong_as_double((long long)(((uint64_t)ahi << 32) | alo));
  b = __longlong_as_double((long long)(((uint64_t)bhi << 32) | blo));
}
template <int N>
__device__ __forceinline__ double wave_sum_scatter_f64(double (&v)[N]) {
  const int lane = threadIdx.x & 63;
  int c = N;
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    if (c > 1) {
      const int h = c / 2;
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        if (i < h) {
          if (m >= 16) {
            // the pair's two results hold, in every lane, its own and its partner's value of
            // the half that lane keeps
            double a = v[i], b = v[i + h];
            swap32_f64(a, b, m);
            v[i] = a + b;
          } else {
            const bool up = lane & m;
            const double keep = up ? v[i + h] : v[i], send = up ? v[i] : v[i + h];
            v[i] = keep + __shfl_xor(send, m);
          }
        }
      }
      c = h;
    } else {
      v[0] += __shfl_xor(v[0], m);
    }
  }
  return v[0];
}

__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float bf_lo(uint32_t v) { return bf16_bits_to_f32(v & 0xFFFF); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return bf16_bits_to_f32(v >> 16); }

// Exact (fp64) router logit of expert e for token row xr, in the oracle's arithmetic: one wave.
// A bf16·bf16 product is exact in fp32, so each term is formed in fp32 and added in fp64:
// the same value as an fp64 fma. GEMMA: Σ (((x·s)·scale)·root)·w in fp64 with
// s = (Σx²/H + eps)^-½ passed in `norm`. Lane l takes columns 2048·i + 512·u + 8l .. +7 into
// accumulator u (i ascending), and the logit is (acc0 + acc1) + (acc2 + acc3). Rows of at most
// 4096 columns issue all their loads (two 2048-column steps) before the first product, so a dot
// costs one memory latency and a short dependency chain.
template <bool gemma>
__device__ __forceinline__ double exact_logit(const RouteArgs &a, const uint16_t *xr,
                                              const uint16_t *wrow, double norm, double root) {
  const int lane = threadIdx.x & 63, H = a.hidden;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  struct Step {
    u32x4 xv[4], wv[4], sv[4];
  };
  // Loads are unconditional (clamped into the row) and masked afterwards: a load under a
  // lane-dependent branch would be waited for before the next one is issued.
  auto load = [&](Step &st, int base) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int h = base + lane * 8 + 512 * u;
      const int hc = min(h, H - 8);
      st.xv[u] = *(const u32x4 *)(xr + hc);
      st.wv[u] = *(const u32x4 *)(wrow + hc);
      st.sv[u] = gemma ? *(const u32x4 *)(a.router_scale + hc) : u32x4{0u, 0u, 0u, 0u};
      if (h >= H) st.wv[u] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto add = [&](const Step &st) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int sh = (k & 1) * 16;
        const float xf = bf16_bits_to_f32((st.xv[u][k >> 1] >> sh) & 0xFFFF);
        const float wf = bf16_bits_to_f32((st.wv[u][k >> 1] >> sh) & 0xFFFF);
        if constexpr (gemma) {
          const double xd = (((double)xf * norm) *
                             (double)bf16_bits_to_f32((st.sv[u][k >> 1] >> sh) & 0xFFFF)) * root;
          acc[u] = fma(xd, (double)wf, acc[u]);
        } else {
          acc[u] += (double)(xf * wf);
        }
      }
    }
  };
  if (H <= 4096) {
    // Both steps' loads first (the second clamped into the row when H ≤ 2048, and not added).
    Step s0, s1;
    load(s0, 0);
    load(s1, 2048);
    add(s0);
    if (H > 2048) add(s1);
  } else {
    for (int base = 0; base < H; base += 2048) {
      Step st;
      load(st, base);
      add(st);
    }
  }
  return wave_sum_f64((acc[0] + acc[1]) + (acc[2] + acc[3]));
}

// Logit of (token t, expert e) in the oracle's arithmetic, whole wave (every lane returns it);
// e == E is the shared expert's gate row.
template <bool gemma>
__device__ __forceinline__ double pair_logit(const RouteArgs &a, int t, int e) {
  const int lane = threadIdx.x & 63, E = a.experts, H = a.hidden;
  double v;
  if (e < E) {
    const uint16_t *xr = a.xr + (size_t)t * H;
    double norm = 1.0, root = 1.0;
    if constexpr (gemma) {
      double xx = 0.0;
      for (int base = 0; base < H; base += 2048) {
        u32x4 xv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int h = base + lane * 8 + 512 * u;
          xv[u] = *(const u32x4 *)(xr + min(h, H - 8));
          if (h >= H) xv[u] = u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          double px = 0.0;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const float xf = bf16_bits_to_f32((xv[u][k >> 1] >> ((k & 1) * 16)) & 0xFFFF);
            px += (double)(xf * xf);
          }
          xx += px;
        }
      }
      xx = wave_sum_f64(xx);
      norm = pow(xx / (double)H + (double)a.eps, -0.5);
      root = pow((double)H, -0.5);
    }
    v = exact_logit<gemma>(a, xr, a.router_w + (size_t)e * H, norm, root);
    if (a.router_b) v += (double)bf16_bits_to_f32(a.router_b[e]);
  } else {
    v = exact_logit<false>(a, a.x + (size_t)t * H, a.shared_gate, 1.0, 1.0);
  }
  return v;
}

// exact_logit of R rows at once (the loads of all R rows of a 2048-column pass in flight
// together): for each row the same per-lane arithmetic, so the same values bit for bit.
template <bool gemma, int R>
__device__ __forceinline__ void exact_logits_rows(const RouteArgs &a, const uint16_t *xr,
                                                  const uint16_t *const (&wrow)[R], double norm,
                                                  double root, double (&out)[R]) {
  const int lane = threadIdx.x & 63, H = a.hidden;
  double acc[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[r][u] = 0.0;
  for (int base = 0; base < H; base += 2048) {
    u32x4 xv[4], sv[4], wv[R][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int h = base + lane * 8 + 512 * u;
      const int hc = min(h, H - 8);
      const bool ok = h < H;
      xv[u] = *(const u32x4 *)(xr + hc);
      sv[u] = gemma ? *(const u32x4 *)(a.router_scale + hc) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        wv[r][u] = *(const u32x4 *)(wrow[r] + hc);
        if (!ok) wv[r][u] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int sh = (k & 1) * 16;
          const float xf = bf16_bits_to_f32((xv[u][k >> 1] >> sh) & 0xFFFF);
          const float wf = bf16_bits_to_f32((wv[r][u][k >> 1] >> sh) & 0xFFFF);
          if constexpr (gemma) {
            const double xd = (((double)xf * norm) *
                               (double)bf16_bits_to_f32((sv[u][k >> 1] >> sh) & 0xFFFF)) * root;
            acc[r][u] = fma(xd, (double)wf, acc[r][u]);
          } else {
            acc[r][u] += (double)(xf * wf);
          }
        }
      }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = wave_sum_f64((acc[r][0] + acc[r][1]) + (acc[r][2] + acc[r][3]));
}

// Logit of (token t, row e; e == E the shared expert's gate row) with the 4 waves of a workgroup
// (H ≤ 4096): wave u forms accumulator u of exact_logit (columns 2048i + 512u + 8l .. +7, i
// ascending) and wave 0 adds the four in exact_logit's order, (acc0 + acc1) + (acc2 + acc3), then
// sums the wave: the same value with a quarter of the products on each wave's dependent chain.
// GEMMA's norm: wave u forms the partial Σx² of each (step, slice u), and every wave adds them in
// pair_logit's order (steps ascending, slices ascending within a step) before the wave sum.
// Every wave of the workgroup calls it (barriers); wave 0 returns the logit, the others 0.
template <bool gemma>
__device__ __forceinline__ double split_pair_logit(const RouteArgs &a, int t, int e, double (*s_acc)[64],
                                                   double (*s_px)[2][64]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.experts, H = a.hidden;
  const bool sg = e == E;                 // the shared expert's gate row: plain dot, no bias
  const bool gm = gemma && !sg;
  const uint16_t *xr = (sg ? a.x : a.xr) + (size_t)t * H;
  const uint16_t *wrow = sg ? a.shared_gate : a.router_w + (size_t)e * H;
  const int u = wave, nb = H > 2048 ? 2 : 1;
  u32x4 xv[2], wv[2], sv[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int h = 2048 * b + lane * 8 + 512 * u;
    const int hc = min(h, H - 8);
    xv[b] = *(const u32x4 *)(xr + hc);
    wv[b] = *(const u32x4 *)(wrow + hc);
    sv[b] = gm ? *(const u32x4 *)(a.router_scale + hc) : u32x4{0u, 0u, 0u, 0u};
    if (h >= H) wv[b] = u32x4{0u, 0u, 0u, 0u};
  }
  double norm = 1.0, root = 1.0;
  if (gm) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int h = 2048 * b + lane * 8 + 512 * u;
      double px = 0.0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float xf = h < H ? bf16_bits_to_f32((xv[b][k >> 1] >> ((k & 1) * 16)) & 0xFFFF) : 0.f;
        px += (double)(xf * xf);
      }
      s_px[u][b][lane] = px;
    }
    __syncthreads();
    double xx = 0.0;
    for (int b = 0; b < nb; ++b)
#pragma unroll
      for (int uu = 0; uu < 4; ++uu) xx += s_px[uu][b][lane];
    xx = wave_sum_f64(xx);
    norm = pow(xx / (double)H + (double)a.eps, -0.5);
    root = pow((double)H, -0.5);
  }
  double acc = 0.0;
  for (int b = 0; b < nb; ++b)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int sh = (k & 1) * 16;
      const float xf = bf16_bits_to_f32((xv[b][k >> 1] >> sh) & 0xFFFF);
      const float wf = bf16_bits_to_f32((wv[b][k >> 1] >> sh) & 0xFFFF);
      if (gm) {
        const double xd = (((double)xf * norm) * (double)bf16_bits_to_f32((sv[b][k >> 1] >> sh) & 0xFFFF)) * root;
        acc = fma(xd, (double)wf, acc);
      } else {
        acc += (double)(xf * wf);
      }
    }
  s_acc[u][lane] = acc;
  __syncthreads();
  if (wave != 0) return 0.0;
  double v = wave_sum_f64((s_acc[0][lane] + s_acc[1][lane]) + (s_acc[2][lane] + s_acc[3][lane]));
  if (!sg && a.router_b) v += (double)bf16_bits_to_f32(a.router_b[e]);
  return v;
}

// split_pair_logit for the FFN block (non-GEMMA router, H ≤ 4096), whose layer input x is not in
// memory: each wave loads token t's residual row in row_sumsq's layout (lane l: columns 2048i +
// 512u + 8l .. +7), sums its squares in row_sumsq's order and butterfly, takes the norm factor f
// and rounds its own slice u to x = bf16(resid·f·norm_w), the values the block's norm kernel
// writes; the products, the per-slice sums and the wave sum are split_pair_logit's. Row E (the
// shared gate) takes the same x. Every global load goes out before the first arithmetic.
__device__ __forceinline__ double block_pair_logit(const RouteArgs &a, int t, int e, double (*s_acc)[64]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.experts, H = a.hidden;
  const bool sg = e == E;
  const uint16_t *wrow = sg ? a.shared_gate : a.router_w + (size_t)e * H;
  const float *x = a.resid + (size_t)t * H;
  const int u = wave, nb = H > 2048 ? 2 : 1;
  f32x4 xv[2][4][2];
  u32x4 wv[2], nv[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int uu = 0; uu < 4; ++uu) {
      const int h = 2048 * i + 512 * uu + 8 * lane;
      const int hc = min(h, H - 8);
      xv[i][uu][0] = *(const f32x4 *)(x + hc);
      xv[i][uu][1] = *(const f32x4 *)(x + hc + 4);
      if (h >= H) xv[i][uu][0] = xv[i][uu][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int h = 2048 * b + 512 * u + 8 * lane;
    const int hc = min(h, H - 8);
    wv[b] = *(const u32x4 *)(wrow + hc);
    nv[b] = *(const u32x4 *)(a.norm_w + hc);
    if (h >= H) wv[b] = u32x4{0u, 0u, 0u, 0u};
  }
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int uu = 0; uu < 4; ++uu)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const double d = xv[i][uu][k >> 2][k & 3];
        ss += d * d;
      }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const double f = norm_factor(ss, H, (double)a.norm_eps, a.norm_pow);
  double acc = 0.0;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if (b >= nb) break;
    f32x4 x0 = xv[b][0][0], x1 = xv[b][0][1];   // slice u of step b (u is wave-uniform)
#pragma unroll
    for (int uu = 1; uu < 4; ++uu)
      if (u == uu) {
        x0 = xv[b][uu][0];
        x1 = xv[b][uu][1];
      }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int sh = (k & 1) * 16;
      const float rv = k < 4 ? x0[k] : x1[k - 4];
      const float nf = bf16_bits_to_f32((nv[b][k >> 1] >> sh) & 0xFFFF);
      const float xf = bf16_bits_to_f32(f64_to_bf16_bits((double)rv * f * (double)nf));
      const float wf = bf16_bits_to_f32((wv[b][k >> 1] >> sh) & 0xFFFF);
      acc += (double)(xf * wf);
    }
  }
  s_acc[u][lane] = acc;
  __syncthreads();
  if (wave != 0) return 0.0;
  double v = wave_sum_f64((s_acc[0][lane] + s_acc[1][lane]) + (s_acc[2][lane] + s_acc[3][lane]));
  if (!sg && a.router_b) v += (double)bf16_bits_to_f32(a.router_b[e]);
  return v;
}

}  // namespace hh
