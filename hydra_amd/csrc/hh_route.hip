// hh_route.hip — router logits, top-k weights and token→expert dispatch.
//
// route_kernel: one 256-thread workgroup per 16-token tile, no cross-workgroup synchronisation.
//   A. Router logits of the tile against every expert with v_mfma_f32_16x16x32_bf16 (exact
//      bf16·bf16 products, fp32 accumulation), the 4 waves splitting K, plus each expert row's
//      norm.
//   B. Per token: every fp32 logit lies within err = 2·H·2^-23·‖x‖·‖w_e‖ of the exact one
//      (recursive summation bound with Cauchy-Schwarz). Experts whose upper bound reaches the
//      K-th largest lower bound are the only ones that can be in the exact top-k; their logits
//      are recomputed in fp64 (the oracle's arithmetic) and the top-k is selected among them
//      with ties to the smaller index. Indices therefore equal those of an fp64 router, and
//      weights are computed from fp64 logits.
//   C. dispatch_kernel then groups the batch's assignments by expert.
//
// Batches of at most 16 tokens skip the screening: logits64_kernel computes every logit in
// fp64 (one wave per (token, expert)) and select_kernel selects and dispatches in one
// workgroup.
//
// Reference: router_topk / router_topk_batch (attention.metal:249, batch.metal:430),
// gemma_router_topk (gemma.metal:158), ReferenceOps.router (ReferenceOps.swift:173-183),
// QwenReferenceOps.router (:159-179), Gemma4ReferenceOps.router (:131-156),
// PrefillRunner.assignments (PrefillRunner.swift:224-246).
#include "hh_common.hpp"

namespace hh {

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o));
  return v;
}

// Exclusive scan of data[0..n) in place (n ≤ 512), 256 threads; returns the total.
__device__ int block_exclusive_scan(int *data, int n, int *s_wave) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int a0 = (2 * tid < n) ? data[2 * tid] : 0;
  int a1 = (2 * tid + 1 < n) ? data[2 * tid + 1] : 0;
  int v = a0 + a1, inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  if (lane == 63) s_wave[wave] = inc;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += s_wave[w];
  int total = s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
  int ex = base + inc - v;
  __syncthreads();
  if (2 * tid < n) data[2 * tid] = ex;
  if (2 * tid + 1 < n) data[2 * tid + 1] = ex + a0;
  __syncthreads();
  return total;
}

// Stable token→expert permutation of the whole batch by one workgroup.
__device__ void dispatch_batch(const RouteArgs &a) {
  __shared__ int s_cnt[kMaxExperts + 1];
  __shared__ int s_off[kMaxExperts + 1];
  __shared__ int s_tiles[kMaxExperts + 1];
  __shared__ int s_run[kMaxExperts];
  __shared__ int s_wcnt[4][kMaxExperts];
  __shared__ int s_wave[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = a.experts, K = a.top_k, T = a.tokens, A = T * K;
  const int TN = a.tile_tokens;
  for (int e = tid; e <= E; e += 256) s_cnt[e] = 0;
  for (int e = tid; e < E; e += 256) {
    s_run[e] = 0;
    for (int w = 0; w < 4; ++w) s_wcnt[w][e] = 0;
  }
  __syncthreads();
  for (int i = tid; i < A; i += 256) atomicAdd(&s_cnt[a.topk_idx[i]], 1);
  __syncthreads();
  for (int e = tid; e < E; e += 256) {
    s_off[e] = s_cnt[e];
    s_tiles[e] = (s_cnt[e] + TN - 1) / TN;
  }
  __syncthreads();
  int routed_positions = block_exclusive_scan(s_off, E, s_wave);
  int routed_tiles = block_exclusive_scan(s_tiles, E, s_wave);
  (void)routed_positions;
  // Stable scatter in chunks of 256 assignments, (t, r) order preserved inside each expert.
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
  for (int base = 0; base < A; base += 256) {
    const int i = base + tid;
    const bool valid = i < A;
    const int e = valid ? a.topk_idx[i] : 0;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      uint64_t m = __ballot(valid && ((e >> b) & 1));
      peers &= ((e >> b) & 1) ? m : ~m;
    }
    const int rank = __popcll(peers & ((1ull << lane) - 1ull));
    if (valid && rank == 0) s_wcnt[wave][e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pos = s_off[e] + s_run[e] + rank;
      for (int w = 0; w < wave; ++w) pos += s_wcnt[w][e];
      const int t = i / K, r = i - t * K;
      a.order[pos] = t * a.slots + r;
    }
    __syncthreads();
    for (int x = tid; x < E; x += 256) {
      s_run[x] += s_wcnt[0][x] + s_wcnt[1][x] + s_wcnt[2][x] + s_wcnt[3][x];
      s_wcnt[0][x] = s_wcnt[1][x] = s_wcnt[2][x] = s_wcnt[3][x] = 0;
    }
    __syncthreads();
  }
  // Segments and work items (expert, first position, tokens), ascending expert order.
  for (int e = tid; e < E; e += 256) {
    a.seg[e] = s_off[e];
    const int n = s_cnt[e];
    for (int j = 0; j * TN < n; ++j)
      a.work[s_tiles[e] + j] = make_int4(e, s_off[e] + j * TN, min(TN, n - j * TN), 0);
  }
  int nwork = routed_tiles;
  if (a.shared_gate) {
    // The shared expert is expert id E over every token, after the routed positions.
    for (int t = tid; t < T; t += 256) a.order[A + t] = t * a.slots + K;
    const int st = (T + TN - 1) / TN;
    for (int j = tid; j < st; j += 256)
      a.work[routed_tiles + j] = make_int4(E, A + j * TN, min(TN, T - j * TN), 0);
    nwork += st;
    if (tid == 0) { a.seg[E] = A; a.seg[E + 1] = A + T; }
  } else if (tid == 0) {
    a.seg[E] = A;
    a.seg[E + 1] = A;
  }
  if (tid == 0) *a.n_work = nwork;
}


constexpr int RT_TOK = 16;          // tokens per route workgroup
constexpr int RT_MAXCAND = 64;      // exact-recompute candidates handled per pass

__device__ __forceinline__ float bf_lo(uint32_t v) { return bf16_bits_to_f32(v & 0xFFFF); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return bf16_bits_to_f32(v >> 16); }

// Projection input of the router for token row `xr` at column block [h, h+8): GEMMA uses
// u = x·scale split exactly into bf16 hi + lo (x·scale has at most 16 significant bits);
// the other routers use x itself (lo = 0).
__device__ __forceinline__ void router_operand(const RouteArgs &a, const uint16_t *xr, int h,
                                               u32x4 &hi, u32x4 &lo) {
  const u32x4 xv = *(const u32x4 *)(xr + h);
  if (a.router != R_GEMMA) {
    hi = xv;
    lo = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  const u32x4 sv = *(const u32x4 *)(a.router_scale + h);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float u0 = bf_lo(xv[k]) * bf_lo(sv[k]), u1 = bf_hi(xv[k]) * bf_hi(sv[k]);
    const uint32_t h0 = f32_to_bf16_bits(u0), h1 = f32_to_bf16_bits(u1);
    const uint32_t l0 = f32_to_bf16_bits(u0 - bf16_bits_to_f32(h0));
    const uint32_t l1 = f32_to_bf16_bits(u1 - bf16_bits_to_f32(h1));
    hi[k] = h0 | (h1 << 16);
    lo[k] = l0 | (l1 << 16);
  }
}

// Exact (fp64) router logit of expert e for token row xr, in the oracle's arithmetic: one wave.
// GEMMA: Σ (((x·s)·scale)·root)·w with s = (Σx²/H + eps)^-½ passed in `norm`.
__device__ double exact_logit(const RouteArgs &a, const uint16_t *xr, const uint16_t *wrow,
                              bool gemma, double norm, double root) {
  const int lane = threadIdx.x & 63, H = a.hidden;
  double acc = 0.0;
  for (int h = lane * 8; h < H; h += 512) {
    const u32x4 xv = *(const u32x4 *)(xr + h);
    const u32x4 wv = *(const u32x4 *)(wrow + h);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      double xd = bf16_bits_to_f32((xv[k >> 1] >> ((k & 1) * 16)) & 0xFFFF);
      const double wd = bf16_bits_to_f32((wv[k >> 1] >> ((k & 1) * 16)) & 0xFFFF);
      if (gemma) xd = ((xd * norm) * (double)bf16_bits_to_f32(a.router_scale[h + k])) * root;
      acc = fma(xd, wd, acc);
    }
  }
  return wave_sum_f64(acc);
}

// Weights of one token's selection (by lane 0): sel_v are fp64 logits in rank order.
__device__ void finish_token(const RouteArgs &a, int t, const double *sel_v, const int *sel_i,
                             double sg_logit) {
  const int K = a.top_k;
  double w[kMaxTopK];
  double total = 0.0;
  // TOPK_SOFTMAX: softmax over the k selected logits (ReferenceOps.swift:178-182).
  // SOFTMAX_TOPK_RENORM and GEMMA: softmax over all experts, renormalised over the k
  // (QwenReferenceOps.swift:159-179, Gemma4ReferenceOps.swift:146-155); the full-softmax
  // denominator cancels, leaving the same softmax of the k selected logits.
  const double peak = sel_v[0];
  for (int r = 0; r < K; ++r) { w[r] = exp(sel_v[r] - peak); total += w[r]; }
  for (int r = 0; r < K; ++r) w[r] /= total;
  if (a.router == R_GEMMA)
    for (int r = 0; r < K; ++r) w[r] *= (double)bf16_bits_to_f32(a.router_pes[sel_i[r]]);
  for (int r = 0; r < K; ++r) {
    a.topk_idx[(size_t)t * K + r] = sel_i[r];
    a.topk_w[(size_t)t * K + r] = (float)w[r];
    a.slot_w[(size_t)t * a.slots + r] = (float)w[r];
  }
  if (a.logits)
    for (int r = 0; r < K; ++r) a.logits[(size_t)t * K + r] = sel_v[r];
  if (a.shared_gate) {
    // σ of the shared gate row, applied to the shared expert's output
    // (QwenReferenceLayer.swift:399-404).
    const double sg = 1.0 / (1.0 + exp(-sg_logit));
    a.slot_w[(size_t)t * a.slots + K] = (float)sg;
    if (a.shared_w) a.shared_w[t] = (float)sg;
  }
}

__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, l16 = lane & 15;
  const int E = a.experts, H = a.hidden, K = a.top_k, T = a.tokens;
  const int t0 = blockIdx.x * RT_TOK;
  const int ntok = min(RT_TOK, T - t0);
  const bool gemma = (a.router == R_GEMMA);

  __shared__ float s_part[4][16][16];          // [wave][expert in tile][token]
  __shared__ float s_wpart[4][16];              // [wave][expert in tile] Σw² partials
  __shared__ float s_logit[RT_TOK][kMaxExperts];
  __shared__ float s_wn[kMaxExperts];           // ‖w_e‖
  __shared__ int s_cand[4][RT_MAXCAND];
  __shared__ double s_exact[4][RT_MAXCAND];

  // ---- A: fp32 logits of the tile, K split over the 4 waves ----
  const int tok_lane = t0 + min(l16, ntok - 1);
  const uint16_t *xr_lane = a.xr + (size_t)tok_lane * H;
  const int nch = H / 128 + ((H % 128) ? 1 : 0);
  const int ntiles = (E + 15) / 16;
  for (int et = 0; et < ntiles; ++et) {
    const int e_lane = min(et * 16 + l16, E - 1);
    const uint16_t *wrow = a.router_w + (size_t)e_lane * H;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float wsq = 0.f;
    for (int c = wave; c < nch; c += 4) {
      const int col = min(128 * c + 32 * g, H - 32);
      const bool ok = 128 * c + 32 * g < H;
      u32x4 wv[4], xh[4], xl[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        wv[v] = ok ? *(const u32x4 *)(wrow + col + 8 * v) : u32x4{0u, 0u, 0u, 0u};
        router_operand(a, xr_lane, col + 8 * v, xh[v], xl[v]);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float w0 = bf_lo(wv[v][k]), w1 = bf_hi(wv[v][k]);
          wsq = __builtin_fmaf(w0, w0, wsq);
          wsq = __builtin_fmaf(w1, w1, wsq);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wv[v]), as_bf16x8(xh[v]), acc, 0, 0, 0);
        if (gemma)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wv[v]), as_bf16x8(xl[v]), acc, 0, 0, 0);
      }
    }
    // D: lane holds experts 4g..4g+3 of the tile for token l16.
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) s_part[wave][4 * g + ii][l16] = acc[ii];
    wsq += __shfl_xor(wsq, 16);
    wsq += __shfl_xor(wsq, 32);
    if (g == 0) s_wpart[wave][l16] = wsq;
    __syncthreads();
    {
      const int el = tid >> 4, tk = tid & 15;   // 256 threads = 16 experts × 16 tokens
      const int e = et * 16 + el;
      if (e < E) {
        float v = ((s_part[0][el][tk] + s_part[1][el][tk]) + s_part[2][el][tk]) + s_part[3][el][tk];
        if (a.router_b) v += bf16_bits_to_f32(a.router_b[e]);
        s_logit[tk][e] = v;
        if (tk == 0)
          s_wn[e] = sqrtf(((s_wpart[0][el] + s_wpart[1][el]) + s_wpart[2][el]) + s_wpart[3][el]);
      }
    }
    __syncthreads();
  }

  // ---- B: per token, candidates → exact logits → top-k ----
  const double root = gemma ? pow((double)H, -0.5) : 1.0;
  for (int tl = wave; tl < ntok; tl += 4) {
    const int t = t0 + tl;
    const uint16_t *xr = a.xr + (size_t)t * H;
    // ‖u‖ of the projection input (u = x, or x·scale for GEMMA) and Σx² for GEMMA's norm.
    double uu = 0.0, xx = 0.0;
    for (int h = lane * 8; h < H; h += 512) {
      const u32x4 xv = *(const u32x4 *)(xr + h);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const double xd = bf16_bits_to_f32((xv[k >> 1] >> ((k & 1) * 16)) & 0xFFFF);
        const double ud = gemma ? xd * (double)bf16_bits_to_f32(a.router_scale[h + k]) : xd;
        uu = fma(ud, ud, uu);
        xx = fma(xd, xd, xx);
      }
    }
    uu = wave_sum_f64(uu);
    xx = wave_sum_f64(xx);
    const double norm = gemma ? pow(xx / (double)H + (double)a.eps, -0.5) : 1.0;
    const double fscale = gemma ? norm * root : 1.0;   // logit = fscale · Σ u·w
    // |fp32 − exact| ≤ fscale·(2·H·2^-23·‖u‖‖w‖) + 2^-22·|logit| (bias add, final scaling).
    const float cb = (float)(fscale * 2.0 * H * 1.1920928955078125e-07 * sqrt(uu));
    // K-th largest lower bound.
    float lb[8], ub[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = lane + 64 * j;
      if (e < E) {
        const float l = (float)(fscale * (double)s_logit[tl][e]);
        const float err = cb * s_wn[e] + 2.384185791015625e-07f * fabsf(l) + 1e-30f;
        lb[j] = l - err;
        ub[j] = l + err;
      } else {
        lb[j] = -INFINITY;
        ub[j] = -INFINITY;
      }
    }
    uint32_t taken = 0;
    float theta = INFINITY;
    for (int r = 0; r < K; ++r) {
      float bv = -INFINITY;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = lane + 64 * j;
        if (e < E && !(taken & (1u << j)) && (lb[j] > bv || bi == 0x7FFFFFFF)) { bv = lb[j]; bi = e; }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
      theta = bv;
    }
    // Exact top-k over the candidates {e : ub_e ≥ θ}, processed in passes of ≤ 64.
    double sel_v[kMaxTopK];
    int sel_i[kMaxTopK];
    for (int r = 0; r < K; ++r) { sel_v[r] = -INFINITY; sel_i[r] = 0x7FFFFFFF; }
    int nsel = 0;
    for (int j = 0; j < 8; ++j) {
      const int e = lane + 64 * j;
      const bool is_c = (e < E) && (ub[j] >= theta);
      const uint64_t m = __ballot(is_c);
      const int nc = __popcll(m);
      if (is_c) s_cand[wave][__popcll(m & ((1ull << lane) - 1ull))] = e;
      __builtin_amdgcn_wave_barrier();
      for (int ci = 0; ci < nc; ++ci) {
        const int ce = s_cand[wave][ci];
        double v = exact_logit(a, xr, a.router_w + (size_t)ce * H, gemma, norm, root);
        if (a.router_b) v += (double)bf16_bits_to_f32(a.router_b[ce]);
        // Insert (v, ce) into the running top-k (descending, ties to the smaller index);
        // candidates arrive in ascending index order, so a tie never displaces an earlier one.
        if (nsel < K || v > sel_v[K - 1]) {
          int pos = min(nsel, K - 1);
          while (pos > 0 && v > sel_v[pos - 1]) {
            sel_v[pos] = sel_v[pos - 1];
            sel_i[pos] = sel_i[pos - 1];
            --pos;
          }
          sel_v[pos] = v;
          sel_i[pos] = ce;
          nsel = min(nsel + 1, K);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    double sg_logit = 0.0;
    if (a.shared_gate)
      sg_logit = exact_logit(a, a.x + (size_t)t * H, a.shared_gate, false, 1.0, 1.0);
    if (lane == 0) finish_token(a, t, sel_v, sel_i, sg_logit);
  }

}

// ---- small batches (T ≤ 16): every logit exactly in fp64, one wave per (token, expert) ----
__global__ __launch_bounds__(256) void logits64_kernel(RouteArgs a) {
  const int wave = threadIdx.x >> 6;
  const int E = a.experts, E1 = E + 1, H = a.hidden;
  const int p = blockIdx.x * 4 + wave;
  if (p >= a.tokens * E1) return;
  const int t = p / E1, e = p - t * E1;
  if (e == E && !a.shared_gate) return;
  const bool gemma = (a.router == R_GEMMA) && e < E;
  const uint16_t *xr = (e < E ? a.xr : a.x) + (size_t)t * H;
  double norm = 1.0, root = 1.0;
  if (gemma) {
    const int lane = threadIdx.x & 63;
    double xx = 0.0;
    for (int h = lane * 8; h < H; h += 512) {
      const u32x4 xv = *(const u32x4 *)(xr + h);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const double xd = bf16_bits_to_f32((xv[k >> 1] >> ((k & 1) * 16)) & 0xFFFF);
        xx = fma(xd, xd, xx);
      }
    }
    xx = wave_sum_f64(xx);
    norm = pow(xx / (double)H + (double)a.eps, -0.5);
    root = pow((double)H, -0.5);
  }
  const uint16_t *wrow = e < E ? a.router_w + (size_t)e * H : a.shared_gate;
  double v = exact_logit(a, xr, wrow, gemma, norm, root);
  if (e < E && a.router_b) v += (double)bf16_bits_to_f32(a.router_b[e]);
  if ((threadIdx.x & 63) == 0) a.lg64[(size_t)t * E1 + e] = v;
}

// Top-k of every token from the exact logits (one wave per token), then the dispatch.
__global__ __launch_bounds__(256) void select_kernel(RouteArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.experts, E1 = E + 1, K = a.top_k;
  for (int t = wave; t < a.tokens; t += 4) {
    const double *lg = a.lg64 + (size_t)t * E1;
    double v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < E ? lg[e] : -INFINITY;
    }
    uint32_t taken = 0;
    double sel_v[kMaxTopK];
    int sel_i[kMaxTopK];
    for (int r = 0; r < K; ++r) {
      double bv = -INFINITY;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = lane + 64 * j;
        if (e < E && !(taken & (1u << j)) && (v[j] > bv || bi == 0x7FFFFFFF)) { bv = v[j]; bi = e; }
      }
      // Larger value first, smaller index on ties (attention.metal:270, ReferenceOps.swift:174-176).
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const double ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
      sel_v[r] = bv;
      sel_i[r] = bi;
    }
    if (lane == 0) finish_token(a, t, sel_v, sel_i, a.shared_gate ? lg[E] : 0.0);
  }
  if (a.want_dispatch) {
    __syncthreads();
    dispatch_batch(a);
  }
}

__global__ __launch_bounds__(256) void dispatch_kernel(RouteArgs a) { dispatch_batch(a); }
}  // namespace hh

namespace hh {
// Router + top-k + dispatch: exact fp64 logits then one selecting workgroup when T ≤ 16;
// the MFMA-screened tiles then the dispatch workgroup otherwise.
hipError_t launch_route(const RouteArgs &a, hipStream_t s, Timing tm) {
  if (a.tokens <= RT_TOK) {
    const int pairs = a.tokens * (a.experts + 1);
    hipExtLaunchKernelGGL(logits64_kernel, dim3((pairs + 3) / 4), dim3(256), 0, s, tm.start,
                          nullptr, 0, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipExtLaunchKernelGGL(select_kernel, dim3(1), dim3(256), 0, s, nullptr, tm.stop, 0, a);
    return hipGetLastError();
  }
  const int tiles = (a.tokens + RT_TOK - 1) / RT_TOK;
  const bool second = a.want_dispatch != 0;
  hipExtLaunchKernelGGL(route_kernel, dim3(tiles), dim3(256), 0, s, tm.start,
                        second ? nullptr : tm.stop, 0, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !second) return e;
  hipExtLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(256), 0, s, nullptr, tm.stop, 0, a);
  return hipGetLastError();
}
// Stand-alone permutation of a given top-k table (hh_permute).
hipError_t launch_permute(const RouteArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(256), 0, s, a);
  return hipGetLastError();
}
}  // namespace hh
