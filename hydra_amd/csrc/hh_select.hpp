// hh_select.hpp — exact top-k selection and routing weights, shared by the router kernels and by
// the decode gate-up kernel (which selects redundantly in every workgroup instead of waiting for a
// separate selection launch).
//
// Reference: ReferenceOps.router (ReferenceOps.swift:173-183), QwenReferenceOps.router
// (QwenReferenceOps.swift:159-179), Gemma4ReferenceOps.router (Gemma4ReferenceOps.swift:131-156),
// router_topk (attention.metal:249-300: larger value first, smaller index on ties).
#pragma once
#include "hh_common.hpp"

namespace hh {

// Exclusive scan of data[0..n) in place (n ≤ 128·NW), 64·NW threads; returns the total.
template <int NW>
__device__ __forceinline__ int block_exclusive_scan(int *data, int n, int *s_wave) {
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
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    base += (w < wave) ? s_wave[w] : 0;
    total += s_wave[w];
  }
  int ex = base + inc - v;
  __syncthreads();
  if (2 * tid < n) data[2 * tid] = ex;
  if (2 * tid + 1 < n) data[2 * tid + 1] = ex + a0;
  __syncthreads();
  return total;
}

// Running exact top-k, descending, ties to the smaller index. Every lane of a wave holds the
// same copy.
struct TopK {
  double v[kMaxTopK];
  int i[kMaxTopK];
  __device__ TopK() {
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r) { v[r] = -INFINITY; i[r] = 0x7FFFFFFF; }
  }
  // One bubble pass with static indices (registers only). The carried entry (the new one,
  // then each displaced one) goes ahead of an entry with a smaller value, or an equal value and
  // a larger index.
  __device__ void insert(double x, int e, int K) {
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r) {
      if (r < K && (x > v[r] || (x == v[r] && e < i[r]))) {
        const double tv = v[r];
        const int ti = i[r];
        v[r] = x;
        i[r] = e;
        x = tv;
        e = ti;
      }
    }
  }
  // Index of rank r (r < kMaxTopK) read with a static index per case, so the arrays stay in
  // registers.
  __device__ int index_of(int r) const {
    int e = 0;
#pragma unroll
    for (int q = 0; q < kMaxTopK; ++q)
      if (q == r) e = i[q];
    return e;
  }
};

// SOFTMAX_TOPK_RENORM and GEMMA rank the experts by fp64 probability exp(l − max) / Σ, ties to
// the smaller index (QwenReferenceOps.swift:164-173, Gemma4ReferenceOps.swift:146-149). The
// probability is monotone in the logit, so it orders the experts as the logit does except where
// distinct logits give the same probability. Where exp(l − max) is 0 (l − max < −745.13: every
// such expert's probability is exactly 0), the reference takes the zero-probability experts by
// increasing index. tk holds the logit top-k; when its last ranks are of that class they are
// replaced by the smallest expert indices outside the non-zero ranks, with logit −∞ (weight 0,
// as the reference's 0 / Σ). Wave-uniform; a no-op unless the K-th logit is 700 below the first.
__device__ __forceinline__ void prob_order(TopK &tk, int K, int router) {
  if (router == R_TOPK_SOFTMAX) return;
  const double top = tk.v[0];
  bool low = false;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) low |= r < K && tk.v[r] - top < -700.0;
  if (!low) return;
  int nz = 0;   // ranks of non-zero probability form a prefix (monotone in the logit)
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r)
    if (r < K && exp(tk.v[r] - top) != 0.0) nz = r + 1;
  int e = 0;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r >= nz && r < K) {
      for (;;) {
        bool used = false;
#pragma unroll
        for (int q = 0; q < kMaxTopK; ++q) used |= q < nz && tk.i[q] == e;
        if (!used) break;
        ++e;
      }
      tk.i[r] = e++;
      tk.v[r] = -INFINITY;
    }
  }
}

// Top-k of one token from its exact logits lg[0..E) (E ≤ 512), whole wave: K rounds of a wave
// arg-max, larger value first and the smaller index on ties.
__device__ __forceinline__ TopK topk_exact(const double *lg, int E, int K) {
  const int lane = threadIdx.x & 63;
  double v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? lg[e] : -INFINITY;
  }
  TopK tk;
  uint32_t taken = 0;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r < K) {
      double bv = -INFINITY;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = lane + 64 * j;
        if (e < E && !(taken & (1u << j)) && (v[j] > bv || bi == 0x7FFFFFFF)) { bv = v[j]; bi = e; }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const double ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
      tk.v[r] = bv;
      tk.i[r] = bi;
    }
  }
  return tk;
}

// Rank counting split over groups of NW consecutive waves of a workgroup, each group selecting
// one token (every wave of a group with identical inputs): wave w counts its share of the
// comparisons, and the shares meet in s_part [waves][64]. Integer counts, so the sum does not
// depend on the split. Every wave of the workgroup must call it (barriers); the second barrier
// lets s_part be reused.
template <int NW>
__device__ __forceinline__ int coop_rank(int part, int (*s_part)[64]) {
  if constexpr (NW == 1) {
    return part;
  } else {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, w0 = w - w % NW;
    s_part[w][lane] = part;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) r += s_part[w0 + k][lane];
    __syncthreads();
    return r;
  }
}
// Range [j0, j1) of n comparisons that wave w of its group of NW takes.
template <int NW> __device__ __forceinline__ void coop_range(int n, int &j0, int &j1) {
  const int w = NW == 1 ? 0 : (int)(threadIdx.x >> 6) % NW;
  j0 = n * w / NW;
  j1 = n * (w + 1) / NW;
}

// The same selection for E ≤ 64 by rank counting: lane e holds logit e and counts the logits
// that precede it (larger, or equal with a smaller index) from a copy in the wave's LDS row
// s_lg[64]; the lanes of rank < K publish themselves in s_ri[8]. Independent LDS reads replace
// the K dependent shuffle chains of topk_exact (the decode critical path). NW > 1: the waves of
// the workgroup select this token together (coop_rank).
template <int NW = 1>
__device__ __forceinline__ TopK topk_rank64(const double *lg, int E, int K, double *s_lg, int *s_ri,
                                            int (*s_part)[64] = nullptr) {
  const int lane = threadIdx.x & 63;
  const double v = lane < E ? lg[lane] : -INFINITY;
  s_lg[lane] = v;
  __builtin_amdgcn_wave_barrier();
  int j0, j1;
  coop_range<NW>(E, j0, j1);
  int rank = 0;
#pragma unroll 8
  for (int j = j0; j < j1; ++j) {
    const double o = s_lg[j];
    rank += (o > v || (o == v && j < lane)) ? 1 : 0;
  }
  rank = coop_rank<NW>(rank, s_part);
  if (lane < E && rank < K) s_ri[rank] = lane;
  __builtin_amdgcn_wave_barrier();
  TopK tk;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r < K) {
      tk.i[r] = s_ri[r];
      tk.v[r] = s_lg[tk.i[r]];
    }
  }
  return tk;
}

// The value of lane l's v (wave-uniform l), without memory.
__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// The same selection for E ≤ 512 (one wave; lane l holds logits l, l + 64, ...) without K
// dependent rounds of shuffles. τ = the K-th largest of the 64 lane maxima bounds the K-th
// largest logit from below (the K lanes with the largest maxima hold K logits ≥ τ), so every
// selected logit is ≥ τ and a candidate's rank among the candidates {v ≥ τ} is its rank among
// all logits (a logit < τ is never ahead of one ≥ τ). Both rankings count the values ahead
// (larger, or equal with a smaller index) from registers by readlane, so ties resolve exactly as
// topk_exact's. s_ri / s_rv[kMaxTopK] and s_ci[kFastCand] / s_cv[kFastCand] are the wave's LDS
// scratch; more candidates than 64 (heavy ties) rank from LDS, more than kFastCand take
// topk_exact.
// NW > 1: groups of NW waves share the 64 lane maxima's ranking (one barrier pair for every
// group, whatever its token); NWC > 1 also splits the candidates' ranking, whose barrier count
// depends on the candidate count: only when every wave of the workgroup ranks the same token.
constexpr int kFastCand = 128;
template <int NW = 1, int NWC = NW>
__device__ __forceinline__ TopK topk_fast(const double *lg, int E, int K, int *s_ri, double *s_rv, int *s_ci,
                                          double *s_cv, int (*s_part)[64] = nullptr) {
  const int lane = threadIdx.x & 63;
  double v[8];
  double m = -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? lg[min(e, E - 1)] : -INFINITY;
    m = fmax(m, v[j]);
  }
  // τ: the lane maximum of rank K−1 among the 64 (ties by lane).
  int j0, j1;
  coop_range<NW>(64, j0, j1);
  int rank = 0;
  for (int j = j0; j < j1; ++j) {
    const double o = readlane_f64(m, j);
    rank += (o > m || (o == m && j < lane)) ? 1 : 0;
  }
  rank = coop_rank<NW>(rank, s_part);
  const uint64_t at_k = __ballot(rank == K - 1);
  const double tau = readlane_f64(m, __ffsll((unsigned long long)at_k) - 1);
  // Candidates v ≥ τ, compacted into LDS (lane-major within each j).
  int nc = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) nc += __popcll(__ballot(lane + 64 * j < E && v[j] >= tau));
  if (nc > kFastCand) return topk_exact(lg, E, K);
  nc = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = lane + 64 * j;
    const bool c = e < E && v[j] >= tau;
    const uint64_t bm = __ballot(c);
    if (c) {
      const int pos = nc + __popcll(bm & ((1ull << lane) - 1ull));
      s_ci[pos] = e;
      s_cv[pos] = v[j];
    }
    nc += __popcll(bm);
  }
  __builtin_amdgcn_wave_barrier();
  // Rank of each candidate among the candidates; ranks < K publish index and value.
  for (int c0 = 0; c0 < nc; c0 += 64) {
    const int ci = c0 + lane;
    const bool mine = ci < nc;
    const double cv = mine ? s_cv[ci] : 0.0;
    const int ce = mine ? s_ci[ci] : 0;
    int r = 0;
    int k0, k1;
    coop_range<NWC>(nc, k0, k1);
    if (nc <= 64) {
      for (int j = k0; j < k1; ++j) {
        const double o = readlane_f64(cv, j);
        const int oe = __builtin_amdgcn_readlane(ce, j);
        r += (o > cv || (o == cv && oe < ce)) ? 1 : 0;
      }
    } else {
      for (int j = k0; j < k1; ++j) {
        const double o = s_cv[j];
        const int oe = s_ci[j];
        r += (o > cv || (o == cv && oe < ce)) ? 1 : 0;
      }
    }
    r = coop_rank<NWC>(r, s_part);
    if (mine && r < K) {
      s_ri[r] = ce;
      s_rv[r] = cv;
    }
  }
  __builtin_amdgcn_wave_barrier();
  TopK tk;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r < K) {
      tk.i[r] = s_ri[r];
      tk.v[r] = s_rv[r];
    }
  }
  __builtin_amdgcn_wave_barrier();
  return tk;
}

// Routing weight of rank `lane` (lanes ≥ K: 0) of one token's selection (whole wave): tk holds
// the fp64 logits in rank order; `e` returns the lane's expert.
// TOPK_SOFTMAX: softmax over the k selected logits (ReferenceOps.swift:178-182).
// SOFTMAX_TOPK_RENORM and GEMMA: softmax over all experts, renormalised over the k
// (QwenReferenceOps.swift:159-179, Gemma4ReferenceOps.swift:146-155); the full-softmax
// denominator cancels, leaving the same softmax of the k selected logits. The sum runs in rank
// order.
__device__ __forceinline__ double token_weight(const RouteArgs &a, const TopK &tk, double &v, int &e) {
  const int K = a.top_k, lane = threadIdx.x & 63;
  v = -INFINITY;
  e = 0;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r)
    if (lane == r) { v = tk.v[r]; e = tk.i[r]; }
  double w = lane < K ? exp(v - tk.v[0]) : 0.0;
  double total = 0.0;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    const double wr = __shfl(w, r);
    if (r < K) total += wr;
  }
  w /= total;
  if (lane < K && a.router == R_GEMMA) w *= (double)bf16_bits_to_f32(a.router_pes[e]);
  return lane < K ? w : 0.0;
}

// Weights of one token's selection (whole wave; lane r < K handles rank r). Writes
// topk_idx/topk_w/slot_w (and logits, shared_w when given).
// COUNT (the selection kernels above 16 tokens): also add each assignment to the multi-block
// dispatch's count of its block (the decode kernels leave it out, which keeps their code as it is).
template <bool COUNT = false>
__device__ __forceinline__ void finish_token(const RouteArgs &a, int t, const TopK &tk, double sg_logit) {
  const int K = a.top_k, lane = threadIdx.x & 63;
  double v;
  int e;
  const double w = token_weight(a, tk, v, e);
  if (lane < K) {
    a.topk_idx[(size_t)t * K + lane] = e;
    if (a.topk_w) a.topk_w[(size_t)t * K + lane] = (float)w;
    a.slot_w[(size_t)t * a.slots + lane] = (float)w;
    if (a.logits) a.logits[(size_t)t * K + lane] = v;
    if (COUNT && a.dcount && a.want_dispatch) {
      // the multi-block dispatch's count of this assignment's block (integer adds: any order)
      const int A = a.tokens * K, i = t * K + lane;
      atomicAdd(&a.dcount[(size_t)(i / dispatch_range(A, dispatch_blocks(A))) * a.experts + e], 1);
    }
  }
  if (a.shared_gate && lane == 0) {
    // σ of the shared gate row, applied to the shared expert's output
    // (QwenReferenceLayer.swift:399-404).
    const double sg = 1.0 / (1.0 + exp(-sg_logit));
    a.slot_w[(size_t)t * a.slots + K] = (float)sg;
    if (a.shared_w) a.shared_w[t] = (float)sg;
  }
}

}  // namespace hh
