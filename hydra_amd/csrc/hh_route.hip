// hh_route.hip — router logits, top-k weights and token→expert dispatch.
//
// Selection is exact: top-k indices equal those of fp64 logits (the oracle's arithmetic).
//   A. Screening logits with v_mfma_f32_16x16x32_bf16 (exact bf16·bf16 products, fp32
//      accumulation) for 16-token × 16-expert tiles, plus each expert row's norm ‖w_e‖.
//   B. Per token (one wave): every fp32 logit lies within err = 2·H·2^-23·‖u‖·‖w_e‖ (+ the
//      rounding of the bias add and final scaling) of the exact one (recursive summation bound
//      with Cauchy-Schwarz). Experts whose upper bound reaches the K-th largest lower bound are
//      the only ones that can be in the exact top-k; their logits are recomputed in fp64 and
//      the top-k is selected among them with ties to the smaller index. Weights come from the
//      fp64 logits.
//   C. Dispatch: the batch's (token, rank) assignments grouped by expert, stable, plus the
//      work list of the expert products.
//
// Batches of at most 16 tokens skip the screening: logits_small_kernel computes every logit in
// fp64 (one wave per (token, expert) pair, spread over many compute units). In the layer, the
// decode gate-up kernel then selects from those logits itself (hh_select.hpp), so routing a
// decode step is one launch and needs no dispatch; the operator entry hh_router_topk runs
// select_small_kernel instead. Larger batches run A over a (token tile × expert tiles) grid
// (route_logits_kernel), B one workgroup per token below 1024 tokens (route_select_kernel) or one
// wave per token from there (route_select_wave_kernel), and C (dispatch_kernel, or the
// multi-block dispatch from 1024 assignments), ordered by the stream.
//
// Reference: router_topk / router_topk_batch (attention.metal:249, batch.metal:430),
// gemma_router_topk (gemma.metal:158), ReferenceOps.router (ReferenceOps.swift:173-183),
// QwenReferenceOps.router (:159-179), Gemma4ReferenceOps.router (:131-156),
// PrefillRunner.assignments (PrefillRunner.swift:224-246).
#include "hh_common.hpp"
#include "hh_select.hpp"
#include "hh_logit.hpp"
#include "hh_norm.hpp"

#include <mutex>

namespace hh {

// Development timeline (built only with -DHH_TRACE): wall-clock stamps (100 MHz) per workgroup of
// the small-batch router kernels and of route_select_kernel, [block][point], read as kernel 0 of
// the decode kernels' timeline.
#ifdef HH_TRACE
constexpr int kRtTraceBlocks = 4096, kRtTracePoints = 8;
static __device__ uint64_t hh_trace_rt[kRtTraceBlocks * kRtTracePoints];
#define HH_RT(point)                                                                               \
  do {                                                                                             \
    if ((threadIdx.x & 63) == 0 && blockIdx.x < kRtTraceBlocks)                                    \
      hh_trace_rt[blockIdx.x * kRtTracePoints + (point)] = wall_clock64();                         \
  } while (0)
hipError_t trace_read_route(void *out, size_t bytes) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(hh_trace_rt), std::min(bytes, sizeof(hh_trace_rt)), 0,
                             hipMemcpyDeviceToHost);
}
hipError_t trace_clear_route() {
  static uint64_t zeros[kRtTraceBlocks * kRtTracePoints];
  return hipMemcpyToSymbol(HIP_SYMBOL(hh_trace_rt), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
// Point 7 of route_select_kernel's rows: the token's candidate count.
#define HH_RT_NC(nc)                                                                               \
  do {                                                                                             \
    if (threadIdx.x == 0 && blockIdx.x < kRtTraceBlocks) hh_trace_rt[blockIdx.x * kRtTracePoints + 7] = (uint64_t)(nc); \
  } while (0)
// The dispatch workgroup's stamps: row kRtTraceBlocks − 1, wave 0.
#define HH_DS(point)                                                                               \
  do {                                                                                             \
    if (threadIdx.x == 0) hh_trace_rt[(kRtTraceBlocks - 1) * kRtTracePoints + (point)] = wall_clock64(); \
  } while (0)
#else
#define HH_DS(point) do {} while (0)
#define HH_RT(point) do {} while (0)
#define HH_RT_NC(nc) do {} while (0)
#endif

// Stable token→expert permutation of the whole batch by one workgroup of NW waves; `idx` is
// the top-k table [T][K] (global or LDS). Wave w owns the contiguous assignment range
// [w·R, (w+1)·R): pass 1 counts its assignments per expert, a scan over (expert, wave) gives every
// wave its first position inside each expert's segment, pass 2 writes the positions (a lane's rank
// among the earlier lanes of its 64-assignment chunk with the same expert, found by ballots over
// the expert id's bits, plus the wave's running count). Two barriers in all, and (t, r) order is
// kept inside each expert.
template <int NW>
__device__ __forceinline__ void dispatch_batch(const RouteArgs &a, const int32_t *idx) {
  constexpr int NT = 64 * NW;
  __shared__ int s_cnt[kMaxExperts + 1];
  __shared__ int s_off[kMaxExperts + 1];
  __shared__ int s_tiles[kMaxExperts + 1];
  __shared__ int s_wc[NW][kMaxExperts];   // pass 1: count per (wave, expert); then running position
  __shared__ int s_wave[NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = a.experts, K = a.top_k, T = a.tokens, A = T * K;
  const int TN = a.tile_tokens;
  const int R = ((A + NW - 1) / NW + 63) & ~63;     // assignments per wave, whole chunks
  const int lo = min(wave * R, A), hi = min(lo + R, A);
  HH_DS(0);
  for (int e = tid; e < NW * kMaxExperts; e += NT) (&s_wc[0][0])[e] = 0;
  __syncthreads();
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
  // Peers of the lane's assignment inside its chunk (same expert), as a lane mask.
  auto peers_of = [&](bool valid, int e) {
    uint64_t peers = __ballot(valid);
    for (int bb = 0; bb < nbits; ++bb) {
      const uint64_t m = __ballot(valid && ((e >> bb) & 1));
      peers &= ((e >> bb) & 1) ? m : ~m;
    }
    return peers;
  };
  // The wave's expert ids are read DCH chunks at a time, all loads issued before the first is
  // used (one memory latency per DCH chunks, not per chunk).
  constexpr int DCH = 16;
  int ev[DCH];
  auto load_ids = [&](int b0) {
#pragma unroll
    for (int k = 0; k < DCH; ++k) {
      const int i = b0 + 64 * k + lane;
      ev[k] = i < hi ? idx[i] : 0;
    }
  };
  for (int b0 = lo; b0 < hi; b0 += 64 * DCH) {
    load_ids(b0);
#pragma unroll
    for (int k = 0; k < DCH; ++k) {
      const int base = b0 + 64 * k;
      if (base >= hi) break;
      const bool valid = base + lane < hi;
      const int e = ev[k];
      const uint64_t peers = peers_of(valid, e);
      if (valid && __popcll(peers & ((1ull << lane) - 1ull)) == 0) s_wc[wave][e] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  }
  HH_DS(1);
  __syncthreads();
  HH_DS(2);
  // Per expert: total count, and each wave's first position relative to the expert's segment.
  for (int e = tid; e < E; e += NT) {
    int run = 0;
    for (int w = 0; w < NW; ++w) {
      const int c = s_wc[w][e];
      s_wc[w][e] = run;
      run += c;
    }
    s_cnt[e] = run;
    s_off[e] = run;
    s_tiles[e] = (run + TN - 1) / TN;
  }
  __syncthreads();
  block_exclusive_scan<NW>(s_off, E, s_wave);
  const int routed_tiles = block_exclusive_scan<NW>(s_tiles, E, s_wave);
  HH_DS(3);
  for (int b0 = lo; b0 < hi; b0 += 64 * DCH) {
    load_ids(b0);
#pragma unroll
    for (int k = 0; k < DCH; ++k) {
      const int base = b0 + 64 * k;
      if (base >= hi) break;
      const int i = base + lane;
      const bool valid = i < hi;
      const int e = ev[k];
      const uint64_t peers = peers_of(valid, e);
      const int rank = __popcll(peers & ((1ull << lane) - 1ull));
      if (valid) {
        const int t = i / K, r = i - t * K;
        a.order[s_off[e] + s_wc[wave][e] + rank] = t * a.slots + r;
      }
      __builtin_amdgcn_wave_barrier();
      if (valid && rank == 0) s_wc[wave][e] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  }
  HH_DS(4);
  __syncthreads();
  HH_DS(5);
  // Segments and work items (expert, first position, tokens), ascending expert order.
  for (int e = tid; e < E; e += NT) {
    a.seg[e] = s_off[e];
    const int n = s_cnt[e];
    for (int j = 0; j * TN < n; ++j)
      a.work[s_tiles[e] + j] = make_int4(e, s_off[e] + j * TN, min(TN, n - j * TN), 0);
  }
  if (a.work_half) {
    // The same segments in items of TN / 2 tokens (the list's users have no shared expert).
    const int TH = TN / 2;
    __syncthreads();   // s_tiles was read above
    for (int e = tid; e < E; e += NT) s_tiles[e] = (s_cnt[e] + TH - 1) / TH;
    __syncthreads();
    const int half_tiles = block_exclusive_scan<NW>(s_tiles, E, s_wave);
    for (int e = tid; e < E; e += NT) {
      const int n = s_cnt[e];
      for (int j = 0; j * TH < n; ++j)
        a.work_half[s_tiles[e] + j] = make_int4(e, s_off[e] + j * TH, min(TH, n - j * TH), 0);
    }
    if (tid == 0) *a.n_work_half = half_tiles;
  }
  int nwork = routed_tiles;
  if (a.shared_gate) {
    // The shared expert is expert id E over every token, after the routed positions.
    for (int t = tid; t < T; t += NT) a.order[A + t] = t * a.slots + K;
    const int st = (T + TN - 1) / TN;
    for (int j = tid; j < st; j += NT)
      a.work[routed_tiles + j] = make_int4(E, A + j * TN, min(TN, T - j * TN), 0);
    nwork += st;
    if (tid == 0) { a.seg[E] = A; a.seg[E + 1] = A + T; }
  } else if (tid == 0) {
    a.seg[E] = A;
    a.seg[E + 1] = A;
  }
  if (tid == 0) *a.n_work = nwork;
  HH_DS(6);
}


// ---- multi-block dispatch (large batches) ---------------------------------------------------------
// The same stable grouping as dispatch_batch over DB_MAX or fewer 256-thread workgroups, in two
// launches: dispatch_count_kernel writes each block's per-expert counts, dispatch_scatter_kernel
// gives every block its first position inside each expert's segment (the segments of all experts
// before it, plus the same expert's counts of the earlier blocks) and writes its assignments'
// positions in (t, r) order, as dispatch_batch does within one workgroup. Every block also forms
// the segment offsets and the work lists' tile offsets and writes the items of the experts
// e ≡ block (mod blocks); block 0 writes the segment table and the item counts. A single
// 1024-thread workgroup was bound by its compute unit's issue rate (≈ 80 instructions per 64
// assignments per pass on 16 waves sharing 4 SIMDs).

__global__ __launch_bounds__(256) void dispatch_count_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  __shared__ int s_c[kMaxExperts];
  const int tid = threadIdx.x, E = a.experts, A = a.tokens * a.top_k;
  const int R = dispatch_range(A, gridDim.x), lo = blockIdx.x * R, hi = min(lo + R, A);
  for (int e = tid; e < E; e += 256) s_c[e] = 0;
  __syncthreads();
  for (int i = lo + tid; i < hi; i += 256) atomicAdd(&s_c[a.topk_idx[i]], 1);
  __syncthreads();
  for (int e = tid; e < E; e += 256) a.dcount[(size_t)blockIdx.x * E + e] = s_c[e];
}

__global__ __launch_bounds__(256) void dispatch_scatter_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  constexpr int NW = 4;
  __shared__ int s_off[kMaxExperts];      // segment offsets (exclusive scan of the totals)
  __shared__ int s_tot[kMaxExperts];
  __shared__ int s_tiles[kMaxExperts];
  __shared__ int s_wc[NW][kMaxExperts];   // per wave: count, then running position
  __shared__ int s_wave[NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = a.experts, K = a.top_k, T = a.tokens, A = T * K, TN = a.tile_tokens;
  const int NB = gridDim.x, b = blockIdx.x;
  const int R = dispatch_range(A, NB), blo = b * R, bhi = min(blo + R, A);
  const int RW = R / NW, lo = min(blo + wave * RW, bhi), hi = min(lo + RW, bhi);
  // Totals, and this block's first position per expert relative to the expert's segment.
  int pre[2] = {0, 0};
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e = tid + 256 * k;
    if (e < E) {
      int c[DB_MAX];   // every block's count in one round of loads
#pragma unroll
      for (int bb = 0; bb < DB_MAX; ++bb) c[bb] = bb < NB ? a.dcount[(size_t)bb * E + e] : 0;
      int p = 0, t = 0;
#pragma unroll
      for (int bb = 0; bb < DB_MAX; ++bb) {
        p += bb < b ? c[bb] : 0;
        t += c[bb];
      }
      pre[k] = p;
      s_tot[e] = t;
      s_off[e] = t;
    }
  }
  for (int e = tid; e < NW * kMaxExperts; e += 256) (&s_wc[0][0])[e] = 0;
  __syncthreads();
  block_exclusive_scan<NW>(s_off, E, s_wave);
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 1;
  auto peers_of = [&](bool valid, int e) {
    uint64_t peers = __ballot(valid);
    for (int bb = 0; bb < nbits; ++bb) {
      const uint64_t m = __ballot(valid && ((e >> bb) & 1));
      peers &= ((e >> bb) & 1) ? m : ~m;
    }
    return peers;
  };
  constexpr int DCH = 8;
  int ev[DCH];
  auto load_ids = [&](int b0) {
#pragma unroll
    for (int k = 0; k < DCH; ++k) {
      const int i = b0 + 64 * k + lane;
      ev[k] = i < hi ? a.topk_idx[i] : 0;
    }
  };
  // Pass 1: the wave's count per expert.
  for (int b0 = lo; b0 < hi; b0 += 64 * DCH) {
    load_ids(b0);
#pragma unroll
    for (int k = 0; k < DCH; ++k) {
      const int base = b0 + 64 * k;
      if (base >= hi) break;
      const bool valid = base + lane < hi;
      const int e = ev[k];
      const uint64_t peers = peers_of(valid, e);
      if (valid && __popcll(peers & ((1ull << lane) - 1ull)) == 0) s_wc[wave][e] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();
  // Each wave's first position per expert: segment offset + earlier blocks + earlier waves.
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e = tid + 256 * k;
    if (e < E) {
      int run = s_off[e] + pre[k];
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const int c = s_wc[w][e];
        s_wc[w][e] = run;
        run += c;
      }
    }
  }
  __syncthreads();
  // Pass 2: positions.
  for (int b0 = lo; b0 < hi; b0 += 64 * DCH) {
    load_ids(b0);
#pragma unroll
    for (int k = 0; k < DCH; ++k) {
      const int base = b0 + 64 * k;
      if (base >= hi) break;
      const int i = base + lane;
      const bool valid = i < hi;
      const int e = ev[k];
      const uint64_t peers = peers_of(valid, e);
      const int rank = __popcll(peers & ((1ull << lane) - 1ull));
      if (valid) {
        const int t = i / K, r = i - t * K;
        a.order[s_wc[wave][e] + rank] = t * a.slots + r;
      }
      __builtin_amdgcn_wave_barrier();
      if (valid && rank == 0) s_wc[wave][e] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  }
  // Work items (expert, first position, tokens) in ascending expert order; this block writes the
  // items of the experts e ≡ b (mod NB).
  for (int e = tid; e < E; e += 256) s_tiles[e] = (s_tot[e] + TN - 1) / TN;
  __syncthreads();
  const int routed_tiles = block_exclusive_scan<NW>(s_tiles, E, s_wave);
  for (int e = b + NB * tid; e < E; e += NB * 256) {
    const int n = s_tot[e];
    for (int j = 0; j * TN < n; ++j) a.work[s_tiles[e] + j] = make_int4(e, s_off[e] + j * TN, min(TN, n - j * TN), 0);
  }
  if (a.work_half) {
    const int TH = TN / 2;
    __syncthreads();   // s_tiles was read above
    for (int e = tid; e < E; e += 256) s_tiles[e] = (s_tot[e] + TH - 1) / TH;
    __syncthreads();
    const int half_tiles = block_exclusive_scan<NW>(s_tiles, E, s_wave);
    for (int e = b + NB * tid; e < E; e += NB * 256) {
      const int n = s_tot[e];
      for (int j = 0; j * TH < n; ++j)
        a.work_half[s_tiles[e] + j] = make_int4(e, s_off[e] + j * TH, min(TH, n - j * TH), 0);
    }
    if (b == 0 && tid == 0) *a.n_work_half = half_tiles;
  }
  int nwork = routed_tiles;
  if (a.shared_gate) {
    // The shared expert is expert id E over every token, after the routed positions.
    for (int t = b * 256 + tid; t < T; t += NB * 256) a.order[A + t] = t * a.slots + K;
    const int st = (T + TN - 1) / TN;
    for (int j = b * 256 + tid; j < st; j += NB * 256)
      a.work[routed_tiles + j] = make_int4(E, A + j * TN, min(TN, T - j * TN), 0);
    nwork += st;
    if (b == 0 && tid == 0) { a.seg[E] = A; a.seg[E + 1] = A + T; }
  } else if (b == 0 && tid == 0) {
    a.seg[E] = A;
    a.seg[E + 1] = A;
  }
  if (b == 0) {
    for (int e = tid; e < E; e += 256) a.seg[e] = s_off[e];
    if (tid == 0) *a.n_work = nwork;
  }
}

constexpr int RT_TOK = 16;          // tokens per route workgroup
constexpr int RT_MAXCAND = 64;      // exact-recompute candidates handled per pass

// Projection input of the router from 8 columns of a token row (xv) and of the GEMMA scale
// (sv): GEMMA uses u = x·scale split exactly into bf16 hi + lo (x·scale has at most 16
// significant bits); the other routers use x itself (lo = 0).
__device__ __forceinline__ void router_operand(bool gemma, const u32x4 &xv, const u32x4 &sv,
                                               u32x4 &hi, u32x4 &lo) {
  if (!gemma) {
    hi = xv;
    lo = u32x4{0u, 0u, 0u, 0u};
    return;
  }
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

// Screening result of one token: candidate count and the GEMMA normaliser of its input.
struct TokenScreen {
  int nc = 0;
  double norm = 1.0;
};

// Screens token t (one wave): bounds every fp32 logit lgf(e) by err_e, θ = the K-th largest
// lower bound, and writes the candidates {e : ub_e ≥ θ} to cl[] in ascending order.
// NW > 1: groups of NW consecutive waves of the workgroup each screen one token together
// (identical results in every wave of a group); the 64-lane ranking splits over a group's waves
// through s_rk [waves][64]. Every wave of the workgroup calls it (one barrier).
template <bool gemma, int NW = 1, class LG, class WN>
__device__ __forceinline__ TokenScreen screen_token(const RouteArgs &a, int t, LG lgf, WN wnf, int *cl,
                                                    int (*s_rk)[64] = nullptr, double coef = -1.0) {
  const int lane = threadIdx.x & 63;
  const int E = a.experts, H = a.hidden, K = a.top_k;
  const uint16_t *xr = a.xr + (size_t)t * H;
  // ‖u‖ of the projection input (u = x, or x·scale for GEMMA) and Σx² for GEMMA's norm.
  double uu = 0.0, xx = 0.0;
  for (int base = 0; base < H; base += 2048) {
    u32x4 xv[4], sv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int h = base + lane * 8 + 512 * u;
      const int hc = min(h, H - 8);
      xv[u] = *(const u32x4 *)(xr + hc);
      sv[u] = gemma ? *(const u32x4 *)(a.router_scale + hc) : u32x4{0u, 0u, 0u, 0u};
      if (h >= H) xv[u] = u32x4{0u, 0u, 0u, 0u};
    }
    // x² and (x·scale) are exact in fp32; partial sums per step in fp32 are not, so they
    // are kept per element pair in fp64 (the sums only feed an error bound and GEMMA's norm).
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      double pu = 0.0, px = 0.0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int sh = (k & 1) * 16;
        const float xf = bf16_bits_to_f32((xv[u][k >> 1] >> sh) & 0xFFFF);
        px += (double)(xf * xf);
        if constexpr (gemma) {
          const double ud = (double)(xf * bf16_bits_to_f32((sv[u][k >> 1] >> sh) & 0xFFFF));
          pu = fma(ud, ud, pu);
        }
      }
      xx += px;
      uu += gemma ? pu : px;
    }
  }
  uu = wave_sum_f64(uu);
  xx = wave_sum_f64(xx);
  TokenScreen ts;
  ts.norm = gemma ? pow(xx / (double)H + (double)a.eps, -0.5) : 1.0;
  const double fscale = gemma ? ts.norm * pow((double)H, -0.5) : 1.0;   // logit = fscale·Σu·w
  // |fp32 − exact| ≤ fscale·(2·H·2^-23·‖u‖‖w‖) + 2^-22·|logit| (bias add, final scaling); a
  // screen with another bound passes its coefficient of ‖u‖·wnf(e) (`coef`).
  const float cb = (float)(fscale * (coef > 0.0 ? coef : 2.0 * H * 1.1920928955078125e-07) * sqrt(uu));
  float lb[8], ub[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = lane + 64 * j;
    if (e < E) {
      const float l = (float)(fscale * (double)lgf(e));
      const float err = cb * wnf(e) + 2.384185791015625e-07f * fabsf(l) + 1e-30f;
      lb[j] = l - err;
      ub[j] = l + err;
    } else {
      lb[j] = -INFINITY;
      ub[j] = -INFINITY;
    }
  }
  // θ = the K-th largest lower bound. τ = the K-th largest of the 64 lane maxima is ≤ θ (the K
  // lanes with the largest maxima hold K bounds ≥ τ), so θ is the K-th largest of the bounds ≥ τ,
  // ranked (larger, or equal and earlier) by readlane from lanes; cl[] is the scratch.
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j) mx = fmaxf(mx, lb[j]);
  int rk = 0;
  {
    const int j0 = NW > 1 ? (64 / NW) * ((int)(threadIdx.x >> 6) % NW) : 0;
#pragma unroll 4
    for (int jj = 0; jj < 64 / NW; ++jj) {
      const int j = j0 + jj;
      const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx), j));
      rk += (o > mx || (o == mx && j < lane)) ? 1 : 0;
    }
  }
  if constexpr (NW > 1) {
    const int w0 = (int)(threadIdx.x >> 6) - (int)(threadIdx.x >> 6) % NW;   // the group's first wave
    s_rk[threadIdx.x >> 6][lane] = rk;
    __syncthreads();
    rk = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) rk += s_rk[w0 + w][lane];
  }
  const float tau = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx), __ffsll((unsigned long long)__ballot(rk == K - 1)) - 1));
  int nq = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool q = lane + 64 * j < E && lb[j] >= tau;
    const uint64_t bm = __ballot(q);
    if (q) cl[nq + __popcll(bm & ((1ull << lane) - 1ull))] = __builtin_bit_cast(int, lb[j]);
    nq += __popcll(bm);
  }
  __builtin_amdgcn_wave_barrier();
  float theta = -INFINITY;
  for (int c0 = 0; c0 < nq; c0 += 64) {
    const int ci = c0 + lane;
    const float cv = ci < nq ? __builtin_bit_cast(float, cl[ci]) : -INFINITY;
    int r = 0;
    if (nq <= 64) {
      for (int j = 0; j < nq; ++j) {
        const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), j));
        r += (o > cv || (o == cv && j < ci)) ? 1 : 0;
      }
    } else {
      for (int j = 0; j < nq; ++j) {
        const float o = __builtin_bit_cast(float, cl[j]);
        r += (o > cv || (o == cv && j < ci)) ? 1 : 0;
      }
    }
    const uint64_t hit = __ballot(ci < nq && r == K - 1);
    if (hit) theta = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), __ffsll((unsigned long long)hit) - 1));
  }
  __builtin_amdgcn_wave_barrier();
  int nc = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = lane + 64 * j;
    const bool is_c = (e < E) && (ub[j] >= theta);
    const uint64_t m = __ballot(is_c);
    if (is_c) cl[nc + __popcll(m & ((1ull << lane) - 1ull))] = e;
    nc += __popcll(m);
  }
  __builtin_amdgcn_wave_barrier();
  ts.nc = nc;
  return ts;
}

// ---- x as fp8 terms (MXFP4 layers) ----------------------------------------------------------------
// One wave quantises 16 blocks of 32 columns of token t (quant_block): lane (g, l16) takes block
// blk0 + l16, columns 8g .. 8g+7 of it.
__device__ __forceinline__ void quant_x_wave(const RouteArgs &a, int t, int blk0) {
  const int lane = threadIdx.x & 63, g = lane >> 4, l16 = lane & 15;
  const int H = a.hidden, nb = H / 32;
  const int b = blk0 + l16, bc = min(b, nb - 1);
  const u32x4 xv = *(const u32x4 *)(a.x + (size_t)t * H + bc * 32 + 8 * g);
  float v[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[2 * k] = bf_lo(xv[k]);
    v[2 * k + 1] = bf_hi(xv[k]);
  }
  uint32_t q[NTX][2], sb[NTX];
  quant_block<NTX>(v, q, sb);
  if (b < nb) {
#pragma unroll
    for (int j = 0; j < NTX; ++j) {
      *(u32x2 *)(a.xq + ((size_t)t * NTX + j) * a.xld + b * 32 + 8 * g) = u32x2{q[j][0], q[j][1]};
      if (g == 0) a.xs[((size_t)t * NTX + j) * (a.xld / 32) + b] = (uint8_t)sb[j];
    }
  }
}

__device__ __forceinline__ int quant_x_waves(const RouteArgs &a) {
  return a.xq ? a.tokens * ((a.hidden / 32 + 15) / 16) : 0;
}

// ---- large batches ---------------------------------------------------------------------------
// Zeroes the multi-block dispatch's count buffer (the selection launch that follows adds to it);
// every workgroup of the calling launch takes a slice.
__device__ __forceinline__ void zero_dispatch_counts(const RouteArgs &a) {
  if (!a.dcount || !a.want_dispatch) return;
  const int n = DB_MAX * a.experts;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) a.dcount[i] = 0;
}

// A: the screening logits lg32 [T][E] on the bf16 MFMA and, from the first token tile, ‖w_e‖
// (the diagonal of W·Wᵀ, accumulated in fp32 like the logits: its relative error ≤ H·2^-24 is
// far inside the factor 4 of slack the screening bound carries). One workgroup per (16-token
// tile, RET consecutive 16-expert tiles), its RLW2 waves splitting K (chunks c ≡ wave mod RLW2;
// lane (g, l16) supplies router row l16 of a tile and token l16 at columns 128c + 32g + 8v). A
// chunk's token operand (GEMMA: the bf16 hi/lo split of x·scale) is loaded and formed once for
// the RET expert tiles. Any order of the fp32 sums lies inside the screening bound. Workgroups
// past the tiles quantise x (MXFP4 layers), one wave per 16 blocks of a token.
constexpr int RLW2 = 8;
template <bool gemma, int RET>
__global__ __launch_bounds__(64 * RLW2) void route_logits_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  zero_dispatch_counts(a);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, l16 = lane & 15;
  const int E = a.experts, T = a.tokens, H = a.hidden;
  const int ntiles = (E + 15) / 16, ngr = (ntiles + RET - 1) / RET;
  const int nlog = ((T + RT_TOK - 1) / RT_TOK) * ngr;
  if ((int)blockIdx.x >= nlog) {
    const int w = ((int)blockIdx.x - nlog) * RLW2 + wave;
    const int per_t = (H / 32 + 15) / 16;
    if (w < quant_x_waves(a)) quant_x_wave(a, w / per_t, 16 * (w % per_t));
    return;
  }
  const int tt = blockIdx.x / ngr, eg = blockIdx.x - tt * ngr;
  const int t0 = tt * RT_TOK, ntok = min(RT_TOK, T - t0);
  const bool want_wn = tt == 0;
  const uint16_t *xr = a.xr + (size_t)(t0 + min(l16, ntok - 1)) * H;
  const uint16_t *wrow[RET];
#pragma unroll
  for (int j = 0; j < RET; ++j) wrow[j] = a.router_w + (size_t)min((eg * RET + j) * 16 + l16, E - 1) * H;
  f32x4 acc[RET], wacc[RET];
#pragma unroll
  for (int j = 0; j < RET; ++j) acc[j] = wacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nch = (H + 127) / 128;
  struct Chunk {
    u32x4 xv[4], sv[4], wv[RET][4];
  };
  // Chunk c's operands (columns past H: clamped loads, zero weights).
  auto load = [&](Chunk &k, int c) {
    const int cc = min(c, nch - 1);
    const int col = min(128 * cc + 32 * g, H - 32);
    const bool ok = 128 * cc + 32 * g < H;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      k.xv[v] = *(const u32x4 *)(xr + col + 8 * v);
      k.sv[v] = gemma ? *(const u32x4 *)(a.router_scale + col + 8 * v) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < RET; ++j) {
        k.wv[j][v] = *(const u32x4 *)(wrow[j] + col + 8 * v);
        if (!ok) k.wv[j][v] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto add = [&](const Chunk &k) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      u32x4 xh, xl;
      router_operand(gemma, k.xv[v], k.sv[v], xh, xl);
#pragma unroll
      for (int j = 0; j < RET; ++j) {
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(k.wv[j][v]), as_bf16x8(xh), acc[j], 0, 0, 0);
        if constexpr (gemma)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(k.wv[j][v]), as_bf16x8(xl), acc[j], 0, 0, 0);
        if (want_wn)
          wacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(k.wv[j][v]), as_bf16x8(k.wv[j][v]), wacc[j], 0, 0, 0);
      }
    }
  };
  for (int c = wave; c < nch; c += RLW2) {
    Chunk k;
    load(k, c);
    add(k);
  }
  __shared__ float s_part[RLW2][RET][16][16];   // [wave][tile][expert in tile][token]
  __shared__ float s_wpart[RLW2][RET][16];
#pragma unroll
  for (int j = 0; j < RET; ++j) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) s_part[wave][j][4 * g + ii][l16] = acc[j][ii];
    // Σw² of row l16 is the diagonal of W·Wᵀ: lane (g = l16 / 4, l16), element l16 % 4.
    if (want_wn && g == (l16 >> 2)) s_wpart[wave][j][l16] = wacc[j][l16 & 3];
  }
  __syncthreads();
  auto wsum = [&](auto get) {
    float p[RLW2];
#pragma unroll
    for (int w = 0; w < RLW2; ++w) p[w] = get(w);
#pragma unroll
    for (int h = 1; h < RLW2; h *= 2)
#pragma unroll
      for (int w = 0; w + h < RLW2; w += 2 * h) p[w] += p[w + h];
    return p[0];
  };
  for (int q = tid; q < RET * 256; q += 64 * RLW2) {
    const int j = q >> 8, el = (q >> 4) & 15, tk = q & 15;
    const int e = (eg * RET + j) * 16 + el;
    if (e < E && tk < ntok) {
      float v = wsum([&](int w) { return s_part[w][j][el][tk]; });
      if (a.router_b) v += bf16_bits_to_f32(a.router_b[e]);
      a.lg32[(size_t)(t0 + tk) * E + e] = v;
      if (want_wn && tk == 0) a.wn[e] = sqrtf(wsum([&](int w) { return s_wpart[w][j][el]; }));
    }
  }
}
// Expert tiles per workgroup of route_logits_kernel: the most (up to 4) that still leave
// 256 logit workgroups.
static int wide_ret(int T, int E) {
  const int tt = (T + RT_TOK - 1) / RT_TOK, nt = (E + 15) / 16;
  for (int r : {4, 2})
    if (tt * ((nt + r - 1) / r) >= 256) return r;
  return 1;
}
template <bool gemma> static void *wide_logits_fn(int ret) {
  return ret == 4 ? (void *)route_logits_kernel<gemma, 4>
                  : ret == 2 ? (void *)route_logits_kernel<gemma, 2> : (void *)route_logits_kernel<gemma, 1>;
}

// B: one workgroup per token. Its 4 waves screen the token together, then wave w computes the
// exact logits of candidates w, w + 4, ... (each row in exact_logits_rows' arithmetic, so the
// values do not depend on how rows are grouped) and wave 1 the shared gate's; wave 0 ranks them
// (TopK's order: larger value, then smaller index, whatever the insertion order) and writes the
// token's routing.


// The GEMMA variant took 129 VGPRs, three workgroups per compute unit; at most 128 gives four
// (five spills).
template <bool gemma>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(gemma ? 4 : 5))) void route_select_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x;
  __shared__ int s_cl[4][kMaxExperts];
  __shared__ int s_rk[4][64];
  __shared__ double s_v[kMaxExperts];
  __shared__ double s_sg;
  const float *lg = a.lg32 + (size_t)t * a.experts;
  const float *wn = a.wn;
  if (wave == 0) HH_RT(0);
  const TokenScreen ts = screen_token<gemma, 4>(a, t, [&](int e) { return lg[e]; },
                                                [&](int e) { return wn[e]; }, s_cl[wave], s_rk);
  if (wave == 0) HH_RT(1);
  HH_RT_NC(ts.nc);
  const double root = gemma ? pow((double)a.hidden, -0.5) : 1.0;
  const uint16_t *xr = a.xr + (size_t)t * a.hidden;
  for (int c = wave; c < ts.nc; c += 4) {
    const int e = s_cl[wave][c];
    const uint16_t *rows[1] = {a.router_w + (size_t)e * a.hidden};
    double v[1];
    exact_logits_rows<gemma, 1>(a, xr, rows, ts.norm, root, v);
    if (a.router_b) v[0] += (double)bf16_bits_to_f32(a.router_b[e]);
    if (lane == 0) s_v[c] = v[0];
  }
  if (wave == 1 && a.shared_gate) {
    const double sg = exact_logit<false>(a, a.x + (size_t)t * a.hidden, a.shared_gate, 1.0, 1.0);
    if (lane == 0) s_sg = sg;
  }
  if (wave == 0) HH_RT(2);
  __syncthreads();
  if (wave == 0) HH_RT(3);
  if (wave != 0) return;
  TopK tk;
  for (int c = 0; c < ts.nc; ++c) tk.insert(s_v[c], s_cl[0][c], a.top_k);
  prob_order(tk, a.top_k, a.router);
  finish_token<true>(a, t, tk, a.shared_gate ? s_sg : 0.0);
}

// B for batches of at least kSelWaveT tokens: one wave per token, four tokens per workgroup, so
// that every token's wave is resident at once (2048 tokens are two waves per SIMD) where the
// four-wave form above ran in rounds of workgroups. The wave screens its token alone
// (screen_token, NW = 1: the same bounds and candidates), computes the candidates' exact
// logits sel_rows() rows at a time (exact_logits_rows: each row's arithmetic is the one-row form's,
// so the same values) and the shared gate's, then ranks them and writes the token's routing:
// the same routing as route_select_kernel's.
constexpr int kSelWaveT = 1024;
// Candidate rows per batch: GEMMA's top-8 screens ≈ 9 candidates, in batches of 4 (5 and 6 were
// slower: 49.5 / 52 against 46 µs at T=2048); the top-4 routers ≈ 4.3, mostly one batch of 5
// (27.4 → 25.2 µs on the 120B layer at T=2048).
template <bool gemma> constexpr int sel_rows() { return gemma ? 4 : 5; }
template <bool gemma>
__global__ __launch_bounds__(256) void route_select_wave_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  __shared__ int s_cl[4][kMaxExperts];
  __shared__ double s_v[4][kMaxExperts];
  if (t >= a.tokens) return;
  if (wave == 0) HH_RT(0);
  const int H = a.hidden;
  const float *lg = a.lg32 + (size_t)t * a.experts;
  const float *wn = a.wn;
  int *cl = s_cl[wave];
  const TokenScreen ts = screen_token<gemma, 1>(a, t, [&](int e) { return lg[e]; }, [&](int e) { return wn[e]; }, cl);
  if (wave == 0) HH_RT(1);
  if (wave == 0) HH_RT_NC(ts.nc);
  const double root = gemma ? pow((double)H, -0.5) : 1.0;
  const uint16_t *xr = a.xr + (size_t)t * H;
  constexpr int RSEL = sel_rows<gemma>();
  for (int c0 = 0; c0 < ts.nc; c0 += RSEL) {
    const uint16_t *rows[RSEL];
    int es[RSEL];
#pragma unroll
    for (int r = 0; r < RSEL; ++r) {
      es[r] = cl[min(c0 + r, ts.nc - 1)];
      rows[r] = a.router_w + (size_t)es[r] * H;
    }
    double v[RSEL];
    exact_logits_rows<gemma, RSEL>(a, xr, rows, ts.norm, root, v);
#pragma unroll
    for (int r = 0; r < RSEL; ++r) {
      if (a.router_b) v[r] += (double)bf16_bits_to_f32(a.router_b[es[r]]);
      if (lane == 0 && c0 + r < ts.nc) s_v[wave][c0 + r] = v[r];
    }
  }
  const double sg = a.shared_gate ? exact_logit<false>(a, a.x + (size_t)t * H, a.shared_gate, 1.0, 1.0) : 0.0;
  if (wave == 0) HH_RT(2);
  __builtin_amdgcn_wave_barrier();
  TopK tk;
  for (int c = 0; c < ts.nc; ++c) tk.insert(s_v[wave][c], cl[c], a.top_k);
  prob_order(tk, a.top_k, a.router);
  finish_token<true>(a, t, tk, sg);
  if (wave == 0) HH_RT(3);
}

// C.
__global__ __launch_bounds__(1024) void dispatch_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  dispatch_batch<16>(a, a.topk_idx);
}

// Batches above 16 tokens: one wave per 16 blocks of a token.
__global__ __launch_bounds__(256) void quant_x_kernel(RouteArgs a) {
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int per_t = (a.hidden / 32 + 15) / 16;
  if (w >= a.tokens * per_t) return;
  quant_x_wave(a, w / per_t, 16 * (w % per_t));
}


// ---- small batches (T ≤ 16): every logit exactly in fp64 -----------------------------------------
// One wave per (token, expert) pair, spread over many compute units (one compute unit's load path
// would take several microseconds to stream even a 32-expert router); expert id E is the shared
// expert's gate row. Writes lg64 [T][E+1].
// Waves past the logits quantise x (MXFP4 layers).
// The FFN block's x terms (MXFP4 layers): as quant_x_wave over token t's layer input, formed
// from the residual stream (norm factor from the whole row, values rounded as norm_row_bf16).
__device__ __forceinline__ void quant_x_wave_block(const RouteArgs &a, int t, int blk0) {
  const int lane = threadIdx.x & 63, g = lane >> 4, l16 = lane & 15;
  const int H = a.hidden, nb = H / 32;
  const int b = blk0 + l16, bc = min(b, nb - 1);
  const float *x = a.resid + (size_t)t * H;
  const int c0 = bc * 32 + 8 * g;
  const f32x4 x0 = *(const f32x4 *)(x + c0), x1 = *(const f32x4 *)(x + c0 + 4);
  const u32x4 nw = *(const u32x4 *)(a.norm_w + c0);
  const double f = norm_factor(row_sumsq(x, H), H, (double)a.norm_eps, a.norm_pow);
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t nbits = (nw[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
    const float xv = k < 4 ? x0[k] : x1[k - 4];
    v[k] = bf16_bits_to_f32(f64_to_bf16_bits((double)xv * f * (double)bf16_bits_to_f32(nbits)));
  }
  uint32_t q[NTX][2], sb[NTX];
  quant_block<NTX>(v, q, sb);
  if (b < nb) {
#pragma unroll
    for (int j = 0; j < NTX; ++j) {
      *(u32x2 *)(a.xq + ((size_t)t * NTX + j) * a.xld + b * 32 + 8 * g) = u32x2{q[j][0], q[j][1]};
      if (g == 0) a.xs[((size_t)t * NTX + j) * (a.xld / 32) + b] = (uint8_t)sb[j];
    }
  }
}

template <bool gemma>
__global__ __launch_bounds__(256) void logits_small_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.experts, E1 = E + 1, H = a.hidden;
  const int p = blockIdx.x * 4 + wave;
  if (wave == 0) HH_RT(0);
  if (p >= a.tokens * E1) {
    const int w = p - a.tokens * E1;
    if (w < quant_x_waves(a)) {
      const int per_t = (H / 32 + 15) / 16;
      quant_x_wave(a, w / per_t, 16 * (w % per_t));
    }
    if (wave == 0) HH_RT(2);
    return;
  }
  const int t = p / E1, e = p - t * E1;
  if (e == E && !a.shared_gate) return;
  const double v = pair_logit<gemma>(a, t, e);
  if (lane == 0) a.lg64[(size_t)t * E1 + e] = v;
  if (wave == 0) HH_RT(1);
}

// The same logits with a 4-wave workgroup per (token, expert) pair (H ≤ 4096): wave u forms
// accumulator u of exact_logit (columns 2048i + 512u + 8l .. +7, i ascending) and wave 0 adds the
// four in exact_logit's order, (acc0 + acc1) + (acc2 + acc3), then sums the wave: the same value
// with a quarter of the products on each wave's dependent chain. GEMMA's norm: wave u forms the
// partial Σx² of each (step, slice u), and every wave adds them in pair_logit's order (steps
// ascending, slices ascending within a step) before the wave sum. Workgroups past the pairs
// quantise x (MXFP4 layers).
template <bool gemma>
__global__ __launch_bounds__(256) void logits_split_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.experts, E1 = E + 1, H = a.hidden;
  const int np = a.tokens * E1;
  __shared__ double s_acc[4][64];
  __shared__ double s_px[4][2][64];
  if (wave == 0) HH_RT(0);
  if ((int)blockIdx.x >= np) {
    const int w = ((int)blockIdx.x - np) * 4 + wave;
    if (w < quant_x_waves(a)) {
      const int per_t = (H / 32 + 15) / 16;
      quant_x_wave(a, w / per_t, 16 * (w % per_t));
    }
    return;
  }
  const int t = blockIdx.x / E1, e = blockIdx.x - t * E1;
  if (e == E && !a.shared_gate) return;   // uniform over the workgroup
  const double v = split_pair_logit<gemma>(a, t, e, s_acc, s_px);
  if (wave == 0 && lane == 0) a.lg64[(size_t)t * E1 + e] = v;
  if (wave == 0) HH_RT(1);
}

// The FFN block's router (a.resid set, bf16 non-GEMMA router, T ≤ 16, H ≤ 4096): workgroup (t, g)
// of BLK_W waves forms token t's layer input x = bf16(resid·f·norm_w) once, into LDS (its threads
// splitting the columns; the norm factor f from every wave's own canonical Σ resid², row_sumsq's
// order), then wave w computes the exact logit of row BLK_W·g + w against it (row E: the shared
// gate) in exact_logit's arithmetic (lane l: columns 2048i + 512u + 8l .. +7, bf16·bf16 products
// exact in fp32 added in fp64 per u, (acc0 + acc1) + (acc2 + acc3), wave sum): the values the
// block's norm kernel followed by the plain router give. Every global load of a wave (router
// row, residual row, its share of the norm weights) goes out before the first arithmetic, so the
// workgroup costs one memory latency. Workgroup (t, 0) also stores x for the expert products;
// workgroups past T·G quantise x (MXFP4 layers).
constexpr int BLK_W = 8;
__host__ __device__ constexpr int block_logit_groups(int E) { return (E + 1 + BLK_W - 1) / BLK_W; }
__global__ __launch_bounds__(64 * BLK_W) void logits_block_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  __shared__ __align__(16) uint16_t s_xn[4096];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int E = a.experts, E1 = E + 1, H = a.hidden;
  const int G = block_logit_groups(E);
  if (wave == 0) HH_RT(0);
  if ((int)blockIdx.x >= a.tokens * G) {
    const int w = ((int)blockIdx.x - a.tokens * G) * BLK_W + wave;
    if (w < quant_x_waves(a)) {
      const int per_t = (H / 32 + 15) / 16;
      quant_x_wave_block(a, w / per_t, 16 * (w % per_t));
    }
    if (wave == 0) HH_RT(2);
    return;
  }
  const int t = blockIdx.x / G, g = blockIdx.x - t * G, e = g * BLK_W + wave;
  const bool live = e < E || (e == E && a.shared_gate);
  const uint16_t *wrow = (e < E || !live) ? a.router_w + (size_t)min(e, E - 1) * H : a.shared_gate;
  const float *x = a.resid + (size_t)t * H;
  // Loads: the router row and the residual row in the canonical layout, and this thread's share
  // of the row (4 columns per step) with its norm weights.
  u32x4 wv[2][4];
  f32x4 xv[2][4][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int h = 2048 * i + 512 * u + 8 * lane;
      const int hc = min(h, H - 8);
      wv[i][u] = *(const u32x4 *)(wrow + hc);
      xv[i][u][0] = *(const f32x4 *)(x + hc);
      xv[i][u][1] = *(const f32x4 *)(x + hc + 4);
      if (h >= H) {
        wv[i][u] = u32x4{0u, 0u, 0u, 0u};
        xv[i][u][0] = xv[i][u][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  constexpr int NS = 4096 / 4 / (64 * BLK_W);   // 4-column groups per thread (H ≤ 4096)
  const int n4 = H / 4;
  f32x4 sx[NS];
  u32x2 sn[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int j = min(tid + 64 * BLK_W * k, n4 - 1);
    sx[k] = ((const f32x4 *)x)[j];
    sn[k] = ((const u32x2 *)a.norm_w)[j];
  }
  // Σ resid² in row_sumsq's order, then the thread's columns of x.
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const double d = xv[i][u][k >> 2][k & 3];
        ss += d * d;
      }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const double f = norm_factor(ss, H, (double)a.norm_eps, a.norm_pow);
  uint16_t *xn_g = (g == 0 && a.xn_out) ? a.xn_out + (size_t)t * H : nullptr;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int j = tid + 64 * BLK_W * k;
    if (j < n4) {
      uint32_t o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t nb = (sn[k][c >> 1] >> (16 * (c & 1))) & 0xFFFFu;
        o[c] = f64_to_bf16_bits((double)sx[k][c] * f * (double)bf16_bits_to_f32(nb));
      }
      const u32x2 pk = {o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      *(u32x2 *)(s_xn + 4 * j) = pk;
      if (xn_g) *(u32x2 *)(xn_g + 4 * j) = pk;
    }
  }
  __syncthreads();
  if (!live) return;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (2048 * i >= H) break;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const u32x4 xb = *(const u32x4 *)(s_xn + min(2048 * i + 512 * u + 8 * lane, H - 8));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int sh = (k & 1) * 16;
        const float xf = bf16_bits_to_f32((xb[k >> 1] >> sh) & 0xFFFF);
        const float wf = bf16_bits_to_f32((wv[i][u][k >> 1] >> sh) & 0xFFFF);
        acc[u] += (double)(xf * wf);
      }
    }
  }
  double v = wave_sum_f64((acc[0] + acc[1]) + (acc[2] + acc[3]));
  if (e < E && a.router_b) v += (double)bf16_bits_to_f32(a.router_b[e]);
  if (lane == 0) a.lg64[(size_t)t * E1 + e] = v;
  if (wave == 0) HH_RT(1);
}

// Top-k and weights of every token from lg64 (operator entry hh_router_topk, T ≤ 16): one
// workgroup, wave w takes tokens w, w + 4, ...
__global__ __launch_bounds__(256) void select_small_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  const int wave = threadIdx.x >> 6;
  const int E1 = a.experts + 1;
  __shared__ int s_ri[4][kMaxTopK];
  __shared__ double s_rv[4][kMaxTopK];
  __shared__ int s_ci[4][kFastCand];
  __shared__ double s_cv[4][kFastCand];
  for (int t = wave; t < a.tokens; t += 4) {
    const double *lg = a.lg64 + (size_t)t * E1;
    TopK tk = topk_fast(lg, a.experts, a.top_k, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave]);
    prob_order(tk, a.top_k, a.router);
    finish_token(a, t, tk, a.shared_gate ? lg[a.experts] : 0.0);
  }
}

// ---- MLX-affine router: fp64 logits of every (token, row) pair -----------------------------
// Rows 0..E-1 are the router, row E the shared gate (whose input x the layer requires to equal
// the router's, so every row reads a.xr). A row's codes are 16-byte vectors v = 0 .. V−1 of NC =
// 128 / BITS columns each (columns NC·v ..; one MLX group holds 64 / NC vectors); lane l takes the
// vectors l, l + 64, ... and its partial sum runs over them in that order, column by column:
// acc = fma(q·scale + bias, x, acc), where q·scale + bias (an 8-bit code times a bf16 scale, plus
// the bf16 bias) and its product with the bf16 x are exact in fp64, so each step rounds once, like
// the reference's fp64 sum (MLXAffine.matvec, Gemma4ReferenceOps.swift:224-239). The logit is the
// wave's xor-butterfly sum of the 64 partials (wave_sum_f64), plus the router bias. That order is
// fixed per (token, row) whatever the batch size or tiling, so decode and prefill get the same
// bits. Each wave takes R consecutive rows and walks its token range 4 tokens at a time (one
// dequantisation per column for 4·R products); T ≤ 16: R = 1, one wave per row and every token
// (the decode router: ≈ E + 1 waves over the whole chip); T > 16: MLX_RT_R rows over 16-token tiles.
template <int BITS>
__device__ __forceinline__ uint32_t mlx_code(const u32x4 &q, int s) {
  if constexpr (BITS == 8) return (q[s >> 2] >> (8 * (s & 3))) & 0xFFu;
  else return (q[s >> 3] >> (4 * (s & 7))) & 0xFu;
}

constexpr int MLX_RT_TILE = 16;   // tokens per wave above 16 tokens
constexpr int MLX_RT_R = 2;       // rows per wave above 16 tokens

// The fp64 logits of rows row_of(0) .. row_of(R−1) (row E: the shared gate) for tokens t0 .. t1−1,
// one wave, in the arithmetic above: lane l's code vectors l, l + 64, ... (J per lane, zero past
// the row) summed column by column in fp64, the R·P wave sums of each P-token group on one
// reduce-scatter butterfly, plus the router bias. `out(v, r, token)` is called by one lane per
// total, for r < nr and tokens < t1 only. A (token, row) value does not depend on R, P, t0, t1,
// the other rows or the token's place in its group.
template <int BITS, int R, int J, int P, class RowOf, class Out>
__device__ __forceinline__ void mlx_rows_logits(const RouteArgs &a, RowOf row_of, int nr, int t0, int t1, Out out) {
  constexpr int NC = 128 / BITS, XV = NC / 8;
  static_assert(R * P == 1 || R * P == 4 || R * P == 8 || R * P == 16, "the reduce-scatter's lane mapping");
  const int lane = threadIdx.x & 63;
  const int E = a.experts, H = a.hidden, T = a.tokens;
  const int V = H / NC, wpr = H * BITS / 32, gpr = H / 64;
  // The rows' code vectors and group (scale, bias) of this lane, once: vectors past the row
  // (J·64 > V) are zero codes with zero scale and bias, adding exactly nothing.
  u32x4 q[R][J];
  double sc[R][J], bi[R][J];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row_of(r);
    const bool sg = row == E;
    const uint32_t *qr = sg ? a.sg_words : a.rq_words + (size_t)row * wpr;
    const uint16_t *sr = sg ? a.sg_scales : a.rq_scales + (size_t)row * gpr;
    const uint16_t *br = sg ? a.sg_biases : a.rq_biases + (size_t)row * gpr;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int v = lane + 64 * j, vc = min(v, V - 1);
      q[r][j] = *(const u32x4 *)(qr + 4 * vc);
      sc[r][j] = (double)bf16_bits_to_f32(sr[vc * NC / 64]);
      bi[r][j] = (double)bf16_bits_to_f32(br[vc * NC / 64]);
      if (v >= V) { q[r][j] = u32x4{0u, 0u, 0u, 0u}; sc[r][j] = 0.0; bi[r][j] = 0.0; }
    }
  }
  for (int t = t0; t < t1; t += P) {
    u32x4 xv[P][J][XV];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const uint16_t *xr = a.xr + (size_t)min(t + p, T - 1) * H;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int vc = min(lane + 64 * j, V - 1);
#pragma unroll
        for (int u = 0; u < XV; ++u) xv[p][j][u] = *(const u32x4 *)(xr + NC * vc + 8 * u);
      }
    }
    double acc[R][P];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) acc[r][p] = 0.0;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        double x[P];
#pragma unroll
        for (int p = 0; p < P; ++p)
          x[p] = (double)bf16_bits_to_f32((xv[p][j][k >> 3][(k & 7) >> 1] >> (16 * (k & 1))) & 0xFFFFu);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const double w = fma((double)mlx_code<BITS>(q[r][j], k), sc[r][j], bi[r][j]);
#pragma unroll
          for (int p = 0; p < P; ++p) acc[r][p] = fma(w, x[p], acc[r][p]);
        }
      }
    // all R·P sums at once; lane l ends with the total of acc index l >> (6 − log2(R·P)) (one
    // sum: the plain butterfly, the same additions)
    constexpr int N = R * P, SH = N == 1 ? 6 : N == 4 ? 4 : N == 8 ? 3 : 2;
    double flat[N];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) flat[r * P + p] = acc[r][p];
    double v;
    if constexpr (N == 1) v = wave_sum_f64(flat[0]);
    else v = wave_sum_scatter_f64<N>(flat);
    const int i = lane >> SH, r = i / P, tp = t + i % P;
    const int row = row_of(min(r, R - 1));
    if (row < E && a.router_b) v += (double)bf16_bits_to_f32(a.router_b[row]);
    if ((lane & ((1 << SH) - 1)) == 0 && r < nr && tp < t1) out(v, r, tp);
  }
}

template <int BITS, int R, int J>
__global__ __launch_bounds__(256) void mlx_router_logits_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  zero_dispatch_counts(a);
  const int wave = threadIdx.x >> 6;
  const int E = a.experts, T = a.tokens;
  const int rows = E + (a.shared_gate ? 1 : 0);
  const int waves_per_tile = (rows + R - 1) / R, blocks_per_tile = (waves_per_tile + 3) / 4;
  const int tile = blockIdx.x / blocks_per_tile;
  const int wid = (blockIdx.x - tile * blocks_per_tile) * 4 + wave;
  if (wid >= waves_per_tile) return;   // no barriers below
  const int tsz = T <= RT_TOK ? T : MLX_RT_TILE;
  const int t0 = tile * tsz, t1 = min(T, t0 + tsz);
  const int r0 = wid * R;
  mlx_rows_logits<BITS, R, J, 4>(a, [&](int r) { return min(r0 + r, rows - 1); }, rows - r0, t0, t1,
                                 [&](double v, int r, int tp) { a.lg64[(size_t)tp * (E + 1) + r0 + r] = v; });
}

// ---- MLX-affine router above 16 tokens: screen on the MFMA, exact logits of the candidates ----
// Screening logit of (token t, row e) on the bf16 MFMA: per 64-column group g, P_g = Σ q·x (codes
// ≤ 255 are exact in bf16, each q·x exact in fp32; the MFMA adds 64 of them in fp32) and
// X_g = Σ x (fp32), then l += s_g·P_g + b_g·X_g in fp32. Against the exact Σ (q·s + b)·x:
// |l − exact| ≤ (63 + 2 + 1 + NG)·u·Σ_c (|s|·q + |b|)·|x| + O(u²) ≤ kMlxScreenCoef·‖v_e‖·‖x_t‖ with
// v_c = |s_g|·q_c + |b_g|, u = 2^-24, NG ≤ 64 groups: the coefficient 256·u is twice that
// (rounding modes aside). Each workgroup takes a 16-token × 16-row tile, its 4 waves the groups
// g ≡ wave (mod 4); in a group, lane group gg supplies columns 16gg .. 16gg+15 (both MFMAs of the
// group, A and B alike, so any column order is the same sum's terms). The first token tile also
// writes ‖v_e‖ (rounded up) to wn. Selection then recomputes the candidates exactly
// (mlx_select_kernel), so the screen's order of additions does not matter.
constexpr double kMlxScreenCoef = 256.0 * 5.9604644775390625e-08;
constexpr int MLX_SG_MAX = 64;   // groups per row (H ≤ 4096)
template <int BITS>
__global__ __launch_bounds__(256) void mlx_screen_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  zero_dispatch_counts(a);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, gg = lane >> 4, l16 = lane & 15;
  const int E = a.experts, H = a.hidden, T = a.tokens, NG = H / 64;
  const int etiles = (E + 15) / 16;
  const int tt = blockIdx.x / etiles, et = blockIdx.x - tt * etiles;
  const int t0 = tt * 16, e0 = et * 16;
  const int ntok = min(16, T - t0);
  __shared__ float2 s_sb[16][MLX_SG_MAX];   // (scale, bias) of the tile's rows; rows past E: 0
  __shared__ float s_part[4][16][16];        // [wave][row][token]
  __shared__ float s_wn[4][16];
  for (int i = tid; i < 16 * NG; i += 256) {
    const int r = i / NG, g = i - r * NG, e = e0 + r;
    float2 v = {0.f, 0.f};
    if (e < E) v = {bf16_bits_to_f32(a.rq_scales[(size_t)e * NG + g]), bf16_bits_to_f32(a.rq_biases[(size_t)e * NG + g])};
    s_sb[r][g] = v;
  }
  __syncthreads();
  const int row = min(e0 + l16, E - 1);
  const bool row_ok = e0 + l16 < E;
  const uint16_t *xr = a.xr + (size_t)(t0 + min(l16, ntok - 1)) * H;
  const uint8_t *qrow = (const uint8_t *)a.rq_words + (size_t)row * (H * BITS / 8);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float vv = 0.f;   // Σ v² of this lane's columns of row l16 (first token tile)
  for (int g = wave; g < NG; g += 4) {
    const int c = 64 * g + 16 * gg;
    // 16 codes of row l16, as two bf16x8 A operands
    u32x4 qv;
    if constexpr (BITS == 8) {
      qv = *(const u32x4 *)(qrow + c);
    } else {
      const u32x2 q = *(const u32x2 *)(qrow + c / 2);
      qv = u32x4{q[0], q[1], 0u, 0u};
    }
    u32x4 a0, a1;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const uint32_t c0 = mlx_code<BITS>(qv, 2 * kk), c1 = mlx_code<BITS>(qv, 2 * kk + 1);
      const uint32_t lo = f32_to_bf16_bits((float)(row_ok ? c0 : 0u)), hi = f32_to_bf16_bits((float)(row_ok ? c1 : 0u));
      const uint32_t pk = lo | (hi << 16);
      if (kk < 4) a0[kk] = pk; else a1[kk - 4] = pk;
      if (tt == 0) {
        const float2 sbv = s_sb[l16][g];
        const float v0 = fabsf(sbv.x) * (float)c0 + fabsf(sbv.y), v1 = fabsf(sbv.x) * (float)c1 + fabsf(sbv.y);
        vv = fmaf(v0, v0, fmaf(v1, v1, vv));
      }
    }
    const u32x4 b0 = *(const u32x4 *)(xr + c), b1 = *(const u32x4 *)(xr + c + 8);
    f32x4 p = {0.f, 0.f, 0.f, 0.f};
    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0), as_bf16x8(b0), p, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1), as_bf16x8(b1), p, 0, 0, 0);
    // Σx of the group for token l16: this lane's 16 columns, then the 4 lane groups
    float xs = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) xs += (bf_lo(b0[q]) + bf_hi(b0[q])) + (bf_lo(b1[q]) + bf_hi(b1[q]));
    xs += __shfl_xor(xs, 16);
    xs += __shfl_xor(xs, 32);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const float2 sbv = s_sb[4 * gg + ii][g];
      acc[ii] += fmaf(sbv.x, p[ii], sbv.y * xs);
    }
  }
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) s_part[wave][4 * gg + ii][l16] = acc[ii];
  if (tt == 0) {
    vv += __shfl_xor(vv, 16);
    vv += __shfl_xor(vv, 32);
    if (gg == 0) s_wn[wave][l16] = vv;
  }
  __syncthreads();
  const int er = tid >> 4, tk = tid & 15, e = e0 + er;
  if (e < E && tk < ntok) {
    float v = (s_part[0][er][tk] + s_part[1][er][tk]) + (s_part[2][er][tk] + s_part[3][er][tk]);
    if (a.router_b) v += bf16_bits_to_f32(a.router_b[e]);
    a.lg32[(size_t)(t0 + tk) * E + e] = v;
    // ‖v_e‖, rounded up: the fp32 sums of squares are within a few hundred ulps
    if (tt == 0 && tk == 0)
      a.wn[e] = sqrtf((s_wn[0][er] + s_wn[1][er]) + (s_wn[2][er] + s_wn[3][er])) * 1.0001f + 1e-30f;
  }
}

// One workgroup per token: the 4 waves screen it (screen_token with the MLX screen's bound), then
// wave w computes the exact logits of candidates w, w + 4, ... with mlx_rows_logits (the decode
// router's values, bit for bit) and wave 1 the shared gate's; wave 0 ranks them and writes the
// token's routing (as route_select_kernel).
template <int BITS, int J>
__global__ __launch_bounds__(256) void mlx_select_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x, E = a.experts;
  __shared__ int s_cl[4][kMaxExperts];
  __shared__ int s_rk[4][64];
  __shared__ double s_v[kMaxExperts];
  __shared__ double s_sg;
  const float *lg = a.lg32 + (size_t)t * E;
  const TokenScreen ts = screen_token<false, 4>(a, t, [&](int e) { return lg[e]; }, [&](int e) { return a.wn[e]; },
                                                s_cl[wave], s_rk, kMlxScreenCoef);
  // wave w: candidates w, w + 4, ... (one row of the one token per pass); wave 1 also the
  // shared gate's row
  const int *cl = s_cl[wave];
  for (int c0 = wave; c0 < ts.nc; c0 += 4)
    mlx_rows_logits<BITS, 1, J, 1>(a, [&](int) { return cl[c0]; }, 1, t, t + 1, [&](double v, int, int) { s_v[c0] = v; });
  if (wave == 1 && a.shared_gate)
    mlx_rows_logits<BITS, 1, J, 1>(a, [&](int) { return E; }, 1, t, t + 1, [&](double v, int, int) { s_sg = v; });
  __syncthreads();
  if (wave != 0) return;
  TopK tk;
  for (int c = 0; c < ts.nc; ++c) tk.insert(s_v[c], s_cl[0][c], a.top_k);
  prob_order(tk, a.top_k, a.router);
  finish_token<true>(a, t, tk, a.shared_gate ? s_sg : 0.0);
}
template <int BITS> void *mlx_select_fn(int H) {
  const int J = (H / (128 / BITS) + 63) / 64;
  if (J <= 1) return (void *)mlx_select_kernel<BITS, 1>;
  if (J <= 2) return (void *)mlx_select_kernel<BITS, 2>;
  if (J <= 4) return (void *)mlx_select_kernel<BITS, 4>;
  return nullptr;
}

// The launch of mlx_router_logits_kernel for a row of H columns (J = vectors per lane).
template <int BITS, int R>
void *mlx_logits_fn(int H) {
  const int J = (H / (128 / BITS) + 63) / 64;
  if (J <= 1) return (void *)mlx_router_logits_kernel<BITS, R, 1>;
  if (J <= 2) return (void *)mlx_router_logits_kernel<BITS, R, 2>;
  if (J <= 4) return (void *)mlx_router_logits_kernel<BITS, R, 4>;
  return nullptr;
}

// Top-k and weights of every token from lg64, one wave per token (batches with an MLX router).
__global__ __launch_bounds__(256) void select_lg64_kernel(RouteArgs a) {
  warm_kernargs<sizeof(RouteArgs)>();
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  __shared__ int s_ri[4][kMaxTopK];
  __shared__ double s_rv[4][kMaxTopK];
  __shared__ int s_ci[4][kFastCand];
  __shared__ double s_cv[4][kFastCand];
  if (t >= a.tokens) return;
  const double *lg = a.lg64 + (size_t)t * (a.experts + 1);
  TopK tk = topk_fast(lg, a.experts, a.top_k, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave]);
  prob_order(tk, a.top_k, a.router);
  finish_token<true>(a, t, tk, a.shared_gate ? lg[a.experts] : 0.0);
}

// The dispatch of a batch's top-k table: one workgroup below DB_MIN_ASSIGN assignments (or
// without a count buffer), else the multi-block scatter, after dispatch_count_kernel unless the
// selection already counted (`counted`).
static hipError_t launch_dispatch(const RouteArgs &a, hipStream_t s, hipEvent_t stop, bool counted) {
  const int A = a.tokens * a.top_k;
  if (A < DB_MIN_ASSIGN || !a.dcount) {
    hipExtLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, s, nullptr, stop, 0, a);
    return hipGetLastError();
  }
  const int nb = dispatch_blocks(A);
  hipError_t e;
  if (!counted) {
    hipExtLaunchKernelGGL(dispatch_count_kernel, dim3(nb), dim3(256), 0, s, nullptr, nullptr, 0, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  hipExtLaunchKernelGGL(dispatch_scatter_kernel, dim3(nb), dim3(256), 0, s, nullptr, stop, 0, a);
  return hipGetLastError();
}

// The MLX-router sequence: exact logits, x terms (MXFP4 layers), selection (unless the layer's
// decode gate-up kernel selects), dispatch (layers above 16 tokens).
hipError_t launch_route_mlx(const RouteArgs &a, hipStream_t s, Timing tm) {
  const int rows = a.experts + (a.shared_gate ? 1 : 0);
  const bool small = a.tokens <= RT_TOK;
  if (!small && a.hidden % 64 == 0 && a.hidden <= 64 * MLX_SG_MAX) {
    // screen on the MFMA, then the candidates' exact logits
    const bool disp = a.want_dispatch != 0;
    void *screen = a.router_bits == 8 ? (void *)mlx_screen_kernel<8> : (void *)mlx_screen_kernel<4>;
    void *select = a.router_bits == 8 ? mlx_select_fn<8>(a.hidden) : mlx_select_fn<4>(a.hidden);
    if (!select) return hipErrorInvalidValue;
    void *args[] = {(void *)&a};
    const int blocks = ((a.tokens + 15) / 16) * ((a.experts + 15) / 16);
    hipError_t e = hipExtLaunchKernel(screen, dim3(blocks), dim3(256), args, 0, s, tm.start, nullptr, 0);
    if (e != hipSuccess) return e;
    if (a.xq) {
      const int qw = a.tokens * ((a.hidden / 32 + 15) / 16);
      hipExtLaunchKernelGGL(quant_x_kernel, dim3((qw + 3) / 4), dim3(256), 0, s, nullptr, nullptr, 0, a);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    e = hipExtLaunchKernel(select, dim3(a.tokens), dim3(256), args, 0, s, nullptr, disp ? nullptr : tm.stop, 0);
    if (e != hipSuccess || !disp) return e;
    return launch_dispatch(a, s, tm.stop, true);
  }
  const int R = small ? 1 : MLX_RT_R;
  const int blocks = (small ? 1 : (a.tokens + MLX_RT_TILE - 1) / MLX_RT_TILE) * (((rows + R - 1) / R + 3) / 4);
  const bool sel = !small || a.want_dispatch == 0;
  const bool disp = !small && a.want_dispatch != 0;
  const bool quant = a.xq != nullptr;
  void *kern = a.router_bits == 8 ? (small ? mlx_logits_fn<8, 1>(a.hidden) : mlx_logits_fn<8, MLX_RT_R>(a.hidden))
                                  : (small ? mlx_logits_fn<4, 1>(a.hidden) : mlx_logits_fn<4, MLX_RT_R>(a.hidden));
  if (!kern) return hipErrorInvalidValue;
  {
    void *args[] = {(void *)&a};
    hipError_t le = hipExtLaunchKernel(kern, dim3(blocks), dim3(256), args, 0, s, tm.start,
                                       (sel || quant) ? nullptr : tm.stop, 0);
    if (le != hipSuccess) return le;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (quant) {
    const int qw = a.tokens * ((a.hidden / 32 + 15) / 16);
    hipExtLaunchKernelGGL(quant_x_kernel, dim3((qw + 3) / 4), dim3(256), 0, s, nullptr,
                          sel ? nullptr : tm.stop, 0, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (!sel) return hipSuccess;
  hipExtLaunchKernelGGL(select_lg64_kernel, dim3((a.tokens + 3) / 4), dim3(256), 0, s, nullptr,
                        disp ? nullptr : tm.stop, 0, a);
  if ((e = hipGetLastError()) != hipSuccess || !disp) return e;
  return launch_dispatch(a, s, tm.stop, true);
}
}  // namespace hh

namespace hh {
hipError_t launch_route(const RouteArgs &a, hipStream_t s, Timing tm) {
  if (a.router_bits) return launch_route_mlx(a, s, tm);
  if (a.tokens <= RT_TOK) {
    // The layer (want_dispatch) selects inside its gate-up kernel; the operator entry selects
    // here.
    const int qwaves = a.xq ? a.tokens * ((a.hidden / 32 + 15) / 16) : 0;
    const bool sel = a.want_dispatch == 0;
    const bool g = a.router == R_GEMMA;
    if (a.resid) {
      // The FFN block's router (the caller admits only bf16 non-GEMMA routers, H ≤ 4096).
      if (g || a.hidden > 4096) return hipErrorInvalidValue;
      const int blocks = a.tokens * block_logit_groups(a.experts) + (qwaves + BLK_W - 1) / BLK_W;
      hipExtLaunchKernelGGL(logits_block_kernel, dim3(blocks), dim3(64 * BLK_W), 0, s, tm.start,
                            sel ? nullptr : tm.stop, 0, a);
    } else if (a.hidden <= 4096 && (!g || a.tokens == 1)) {
      // (GEMMA: every workgroup also forms its token's norm, which costs more than the split
      // saves once the batch fills the machine; measured T=8 route 8.6 → 11.0 µs.)
      const int pairs = a.tokens * (a.experts + 1);
      hipExtLaunchKernelGGL(g ? logits_split_kernel<true> : logits_split_kernel<false>,
                            dim3(pairs + (qwaves + 3) / 4), dim3(256), 0, s, tm.start, sel ? nullptr : tm.stop,
                            0, a);
    } else {
      const int waves = a.tokens * (a.experts + 1) + qwaves;
      hipExtLaunchKernelGGL(g ? logits_small_kernel<true> : logits_small_kernel<false>,
                            dim3((waves + 3) / 4), dim3(256), 0, s, tm.start, sel ? nullptr : tm.stop,
                            0, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !sel) return e;
    hipExtLaunchKernelGGL(select_small_kernel, dim3(1), dim3(256), 0, s, nullptr, tm.stop, 0, a);
    return hipGetLastError();
  }
  const int ttiles = (a.tokens + RT_TOK - 1) / RT_TOK;
  const int etiles = (a.experts + 15) / 16;
  const bool third = a.want_dispatch != 0;
  const bool g = a.router == R_GEMMA;
  const int qw = a.xq ? a.tokens * ((a.hidden / 32 + 15) / 16) : 0;
  {
    const int ret = wide_ret(a.tokens, a.experts);
    void *k = g ? wide_logits_fn<true>(ret) : wide_logits_fn<false>(ret);
    void *args[] = {(void *)&a};
    const int blocks = ttiles * ((etiles + ret - 1) / ret) + (qw + RLW2 - 1) / RLW2;
    hipError_t le = hipExtLaunchKernel(k, dim3(blocks), dim3(64 * RLW2), args, 0, s, tm.start, nullptr, 0);
    if (le != hipSuccess) return le;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.tokens >= kSelWaveT && a.hidden <= 4096)
    hipExtLaunchKernelGGL(g ? route_select_wave_kernel<true> : route_select_wave_kernel<false>, dim3((a.tokens + 3) / 4),
                          dim3(256), 0, s, nullptr, third ? nullptr : tm.stop, 0, a);
  else
    hipExtLaunchKernelGGL(g ? route_select_kernel<true> : route_select_kernel<false>, dim3(a.tokens), dim3(256), 0, s,
                          nullptr, third ? nullptr : tm.stop, 0, a);
  e = hipGetLastError();
  if (e != hipSuccess || !third) return e;
  return launch_dispatch(a, s, tm.stop, true);
}
// Stand-alone permutation of a given top-k table (hh_permute).
hipError_t launch_permute(const RouteArgs &a, hipStream_t s) { return launch_dispatch(a, s, nullptr, false); }
}  // namespace hh
