// hh_common.hpp — shared device helpers and kernel argument blocks of HydraHIP (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

namespace hh {

enum Quant { Q_MXFP4 = 0, Q_MLX4 = 1, Q_MLX8 = 2, Q_BF16 = 3 };
enum Act { A_SWIGLU_OAI = 0, A_SILU = 1, A_GELU_TANH = 2 };
// Multi-block dispatch (hh_route.hip): at most DB_MAX blocks, taken from DB_MIN_ASSIGN (token, rank)
// assignments on; the count buffer holds DB_MAX · E words [block][expert]. In the layer the
// router-logits launch zeroes it and the selection adds each assignment's count (finish_token).
constexpr int DB_MAX = 64, DB_MIN_ASSIGN = 1024;
__host__ __device__ inline int dispatch_blocks(int A) {
  const int nb = (A + 255) / 256;
  return nb < 1 ? 1 : (nb > DB_MAX ? DB_MAX : nb);
}
// Assignments per block: whole 256-assignment groups (4 waves × 64).
__host__ __device__ inline int dispatch_range(int A, int nb) { return (((A + nb - 1) / nb) + 255) & ~255; }

enum Router { R_TOPK_SOFTMAX = 0, R_SOFTMAX_TOPK_RENORM = 1, R_GEMMA = 2 };

constexpr int kMaxTopK = 8;
constexpr int kMaxExperts = 512;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- bf16 (the reference's BF16.toFloat / fromFloat, BF16.swift:20-33) ----------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if (f != f) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// e8m0 scale byte → fp32 factor 2^(s-127), exactly (s = 0 is the subnormal 2^-127, s = 255 is
// +inf as in the reference's exp2, MXFP4.swift:37-42).
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  return __uint_as_float(s == 0 ? 0x00400000u : (s << 23));
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4 &v) { return __builtin_bit_cast(bf16x8, v); }

// 8 MXFP4 values (one dword, low nibble first) → 8 bf16 scaled by 2^(s-127). The values are
// e2m1·2^k, exact in bf16.
__device__ __forceinline__ bf16x8 mxfp4_to_bf16(uint32_t w, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  u32x4 r = {__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
             __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)};
  return as_bf16x8(r);
}

// ---- fp8 e4m3 activation terms for the scaled MXFP4 products ---------------------------------
// A block of 32 activations (of one token, along K) is written as NTERM fp8 e4m3 terms with an
// e8m0 scale each: v ≈ Σ_t q_t·2^(b_t-127). b_0 puts the block's largest magnitude in [128, 256)
// and b_t = b_0 - 4t; each term takes the exact residual of the previous ones (r − dec(q)·2^b is
// exact in fp32), so NTERM terms keep ~4·NTERM significant bits of every element not far below the
// block maximum: 2 terms reproduce a bf16 element exactly when it is ≥ 2^-13 of the block maximum,
// 3 terms keep an fp32 activation to ~2^-13 relative. The block is spread over the 4 lanes
// l, l^16, l^32, l^48 (lane groups of a wave), 8 values each; the result depends only on the 32
// values, not on how they are spread.
constexpr int NTX = 2;   // terms of the expert input x
constexpr int NTH = 3;   // terms of the activation h

// Exchanges across the 4 lane groups (rows of 16 lanes) on gfx950's row swaps, VALU instructions
// (a shuffle is an LDS-crossbar round trip): with both operands v, permlane32_swap leaves
// (v[l], v[l ^ 32]) in the two results of every lane, in one order or the other, and
// permlane16_swap (v[l], v[l ^ 16]). Every lane of the wave must be active.
__device__ __forceinline__ float max_lane_groups(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
// (g0 + g1) + (g2 + g3) of a value held by the 4 lane groups, identical in every lane (the two
// operands of each addition come in either order: the same sum).
__device__ __forceinline__ float sum_lane_groups(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// quant_block's term bytes regrouped for 8-byte stores: lane group g holds, for j = 0..3, the
// 2 bytes at columns 2g + 8j of its token's 32-column block ((d0, d1) = pieces (0 | 1 << 16,
// 2 | 3 << 16)); afterwards it holds columns 8g .. 8g + 7 ((e0, e1)), i.e. piece g of groups
// 0..3 in order: a 4 × 4 transpose of 16-bit pieces across the lane groups (a dword swap between
// groups g and g ^ 2, then a half-dword swap between g and g ^ 1). Every lane must be active.
__device__ __forceinline__ void transpose_pieces(uint32_t d0, uint32_t d1, int g, uint32_t &e0, uint32_t &e1) {
  // Groups 0, 1 keep d0 and take d0 of g + 2; groups 2, 3 keep d1 and take d1 of g − 2.
  const auto r = __builtin_amdgcn_permlane32_swap(d0, d1, false, false);
  const uint32_t A = r[0], B = r[1];   // (0,1): A = own d0, B = d0 of g+2; (2,3): A = d1 of g−2, B = own d1
  const bool odd = g & 1;
  const uint32_t S = odd ? ((A & 0xFFFFu) | (B << 16)) : ((A >> 16) | (B & 0xFFFF0000u));
  const auto q = __builtin_amdgcn_permlane16_swap(S, S, false, false);
  const uint32_t R = odd ? q[0] : q[1];   // S of g ^ 1
  e0 = odd ? ((R & 0xFFFFu) | (A & 0xFFFF0000u)) : ((A & 0xFFFFu) | (R << 16));
  e1 = odd ? ((R >> 16) | (B & 0xFFFF0000u)) : ((B & 0xFFFFu) | (R & 0xFFFF0000u));
}

template <int NTERM>
__device__ __forceinline__ void quant_block(const float (&v)[8], uint32_t (&q)[NTERM][2],
                                            uint32_t (&sb)[NTERM]) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = max_lane_groups(amax);
  const int eb = (int)((__float_as_uint(amax) >> 23) & 0xFF);   // biased exponent (0: zero/tiny)
  const int b0 = eb > 7 ? eb - 7 : 0;
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = v[i];
#pragma unroll
  for (int t = 0; t < NTERM; ++t) {
    const int bt = b0 - 4 * t > 0 ? b0 - 4 * t : 0;
    sb[t] = (uint32_t)bt;
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = fminf(fmaxf(__builtin_amdgcn_ldexpf(r[i], 127 - bt), -448.f), 448.f);
    int w0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    w0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], w0, true);
    int w1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
    w1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], w1, true);
    q[t][0] = (uint32_t)w0;
    q[t][1] = (uint32_t)w1;
    if (t + 1 < NTERM) {
      const float d[8] = {__builtin_amdgcn_cvt_f32_fp8(w0, 0), __builtin_amdgcn_cvt_f32_fp8(w0, 1),
                          __builtin_amdgcn_cvt_f32_fp8(w0, 2), __builtin_amdgcn_cvt_f32_fp8(w0, 3),
                          __builtin_amdgcn_cvt_f32_fp8(w1, 0), __builtin_amdgcn_cvt_f32_fp8(w1, 1),
                          __builtin_amdgcn_cvt_f32_fp8(w1, 2), __builtin_amdgcn_cvt_f32_fp8(w1, 3)};
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] -= __builtin_amdgcn_ldexpf(d[i], bt - 127);
    }
  }
}

// quant_block with one value per lane, the block held by the 32 lanes of a half wave (lane & 31
// = position in the block): the same term bytes and scales, since the block maximum is the same
// and every other step is per element. q[t] holds the value's byte of term t.
template <int NTERM>
__device__ __forceinline__ void quant_lane(float v, uint32_t (&q)[NTERM], uint32_t (&sb)[NTERM]) {
  float amax = fabsf(v);
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  const int eb = (int)((__float_as_uint(amax) >> 23) & 0xFF);
  const int b0 = eb > 7 ? eb - 7 : 0;
  float r = v;
#pragma unroll
  for (int t = 0; t < NTERM; ++t) {
    const int bt = b0 - 4 * t > 0 ? b0 - 4 * t : 0;
    sb[t] = (uint32_t)bt;
    const float y = fminf(fmaxf(__builtin_amdgcn_ldexpf(r, 127 - bt), -448.f), 448.f);
    const int w = __builtin_amdgcn_cvt_pk_fp8_f32(y, 0.f, 0, false);
    q[t] = (uint32_t)w & 0xFFu;
    if (t + 1 < NTERM) r -= __builtin_amdgcn_ldexpf(__builtin_amdgcn_cvt_f32_fp8(w, 0), bt - 127);
  }
}

// ---- gated activations (device twins of the oracle's act_pair) ------------------------------
// 1 / (1 + e^-z) in fp32 to a few ulps, with no compare or division step: e^x = 2^n · 2^f by
// Cody–Waite reduction (x·log2 e formed as a head and a tail: the fma recovers the head's
// rounding error, the tail carries log2 e's bits below fp32), 2^f on v_exp_f32, 2^n by ldexp;
// the reciprocal of d = 1 + e^x is v_rcp_f32 and one Newton step r += r·(1 − d·r). x is clamped
// to [−104, 80]: below, 2^n underflows to 0 (the factor is 1); above, the factor (< 2e-35) is
// formed without overflow. The library expf and the IEEE division test ranges and scale their
// operands through the one condition register (VCC), which chains every activation of a block
// to the previous one; these steps leave independent activations free to interleave.
__device__ __forceinline__ float sigmoid_f32(float z) {
  const float x = fminf(fmaxf(-z, -104.0f), 80.0f);
  const float log2e_hi = 1.44269502e+00f, log2e_lo = 1.92596299e-08f;
  const float ph = x * log2e_hi;
  const float pl = __builtin_fmaf(x, log2e_hi, -ph) + x * log2e_lo;
  const float n = __builtin_rintf(ph);
  const float e = __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), (int)n);
  const float d = 1.0f + e;
  const float r = __builtin_amdgcn_rcpf(d);
  return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}
// ReferenceOps.swiglu (ReferenceOps.swift:87-99).
__device__ __forceinline__ float act_swiglu(float g, float u, float alpha, float limit) {
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  return g * sigmoid_f32(alpha * g) * (u + 1.0f);
}
// QwenReferenceOps.siluMultiply (QwenReferenceOps.swift:149-151).
__device__ __forceinline__ float act_silu(float g, float u) { return g * sigmoid_f32(g) * u; }
// Gemma4ReferenceOps.gelu (Gemma4ReferenceOps.swift:37-40), with (1 + tanh y) / 2 = 1 / (1 + e^-2y);
// the tanh argument is clamped to ±15, where tanh is 1 to within float precision (as
// gemma.metal:77-88 does).
__device__ __forceinline__ float act_gelu(float g, float u) {
  float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
  inner = fminf(fmaxf(inner, -15.0f), 15.0f);
  return g * sigmoid_f32(2.0f * inner) * u;
}
__device__ __forceinline__ float activate(int act, float g, float u, float alpha, float limit) {
  if (act == A_SWIGLU_OAI) return act_swiglu(g, u, alpha, limit);
  if (act == A_SILU) return act_silu(g, u);
  return act_gelu(g, u);
}
// N independent activations, the kind tested once: the N chains (exponential, division) form one
// block, which the compiler interleaves (a test per element gives N blocks run one after the
// other, each waiting out its own latencies). Each element's arithmetic is activate's.
template <int N>
__device__ __forceinline__ void activate_n(int act, const float (&g)[N], const float (&u)[N], float (&y)[N],
                                           float alpha, float limit) {
  if (act == A_SWIGLU_OAI) {
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = act_swiglu(g[i], u[i], alpha, limit);
  } else if (act == A_SILU) {
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = act_silu(g[i], u[i]);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = act_gelu(g[i], u[i]);
  }
}

// ---- kernel argument blocks -----------------------------------------------------------------
// One group of experts sharing a shape: [0] the routed experts, [1] the shared expert.
struct ExpertGroup {
  const uint8_t *blobs;   // blob of expert 0 of the group
  uint64_t stride;        // bytes between consecutive blobs
  int32_t inter;          // I of the group
  uint32_t down_bytes;    // MXFP4: the down matrix's bytes when its tensors are not one blob (an
                          // operator-level projection); 0: the blob's off[4] − off[3]
  uint64_t off[9];        // sub-tensor offsets inside a blob (reference blob layout)
};

struct GemmArgs {
  ExpertGroup grp[2];
  int32_t hidden, experts, top_k, slots;   // slots = top_k + (shared ? 1 : 0)
  int32_t quant, act, expert_bias, group;
  float alpha, limit;
  int32_t ldh;                  // row stride (elements) of h_hi / h_lo; multiple of 64
  int32_t max_work;             // grid rows of work items
  int32_t row_tiles;            // workgroup row tiles along the output dimension
  int32_t xcd_rows;             // persistent prefill: row-tile parts P of the 8 XCDs (1, 2, 4, 8; 0 = 8)
  const uint16_t *x;            // bf16 [T][H]
  const int32_t *order;         // [positions] slot id (t·slots + r) of each permuted position (T > 16)
  const int4 *work;             // [max_work] {expert (E = shared), pos0, n, 0}
  const int32_t *n_work;        // device count of valid work items
  uint16_t *h_hi, *h_lo;        // bf16 [T·slots][ldh]: activation of each slot, hi + lo split
  // MXFP4 (scaled fp4 × fp8 products): the operands as fp8 e4m3 terms with e8m0 block scales.
  const uint8_t *xq, *xs;       // x: [T][NTX][xld] bytes, scales [T][NTX][xld/32]
  uint8_t *hq, *hs;             // h: [T·slots][NTH][hld] bytes, scales [T·slots][NTH][hld/32]
  int32_t xld, hld;             // row lengths (multiples of 128)
  const float *slot_w;          // fp32 [T·slots] routing weight of each slot
  float *slot_out;              // fp32 [T·slots][H] (T > 16)
  float *y;                     // fp32 [T][H] layer output (written directly by the decode path)
  const float *resid;           // fp32 [T][H] residual added to the mixture (y = resid + Σ slots), or null
};

// Decode attention (hh_attn.hip).
struct AttnArgs {
  const float *q;              // [qh][d]
  const uint16_t *k, *v;       // fp16 [rows][kvh][d]
  const uint16_t *sinks;       // bf16 [qh]
  int qh, kvh, d, keys, ring, start, chunks, per_chunk;
  float scale;
  float *pmax, *pden, *pout;   // [qh][chunks], [qh][chunks], [qh][chunks][d]
  float *out;                  // [qh][d]
};
constexpr int kAttnQM = 8;     // most query heads per kv head
constexpr int kAttnMaxChunks = 1024;

struct RouteArgs {
  const uint16_t *x;            // bf16 [T][H] expert input (and shared-gate input)
  const uint16_t *xr;           // bf16 [T][H] router input
  const uint16_t *router_w;     // bf16 [E][H]
  const uint16_t *router_b;     // bf16 [E] or null
  const uint16_t *router_scale; // bf16 [H] (GEMMA)
  const uint16_t *router_pes;   // bf16 [E] (GEMMA)
  const uint16_t *shared_gate;  // bf16 [H] or null
  // MLX-affine router (router_bits 4 or 8; 0 = the bf16 router above): words [E][H·bits/32],
  // scales / biases bf16 [E][H/64]; the shared gate row in the same format (sg_*), or null.
  int32_t router_bits;
  const uint32_t *rq_words;
  const uint16_t *rq_scales, *rq_biases;
  const uint32_t *sg_words;
  const uint16_t *sg_scales, *sg_biases;
  int32_t tokens, hidden, experts, top_k, slots, router, tile_tokens, want_dispatch;
  float eps;
  // FFN block, batches of ≤ 16 tokens with a bf16 router: the router kernel forms the layer input
  // itself from the fp32 residual stream, rmsnorm(resid)·norm_w rounded to bf16 (norm_row_bf16),
  // and writes it to xn_out for the expert products (non-MXFP4 layers); null otherwise.
  const float *resid;
  const uint16_t *norm_w;
  float norm_eps;
  int32_t norm_pow;
  uint16_t *xn_out;
  double *logits;               // fp64 [T][K] exact logits of the selected experts, or null
  double *lg64;                 // fp64 [T][E+1] exact logits (batches of ≤ 16 tokens, or any batch with an MLX router; column E: shared gate)
  uint8_t *xq, *xs;             // MXFP4 layers: x as fp8 terms (GemmArgs::xq), or null
  int32_t xld;
  float *lg32;                  // fp32 [T][E] screening logits (batches above 16 tokens)
  float *wn;                    // fp32 [E] router row norms
  int32_t *topk_idx;            // [T][K]
  float *topk_w;                // [T][K]
  float *slot_w;                // [T·slots]
  float *shared_w;              // [T] or null
  // dispatch outputs
  int32_t *seg;                 // [E+2] segment offsets (routed experts, then shared)
  int32_t *order;               // [positions]
  int4 *work;                   // [max_work]
  int32_t *n_work;              // [1]
  int32_t max_work;
  // Optional (null: not written): the same routed segments in items of tile_tokens / 2 tokens,
  // for a down phase with half the gate-up's token tile (no shared expert).
  int4 *work_half;              // [max_work_half]
  int32_t *dcount;              // [dispatch blocks][E]: per-block expert counts (multi-block dispatch)
  int32_t *n_work_half;         // [1]
  int32_t max_work_half;
};

// The kernel's argument block into the scalar cache in one round: one dword of each 64-byte line
// is read at entry and the reads are awaited together. Otherwise each field is read where it is
// first used, and every line's first touch is a round trip of its own on a cold compute unit
// (the argument reads of a decode kernel form chains of several).
template <size_t BYTES> __device__ __forceinline__ void warm_kernargs() {
  const uint32_t *k = (const uint32_t *)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t x = 0;
#pragma unroll
  for (size_t i = 0; i < (BYTES + 63) / 64; ++i) x ^= k[16 * i];
  __builtin_amdgcn_sched_barrier(0);   // nothing that waits on a field is scheduled among the reads
  asm volatile("" ::"s"(x));
  __builtin_amdgcn_sched_barrier(0);
}

// Optional profiling events of a launch sequence: `start` is attached to the first kernel's
// dispatch packet and `stop` to the last one's (hipExtLaunchKernelGGL), so the interval covers
// exactly the kernels' execution, as a kernel trace would. Null events launch normally.
// Cache policy of device-scope buffer loads and stores on gfx950 (the sc1 bit): a load misses in
// caches that are not coherent across the device, a store completes once it is visible across
// the device. Data exchanged between workgroups of one launch moves this way.
constexpr int kDevScope = 16;

// Fused decode (one launch per MXFP4 layer), see decode_mx.
struct FuseArgs {
  uint32_t *flags;    // [R] router workgroups, then the gate-up items
  uint32_t *status;   // bit 0: a wait timed out
  uint32_t epoch;     // this call's flag value (never repeats for a buffer)
  uint32_t seq;       // one-launch decode: the context's count of earlier one-launch calls
  uint32_t *ctr;      // one-launch decode: the two counter regions (2·64 words)
  int32_t R, U, D;    // workgroups per role
};

struct Timing {
  hipEvent_t start = nullptr, stop = nullptr;
};

}  // namespace hh
