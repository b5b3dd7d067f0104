// hh_gemm.hip — grouped expert products on gfx950 MFMA, shared by decode and prefill.
//
// Two products per layer:
//   PH_UP   : h[s][i] = act(gate_i · x_t + b, up_i · x_t + b) for every slot s = t·slots + r
//             (token t, rank r; rank `top_k` is the shared expert), stored as bf16 hi + lo so
//             the down product sees the fp32 activation to ~2^-17 relative;
//   PH_DOWN : slot value w(t, r) · (down_j · h[s] + b_j); the slots of a token are summed in rank
//             order into y.
//
// Canonical arithmetic. Every output element (row j, slot s) is TWO accumulation chains over the
// K dimension, summed at the end (acc_even + acc_odd): chain p takes the chunks c ≡ p (mod 2) in
// increasing order, each chunk a fixed sequence of v_mfma_f32_16x16x32_bf16 steps (MXFP4/BF16:
// 128-column chunks, 4 steps; MLX: one 64-column affine group, 2 steps into a group partial P,
// then acc = fma(s, P, acc), acc = fma(b, Σx, acc)). Two chains halve the dependent-MFMA latency
// of a decode wave, which owns a single 16-row tile. Decode and prefill kernels differ only in
// how rows and tokens are tiled over waves and how the B operand reaches the registers; each
// output element sees the same MFMA sequence with the same operands, so a T-token call equals
// T one-token calls bit for bit. No split-K across waves, no atomics.
//
// Kernels:
//   up_small / down_small (T ≤ 16, decode): up_small selects the top-k itself from the exact
//     fp64 logits (every workgroup redundantly, hh_select.hpp), takes the u-th distinct expert of
//     the batch (in order of first appearance in the (token, rank) table), and computes 32
//     intermediates of it for all its tokens: 4 waves = {gate, up} × 2 tiles of 16 rows, each
//     wave issuing its whole weight stream at once (one 16-byte load per lane per chunk), the
//     tokens' x rows staged in LDS. down_small computes 16 hidden rows of one token for all of
//     its slots (one wave per slot) and sums them in rank order in the epilogue: no slot buffer,
//     no combine launch.
//   prefill_gemm (T > 16): a work list of (expert, first position, ≤ 16·NT tokens) from the
//     device-side dispatch; 4 waves on different row tiles share the B chunk staged in LDS;
//     slot values go to slot_out and combine_kernel sums them in rank order.
//
// MFMA operand mapping (16x16x32, lane l, lane group g = l/16): A lane l supplies row l%16,
// B lane l supplies token column l%16, each with 8 consecutive K values; D lane l holds rows
// 4g..4g+3 of column l%16. The K slots are assigned per format:
//   MXFP4, BF16: chunk c of 128 columns; MFMA step v∈0..3 takes lane group g's columns
//                128c + 32g + 8v .. +8 (g's 16-byte MXFP4 block 4c+g, or its 64 bytes of bf16)
//   MLX4/MLX8  : chunk c = affine group c (64 columns); step v∈0..1 takes columns
//                64c + 16g + 8v .. +8, so both steps stay inside one group and the affine
//                factorisation s·Σq·x + b·Σx applies per group.
//
// Reference kernels replaced: mxfp4_gemv_vectorized (mxfp4.metal:119), mxfp4_gemm_gathered /
// mxfp4_gemm_tiled (batch.metal:96, tiled.metal:127), bf16_gemv (dense.metal:14),
// mlx_affine_gemv_t / mlx_affine_gemm_t (gemma.metal:248, :460), swiglu(_batch),
// qwen_silu_multiply, gelu_mul, write_expert_scaled, scatter_expert(_scaled), sum_expert_slices.
#include "hh_common.hpp"
#include "hh_select.hpp"
#include "hh_logit.hpp"

#include <algorithm>
#include <type_traits>
#include <mutex>
#include <vector>

namespace hh {

enum { PH_UP = 0, PH_DOWN = 1 };

__device__ __forceinline__ f32x4 mfma(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Two unsigned integers < 256 → packed bf16 pair (exact: 8 significant bits).
__device__ __forceinline__ uint32_t u8pair_to_bf16x2(uint32_t lo, uint32_t hi) {
  uint32_t a = __float_as_uint((float)lo), b = __float_as_uint((float)hi);
  return (a >> 16) | (b & 0xFFFF0000u);
}

// 8 4-bit MLX values of one word (low-order first) → bf16 integers.
__device__ __forceinline__ bf16x8 mlx4_to_bf16(uint32_t w) {
  u32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    r[k] = u8pair_to_bf16x2((w >> (8 * k)) & 0xF, (w >> (8 * k + 4)) & 0xF);
  return as_bf16x8(r);
}

// 8 8-bit MLX values of two words → bf16 integers.
__device__ __forceinline__ bf16x8 mlx8_to_bf16(uint32_t w0, uint32_t w1) {
  u32x4 r = {u8pair_to_bf16x2(w0 & 0xFF, (w0 >> 8) & 0xFF),
             u8pair_to_bf16x2((w0 >> 16) & 0xFF, w0 >> 24),
             u8pair_to_bf16x2(w1 & 0xFF, (w1 >> 8) & 0xFF),
             u8pair_to_bf16x2((w1 >> 16) & 0xFF, w1 >> 24)};
  return as_bf16x8(r);
}

template <int FMT> struct Fmt;

// ---- MXFP4: 128-column chunks, one 16-byte block per lane -----------------------------------
template <> struct Fmt<Q_MXFP4> {
  static constexpr int CHUNK = 128, NB = 4;  // B vectors (16 B) per lane per chunk
  struct A { u32x4 w; uint32_t s; };
  struct Row { const uint8_t *w; const uint8_t *s; };
  __device__ static Row row(const uint8_t *blocks, const uint8_t *scales, int r, int K) {
    return {blocks + (size_t)r * (K / 2), scales + (size_t)r * (K / 32)};
  }
  __device__ static void load(A &a, const Row &rw, int c, int g, int K) {
    int kb = min(4 * c + g, K / 32 - 1);
    a.w = *(const u32x4 *)(rw.w + kb * 16);
    a.s = rw.s[kb];
  }
  __device__ static int bcol(int c, int g, int K) { return min(128 * c + 32 * g, K - 32); }
  __device__ static bool lane_valid(int c, int g, int K) { return 128 * c + 32 * g < K; }
};

// ---- MXFP4 blocks without their scales (decode kernels stage a tile's scales in LDS) ----------
constexpr int Q_MXFP4_W = 4;
// Rows are read through a buffer resource over the whole weight matrix of the expert: the lane's
// row offset is computed once and a chunk's offset (64 bytes per chunk) goes into the
// instruction's immediate field, so a stream of chunks costs no address registers. Chunks are
// not clamped: a lane past K reads the next row (its weights are zeroed by lane_valid) and reads
// past the matrix return zeros. Streams of this format walk K with stride 1.
template <> struct Fmt<Q_MXFP4_W> {
  static constexpr int CHUNK = 128, NB = 4;
  struct A { u32x4 w; };
  struct Row {
    __amdgpu_buffer_rsrc_t rs;
    int voff;   // row · K/2 + 16·(lane group): the lane's block of chunk 0
  };
  __device__ static Row row(const uint8_t *matrix, uint64_t bytes, int r, int K) {
    Row rw;
    rw.rs = __builtin_amdgcn_make_buffer_rsrc((void *)matrix, (short)0, (int)bytes, 0x00020000);
    rw.voff = r * (K / 2) + 16 * ((threadIdx.x & 63) >> 4);
    return rw;
  }
  __device__ static void load(A &a, const Row &rw, int c, int, int) {
    a.w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw.rs, rw.voff + 64 * c, 0, 0));
  }
  __device__ static bool lane_valid(int c, int g, int K) { return 128 * c + 32 * g < K; }
};

// ---- BF16: 128-column chunks; step v (32 columns) of a chunk holds, in lane (g, l16), row l16's
// columns 128c + 32v + 8g .. +7: a lane's four 16-byte pieces lie 64 bytes apart, so a load of
// one step reads 64 contiguous bytes of each of 16 rows. K is a multiple of 64: a step lies wholly
// inside or wholly past K, and steps past K are skipped (uniformly) by every kernel.
template <> struct Fmt<Q_BF16> {
  static constexpr int CHUNK = 128, NB = 4, VS = 32;   // VS: B columns between steps
  struct A { u32x4 w[4]; };
  struct Row { const uint8_t *w; };
  __device__ static Row row(const uint8_t *base, int r, int K) { return {base + (size_t)r * K * 2}; }
  __device__ static void load(A &a, const Row &rw, int c, int g, int K) {
#pragma unroll
    for (int s = 0; s < 4; ++s) a.w[s] = *(const u32x4 *)(rw.w + 2 * min(128 * c + 32 * s + 8 * g, K - 8));
  }
  __device__ static int bcol(int c, int g, int) { return 128 * c + 8 * g; }
  __device__ static bool step_ok(int c, int v, int K) { return 128 * c + 32 * v < K; }
};

// ---- MLX affine: 64-column chunks (one group) ------------------------------------------------
// The lane's stage also carries its row's group scale and bias (bf16 pair); the D rows' values
// are fetched from the lanes of those rows by shuffle (affine_sb).
template <int BITS> struct FmtMLX {
  static constexpr int CHUNK = 64, NB = 2, VS = 8;
  struct A { uint32_t w[BITS / 2]; uint32_t sb; };  // 4-bit: 2 words (16 values); 8-bit: 4 words
  struct Row { const uint8_t *w; const uint16_t *sc, *bi; };
  __device__ static Row row(const uint8_t *words, const uint8_t *scales, const uint8_t *biases,
                            int r, int K) {
    return {words + (size_t)r * (K * BITS / 8), (const uint16_t *)scales + (size_t)r * (K / 64),
            (const uint16_t *)biases + (size_t)r * (K / 64)};
  }
  __device__ static void load(A &a, const Row &rw, int c, int g, int K) {
    const uint8_t *p = rw.w + (64 * c + 16 * g) * BITS / 8;
    if constexpr (BITS == 4) {
      u32x2 v = *(const u32x2 *)p;
      a.w[0] = v[0]; a.w[1] = v[1];
    } else {
      u32x4 v = *(const u32x4 *)p;
      a.w[0] = v[0]; a.w[1] = v[1]; a.w[2] = v[2]; a.w[3] = v[3];
    }
    a.sb = (uint32_t)rw.sc[c] | ((uint32_t)rw.bi[c] << 16);
  }
  // The codes only (the group's scale and bias come from elsewhere: MlxSb).
  __device__ static void load_w(A &a, const Row &rw, int c, int g, int K) {
    const uint8_t *p = rw.w + (64 * c + 16 * g) * BITS / 8;
    if constexpr (BITS == 4) {
      u32x2 v = *(const u32x2 *)p;
      a.w[0] = v[0]; a.w[1] = v[1];
    } else {
      u32x4 v = *(const u32x4 *)p;
      a.w[0] = v[0]; a.w[1] = v[1]; a.w[2] = v[2]; a.w[3] = v[3];
    }
    a.sb = 0u;
  }
  __device__ static bf16x8 decode(const A &a, int j) {
    if constexpr (BITS == 4) return mlx4_to_bf16(a.w[j]);
    else return mlx8_to_bf16(a.w[2 * j], a.w[2 * j + 1]);
  }
  __device__ static int bcol(int c, int g, int) { return 64 * c + 16 * g; }
};
template <> struct Fmt<Q_MLX4> : FmtMLX<4> {};
template <> struct Fmt<Q_MLX8> : FmtMLX<8> {};

template <int FMT> constexpr bool is_mlx() { return FMT == Q_MLX4 || FMT == Q_MLX8; }

// ---- shared pieces of the canonical arithmetic -------------------------------------------------

// Sum of 8 bf16 values of one 16-byte vector, in index order.
__device__ __forceinline__ float sum8_bf16(const u32x4 &v) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    s += bf16_bits_to_f32(v[k] & 0xFFFF);
    s += bf16_bits_to_f32(v[k] >> 16);
  }
  return s;
}

// One 16-row A tile of a wave: the lane's weight row.
template <int FMT> struct ATile {
  typename Fmt<FMT>::Row row;
};

// Tiles of a wave whose first output row is rb: PH_UP takes RT gate tiles then RT up tiles of
// intermediates rb + 16q, PH_DOWN RT tiles of hidden rows rb + 16q. Rows past out_dim are
// clamped into the matrix (their results are never stored).
// One 16-row A tile: output rows r0 .. r0+15 (lane l16 takes r0 + l16); PH_UP picks the gate
// (is_up false) or the up matrix.
template <int PH, int FMT>
__device__ __forceinline__ ATile<FMT> tile_of(const uint8_t *blob, const ExpertGroup &grp, int r0, bool is_up,
                                              int K, int l16) {
  ATile<FMT> t;
  const int orow = r0 + l16;
  const int I = grp.inter;
  if constexpr (FMT == Q_MXFP4) {
    // GPT-OSS gate_up rows interleave gate and up (ReferenceLayer.swift:11).
    if (PH == PH_UP) t.row = Fmt<FMT>::row(blob + grp.off[0], blob + grp.off[1], 2 * orow + (is_up ? 1 : 0), K);
    else t.row = Fmt<FMT>::row(blob + grp.off[3], blob + grp.off[4], orow, K);
  } else if constexpr (FMT == Q_MXFP4_W) {
    // The matrix extends to the next sub-tensor of the blob (its scales).
    if (PH == PH_UP) t.row = Fmt<FMT>::row(blob + grp.off[0], grp.off[1] - grp.off[0], 2 * orow + (is_up ? 1 : 0), K);
    else t.row = Fmt<FMT>::row(blob + grp.off[3], grp.down_bytes ? grp.down_bytes : grp.off[4] - grp.off[3], orow, K);
  } else if constexpr (FMT == Q_BF16) {
    // Gemma gate_up: gate = rows 0..I-1, up = rows I..2I-1 (Gemma4Weights.swift:107-112).
    if (PH == PH_UP) t.row = Fmt<FMT>::row(blob + grp.off[0], orow + (is_up ? I : 0), K);
    else t.row = Fmt<FMT>::row(blob + grp.off[1], orow, K);
  } else {
    const int mat = (PH == PH_UP) ? (is_up ? 1 : 0) : 2;
    t.row = Fmt<FMT>::row(blob + grp.off[3 * mat], blob + grp.off[3 * mat + 1], blob + grp.off[3 * mat + 2],
                          orow, K);
  }
  return t;
}

template <int PH, int FMT, int RT>
__device__ __forceinline__ void wave_tiles(ATile<FMT> (&t)[(PH == PH_UP ? 2 : 1) * RT],
                                           const uint8_t *blob, const ExpertGroup &grp, int rb,
                                           int out_dim, int K, int l16) {
  constexpr int NM = (PH == PH_UP ? 2 : 1) * RT;
#pragma unroll
  for (int m = 0; m < NM; ++m)
    t[m] = tile_of<PH, FMT>(blob, grp, min(rb + 16 * (m % RT), out_dim - 16), (PH == PH_UP) && (m >= RT), K, l16);
}

// The MFMA sequence of chunk c for NM A tiles × NT token tiles. `bv(st, hh, v)` returns the
// lane's 8 B values of token tile st, term hh (x | h_hi, h_lo), step v, at columns
// Fmt::bcol(c, g, K) + 8v.
// MLX: `sbf(m)`, when given, returns the (scale | bias << 16) words of D rows 4g .. 4g+3 of tile m
// for this chunk; otherwise they come from the A operands' rows by shuffles.
template <int FMT, int NM, int NT, int NH, class BV, class SBF = std::nullptr_t>
__device__ __forceinline__ void chunk_mfma(f32x4 (&acc)[NM][NT], const typename Fmt<FMT>::A (&w)[NM],
                                           const ATile<FMT> (&at)[NM], BV bv, int c, int g, int K,
                                           SBF sbf = nullptr) {
  using F = Fmt<FMT>;
  if constexpr (FMT == Q_BF16) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (!F::step_ok(c, v, K)) break;
      u32x4 b[NT][NH];
#pragma unroll
      for (int st = 0; st < NT; ++st)
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) b[st][hh] = bv(st, hh, v);
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int st = 0; st < NT; ++st)
#pragma unroll
          for (int hh = 0; hh < NH; ++hh) acc[m][st] = mfma(as_bf16x8(w[m].w[v]), as_bf16x8(b[st][hh]), acc[m][st]);
    }
  } else if constexpr (!is_mlx<FMT>()) {
    const bool ok = F::lane_valid(c, g, K);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      u32x4 b[NT][NH];
#pragma unroll
      for (int st = 0; st < NT; ++st)
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) b[st][hh] = bv(st, hh, v);
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        bf16x8 av;
        av = mxfp4_to_bf16(ok ? w[m].w[v] : 0u, e8m0_to_f32(w[m].s));
#pragma unroll
        for (int st = 0; st < NT; ++st)
#pragma unroll
          for (int hh = 0; hh < NH; ++hh) acc[m][st] = mfma(av, as_bf16x8(b[st][hh]), acc[m][st]);
      }
    }
  } else {
    // MLX affine, one 64-column group: P = Σ q·x on the bf16 MFMA (steps v = 0, 1: word v of the
    // lane's codes), G = Σ x on the MFMA with an all-ones A operand (every row of its D holds the
    // column sums, so each lane gets its column's), then acc += s·P + b·G per D row
    // (gemma.metal:234-236's factorisation). 4-bit codes enter the MFMA as bf16 (128 + q), two
    // per instruction pair: ((w >> 4k) & 0x000F000F) | 0x43004300 holds codes k and k+4, so the
    // B values are paired the same way (x_k, x_{k+4}) and the 128·G term goes into the bias:
    // acc += s·P' + (b − 128·s)·G.
    u32x4 b[NT][NH][2];
#pragma unroll
    for (int st = 0; st < NT; ++st)
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          const u32x4 raw = bv(st, hh, v);
          if constexpr (FMT == Q_MLX4) {
            // (x0,x1)(x2,x3)(x4,x5)(x6,x7) → (x0,x4)(x1,x5)(x2,x6)(x3,x7)
            b[st][hh][v] = u32x4{__builtin_amdgcn_perm(raw[2], raw[0], 0x05040100u),
                                 __builtin_amdgcn_perm(raw[2], raw[0], 0x07060302u),
                                 __builtin_amdgcn_perm(raw[3], raw[1], 0x05040100u),
                                 __builtin_amdgcn_perm(raw[3], raw[1], 0x07060302u)};
          } else {
            b[st][hh][v] = raw;
          }
        }
    f32x4 P[NM][NT], G[NT];
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      G[st] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < NM; ++m) P[m][st] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};   // bf16 1.0
#pragma unroll
    for (int v = 0; v < 2; ++v) {
#pragma unroll
      for (int st = 0; st < NT; ++st)
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) G[st] = mfma(as_bf16x8(ones), as_bf16x8(b[st][hh][v]), G[st]);
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        bf16x8 av;
        if constexpr (FMT == Q_MLX4) {
          const uint32_t wv = w[m].w[v];
          u32x4 r;
#pragma unroll
          for (int k = 0; k < 4; ++k) r[k] = ((wv >> (4 * k)) & 0x000F000Fu) | 0x43004300u;
          av = as_bf16x8(r);
        } else {
          av = F::decode(w[m], v);
        }
#pragma unroll
        for (int st = 0; st < NT; ++st)
#pragma unroll
          for (int hh = 0; hh < NH; ++hh) P[m][st] = mfma(av, as_bf16x8(b[st][hh][v]), P[m][st]);
      }
    }
    // D row 4g + ii is the A row of lane 4g + ii: its scale and bias by shuffle (all four
    // shuffles issued before the first is used).
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      uint32_t sbs[4];
      if constexpr (std::is_same_v<SBF, std::nullptr_t>) {
        const int sbl = (int)w[m].sb;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) sbs[ii] = (uint32_t)__shfl(sbl, 4 * g + ii);
      } else {
        const u32x4 v = sbf(m);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) sbs[ii] = v[ii];
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const uint32_t sbv = sbs[ii];
        const float sc = bf16_bits_to_f32(sbv & 0xFFFF);
        const float bi0 = bf16_bits_to_f32(sbv >> 16);
        const float bi = FMT == Q_MLX4 ? __builtin_fmaf(-128.f, sc, bi0) : bi0;
#pragma unroll
        for (int st = 0; st < NT; ++st) {
          acc[m][st][ii] = __builtin_fmaf(sc, P[m][st][ii], acc[m][st][ii]);
          acc[m][st][ii] = __builtin_fmaf(bi, G[st][ii], acc[m][st][ii]);
        }
      }
    }
  }
}

// Weight stream of one wave over its chunks c = c0, c0 + cs, c0 + 2·cs, ... < nch with a DA-deep
// register ring: the A operand of the next DA chunks is in flight while a chunk is computed; a
// wave with at most DA chunks issues its whole stream at once. The loop body is instantiated DA
// times. Refills are issued only when another round follows (a round's refills past the last
// chunk reload it, clamped, so the rounds before the last need no per-load test): a duplicate
// load costs as much of the address/L1 path as a real one.
template <int FMT> constexpr bool unit_stride() { return FMT == Q_MXFP4_W; }
// NOSB (MLX): the stream carries the codes only; the scales and biases are staged (MlxSb).
template <int FMT, int NM, int DA, bool NOSB = false> struct AStream {
  typename Fmt<FMT>::A s[DA][NM];
  int c0, cs, n;   // first chunk, chunk stride, chunks of this wave
  __device__ __forceinline__ AStream(int first, int stride, int nch)
      : c0(first), cs(stride), n(nch > first ? (nch - first + stride - 1) / stride : 0) {}
  __device__ __forceinline__ void load(int slot, const ATile<FMT> (&at)[NM], int i, int nch, int g, int K) {
    int c;
    if constexpr (unit_stride<FMT>()) c = c0 + i;
    else c = min(c0 + cs * min(i, max(n - 1, 0)), nch - 1);
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      if constexpr (NOSB) Fmt<FMT>::load_w(s[slot][m], at[m].row, c, g, K);
      else Fmt<FMT>::load(s[slot][m], at[m].row, c, g, K);
    }
  }
  // The first P (default: all DA) stages; run_pf<ONE, P> issues the rest as it goes.
  template <int P = DA> __device__ __forceinline__ void fill(const ATile<FMT> (&at)[NM], int nch, int g, int K) {
#pragma unroll
    for (int u = 0; u < P; ++u) load(u, at, u, nch, g, K);
  }
  // Runs this wave's chunks through `body(stage, c)`.
  template <class Body>
  __device__ __forceinline__ void run(const ATile<FMT> (&at)[NM], int nch, int g, int K, Body body) {
    for (int i0 = 0; i0 < n; i0 += DA) {
      const bool more = i0 + DA < n;
#pragma unroll
      for (int u = 0; u < DA; ++u) {
        if (i0 + u < n) body(s[u], c0 + cs * (i0 + u));
        if (more) load(u, at, i0 + u + DA, nch, g, K);
      }
    }
  }
  // As run, with the chunk's other operands read one chunk ahead: `pre(c)` issues them (LDS
  // reads) and `body(stage, c, ops)` consumes them, so each chunk's operand latency hides behind
  // the previous chunk's MFMAs. A wave whose chunks fit the ring (n ≤ DA) runs straight-line code
  // without refills, which keeps every weight wait exact (a refill inside the loop forces
  // conservative waits).
  // ONE: the caller guarantees one round from chunk 0 with stride 1 (n ≤ DA, c0 = 0, cs = 1), and
  // only that code is generated.
  // P < DA (ONE only): the stream was filled with its first P chunks and chunk u + P is issued
  // after chunk u is computed, so at most P loads of the wave are in flight. The memory system
  // returns a saturating stream at the rate it accepts new loads, so the later chunks' data is
  // not delayed, while the MFMAs of the early chunks overlap the stream and the workgroup's
  // staging barrier (before the first chunk) waits only for loads issued ahead of it.
  // NC > 0 (ONE only): the stream's chunk count is NC, known at compile time, so the per-chunk
  // guards vanish and the unrolled chunks form one straight block (no register copies at merges).
  template <bool ONE = false, int P = DA, int NC = 0, class Pre, class Body>
  __device__ __forceinline__ void run_pf(const ATile<FMT> (&at)[NM], int nch, int g, int K, Pre pre, Body body) {
    static_assert(P == DA || ONE, "a partial fill needs the single-round stream");
    static_assert(NC == 0 || (ONE && NC <= DA), "a static chunk count needs the single-round stream");
    if (n <= 0) return;
    if constexpr (ONE) {
      rounds<true, true, P, NC>(at, nch, g, K, pre, body);
    } else {
      if (n <= DA && c0 == 0 && cs == 1) rounds<true, true>(at, nch, g, K, pre, body);
      else if (n <= DA) rounds<true, false>(at, nch, g, K, pre, body);
      else rounds<false, false>(at, nch, g, K, pre, body);
    }
  }
  // One round of NC chunks at this wave's first chunk and stride, NC known at compile time (the
  // caller guarantees n == NC ≤ DA): every chunk's wait is exact. The first P chunks were issued
  // by fill<P>; chunk u + P is issued after chunk u is computed.
  // `pre(c)` / `body(stage, c, ops)` as in run_pf.
  template <int NC, int P = DA, class Pre, class Body>
  __device__ __forceinline__ void run_static(const ATile<FMT> (&at)[NM], int nch, int g, int K, Pre pre, Body body) {
    static_assert(NC > 0 && NC <= DA && P <= NC, "a static single round");
    rounds<true, false, P, NC>(at, nch, g, K, pre, body);
  }
  // UNIT: chunk u of the ring is chunk u of K (one round, first chunk 0, stride 1), so chunk
  // indices, and the operand offsets derived from them, are compile-time constants.
  template <bool ONE, bool UNIT, int P = DA, int NC = 0, class Pre, class Body>
  __device__ __forceinline__ void rounds(const ATile<FMT> (&at)[NM], int nch, int g, int K, Pre pre, Body body) {
    auto op = pre(UNIT ? 0 : c0);
    for (int i0 = 0; i0 < n; i0 += DA) {
      const bool more = !ONE && i0 + DA < n;
#pragma unroll
      for (int u = 0; u < DA; ++u) {
        if (NC > 0 ? u < NC : i0 + u < n) {
          const int cn = UNIT ? min(u + 1, DA - 1) : c0 + cs * min(i0 + u + 1, n - 1);
          const auto nx = pre(cn);
          body(s[u], UNIT ? u : c0 + cs * (i0 + u), op);
          op = nx;
        }
        if constexpr (P < DA) {
          if (u + P < (NC > 0 ? NC : DA)) load(u + P, at, u + P, nch, g, K);
        }
        if (more) load(u, at, i0 + u + DA, nch, g, K);
      }
      if (ONE) break;
    }
  }
};

// acc = p0 + p1 per element (the two chains of the canonical arithmetic).
__device__ __forceinline__ f32x4 sum_chains(const f32x4 &p0, const f32x4 &p1) {
  f32x4 r;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) r[ii] = p0[ii] + p1[ii];
  return r;
}

// Activations of 4 intermediates i0..i0+3: bias (GPT-OSS gate_up bias, interleaved like the
// rows) and the gated activation.
template <int FMT>
__device__ __forceinline__ f32x4 up_values(const GemmArgs &a, const uint8_t *blob, const ExpertGroup &grp,
                                           int i0, const f32x4 &gate, const f32x4 &up) {
  float gb[4] = {0.f, 0.f, 0.f, 0.f}, ub[4] = {0.f, 0.f, 0.f, 0.f};
  if (FMT == Q_MXFP4 && a.expert_bias) {
    const uint16_t *bias = (const uint16_t *)(blob + grp.off[2]);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      gb[ii] = bf16_bits_to_f32(bias[2 * (i0 + ii)]);
      ub[ii] = bf16_bits_to_f32(bias[2 * (i0 + ii) + 1]);
    }
  }
  float gv[4], uv[4], yv[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    gv[ii] = gate[ii] + gb[ii];
    uv[ii] = up[ii] + ub[ii];
  }
  activate_n<4>(a.act, gv, uv, yv, a.alpha, a.limit);
  return f32x4{yv[0], yv[1], yv[2], yv[3]};
}

// up_values with the GPT-OSS bias of the 4 intermediates already loaded: 16 bytes from the bias
// row at element 2·i0, (gate, up) bf16 pairs in order.
__device__ __forceinline__ f32x4 up_values_mx(const GemmArgs &a, const u32x4 &bias, const f32x4 &gate,
                                              const f32x4 &up) {
  float gv[4], uv[4], yv[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    gv[ii] = gate[ii] + bf16_bits_to_f32(bias[ii] & 0xFFFFu);
    uv[ii] = up[ii] + bf16_bits_to_f32(bias[ii] >> 16);
  }
  activate_n<4>(a.act, gv, uv, yv, a.alpha, a.limit);
  return f32x4{yv[0], yv[1], yv[2], yv[3]};
}

// Gate-up epilogue of 4 intermediates i0..i0+3 of slot `slot`: bias, activation, bf16 hi/lo.
template <int FMT>
__device__ __forceinline__ void up_epilogue(const GemmArgs &a, const uint8_t *blob,
                                            const ExpertGroup &grp, int i0, int slot,
                                            const f32x4 &gate, const f32x4 &up) {
  const f32x4 yv = up_values<FMT>(a, blob, grp, i0, gate, up);
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const float y = yv[ii];
    hi[ii] = f32_to_bf16_bits(y);
    lo[ii] = f32_to_bf16_bits(y - bf16_bits_to_f32(hi[ii]));
  }
  const size_t o = (size_t)slot * a.ldh + i0;
  *(u32x2 *)(a.h_hi + o) = u32x2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
  *(u32x2 *)(a.h_lo + o) = u32x2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
}

// Slot values of hidden rows h0..h0+3: routing weight × (product + bias)
// (write_expert_scaled, dense.metal:131-145).
template <int FMT>
__device__ __forceinline__ f32x4 down_value(const GemmArgs &a, const uint8_t *blob,
                                            const ExpertGroup &grp, int h0, int slot,
                                            const f32x4 &r) {
  const float w = a.slot_w[slot];
  float db[4] = {0.f, 0.f, 0.f, 0.f};
  if (FMT == Q_MXFP4 && a.expert_bias) {
    const uint16_t *bias = (const uint16_t *)(blob + grp.off[5]);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) db[ii] = bf16_bits_to_f32(bias[h0 + ii]);
  }
  f32x4 o;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) o[ii] = w * (r[ii] + db[ii]);
  return o;
}

// Prefill block order: hardware places block b on XCD b % 8. XCD x takes the row tiles
// [x·rtx, x·rtx + rtx) (rtx = ⌈row_tiles / 8⌉) and walks the work items in order, an item's row
// tiles consecutively: the item's activation operand is fetched about once per XCD and reused
// from its L2 by the item's row tiles, and an expert's weight rows by its consecutive items.
// (Row-tile-major order re-read every item's operand from HBM once per row tile.)
__device__ __forceinline__ void prefill_tile(int b, int row_tiles, int &rt, int &wi) {
  const int rtx = (row_tiles + 7) >> 3;
  const int x = b & 7, j = b >> 3;
  wi = j / rtx;
  rt = x * rtx + (j - wi * rtx);
}

// Copies vectors v ∈ [base, base + threads·NB) ∩ [0, n) with `threads` threads (thread index
// `id`): the loads of the batch are all issued before any store, so a batch costs one memory
// latency (a load-store loop would wait for each load in turn, and, completion being in order,
// for every load issued before it).
template <int NB, class Src, class Dst>
__device__ __forceinline__ void stage_batch(int base, int id, int threads, int n, Src src, Dst dst) {
  u32x4 r[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const int v = base + id + threads * k;
    if (v < n) r[k] = src(v);
  }
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const int v = base + id + threads * k;
    if (v < n) dst(v, r[k]);
  }
}

// Development timeline (built only with -DHH_TRACE): per workgroup, wall-clock stamps (100 MHz)
// at fixed points of the decode kernels, [kernel][block][point]; the last call's values.
#ifdef HH_TRACE
constexpr int kTraceBlocks = 4096, kTracePoints = 8;
static __device__ uint64_t hh_trace_buf[3 * kTraceBlocks * kTracePoints];
#define HH_TR(kern, point)                                                                     \
  do {                                                                                         \
    if (threadIdx.x == 0 && blockIdx.x < kTraceBlocks)                                         \
      hh_trace_buf[((kern) * kTraceBlocks + blockIdx.x) * kTracePoints + (point)] = wall_clock64(); \
  } while (0)
// Per-step stamps (core clock) of MFMA wave 0 of workgroup 0 of the MXFP4 prefill gate-up:
// hh_trace_buf[2][step][point], steps < kTraceBlocks.
#define HH_TRS(step, point)                                                                      \
  do {                                                                                           \
    if (threadIdx.x == 0 && blockIdx.x == 0 && (step) < kTraceBlocks)                            \
      hh_trace_buf[(2 * kTraceBlocks + (step)) * kTracePoints + (point)] = clock64();            \
  } while (0)
#else
#define HH_TR(kern, point) do {} while (0)
#define HH_TRS(step, point) do {} while (0)
#endif

// ---- decode prologue -----------------------------------------------------------------------------
// Every decode gate-up workgroup selects the top-k of every token of the batch itself from the
// exact fp64 logits (wave w: tokens w, w + NW, ...) into s_idx [T][K], so the decode step needs no
// selection or dispatch launch; workgroup 0 also writes the routing outputs.
template <int NW>
__device__ __forceinline__ void select_batch(const GemmArgs &a, const RouteArgs &ra, int *s_idx) {
  __shared__ double s_lg[NW][64];
  __shared__ int s_ri[NW][kMaxTopK];
  __shared__ int s_ci[NW][kFastCand];
  __shared__ double s_cv[NW][kFastCand];
  __shared__ double s_rv[NW][kMaxTopK];
  __shared__ int s_rk[NW][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int T = ra.tokens, E = a.experts, K = a.top_k;
  const bool has_shared = a.slots > K;
  if (T == 1 || (T == 2 && NW % 2 == 0)) {
    // One or two tokens: groups of NW / T waves rank a token together; the group's first wave
    // publishes.
    constexpr int G1 = NW, G2 = NW / 2 > 0 ? NW / 2 : 1;
    const int G = T == 1 ? G1 : G2, t = wave / G;
    const double *lg = ra.lg64 + (size_t)t * (E + 1);
    TopK tk = T == 1 ? (E <= 64 ? topk_rank64<G1>(lg, E, K, s_lg[wave], s_ri[wave], s_rk)
                                      : topk_fast<G1>(lg, E, K, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave], s_rk))
                           : (E <= 64 ? topk_rank64<G2>(lg, E, K, s_lg[wave], s_ri[wave], s_rk)
                                      : topk_fast<G2, 1>(lg, E, K, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave], s_rk));
    prob_order(tk, K, ra.router);
    if (wave % G == 0) {
      if (lane < K) s_idx[t * K + lane] = tk.index_of(lane);
      if (blockIdx.x == 0) finish_token(ra, t, tk, has_shared ? lg[E] : 0.0);
    }
  } else {
    for (int t = wave; t < T; t += NW) {
      const double *lg = ra.lg64 + (size_t)t * (E + 1);
      TopK tk = E <= 64 ? topk_rank64(lg, E, K, s_lg[wave], s_ri[wave])
                              : topk_fast(lg, E, K, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave]);
      if (t == wave) HH_TR(1, 5);
      prob_order(tk, K, ra.router);
      if (lane < K) s_idx[t * K + lane] = tk.index_of(lane);
      if (blockIdx.x == 0) finish_token(ra, t, tk, has_shared ? lg[E] : 0.0);
    }
    HH_TR(1, 6);
  }
  __syncthreads();
}

// The j-th set bit of m.
__device__ __forceinline__ int nth_bit(uint64_t m, int j) {
  for (int k = 0; k < j; ++k) m &= m - 1;
  return __ffsll((long long)m) - 1;
}

// The decode plan, computed by every wave in registers from the batch's top-k table s_idx
// [T][K] (LDS): the distinct experts in order of first appearance in (token, rank) order and
// the tokens of each. Lane l holds entries l and 64 + l (T·K ≤ 128).
struct Plan {
  int pe[2];
  bool pf[2];
  uint64_t ptm[2];
  uint64_t m0, m1;
  int n0, nu, E, T;
  __device__ __forceinline__ Plan(const int *s_idx, int T_, int K, int E_) : E(E_), T(T_) {
    const int lane = threadIdx.x & 63, n = T * K;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      pe[h] = lane + 64 * h < n ? s_idx[lane + 64 * h] : -1;
      pf[h] = lane + 64 * h < n;
      ptm[h] = 0ull;
    }
    for (int j = 0, tj = 0, rj = 0; j < n; ++j) {
      const int ej = __builtin_amdgcn_readlane(j < 64 ? pe[0] : pe[1], j & 63);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (ej == pe[h]) {
          if (j < lane + 64 * h) pf[h] = false;
          ptm[h] |= 1ull << tj;
        }
      if (++rj == K) { rj = 0; ++tj; }
    }
    m0 = __ballot(pf[0]);
    m1 = __ballot(pf[1]);
    n0 = __popcll(m0);
    nu = n0 + __popcll(m1);
  }
  // Distinct expert u (< nu) and its token mask; u ≥ nu is the shared expert, every token.
  __device__ __forceinline__ void entry(int u, int &e, uint64_t &tm) const {
    if (u >= nu) {
      e = E;
      tm = (1ull << T) - 1ull;
      return;
    }
    const int h = u < n0 ? 0 : 1;
    const int l = nth_bit(h ? m1 : m0, h ? u - n0 : u);
    const int ev = h ? pe[1] : pe[0];
    const uint64_t tv = h ? ptm[1] : ptm[0];
    e = __builtin_amdgcn_readlane(ev, l);
    tm = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(tv >> 32), l) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tv, l);
  }
  // Plan index of routed expert e (wave-uniform; e must occur in the table).
  __device__ __forceinline__ int index_of(int e) const {
    const uint64_t h0 = __ballot(pf[0] && pe[0] == e), h1 = __ballot(pf[1] && pe[1] == e);
    if (h0) return __popcll(m0 & ((1ull << (__ffsll((unsigned long long)h0) - 1)) - 1ull));
    return n0 + __popcll(m1 & ((1ull << (__ffsll((unsigned long long)h1) - 1)) - 1ull));
  }
};

// Rank of expert e in token t's selection (the shared expert is rank K).
__device__ __forceinline__ int rank_of(const int *s_idx, int t, int e, int K, bool shared) {
  int r = K;
  if (!shared)
    for (int rr = 0; rr < K; ++rr)
      if (s_idx[t * K + rr] == e) r = rr;
  return r;
}

// ---- MLX decode: group scales and biases staged per item ------------------------------------------
// The (scale | bias << 16) word of every (chunk, row) of NTL 16-row tiles in LDS, sb[tile][chunk]
// [row]: lane (g, l16) reads D rows 4g .. 4g+3 of a chunk as one 16-byte vector (chunk_mfma's
// sbf), in place of two 2-byte loads per chunk in every lane of the weight stream and four
// shuffles. `src(tile, kind, row)` is the row's first scale (kind 0) or bias (kind 1). Rows of a
// multiple of 8 chunks come as 16-byte vectors of 8 values (loads issued by mlx_sb_load before
// the weight stream, stored by mlx_sb_store after it); other rows value by value.
// Staged chunks per row (the kernels take the staged variant when K fits, the per-chunk loads
// otherwise): gate-up tiles K ≤ 4096; down tiles K ≤ 4096 with at most 4 slots per workgroup,
// K ≤ 2048 with 9 (a 16-row tile per 64·KS threads).
constexpr int kMlxSbChunks = 64;
template <int SMAX> constexpr int mlx_sb_chunks_down() { return SMAX > 4 ? 32 : 64; }
constexpr int kMlxSbNB = 2;        // 16-byte vectors per thread (NTL · 32 · K/512 ≤ 2 · threads)
template <int NTL, class Src>
__device__ __forceinline__ void mlx_sb_load(u32x4 (&r)[kMlxSbNB], int nch, int tid, int nth, Src src) {
  if (nch & 7) return;
  const int vpr = nch >> 3, n = NTL * 32 * vpr;
#pragma unroll
  for (int k = 0; k < kMlxSbNB; ++k) {
    const int v = min(tid + nth * k, n - 1);
    const int row = (v / vpr) & 15, kind = (v / (16 * vpr)) & 1, tile = v / (32 * vpr);
    r[k] = *(const u32x4 *)(src(tile, kind, row) + 8 * (v % vpr));
  }
}
template <int NTL, int CH, class Src>
__device__ __forceinline__ void mlx_sb_store(const u32x4 (&r)[kMlxSbNB], uint32_t (*sb)[CH][16], int nch,
                                             int tid, int nth, Src src) {
  if ((nch & 7) == 0) {
    const int vpr = nch >> 3, n = NTL * 32 * vpr;
#pragma unroll
    for (int k = 0; k < kMlxSbNB; ++k) {
      const int v = tid + nth * k;
      if (v >= n) break;
      const int row = (v / vpr) & 15, kind = (v / (16 * vpr)) & 1, tile = v / (32 * vpr), c0 = 8 * (v % vpr);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        ((uint16_t *)&sb[tile][c0 + j][row])[kind] = (uint16_t)(r[k][j >> 1] >> (16 * (j & 1)));
    }
  } else {
    for (int v = tid; v < NTL * 32 * nch; v += nth) {
      const int c = v % nch, row = (v / nch) & 15, kind = (v / (16 * nch)) & 1, tile = v / (32 * nch);
      ((uint16_t *)&sb[tile][c][row])[kind] = src(tile, kind, row)[c];
    }
  }
}

// ---- decode: gate-up ----------------------------------------------------------------------------
constexpr int SMALL_T = 16;       // largest batch of the decode kernels
constexpr int UP_ROWS = 32;       // intermediates per up_small workgroup (2 tiles × {gate, up})
constexpr int MX_ONE_CHUNKS = 24; // MXFP4 decode rows of at most this many 128-column chunks stream in one round
#ifndef HH_MX_PF
#define HH_MX_PF 6
#endif
constexpr int MX_PF = HH_MX_PF;   // chunks a single-round MXFP4 decode wave issues before its staging barrier
// The one-token gate-up instantiation issues 10 (measured: T=1 gate-up 15.0 → 14.5 µs; 10 and
// more made the T ≥ 2 kernels and the down kernel slower).
constexpr int MX_PF_T1 = 10;
constexpr int kFusedMaxE = 128;   // experts of layers that take the fused decode kernel
// Batches that take the two-launch decode (the router inside the gate-up launch). Larger batches
// measured no faster (T = 4: 69.3k against 69.1–69.8k tokens/s) or slower (T = 8: 75k against
// 92k): every gate-up workgroup quantises every token's x itself, and the LDS copy of the logits
// leaves fewer workgroups per compute unit.
constexpr int kFusedRouterT = 2;
constexpr int LDS_PAD = 8;        // bf16 elements of padding per staged row (bank spread)

// Persistent: work items (row tile rt of 16·TPW intermediates, u) with u < nu the batch's
// distinct routed experts in order of first appearance in the (token, rank) table and u = nu the
// shared expert when there is one; item it = blockIdx.x, blockIdx.x + gridDim.x, ... Every
// workgroup selects the batch's top-k once (at T = 1 the grid holds one workgroup per item).
// 4·TPW waves: wave w takes tile q (16 intermediates; w & 1 when TPW = 2), gate or up rows, and
// chunk parity p (the even or odd chain of the canonical arithmetic). TPW = 1 gives twice the
// workgroups of half the size, which spreads a decode step's few experts over more compute units.
// SBS (MLX, K ≤ 64·kMlxSbChunks): the group scales and biases staged per item (MlxSb).
// NCW > 0: every wave's stream is exactly NCW chunks (K of 2·NCW chunks, checked on the host), all
// issued before the staging barrier and waited for one by one (DA == NCW).
template <int FMT, int DA, int TPW, int XB, bool SBS = false, int NCW = 0>
__global__ __launch_bounds__(256 * TPW) void up_small(GemmArgs a, RouteArgs ra, FuseArgs) {
  warm_kernargs<sizeof(GemmArgs) + sizeof(RouteArgs) + sizeof(FuseArgs)>();
  constexpr int NTH = 256 * TPW, NWV = 4 * TPW, ROWS = 16 * TPW;
  constexpr int NM = 1;
  extern __shared__ __align__(16) uint16_t s_x[];   // [ntok][H + LDS_PAD]
  __shared__ int s_idx[SMALL_T * kMaxTopK];
  __shared__ f32x4 s_part[3][2][64];                // [gate odd | up even | up odd][q][lane]
  constexpr bool SB = SBS && is_mlx<FMT>();         // MLX: scales and biases staged per item
  __shared__ __align__(16) uint32_t s_sb[SB ? 2 * TPW : 1][SB ? kMlxSbChunks : 1][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int T = ra.tokens, E = a.experts, K = a.top_k, S = a.slots, H = a.hidden;
  const bool has_shared = S > K;

  // Every token's x into LDS (row t), independent of the routing: the first batch of loads
  // (XB vectors per thread) goes out before the selection and is stored with the first item, or,
  // for batches of several tokens, right after the selection (before any weight stream).
  const int ldx = H + LDS_PAD;
  const int per_row = H / 8, nvec = T * per_row;
  auto xsrc = [&](int v) {
    const int t = v / per_row, qq = v - t * per_row;
    return *(const u32x4 *)(a.x + (size_t)t * H + 8 * qq);
  };
  auto xdst = [&](int v, const u32x4 &val) {
    const int t = v / per_row, qq = v - t * per_row;
    *(u32x4 *)(s_x + (size_t)t * ldx + 8 * qq) = val;
  };
  u32x4 xr[XB];
#pragma unroll
  for (int k = 0; k < XB; ++k)
    if (tid + NTH * k < nvec) xr[k] = xsrc(tid + NTH * k);
  HH_TR(1, 0);
  select_batch<NWV>(a, ra, s_idx);
  HH_TR(1, 1);
  const Plan plan(s_idx, T, K, E);
  const int rtr = (a.grp[0].inter + ROWS - 1) / ROWS;
  const int nitems = plan.nu * rtr + (has_shared ? (a.grp[1].inter + ROWS - 1) / ROWS : 0);

  const int q = TPW == 2 ? (wave & 1) : 0;
  const bool is_up = TPW == 2 ? (wave & 2) != 0 : (wave & 1) != 0;
  const int par = TPW == 2 ? wave >> 2 : wave >> 1;
  const int nch = (H + Fmt<FMT>::CHUNK - 1) / Fmt<FMT>::CHUNK;
  bool x_pending = true;
  auto store_x = [&]() {
#pragma unroll
    for (int k = 0; k < XB; ++k)
      if (tid + NTH * k < nvec) xdst(tid + NTH * k, xr[k]);
    for (int base = NTH * XB; base < nvec; base += NTH * 4) stage_batch<4>(base, tid, NTH, nvec, xsrc, xdst);
    x_pending = false;
  };
  if constexpr (XB > 2) store_x();
  for (int it = blockIdx.x; it < nitems; it += gridDim.x) {
    const bool sh = it >= plan.nu * rtr;
    const int u = sh ? plan.nu : it / rtr;
    const int rt = sh ? it - plan.nu * rtr : it % rtr;
    int e;
    uint64_t tm;
    plan.entry(u, e, tm);
    const int ntok = __popcll(tm);
    const ExpertGroup &grp = a.grp[sh ? 1 : 0];
    const uint8_t *blob = grp.blobs + (sh ? 0 : (size_t)e * grp.stride);
    const int rb = rt * ROWS + 16 * q;
    ATile<FMT> at[NM] = {tile_of<PH_UP, FMT>(blob, grp, rb, is_up, H, l16)};
    // MLX tiles: gate rows of tile qq (tile index qq), then up rows (TPW + qq).
    auto sb_src = [&](int tile, int kind, int row) {
      const int mat = tile / TPW, orow = min(rt * ROWS + 16 * (tile % TPW) + row, grp.inter - 1);
      return (const uint16_t *)(blob + grp.off[3 * mat + 1 + kind]) + (size_t)orow * (H / 64);
    };
    u32x4 sbr[kMlxSbNB];
    if constexpr (SB) mlx_sb_load<2 * TPW>(sbr, nch, tid, NTH, sb_src);
    // The weight stream, then (first item) the x stores, which wait for the x loads only, and
    // any further batches, and the staged scales and biases.
    AStream<FMT, NM, DA, SB> as(par, 2, nch);
    as.fill(at, nch, g, H);
    if (x_pending) store_x();
    if constexpr (SB) mlx_sb_store<2 * TPW, kMlxSbChunks>(sbr, s_sb, nch, tid, NTH, sb_src);
    __syncthreads();
    if (it == (int)blockIdx.x) HH_TR(1, 2);

    // Token column l16 = the l16-th token of the expert (padding columns repeat the last one).
    const int my_t = nth_bit(tm, min(l16, ntok - 1));
    const uint16_t *brow = s_x + (size_t)my_t * ldx;
    f32x4 acc[NM][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}};
    const int my_tile = (is_up ? TPW : 0) + q;
    auto chunk = [&](const typename Fmt<FMT>::A (&w)[NM], int c) {
      const int col = Fmt<FMT>::bcol(c, g, H);
      auto bv = [&](int, int, int v) { return *(const u32x4 *)(brow + col + Fmt<FMT>::VS * v); };
      if constexpr (SB)
        chunk_mfma<FMT, NM, 1, 1>(acc, w, at, bv, c, g, H,
                                  [&](int) { return *(const u32x4 *)&s_sb[my_tile][c][4 * g]; });
      else
        chunk_mfma<FMT, NM, 1, 1>(acc, w, at, bv, c, g, H);
    };
    if constexpr (NCW > 0) {
      static_assert(SB, "the single-round stream takes the staged scales and biases");
      // The chunk's x vectors and (scale | bias) words read one chunk ahead.
      struct Ops { u32x4 b[2], sb; };
      as.template run_static<NCW>(
          at, nch, g, H,
          [&](int c) {
            const int col = Fmt<FMT>::bcol(c, g, H);
            Ops o;
            o.b[0] = *(const u32x4 *)(brow + col);
            o.b[1] = *(const u32x4 *)(brow + col + Fmt<FMT>::VS);
            o.sb = *(const u32x4 *)&s_sb[my_tile][c][4 * g];
            return o;
          },
          [&](const typename Fmt<FMT>::A (&w)[NM], int c, const Ops &o) {
            chunk_mfma<FMT, NM, 1, 1>(acc, w, at, [&](int, int, int v) { return o.b[v]; }, c, g, H,
                                      [&](int) { return o.sb; });
          });
    } else {
      as.run(at, nch, g, H, chunk);
    }
    // Chains and gate/up meet in the (gate, even) wave of each tile. The next item's partials
    // are written only after its first barrier, which this item's epilogue wave reaches last.
    const int slot_of_part = (is_up ? 1 : 0) * 2 + par;   // 0: gate even (keeps), 1: gate odd, 2: up even, 3: up odd
    if (slot_of_part > 0) s_part[slot_of_part - 1][q][lane] = acc[0][0];
    __syncthreads();
    if (it == (int)blockIdx.x) HH_TR(1, 3);
    if (slot_of_part == 0 && l16 < ntok) {
      const int r = rank_of(s_idx, my_t, e, K, sh);
      up_epilogue<FMT>(a, blob, grp, rb + 4 * g, my_t * S + r, sum_chains(acc[0][0], s_part[0][q][lane]),
                       sum_chains(s_part[1][q][lane], s_part[2][q][lane]));
    }
    if (it == (int)blockIdx.x) HH_TR(1, 4);
  }
}

// ---- MXFP4 on the scaled MFMA -------------------------------------------------------------------
typedef int v8i __attribute__((ext_vector_type(8)));

// D += A·B, v_mfma_scale_f32_16x16x128_f8f6f4 with A = 16 rows × 128 K of fp4 e2m1 and B =
// 128 K × 16 columns of fp8 e4m3. A lane (g, l16): row l16, the 32 values of K block g (low nibble
// first: exactly one MXFP4 block as stored) and that block's e8m0 scale. B lane (g, l16): column
// l16, K 16g..16g+15 in bytes 0-15 and K 64+16g..64+16g+15 in bytes 16-31, and the e8m0 scale of
// K block g. D as the 16x16 bf16 MFMA.
__device__ __forceinline__ f32x4 smfma(const u32x4 &a, const u32x4 &blo, const u32x4 &bhi, uint32_t sa,
                                       uint32_t sb, const f32x4 &c) {
  const v8i av = {(int)a[0], (int)a[1], (int)a[2], (int)a[3], 0, 0, 0, 0};
  const v8i bv = {(int)blo[0], (int)blo[1], (int)blo[2], (int)blo[3],
                  (int)bhi[0], (int)bhi[1], (int)bhi[2], (int)bhi[3]};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 4, 0, 0, (int)sa, 0, (int)sb);
}

// B operand of chunk c from one term row (bytes, K columns) and its block scales `srow`; columns
// at or past K read as zero and their blocks' scales as 2^0, so only finite values meet the zeroed
// weights of a tail chunk.
struct MxB {
  u32x4 lo, hi;
  uint32_t s;
};
__device__ __forceinline__ MxB mx_b(const uint8_t *row, const uint8_t *srow, int c, int g, int K) {
  const int k0 = 128 * c + 16 * g;
  MxB b;
  b.lo = *(const u32x4 *)(row + k0);
  b.hi = *(const u32x4 *)(row + k0 + 64);
  b.s = srow[4 * c + g];
  if (k0 >= K) b.lo = u32x4{0u, 0u, 0u, 0u};
  if (k0 + 64 >= K) b.hi = u32x4{0u, 0u, 0u, 0u};
  if (128 * c + 32 * g >= K) b.s = 127u;
  return b;
}

// One chunk of the canonical MXFP4 arithmetic: acc += A·B_t for the terms t in order.
template <int NM, int NT, int NTERM, class BF>
__device__ __forceinline__ void chunk_mx(f32x4 (&acc)[NM][NT], const u32x4 (&w)[NM], const uint32_t (&sa)[NM], BF bf,
                                         int c, int g, int K) {
  const bool ok = Fmt<Q_MXFP4>::lane_valid(c, g, K);
#pragma unroll
  for (int t = 0; t < NTERM; ++t)
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      const MxB b = bf(st, t);
#pragma unroll
      for (int m = 0; m < NM; ++m)
        acc[m][st] = smfma(ok ? w[m] : u32x4{0u, 0u, 0u, 0u}, b.lo, b.hi, sa[m] & 0xFFu, b.s, acc[m][st]);
    }
}

// The operands of one chunk that come from LDS, read unmasked: the B operand of every term and
// the e8m0 scale of the wave's weight block.
template <int NTERM> struct MxOps {
  MxB b[NTERM];
  uint32_t sa;
};
template <int NTERM>
__device__ __forceinline__ MxOps<NTERM> mx_ops(const uint8_t *brow, int RS, int ld, const uint8_t *my_sc, int nsb,
                                               int c, int g) {
  MxOps<NTERM> o;
  const int k0 = 128 * c + 16 * g;
#pragma unroll
  for (int t = 0; t < NTERM; ++t) {
    o.b[t].lo = *(const u32x4 *)(brow + t * RS + k0);
    o.b[t].hi = *(const u32x4 *)(brow + t * RS + k0 + 64);
    o.b[t].s = brow[t * RS + ld + 4 * c + g];
  }
  o.sa = my_sc[min(4 * c + g, nsb - 1)];
  return o;
}
// chunk_mx for one tile and one token tile with pre-read operands, which come from rows staged by
// MxStage (zero past K, scales 2^0 there): the same values mx_b's masks give. Lanes whose weight
// block lies past K take zero weights, as in chunk_mx.
// `full`: the chunk lies wholly inside K (no lane needs the test).
template <int NTERM>
__device__ __forceinline__ void chunk_mx1(f32x4 &acc, const u32x4 &w, const MxOps<NTERM> &o, int c, int g, int K,
                                          bool full = false) {
  const u32x4 wv = (full || Fmt<Q_MXFP4>::lane_valid(c, g, K)) ? w : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int t = 0; t < NTERM; ++t) acc = smfma(wv, o.b[t].lo, o.b[t].hi, o.sa & 0xFFu, o.b[t].s, acc);
}

// Stages the e8m0 scales of `rows` consecutive weight rows (rows · K/32 bytes, 16-byte aligned)
// into LDS: one 16-byte vector per thread and step.
__device__ __forceinline__ int scale_vectors(int rows, int K) { return rows * (K / 32) / 16; }

// The NTH fp8 terms of 8 activations of slot `slot` (intermediates ia..ia+3 in q[t][0], ib..ib+3
// in q[t][1]) and, from lane group 0, the scales of their block blk.
template <bool DEV = false>
__device__ __forceinline__ void store_hq(const GemmArgs &a, int slot, int blk, int ia, int ib,
                                         const uint32_t (&q)[NTH][2], const uint32_t (&sb)[NTH], int g) {
  // DEV: device-scope stores (sc1) through a buffer resource based at hq (hs lies after it), for
  // readers in other workgroups of the same launch.
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)a.hq, (short)0, 0x7FFFFFF0, 0x00020000);
#pragma unroll
  for (int t = 0; t < NTH; ++t) {
    uint8_t *row = a.hq + ((size_t)slot * NTH + t) * a.hld;
    uint8_t *srow = a.hs + ((size_t)slot * NTH + t) * (a.hld / 32) + blk;
    if constexpr (DEV) {
      __builtin_amdgcn_raw_buffer_store_b32(q[t][0], rs, (int)(row + ia - a.hq), 0, kDevScope);
      __builtin_amdgcn_raw_buffer_store_b32(q[t][1], rs, (int)(row + ib - a.hq), 0, kDevScope);
      if (g == 0) __builtin_amdgcn_raw_buffer_store_b8((uint8_t)sb[t], rs, (int)(srow - a.hq), 0, kDevScope);
    } else {
      *(uint32_t *)(row + ia) = q[t][0];
      *(uint32_t *)(row + ib) = q[t][1];
      if (g == 0) *srow = (uint8_t)sb[t];
    }
  }
}

// A staged operand row in LDS: `ld` bytes of one term followed by its ld/32 scale bytes.
__host__ __device__ __forceinline__ int mx_row_bytes(int ld) { return ld + ld / 32 + 16; }

// Copies the NTERM term rows (and scales) of `nrows` operand rows into LDS rows of
// mx_row_bytes(ld): LDS row rr = (j, t) ← q + (row_of(j)·NTERM + t)·ld and s + (…)·ld/32, the
// first `cols` columns only (cols a multiple of 16; the MFMA operand reads mask columns past K),
// in 16-byte vectors v = id + threads·k. The first NB vectors of each thread can be loaded before
// other loads are issued (load_first) and stored after them (store_first): completion counts
// are in order, so stores issued after a weight stream would otherwise wait for all of it.
// DEV: the rows were written by other workgroups of the same launch with device-scope stores;
// they are read with device-scope loads (sc1), which miss in caches that may hold older
// contents, through a buffer resource based at q (sc lies after q).
template <int NTERM, int NB, class RowOf, bool DEV = false> struct MxStage {
  uint8_t *dst;
  const uint8_t *q, *sc;
  int ld, cols, nrows, n, dv, per_row, RS, id, threads;
  RowOf row_of;
  u32x4 r[NB];
  __device__ __forceinline__ MxStage(uint8_t *dst_, const uint8_t *q_, const uint8_t *sc_, int ld_, int cols_,
                                     int nrows_, RowOf row_of_, int id_, int threads_)
      : dst(dst_), q(q_), sc(sc_), ld(ld_), cols(cols_), nrows(nrows_), dv(cols_ / 16),
        per_row(cols_ / 16 + (cols_ / 32 + 15) / 16), RS(mx_row_bytes(ld_)), id(id_), threads(threads_),
        row_of(row_of_) {
    n = nrows * NTERM * per_row;
  }
  __device__ __forceinline__ u32x4 src(int v) const {
    const int rr = v / per_row;
    return src_at(rr, v - rr * per_row);
  }
  // Vector qq of staged row rr.
  __device__ __forceinline__ u32x4 src_at(int rr, int qq) const {
    const size_t grow = (size_t)row_of(rr / NTERM) * NTERM + rr % NTERM;
    // One load from a selected address (two loads under a lane-dependent branch would serialise).
    const uint8_t *p = qq < dv ? q + grow * ld + 16 * qq : sc + grow * (ld / 32) + 16 * (qq - dv);
    if constexpr (DEV) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)q, (short)0, 0x7FFFFFF0, 0x00020000);
      return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(p - q), 0, kDevScope));
    } else {
      return *(const u32x4 *)p;
    }
  }
  // Scale bytes of blocks at or past `cols` (the tail of the last scale vector) are stored as 127
  // (2^0), so the MFMA operands of the last chunk need no masks.
  __device__ __forceinline__ void put(int v, u32x4 val) const {
    const int rr = v / per_row;
    put_at(rr, v - rr * per_row, val);
  }
  __device__ __forceinline__ void put_at(int rr, int qq, u32x4 val) const {
    if (qq >= dv) {
      const int nvalid = cols / 32 - 16 * (qq - dv);
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          if (4 * d + b >= nvalid) val[d] = (val[d] & ~(0xFFu << (8 * b))) | (0x7Fu << (8 * b));
    }
    *(u32x4 *)(dst + (size_t)rr * RS + (qq < dv ? 16 * qq : ld + 16 * (qq - dv))) = val;
  }
  // Zeros columns cols .. (cols rounded up to 128) of every staged row: the last chunk's operand
  // past K. Disjoint from the bytes put() writes.
  __device__ __forceinline__ void pad() const {
    const int nz = (((cols + 127) & ~127) - cols) / 16;
    for (int v = id; v < nrows * NTERM * nz; v += threads) {
      const int rr = v / nz;
      *(u32x4 *)(dst + (size_t)rr * RS + cols + 16 * (v - rr * nz)) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  // The (row, vector) coordinates of vectors id, id + threads, ...: one division, then a step of
  // `threads` vectors (under a row when threads < per_row, so one carry at most; otherwise the
  // whole rows of the step are added first).
  struct Walk {
    int rr, qq, dr, dq;
  };
  __device__ __forceinline__ Walk walk() const {
    Walk w;
    w.rr = id / per_row;
    w.qq = id - w.rr * per_row;
    w.dr = threads / per_row;
    w.dq = threads - w.dr * per_row;
    return w;
  }
  __device__ __forceinline__ void step(Walk &w) const {
    w.rr += w.dr;
    w.qq += w.dq;
    if (w.qq >= per_row) {
      w.qq -= per_row;
      ++w.rr;
    }
  }
  // Unconditional (clamped) loads keep the completion counts exact.
  __device__ __forceinline__ void load_first() {
    const int rl = (n - 1) / per_row, ql = n - 1 - rl * per_row;
    Walk w = walk();
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const bool in = id + threads * k < n;
      r[k] = src_at(in ? w.rr : rl, in ? w.qq : ql);
      step(w);
    }
  }
  __device__ __forceinline__ void store_first() {
    Walk w = walk();
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      if (id + threads * k < n) put_at(w.rr, w.qq, r[k]);
      step(w);
    }
  }
  __device__ __forceinline__ void rest() {
    for (int base = threads * NB; base < n; base += threads * 4)
      stage_batch<4>(base, id, threads, n, [&](int v) { return src(v); }, [&](int v, const u32x4 &x) { put(v, x); });
  }
};
template <int NTERM, int NB, bool DEV = false, class RowOf>
__device__ __forceinline__ MxStage<NTERM, NB, RowOf, DEV> mx_stage(uint8_t *dst, const uint8_t *q, const uint8_t *sc,
                                                                    int ld, int cols, int nrows, RowOf row_of, int id,
                                                                    int threads) {
  return MxStage<NTERM, NB, RowOf, DEV>(dst, q, sc, ld, cols, nrows, row_of, id, threads);
}

// Data between workgroups of one launch (the fused decode kernels) is announced by words that
// hold the epoch of the call that wrote them; epochs never repeat for a buffer, so no word is
// ever cleared.
// Logit records of the fused router: 16 bytes {value lo, value hi, epoch, check} with check =
// lo ^ hi ^ epoch ^ kRecSalt, written by one device-scope 16-byte store into each of the 8
// replicas (one per XCD, so the pollers of one XCD share a copy). A reader accepts a record
// whose epoch is the call's and whose check matches: a record whose dwords came from two
// different stores fails the check (the value bits differ between calls).
constexpr uint32_t kRecSalt = 0x9E3779B9u;
constexpr int kRecReplicas = 8;
__device__ __forceinline__ void store_logit_record(uint32_t *recs, int R, int i, double v, uint32_t epoch, int lane) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)b, hi = (uint32_t)(b >> 32);
  if (lane < kRecReplicas) {
    const u32x4 rec = {lo, hi, epoch, lo ^ hi ^ epoch ^ kRecSalt};
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)recs, (short)0, 0x7FFFFFF0, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b128(rec, rs, 16 * (lane * R + i), 0, kDevScope);
  }
}
// Whole wave: the n logits of replica `rep` into dst[0..n) once every record holds `epoch`
// (device-scope loads, one round trip per poll); false past the deadline.
__device__ __forceinline__ bool wait_logit_records(const uint32_t *recs, int R, int rep, int n, uint32_t epoch,
                                                   uint64_t deadline, double *dst) {
  const int lane = threadIdx.x & 63;
  const uint32_t *base = recs + 4 * (size_t)rep * R;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7FFFFFF0, 0x00020000);
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int i = i0 + lane;
    for (;;) {
      bool ok = true;
      if (i < n) {
        const u32x4 r = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * i, 0, kDevScope));
        ok = r[2] == epoch && r[3] == (r[0] ^ r[1] ^ epoch ^ kRecSalt);
        if (ok) dst[i] = __longlong_as_double((long long)(((uint64_t)r[1] << 32) | r[0]));
      }
      if (__ballot(!ok) == 0ull) break;
      if (wall_clock64() > deadline) return false;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return true;
}
// Before a flag store: this wave's device-scope data stores have completed.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// x of every token as NTX fp8 terms into LDS rows (t, j) of RS bytes, the layout MxStage gives:
// term bytes at their columns, block scales after `xld`, the last chunk's columns past H zero
// and their scales 2^0. Lane (g, l16) of a wave takes block 16·k + l16, columns 8g .. 8g+7
// (quant_block).
__device__ __forceinline__ void quant_x_lds(const uint16_t *x, int T, int H, int xld, uint8_t *s_xb, int RS) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const int nb = H / 32, per_t = (nb + 15) / 16, nw = T * per_t;
  // A wave's tasks w, w + 4, ... in batches of QXB: every load of a batch is issued before the
  // first is used (one memory latency per batch, not per task).
  constexpr int QXB = 6;
  for (int w0 = wave; w0 < nw; w0 += 4 * QXB) {
    u32x4 xb[QXB];
#pragma unroll
    for (int k = 0; k < QXB; ++k) {
      const int w = min(w0 + 4 * k, nw - 1), t = w / per_t, bc = min(16 * (w - t * per_t) + l16, nb - 1);
      xb[k] = *(const u32x4 *)(x + (size_t)t * H + bc * 32 + 8 * g);
    }
#pragma unroll
    for (int k = 0; k < QXB; ++k) {
    const int w = w0 + 4 * k;
    if (w >= nw) break;
    const int t = w / per_t, b = 16 * (w - t * per_t) + l16;
    const u32x4 xv = xb[k];
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
        uint8_t *row = s_xb + (size_t)(t * NTX + j) * RS;
        *(u32x2 *)(row + b * 32 + 8 * g) = u32x2{q[j][0], q[j][1]};
        if (g == 0) row[xld + b] = (uint8_t)sb[j];
      }
    }
    }
  }
  const int hp = (H + 127) & ~127, nz = (hp - H) / 16, ns = (hp - H) / 32;
  for (int v = tid; v < T * NTX * (nz + ns); v += 256) {
    const int rr = v / (nz + ns), k = v - rr * (nz + ns);
    uint8_t *row = s_xb + (size_t)rr * RS;
    if (k < nz) *(u32x4 *)(row + H + 16 * k) = u32x4{0u, 0u, 0u, 0u};
    else row[xld + H / 32 + (k - nz)] = 127;
  }
}

// quant_x_lds for the FFN block (ra.resid set, T ≤ 2): x = bf16(resid·f·norm_w) formed from the
// residual rows as the block's norm kernel rounds it (f from row_sumsq, every wave for every
// token), then quantised as quant_x_lds into the same LDS layout.
__device__ __forceinline__ void quant_x_lds_block(const RouteArgs &ra, int T, int H, int xld, uint8_t *s_xb, int RS) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const int nb = H / 32, per_t = (nb + 15) / 16, nw = T * per_t;
  double f[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
    if (t < T) f[t] = norm_factor(row_sumsq(ra.resid + (size_t)t * H, H), H, (double)ra.norm_eps, ra.norm_pow);
  constexpr int QXB = 4;
  for (int w0 = wave; w0 < nw; w0 += 4 * QXB) {
    f32x4 xb[QXB][2];
    u32x4 nv[QXB];
#pragma unroll
    for (int k = 0; k < QXB; ++k) {
      const int w = min(w0 + 4 * k, nw - 1), t = w / per_t, bc = min(16 * (w - t * per_t) + l16, nb - 1);
      const float *xr = ra.resid + (size_t)t * H + bc * 32 + 8 * g;
      xb[k][0] = *(const f32x4 *)xr;
      xb[k][1] = *(const f32x4 *)(xr + 4);
      nv[k] = *(const u32x4 *)(ra.norm_w + bc * 32 + 8 * g);
    }
#pragma unroll
    for (int k = 0; k < QXB; ++k) {
      const int w = w0 + 4 * k;
      if (w >= nw) break;
      const int t = w / per_t, b = 16 * (w - t * per_t) + l16;
      const double ft = t == 0 ? f[0] : f[1];
      float v[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float nf = bf16_bits_to_f32((nv[k][c >> 1] >> (16 * (c & 1))) & 0xFFFFu);
        const float xv = c < 4 ? xb[k][0][c] : xb[k][1][c - 4];
        v[c] = bf16_bits_to_f32(f64_to_bf16_bits((double)xv * ft * (double)nf));
      }
      uint32_t q[NTX][2], sb[NTX];
      quant_block<NTX>(v, q, sb);
      if (b < nb) {
#pragma unroll
        for (int j = 0; j < NTX; ++j) {
          uint8_t *row = s_xb + (size_t)(t * NTX + j) * RS;
          *(u32x2 *)(row + b * 32 + 8 * g) = u32x2{q[j][0], q[j][1]};
          if (g == 0) row[xld + b] = (uint8_t)sb[j];
        }
      }
    }
  }
  const int hp = (H + 127) & ~127, nz = (hp - H) / 16, ns = (hp - H) / 32;
  for (int v = tid; v < T * NTX * (nz + ns); v += 256) {
    const int rr = v / (nz + ns), k = v - rr * (nz + ns);
    uint8_t *row = s_xb + (size_t)rr * RS;
    if (k < nz) *(u32x4 *)(row + H + 16 * k) = u32x4{0u, 0u, 0u, 0u};
    else row[xld + H / 32 + (k - nz)] = 127;
  }
}


// Decode gate-up on the scaled MFMA, persistent: the grid holds about two workgroups per compute
// unit; each selects the top-k of the batch once, lists the batch's distinct experts in LDS (in
// order of first appearance in the (token, rank) table, the shared expert last) and stages every
// token's x terms, then takes work items it = blockIdx.x, blockIdx.x + gridDim.x, ... An item is
// 32 intermediates of one expert. 4 waves: wave w takes tile q = w & 1 (16 intermediates) and the
// gate (w < 2) or up rows over the whole K (both chains); the item's 64 rows' e8m0 scales come
// through LDS. The gate waves combine gate and up and write the block's activations to LDS; wave
// 0 writes them as NTH fp8 terms. Each item issues its whole weight stream at once; co-resident
// workgroups hide one another's latency.
// NCH > 0 (ONE only): every row of the layer has exactly NCH chunks (checked on the host).
// FR (fused router): the grid's first f.R workgroups are the router, one per (token, row) pair
// (split_pair_logit, the router kernel's arithmetic), each storing its logit as a checksummed
// record into the 8 per-XCD replicas (store_logit_record); the other workgroups quantise x into
// LDS themselves (the router kernel's terms, quant_block), then wave 0 polls its XCD's replica
// until every record carries the call's epoch (wait_logit_records: device-scope loads, no
// fences, the logits arriving with the same load that shows them ready) and the selection reads
// them from LDS. Router workgroups wait for nothing and have the smaller indices, which the
// dispatcher starts first, so every wait is for workgroups that run. Waits are bounded (10 ms);
// a workgroup that times out sets bit 0 of *f.status and stops.
template <int DA, bool ONE, int XB, int NCH = 0, int FR = 0>
__global__ __launch_bounds__(256, 2) void up_small_mx(GemmArgs a, RouteArgs ra, FuseArgs f) {
  warm_kernargs<sizeof(GemmArgs) + sizeof(RouteArgs) + sizeof(FuseArgs)>();
  constexpr int NM = 1;
  extern __shared__ __align__(16) uint8_t s_xb[];   // [T][NTX] rows of mx_row_bytes(xld), then [64][H/32] scales
  __shared__ int s_idx[SMALL_T * kMaxTopK];
  __shared__ f32x4 s_up[2][64], s_gate[2][64];
  __shared__ u32x4 s_bias[2][4];
  __shared__ float s_hv[SMALL_T][UP_ROWS];
  __shared__ double s_lg[4][64];
  __shared__ int s_ri[4][kMaxTopK];
  __shared__ int s_ci[4][kFastCand];
  __shared__ double s_cv[4][kFastCand];
  __shared__ double s_rv[4][kMaxTopK];
  __shared__ int s_rk[4][64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  // The instances with two x vectors per thread (XB = 2) are launched for one token only
  // (up_small_k): their token count is compiled in.
  constexpr bool T1 = XB <= 2;
  const int T = T1 ? 1 : ra.tokens, E = a.experts, K = a.top_k, S = a.slots, H = a.hidden;
  const bool has_shared = S > K;
  // The gate-up role's workgroup index and count.
  const int bx = FR ? (int)blockIdx.x - f.R : (int)blockIdx.x;
  const int gx = FR ? (int)gridDim.x - f.R : (int)gridDim.x;
  [[maybe_unused]] __shared__ double s_lgall[FR ? kFusedRouterT : 1][FR ? kFusedMaxE + 1 : 1];
  [[maybe_unused]] __shared__ int s_flag;
  [[maybe_unused]] uint64_t deadline = 0;
  if constexpr (FR) {
    deadline = wall_clock64() + 1000000;   // 10 ms at 100 MHz
    if (bx < 0) {
      // ---- router: logit of pair blockIdx.x ----
      HH_TR(1, 0);
      __shared__ double s_acc[4][64];
      __shared__ double s_px[4][2][64];
      const int E1 = E + 1, t = (int)blockIdx.x / E1, e = (int)blockIdx.x - t * E1;
      double v = 0.0;
      if (e < E || has_shared) {
        if constexpr (FR == 2) v = block_pair_logit(ra, t, e, s_acc);
        else v = split_pair_logit<false>(ra, t, e, s_acc, s_px);
      }
      if (wave == 0) store_logit_record(f.flags, f.R, (int)blockIdx.x, v, f.epoch, lane);
      HH_TR(1, 1);
      return;
    }
  }

  // x terms of every token: first batch of loads now (they do not depend on the routing), stored
  // with the first item. FR: quantised here into the same LDS rows while the router runs.
  const int RS = mx_row_bytes(a.xld);
  HH_TR(1, 0);
  auto xs = mx_stage<NTX, XB>(s_xb, a.xq, a.xs, a.xld, a.hidden, T, [](int j) { return j; }, tid, 256);
  if constexpr (FR) {
    if constexpr (FR == 2) quant_x_lds_block(ra, T, H, a.xld, s_xb, RS);
    else quant_x_lds(ra.x, T, H, a.xld, s_xb, RS);
    HH_TR(1, 6);
    if (wave == 0) {
      // the records of this workgroup's XCD (workgroups are dealt to the 8 XCDs round robin)
      const bool ok = wait_logit_records(f.flags, f.R, (int)blockIdx.x % kRecReplicas, f.R, f.epoch,
                                         deadline, &s_lgall[0][0]);
      if (lane == 0) s_flag = ok ? 1 : 0;
    }
    __syncthreads();
    if (!s_flag) {
      if (tid == 0) atomicOr(f.status, 1u);
      return;
    }
    HH_TR(1, 7);
  } else {
    xs.load_first();
  }
  // The fp64 logits of token t: the router's output, or (FR) the workgroup's LDS copy.
  auto logits_of = [&](int t) -> const double * {
    if constexpr (FR) return &s_lgall[0][0] + (size_t)t * (E + 1);
    else return ra.lg64 + (size_t)t * (E + 1);
  };
  // Top-k of every token (wave w: tokens w, w + 4, ...; one token: the 4 waves rank it
  // together); workgroup 0 writes the routing outputs.
  if (T1 || T <= 2) {
    // One or two tokens: groups of 4 / T waves rank a token together.
    const int G = (T1 || T == 1) ? 4 : 2, t = T1 ? 0 : wave / G;
    const double *lg = logits_of(t);
#ifdef HH_TRACE
    if (!FR) { volatile double first = lg[lane % E]; (void)first; HH_TR(1, 6); }
#endif
    TopK tk = (T1 || T == 1) ? (E <= 64 ? topk_rank64<4>(lg, E, K, s_lg[wave], s_ri[wave], s_rk)
                                      : topk_fast<4>(lg, E, K, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave], s_rk))
                           : (E <= 64 ? topk_rank64<2>(lg, E, K, s_lg[wave], s_ri[wave], s_rk)
                                      : topk_fast<2, 1>(lg, E, K, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave], s_rk));
    prob_order(tk, K, ra.router);
    if (!FR) HH_TR(1, 7);
    if (wave % G == 0) {
      if (lane < K) s_idx[t * K + lane] = tk.index_of(lane);
      if (bx == 0) finish_token(ra, t, tk, has_shared ? lg[E] : 0.0);
    }
  } else {
    for (int t = wave; t < T; t += 4) {
      const double *lg = logits_of(t);
      TopK tk = E <= 64 ? topk_rank64(lg, E, K, s_lg[wave], s_ri[wave])
                              : topk_fast(lg, E, K, s_ri[wave], s_rv[wave], s_ci[wave], s_cv[wave]);
      prob_order(tk, K, ra.router);
      if (lane < K) s_idx[t * K + lane] = tk.index_of(lane);
      if (bx == 0) finish_token(ra, t, tk, has_shared ? lg[E] : 0.0);
    }
  }
  __syncthreads();
  HH_TR(1, 1);
  const Plan plan(s_idx, T, K, E);
  const int nu = plan.nu;
  const int rtr = a.grp[0].inter / UP_ROWS;
  const int nitems = nu * rtr + (has_shared ? a.grp[1].inter / UP_ROWS : 0);

  const int q = wave & 1;
  const bool is_up = wave >= 2;
  const int nch = (H + 127) / 128;
  const int nsb = H / 32;                            // scale bytes per row
  uint8_t *s_sc = s_xb + (size_t)T * NTX * RS;      // [64][nsb]
  const int nsv = scale_vectors(64, H);
  bool x_pending = !FR;
  if constexpr (XB > 2 && !FR) {
    // Batches of several tokens: the x terms landed during the selection; they are stored before
    // the first item's weight stream takes its registers.
    xs.store_first();
    xs.rest();
    xs.pad();
    x_pending = false;
  }
  for (int it = bx; it < nitems; it += gx) {
    const bool sh = it >= nu * rtr;
    const int u = sh ? nu : it / rtr;
    const int rt = sh ? it - nu * rtr : it % rtr;
    int e;
    uint64_t tm;
    plan.entry(u, e, tm);
    const int ntok = __popcll(tm);
    const ExpertGroup &grp = a.grp[sh ? 1 : 0];
    const uint8_t *blob = grp.blobs + (sh ? 0 : (size_t)e * grp.stride);
    const int rb = rt * UP_ROWS + 16 * q;

    // The item's 64 gate_up rows' scales (contiguous: rows 64·rt ..), first loads out before the
    // weight stream, stored after it (with the x terms on the first item).
    const uint8_t *gsc = blob + grp.off[1] + (size_t)rt * 64 * nsb;
    u32x4 scv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) scv[k] = *(const u32x4 *)(gsc + 16 * min(tid + 256 * k, nsv - 1));
    // The gate waves' bias (4 intermediates per lane), loaded ahead of the weight stream.
    u32x4 bias = {0u, 0u, 0u, 0u};
    if (!is_up && a.expert_bias) bias = *(const u32x4 *)(blob + grp.off[2] + 4 * (rb + 4 * g));
    ATile<Q_MXFP4_W> at[NM] = {tile_of<PH_UP, Q_MXFP4_W>(blob, grp, rb, is_up, H, l16)};
    constexpr int PF = ONE ? (XB <= 2 ? MX_PF_T1 : MX_PF) : DA;
    AStream<Q_MXFP4_W, NM, DA> as(0, 1, nch);
    as.template fill<PF>(at, nch, g, H);
    if (x_pending) {
      xs.store_first();
      xs.rest();
      xs.pad();
      x_pending = false;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (tid + 256 * k < nsv) *(u32x4 *)(s_sc + 16 * (tid + 256 * k)) = scv[k];
    for (int v = tid + 512; v < nsv; v += 256) *(u32x4 *)(s_sc + 16 * v) = *(const u32x4 *)(gsc + 16 * v);
    __syncthreads();
    if (it == bx) HH_TR(1, 2);

    const uint8_t *my_sc = s_sc + (2 * (16 * q + l16) + (is_up ? 1 : 0)) * nsb;
    // The lane group as a value opaque to the compiler in each item: otherwise every chunk's
    // item-invariant operand addresses and masks are hoisted out of the item loop and held
    // (spilled) across it.
    int gi = g;
    asm volatile("" : "+v"(gi));
    const int my_t = nth_bit(tm, min(l16, ntok - 1));   // token of column l16 (padding repeats)
    const uint8_t *brow = s_xb + (size_t)my_t * NTX * RS;
    f32x4 acc[NM][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}};
    as.template run_pf<ONE, PF, NCH>(
        at, nch, gi, H, [&](int c) { return mx_ops<NTX>(brow, RS, a.xld, my_sc, nsb, c, gi); },
        [&](const Fmt<Q_MXFP4_W>::A (&w)[NM], int c, const MxOps<NTX> &o) {
          chunk_mx1<NTX>(acc[0][0], w[0].w, o, c, gi, H, NCH > 0 && c < NCH - 1);
        });
    const f32x4 res = acc[0][0];
    if (nitems > gx) {
      // Workgroups with further items: the gate waves form the activations and wave 0 writes the
      // terms, while the other waves go on to the next item's weight stream.
      if (is_up) s_up[q][lane] = res;
      __syncthreads();
      if (it == bx) HH_TR(1, 3);
      if (!is_up && l16 < ntok) {
        const f32x4 y = up_values_mx(a, bias, res, s_up[q][lane]);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) s_hv[l16][16 * q + 4 * g + ii] = y[ii];
      }
      __syncthreads();
      if (wave == 0) {
        // Lane (g, l16): activations 8g .. 8g+7 of the block of token column l16.
        const int j = min(l16, ntok - 1);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = s_hv[j][8 * g + i];
        uint32_t hq[NTH][2], sb[NTH];
        quant_block<NTH>(v, hq, sb);
        if (l16 < ntok) {
          const int t = nth_bit(tm, l16);
          const int slot = t * S + rank_of(s_idx, t, e, K, sh);
          store_hq(a, slot, rt, rt * UP_ROWS + 8 * g, rt * UP_ROWS + 8 * g + 4, hq, sb, g);
        }
      }
      if (it == bx) HH_TR(1, 4);
      continue;
    }
    // One item per workgroup: the epilogue spread over the workgroup, one (token column j,
    // intermediate k) per thread: the gate and up sums (lane (g, l16) of tile q holds
    // intermediates 16q + 4g + ii of column l16) and the gate bias through LDS, the activation,
    // then the block's NTH fp8 terms with the block on the 32 lanes of a half wave (quant_lane:
    // quant_block's bytes). Its dependent chain is a fraction of the one-wave epilogue's.
    if (is_up) {
      s_up[q][lane] = res;
    } else {
      s_gate[q][lane] = res;
      if (l16 == 0) s_bias[q][g] = bias;
    }
    __syncthreads();
    if (it == bx) HH_TR(1, 3);
    const int nv = ntok * UP_ROWS;
    for (int i = tid; i < nv; i += 256) {
      const int j = i >> 5, k = i & 31, kq = k >> 4, kg = (k >> 2) & 3, ii = k & 3;
      const uint32_t bb = s_bias[kq][kg][ii];
      s_hv[j][k] = activate(a.act, s_gate[kq][16 * kg + j][ii] + bf16_bits_to_f32(bb & 0xFFFFu),
                            s_up[kq][16 * kg + j][ii] + bf16_bits_to_f32(bb >> 16), a.alpha, a.limit);
    }
    __syncthreads();
    for (int i = tid; i < nv; i += 256) {   // whole half waves: nv is a multiple of 32
      const int j = i >> 5, k = i & 31;
      uint32_t hq[NTH], sb[NTH];
      quant_lane<NTH>(s_hv[j][k], hq, sb);
      const int t = nth_bit(tm, j);
      const int slot = t * S + rank_of(s_idx, t, e, K, sh);
#pragma unroll
      for (int tt = 0; tt < NTH; ++tt) {
        a.hq[((size_t)slot * NTH + tt) * a.hld + rt * UP_ROWS + k] = (uint8_t)hq[tt];
        if (k == 0) a.hs[((size_t)slot * NTH + tt) * (a.hld / 32) + rt] = (uint8_t)sb[tt];
      }
    }
    if (it == bx) HH_TR(1, 4);
    // s_hv and s_sc are rewritten by the next item only after its first barrier.
  }
  HH_TR(1, 5);
}

// ---- decode: down + combine -----------------------------------------------------------------------
// Item order of down_small, XCD-aware: workgroups are dealt to the 8 XCDs round robin by index
// and the grid is a multiple of 8, so item it runs on XCD it % 8. The T tokens of row tile rt
// are consecutive items of one XCD (rt ≡ it (mod 8)): the tokens that share an expert read its
// 16 rows at about the same time through the same L2 instead of once per token from HBM. Row
// tiles are padded to a multiple of 8; padding items have rt ≥ the row tile count.
__host__ __device__ constexpr int down_small_items(int row_tiles, int T) { return 8 * ((row_tiles + 7) / 8) * T; }
__device__ __forceinline__ void down_small_item(int it, int T, int &rt, int &t) {
  const int x = it & 7, j = it >> 3, jt = j / T;
  t = j - jt * T;
  rt = x + 8 * jt;
}
// Persistent: work items (16 hidden rows, token t) = it = blockIdx.x, blockIdx.x + gridDim.x, ...
// Wave (r, p): slot r of the token (expert topk_idx[t][r], or the
// shared expert), chunk parity p when KS = 2 (both chains in one wave when KS = 1). The epilogue
// sums the chains, then the slots in rank order (sum_expert_slices, dense.metal:147;
// ReferenceLayer.swift:194-202). SMAX = the most slots a token has under this instantiation.
// SBS (MLX, K ≤ 64·mlx_sb_chunks_down<SMAX>): each slot's scales and biases staged (MlxSb).
template <int FMT, int DA, int SMAX, int KS, bool SBS = false>
__global__ __launch_bounds__(64 * SMAX * KS) void down_small(GemmArgs a, const int32_t *topk_idx) {
  warm_kernargs<sizeof(GemmArgs) + sizeof(void *)>();
  constexpr int NM = 1;
  extern __shared__ __align__(16) uint16_t s_h[];   // [slots][2][ldh + LDS_PAD]
  __shared__ f32x4 s_odd[KS > 1 ? SMAX : 1][4];     // odd chain, lanes l16 == 0
  constexpr bool SB = SBS && is_mlx<FMT>();         // MLX: each slot's scales and biases staged
  constexpr int SBCH = mlx_sb_chunks_down<SMAX>();
  __shared__ __align__(16) uint32_t s_sbd[SB ? SMAX : 1][SB ? SBCH : 1][16];
  __shared__ float s_o[SMAX][16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int S = a.slots, K = a.top_k, H = a.hidden, E = a.experts;
  const int T = a.max_work;              // tokens of the batch
  const int nitems = down_small_items(a.row_tiles, T);
  const int r = wave % S, par = wave / S;
  HH_TR(2, 0);
  for (int it = blockIdx.x; it < nitems; it += gridDim.x) {
  int rt, t;
  down_small_item(it, T, rt, t);
  if (rt >= a.row_tiles) continue;       // padding item (uniform over the workgroup)
  const int slot = t * S + r;
  if (it == (int)blockIdx.x) HH_TR(2, 6);
  const int e = r < K ? topk_idx[t * K + r] : E;
  const int gsel = e == E ? 1 : 0;
  const ExpertGroup &grp = a.grp[gsel];
  const uint8_t *blob = grp.blobs + (gsel ? 0 : (size_t)e * grp.stride);
  const int I = grp.inter;
  const int rb = rt * 16;
  // The residual of the item's 16 rows (FFN block), loaded ahead of the weight stream.
  const float rv = (a.resid && tid < 16) ? a.resid[(size_t)t * H + rb + tid] : 0.f;

  ATile<FMT> at[NM];
  wave_tiles<PH_DOWN, FMT, 1>(at, blob, grp, rb, H, I, l16);
  const int nch = (I + Fmt<FMT>::CHUNK - 1) / Fmt<FMT>::CHUNK;
  f32x4 acc[2][NM][1];
#pragma unroll
  for (int p = 0; p < 2; ++p) acc[p][0][0] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (FMT == Q_MXFP4) {
    // This slot's activation terms and its 16 weight rows' scales into LDS (the slot's waves
    // share them): first loads out before the weight stream, stored after it.
    uint8_t *sbm = (uint8_t *)s_h;
    const int RS = mx_row_bytes(a.hld);
    const int nsb = I / 32, nsv = scale_vectors(16, I);
    const int imax = max(a.grp[0].inter, a.grp[1].inter);   // per-slot LDS stride as on the host
    const int slot_bytes = NTH * RS + 16 * ((16 * (imax / 32) + 15) / 16);
    uint8_t *my_lds = sbm + (size_t)r * slot_bytes;
    uint8_t *s_sc = my_lds + NTH * RS;
    const uint8_t *gsc = blob + grp.off[4] + (size_t)rb * nsb;
    const int sid = par * 64 + lane, sth = 64 * KS;
    u32x4 scv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) scv[k] = *(const u32x4 *)(gsc + 16 * min(sid + sth * k, nsv - 1));
    auto hs = mx_stage<NTH, 9>(my_lds, a.hq, a.hs, a.hld, I, 1, [&](int) { return slot; }, sid, sth);
    hs.load_first();
    ATile<Q_MXFP4_W> aw[NM] = {tile_of<PH_DOWN, Q_MXFP4_W>(blob, grp, rb, false, I, l16)};
    static_assert(KS == 1, "MXFP4 accumulates one chain over K");
    constexpr int PF = DA >= MX_ONE_CHUNKS ? MX_PF : DA;
    AStream<Q_MXFP4_W, NM, DA> as(0, 1, nch);
    as.template fill<PF>(aw, nch, g, I);
    if (it == (int)blockIdx.x) HH_TR(2, 5);
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (sid + sth * k < nsv) *(u32x4 *)(s_sc + 16 * (sid + sth * k)) = scv[k];
    for (int v = sid + 2 * sth; v < nsv; v += sth) *(u32x4 *)(s_sc + 16 * v) = *(const u32x4 *)(gsc + 16 * v);
    hs.store_first();
    if (it == (int)blockIdx.x) HH_TR(2, 4);
    hs.rest();
    hs.pad();
    __syncthreads();
    if (it == (int)blockIdx.x) HH_TR(2, 1);
    const uint8_t *brow = my_lds;
    const uint8_t *my_sc = s_sc + l16 * nsb;
    // MXFP4: one chain. DA ≥ MX_ONE instantiations run only for rows of at most DA chunks.
    as.template run_pf<(DA >= MX_ONE_CHUNKS), PF>(
        aw, nch, g, I, [&](int c) { return mx_ops<NTH>(brow, RS, a.hld, my_sc, nsb, c, g); },
        [&](const Fmt<Q_MXFP4_W>::A (&w)[NM], int c, const MxOps<NTH> &o) {
          chunk_mx1<NTH>(acc[0][0][0], w[0].w, o, c, g, I);
        });
  } else {
  // This slot's activation (hi, lo) into LDS (the slot's two waves share it): the loads go out
  // before the weight stream (see stage_batch), the stores after it.
  const int ldb = a.ldh + LDS_PAD;
  uint16_t *sb = s_h + (size_t)r * 2 * ldb;
  const int per_row = I / 8, nvec = 2 * per_row;
  auto hsrc = [&](int v) {
    const int hh = v / per_row, qq = v - hh * per_row;
    return *(const u32x4 *)((hh ? a.h_lo : a.h_hi) + (size_t)slot * a.ldh + 8 * qq);
  };
  auto hdst = [&](int v, const u32x4 &val) {
    const int hh = v / per_row, qq = v - hh * per_row;
    *(u32x4 *)(sb + hh * ldb + 8 * qq) = val;
  };
  // 64·KS·HB vectors in the first batch: both terms of I ≤ 3072 (SMAX 4, KS 2) or I ≤ 1024.
  constexpr int HB = (SMAX <= 4 && KS == 2) ? 6 : 4;
  const int sid = par * 64 + lane, sth = 64 * KS;
  u32x4 hr[HB];
#pragma unroll
  for (int k = 0; k < HB; ++k)
    if (sid + sth * k < nvec) hr[k] = hsrc(sid + sth * k);
  // MLX: the slot's 16 down rows' scales and biases, staged by the slot's waves.
  auto sb_src = [&](int, int kind, int row) {
    return (const uint16_t *)(blob + grp.off[7 + kind]) + (size_t)min(rb + row, H - 1) * (I / 64);
  };
  u32x4 sbr[kMlxSbNB];
  if constexpr (SB) mlx_sb_load<1>(sbr, nch, sid, sth, sb_src);
  AStream<FMT, NM, DA, SB> as(KS > 1 ? par : 0, KS, nch);
  as.fill(at, nch, g, I);
#pragma unroll
  for (int k = 0; k < HB; ++k)
    if (sid + sth * k < nvec) hdst(sid + sth * k, hr[k]);
  for (int base = sth * HB; base < nvec; base += sth * 4) stage_batch<4>(base, sid, sth, nvec, hsrc, hdst);
  if constexpr (SB) mlx_sb_store<1, SBCH>(sbr, &s_sbd[r], nch, sid, sth, sb_src);
  __syncthreads();
  if (it == (int)blockIdx.x) HH_TR(2, 1);

  as.run(at, nch, g, I, [&](const typename Fmt<FMT>::A (&w)[NM], int c) {
    const int col = Fmt<FMT>::bcol(c, g, I);
    auto bv = [&](int, int hh, int v) { return *(const u32x4 *)(sb + hh * ldb + col + Fmt<FMT>::VS * v); };
    if constexpr (SB) {
      auto sbf = [&](int) { return *(const u32x4 *)&s_sbd[r][c][4 * g]; };
      if (KS == 1 && (c & 1)) chunk_mfma<FMT, NM, 1, 2>(acc[1], w, at, bv, c, g, I, sbf);
      else chunk_mfma<FMT, NM, 1, 2>(acc[0], w, at, bv, c, g, I, sbf);
    } else {
      if (KS == 1 && (c & 1)) chunk_mfma<FMT, NM, 1, 2>(acc[1], w, at, bv, c, g, I);
      else chunk_mfma<FMT, NM, 1, 2>(acc[0], w, at, bv, c, g, I);
    }
  });
  }
  if constexpr (KS > 1) {
    if (par == 1 && l16 == 0) s_odd[r][g] = acc[0][0][0];
    __syncthreads();
    if (par == 0 && l16 == 0) acc[1][0][0] = s_odd[r][g];
  }
  if (par == 0 && l16 == 0) {
    const f32x4 o = down_value<FMT>(a, blob, grp, rb + 4 * g, slot,
                                    FMT == Q_MXFP4 ? acc[0][0][0] : sum_chains(acc[0][0][0], acc[1][0][0]));
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) s_o[r][4 * g + ii] = o[ii];
  }
  __syncthreads();
  if (it == (int)blockIdx.x) HH_TR(2, 2);
  if (tid < 16) {
    float y = s_o[0][tid];
    for (int qq = 1; qq < S; ++qq) y += s_o[qq][tid];
    const size_t o = (size_t)t * H + rb + tid;
    if (a.resid) y = rv + y;
    a.y[o] = y;
  }
  __syncthreads();   // the next item rewrites the LDS rows and s_o
  }
  HH_TR(2, 3);
}

// ---- decode, fused: one launch per MXFP4 layer ------------------------------------------------------
// Workgroups take one of three roles by blockIdx, in dependency order:
//   [0, R)        router: one workgroup per (token, row) pair (split_pair_logit) writes its logit
//                 as a record into the 8 replicas (store_logit_record), as up_small_mx's FR role.
//   [R, R+U)      gate-up: quantise x into LDS (every workgroup itself), wait for the records of
//                 its XCD's replica, select the top-k and build the plan (as up_small_mx), then
//                 items it = role index, + U, ...; an item's h terms go to the exchange buffer with
//                 device-scope stores, then the item adds one to its expert's counter.
//   [R+U, R+U+D)  down: the same records and selection, then items (16 hidden rows, token), wave
//                 r = slot r: issue the weight stream and scales, wait until the counter of the
//                 slot's expert holds all its gate-up items, stage its h terms with device-scope
//                 loads and compute; the rank-ordered slot sum goes to y.
// Counters sit in two regions of kFusedCtr words at f.ctr, apart from the records (whose extent
// varies with the batch size); the context's n-th one-launch
// call (f.seq = n) counts in region n & 1 with atomic adds, and its first gate-up workgroup
// zeroes the other region for the next one-launch call (which starts only after this launch
// ends). Data passed between workgroups is
// written with device-scope stores, completed (vmcnt 0) before the record or counter that
// announces it, and read with device-scope loads issued after the announcement was read, so a
// reader sees it on any XCD without cache maintenance. Workgroups only wait for workgroups of
// smaller index, which the dispatcher starts first. Waits are bounded (10 ms): a workgroup that
// times out sets bit 0 of `status` and its outputs are NaN.
constexpr int kFusedCtr = 64;   // counter words per region (distinct experts of a call ≤ 16·4)
// Whole wave: true once *c holds n, false past the deadline. Polls are spaced (≈ 0.2 µs) so
// that hundreds of waiting waves leave the memory atomics to the writers.
__device__ __forceinline__ bool wait_count(const uint32_t *c, uint32_t n, uint64_t deadline) {
  for (;;) {
    uint32_t v = 0;
    if ((threadIdx.x & 63) == 0) v = __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(v) == n) return true;
    if (wall_clock64() > deadline) return false;
    __builtin_amdgcn_s_sleep(8);
  }
}

template <bool GEMMA>
__global__ __launch_bounds__(256, 2) void decode_mx(GemmArgs a, RouteArgs ra, FuseArgs f) {
  constexpr int NM = 1, DA = MX_ONE_CHUNKS;
  extern __shared__ __align__(16) uint8_t s_dyn[];
  __shared__ int s_idx[SMALL_T * kMaxTopK];
  __shared__ float s_w[SMALL_T * kMaxTopK];
  __shared__ f32x4 s_up[2][64];
  __shared__ float s_hv[SMALL_T][UP_ROWS];
  __shared__ double s_lg[4][64];
  __shared__ double s_lgall[SMALL_T * (kFusedMaxE + 1)];
  __shared__ int s_ri[4][kMaxTopK];
  __shared__ float s_o[4][16];
  __shared__ int s_flag, s_bad;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int T = ra.tokens, E = a.experts, E1 = E + 1, K = a.top_k, S = a.slots, H = a.hidden;
  const int b = blockIdx.x;
  const uint64_t deadline = wall_clock64() + 1000000;   // 10 ms at 100 MHz
  uint32_t *ctr_base = f.ctr;
  uint32_t *ctr = ctr_base + kFusedCtr * (f.seq & 1);                   // this call's, per plan expert

  // ---- router ----
  if (b < f.R) {
    __shared__ double s_acc[4][64];
    __shared__ double s_px[4][2][64];
    const int t = b / E1, e = b - t * E1;
    double v = 0.0;
    if (e < E || ra.shared_gate) v = split_pair_logit<GEMMA>(ra, t, e, s_acc, s_px);
    if (wave == 0) store_logit_record(f.flags, f.R, b, v, f.epoch, lane);
    return;
  }

  const bool up_role = b < f.R + f.U;
  if (up_role) HH_TR(1, 0); else HH_TR(2, 0);
  if (tid == 0) s_bad = 0;
  // Gate-up workgroups quantise x while the router runs.
  const int RS = mx_row_bytes(a.xld);
  if (up_role) quant_x_lds(ra.x, T, H, a.xld, s_dyn, RS);
  if (wave == 0) {
    const bool ok = wait_logit_records(f.flags, f.R, b % kRecReplicas, f.R, f.epoch, deadline, s_lgall);
    if (lane == 0) s_flag = ok ? 1 : 0;
  }
  __syncthreads();
  if (!s_flag) {
    if (tid == 0) atomicOr(f.status, 1u);
    if (!up_role) {
      // Down items of this workgroup: NaN rows.
      for (int it = b - f.R - f.U; it < a.row_tiles * T; it += f.D)
        if (tid < 16) a.y[(size_t)(it % T) * H + (it / T) * 16 + tid] = __builtin_nanf("");
    }
    return;
  }
  // Top-k of every token (wave w: tokens w, w + 4, ...). The first gate-up workgroup writes the
  // routing outputs; down workgroups keep the weights.
  for (int t = wave; t < T; t += 4) {
    const double *lg = s_lgall + (size_t)t * E1;
    TopK tk = E <= 64 ? topk_rank64(lg, E, K, s_lg[wave], s_ri[wave]) : topk_exact(lg, E, K);
    prob_order(tk, K, ra.router);
    if (lane < K) s_idx[t * K + lane] = tk.index_of(lane);
    if (b == f.R) finish_token(ra, t, tk, ra.shared_gate ? lg[E] : 0.0);
    if (!up_role) {
      double v;
      int e;
      const double w = token_weight(ra, tk, v, e);
      if (lane < K) s_w[t * K + lane] = (float)w;
    }
  }
  __syncthreads();
  const Plan plan(s_idx, T, K, E);
  const int nu = plan.nu;
  const int rtr = a.grp[0].inter / UP_ROWS;
  const int nitems = nu * rtr;
  if (up_role) HH_TR(1, 1); else HH_TR(2, 1);

  if (up_role) {
    if (b == f.R && tid < kFusedCtr)   // the next call's counters
      __hip_atomic_store(ctr_base + kFusedCtr * ((f.seq + 1) & 1) + tid, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // ---- gate-up: as up_small_mx with x already in LDS ----
    const int q = wave & 1;
    const bool is_up = wave >= 2;
    const int nch = (H + 127) / 128;
    const int nsb = H / 32;
    uint8_t *s_sc = s_dyn + (size_t)T * NTX * RS;   // [64][nsb]
    const int nsv = scale_vectors(64, H);
    for (int it = b - f.R; it < nitems; it += f.U) {
      const int u = it / rtr, rt = it - u * rtr;
      int e;
      uint64_t tm;
      plan.entry(u, e, tm);
      const int ntok = __popcll(tm);
      const ExpertGroup &grp = a.grp[0];
      const uint8_t *blob = grp.blobs + (size_t)e * grp.stride;
      const int rb = rt * UP_ROWS + 16 * q;
      const uint8_t *gsc = blob + grp.off[1] + (size_t)rt * 64 * nsb;
      u32x4 scv[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) scv[k] = *(const u32x4 *)(gsc + 16 * min(tid + 256 * k, nsv - 1));
      u32x4 bias = {0u, 0u, 0u, 0u};
      if (!is_up && a.expert_bias) bias = *(const u32x4 *)(blob + grp.off[2] + 4 * (rb + 4 * g));
      ATile<Q_MXFP4_W> at[NM] = {tile_of<PH_UP, Q_MXFP4_W>(blob, grp, rb, is_up, H, l16)};
      AStream<Q_MXFP4_W, NM, DA> as(0, 1, nch);
      as.fill(at, nch, g, H);
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (tid + 256 * k < nsv) *(u32x4 *)(s_sc + 16 * (tid + 256 * k)) = scv[k];
      for (int v = tid + 512; v < nsv; v += 256) *(u32x4 *)(s_sc + 16 * v) = *(const u32x4 *)(gsc + 16 * v);
      __syncthreads();
      const uint8_t *my_sc = s_sc + (2 * (16 * q + l16) + (is_up ? 1 : 0)) * nsb;
      int gi = g;
      asm volatile("" : "+v"(gi));
      const int my_t = nth_bit(tm, min(l16, ntok - 1));
      const uint8_t *brow = s_dyn + (size_t)my_t * NTX * RS;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      as.template run_pf<true>(
          at, nch, gi, H, [&](int c) { return mx_ops<NTX>(brow, RS, a.xld, my_sc, nsb, c, gi); },
          [&](const Fmt<Q_MXFP4_W>::A (&w)[NM], int c, const MxOps<NTX> &o) { chunk_mx1<NTX>(acc, w[0].w, o, c, gi, H); });
      if (is_up) s_up[q][lane] = acc;
      if (it == b - f.R) HH_TR(1, 2);
      __syncthreads();
      if (!is_up && l16 < ntok) {
        const f32x4 y = up_values_mx(a, bias, acc, s_up[q][lane]);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) s_hv[l16][16 * q + 4 * g + ii] = y[ii];
      }
      __syncthreads();
      if (wave == 0) {
        const int j = min(l16, ntok - 1);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = s_hv[j][8 * g + i];
        uint32_t hq[NTH][2], sb[NTH];
        quant_block<NTH>(v, hq, sb);
        if (l16 < ntok) {
          const int t = nth_bit(tm, l16);
          const int slot = t * S + rank_of(s_idx, t, e, K, false);
          store_hq<true>(a, slot, rt, rt * UP_ROWS + 8 * g, rt * UP_ROWS + 8 * g + 4, hq, sb, g);
        }
        wait_stores();
        if (lane == 0) __hip_atomic_fetch_add(ctr + u, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (it == b - f.R) HH_TR(1, 3);
      }
    }
    return;
  }

  // ---- down: wave r = slot r of the item's token ----
  const int r = wave;
  const int I = a.grp[0].inter;
  const int nch = (I + 127) / 128;
  const int nsb = I / 32, nsv = scale_vectors(16, I);
  const int RSH = mx_row_bytes(a.hld);
  const int slot_bytes = NTH * RSH + 16 * ((16 * nsb + 15) / 16);
  uint8_t *my_lds = s_dyn + (size_t)r * slot_bytes;
  uint8_t *s_sc = my_lds + NTH * RSH;
  for (int it = b - f.R - f.U; it < a.row_tiles * T; it += f.D) {
    const int rt = it / T, t = it - rt * T;
    const int rb = rt * 16;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (r < K) {
      const int slot = t * S + r;
      const int e = s_idx[t * K + r];
      const ExpertGroup &grp = a.grp[0];
      const uint8_t *blob = grp.blobs + (size_t)e * grp.stride;
      const uint8_t *gsc = blob + grp.off[4] + (size_t)rb * nsb;
      u32x4 scv[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) scv[k] = *(const u32x4 *)(gsc + 16 * min(lane + 64 * k, nsv - 1));
      ATile<Q_MXFP4_W> aw[NM] = {tile_of<PH_DOWN, Q_MXFP4_W>(blob, grp, rb, false, I, l16)};
      AStream<Q_MXFP4_W, NM, DA> as(0, 1, nch);
      as.fill(aw, nch, g, I);
      if (it == b - f.R - f.U && r == 0) HH_TR(2, 2);
      float db[4] = {0.f, 0.f, 0.f, 0.f};
      if (a.expert_bias && l16 == 0) {
        const uint16_t *bias = (const uint16_t *)(blob + grp.off[5]);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) db[ii] = bf16_bits_to_f32(bias[rb + 4 * g + ii]);
      }
      // The h terms of this slot exist once every gate-up item of its expert is done.
      const int u = plan.index_of(e);
      const bool ok = wait_count(ctr + u, (uint32_t)rtr, deadline);
      if (!ok && lane == 0) {
        s_bad = 1;
        atomicOr(f.status, 1u);
      }
      if (it == b - f.R - f.U && r == 0) HH_TR(2, 3);
      // The lane id as a value opaque to the compiler in each item, so the staging addresses are
      // computed here rather than hoisted out of the item loop and held across it.
      int li = lane;
      asm volatile("" : "+v"(li));
      auto hs = mx_stage<NTH, 9, true>(my_lds, a.hq, a.hs, a.hld, I, 1, [&](int) { return slot; }, li, 64);
      hs.load_first();
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (li + 64 * k < nsv) *(u32x4 *)(s_sc + 16 * (li + 64 * k)) = scv[k];
      for (int v = li + 128; v < nsv; v += 64) *(u32x4 *)(s_sc + 16 * v) = *(const u32x4 *)(gsc + 16 * v);
      hs.store_first();
      hs.rest();
      hs.pad();
      __builtin_amdgcn_s_waitcnt(0xc07f);   // this wave's LDS stores (lgkmcnt 0)
      __builtin_amdgcn_wave_barrier();
      if (it == b - f.R - f.U && r == 0) HH_TR(2, 4);
      const uint8_t *my_sc = s_sc + l16 * nsb;
      int gi = g;
      asm volatile("" : "+v"(gi));
      as.template run_pf<true>(
          aw, nch, gi, I, [&](int c) { return mx_ops<NTH>(my_lds, RSH, a.hld, my_sc, nsb, c, gi); },
          [&](const Fmt<Q_MXFP4_W>::A (&w)[NM], int c, const MxOps<NTH> &o) { chunk_mx1<NTH>(acc, w[0].w, o, c, gi, I); });
      if (it == b - f.R - f.U && r == 0) HH_TR(2, 5);
      if (l16 == 0) {
        const float w = s_w[t * K + r];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) s_o[r][4 * g + ii] = w * (acc[ii] + db[ii]);
      }
    }
    __syncthreads();
    if (tid < 16) {
      float y = s_o[0][tid];
      for (int qq = 1; qq < K; ++qq) y += s_o[qq][tid];
      a.y[(size_t)t * H + rb + tid] = s_bad ? __builtin_nanf("") : y;
    }
    if (it == b - f.R - f.U) HH_TR(2, 6);
    __syncthreads();   // the next item rewrites the LDS rows and s_o
  }
}

// ---- prefill, MXFP4, producer/consumer workgroups ----------------------------------------------------
// 8 waves: waves 4-7 load, waves 0-3 multiply. Per 128-column chunk the loaders bring the chunk of
// the workgroup's 128 weight rows (8 KiB of fp4 blocks) and of the pass's NTOK token operands
// (NTERM fp8 terms × 128 B each, XOR-swizzled by token, plus their block scales) into a
// double-buffered LDS stage, keeping R chunks in flight in their registers; the weight rows' e8m0
// scales for the whole K are staged once. One barrier per chunk. The MFMA waves form a 2 × 2
// grid of 64 rows × 16·NTW tokens (4 row tiles × NTW token tiles each). Weight rows are the
// matrix's consecutive rows: for gate_up (gate/up interleaved, ReferenceLayer.swift:11) a tile
// holds 8 intermediates' gate and up rows, so each lane pairs gate and up in its own D fragment,
// and a wave's 64 rows are one 32-intermediate block of the activation terms. Per output
// element the arithmetic is the canonical one (the decode kernels' bits).
template <int PH, int NTW>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void prefill_mx2(GemmArgs a) {
  constexpr int NTERM = (PH == PH_UP) ? NTX : NTH;
  constexpr int NTOK = 32 * NTW;            // tokens per pass
  constexpr int MR = 128;                   // weight rows per workgroup
  constexpr int AV = MR * 4;                // 16-byte weight vectors per chunk
  constexpr int BV = NTERM * NTOK * 8;      // 16-byte operand vectors per chunk
  constexpr int BS = NTERM * NTOK;          // operand scale dwords per chunk
  constexpr int APL = AV / 256;             // per loader thread
  constexpr int BPL = (BV + 255) / 256;
  // Loader ring depth (chunks in flight), within the 128 registers that let two workgroups
  // share a compute unit.
  constexpr int R = (APL + BPL) * 4 * 3 <= 80 ? 3 : 2;
  static_assert(AV % 256 == 0 && BS <= 256, "loader assignment");
  __shared__ __align__(16) u32x4 sA[2][AV];
  __shared__ __align__(16) u32x4 sB[2][BV];
  __shared__ uint32_t sBs[2][BS];
  __shared__ float sBias[MR];                       // bias of the workgroup's weight rows
  extern __shared__ __align__(16) uint8_t sAS[];   // [MR][K/32] weight scales

  int rt, wi;
  prefill_tile(blockIdx.x, a.row_tiles, rt, wi);
  if (rt >= a.row_tiles || wi >= *a.n_work) return;
  const int4 item = a.work[wi];
  const int e = item.x, pos0 = item.y, nitem = item.z;
  const int gsel = (e == a.experts) ? 1 : 0;
  const ExpertGroup &grp = a.grp[gsel];
  const uint8_t *blob = grp.blobs + (gsel ? 0 : (size_t)e * grp.stride);
  const int I = grp.inter, H = a.hidden;
  const int out_dim = (PH == PH_UP) ? 2 * I : H;    // weight rows of the matrix
  const int K = (PH == PH_UP) ? H : I;
  const int r0 = rt * MR;
  if (r0 >= out_dim) return;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int nch = (K + 127) / 128, nsb = K / 32;
  const uint8_t *wblk = blob + grp.off[PH == PH_UP ? 0 : 3];
  const uint8_t *wsc = blob + grp.off[PH == PH_UP ? 1 : 4];
  const int ld = PH == PH_UP ? a.xld : a.hld;
  const uint8_t *qbase = PH == PH_UP ? a.xq : a.hq;
  const uint8_t *sbase = PH == PH_UP ? a.xs : a.hs;

  // Weight scales of the valid rows (16-row granular), whole K, and the rows' biases.
  const int vrows = min(MR, out_dim - r0);
  for (int v = tid; v < vrows * nsb / 16; v += 512)
    *(u32x4 *)(sAS + 16 * v) = *(const u32x4 *)(wsc + (size_t)r0 * nsb + 16 * v);
  if (tid < MR) {
    const uint16_t *bias = (const uint16_t *)(blob + grp.off[PH == PH_UP ? 2 : 5]);
    sBias[tid] = a.expert_bias ? bf16_bits_to_f32(bias[min(r0 + tid, out_dim - 1)]) : 0.f;
  }

  for (int t0 = 0; t0 < nitem; t0 += NTOK) {
    const int ntok = min(NTOK, nitem - t0);
    auto slot_of = [&](int n) { return a.order[pos0 + t0 + min(n, ntok - 1)]; };
    if (wave >= 4) {
      // ---- loaders ----
      const int lt = tid - 256;
      const uint8_t *asrc[APL];
      int ag[APL];
      const uint8_t *bsrc[BPL];
      const uint8_t *ssrc;
#pragma unroll
      for (int k = 0; k < APL; ++k) {
        // Vector v = (tile j, lane i): row 16j + i%16, block g = i/16 of the chunk.
        const int v = lt + 256 * k, j = v >> 6, i = v & 63;
        const int r = min(r0 + 16 * j + (i & 15), out_dim - 1);
        asrc[k] = wblk + (size_t)r * (K / 2);
        ag[k] = i >> 4;
      }
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const int v = min(lt + 256 * k, BV - 1);
        const int tt = v / (NTOK * 8), sl = v % (NTOK * 8), n = sl >> 3, sg = (sl & 7) ^ (n & 7);
        const int row = PH == PH_UP ? slot_of(n) / a.slots : slot_of(n);
        bsrc[k] = qbase + ((size_t)row * NTERM + tt) * ld + 16 * sg;
      }
      {
        const int v = min(lt, BS - 1), tt = v / NTOK, n = v % NTOK;
        const int row = PH == PH_UP ? slot_of(n) / a.slots : slot_of(n);
        ssrc = sbase + ((size_t)row * NTERM + tt) * (ld / 32);
      }
      u32x4 ra[R][APL], rb[R][BPL];
      uint32_t rs[R];
      auto issue = [&](int u, int c) {
        const int cc = min(c, nch - 1);
#pragma unroll
        for (int k = 0; k < APL; ++k) ra[u][k] = *(const u32x4 *)(asrc[k] + 16 * min(4 * cc + ag[k], nsb - 1));
#pragma unroll
        for (int k = 0; k < BPL; ++k) rb[u][k] = *(const u32x4 *)(bsrc[k] + 128 * cc);
        rs[u] = *(const uint32_t *)(ssrc + 4 * cc);
      };
      auto put = [&](int u, int buf) {
#pragma unroll
        for (int k = 0; k < APL; ++k) sA[buf][lt + 256 * k] = ra[u][k];
#pragma unroll
        for (int k = 0; k < BPL; ++k)
          if (lt + 256 * k < BV) sB[buf][lt + 256 * k] = rb[u][k];
        if (lt < BS) sBs[buf][lt] = rs[u];
      };
#pragma unroll
      for (int u = 0; u < R; ++u) issue(u, u);
      for (int c0 = 0; c0 < nch; c0 += R) {
#pragma unroll
        for (int u = 0; u < R; ++u) {
          const int c = c0 + u;
          if (c < nch) {
            put(u, c & 1);
            __syncthreads();
            issue(u, c + R);
          }
        }
      }
    } else {
      // ---- MFMA waves ----
      const int wr = wave & 1, wt = wave >> 1;
      const int rw = r0 + 64 * wr;              // first weight row of this wave
      // Epilogue operands fetched now, off the critical path: slot ids and routing weights.
      int eslot[NTW];
      float ew[NTW];
#pragma unroll
      for (int st = 0; st < NTW; ++st) {
        eslot[st] = slot_of(16 * NTW * wt + 16 * st + l16);
        ew[st] = PH == PH_DOWN ? a.slot_w[eslot[st]] : 0.f;
      }
      f32x4 acc[4][NTW];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int st = 0; st < NTW; ++st) acc[j][st] = f32x4{0.f, 0.f, 0.f, 0.f};
      auto compute = [&](int c) {
        const int buf = c & 1;
        const bool ok = 128 * c + 32 * g < K;
        u32x4 w[4];
        uint32_t sa[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          w[j] = ok ? sA[buf][(4 * wr + j) * 64 + lane] : u32x4{0u, 0u, 0u, 0u};
          sa[j] = sAS[(64 * wr + 16 * j + l16) * nsb + min(4 * c + g, nsb - 1)];
        }
#pragma unroll
        for (int t = 0; t < NTERM; ++t)
#pragma unroll
          for (int st = 0; st < NTW; ++st) {
            const int n = 16 * NTW * wt + 16 * st + l16;
            const int k0 = 128 * c + 16 * g;
            u32x4 blo = sB[buf][(t * NTOK + n) * 8 + (g ^ (n & 7))];
            u32x4 bhi = sB[buf][(t * NTOK + n) * 8 + ((4 + g) ^ (n & 7))];
            uint32_t bs = (sBs[buf][t * NTOK + n] >> (8 * g)) & 0xFFu;
            if (k0 >= K) blo = u32x4{0u, 0u, 0u, 0u};
            if (k0 + 64 >= K) bhi = u32x4{0u, 0u, 0u, 0u};
            if (!ok) bs = 127u;
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j][st] = smfma(w[j], blo, bhi, sa[j], bs, acc[j][st]);
          }
      };
      for (int c = 0; c < nch; ++c) {
        __syncthreads();
        compute(c);
      }
      // ---- epilogue ----
      if (rw < out_dim) {
#pragma unroll
        for (int st = 0; st < NTW; ++st) {
          const int n = 16 * NTW * wt + 16 * st + l16;
          const int slot = eslot[st];
          if constexpr (PH == PH_UP) {
            // Tile j, lane group g: rows rw + 16j + 4g + {0..3} = (gate, up) of intermediates
            // rw/2 + 8j + 2g + {0, 1}.
            float v[8], gv[8], uv[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const f32x4 d = acc[j][st];
              const float *bb = sBias + 64 * wr + 16 * j + 4 * g;
              gv[2 * j] = d[0] + bb[0];
              uv[2 * j] = d[1] + bb[1];
              gv[2 * j + 1] = d[2] + bb[2];
              uv[2 * j + 1] = d[3] + bb[3];
            }
            activate_n<8>(a.act, gv, uv, v, a.alpha, a.limit);
            uint32_t hq[NTH][2], sb[NTH];
            quant_block<NTH>(v, hq, sb);
            if (n < ntok) {
              const int i0 = rw / 2;
#pragma unroll
              for (int t = 0; t < NTH; ++t) {
                uint8_t *row = a.hq + ((size_t)slot * NTH + t) * a.hld + i0 + 2 * g;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                  *(uint16_t *)(row + 8 * j) = (uint16_t)(hq[t][j >> 1] >> (16 * (j & 1)));
                if (g == 0) a.hs[((size_t)slot * NTH + t) * (a.hld / 32) + i0 / 32] = (uint8_t)sb[t];
              }
            }
          } else {
            if (n < ntok) {
              const float wgt = ew[st];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const int h0 = rw + 16 * j + 4 * g;
                const f32x4 r = acc[j][st];
                const float *bb = sBias + 64 * wr + 16 * j + 4 * g;
                f32x4 o;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) o[ii] = wgt * (r[ii] + bb[ii]);   // down_value's arithmetic
                *(f32x4 *)(a.slot_out + (size_t)slot * H + h0) = o;
              }
            }
          }
        }
      }
    }
    __syncthreads();   // the next pass restages the buffers
  }
}

#ifndef HH_GEMM_KERNELS_ONLY
// y[t][j] = Σ_r slot[t·slots + r][j] in rank order (sum_expert_slices, dense.metal:147; the
// shared expert's slot comes last as in QwenReferenceLayer.swift:399-404).
__global__ __launch_bounds__(256) void combine_kernel(const float *slot_out, int slots, int H,
                                                      int T, float *y, const float *resid) {
  const size_t n4 = (size_t)T * H / 4;
  for (size_t q = blockIdx.x * 256ull + threadIdx.x; q < n4; q += (size_t)gridDim.x * 256) {
    const size_t t = (q * 4) / H, j = (q * 4) % H;
    const f32x4 *src = (const f32x4 *)(slot_out + t * slots * H + j);
    f32x4 s = src[0];
    for (int r = 1; r < slots; ++r) {
      const f32x4 v = src[(size_t)r * H / 4];
      s[0] += v[0]; s[1] += v[1]; s[2] += v[2]; s[3] += v[3];
    }
    if (resid) {   // the residual stream: y = resid + mixture (ReferenceLayer.swift:202)
      const f32x4 r = *(const f32x4 *)(resid + t * H + j);
      s[0] = r[0] + s[0]; s[1] = r[1] + s[1]; s[2] = r[2] + s[2]; s[3] = r[3] + s[3];
    }
    *(f32x4 *)(y + t * H + j) = s;
  }
}
#endif

// ---- prefill, MXFP4: persistent pipeline with direct-to-LDS loads -----------------------------
// One 512-thread workgroup per compute unit takes tasks τ = blockIdx.x, + gridDim.x, ... in
// prefill_tile order (a task: 128 weight rows × one work item of ≤ 32 tokens). Waves 4-7 load,
// waves 0-3 multiply (2×2: 64 rows × 16 tokens each). The loaders stream every task's 128-column
// chunks (weight blocks, the rows' block scales, the tokens' fp8 terms and their scales) straight
// into a ring of S LDS stages with global_load_lds, S−1 chunks ahead of the MFMA waves and across
// task boundaries, so neither a chunk's memory latency nor a task's start is waited for. Each
// loader wave issues at least L loads per chunk, so "the oldest chunk has landed" is the fixed wait
// vmcnt((S−2)·L); the task switches' extra loads (work item and slot ids, fetched into LDS one and
// two tasks ahead) only make that wait stricter. The arithmetic per output element is
// prefill_mx2's: one chain over the chunks, the terms in order.
// RR: 128-row halves of the weight tile (MR = 128·RR rows); TT: 32-token halves of the token tile.
template <int PH, int RR, int TT> struct Mx3 {
  static constexpr int NTERM = PH == PH_UP ? NTX : NTH;
  static constexpr int NTOK = 32 * TT, MR = 128 * RR;
  static constexpr int B_INS = NTERM * NTOK / 8;            // 1 KB operand loads per chunk
  static constexpr int BPW = B_INS / 4;                     // per loader wave
  static constexpr int BS_DW = NTERM * NTOK;                // operand scale dwords per chunk
  static constexpr int L = 2 * RR + BPW + 1 + 1;            // loads per loader wave per chunk
  static constexpr int OFF_B = 8192 * RR;                   // after 8·RR weight tiles of 1 KB
  static constexpr int OFF_BS = OFF_B + B_INS * 1024;
  static constexpr int OFF_SC = OFF_BS + 256 * ((BS_DW + 63) / 64);
  static constexpr int STAGE = OFF_SC + 512 * RR;           // + MR rows × 4 block-scale bytes
  static constexpr int S_FIT = (150 * 1024 - 1792) / STAGE;
  static constexpr int S = S_FIT > 8 ? 8 : S_FIT;
  static constexpr int OFF_INFO = S * STAGE;                // [3][64] work item (4 dwords used)
  static constexpr int OFF_ORDER = OFF_INFO + 3 * 256;      // [3][64] slot ids (32 used)
  static constexpr int OFF_JUNK = OFF_ORDER + 3 * 256;      // sink of loads no stage needs
  static constexpr int LDS = OFF_JUNK + 256;
  static_assert(B_INS % 4 == 0 && BS_DW <= 256 && NTOK <= 64 && S >= 3 && (S - 2) * L <= 63, "loader layout");
};

// Workgroup barrier without __syncthreads' release fence: the fence would make every wave wait for
// all of its direct-to-LDS loads (vmcnt(0)) before the barrier; the pipeline orders LDS itself
// with explicit waits. A compiler memory barrier keeps LDS accesses on their side.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) void *lds_ptr_t;
__device__ __forceinline__ void lds_load16(const void *g, uint8_t *l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void *g, uint8_t *l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 4, 0, 0);
}

// Task ids of one workgroup of a persistent prefill kernel: τ = b, b + G, ... (G a multiple of
// 8, so τ mod 8 is the workgroup's XCD), skipping tasks past the row tiles or the work items.
// The 8 XCDs form P row-tile parts × 8/P work-item parts: XCD x takes row tiles of part x mod P
// and work items of part x / P, work item by work item (each item's row tiles consecutively).
// An expert's slice of weight rows stays in the XCD's L2 across the expert's consecutive items,
// and an item's operand rows are fetched by the P XCDs of its item part.
struct Mx3Tasks {
  int b, G, RT, nwork, P, rtp, nq, lim;
  __device__ __forceinline__ Mx3Tasks(int b_, int G_, int RT_, int nwork_, int P_)
      : b(b_), G(G_), RT(RT_), nwork(nwork_), P(P_ == 1 || P_ == 2 || P_ == 4 ? P_ : 8) {
    rtp = (RT + P - 1) / P;
    nq = (nwork + 8 / P - 1) / (8 / P);
    lim = 8 * rtp * nq;
  }
  __device__ __forceinline__ void tile(int tau, int &rt, int &wi) const {
    const int x = tau & 7, j = tau >> 3, q = j / rtp;
    rt = (x & (P - 1)) * rtp + (j - q * rtp);
    wi = (x / P) * nq + q;
  }
  __device__ __forceinline__ int first() const { return fix(b); }
  __device__ __forceinline__ int next(int tau) const { return fix(tau + G); }
  __device__ __forceinline__ int fix(int tau) const {
    for (; tau < lim; tau += G) {
      int rt, wi;
      tile(tau, rt, wi);
      if (rt < RT && wi < nwork) return tau;
    }
    return lim;
  }
};

template <int PH, int RR, int TT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mx3(GemmArgs a) {
  using C = Mx3<PH, RR, TT>;
  constexpr int NTERM = C::NTERM, NTOK = C::NTOK, S = C::S, L = C::L;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const ExpertGroup &grp = a.grp[0];
  const int I = grp.inter, H = a.hidden;
  const int out_dim = PH == PH_UP ? 2 * I : H;
  const int K = PH == PH_UP ? H : I;
  const int nch = (K + 127) / 128, nsb = K / 32;
  const int ld = PH == PH_UP ? a.xld : a.hld;
  const uint8_t *qbase = PH == PH_UP ? a.xq : a.hq;
  const uint8_t *sbase = PH == PH_UP ? a.xs : a.hs;
  const int RT = a.row_tiles, rtx = (RT + 7) >> 3;
  const int nwork = *a.n_work;
  const Mx3Tasks tasks((int)blockIdx.x, (int)gridDim.x, RT, nwork, a.xcd_rows);
  // Number of chunks this workgroup computes.
  int nsteps = 0;
  for (int tau = tasks.first(); tau < tasks.lim; tau = tasks.next(tau)) nsteps += nch;
  if (nsteps == 0) return;
  uint8_t *info = lds + C::OFF_INFO, *order = lds + C::OFF_ORDER, *junk = lds + C::OFF_JUNK;
  auto item_of = [&](int slot) { return *(const int4 *)(info + 256 * slot); };

  if (wave >= 4) {
    // ---- loaders ----
    const int lw = wave - 4;
    // Work item (lanes 0-3) and slot ids (lanes 0-31) of a task into its LDS slot (other lanes
    // repeat valid entries). Every loader wave fetches them (the same values), so each one's own
    // vmcnt tells it they have landed.
    auto fetch_info = [&](int tau, int slot) {
      int rt, wi;
      tasks.tile(min(tau, tasks.lim - 1), rt, wi);
      lds_load4((const int *)(a.work + min(wi, nwork - 1)) + min(lane, 3), info + 256 * slot);
    };
    auto fetch_order = [&](int slot) {
      const int4 it = item_of(slot);
      lds_load4(a.order + it.y + min(lane, it.z - 1), order + 256 * slot);
    };
    // Per-task source pointers.
    const uint8_t *asrc[2 * RR], *bsrc[C::BPW], *bssrc, *scsrc;
    auto start_task = [&](int tau, int slot) {
      int rt, wi;
      tasks.tile(tau, rt, wi);
      const int4 it = item_of(slot);
      const int r0 = rt * C::MR;
      const uint8_t *blob = grp.blobs + (size_t)it.x * grp.stride;
      const uint8_t *wblk = blob + grp.off[PH == PH_UP ? 0 : 3];
      const uint8_t *wsc = blob + grp.off[PH == PH_UP ? 1 : 4];
      const int *ord = (const int *)(order + 256 * slot);
      auto row_of = [&](int n) {
        const int sl = ord[min(n, it.z - 1)];
        return PH == PH_UP ? sl / a.slots : sl;
      };
#pragma unroll
      for (int k = 0; k < 2 * RR; ++k) {
        const int j = 2 * RR * lw + k;   // 16-row tile of the chunk
        asrc[k] = wblk + (size_t)min(r0 + 16 * j + l16, out_dim - 1) * (K / 2);
      }
#pragma unroll
      for (int k = 0; k < C::BPW; ++k) {
        const int v = (lw * C::BPW + k) * 64 + lane;
        const int t = v / (NTOK * 8), sl = v % (NTOK * 8), n = sl >> 3, sg = (sl & 7) ^ (n & 7);
        bsrc[k] = qbase + ((size_t)row_of(n) * NTERM + t) * ld + 16 * sg;
      }
      {
        const int d = min(lw * 64 + lane, C::BS_DW - 1), t = d / NTOK, n = d % NTOK;
        bssrc = sbase + ((size_t)row_of(n) * NTERM + t) * (ld / 32);
      }
      // Block scales: one row's 4 bytes of a chunk per lane (4-byte loads from 2-byte-aligned
      // rows are exact; a 2-byte direct-to-LDS load would write a whole dword per lane).
      scsrc = wsc + (size_t)min(r0 + min(lw, 2 * RR - 1) * 64 + lane, out_dim - 1) * nsb;
    };
    // Chunk c of the current task into stage st.
    auto issue = [&](int c, int st) {
      uint8_t *stg = lds + st * C::STAGE;
#pragma unroll
      for (int k = 0; k < 2 * RR; ++k)
        lds_load16(asrc[k] + 16 * min(4 * c + g, nsb - 1), stg + 1024 * (2 * RR * lw + k));
#pragma unroll
      for (int k = 0; k < C::BPW; ++k) lds_load16(bsrc[k] + 128 * c, stg + C::OFF_B + 1024 * (lw * C::BPW + k));
      lds_load4(bssrc + 4 * c, lw * 64 < C::BS_DW ? stg + C::OFF_BS + 256 * lw : junk);
      lds_load4(scsrc + 4 * c, lw < 2 * RR ? stg + C::OFF_SC + 256 * lw : junk);
    };
    // Prologue: work items of the first two tasks and the first task's slot ids, then the first
    // S−1 chunks.
    int tq[3];   // task ids: issuing, next, the one after
    tq[0] = tasks.first();
    tq[1] = tasks.next(tq[0]);
    tq[2] = tasks.next(tq[1]);
    fetch_info(tq[0], 0);
    fetch_info(tq[1], 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    fetch_order(0);
    fetch_order(1);
    fetch_info(tq[2], 2);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int slot = 0, lc = 0;
    start_task(tq[0], 0);
    int q = 0;   // chunks issued
    auto issue_next = [&]() {
      issue(lc, q % S);
      ++q;
      if (++lc == nch) {
        lc = 0;
        // Next task: its work item and slot ids have landed (fetched ≥ one task ago).
        tq[0] = tq[1];
        tq[1] = tq[2];
        tq[2] = tasks.next(tq[2]);
        slot = slot == 2 ? 0 : slot + 1;
        if (tq[0] < tasks.lim) {
          start_task(tq[0], slot);
          const int s1 = slot == 2 ? 0 : slot + 1, s2 = s1 == 2 ? 0 : s1 + 1;
          fetch_order(s1);            // slot ids of the next task (its work item landed)
          fetch_info(tq[2], s2);      // work item of the task after it
        }
      }
    };
    // At every barrier the chunk being computed and the next one (whose operands the MFMA waves
    // read ahead) have landed: after issuing chunk q, wait until at most S−3 chunks' loads are
    // outstanding.
    for (int u = 0; u < S - 1 && q < nsteps; ++u) issue_next();
    if (q >= S - 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 3) * L) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (int step = 0; step < nsteps; ++step) {
      ring_barrier();
      if (q < nsteps) {
        issue_next();
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 3) * L) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }
    return;
  }

  // ---- MFMA waves ----
  // Wave (wr, wt): weight rows r0 + 64·RR·wr + 16j (j < 4·RR), tokens 16·TT·wt + 16·tt + l16.
  const int wr = wave & 1, wt = wave >> 1;
  constexpr int NJ = 4 * RR;
  f32x4 acc[NJ][TT];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[j][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  int tau = tasks.first(), slot = 0, c = 0;
  int ntok = 0, r0 = 0;
  int eslot[TT];
  float ew[TT];
  uint16_t braw[NJ][4];   // bias bits of the lane's rows, loaded at the task's start, used at its end
  auto task_begin = [&]() {
    int rt, wi;
    tasks.tile(tau, rt, wi);
    const int4 it = item_of(slot);
    r0 = rt * C::MR;
    ntok = __builtin_amdgcn_readfirstlane(it.z);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      eslot[tt] = ((const int *)(order + 256 * slot))[min(16 * TT * wt + 16 * tt + l16, ntok - 1)];
      ew[tt] = PH == PH_DOWN ? a.slot_w[eslot[tt]] : 0.f;
    }
    // Unconditional loads (a branch on expert_bias would make the compiler wait for them here).
    const uint16_t *bp = (const uint16_t *)(grp.blobs + (size_t)it.x * grp.stride + grp.off[PH == PH_UP ? 2 : 5]);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) braw[j][ii] = bp[min(r0 + 64 * RR * wr + 16 * j + 4 * g + ii, out_dim - 1)];
  };
  // Operands of a chunk, read from its stage one step ahead of its MFMAs (raw: the chunk's masks
  // are applied at use).
  struct Ops {
    u32x4 w[NJ], blo[NTERM][TT], bhi[NTERM][TT];
    uint32_t sa[NJ], bs[NTERM][TT];
  };
  auto read_ops = [&](int st) {
    const uint8_t *stg = lds + st * C::STAGE;
    Ops o;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      o.w[j] = *(const u32x4 *)(stg + 1024 * (NJ * wr + j) + 16 * lane);
      o.sa[j] = stg[C::OFF_SC + 4 * (64 * RR * wr + 16 * j + l16) + g];
    }
    const u32x4 *sb = (const u32x4 *)(stg + C::OFF_B);
#pragma unroll
    for (int t = 0; t < NTERM; ++t)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int n = 16 * TT * wt + 16 * tt + l16;
        o.blo[t][tt] = sb[(t * NTOK + n) * 8 + (g ^ (n & 7))];
        o.bhi[t][tt] = sb[(t * NTOK + n) * 8 + ((4 + g) ^ (n & 7))];
        o.bs[t][tt] = (((const uint32_t *)(stg + C::OFF_BS))[t * NTOK + n] >> (8 * g)) & 0xFFu;
      }
    return o;
  };
  ring_barrier();
  Ops cur = read_ops(0);
  for (int step = 0; step < nsteps; ++step) {
    if (c == 0) task_begin();
    Ops nxt;
    if (step + 1 < nsteps) nxt = read_ops((step + 1) % S);
    if (128 * (c + 1) <= K) {
      // A whole chunk (every chunk but a partial last one): no lane masks.
#pragma unroll
      for (int t = 0; t < NTERM; ++t)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[j][tt] = smfma(cur.w[j], cur.blo[t][tt], cur.bhi[t][tt], cur.sa[j], cur.bs[t][tt], acc[j][tt]);
    } else {
      const bool ok = 128 * c + 32 * g < K;
      const int k0 = 128 * c + 16 * g;
#pragma unroll
      for (int t = 0; t < NTERM; ++t)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          // Lanes past K take zero weights; their scale byte may be any byte of the blob, so 2^0
          // (the product is the same signed zero).
          const u32x4 blo = k0 >= K ? u32x4{0u, 0u, 0u, 0u} : cur.blo[t][tt];
          const u32x4 bhi = k0 + 64 >= K ? u32x4{0u, 0u, 0u, 0u} : cur.bhi[t][tt];
          const uint32_t bs = ok ? cur.bs[t][tt] : 127u;
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[j][tt] = smfma(ok ? cur.w[j] : u32x4{0u, 0u, 0u, 0u}, blo, bhi, ok ? cur.sa[j] : 127u, bs, acc[j][tt]);
        }
    }
    const bool more = step + 1 < nsteps;
    if (++c < nch) {
      if (more) ring_barrier();
      cur = nxt;
      continue;
    }
    // ---- epilogue of the task ----
    c = 0;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      if (16 * TT * wt + 16 * tt >= ntok) break;   // padding tiles (also wt > 0 past the tokens)
      const int n = 16 * TT * wt + 16 * tt + l16;
#pragma unroll
      for (int h = 0; h < RR; ++h) {
        const int rw = r0 + 64 * RR * wr + 64 * h;   // a 64-row block: 32 intermediates of gate-up
        if (rw >= out_dim) continue;
        float bias[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) bias[j][ii] = a.expert_bias ? bf16_bits_to_f32(braw[4 * h + j][ii]) : 0.f;
        if constexpr (PH == PH_UP) {
          float v[8], gv[8], uv[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f32x4 d = acc[4 * h + j][tt];
            gv[2 * j] = d[0] + bias[j][0];
            uv[2 * j] = d[1] + bias[j][1];
            gv[2 * j + 1] = d[2] + bias[j][2];
            uv[2 * j + 1] = d[3] + bias[j][3];
          }
          activate_n<8>(a.act, gv, uv, v, a.alpha, a.limit);
          uint32_t hq[NTH][2], sbq[NTH];
          quant_block<NTH>(v, hq, sbq);
          if (n < ntok) {
            const int i0 = rw / 2;
#pragma unroll
            for (int t = 0; t < NTH; ++t) {
              uint8_t *row = a.hq + ((size_t)eslot[tt] * NTH + t) * a.hld + i0 + 2 * g;
#pragma unroll
              for (int j = 0; j < 4; ++j) *(uint16_t *)(row + 8 * j) = (uint16_t)(hq[t][j >> 1] >> (16 * (j & 1)));
              if (g == 0) a.hs[((size_t)eslot[tt] * NTH + t) * (a.hld / 32) + i0 / 32] = (uint8_t)sbq[t];
            }
          }
        } else {
          if (n < ntok) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int h0 = rw + 16 * j + 4 * g;
              f32x4 o;
#pragma unroll
              for (int ii = 0; ii < 4; ++ii) o[ii] = ew[tt] * (acc[4 * h + j][tt][ii] + bias[j][ii]);   // down_value's arithmetic
              *(f32x4 *)(a.slot_out + (size_t)eslot[tt] * H + h0) = o;
            }
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[j][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    tau = tasks.next(tau);
    slot = slot == 2 ? 0 : slot + 1;
    if (more) ring_barrier();
    cur = nxt;
  }
}

// ---- prefill, MXFP4: weight rows in registers, token operand through an LDS ring -----------------
// prefill_mx3's persistent task order and loader protocol, with the weight operand taken out of
// LDS: each MFMA wave owns 64 distinct weight rows of the task's 256-row tile (one 32-intermediate
// block of gate-up) and streams them straight into a DA-deep register ring that runs across task
// boundaries (the wave reads the next task's work item from the loaders' LDS copy when its stream
// crosses into it). The loaders only stage the 32 tokens' fp8 terms, their scales and the weight
// rows' block scales, so a stage is ~9 KB and the ring holds S = 12 of them: with the weight
// rows in the register file, about twice as many bytes are in flight per compute unit as when
// everything passes through LDS. Per output element the arithmetic is the canonical one.
// TT: 16-token tiles per wave (the whole token tile): 2 (32-token work items) or 4 (64).
#ifndef HH_MXA_DA
#define HH_MXA_DA 4
#endif
#ifndef HH_MXA_RA
#define HH_MXA_RA 1
#endif
template <int PH, int TT_ = 2> struct MxA {   // PH_UP (down's three terms leave too few registers)
  static constexpr int NTERM = PH == PH_UP ? NTX : NTH;
  static constexpr int TT = TT_, NTOK = 16 * TT, MR = 256, NJ = 4;
  // RA: an even step also reads the next step's operands (32-token items; 64-token items leave
  // no registers for a second set). DA: the weight ring's depth in chunks.
  static constexpr bool RA = TT == 2 && HH_MXA_RA;
  static constexpr int DA = TT == 2 ? HH_MXA_DA : 2;
  static constexpr int B_INS = NTERM * NTOK / 8;            // 1 KB operand loads per chunk
  static constexpr int BPW = B_INS / 4;                     // per loader wave
  static constexpr int BS_DW = NTERM * NTOK;                // operand scale dwords per chunk
  static constexpr int L = BPW + 1 + 1;                     // loads per loader wave per chunk
  static constexpr int OFF_BS = B_INS * 1024;
  static constexpr int OFF_SC = OFF_BS + 256 * ((BS_DW + 63) / 64);
  static constexpr int STAGE = OFF_SC + 4 * 256;            // + 256 rows × 4 block-scale bytes
  static constexpr int S = TT == 2 ? 12 : 8;
  static constexpr int OFF_INFO = S * STAGE;                // [3][64] work item (4 dwords used)
  static constexpr int OFF_ORDER = OFF_INFO + 3 * 256;      // [3][64] slot ids (NTOK used)
  static constexpr int OFF_BIAS = OFF_ORDER + 3 * 256;      // [3][256] bf16 bias of the tile's rows
  static constexpr int OFF_JUNK = OFF_BIAS + 3 * 512;       // sink of loads no stage needs
  static constexpr int LDS = OFF_JUNK + 256;
  static_assert(B_INS % 4 == 0 && BS_DW <= 256 && (S - 2) * L <= 63 && DA % 2 == 0 && LDS <= 160 * 1024, "loader layout");
};

template <int PH, int TT_>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mxa(GemmArgs a) {
  using C = MxA<PH, TT_>;
  constexpr int NTERM = C::NTERM, NTOK = C::NTOK, S = C::S, L = C::L, NJ = C::NJ, DA = C::DA;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const ExpertGroup &grp = a.grp[0];
  const int I = grp.inter, H = a.hidden;
  const int out_dim = PH == PH_UP ? 2 * I : H;
  const int K = PH == PH_UP ? H : I;
  const int nch = (K + 127) / 128, nsb = K / 32;
  const int ld = PH == PH_UP ? a.xld : a.hld;
  const uint8_t *qbase = PH == PH_UP ? a.xq : a.hq;
  const uint8_t *sbase = PH == PH_UP ? a.xs : a.hs;
  const int RT = a.row_tiles, rtx = (RT + 7) >> 3;
  const int nwork = *a.n_work;
  const Mx3Tasks tasks((int)blockIdx.x, (int)gridDim.x, RT, nwork, a.xcd_rows);
  int nsteps = 0;
  for (int tau = tasks.first(); tau < tasks.lim; tau = tasks.next(tau)) nsteps += nch;
  if (nsteps == 0) return;
  uint8_t *info = lds + C::OFF_INFO, *order = lds + C::OFF_ORDER, *junk = lds + C::OFF_JUNK;
  auto item_of = [&](int slot) { return *(const int4 *)(info + 256 * slot); };

  if (wave >= 4) {
    // ---- loaders (prefill_mx3's, without the weight blocks) ----
    const int lw = wave - 4;
    auto fetch_info = [&](int tau, int slot) {
      int rt, wi;
      tasks.tile(min(tau, tasks.lim - 1), rt, wi);
      lds_load4((const int *)(a.work + min(wi, nwork - 1)) + min(lane, 3), info + 256 * slot);
    };
    // Slot ids and the tile rows' bias of a task whose work item has landed.
    auto fetch_order = [&](int tau, int slot) {
      const int4 it = item_of(slot);
      lds_load4(a.order + it.y + min(lane, it.z - 1), order + 256 * slot);
      int rt, wi;
      tasks.tile(min(tau, tasks.lim - 1), rt, wi);
      const uint8_t *bp = grp.blobs + (size_t)it.x * grp.stride + grp.off[PH == PH_UP ? 2 : 5];
#pragma unroll
      for (int k = 0; k < 2; ++k)
        lds_load4(bp + 2 * min(rt * C::MR + 2 * (64 * k + lane), out_dim - 2), lds + C::OFF_BIAS + 512 * slot + 256 * k);
    };
    const uint8_t *bsrc[C::BPW], *bssrc, *scsrc;
    auto start_task = [&](int tau, int slot) {
      int rt, wi;
      tasks.tile(tau, rt, wi);
      const int4 it = item_of(slot);
      const int r0 = rt * C::MR;
      const uint8_t *wsc = grp.blobs + (size_t)it.x * grp.stride + grp.off[PH == PH_UP ? 1 : 4];
      const int *ord = (const int *)(order + 256 * slot);
      auto row_of = [&](int n) {
        const int sl = ord[min(n, it.z - 1)];
        return PH == PH_UP ? sl / a.slots : sl;
      };
#pragma unroll
      for (int k = 0; k < C::BPW; ++k) {
        const int v = (lw * C::BPW + k) * 64 + lane;
        const int t = v / (NTOK * 8), sl = v % (NTOK * 8), n = sl >> 3, sg = (sl & 7) ^ (n & 7);
        bsrc[k] = qbase + ((size_t)row_of(n) * NTERM + t) * ld + 16 * sg;
      }
      {
        const int d = min(lw * 64 + lane, C::BS_DW - 1), t = d / NTOK, n = d % NTOK;
        bssrc = sbase + ((size_t)row_of(n) * NTERM + t) * (ld / 32);
      }
      // Block scales of rows r0 + 64·lw + lane: one row's 4 bytes of a chunk per lane.
      scsrc = wsc + (size_t)min(r0 + lw * 64 + lane, out_dim - 1) * nsb;
    };
    auto issue = [&](int c, int st) {
      uint8_t *stg = lds + st * C::STAGE;
#pragma unroll
      for (int k = 0; k < C::BPW; ++k) lds_load16(bsrc[k] + 128 * c, stg + 1024 * (lw * C::BPW + k));
      lds_load4(bssrc + 4 * c, lw * 64 < C::BS_DW ? stg + C::OFF_BS + 256 * lw : junk);
      lds_load4(scsrc + 4 * c, stg + C::OFF_SC + 256 * lw);
    };
    int tq[3];
    tq[0] = tasks.first();
    tq[1] = tasks.next(tq[0]);
    tq[2] = tasks.next(tq[1]);
    fetch_info(tq[0], 0);
    fetch_info(tq[1], 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    fetch_order(tq[0], 0);
    fetch_order(tq[1], 1);
    fetch_info(tq[2], 2);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int slot = 0, lc = 0;
    start_task(tq[0], 0);
    int q = 0;
    auto issue_next = [&]() {
      issue(lc, q % S);
      ++q;
      if (++lc == nch) {
        lc = 0;
        tq[0] = tq[1];
        tq[1] = tq[2];
        tq[2] = tasks.next(tq[2]);
        slot = slot == 2 ? 0 : slot + 1;
        if (tq[0] < tasks.lim) {
          start_task(tq[0], slot);
          const int s1 = slot == 2 ? 0 : slot + 1, s2 = s1 == 2 ? 0 : s1 + 1;
          fetch_order(tq[1], s1);
          fetch_info(tq[2], s2);
        }
      }
    };
    // One barrier per two chunks: at barrier k chunks 2k and 2k+1 have landed; after it the
    // slots of chunks 2k−2 and 2k−1 (computed before it) take chunks 2k+S−2 and 2k+S−1.
    for (int u = 0; u < S - 2 && q < nsteps; ++u) issue_next();
    if (q >= S - 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 4) * L) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int nbar = (nsteps + 1) / 2;
    for (int k = 0; k < nbar; ++k) {
      ring_barrier();
      if (q + 2 <= nsteps) {
        issue_next();
        issue_next();
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 4) * L) : "memory");
      } else {
        while (q < nsteps) issue_next();
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }
    return;
  }

  // ---- MFMA waves: rows 64·wave .. +63 of the tile (NJ = 4 tiles of 16), every token ----
  constexpr int TT = C::TT;
  f32x4 acc[NJ][TT];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[j][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Weight stream: chunk qa (of this workgroup's flat chunk sequence) of the load task.
  int la_tau = tasks.first(), la_slot = 0, la_c = 0;
  const uint8_t *arow[NJ];
  auto la_rows = [&]() {
    int rt, wi;
    tasks.tile(la_tau, rt, wi);
    const int4 it = item_of(la_slot);
    const uint8_t *wblk = grp.blobs + (size_t)it.x * grp.stride + grp.off[PH == PH_UP ? 0 : 3];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      arow[j] = wblk + (size_t)min(rt * C::MR + 64 * wave + 16 * j + l16, out_dim - 1) * (K / 2);
  };
  u32x4 ar[DA][NJ];
  // Unconditional: past the last task the stream re-reads the last task's rows (never used). A
  // load under a branch becomes a copy at the merge, which waits for the data: the ring would be
  // one chunk deep.
  auto load_a = [&](u32x4 (&dst)[NJ]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) dst[j] = *(const u32x4 *)(arow[j] + 16 * min(4 * la_c + g, nsb - 1));
    if (la_tau >= tasks.lim) return;
    if (++la_c == nch) {
      la_c = 0;
      la_tau = tasks.next(la_tau);
      la_slot = la_slot == 2 ? 0 : la_slot + 1;
      if (la_tau < tasks.lim) la_rows();
    }
  };
  int tau = tasks.first(), slot = 0, c = 0;
  int ntok = 0, r0 = 0;
  int eslot[TT];
  float ew[TT];
  auto task_begin = [&]() {
    int rt, wi;
    tasks.tile(tau, rt, wi);
    const int4 it = item_of(slot);
    r0 = rt * C::MR;
    ntok = __builtin_amdgcn_readfirstlane(it.z);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      eslot[tt] = ((const int *)(order + 256 * slot))[min(16 * tt + l16, ntok - 1)];
      ew[tt] = PH == PH_DOWN ? a.slot_w[eslot[tt]] : 0.f;
    }
  };
  struct Ops {
    u32x4 blo[NTERM][TT], bhi[NTERM][TT];
    uint32_t sa[NJ], bs[NTERM][TT];
  };
  auto read_ops = [&](int st) {
    const uint8_t *stg = lds + st * C::STAGE;
    Ops o;
#pragma unroll
    for (int j = 0; j < NJ; ++j) o.sa[j] = stg[C::OFF_SC + 4 * (64 * wave + 16 * j + l16) + g];
    const u32x4 *sb = (const u32x4 *)stg;
#pragma unroll
    for (int t = 0; t < NTERM; ++t)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int n = 16 * tt + l16;
        o.blo[t][tt] = sb[(t * NTOK + n) * 8 + (g ^ (n & 7))];
        o.bhi[t][tt] = sb[(t * NTOK + n) * 8 + ((4 + g) ^ (n & 7))];
        o.bs[t][tt] = (((const uint32_t *)(stg + C::OFF_BS))[t * NTOK + n] >> (8 * g)) & 0xFFu;
      }
    return o;
  };
  ring_barrier();   // the loaders' first task copies have landed
  la_rows();
#pragma unroll
  for (int u = 0; u < DA; ++u) load_a(ar[u]);
  bool done = false;
  // Barrier k lands chunks 2k and 2k + 1: with RA an even step reads its own operands and the
  // next (odd) step's, whose LDS latency then passes under the even step's MFMAs. DA is even and
  // k0 a multiple of DA, so the parity of `step` is that of the unrolled copy u.
  Ops nx;
  for (int k0 = 0; !done; k0 += DA) {
#pragma unroll
    for (int u = 0; u < DA; ++u) {
      const int step = k0 + u;
      if (PH == PH_UP) HH_TRS(step, 0);
      if (c == 0) task_begin();
      Ops cur;
      if (C::RA && (u & 1)) {
        cur = nx;
      } else {
        cur = read_ops(step % S);
        if (C::RA) nx = read_ops((step + 1) % S);   // past the last step: a stage no step reads
      }
#ifdef HH_TRACE_STEPS
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
      if (PH == PH_UP) HH_TRS(step, 1);
      const bool more = step + 1 < nsteps;
      if (128 * (c + 1) > K) {
        // A partial last chunk: lanes past K take zero weights and operand terms; their scale
        // bytes may be any bytes, so 2^0 (the product is the same signed zero). Masked in place.
        const bool ok = 128 * c + 32 * g < K;
        const int kk = 128 * c + 16 * g;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          if (!ok) ar[u][j] = u32x4{0u, 0u, 0u, 0u};
          if (!ok) cur.sa[j] = 127u;
        }
#pragma unroll
        for (int t = 0; t < NTERM; ++t)
#pragma unroll
          for (int tt = 0; tt < TT; ++tt) {
            if (kk >= K) cur.blo[t][tt] = u32x4{0u, 0u, 0u, 0u};
            if (kk + 64 >= K) cur.bhi[t][tt] = u32x4{0u, 0u, 0u, 0u};
            if (!ok) cur.bs[t][tt] = 127u;
          }
      }
      // Token tiles wholly past the item's tokens (padding) are skipped: never stored.
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        if (tt > 0 && 16 * tt >= ntok) break;
#pragma unroll
        for (int t = 0; t < NTERM; ++t)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[j][tt] = smfma(ar[u][j], cur.blo[t][tt], cur.bhi[t][tt], cur.sa[j], cur.bs[t][tt], acc[j][tt]);
      }
      if (PH == PH_UP) HH_TRS(step, 2);
      load_a(ar[u]);   // the chunk DA ahead into the slot just consumed
      if (PH == PH_UP) HH_TRS(step, 3);
      if (++c == nch) {
        // ---- epilogue of the task ----
        c = 0;
        const int rw = r0 + 64 * wave;   // a 64-row block: 32 intermediates of gate-up
        if (rw < out_dim) {
          // The tile rows' bias from the task's LDS copy (rows past out_dim: another row's, never
          // stored).
          const uint8_t *bl = lds + C::OFF_BIAS + 512 * slot;
          float bias[NJ][4];
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const u32x2 bw = *(const u32x2 *)(bl + 2 * (64 * wave + 16 * j + 4 * g));
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
              bias[j][ii] = a.expert_bias ? bf16_bits_to_f32((bw[ii >> 1] >> (16 * (ii & 1))) & 0xFFFFu) : 0.f;
          }
#pragma unroll
          for (int tt = 0; tt < TT; ++tt) {
            if (16 * tt >= ntok) break;   // padding tiles
            const int n = 16 * tt + l16;
            if constexpr (PH == PH_UP) {
              float v[8], gv[8], uv[8];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const f32x4 d = acc[j][tt];
                gv[2 * j] = d[0] + bias[j][0];
                uv[2 * j] = d[1] + bias[j][1];
                gv[2 * j + 1] = d[2] + bias[j][2];
                uv[2 * j + 1] = d[3] + bias[j][3];
              }
              activate_n<8>(a.act, gv, uv, v, a.alpha, a.limit);
              uint32_t hq[NTH][2], sbq[NTH];
              quant_block<NTH>(v, hq, sbq);
              // Each lane's 8 contiguous bytes of every term (one store each).
              uint32_t he[NTH][2];
#pragma unroll
              for (int t = 0; t < NTH; ++t) transpose_pieces(hq[t][0], hq[t][1], g, he[t][0], he[t][1]);
              if (n < ntok) {
                const int i0 = rw / 2;
#pragma unroll
                for (int t = 0; t < NTH; ++t) {
                  uint8_t *row = a.hq + ((size_t)eslot[tt] * NTH + t) * a.hld + i0;
                  *(u32x2 *)(row + 8 * g) = u32x2{he[t][0], he[t][1]};
                  if (g == 0) a.hs[((size_t)eslot[tt] * NTH + t) * (a.hld / 32) + i0 / 32] = (uint8_t)sbq[t];
                }
              }
            } else {
              if (n < ntok) {
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                  const int h0 = rw + 16 * j + 4 * g;
                  f32x4 o;
#pragma unroll
                  for (int ii = 0; ii < 4; ++ii) o[ii] = ew[tt] * (acc[j][tt][ii] + bias[j][ii]);   // down_value's arithmetic
                  *(f32x4 *)(a.slot_out + (size_t)eslot[tt] * H + h0) = o;
                }
              }
            }
          }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int tt = 0; tt < TT; ++tt) acc[j][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        tau = tasks.next(tau);
        slot = slot == 2 ? 0 : slot + 1;
      }
      if (!more) {
        done = true;
        break;
      }
      if (PH == PH_UP) HH_TRS(step, 4);
      if (step & 1) ring_barrier();   // one barrier per two chunks
      if (PH == PH_UP) HH_TRS(step, 5);
    }
  }
}

// ---- prefill, BF16 and MLX affine: an LDS ring filled by loader waves -----------------------------
// 8 waves, one workgroup per compute unit, persistent over the tasks τ = blockIdx, + gridDim, ...
// (a task = one work item of ≤ 32 tokens × one row tile, in prefill_tile's XCD-aware order).
// Waves 4-7 load: each stage (SCOLS columns of K) brings, by direct-to-LDS loads, the weight
// operand of the row tile (per MFMA wave: NM tiles of 16 rows, laid out exactly as that wave's
// lanes read them), the MLX group scales and biases, and the TOK token rows of the activation
// (x, or h_hi and h_lo) in 16-byte segments XOR-swizzled by token so the MFMA reads are
// bank-conflict free. S stages are in flight; the ring runs on across task boundaries (each
// task's work item and slot ids also travel by direct-to-LDS loads, ahead of its first stage).
// Waves 0-3 multiply: wave w owns output rows rb .. rb + 16·RT of the tile (gate and up tiles of
// the same intermediates for gate-up) for all 32 tokens, and reads each stage's operands one
// stage ahead of its MFMAs. The arithmetic per output element is chunk_mfma's, the decode
// kernels' bits: two chains over the chunks (even / odd), steps in order.
template <int PH, int FMT, int RT, int NT_> struct Ring {
  static constexpr int NT = NT_, TOK = 16 * NT;
  static constexpr int NM = (PH == PH_UP ? 2 : 1) * RT;
  static constexpr int NH = PH == PH_UP ? 1 : 2;
  static constexpr bool MLX = is_mlx<FMT>();
  // K columns per stage: two MLX groups; BF16 two 32-column steps (128-column stages leave
  // 64-token tiles too few stages in LDS).
  static constexpr int SCOLS = MLX ? 128 : 64;
  static constexpr int SPS = MLX ? 2 : SCOLS / 32;              // MLX groups / BF16 steps per stage
  static constexpr int SEGS = SCOLS / 8;                        // 16-byte segments per token row
  static constexpr int RPI = 1024 / (SCOLS * 2);                // token rows per 1 KiB load
  static constexpr int A_INS = FMT == Q_MLX4 ? 1 : SPS;         // 1 KiB weight loads per tile
  static constexpr int B_INS = NH * TOK / RPI;                  // 1 KiB operand loads per stage
  static constexpr int BPW = B_INS / 4;
  static constexpr int SB_INS = MLX ? 4 : 0;                    // {scale, bias} × 2 groups
  static constexpr int L = NM * A_INS + BPW + SB_INS;           // loads per loader wave per stage
  static constexpr int OFF_B = 4 * NM * A_INS * 1024;
  static constexpr int OFF_SB = OFF_B + B_INS * 1024;
  static constexpr int STAGE = OFF_SB + (MLX ? 4096 : 0);
  static constexpr int NO = (TOK + 63) / 64;                    // slot-id registers per lane
  static constexpr int INFO = 256 + 256 * NO;                   // work item, slot ids
  static constexpr int S_LDS = (148 * 1024) / STAGE, S_CNT = 3 + 63 / L;
  static constexpr int S = S_LDS < S_CNT ? (S_LDS < 8 ? S_LDS : 8) : (S_CNT < 8 ? S_CNT : 8);
  static constexpr int NSLOT = S + 1;                           // task info slots (≤ S tasks ahead)
  static constexpr int OFF_INFO = S * STAGE;
  static constexpr int LDS = OFF_INFO + NSLOT * INFO;
  static constexpr int ROWS = 64 * RT;
  // The B operand of the next stage is read ahead too, except for wide token tiles (measured
  // slower there: gate-up 567 → 617 µs).
  static constexpr bool RA_B = NT <= 2;
  static_assert(B_INS % 4 == 0 && S >= 3 && NM <= 4 && LDS <= 160 * 1024, "ring layout");
  __device__ static int swz(int n) {
    return SEGS == 16 ? (n & 15) : (SEGS == 8 ? ((n >> 1) & 7) : ((n >> 2) & 3));
  }
};

__device__ __forceinline__ void lds_load2(const void *g, uint8_t *l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 2, 0, 0);
}
template <int N> __device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

template <int PH, int FMT, int RT, int NT_>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_ring(GemmArgs a) {
  using C = Ring<PH, FMT, RT, NT_>;
  using F = Fmt<FMT>;
  constexpr int NM = C::NM, NT = C::NT, NH = C::NH, TOK = C::TOK, S = C::S, L = C::L;
  constexpr int SCOLS = C::SCOLS, SEGS = C::SEGS, SPS = C::SPS, NO = C::NO;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int H = a.hidden, E = a.experts;
  const int RTL = a.row_tiles, rtx = (RTL + 7) >> 3;
  const int nwork = *a.n_work;
  const Mx3Tasks tasks((int)blockIdx.x, (int)gridDim.x, RTL, nwork, a.xcd_rows);
  if (tasks.first() >= tasks.lim) return;
  auto group_of = [&](int e) -> const ExpertGroup & { return a.grp[e == E ? 1 : 0]; };
  auto k_of = [&](int e) { return PH == PH_UP ? H : group_of(e).inter; };
  auto nst_of = [&](int e) { return (k_of(e) + SCOLS - 1) / SCOLS; };
  auto work_of = [&](int tau) {
    int rt, wi;
    tasks.tile(min(tau, tasks.lim - 1), rt, wi);
    return a.work[min(wi, nwork - 1)];
  };
  // A task's copy for the MFMA waves: its work item, then its slot ids.
  auto send_info = [&](int tau, const int4 &w, int slot) {
    int rt, wi;
    tasks.tile(tau, rt, wi);
    uint8_t *info = lds + C::OFF_INFO + C::INFO * slot;
    lds_load4((const int *)(a.work + wi) + min(lane, 3), info);
#pragma unroll
    for (int k = 0; k < NO; ++k) lds_load4(a.order + w.y + min(64 * k + lane, w.z - 1), info + 256 * (k + 1));
  };

  if (wave >= 4) {
    // ---- loaders ----
    const int lw = wave - 4;
    int tau = tasks.first(), slot = 0;
    int4 wn = work_of(tau), wnn = work_of(tasks.next(tau));
    int on[NO];
#pragma unroll
    for (int k = 0; k < NO; ++k) on[k] = a.order[wn.y + min(64 * k + lane, wn.z - 1)];
    int K = 0, nst = 0, ls = 0, q = 0;     // task K, its stages, stage within it, stages issued
    ATile<FMT> at[NM];
    const uint16_t *brow[C::BPW];
    bool more = true;
    send_info(tau, wn, 0);   // the first task's copy, waited for here
    wait_vm<0>();
    auto begin_task = [&]() {
      const int4 cur = wn;
      int o[NO];
#pragma unroll
      for (int k = 0; k < NO; ++k) o[k] = on[k];
      int rt, wi;
      tasks.tile(tau, rt, wi);
      // The next task's copy goes out a task ahead: it lands long before that task's first stage
      // is read.
      const int t1 = tasks.next(tau);
      if (t1 < tasks.lim) send_info(t1, wnn, slot == C::NSLOT - 1 ? 0 : slot + 1);
      const int e = cur.x;
      const ExpertGroup &grp = group_of(e);
      const uint8_t *blob = grp.blobs + (e == E ? 0 : (size_t)e * grp.stride);
      K = k_of(e);
      nst = nst_of(e);
      const int out_dim = PH == PH_UP ? grp.inter : H;
      wave_tiles<PH, FMT, RT>(at, blob, grp, rt * C::ROWS + lw * 16 * RT, out_dim, K, l16);
#pragma unroll
      for (int i = 0; i < C::BPW; ++i) {
        const int j = lw * C::BPW + i;
        const int hh = j / (TOK / C::RPI);
        const int n = min(C::RPI * (j % (TOK / C::RPI)) + lane / SEGS, cur.z - 1);
        int sl = 0;
#pragma unroll
        for (int k = 0; k < NO; ++k) {
          const int v = __shfl(o[k], n & 63);
          if ((n >> 6) == k) sl = v;
        }
        brow[i] = PH == PH_UP ? a.x + (size_t)(sl / a.slots) * H : (hh ? a.h_lo : a.h_hi) + (size_t)sl * a.ldh;
      }
      // Prefetch: the next task's slot ids, the work item of the one after.
      wn = wnn;
#pragma unroll
      for (int k = 0; k < NO; ++k) on[k] = a.order[wn.y + min(64 * k + lane, wn.z - 1)];
      wnn = work_of(tasks.next(t1));
    };
    auto issue = [&](int s, int st) {
      uint8_t *stg = lds + st * C::STAGE;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        uint8_t *dst = stg + (lw * NM + m) * C::A_INS * 1024;
        const uint8_t *w = at[m].row.w;
        if constexpr (FMT == Q_BF16) {
#pragma unroll
          for (int j = 0; j < SPS; ++j) lds_load16(w + 2 * min(SCOLS * s + 32 * j + 8 * g, K - 8), dst + 1024 * j);
        } else if constexpr (FMT == Q_MLX4) {
          lds_load16(w + min(64 * s + 16 * g, K / 2 - 16), dst);
        } else {
#pragma unroll
          for (int p = 0; p < 2; ++p) lds_load16(w + min(128 * s + 64 * p + 16 * g, K - 16), dst + 1024 * p);
        }
      }
      if constexpr (C::MLX) {
        // Group scales and biases of the wave's rows: lane (m, r) holds tile m's row r (one
        // dword per lane; tiles past NM repeat the last).
        typename F::Row r = at[0].row;
#pragma unroll
        for (int m = 1; m < NM; ++m)
          if ((lane >> 4) >= m) r = at[m].row;
        const int ng = K / 64;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int gi = min(2 * s + p, ng - 1);
          lds_load2(r.sc + gi, stg + C::OFF_SB + lw * 1024 + p * 256);
          lds_load2(r.bi + gi, stg + C::OFF_SB + lw * 1024 + 512 + p * 256);
        }
      }
#pragma unroll
      for (int i = 0; i < C::BPW; ++i) {
        const int j = lw * C::BPW + i;
        const int n = C::RPI * (j % (TOK / C::RPI)) + lane / SEGS;
        const int seg = (lane % SEGS) ^ C::swz(n);
        lds_load16(brow[i] + min(SCOLS * s + 8 * seg, K - 8), stg + C::OFF_B + 1024 * j);
      }
    };
    auto issue_next = [&]() {
      if (ls == 0) begin_task();
      issue(ls, q % S);
      asm volatile("" ::: "memory");   // stages (and task copies) issue in program order
      ++q;
      if (++ls == nst) {
        ls = 0;
        tau = tasks.next(tau);
        slot = slot == C::NSLOT - 1 ? 0 : slot + 1;
        more = tau < tasks.lim;
      }
    };
    for (int u = 0; u < S - 1 && more; ++u) issue_next();
    if (q >= S - 1) wait_vm<(S - 3) * L>();
    else wait_vm<0>();
    for (int step = 0; more || step < q; ++step) {
      ring_barrier();
      if (more) {
        issue_next();
        wait_vm<(S - 3) * L>();
      } else {
        wait_vm<0>();
      }
    }
    return;
  }

  // ---- MFMA waves ----
  constexpr int NP = C::MLX ? 2 : 1;
  struct AOps { typename F::A w[NP][NM]; };
  struct BOps { u32x4 b[NP][NT][NH][C::MLX ? 2 : SPS]; };
  auto read_a = [&](int st) {
    const uint8_t *stg = lds + st * C::STAGE;
    AOps o;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const uint8_t *ab = stg + (wave * NM + m) * C::A_INS * 1024;
      if constexpr (FMT == Q_BF16) {
#pragma unroll
        for (int j = 0; j < SPS; ++j) o.w[0][m].w[j] = *(const u32x4 *)(ab + 1024 * j + 16 * lane);
      } else {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if constexpr (FMT == Q_MLX4) {
            const u32x2 v = *(const u32x2 *)(ab + 16 * ((2 * p + (g >> 1)) * 16 + l16) + 8 * (g & 1));
            o.w[p][m].w[0] = v[0];
            o.w[p][m].w[1] = v[1];
          } else {
            const u32x4 v = *(const u32x4 *)(ab + 1024 * p + 16 * lane);
#pragma unroll
            for (int k = 0; k < 4; ++k) o.w[p][m].w[k] = v[k];
          }
          const uint8_t *sbp = stg + C::OFF_SB + wave * 1024 + p * 256 + 4 * (16 * m + l16);
          o.w[p][m].sb = (*(const uint32_t *)sbp & 0xFFFFu) | (*(const uint32_t *)(sbp + 512) << 16);
        }
      }
    }
    return o;
  };
  auto read_b = [&](int st) {
    const uint8_t *stg = lds + st * C::STAGE;
    BOps o;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int st2 = 0; st2 < NT; ++st2)
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
          for (int v = 0; v < (C::MLX ? 2 : SPS); ++v) {
            const int n = 16 * st2 + l16;
            const int seg = C::MLX ? 8 * p + 2 * g + v : 4 * v + g;
            o.b[p][st2][hh][v] =
                *(const u32x4 *)(stg + C::OFF_B + (hh * TOK + n) * (SCOLS * 2) + 16 * (seg ^ C::swz(n)));
          }
    return o;
  };

  // The two chains of the canonical arithmetic. MLX: acc[c & 1] with c static per half-stage.
  // BF16 (a stage is part of one chunk): acc[0] holds the chain of chunk parity cpar and acc[1] the
  // other; they trade places when the parity changes (at most once per chunk), so the MFMAs
  // address fixed registers, and the epilogue's acc[0] + acc[1] is the same sum either way (fp
  // addition commutes).
  f32x4 acc[2][NM][NT];
  int cpar = 0;
  auto zero = [&]() {
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int st = 0; st < NT; ++st) acc[p][m][st] = f32x4{0.f, 0.f, 0.f, 0.f};
    cpar = 0;
  };
  zero();
  int tau = tasks.first(), slot = 0, ls = 0, nst = 0, K = 0, e = 0, ntok = 0, rt = 0;
  float ew[PH == PH_DOWN ? NT : 1];
  const ATile<FMT> at_unused[NM] = {};
  ring_barrier();
  AOps cur = read_a(0);
  BOps curb;
  if constexpr (C::RA_B) curb = read_b(0);
  for (int step = 0;; ++step) {
    if (PH == PH_UP) HH_TRS(step, 0);
    if (ls == 0) {
      const uint8_t *info = lds + C::OFF_INFO + C::INFO * slot;
      const int4 it = *(const int4 *)info;
      e = it.x;
      ntok = it.z;
      K = k_of(e);
      nst = nst_of(e);
      int wi;
      tasks.tile(tau, rt, wi);
      if constexpr (PH == PH_DOWN) {
#pragma unroll
        for (int st = 0; st < NT; ++st) ew[st] = a.slot_w[((const int *)(info + 256))[min(16 * st + l16, ntok - 1)]];
      }
    }
    // Is there a stage after this one (this task's next, or the next task's first)?
    const bool last_stage = ls + 1 == nst;
    const int tau_n = last_stage ? tasks.next(tau) : tau;
    const bool more = !last_stage || tau_n < tasks.lim;
    const int st_n = (step + 1) % S;
    AOps nxt;
    BOps nxtb;
    if (more) {
      nxt = read_a(st_n);
      if constexpr (C::RA_B) nxtb = read_b(st_n);
    }
    if constexpr (!C::RA_B) curb = read_b(step % S);
#ifdef HH_TRACE_STEPS
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
    if (PH == PH_UP) HH_TRS(step, 1);
    if constexpr (FMT == Q_BF16) {
      const int c = (SCOLS * ls) >> 7;
      auto steps = [&](f32x4 (&ac)[NM][NT]) {
#pragma unroll
        for (int j = 0; j < SPS; ++j) {
          const int v = ((SCOLS * ls) & 127) / 32 + j;
          if (!F::step_ok(c, v, K)) break;
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int st = 0; st < NT; ++st)
#pragma unroll
              for (int hh = 0; hh < NH; ++hh)
                ac[m][st] = mfma(as_bf16x8(cur.w[0][m].w[j]), as_bf16x8(curb.b[0][st][hh][j]), ac[m][st]);
        }
      };
      if ((c & 1) != cpar) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int st = 0; st < NT; ++st) {
            const f32x4 t = acc[0][m][st];
            acc[0][m][st] = acc[1][m][st];
            acc[1][m][st] = t;
          }
        cpar ^= 1;
      }
      steps(acc[0]);
    } else {
      // The (scale | bias) words of D rows 4g .. 4g+3 straight from the stage (16 contiguous
      // bytes of each), instead of the lane's own row's words moved across lanes by shuffles.
      const uint8_t *sbb = lds + (step % S) * C::STAGE + C::OFF_SB + wave * 1024 + 16 * g;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int c = 2 * ls + p;
        if (64 * c >= K) break;
        chunk_mfma<FMT, NM, NT, NH>(acc[c & 1], cur.w[p], at_unused,
                                    [&](int st, int hh, int v) { return curb.b[p][st][hh][v]; }, c, g, K,
                                    [&](int m) {
                                      const u32x4 sv = *(const u32x4 *)(sbb + p * 256 + 64 * m);
                                      const u32x4 bv = *(const u32x4 *)(sbb + 512 + p * 256 + 64 * m);
                                      u32x4 r;
#pragma unroll
                                      for (int ii = 0; ii < 4; ++ii) r[ii] = (sv[ii] & 0xFFFFu) | (bv[ii] << 16);
                                      return r;
                                    });
      }
    }
    if (last_stage) {
      // ---- epilogue of the task ----
      const ExpertGroup &grp = group_of(e);
      const int out_dim = PH == PH_UP ? grp.inter : H;
      const int rb = rt * C::ROWS + wave * 16 * RT;
      const int *slots = (const int *)(lds + C::OFF_INFO + C::INFO * slot + 256);   // still this task's
#pragma unroll
      for (int st = 0; st < NT; ++st) {
        if (16 * st + l16 >= ntok) continue;
        const int es = slots[16 * st + l16];
#pragma unroll
        for (int q = 0; q < RT; ++q) {
          if (rb + 16 * q >= out_dim) continue;
          if constexpr (PH == PH_UP) {
            up_epilogue<FMT>(a, nullptr, grp, rb + 16 * q + 4 * g, es,
                             sum_chains(acc[0][q][st], acc[1][q][st]), sum_chains(acc[0][RT + q][st], acc[1][RT + q][st]));
          } else {
            const f32x4 r = sum_chains(acc[0][q][st], acc[1][q][st]);
            f32x4 o;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) o[ii] = ew[st] * (r[ii] + 0.f);   // down_value's arithmetic
            *(f32x4 *)(a.slot_out + (size_t)es * H + rb + 16 * q + 4 * g) = o;
          }
        }
      }
      zero();
      tau = tau_n;
      slot = slot == C::NSLOT - 1 ? 0 : slot + 1;
      ls = 0;
    } else {
      ++ls;
    }
    if (PH == PH_UP) HH_TRS(step, 2);
    if (!more) break;
    ring_barrier();
    if (PH == PH_UP) HH_TRS(step, 3);
    cur = nxt;
    if constexpr (C::RA_B) curb = nxtb;
  }
}

// Row tiles per MFMA wave of the ring kernel: gate-up one (a gate and an up tile), down two.
template <int PH, int FMT> constexpr int ring_rt() {
  return PH == PH_DOWN ? 2 : 1;
}

// ---- launch table -----------------------------------------------------------------------------
typedef void (*GemmKernel)(GemmArgs);
typedef void (*UpSmallKernel)(GemmArgs, RouteArgs, FuseArgs);
typedef void (*DownSmallKernel)(GemmArgs, const int32_t *);

// Register ring depth of the decode weight stream, in chunks (per lane per chunk: MXFP4 16 B +
// a scale, MLX4 8 B, MLX8 16 B (+ a scale|bias pair), BF16 64 B).
template <int FMT> constexpr int decode_depth() { return FMT == Q_BF16 ? 4 : (FMT == Q_MXFP4 ? 24 : 8); }

// MXFP4 streams of at most MX_ONE chunks (K ≤ 3072) run the single-round kernels (the whole row
// in flight, no ring refills); longer rows take the ring variants.
constexpr int MX_ONE = MX_ONE_CHUNKS;
// One token's x (MXFP4: 2 terms × (H/16 + scale vectors) 16-byte vectors, 372 at H = 2880; the
// others: H/8 vectors) fits the first round of staging loads at two vectors per thread; larger
// batches issue twelve per thread before the selection, so T ≤ 8 stages in one round (T = 8 took
// four).
constexpr int MX_XB_WIDE = 12;
// Rows of exactly MX_STATIC chunks (K = 2817..2944: GPT-OSS's 2880) take variants with the chunk
// count compiled in (`st`).
constexpr int MX_STATIC = 23;
// MLX gate-up rows of exactly 2·MLX_NCW chunks (K = 2048: Qwen3.5-35B-A3B) take the single-round
// stream of MLX_NCW chunks per wave.
constexpr int MLX_NCW = 16;
#ifndef HH_GEMM_KERNELS_ONLY
// fr: 0 none, 1 the fused router over x, 2 the fused router over the FFN block's residual.
UpSmallKernel up_small_block_k(bool st, int T);
template <int FMT> static UpSmallKernel up_small_k(bool one, int T, bool st = false, bool stat = false, int fr = 0) {
  if constexpr (FMT == Q_MXFP4) {
    if (fr == 2) return up_small_block_k(st, T);   // the fused router: single-round rows only
    if (fr) {
      if (st) return T == 1 ? up_small_mx<MX_ONE, true, 2, MX_STATIC, 1> : up_small_mx<MX_ONE, true, MX_XB_WIDE, MX_STATIC, 1>;
      return T == 1 ? up_small_mx<MX_ONE, true, 2, 0, 1> : up_small_mx<MX_ONE, true, MX_XB_WIDE, 0, 1>;
    }
    if (one && st) return T == 1 ? up_small_mx<MX_ONE, true, 2, MX_STATIC> : up_small_mx<MX_ONE, true, MX_XB_WIDE, MX_STATIC>;
    if (T == 1) return one ? up_small_mx<MX_ONE, true, 2> : up_small_mx<16, false, 2>;
    return one ? up_small_mx<MX_ONE, true, MX_XB_WIDE> : up_small_mx<16, false, MX_XB_WIDE>;
  }
  else if constexpr (is_mlx<FMT>()) {
    if (st && T == 1 && stat) return up_small<FMT, MLX_NCW, 1, 2, true, MLX_NCW>;
    if (st) return T == 1 ? up_small<FMT, decode_depth<FMT>(), 1, 2, true> : up_small<FMT, decode_depth<FMT>(), 1, MX_XB_WIDE, true>;
    return T == 1 ? up_small<FMT, decode_depth<FMT>(), 1, 2> : up_small<FMT, decode_depth<FMT>(), 1, MX_XB_WIDE>;
  }
  else if (T == 1) return up_small<FMT, decode_depth<FMT>(), 1, 2>;
  else return up_small<FMT, decode_depth<FMT>(), 1, MX_XB_WIDE>;
}
// Waves per slot of down_small: MXFP4's canonical arithmetic is one chain over K (one wave per
// slot); the others split K by chunk parity over two waves when the workgroup has room.
template <int FMT> constexpr int down_ks(int slots) { return (FMT == Q_MXFP4 || slots > 4) ? 1 : 2; }

template <int FMT> static DownSmallKernel down_small_k(int slots, bool one, bool st = false) {
  // Nine waves leave a third of the register file per wave: a shallower ring (also the MXFP4
  // kernel for rows longer than MX_ONE chunks).
  constexpr int D9 = decode_depth<FMT>() > 8 ? 8 : decode_depth<FMT>();
  if (slots > 4 || !one) {
    if constexpr (is_mlx<FMT>())
      if (st) return down_small<FMT, D9, kMaxTopK + 1, 1, true>;
    return down_small<FMT, D9, kMaxTopK + 1, 1>;
  }
  if constexpr (is_mlx<FMT>())
    if (st) return down_small<FMT, decode_depth<FMT>(), 4, down_ks<FMT>(4), true>;
  return down_small<FMT, decode_depth<FMT>(), 4, down_ks<FMT>(4)>;
}
// MLX: whether the staged-scale variants take this layer (the rows' chunk counts fit LDS).
static bool mlx_staged_up(int hidden) { return hidden <= 64 * kMlxSbChunks; }
static bool mlx_staged_down(int slots, int imax) {
  return imax <= 64 * (slots > 4 ? mlx_sb_chunks_down<kMaxTopK + 1>() : mlx_sb_chunks_down<4>());
}

// The ring kernel of a BF16 / MLX phase: 64-token work items (BF16 layers whose experts average
// 64 or more tokens) or 32-token ones.
template <int PH, int FMT> static GemmKernel ring_pick(int nt, size_t *lds) {
  constexpr int RT = ring_rt<PH, FMT>();
  if constexpr (FMT == Q_BF16) {
    if (nt > 2) {
      if (lds) *lds = Ring<PH, FMT, RT, 4>::LDS;
      return prefill_ring<PH, FMT, RT, 4>;
    }
  }
  if (lds) *lds = Ring<PH, FMT, RT, 2>::LDS;
  return prefill_ring<PH, FMT, RT, 2>;
}

template <int PH, int FMT>
static GemmKernel pick(int nt) {
  if constexpr (FMT == Q_MXFP4) return nt <= 2 ? prefill_mx2<PH, 1> : prefill_mx2<PH, 2>;
  else return ring_pick<PH, FMT>(nt, nullptr);
}

// Output rows per prefill workgroup: intermediates (gate-up) or hidden rows (down). The MXFP4
// kernel covers 128 weight rows: 64 intermediates of the interleaved gate_up matrix.
int gemm_rows_per_block(int quant, int phase) {
  if (quant == Q_MXFP4) return phase == PH_UP ? 64 : 128;
  return 64 * (phase == PH_UP ? ring_rt<PH_UP, Q_BF16>() : ring_rt<PH_DOWN, Q_BF16>());
}

static GemmKernel gemm_kernel(int phase, int quant, int nt) {
  switch (quant) {
  case Q_MXFP4: return phase == PH_UP ? pick<PH_UP, Q_MXFP4>(nt) : pick<PH_DOWN, Q_MXFP4>(nt);
  case Q_BF16: return phase == PH_UP ? pick<PH_UP, Q_BF16>(nt) : pick<PH_DOWN, Q_BF16>(nt);
  case Q_MLX4: return phase == PH_UP ? pick<PH_UP, Q_MLX4>(nt) : pick<PH_DOWN, Q_MLX4>(nt);
  default: return phase == PH_UP ? pick<PH_UP, Q_MLX8>(nt) : pick<PH_DOWN, Q_MLX8>(nt);
  }
}

// Dynamic LDS of the ring kernel of (phase, quant, token tile).
static size_t ring_lds(int phase, int quant, int nt) {
  size_t lds = 0;
  switch (quant) {
  case Q_BF16: (void)(phase == PH_UP ? ring_pick<PH_UP, Q_BF16>(nt, &lds) : ring_pick<PH_DOWN, Q_BF16>(nt, &lds)); break;
  case Q_MLX4: (void)(phase == PH_UP ? ring_pick<PH_UP, Q_MLX4>(nt, &lds) : ring_pick<PH_DOWN, Q_MLX4>(nt, &lds)); break;
  default: (void)(phase == PH_UP ? ring_pick<PH_UP, Q_MLX8>(nt, &lds) : ring_pick<PH_DOWN, Q_MLX8>(nt, &lds)); break;
  }
  return lds;
}

static int device_cus() {
  static int ncu = 0;
  if (!ncu) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu < 8) ncu = 256;
    ncu &= ~7;   // prefill_tile's order assumes 8 | gridDim for persistent grids
  }
  return ncu;
}

// Whether prefill_mx3 takes a phase: MXFP4 without a shared expert, work items of 32 tokens, and
// rows of at least S chunks (task switches are prefetched one task ahead inside the chunk ring).
// Gate-up over batches of 64 or more work items takes 256-row tiles (twice the products per staged
// byte); down, and smaller batches, 128-row tiles (down's deeper ring measured faster).
template <int PH, int RR, int TT> static bool mx3_fits(const GemmArgs &a) {
  const int K = PH == PH_UP ? a.hidden : a.grp[0].inter;
  return (K + 127) / 128 >= Mx3<PH, RR, TT>::S;
}
static bool mx3_wide(int phase, const GemmArgs &a) { return a.max_work >= 64; }
static bool use_mx3(int phase, const GemmArgs &a, int nt) {
  if (a.slots != a.top_k || nt != 2) return false;
  if (!mx3_wide(phase, a)) return phase == PH_UP ? mx3_fits<PH_UP, 1, 1>(a) : mx3_fits<PH_DOWN, 1, 1>(a);
  return phase == PH_UP ? mx3_fits<PH_UP, 2, 1>(a) : mx3_fits<PH_DOWN, 2, 1>(a);
}

template <int PH, int RR, int TT> static hipError_t launch_mx3(GemmArgs a, hipStream_t s, Timing tm) {
  static std::once_flag once;
  std::call_once(once, [] {
    (void)hipFuncSetAttribute((const void *)prefill_mx3<PH, RR, TT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    (void)hipGetLastError();
  });
  // Row tiles of this variant: MR weight rows (MR / 2 intermediates of the interleaved gate_up).
  constexpr int rows = PH == PH_UP ? Mx3<PH, RR, TT>::MR / 2 : Mx3<PH, RR, TT>::MR;
  a.row_tiles = ((PH == PH_UP ? a.ldh : a.hidden) + rows - 1) / rows;
  hipExtLaunchKernelGGL(prefill_mx3<PH, RR, TT>, dim3(device_cus()), dim3(512), Mx3<PH, RR, TT>::LDS, s, tm.start,
                        tm.stop, 0, a);
  return hipGetLastError();
}

// Whether prefill_mxa takes a phase: gate-up of MXFP4 layers without a shared expert, 32-token
// work items in batches of 64 or more, or 64-token ones; rows of at least S chunks (a wave's
// weight stream reads the next task's copy, which the loaders rewrite S chunks later). Down's three
// operand terms leave too few registers for the weight ring.
static bool use_mxa(int phase, const GemmArgs &a, int nt) {
  if (phase != PH_UP || a.slots != a.top_k) return false;
  if (nt == 2) return a.max_work >= 64 && (a.hidden + 127) / 128 >= MxA<PH_UP, 2>::S;
  return nt == 4 && (a.hidden + 127) / 128 >= MxA<PH_UP, 4>::S;
}

template <int PH, int TT> static hipError_t launch_mxa(GemmArgs a, hipStream_t s, Timing tm) {
  static std::once_flag once;
  std::call_once(once, [] {
    (void)hipFuncSetAttribute((const void *)prefill_mxa<PH, TT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    (void)hipGetLastError();
  });
  constexpr int rows = PH == PH_UP ? MxA<PH, TT>::MR / 2 : MxA<PH, TT>::MR;
  a.row_tiles = ((PH == PH_UP ? a.ldh : a.hidden) + rows - 1) / rows;
  hipExtLaunchKernelGGL(prefill_mxa<PH, TT>, dim3(device_cus()), dim3(512), MxA<PH, TT>::LDS, s, tm.start, tm.stop, 0,
                        a);
  return hipGetLastError();
}

hipError_t launch_gemm(int phase, int quant, int nt, const GemmArgs &args, hipStream_t s, Timing tm) {
  // Persistent kernels: XCD split into row-tile parts × work-item parts (Mx3Tasks). Measured on
  // the benchmark layers (prefill T = 512..2048) against 8 row-tile parts: BF16 gate-up 832 →
  // 615 µs with 4 or 2 parts, BF16 down 414 → 371 µs with 2; MLX 3-5 % faster with 4; MXFP4
  // within ±2 % (its down fetches 18 % fewer bytes with 4).
  GemmArgs a = args;
  a.xcd_rows = (quant == Q_BF16 && phase == PH_DOWN) ? 2 : 4;
  if (quant == Q_MXFP4 && use_mxa(phase, a, nt))
    return nt == 2 ? launch_mxa<PH_UP, 2>(a, s, tm) : launch_mxa<PH_UP, 4>(a, s, tm);
  if (quant == Q_MXFP4 && nt == 4 && phase == PH_DOWN && a.slots == a.top_k &&
      (a.grp[0].inter + 127) / 128 >= Mx3<PH_DOWN, 1, 2>::S)
    return launch_mx3<PH_DOWN, 1, 2>(a, s, tm);
  if (quant == Q_MXFP4 && use_mx3(phase, a, nt)) {
    if (!mx3_wide(phase, a)) return phase == PH_UP ? launch_mx3<PH_UP, 1, 1>(a, s, tm) : launch_mx3<PH_DOWN, 1, 1>(a, s, tm);
    return phase == PH_UP ? launch_mx3<PH_UP, 2, 1>(a, s, tm) : launch_mx3<PH_DOWN, 2, 1>(a, s, tm);
  }
  if (quant != Q_MXFP4) {
    // BF16 / MLX: the persistent ring kernel, one workgroup per compute unit.
    static std::once_flag once;
    std::call_once(once, [] {
      for (int ph = 0; ph < 2; ++ph)
        for (int q : {Q_BF16, Q_MLX4, Q_MLX8})
          for (int nt : {2, 4}) {
            (void)hipFuncSetAttribute((const void *)gemm_kernel(ph, q, nt), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      160 * 1024);
            (void)hipGetLastError();
          }
    });
    if (a.max_work == 0) return hipSuccess;
    hipExtLaunchKernelGGL(gemm_kernel(phase, quant, nt), dim3(device_cus()), dim3(512), ring_lds(phase, quant, nt), s,
                          tm.start, tm.stop, 0, a);
    return hipGetLastError();
  }
  // prefill_tile: 8 XCDs × ⌈row_tiles / 8⌉ row tiles × work items.
  const unsigned blocks = 8u * (unsigned)((a.row_tiles + 7) / 8) * (unsigned)a.max_work;
  if (blocks == 0) return hipSuccess;
  const bool mx = quant == Q_MXFP4;
  // MXFP4: 8 waves, the weight rows' scales (128 rows × K/32 bytes) in dynamic LDS.
  const size_t lds = mx ? (size_t)128 * ((phase == PH_UP ? a.hidden : a.ldh) / 32) : 0;
  hipExtLaunchKernelGGL(gemm_kernel(phase, quant, nt), dim3(blocks), dim3(mx ? 512 : 256), lds, s, tm.start,
                        tm.stop, 0, a);
  return hipGetLastError();
}

hipError_t launch_down_small(int quant, GemmArgs a, const int32_t *topk_idx, int T, hipStream_t s,
                             Timing tm_down);

// Decode (T ≤ 16). `a.row_tiles` is set here per phase.
// Workgroups of `kernel` resident per compute unit at `threads` threads and `lds` bytes of dynamic
// LDS (at least 1), from the runtime's occupancy calculator, cached per (kernel, lds).
static int resident_per_cu(const void *kernel, int threads, size_t lds) {
  struct Entry { const void *k; size_t lds; int n; };
  static std::mutex mu;
  static std::vector<Entry> cache;
  std::lock_guard<std::mutex> lock(mu);
  for (const Entry &en : cache)
    if (en.k == kernel && en.lds == lds) return en.n;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess || n < 1) {
    (void)hipGetLastError();
    n = 1;
  }
  cache.push_back({kernel, lds, n});
  return n;
}

bool fused_router_fits(int quant, int H, int E, int router, int T) {
  return quant == Q_MXFP4 && router != R_GEMMA && H <= 4096 && (H + 127) / 128 <= MX_ONE && E <= kFusedMaxE &&
         T >= 1 && T <= kFusedRouterT;
}
// Flag-buffer words of the fused router's logit records: 8 replicas × T·(E+1) records × 4.
int fused_router_flags(int T, int E) { return 4 * kRecReplicas * T * (E + 1); }

hipError_t launch_small(int quant, GemmArgs a, const RouteArgs &ra, hipStream_t s, Timing tm_up,
                        Timing tm_down, const FuseArgs *fr) {
  const int T = ra.tokens;
  if (T < 1 || T > SMALL_T) return hipErrorInvalidValue;
  const int S = a.slots;
  const int maxu = std::min(a.experts, T * a.top_k) + (S > a.top_k ? 1 : 0);
  const bool mx = quant == Q_MXFP4;
  const bool one_up = !mx || (a.hidden + 127) / 128 <= MX_ONE;
  UpSmallKernel up;
  switch (quant) {
  // The MXFP4 static-count variant needs every up row (over H) at MX_STATIC chunks.
  case Q_MXFP4: up = up_small_k<Q_MXFP4>(one_up, T, (a.hidden + 127) / 128 == MX_STATIC, false, !fr ? 0 : ra.resid ? 2 : 1); break;
  case Q_BF16: up = up_small_k<Q_BF16>(true, T); break;
  case Q_MLX4: up = up_small_k<Q_MLX4>(true, T, mlx_staged_up(a.hidden), (a.hidden + 63) / 64 == 2 * MLX_NCW); break;
  default: up = up_small_k<Q_MLX8>(true, T, mlx_staged_up(a.hidden), (a.hidden + 63) / 64 == 2 * MLX_NCW); break;
  }
  // The decode kernels stage rows in dynamic LDS beyond the default 64 KiB window (gfx950 has
  // 160 KiB per compute unit).
  static std::once_flag lds_once;
  std::call_once(lds_once, [] {
    const void *ks[] = {(const void *)up_small_k<Q_MXFP4>(true, 1), (const void *)up_small_k<Q_MXFP4>(false, 1),
                        (const void *)up_small_k<Q_MXFP4>(true, SMALL_T), (const void *)up_small_k<Q_MXFP4>(false, SMALL_T),
                        (const void *)up_small_k<Q_BF16>(true, 1), (const void *)up_small_k<Q_MLX4>(true, 1),
                        (const void *)up_small_k<Q_MLX8>(true, 1), (const void *)up_small_k<Q_BF16>(true, SMALL_T),
                        (const void *)up_small_k<Q_MLX4>(true, SMALL_T), (const void *)up_small_k<Q_MLX8>(true, SMALL_T),
                        (const void *)down_small_k<Q_MXFP4>(4, true), (const void *)down_small_k<Q_BF16>(4, true),
                        (const void *)down_small_k<Q_MLX4>(4, true), (const void *)down_small_k<Q_MLX8>(4, true),
                        (const void *)down_small_k<Q_MXFP4>(9, true), (const void *)down_small_k<Q_BF16>(9, true),
                        (const void *)down_small_k<Q_MLX4>(9, true), (const void *)down_small_k<Q_MLX8>(9, true),
                        (const void *)up_small_k<Q_MXFP4>(true, 1, true), (const void *)up_small_k<Q_MXFP4>(true, SMALL_T, true),
                        (const void *)up_small_k<Q_MLX4>(true, 1, true), (const void *)up_small_k<Q_MLX4>(true, SMALL_T, true),
                        (const void *)up_small_k<Q_MLX8>(true, 1, true), (const void *)up_small_k<Q_MLX8>(true, SMALL_T, true),
                        (const void *)up_small_k<Q_MLX4>(true, 1, true, true), (const void *)up_small_k<Q_MLX8>(true, 1, true, true),
                        (const void *)down_small_k<Q_MLX4>(4, true, true), (const void *)down_small_k<Q_MLX4>(9, true, true),
                        (const void *)down_small_k<Q_MLX8>(4, true, true), (const void *)down_small_k<Q_MLX8>(9, true, true),
                        (const void *)up_small_k<Q_MXFP4>(true, 1, true, false, true), (const void *)up_small_k<Q_MXFP4>(true, SMALL_T, true, false, true),
                        (const void *)up_small_k<Q_MXFP4>(true, 1, false, false, true), (const void *)up_small_k<Q_MXFP4>(true, SMALL_T, false, false, true),
                        (const void *)up_small_k<Q_MXFP4>(true, 1, true, false, 2), (const void *)up_small_k<Q_MXFP4>(true, SMALL_T, true, false, 2),
                        (const void *)up_small_k<Q_MXFP4>(true, 1, false, false, 2), (const void *)up_small_k<Q_MXFP4>(true, SMALL_T, false, false, 2)};
    // Best effort: HIP on gfx950 accepts launches up to the hardware LDS size without it, and
    // a runtime that rejects the attribute must not leave its error for the launch check below.
    for (const void *k : ks) {
      (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      (void)hipGetLastError();
    }
  });
  static int ncu = 0;
  if (!ncu) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0) ncu = 256;
  }
  a.row_tiles = a.ldh / (mx ? UP_ROWS : 16);   // up_small: one 16-intermediate tile per workgroup
  const size_t lds_up = mx ? (size_t)T * NTX * mx_row_bytes(a.xld) + 64 * (a.hidden / 32)
                           : (size_t)T * (a.hidden + LDS_PAD) * 2;
  // Persistent: as many workgroups per compute unit as are co-resident (registers, and the staged
  // x rows in LDS), up to two (MXFP4, whose launch bounds hold two) or four (the others): a grid
  // larger than that leaves workgroups waiting for earlier ones to exit.
  const int up_per_cu = std::min(mx ? 2 : 4, resident_per_cu((const void *)up, 256, lds_up));
  const int up_grid = std::min(up_per_cu * ncu, a.row_tiles * maxu);
  FuseArgs f{};
  if (fr) {
    if (!fused_router_fits(quant, a.hidden, a.experts, ra.router, T)) return hipErrorInvalidValue;
    f = *fr;
    f.R = T * (a.experts + 1);
  }
  hipExtLaunchKernelGGL(up, dim3(f.R + up_grid), dim3(256), lds_up, s, tm_up.start, tm_up.stop, 0, a, ra, f);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_down_small(quant, a, ra.topk_idx, T, s, tm_down);
}

// The decode down product alone (the second launch of launch_small): slot values of T ≤ 16
// tokens summed in rank order into a.y. Also the operator-level projection's T ≤ 16 path.
#ifdef HH_TRACE
hipError_t trace_read(void *out, size_t bytes) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(hh_trace_buf), std::min(bytes, sizeof(hh_trace_buf)), 0,
                             hipMemcpyDeviceToHost);
}
hipError_t trace_clear() {
  static uint64_t zeros[3 * kTraceBlocks * kTracePoints];
  return hipMemcpyToSymbol(HIP_SYMBOL(hh_trace_buf), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
#endif

hipError_t launch_down_small(int quant, GemmArgs a, const int32_t *topk_idx, int T, hipStream_t s,
                             Timing tm_down) {
  if (T < 1 || T > SMALL_T) return hipErrorInvalidValue;
  const int S = a.slots;
  const int imax = std::max(a.grp[0].inter, a.grp[1].inter);
  const bool mx = quant == Q_MXFP4;
  const bool one_down = !mx || (imax + 127) / 128 <= MX_ONE;
  DownSmallKernel down;
  switch (quant) {
  case Q_MXFP4: down = down_small_k<Q_MXFP4>(S, one_down); break;
  case Q_BF16: down = down_small_k<Q_BF16>(S, true); break;
  case Q_MLX4: down = down_small_k<Q_MLX4>(S, true, mlx_staged_down(S, imax)); break;
  default: down = down_small_k<Q_MLX8>(S, true, mlx_staged_down(S, imax)); break;
  }
  static std::once_flag lds_once;
  std::call_once(lds_once, [] {
    for (int sl : {1, 2, 3, 4, 5, 6, 7, 8, 9})
      for (const void *k : {(const void *)down_small_k<Q_MXFP4>(sl, true), (const void *)down_small_k<Q_MXFP4>(sl, false),
                            (const void *)down_small_k<Q_BF16>(sl, true), (const void *)down_small_k<Q_MLX4>(sl, true),
                            (const void *)down_small_k<Q_MLX8>(sl, true), (const void *)down_small_k<Q_MLX4>(sl, true, true),
                            (const void *)down_small_k<Q_MLX8>(sl, true, true)}) {
        (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipGetLastError();
      }
  });
  static int ncu = 0;
  if (!ncu) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0) ncu = 256;
  }
  a.row_tiles = a.hidden / 16;
  // MXFP4: per slot the activation terms and 16 rows of weight scales (of the larger group).
  const size_t lds_down = mx ? (size_t)S * (NTH * mx_row_bytes(a.hld) + 16 * ((16 * (imax / 32) + 15) / 16))
                             : (size_t)S * 2 * (a.ldh + LDS_PAD) * 2;
  a.max_work = T;
  const int ks = (mx || S > 4 || !one_down) ? 1 : 2;
  // Persistent, a multiple of 8 workgroups: up to two per compute unit, as many as are co-resident.
  const int down_per_cu = std::min(2, resident_per_cu((const void *)down, 64 * S * ks, lds_down));
  const int down_grid = std::min(down_small_items(a.row_tiles, T), std::max(8, (down_per_cu * ncu) & ~7));
  hipExtLaunchKernelGGL(down, dim3(down_grid), dim3(64 * S * ks), lds_down, s, tm_down.start,
                        tm_down.stop, 0, a, topk_idx);
  return hipGetLastError();
}

// Fused decode (MXFP4, T ≤ 16, no shared expert, top_k ≤ 4, H and I ≤ MX_ONE chunks).
// Dynamic LDS: the larger of the gate-up role (x terms of T tokens + 64 rows of scales) and
// the down role (4 slots of h terms + 16 rows of scales).
size_t decode_fused_lds(const GemmArgs &a, int T) {
  const size_t up = (size_t)T * NTX * mx_row_bytes(a.xld) + 64 * (size_t)(a.hidden / 32);
  const int nsb = a.grp[0].inter / 32;
  const size_t down = 4 * ((size_t)NTH * mx_row_bytes(a.hld) + 16 * (size_t)((16 * nsb + 15) / 16));
  return std::max(up, down);
}
bool decode_fused_fits(int H, int I, int E, int K, int shared_inter) {
  return shared_inter == 0 && K <= 4 && E <= kFusedMaxE && (H + 127) / 128 <= MX_ONE && (I + 127) / 128 <= MX_ONE && H % 32 == 0 &&
         I % 32 == 0;
}
// Flag-buffer words of a T-token call's logit records (8 replicas × T·(E+1) × 4 words); the
// counters (2·kFusedCtr words) are at the end of the buffer.
int decode_fused_flags(int T, int E, int K, int I) {
  (void)I;
  (void)K;
  return 4 * kRecReplicas * T * (E + 1);
}
hipError_t launch_decode_fused(bool gemma, GemmArgs a, const RouteArgs &ra, FuseArgs f, hipStream_t s, Timing tm) {
  const int T = ra.tokens;
  if (T < 1 || T > SMALL_T) return hipErrorInvalidValue;
  static int ncu = 0;
  if (!ncu) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0) ncu = 256;
  }
  static std::once_flag lds_once;
  std::call_once(lds_once, [] {
    for (const void *k : {(const void *)decode_mx<false>, (const void *)decode_mx<true>}) {
      (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      (void)hipGetLastError();
    }
  });
  const int nup = std::min(a.experts, T * a.top_k) * (a.grp[0].inter / UP_ROWS);
  a.row_tiles = a.hidden / 16;
  f.R = T * (a.experts + 1);
  // Every gate-up item has its own workgroup: every down item needs all items of its experts, so
  // a second round of items would hold up the whole layer. Down workgroups beyond the resident
  // capacity start as earlier ones finish.
  f.U = std::max(1, nup);
  f.D = std::min(a.row_tiles * T, ncu);
  const size_t lds = decode_fused_lds(a, T);
  hipExtLaunchKernelGGL(gemma ? decode_mx<true> : decode_mx<false>, dim3(f.R + f.U + f.D), dim3(256), lds, s,
                        tm.start, tm.stop, 0, a, ra, f);
  return hipGetLastError();
}

hipError_t launch_combine(const float *slot_out, int slots, int H, int T, float *y,
                          const float *resid, hipStream_t s, Timing tm) {
  const size_t n4 = (size_t)T * H / 4;
  unsigned blocks = (unsigned)std::min<size_t>((n4 + 255) / 256, 4096);
  if (blocks == 0) return hipSuccess;
  hipExtLaunchKernelGGL(combine_kernel, dim3(blocks), dim3(256), 0, s, tm.start, tm.stop, 0,
                        slot_out, slots, H, T, y, resid);
  return hipGetLastError();
}

#else
// The FFN block's MXFP4 gate-up kernels with the fused router, compiled in a translation unit of
// their own (hh_gemm_block.hip): adding them leaves the code object of the other kernels as it
// was (the decode kernels' speed had moved with it).
UpSmallKernel up_small_block_k(bool st, int T) {
  if (st) return T == 1 ? up_small_mx<MX_ONE, true, 2, MX_STATIC, 2> : up_small_mx<MX_ONE, true, MX_XB_WIDE, MX_STATIC, 2>;
  return T == 1 ? up_small_mx<MX_ONE, true, 2, 0, 2> : up_small_mx<MX_ONE, true, MX_XB_WIDE, 0, 2>;
}

#endif

}  // namespace hh
