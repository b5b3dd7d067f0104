// hh_gemm.hip — grouped expert products on gfx950 MFMA, shared by decode and prefill.
//
// Two kernels per weight format:
//   PH_UP   : h[p][i] = act(gate_i · x_t + b, up_i · x_t + b) for every permuted position p
//             (token t, rank r) of an expert, stored as bf16 hi + lo so the down product sees
//             the fp32 activation to ~2^-17 relative;
//   PH_DOWN : slot[t·slots + r][j] = w(t, r) · (down_j · h[p] + b_j), one slot per (token,
//             rank); the combine then sums slots in rank order.
//
// Work decomposition. A 1-D grid of (row tile × work item) workgroups of 4 waves. A work item
// is (expert, first position, tokens ≤ 16·NT) from the device-side dispatch; a wave owns RT
// tiles of 16 output rows and NT token tiles of 16, and walks the whole K dimension in a fixed
// order with v_mfma_f32_16x16x32_bf16. The block index is remapped so that consecutive work
// items of one row tile (the token tiles of one expert, which share its weights) run on the
// same XCD and hit the same L2.
//
// Bit-exactness of prefill against token-by-token decode: every output element is produced by
// the same sequence of MFMAs with the same operands whatever T, NT, RT or the tile placement
// (no split-K, no atomics, fixed K order, rank-ordered combine); padding token lanes read a
// valid row and are never stored.
//
// MFMA operand mapping (16x16x32, lane l, lane group g = l/16): A lane l supplies row l%16,
// B lane l supplies token column l%16, each with 8 consecutive K values; D lane l holds rows
// 4g..4g+3 of column l%16. The K slots are assigned per format:
//   MXFP4, BF16: chunk c of 128 columns; MFMA s∈0..3 takes lane group g's columns
//                128c + 32g + 8s .. +8 (g's 16-byte MXFP4 block 4c+g, or its 64 bytes of bf16)
//   MLX4/MLX8  : chunk c = affine group c (64 columns); MFMA j∈0..1 takes columns
//                64c + 16g + 8j .. +8, so both MFMAs stay inside one group and the affine
//                factorisation s·Σq·x + b·Σx applies per group.
//
// Reference kernels replaced: mxfp4_gemv_vectorized (mxfp4.metal:119), mxfp4_gemm_gathered /
// mxfp4_gemm_tiled (batch.metal:96, tiled.metal:127), bf16_gemv (dense.metal:14),
// mlx_affine_gemv_t / mlx_affine_gemm_t (gemma.metal:248, :460), swiglu(_batch),
// qwen_silu_multiply, gelu_mul, write_expert_scaled, scatter_expert(_scaled).
#include "hh_common.hpp"

#include <algorithm>

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

// ---- BF16: 128-column chunks, 64 bytes per lane ---------------------------------------------
template <> struct Fmt<Q_BF16> {
  static constexpr int CHUNK = 128, NB = 4;
  struct A { u32x4 w[4]; };
  struct Row { const uint8_t *w; };
  __device__ static Row row(const uint8_t *base, int r, int K) { return {base + (size_t)r * K * 2}; }
  __device__ static void load(A &a, const Row &rw, int c, int g, int K) {
    int col = min(128 * c + 32 * g, K - 32);
    const u32x4 *p = (const u32x4 *)(rw.w + col * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s) a.w[s] = p[s];
  }
  __device__ static int bcol(int c, int g, int K) { return min(128 * c + 32 * g, K - 32); }
  __device__ static bool lane_valid(int c, int g, int K) { return 128 * c + 32 * g < K; }
};

// ---- MLX affine: 64-column chunks (one group) ------------------------------------------------
template <int BITS> struct FmtMLX {
  static constexpr int CHUNK = 64, NB = 2;
  struct A { uint32_t w[BITS / 2]; };  // 4-bit: 2 words (16 values); 8-bit: 4 words
  struct Row { const uint8_t *w; };
  __device__ static Row row(const uint8_t *words, int r, int K) {
    return {words + (size_t)r * (K * BITS / 8)};
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
  }
  __device__ static bf16x8 decode(const A &a, int j) {
    if constexpr (BITS == 4) return mlx4_to_bf16(a.w[j]);
    else return mlx8_to_bf16(a.w[2 * j], a.w[2 * j + 1]);
  }
  __device__ static int bcol(int c, int g, int) { return 64 * c + 16 * g; }
};
template <> struct Fmt<Q_MLX4> : FmtMLX<4> {};
template <> struct Fmt<Q_MLX8> : FmtMLX<8> {};

// ---- the kernel -------------------------------------------------------------------------------
// Σ of one value held by the 4 lane groups of a token column, in a fixed pairing:
// (g0 + g1) + (g2 + g3), identical in every lane.
__device__ __forceinline__ float sum_lane_groups(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

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

// Σ of the group's 64 B values of one token column (x, or h_hi + h_lo) from the lane's 2×NH
// vectors, in a fixed order (hi then lo per MFMA step, steps in order), then across the lane
// groups. Shared by every kernel so the affine bias term is computed identically.
template <int NH>
__device__ __forceinline__ float group_sum(const u32x4 (&bv)[NH][2]) {
  float v = 0.f;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    v += sum8_bf16(bv[0][jj]);
    if (NH > 1) v += sum8_bf16(bv[NH - 1][jj]);
  }
  return sum_lane_groups(v);
}

// The 4 K partials of an output element, summed in partial order.
__device__ __forceinline__ f32x4 sum_partials4(const f32x4 &p0, const f32x4 &p1, const f32x4 &p2,
                                               const f32x4 &p3) {
  f32x4 r;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) r[ii] = ((p0[ii] + p1[ii]) + p2[ii]) + p3[ii];
  return r;
}

// Gate-up epilogue of 4 intermediates i0..i0+3 of position `pos`: bias, activation, bf16 hi/lo.
template <int FMT>
__device__ __forceinline__ void up_epilogue(const GemmArgs &a, const uint8_t *blob,
                                            const ExpertGroup &grp, int i0, int pos,
                                            const f32x4 &gate, const f32x4 &up) {
  float gb[4] = {0.f, 0.f, 0.f, 0.f}, ub[4] = {0.f, 0.f, 0.f, 0.f};
  if (FMT == Q_MXFP4 && a.expert_bias) {
    const uint16_t *bias = (const uint16_t *)(blob + grp.off[2]);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      gb[ii] = bf16_bits_to_f32(bias[2 * (i0 + ii)]);
      ub[ii] = bf16_bits_to_f32(bias[2 * (i0 + ii) + 1]);
    }
  }
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const float y = activate(a.act, gate[ii] + gb[ii], up[ii] + ub[ii], a.alpha, a.limit);
    hi[ii] = f32_to_bf16_bits(y);
    lo[ii] = f32_to_bf16_bits(y - bf16_bits_to_f32(hi[ii]));
  }
  const size_t o = (size_t)pos * a.ldh + i0;
  *(u32x2 *)(a.h_hi + o) = u32x2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
  *(u32x2 *)(a.h_lo + o) = u32x2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
}

// Down epilogue of hidden rows h0..h0+3 of position `pos`: bias, routing weight, slot store.
template <int FMT>
__device__ __forceinline__ void down_epilogue(const GemmArgs &a, const uint8_t *blob,
                                              const ExpertGroup &grp, int h0, int pos,
                                              const f32x4 &r) {
  const int slot_id = a.order[pos];
  const float w = a.slot_w[slot_id];
  float db[4] = {0.f, 0.f, 0.f, 0.f};
  if (FMT == Q_MXFP4 && a.expert_bias) {
    const uint16_t *bias = (const uint16_t *)(blob + grp.off[5]);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) db[ii] = bf16_bits_to_f32(bias[h0 + ii]);
  }
  f32x4 o;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) o[ii] = w * (r[ii] + db[ii]);
  *(f32x4 *)(a.slot_out + (size_t)slot_id * a.hidden + h0) = o;
}

// KS = K partials per output element: partial p accumulates chunks c ≡ p (mod KS) in increasing
// order and the partials are summed in p order. The workgroup's 4 waves are 4/KS row groups ×
// KS partials. Every variant used on one layer shares KS, so a token's result does not depend
// on which variant (decode or prefill tiling) computed it.
//
// Pipeline: the weight (A) operand of the next DA chunks and the B operand of the next DB
// chunks are in flight while a chunk is computed.
//
// TP > 0 (decode): the B rows of up to TP tokens are staged once per workgroup in LDS
// ([NH][TP][K] bf16, dynamic shared memory) and read from there, so the vector memory unit
// only carries weight bytes; a work item with more tokens takes several passes.
template <int PH, int FMT, int RT, int NT, int DA, int DB, int KS, int TP>
__global__ __launch_bounds__(256) void expert_gemm(GemmArgs a) {
  using F = Fmt<FMT>;
  constexpr bool MLX = (FMT == Q_MLX4 || FMT == Q_MLX8);
  constexpr int NM = (PH == PH_UP) ? 2 * RT : RT;   // A matrices (row tiles) per wave
  constexpr int NBV = F::NB;                          // B vectors per token tile per chunk
  constexpr int NH = (PH == PH_UP) ? 1 : 2;           // B operand terms (x | h_hi, h_lo)
  constexpr int RG = 4 / KS;                          // row groups per workgroup
  constexpr int ROWS = RG * 16 * RT;                  // output rows per workgroup
  constexpr int TOK = TP > 0 ? TP : 16 * NT;          // tokens per pass
  static_assert(KS == 1 || KS == 2 || KS == 4, "KS divides the 4 waves");
  static_assert(TP == 0 || (NT == 1 && TP <= 16), "LDS-staged B uses one 16-column tile");
  extern __shared__ __align__(16) uint16_t s_b[];     // [NH][TP][K] when TP > 0
  static_assert(DA % DB == 0, "the B ring depth divides the A ring depth");

  // XCD-aware block order: hardware places block b on XCD b % 8; give each XCD a contiguous
  // range of logical ids, logical = row_tile · max_work + work_item.
  const int nblk = gridDim.x;
  const int b = blockIdx.x;
  const int xcd = b & 7, slot = b >> 3;
  const int per = (nblk + 7) >> 3;
  int rem = nblk & 7;
  if (rem == 0) rem = 8;
  const int logical = (xcd < rem ? xcd * per : rem * per + (xcd - rem) * (per - 1)) + slot;
  const int rt = logical / a.max_work;
  const int wi = logical - rt * a.max_work;
  if (rt >= a.row_tiles || wi >= *a.n_work) return;

  const int4 item = a.work[wi];
  const int e = item.x, pos0 = item.y, nitem = item.z;
  const int gsel = (e == a.experts) ? 1 : 0;
  const ExpertGroup &grp = a.grp[gsel];
  const uint8_t *blob = grp.blobs + (gsel ? 0 : (size_t)e * grp.stride);
  const int I = grp.inter, H = a.hidden;
  const int out_dim = (PH == PH_UP) ? I : H;
  const int K = (PH == PH_UP) ? H : I;
  if (rt * ROWS >= out_dim) return;                     // whole workgroup beyond this expert

  const int tid = threadIdx.x, lane = tid & 63;
  // The wave index is uniform across the wave; readfirstlane lets the compiler keep it (and
  // the loop bounds derived from it) in scalar registers, so the K loop has scalar control
  // flow and the load pipeline gets exact wait counts.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int rg = wave / KS, kp = wave % KS;             // row group, K partial
  const int rb = rt * ROWS + rg * 16 * RT;              // first output row of this wave

  // A rows of this lane (row l16 of each 16-row tile).
  typename F::Row arow[NM];
  const uint8_t *mscale[NM];   // MLX: scales of the matrix of tile m (bf16 [rows][K/64])
  const uint8_t *mbias[NM];    // MLX: biases
  int tile_row0[NM];           // first matrix row of tile m (for the D-row scales)
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int q = m % RT;
    const bool is_up = (PH == PH_UP) && (m >= RT);
    const int r0 = min(rb + 16 * q, out_dim - 16);
    const int orow = r0 + l16;   // output row (intermediate or hidden)
    tile_row0[m] = r0;
    if constexpr (FMT == Q_MXFP4) {
      if (PH == PH_UP) arow[m] = F::row(blob + grp.off[0], blob + grp.off[1], 2 * orow + (is_up ? 1 : 0), K);
      else arow[m] = F::row(blob + grp.off[3], blob + grp.off[4], orow, K);
    } else if constexpr (FMT == Q_BF16) {
      if (PH == PH_UP) arow[m] = F::row(blob + grp.off[0], orow + (is_up ? I : 0), K);
      else arow[m] = F::row(blob + grp.off[1], orow, K);
    } else {
      const int mat = (PH == PH_UP) ? (is_up ? 1 : 0) : 2;
      arow[m] = F::row(blob + grp.off[3 * mat], orow, K);
      mscale[m] = blob + grp.off[3 * mat + 1];
      mbias[m] = blob + grp.off[3 * mat + 2];
    }
  }

  const int nch = (K + F::CHUNK - 1) / F::CHUNK;
  // This wave's chunks: c = kp, kp + KS, ...
  const int my_n = nch > kp ? (nch - kp + KS - 1) / KS : 0;

  __shared__ f32x4 s_red[KS > 1 ? 4 : 1][NM][NT][64];

  for (int t0 = 0; t0 < nitem; t0 += TOK) {
    const int ntok = min(TOK, nitem - t0);
    // B rows of this lane (token column l16 of each token tile).
    const uint16_t *brow[NT][NH];
    int bpos[NT];
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      const int j = 16 * st + l16;
      const int p = pos0 + t0 + (j < ntok ? j : 0);
      bpos[st] = p;
      if (TP > 0) {
        // LDS rows of the pass; padding columns repeat row 0.
        brow[st][0] = s_b + (size_t)(j < ntok ? j : 0) * K;
        if (NH > 1) brow[st][NH - 1] = s_b + (size_t)(TP + (j < ntok ? j : 0)) * K;
      } else if (PH == PH_UP) {
        const int slot_id = a.order[p];
        brow[st][0] = a.x + (size_t)(slot_id / a.slots) * H;
      } else {
        brow[st][0] = a.h_hi + (size_t)p * a.ldh;
        if (NH > 1) brow[st][NH - 1] = a.h_lo + (size_t)p * a.ldh;
      }
    }
    if constexpr (TP > 0) {
      // Stage the pass's B rows: K/8 16-byte vectors per row, all 256 threads.
      const int per_row = K / 8;
      const int total = NH * ntok * per_row;
      for (int v = tid; v < total; v += 256) {
        const int hh = v / (ntok * per_row);
        const int rem2 = v - hh * ntok * per_row;
        const int j = rem2 / per_row, q = rem2 - j * per_row;
        const int p = pos0 + t0 + j;
        const uint16_t *src;
        if (PH == PH_UP) src = a.x + (size_t)(a.order[p] / a.slots) * H;
        else src = (hh == 0 ? a.h_hi : a.h_lo) + (size_t)p * a.ldh;
        *(u32x4 *)(s_b + (size_t)(hh * TP + j) * K + 8 * q) = *(const u32x4 *)(src + 8 * q);
      }
      __syncthreads();
    }

    f32x4 acc[NM][NT];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int st = 0; st < NT; ++st) acc[m][st] = f32x4{0.f, 0.f, 0.f, 0.f};

    struct StageA { typename F::A w[NM]; };
    struct StageB { u32x4 bv[NT][NH][NBV]; };
    StageA sa[DA];
    StageB sb[DB];

    // Chunk of pipeline step i, clamped into [0, nch): steps past the wave's last chunk reload
    // it, and a wave with no chunk at all (K shorter than KS chunks) loads chunk nch - 1, never
    // a negative one.
    const int last = my_n > 0 ? my_n - 1 : 0;
    auto chunk_of = [&](int i) { return min(kp + KS * min(i, last), nch - 1); };
    auto load_a = [&](StageA &s, int i) {
      const int c = chunk_of(i);
#pragma unroll
      for (int m = 0; m < NM; ++m) F::load(s.w[m], arow[m], c, g, K);
    };
    auto load_b = [&](StageB &s, int i) {
      const int c = chunk_of(i);
      const int col = F::bcol(c, g, K);
#pragma unroll
      for (int st = 0; st < NT; ++st)
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
          const u32x4 *p = (const u32x4 *)(brow[st][hh] + col);
#pragma unroll
          for (int v = 0; v < NBV; ++v) s.bv[st][hh][v] = p[v];
        }
    };

    auto compute_stage = [&](const StageA &s, const StageB &sbv, int i) {
      const int c = kp + KS * i;
      if constexpr (!MLX) {
        const bool ok = F::lane_valid(c, g, K);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            bf16x8 av;
            if constexpr (FMT == Q_MXFP4) av = mxfp4_to_bf16(ok ? s.w[m].w[v] : 0u, e8m0_to_f32(s.w[m].s));
            else av = as_bf16x8(ok ? s.w[m].w[v] : u32x4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int st = 0; st < NT; ++st)
#pragma unroll
              for (int hh = 0; hh < NH; ++hh) acc[m][st] = mfma(av, as_bf16x8(sbv.bv[st][hh][v]), acc[m][st]);
          }
        }
      } else {
        f32x4 P[NM][NT];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int st = 0; st < NT; ++st) P[m][st] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            const bf16x8 av = F::decode(s.w[m], jj);
#pragma unroll
            for (int st = 0; st < NT; ++st)
#pragma unroll
              for (int hh = 0; hh < NH; ++hh) P[m][st] = mfma(av, as_bf16x8(sbv.bv[st][hh][jj]), P[m][st]);
          }
        }
        // Σ of the group's 64 B values of each token column (x, or h_hi + h_lo), from the
        // operands already in registers: 16 per lane in index order, then the lane groups.
        float gsum[NT];
#pragma unroll
        for (int st = 0; st < NT; ++st) {
          u32x4 gb2[NH][2];
#pragma unroll
          for (int hh = 0; hh < NH; ++hh) { gb2[hh][0] = sbv.bv[st][hh][0]; gb2[hh][1] = sbv.bv[st][hh][1]; }
          gsum[st] = group_sum<NH>(gb2);
        }
        // acc += s·P + b·Σ per D row (affine factorisation, gemma.metal:234-236).
#pragma unroll
        for (int m = 0; m < NM; ++m) {
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const size_t ri = (size_t)(tile_row0[m] + 4 * g + ii) * (K / 64) + c;
            const float sc = bf16_bits_to_f32(((const uint16_t *)mscale[m])[ri]);
            const float bi = bf16_bits_to_f32(((const uint16_t *)mbias[m])[ri]);
#pragma unroll
            for (int st = 0; st < NT; ++st) {
              acc[m][st][ii] = __builtin_fmaf(sc, P[m][st][ii], acc[m][st][ii]);
              acc[m][st][ii] = __builtin_fmaf(bi, gsum[st], acc[m][st][ii]);
            }
          }
        }
      }
    };

    // Software pipeline over this wave's chunks. Loads past the last chunk are clamped to it
    // (valid, already cached) so the steady-state loop has no branches.
#pragma unroll
    for (int u = 0; u < DA; ++u) load_a(sa[u], u);
#pragma unroll
    for (int u = 0; u < DB; ++u) load_b(sb[u], u);
    int i0 = 0;
    for (; i0 + DA <= my_n; i0 += DA) {
#pragma unroll
      for (int u = 0; u < DA; ++u) {
        compute_stage(sa[u], sb[u % DB], i0 + u);
        load_a(sa[u], i0 + u + DA);
        load_b(sb[u % DB], i0 + u + DB);
      }
    }
#pragma unroll
    for (int u = 0; u < DA; ++u) {
      if (i0 + u < my_n) {
        compute_stage(sa[u], sb[u % DB], i0 + u);
        if (i0 + u + DB < my_n) load_b(sb[u % DB], i0 + u + DB);
      }
    }

    // ---- reduce the KS partials in a fixed order, then the epilogue ----
    if constexpr (KS > 1) {
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int st = 0; st < NT; ++st) s_red[wave][m][st][lane] = acc[m][st];
      __syncthreads();
    }
    // The waves of a row group finish token tiles st ≡ kp (mod KS).
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      if ((st % KS) != kp) continue;
      const int j = 16 * st + l16;
      f32x4 r[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if constexpr (KS == 1) {
          r[m] = acc[m][st];
        } else {
          f32x4 sum = s_red[rg * KS][m][st][lane];
#pragma unroll
          for (int p = 1; p < KS; ++p) {
            const f32x4 pp = s_red[rg * KS + p][m][st][lane];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) sum[ii] = sum[ii] + pp[ii];
          }
          r[m] = sum;
        }
      }
      if (j >= ntok) continue;
#pragma unroll
      for (int q = 0; q < RT; ++q) {
        if (rb + 16 * q >= out_dim) continue;
        if constexpr (PH == PH_UP) up_epilogue<FMT>(a, blob, grp, rb + 16 * q + 4 * g, bpos[st], r[q], r[RT + q]);
        else down_epilogue<FMT>(a, blob, grp, rb + 16 * q + 4 * g, bpos[st], r[q]);
      }
    }
    if constexpr (KS > 1 || TP > 0) __syncthreads();   // s_red / s_b are reused by the next pass
  }
}

// ---- prefill: B chunks staged once per workgroup, waves on different rows ---------------------
// The 4 waves own 4·RT consecutive 16-row tiles and walk all of K together: the B operand of
// each chunk (TOK = 16·NT tokens × one chunk of columns, x or h_hi + h_lo) is loaded once by the
// whole workgroup into LDS (double-buffered, 16-byte segments XOR-swizzled by row so the MFMA
// reads are bank-conflict free) and shared by the 4 waves. Each wave keeps the 4 K partials
// (chunk c → partial c mod 4) in separate accumulators and sums them in partial order, which is
// the arithmetic expert_gemm performs with its 4 waves: a token's result is the same bits
// whichever kernel computed it.
template <int PH, int FMT, int RT, int NT, int DA>
__global__ __launch_bounds__(256) void prefill_gemm(GemmArgs a) {
  using F = Fmt<FMT>;
  constexpr bool MLX = (FMT == Q_MLX4 || FMT == Q_MLX8);
  constexpr int NM = (PH == PH_UP) ? 2 * RT : RT;
  constexpr int NBV = F::NB;                          // B vectors per lane per chunk
  constexpr int NH = (PH == PH_UP) ? 1 : 2;
  constexpr int ROWS = 4 * 16 * RT;
  constexpr int TOK = 16 * NT;
  constexpr int NSEG = F::CHUNK / 8;                  // 16-byte segments per B row chunk
  constexpr int BVEC = NH * TOK * NSEG;               // 16-byte vectors per B chunk
  constexpr int BPT = (BVEC + 255) / 256;             // per thread
  static_assert(DA == 1 || DA == 2 || DA == 4, "DA divides the 4-chunk unroll");
  __shared__ __align__(16) u32x4 s_bv[2][BVEC];

  const int nblk = gridDim.x;
  const int b = blockIdx.x;
  const int xcd = b & 7, slot = b >> 3;
  const int per = (nblk + 7) >> 3;
  int rem = nblk & 7;
  if (rem == 0) rem = 8;
  const int logical = (xcd < rem ? xcd * per : rem * per + (xcd - rem) * (per - 1)) + slot;
  const int rt = logical / a.max_work;
  const int wi = logical - rt * a.max_work;
  if (rt >= a.row_tiles || wi >= *a.n_work) return;

  const int4 item = a.work[wi];
  const int e = item.x, pos0 = item.y, nitem = item.z;
  const int gsel = (e == a.experts) ? 1 : 0;
  const ExpertGroup &grp = a.grp[gsel];
  const uint8_t *blob = grp.blobs + (gsel ? 0 : (size_t)e * grp.stride);
  const int I = grp.inter, H = a.hidden;
  const int out_dim = (PH == PH_UP) ? I : H;
  const int K = (PH == PH_UP) ? H : I;
  if (rt * ROWS >= out_dim) return;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int rb = rt * ROWS + wave * 16 * RT;

  typename F::Row arow[NM];
  const uint8_t *mscale[NM];
  const uint8_t *mbias[NM];
  int tile_row0[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int q = m % RT;
    const bool is_up = (PH == PH_UP) && (m >= RT);
    const int r0 = min(rb + 16 * q, out_dim - 16);
    const int orow = r0 + l16;
    tile_row0[m] = r0;
    if constexpr (FMT == Q_MXFP4) {
      if (PH == PH_UP) arow[m] = F::row(blob + grp.off[0], blob + grp.off[1], 2 * orow + (is_up ? 1 : 0), K);
      else arow[m] = F::row(blob + grp.off[3], blob + grp.off[4], orow, K);
    } else if constexpr (FMT == Q_BF16) {
      if (PH == PH_UP) arow[m] = F::row(blob + grp.off[0], orow + (is_up ? I : 0), K);
      else arow[m] = F::row(blob + grp.off[1], orow, K);
    } else {
      const int mat = (PH == PH_UP) ? (is_up ? 1 : 0) : 2;
      arow[m] = F::row(blob + grp.off[3 * mat], orow, K);
      mscale[m] = blob + grp.off[3 * mat + 1];
      mbias[m] = blob + grp.off[3 * mat + 2];
    }
  }
  const int nch = (K + F::CHUNK - 1) / F::CHUNK;

  for (int t0 = 0; t0 < nitem; t0 += TOK) {
    const int ntok = min(TOK, nitem - t0);
    // Staging assignment: vector v = tid + 256·k ↦ (term hh, token row n, segment sg).
    const uint16_t *bsrc[BPT];
    int bcol[BPT], bdst[BPT];
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
      const int v = min(tid + 256 * k, BVEC - 1);
      const int hh = v / (TOK * NSEG);
      const int n = (v / NSEG) % TOK;
      const int sg = v % NSEG;
      const int p = pos0 + t0 + (n < ntok ? n : 0);
      const uint16_t *row;
      if (PH == PH_UP) row = a.x + (size_t)(a.order[p] / a.slots) * H;
      else row = (hh == 0 ? a.h_hi : a.h_lo) + (size_t)p * a.ldh;
      bsrc[k] = row;
      bcol[k] = 8 * sg;
      bdst[k] = (hh * TOK + n) * NSEG + (sg ^ (n & (NSEG - 1)));
    }
    u32x4 breg[BPT];
    auto load_b = [&](int c) {
      // Columns past K (a tail chunk, or K shorter than a chunk) are clamped into the row:
      // those B values only meet zeroed weights.
      const int cc = min(c, nch - 1);
#pragma unroll
      for (int k = 0; k < BPT; ++k)
        breg[k] = *(const u32x4 *)(bsrc[k] + min(cc * F::CHUNK + bcol[k], K - 8));
    };
    auto store_b = [&](int buf) {
#pragma unroll
      for (int k = 0; k < BPT; ++k)
        if (tid + 256 * k < BVEC) s_bv[buf][bdst[k]] = breg[k];
    };
    int bpos[NT];
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      const int j = 16 * st + l16;
      bpos[st] = pos0 + t0 + (j < ntok ? j : 0);
    }

    f32x4 acc[4][NM][NT];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp)
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int st = 0; st < NT; ++st) acc[pp][m][st] = f32x4{0.f, 0.f, 0.f, 0.f};

    typename F::A sa[DA][NM];
    auto load_a = [&](typename F::A (&w)[NM], int c) {
      const int cc = min(c, nch - 1);
#pragma unroll
      for (int m = 0; m < NM; ++m) F::load(w[m], arow[m], cc, g, K);
    };

    // B operand of token tile st, MFMA step v, term hh from LDS buffer buf.
    auto bvec = [&](int buf, int st, int hh, int v) -> u32x4 {
      const int n = 16 * st + l16;
      const int sg = MLX ? (2 * g + v) : (4 * g + v);
      return s_bv[buf][(hh * TOK + n) * NSEG + (sg ^ (n & (NSEG - 1)))];
    };

    auto compute = [&](const typename F::A (&w)[NM], int buf, int c, f32x4 (&ac)[NM][NT]) {
      if constexpr (!MLX) {
        const bool ok = F::lane_valid(c, g, K);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          u32x4 bv[NT][NH];
#pragma unroll
          for (int st = 0; st < NT; ++st)
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) bv[st][hh] = bvec(buf, st, hh, v);
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            bf16x8 av;
            if constexpr (FMT == Q_MXFP4) av = mxfp4_to_bf16(ok ? w[m].w[v] : 0u, e8m0_to_f32(w[m].s));
            else av = as_bf16x8(ok ? w[m].w[v] : u32x4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int st = 0; st < NT; ++st)
#pragma unroll
              for (int hh = 0; hh < NH; ++hh) ac[m][st] = mfma(av, as_bf16x8(bv[st][hh]), ac[m][st]);
          }
        }
      } else {
        u32x4 bv[NT][NH][2];
#pragma unroll
        for (int st = 0; st < NT; ++st)
#pragma unroll
          for (int hh = 0; hh < NH; ++hh)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) bv[st][hh][jj] = bvec(buf, st, hh, jj);
        f32x4 P[NM][NT];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int st = 0; st < NT; ++st) P[m][st] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            const bf16x8 av = F::decode(w[m], jj);
#pragma unroll
            for (int st = 0; st < NT; ++st)
#pragma unroll
              for (int hh = 0; hh < NH; ++hh) P[m][st] = mfma(av, as_bf16x8(bv[st][hh][jj]), P[m][st]);
          }
        float gsum[NT];
#pragma unroll
        for (int st = 0; st < NT; ++st) gsum[st] = group_sum<NH>(bv[st]);
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const size_t ri = (size_t)(tile_row0[m] + 4 * g + ii) * (K / 64) + c;
            const float sc = bf16_bits_to_f32(((const uint16_t *)mscale[m])[ri]);
            const float bi = bf16_bits_to_f32(((const uint16_t *)mbias[m])[ri]);
#pragma unroll
            for (int st = 0; st < NT; ++st) {
              ac[m][st][ii] = __builtin_fmaf(sc, P[m][st][ii], ac[m][st][ii]);
              ac[m][st][ii] = __builtin_fmaf(bi, gsum[st], ac[m][st][ii]);
            }
          }
      }
    };

    // Prologue: B of chunk 0 in LDS, B of chunk 1 in registers, A of chunks 0..DA-1 in flight.
    load_b(0);
    store_b(0);
    load_b(1);
#pragma unroll
    for (int u = 0; u < DA; ++u) load_a(sa[u], u);
    __syncthreads();
    // Chunk c: compute from LDS buffer c % 2; then stage B of c + 1 into the other buffer and
    // fetch B of c + 2 and A of c + DA; one barrier per chunk.
    for (int c0 = 0; c0 < nch; c0 += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = c0 + u;
        if (c < nch) {
          compute(sa[u % DA], u & 1, c, acc[u]);
          load_a(sa[u % DA], c + DA);
          store_b((u + 1) & 1);
          load_b(c + 2);
          __syncthreads();
        }
      }
    }

    // Epilogue: partials summed in order, 4 intermediates / hidden rows per lane.
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      const int j = 16 * st + l16;
      if (j >= ntok) continue;
#pragma unroll
      for (int q = 0; q < RT; ++q) {
        if (rb + 16 * q >= out_dim) continue;
        if constexpr (PH == PH_UP) {
          const f32x4 gate = sum_partials4(acc[0][q][st], acc[1][q][st], acc[2][q][st], acc[3][q][st]);
          const f32x4 up = sum_partials4(acc[0][RT + q][st], acc[1][RT + q][st], acc[2][RT + q][st],
                                         acc[3][RT + q][st]);
          up_epilogue<FMT>(a, blob, grp, rb + 16 * q + 4 * g, bpos[st], gate, up);
        } else {
          const f32x4 r = sum_partials4(acc[0][q][st], acc[1][q][st], acc[2][q][st], acc[3][q][st]);
          down_epilogue<FMT>(a, blob, grp, rb + 16 * q + 4 * g, bpos[st], r);
        }
      }
    }
    __syncthreads();   // the next pass restages s_bv
  }
}

// y[t][j] = Σ_r slot[t·slots + r][j] in rank order (sum_expert_slices, dense.metal:147; the
// shared expert's slot comes last as in QwenReferenceLayer.swift:399-404).
__global__ __launch_bounds__(256) void combine_kernel(const float *slot_out, int slots, int H,
                                                      int T, float *y) {
  const size_t n4 = (size_t)T * H / 4;
  for (size_t q = blockIdx.x * 256ull + threadIdx.x; q < n4; q += (size_t)gridDim.x * 256) {
    const size_t t = (q * 4) / H, j = (q * 4) % H;
    const f32x4 *src = (const f32x4 *)(slot_out + t * slots * H + j);
    f32x4 s = src[0];
    for (int r = 1; r < slots; ++r) {
      const f32x4 v = src[(size_t)r * H / 4];
      s[0] += v[0]; s[1] += v[1]; s[2] += v[2]; s[3] += v[3];
    }
    *(f32x4 *)(y + t * H + j) = s;
  }
}

// ---- launch table -----------------------------------------------------------------------------
typedef void (*GemmKernel)(GemmArgs);

// Decode: one 16-row tile and one 16-token tile per workgroup, deep pipelining. Prefill: 32 rows
// and 64 (gate-up) or 32 (down, whose B operand is twice as wide) tokens per pass.
constexpr int LAYER_KS = 4;

constexpr int DECODE_TP = 4;   // tokens per LDS pass in decode

template <int PH, int FMT>
static GemmKernel pick(int nt) {
  constexpr int DA_DECODE = (FMT == Q_BF16) ? 2 : 4;
  if (nt <= 1) return expert_gemm<PH, FMT, 1, 1, DA_DECODE, 1, LAYER_KS, DECODE_TP>;
  // Prefill: 4 waves × RT 16-row tiles × 32 tokens (BF16 keeps one tile per wave: its
  // weight operand is 4× wider per chunk).
  constexpr int RT_P = (FMT == Q_BF16) ? 1 : 2;
  return prefill_gemm<PH, FMT, RT_P, 2, 2>;
}

int gemm_rows_per_block(int nt, int quant) {
  if (nt <= 1) return (4 / LAYER_KS) * 16;
  return 4 * 16 * (quant == Q_BF16 ? 1 : 2);
}

static GemmKernel gemm_kernel(int phase, int quant, int nt) {
  switch (quant) {
  case Q_MXFP4: return phase == PH_UP ? pick<PH_UP, Q_MXFP4>(nt) : pick<PH_DOWN, Q_MXFP4>(nt);
  case Q_BF16: return phase == PH_UP ? pick<PH_UP, Q_BF16>(nt) : pick<PH_DOWN, Q_BF16>(nt);
  case Q_MLX4: return phase == PH_UP ? pick<PH_UP, Q_MLX4>(nt) : pick<PH_DOWN, Q_MLX4>(nt);
  default: return phase == PH_UP ? pick<PH_UP, Q_MLX8>(nt) : pick<PH_DOWN, Q_MLX8>(nt);
  }
}

hipError_t launch_gemm(int phase, int quant, int nt, const GemmArgs &a, hipStream_t s, Timing tm) {
  const unsigned blocks = (unsigned)a.row_tiles * (unsigned)a.max_work;
  if (blocks == 0) return hipSuccess;
  // Decode stages DECODE_TP B rows (x, or h_hi and h_lo) of up to K = max(H, ldh) columns.
  const size_t kmax = (size_t)std::max(a.hidden, a.ldh);
  const size_t lds = nt <= 1 ? (size_t)DECODE_TP * kmax * 2 * (phase == PH_UP ? 1 : 2) : 0;
  hipExtLaunchKernelGGL(gemm_kernel(phase, quant, nt), dim3(blocks), dim3(256), lds, s, tm.start,
                        tm.stop, 0, a);
  return hipGetLastError();
}

hipError_t launch_combine(const float *slot_out, int slots, int H, int T, float *y, hipStream_t s,
                          Timing tm) {
  const size_t n4 = (size_t)T * H / 4;
  unsigned blocks = (unsigned)std::min<size_t>((n4 + 255) / 256, 4096);
  if (blocks == 0) return hipSuccess;
  hipExtLaunchKernelGGL(combine_kernel, dim3(blocks), dim3(256), 0, s, tm.start, tm.stop, 0,
                        slot_out, slots, H, T, y);
  return hipGetLastError();
}

}  // namespace hh
