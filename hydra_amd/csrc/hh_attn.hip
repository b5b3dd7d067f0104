// hh_attn.hip — decode attention with per-head sinks over an fp16 key/value history.
//
// Reference: attention_decode_split + attention_decode_merge (attention.metal:307-450), driven
// by ForwardEncoder.attention (ForwardEncoder.swift:1107-1160); semantics of
// ReferenceLayer.decode (ReferenceLayer.swift:150-180): keys start .. start + n - 1 are visible,
// key position p is cache row p % ring (ring 0: row p), the sink enters the softmax
// denominator only.
//
// MI355X layout of the work: the reference gives every query head its own threadgroups, so the
// q_mult heads of a kv head each read the same key/value rows. Here a workgroup owns (kv head,
// chunk of keys) and computes all q_mult (≤ 8) query heads of that kv head from one read of
// each row, so HBM sees the history once per call. Each of the 4 waves takes 64-key tiles:
//   phase 1, on the fp16 MFMA: S [64 keys × 16 head columns] = K·q^T with the key rows as the A
//            operand (fp16, as stored) and the scaled queries as an fp16 pair hi + lo held in
//            registers for the whole call (every product exact in fp32, q to ~2^-22); online
//            softmax per head column (16 logits per lane, then the 4 lane groups);
//   phase 2, on the fp16 MFMA: O [16 head rows × head_dim] += P·V, with the probabilities as an
//            fp16 pair hi + lo straight from the phase-1 registers (the MFMA's k order follows
//            the lanes' keys) and the value tile staged in the wave's LDS rows (16-byte loads in,
//            column reads out).
// The waves' states merge in LDS and the workgroup writes an unnormalised partial (max, sum,
// head_dim sums) per (query head, chunk); attn_merge_kernel combines the chunks of a head in
// chunk order. As in the reference, every partial starts from the sink as its running maximum
// and only chunk 0's wave 0 gives the sink its weight, so an empty chunk stays finite.
#include "hh_common.hpp"

namespace hh {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));



// Wave reductions on DPP (register moves, no LDS round trip): row_shr 1, 2, 4, 8 leave each
// 16-lane row's result in its lane 15, row_bcast 15 and 31 carry it to lane 63, read back
// with readlane. Lanes whose DPP source is outside the row or masked take the identity.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float identity, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, identity),
                                                               __builtin_bit_cast(int, v), CTRL, ROWS,
                                                               0xf, false));
}
__device__ __forceinline__ float wave_max(float v) {
  const float id = -INFINITY;
  v = fmaxf(v, dpp_f<0x111, 0xf>(id, v));
  v = fmaxf(v, dpp_f<0x112, 0xf>(id, v));
  v = fmaxf(v, dpp_f<0x114, 0xf>(id, v));
  v = fmaxf(v, dpp_f<0x118, 0xf>(id, v));
  v = fmaxf(v, dpp_f<0x142, 0xa>(id, v));
  v = fmaxf(v, dpp_f<0x143, 0xc>(id, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0x111, 0xf>(0.f, v);
  v += dpp_f<0x112, 0xf>(0.f, v);
  v += dpp_f<0x114, 0xf>(0.f, v);
  v += dpp_f<0x118, 0xf>(0.f, v);
  v += dpp_f<0x142, 0xa>(0.f, v);
  v += dpp_f<0x143, 0xc>(0.f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

template <int D>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
  warm_kernargs<sizeof(AttnArgs)>();
  constexpr int QM = kAttnQM, DG = D / 8, JG = 64 / DG, KPL = 64 / JG, NDC = D / 32, NN = D / 16;
  constexpr int VST = D + 4;   // halves per staged value row: rows 4 keys apart land 8 banks apart
  __shared__ __align__(16) float s_q[QM][D];
  __shared__ __align__(16) _Float16 s_v[4][64 * VST];
  __shared__ float s_m[4][QM], s_l[4][QM];
  __shared__ float s_acc[4][QM][D];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int kvh = blockIdx.x % a.kvh, chunk = blockIdx.x / a.kvh;
  const int qm = a.qh / a.kvh;
  const int h0 = kvh * qm;
  for (int i = tid; i < QM * D; i += 256) {
    const int h = i / D, c = i - h * D;
    s_q[h][c] = h < qm ? a.q[(size_t)(h0 + h) * D + c] * a.scale : 0.f;
  }
  __syncthreads();
  // The scaled queries as the B operand of the QK^T MFMAs: lane (g, l16) holds head l16's
  // dimensions 32·dc + 8g .. +7 as an fp16 pair hi + lo (the fp32 value to ~2^-22 relative;
  // each product with an fp16 key is exact in fp32); zero for heads ≥ qm.
  f16x8 qhi[NDC], qlo[NDC];
#pragma unroll
  for (int dc = 0; dc < NDC; ++dc)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = l16 < QM ? s_q[l16][32 * dc + 8 * g + e] : 0.f;
      const _Float16 hi = (_Float16)x;
      qhi[dc][e] = hi;
      qlo[dc][e] = (_Float16)(x - (float)hi);
    }
  const int first = chunk * a.per_chunk;
  const int last = min(first + a.per_chunk, a.keys);
  // Running maximum and denominator of head l16 (every lane group holds the same values).
  float M = l16 < qm ? bf16_bits_to_f32(a.sinks[h0 + l16]) : 0.f;
  float L = (chunk == 0 && wave == 0) ? 1.f : 0.f;
  // Unnormalised output: acc[n][i] = head 4g + i, dimension 16n + l16 (the PV MFMA's layout).
  f32x4 acc[NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const size_t row_stride = (size_t)a.kvh * D;   // elements between cache rows
  auto row_of = [&](int key) -> size_t {
    const long long pos = (long long)a.start + key;
    return (size_t)(a.ring > 0 ? pos % a.ring : pos);
  };
  const int jg = lane / DG, dg = lane - jg * DG;
  _Float16 *sv = s_v[wave];
  for (int base = first + 64 * wave; base < last; base += 256) {
    // The tile's key rows (16-key subtile st, lane (g, l16): key base + 16·st + l16, dimensions
    // 32·dc + 8g .. +7) and value rows (lane (jg, dg): keys jg·KPL .. +KPL−1, dimensions
    // 8·dg .. +7) are all issued before any arithmetic: one memory latency per tile. Rows past
    // the chunk read row `first` (in bounds) and are masked (their probabilities are zero).
    f16x8 kr[4][NDC], vr[KPL];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int key = base + 16 * st + l16;
      const f16x8 *kp = (const f16x8 *)(a.k + row_of(key < last ? key : first) * row_stride + (size_t)kvh * D);
#pragma unroll
      for (int dc = 0; dc < NDC; ++dc) kr[st][dc] = kp[4 * dc + g];
    }
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int j = base + jg * KPL + i;
      vr[i] = *(const f16x8 *)(a.v + row_of(j < last ? j : first) * row_stride + (size_t)kvh * D + 8 * dg);
    }
    // Phase 1: S = K·q^T on the fp16 MFMA; sc[st][i] is the logit of key base + 16·st + 4g + i
    // for head l16.
    f32x4 sc[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      sc[st] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dc = 0; dc < NDC; ++dc) {
        sc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[st][dc], qhi[dc], sc[st], 0, 0, 0);
        sc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[st][dc], qlo[dc], sc[st], 0, 0, 0);
      }
    }
    // The value tile into the wave's LDS rows (row = key − base), read back column-wise below.
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const u32x4 w = __builtin_bit_cast(u32x4, vr[i]);
      u32x2 *dst = (u32x2 *)(sv + (jg * KPL + i) * VST + 8 * dg);
      dst[0] = u32x2{w[0], w[1]};
      dst[1] = u32x2{w[2], w[3]};
    }
    // Online softmax of head l16 over the tile's 64 keys: 16 per lane, then the 4 lane groups.
    float mt = -INFINITY;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (base + 16 * st + 4 * g + i < last) mt = fmaxf(mt, sc[st][i]);
    mt = max_lane_groups(mt);
    const float mn = fmaxf(M, mt);
    const float corr = __expf(M - mn);
    float ps = 0.f;
    // P as the A operand of the PV MFMAs (head l16's row; k index (kc, g, e) stands for key
    // 16·(2kc + e/4) + 4g + e%4, the lane's own logits), as an fp16 pair hi + lo.
    f16x8 phi[2], plo[2];
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = base + 16 * st + 4 * g + i < last ? __expf(sc[st][i] - mn) : 0.f;
        ps += p;
        const _Float16 hi = (_Float16)p;
        phi[st >> 1][4 * (st & 1) + i] = hi;
        plo[st >> 1][4 * (st & 1) + i] = (_Float16)(p - (float)hi);
      }
    ps = sum_lane_groups(ps);
    L = L * corr + ps;
    M = mn;
    // Lane (g, l16) holds output rows 4g .. 4g + 3: their heads' rescale factors.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ci = __shfl(corr, 4 * g + i);
#pragma unroll
      for (int n = 0; n < NN; ++n) acc[n][i] *= ci;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // Phase 2: O[h][d] += Σ_key P[h][key]·V[key][d] on the fp16 MFMA; B = the value column
    // 16n + l16 at the lane's keys (the k order of P), read from the staged rows.
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        f16x8 vb;
#pragma unroll
        for (int e = 0; e < 8; ++e) vb[e] = sv[(16 * (2 * kc + (e >> 2)) + 4 * g + (e & 3)) * VST + 16 * n + l16];
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(phi[kc], vb, acc[n], 0, 0, 0);
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(plo[kc], vb, acc[n], 0, 0, 0);
      }
    __builtin_amdgcn_wave_barrier();   // the staged rows are rewritten by the next tile
  }
  // The waves' states merge in LDS.
  if (lane < QM) {   // lane h: head h's state
    s_m[wave][lane] = M;
    s_l[wave][lane] = L;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (4 * g + i < QM)
#pragma unroll
      for (int n = 0; n < NN; ++n) s_acc[wave][4 * g + i][16 * n + l16] = acc[n][i];
  __syncthreads();
  for (int i = tid; i < qm * D; i += 256) {
    const int h = i / D, c = i - h * D;
    float gm = s_m[0][h];
    for (int w = 1; w < 4; ++w) gm = fmaxf(gm, s_m[w][h]);
    float den = 0.f, o = 0.f;
    for (int w = 0; w < 4; ++w) {
      const float f = __expf(s_m[w][h] - gm);
      den += s_l[w][h] * f;
      o += s_acc[w][h][c] * f;
    }
    const size_t slot = (size_t)(h0 + h) * a.chunks + chunk;
    a.pout[slot * D + c] = o;
    if (c == 0) {
      a.pmax[slot] = gm;
      a.pden[slot] = den;
    }
  }
}

// One workgroup of 64 per query head. Lanes take chunks for the maximum and the denominator
// (wave reductions), the chunk weights go to LDS, then lane i sums dimension i (and i + 64) over
// the chunks in order, loads issued eight chunks at a time.
template <int D>
__global__ __launch_bounds__(64) void attn_merge_kernel(AttnArgs a) {
  warm_kernargs<sizeof(AttnArgs)>();
  __shared__ float s_f[kAttnMaxChunks];
  const int h = blockIdx.x, lane = threadIdx.x;
  const float *pm = a.pmax + (size_t)h * a.chunks, *pd = a.pden + (size_t)h * a.chunks;
  float g = -INFINITY;
  for (int c = lane; c < a.chunks; c += 64) g = fmaxf(g, pm[c]);
  g = wave_max(g);
  float den = 0.f;
  for (int c = lane; c < a.chunks; c += 64) den += pd[c] * __expf(pm[c] - g);
  den = wave_sum(den);
  const float inv = 1.f / den;
  for (int c = lane; c < a.chunks; c += 64) s_f[c] = __expf(pm[c] - g) * inv;
  __syncthreads();
  const float *po = a.pout + (size_t)h * a.chunks * D;
#pragma unroll
  for (int r = 0; r < D / 64; ++r) {
    const int i = lane + 64 * r;
    float sum = 0.f;
    int c = 0;
    for (; c + 8 <= a.chunks; c += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = po[(size_t)(c + u) * D + i];
#pragma unroll
      for (int u = 0; u < 8; ++u) sum = fmaf(v[u], s_f[c + u], sum);
    }
    for (; c < a.chunks; ++c) sum = fmaf(po[(size_t)c * D + i], s_f[c], sum);
    a.out[(size_t)h * D + i] = sum;
  }
}

hipError_t launch_attention_decode(const AttnArgs &a, hipStream_t s) {
  if (a.d == 64) {
    hipLaunchKernelGGL(attn_split_kernel<64>, dim3(a.kvh * a.chunks), dim3(256), 0, s, a);
    hipLaunchKernelGGL(attn_merge_kernel<64>, dim3(a.qh), dim3(64), 0, s, a);
  } else {
    hipLaunchKernelGGL(attn_split_kernel<128>, dim3(a.kvh * a.chunks), dim3(256), 0, s, a);
    hipLaunchKernelGGL(attn_merge_kernel<128>, dim3(a.qh), dim3(64), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace hh
