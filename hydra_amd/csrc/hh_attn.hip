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
//   phase 1, lane = key: the key row (head_dim fp16, 16-byte loads) against the q_mult queries
//            (LDS broadcast reads), one fp32 logit per head; online softmax per head across the
//            wave (max and sum reductions);
//   phase 2, lane = (key group, 8 dims): the value rows of its keys (16-byte loads), weighted by
//            the tile's probabilities (LDS), into q_mult × 8 fp32 accumulators.
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
  constexpr int QM = kAttnQM, DG = D / 8, JG = 64 / DG, KPL = 64 / JG;
  __shared__ __align__(16) float s_q[QM][D];
  __shared__ __align__(16) float s_p[4][64][QM];
  __shared__ float s_m[4][QM], s_l[4][QM];
  __shared__ float s_acc[4][QM][D];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kvh = blockIdx.x % a.kvh, chunk = blockIdx.x / a.kvh;
  const int qm = a.qh / a.kvh;
  const int h0 = kvh * qm;
  for (int i = tid; i < QM * D; i += 256) {
    const int h = i / D, c = i - h * D;
    s_q[h][c] = h < qm ? a.q[(size_t)(h0 + h) * D + c] * a.scale : 0.f;
  }
  __syncthreads();
  const int first = chunk * a.per_chunk;
  const int last = min(first + a.per_chunk, a.keys);
  float M[QM], L[QM], acc[QM][8];
#pragma unroll
  for (int h = 0; h < QM; ++h) {
    M[h] = h < qm ? bf16_bits_to_f32(a.sinks[h0 + h]) : 0.f;
    L[h] = (chunk == 0 && wave == 0) ? 1.f : 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
  }
  const size_t row_stride = (size_t)a.kvh * D;   // elements between cache rows
  auto row_of = [&](int key) -> size_t {
    const long long pos = (long long)a.start + key;
    return (size_t)(a.ring > 0 ? pos % a.ring : pos);
  };
  const int jg = lane / DG, dg = lane - jg * DG;
  for (int base = first + 64 * wave; base < last; base += 256) {
    // Phase 1: lane = key base + lane.
    const int key = base + lane;
    const bool valid = key < last;
    // The tile's key rows (lane = key) and value rows (lane = key group, dims) are both issued
    // before any arithmetic: one memory latency per tile. Rows past the chunk read row `first`
    // (in bounds) and are masked.
    f16x8 kr[DG], vr[KPL];
    {
      const f16x8 *kp = (const f16x8 *)(a.k + row_of(valid ? key : first) * row_stride + (size_t)kvh * D);
#pragma unroll
      for (int c = 0; c < DG; ++c) kr[c] = kp[c];
#pragma unroll
      for (int i = 0; i < KPL; ++i) {
        const int j = base + jg * KPL + i;
        vr[i] = *(const f16x8 *)(a.v + row_of(j < last ? j : first) * row_stride + (size_t)kvh * D + 8 * dg);
      }
    }
    float s[QM];
#pragma unroll
    for (int h = 0; h < QM; ++h) s[h] = 0.f;
    if (valid) {
#pragma unroll
      for (int c = 0; c < DG; ++c) {
        float kf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] = (float)kr[c][e];
#pragma unroll
        for (int h = 0; h < QM; ++h) {
          // 16-byte broadcast reads of the query (every lane reads the same address).
          const f32x4 qa = *(const f32x4 *)&s_q[h][8 * c], qb = *(const f32x4 *)&s_q[h][8 * c + 4];
          s[h] = fmaf(qa[0], kf[0], s[h]);
          s[h] = fmaf(qa[1], kf[1], s[h]);
          s[h] = fmaf(qa[2], kf[2], s[h]);
          s[h] = fmaf(qa[3], kf[3], s[h]);
          s[h] = fmaf(qb[0], kf[4], s[h]);
          s[h] = fmaf(qb[1], kf[5], s[h]);
          s[h] = fmaf(qb[2], kf[6], s[h]);
          s[h] = fmaf(qb[3], kf[7], s[h]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < QM; ++h) {
      const float mt = wave_max(valid ? s[h] : -INFINITY);
      const float mn = fmaxf(M[h], mt);
      const float corr = __expf(M[h] - mn);
      const float p = valid ? __expf(s[h] - mn) : 0.f;
      L[h] = L[h] * corr + wave_sum(p);
      M[h] = mn;
      s_p[wave][lane][h] = p;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] *= corr;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // Phase 2: lane = (key group jg, dims 8·dg .. 8·dg + 7).
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int j = jg * KPL + i;
      const f16x8 vv = vr[i];   // a masked key has p = 0
      const f32x4 pa = *(const f32x4 *)&s_p[wave][j][0], pb = *(const f32x4 *)&s_p[wave][j][4];
      const float pj[QM] = {pa[0], pa[1], pa[2], pa[3], pb[0], pb[1], pb[2], pb[3]};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float vf = (float)vv[e];
#pragma unroll
        for (int h = 0; h < QM; ++h) acc[h][e] = fmaf(pj[h], vf, acc[h][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();   // s_p is rewritten by the next tile
  }
  // Sum the key groups of the wave (lanes with the same dg), then merge the waves in LDS.
#pragma unroll
  for (int h = 0; h < QM; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int o = DG; o < 64; o <<= 1) acc[h][e] += __shfl_xor(acc[h][e], o);
  if (lane < QM) {
#pragma unroll
    for (int h = 0; h < QM; ++h)
      if (lane == h) {
        s_m[wave][h] = M[h];
        s_l[wave][h] = L[h];
      }
  }
  if (jg == 0) {
#pragma unroll
    for (int h = 0; h < QM; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[wave][h][8 * dg + e] = acc[h][e];
  }
  __syncthreads();
  for (int i = tid; i < qm * D; i += 256) {
    const int h = i / D, c = i - h * D;
    float g = s_m[0][h];
    for (int w = 1; w < 4; ++w) g = fmaxf(g, s_m[w][h]);
    float den = 0.f, o = 0.f;
    for (int w = 0; w < 4; ++w) {
      const float f = __expf(s_m[w][h] - g);
      den += s_l[w][h] * f;
      o += s_acc[w][h][c] * f;
    }
    const size_t slot = (size_t)(h0 + h) * a.chunks + chunk;
    a.pout[slot * D + c] = o;
    if (c == 0) {
      a.pmax[slot] = g;
      a.pden[slot] = den;
    }
  }
}

// One workgroup of 64 per query head. Lanes take chunks for the maximum and the denominator
// (wave reductions), the chunk weights go to LDS, then lane i sums dimension i (and i + 64) over
// the chunks in order, loads issued eight chunks at a time.
template <int D>
__global__ __launch_bounds__(64) void attn_merge_kernel(AttnArgs a) {
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
