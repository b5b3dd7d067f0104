// hh_api.hip — the C ABI of include/hydra_hip.h: context, validation, scratch arena and the
// per-layer launch sequence (route → gate-up → down → combine), all on the context's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "hh_common.hpp"
#include "hydra_hip.h"

namespace hh {
hipError_t launch_route(const RouteArgs &a, hipStream_t s, Timing tm = {});
hipError_t launch_permute(const RouteArgs &a, hipStream_t s);
hipError_t launch_gemm(int phase, int quant, int nt, const GemmArgs &a, hipStream_t s, Timing tm);
hipError_t launch_small(int quant, GemmArgs a, const RouteArgs &ra, hipStream_t s, Timing tm_up,
                        Timing tm_down, const FuseArgs *fr = nullptr);
bool fused_router_fits(int quant, int H, int E, int router, int T);
int fused_router_flags(int T, int E);
int gemm_rows_per_block(int quant, int phase);
size_t decode_fused_lds(const GemmArgs &a, int T);
bool decode_fused_fits(int H, int I, int E, int K, int shared_inter);
int decode_fused_flags(int T, int E, int K, int I);
hipError_t launch_decode_fused(bool gemma, GemmArgs a, const RouteArgs &ra, FuseArgs f, hipStream_t s, Timing tm);
hipError_t launch_combine(const float *slot_out, int slots, int H, int T, float *y,
                          const float *resid, hipStream_t s, Timing tm);
hipError_t launch_block_norm(const float *hidden, const uint16_t *weight, int H, float eps,
                             int pow_form, int T, uint16_t *xn, uint16_t *xr, hipStream_t s);
hipError_t launch_block_gemma_finish(float *hidden, const float *mix, const float *dense,
                                     const uint16_t *n1, const uint16_t *n2, const uint16_t *n,
                                     const uint16_t *scalar, int H, float eps, int T,
                                     hipStream_t s);
hipError_t launch_attention_decode(const AttnArgs &a, hipStream_t s);
#ifdef HH_TRACE
hipError_t trace_read(void *out, size_t bytes);
hipError_t trace_clear();
hipError_t trace_read_route(void *out, size_t bytes);
hipError_t trace_clear_route();
#endif
hipError_t launch_down_small(int quant, GemmArgs a, const int32_t *topk_idx, int T, hipStream_t s,
                             Timing tm_down);
hipError_t launch_proj_prepare(const GemmArgs &a, const float *x, int T, int cols, int32_t *topk,
                               int32_t *order, int tile_tokens, hipStream_t s);
hipError_t launch_combine_weighted(const float *slots, const float *w, int T, int count, int size,
                                   float *y, hipStream_t s);
hipError_t launch_mxfp4_dequant(const uint8_t *blocks, const uint8_t *scales, int64_t n,
                                float *out, hipStream_t s);
hipError_t launch_mlx_dequant(const uint32_t *words, const uint16_t *scales,
                              const uint16_t *biases, int rows, int cols, int bits, int group,
                              float *out, hipStream_t s);
hipError_t launch_activation(int act, float alpha, float limit, const float *gate,
                             const float *up, int64_t n, float *out, hipStream_t s);
}  // namespace hh

struct hh_ctx {
  // Flags of the fused decode kernel: allocated and zeroed once, then only ever written with
  // flag values; `epoch` is the value of the last call.
  uint32_t *flags = nullptr;
  uint32_t epoch = 0;
  uint32_t fused_calls = 0;    // one-launch decode calls so far (the counter region parity)
  int decode_fused = -1;   // 1 on, 0 off, -1 the environment's choice
  int device = 0;
  hipStream_t stream = nullptr;
  uint8_t *arena = nullptr;
  size_t arena_bytes = 0;
  int64_t dispatches = 0;
  // Profiling: a pool of events, a start/stop pair per phase of each profiled forward call.
  bool profile = false;
  std::vector<hipEvent_t> events;
  size_t events_used = 0;
  // Graph capture: calls are recorded, not run; dispatches counted while recording are moved
  // to the graph and added back per launch.
  bool capturing = false;
  int64_t capture_base = 0;
  // Decode attention partials (per query head and chunk), grown on demand.
  float *attn = nullptr;
  size_t attn_bytes = 0;
  // Instantiated graphs of this context that are not yet destroyed: they hold the arena's and
  // the attention partials' device addresses, so neither may be reallocated while any exist.
  int live_graphs = 0;
  // This device's copy of the static scratch array (hh_moe_forward_noalloc), or NULL when its
  // address could not be resolved (scratch_error then says why).
  uint8_t *scratch = nullptr;
  std::string scratch_error;
};

struct hh_graph {
  hh_ctx *ctx = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int64_t dispatches = 0;
};

// Scratch of hh_moe_forward_noalloc: a fixed array in every device's memory, held from module
// load until the process ends. Host code never uses this name as an address (on the host it is
// only a stand-in for the symbol); static_scratch() resolves each device's copy once.
static __device__ __align__(256) uint8_t scratch[HH_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_error;

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device `device`, resolved by
// hipGetSymbolAddress on the first call per device and kept; NULL (with *err set) on failure.
uint8_t *static_scratch(int device, std::string *err) {
  if (device < 0 || device >= kMaxDevices) {
    *err = "device index beyond the static scratch table";
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return nullptr;
    }
    g_scratch_ptr[device] = (uint8_t *)p;
  }
  return g_scratch_ptr[device];
}

int fail(int code, const std::string &msg) {
  g_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(HH_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HH_HIP(call)                                  \
  do {                                                \
    hipError_t e_ = (call);                           \
    if (e_ != hipSuccess) return hip_fail(e_, #call); \
  } while (0)

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

constexpr int kMaxTokens = 1 << 16;  // tokens per call

// Scratch carve-up for T tokens of a layer shaped like d. All offsets 256-byte aligned.
struct Scratch {
  size_t lg64, lg32, wn, topk_idx, topk_w, slot_w, seg, order, work, n_work, h_hi, h_lo, slot_out, dcount;
  size_t xq, xs, hq, hs, status, total;
  size_t work_half, n_work_half;   // half_down: the down phase's items of tile_tokens / 2
  int slots, positions, ldh, max_work, tile_tokens, nt;
  int max_work_half;
  bool half_down;
  int xld, hld;   // MXFP4: row lengths of the fp8 operand terms (multiples of 512)
};

constexpr int kSmallT = 16;  // batches up to this size take the decode kernels

int token_tile_nt(const hh_moe_desc &d, int T) {
  // Prefill work items of 16·nt tokens: MXFP4 32 or 64 (below), BF16 64 once experts
  // average 64 tokens or more (the weight tile is then read once per 64 tokens), else 32.
  if (d.quant == HH_QUANT_BF16 && (int64_t)T * d.top_k >= 64 * (int64_t)d.experts) return 4;
  // MXFP4 without a shared expert, experts averaging 16 or more tokens, rows long enough for the
  // LDS rings: 64-token items for the gate-up (its 256 × 64 tiles skip the MFMAs of padding token
  // tiles, and an expert's rows are read once per 64 tokens); the down product runs the same
  // segments as 32-token items (Scratch::half_down).
  if (d.quant == HH_QUANT_MXFP4 && d.shared_intermediate == 0 && (int64_t)T * d.top_k >= 16 * (int64_t)d.experts &&
      d.hidden >= 1024 && d.intermediate >= 1024)
    return 4;
  return 2;
}

Scratch plan(const hh_moe_desc &d, int T) {
  Scratch s{};
  const int E = d.experts, K = d.top_k, H = d.hidden;
  const bool shared = d.shared_intermediate > 0;
  s.slots = K + (shared ? 1 : 0);
  s.positions = T * K + (shared ? T : 0);
  s.ldh = (int)align_up((size_t)std::max(d.intermediate, d.shared_intermediate), 64);
  s.nt = token_tile_nt(d, T);
  s.tile_tokens = 16 * s.nt;
  const int A = T * K;
  s.max_work = std::min(E, A) + (A + s.tile_tokens - 1) / s.tile_tokens +
               (shared ? (T + s.tile_tokens - 1) / s.tile_tokens : 0);
  size_t c = 0;
  auto take = [&](size_t bytes) {
    size_t o = c;
    c = align_up(c + bytes, 256);
    return o;
  };
  s.lg64 = take(sizeof(double) * (size_t)std::min(T, 16) * (E + 1));
  s.lg32 = take(sizeof(float) * (size_t)T * E);
  s.wn = take(sizeof(float) * (size_t)E);
  s.topk_idx = take(sizeof(int32_t) * (size_t)A);
  s.topk_w = take(sizeof(float) * (size_t)A);
  s.slot_w = take(sizeof(float) * (size_t)T * s.slots);
  s.seg = take(sizeof(int32_t) * (size_t)(E + 2));
  s.order = take(sizeof(int32_t) * (size_t)s.positions);
  s.work = take(sizeof(int4) * (size_t)s.max_work);
  s.n_work = take(sizeof(int32_t));
  s.dcount = take((size_t)A >= (size_t)hh::DB_MIN_ASSIGN ? sizeof(int32_t) * hh::DB_MAX * E : 0);
  // MXFP4 batches of 64-token items: the down product takes 32-token items of 256 rows, which
  // re-read the three activation terms half as often per row as 128-row tiles (a 256 × 64 tile
  // does not fit the register file).
  s.half_down = d.quant == HH_QUANT_MXFP4 && s.nt == 4 && !shared;
  s.max_work_half = s.half_down ? std::min(E, A) + (A + s.tile_tokens / 2 - 1) / (s.tile_tokens / 2) : 0;
  s.work_half = take(sizeof(int4) * (size_t)s.max_work_half);
  s.n_work_half = take(s.half_down ? sizeof(int32_t) : 0);
  const bool mx = d.quant == HH_QUANT_MXFP4;
  s.h_hi = take(mx ? 0 : sizeof(uint16_t) * (size_t)s.positions * s.ldh);
  s.h_lo = take(mx ? 0 : sizeof(uint16_t) * (size_t)s.positions * s.ldh);
  s.xld = (int)align_up((size_t)H, 512);
  s.hld = (int)align_up((size_t)s.ldh, 512);
  s.xq = take(mx ? (size_t)T * hh::NTX * s.xld : 0);
  s.xs = take(mx ? (size_t)T * hh::NTX * (s.xld / 32) : 0);
  s.hq = take(mx ? (size_t)s.positions * hh::NTH * s.hld : 0);
  s.hs = take(mx ? (size_t)s.positions * hh::NTH * (s.hld / 32) : 0);
  // Above 16 tokens the slot outputs are written only after routing, so an MLX router's fp64
  // logits [T][E+1] share their region.
  s.slot_out = take(T > kSmallT ? std::max(sizeof(float) * (size_t)T * s.slots * H,
                                           sizeof(double) * (size_t)T * (E + 1))
                                : 0);
  s.status = take(sizeof(uint32_t));
  s.total = c;
  return s;
}

int ensure_arena(hh_ctx *ctx, size_t bytes) {
  if (ctx->arena_bytes >= bytes) return HH_OK;
  if (ctx->capturing)
    return fail(HH_EINVAL, "the scratch arena must cover the call before capture (hh_ctx_reserve)");
  if (ctx->live_graphs > 0)
    return fail(HH_EINVAL, "the call needs a larger scratch arena, but graphs of this context still "
                           "use the current one (reserve before capture, or destroy the graphs)");
  HH_HIP(hipSetDevice(ctx->device));
  if (ctx->arena) {
    HH_HIP(hipStreamSynchronize(ctx->stream));
    HH_HIP(hipFree(ctx->arena));
    ctx->arena = nullptr;
    ctx->arena_bytes = 0;
  }
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) return fail(HH_ENOMEM, "scratch arena allocation failed");
  ctx->arena = (uint8_t *)p;
  ctx->arena_bytes = bytes;
  return HH_OK;
}

// Flag words of the fused decode kernels (the one-launch kernel's flags, the two-launch
// decode's logit records), per context.
constexpr size_t kFlagBytes = 1024 * 1024;

int ensure_flags(hh_ctx *ctx) {
  if (ctx->flags) return HH_OK;
  void *p = nullptr;
  if (hipMalloc(&p, kFlagBytes) != hipSuccess) return fail(HH_ENOMEM, "flag buffer allocation failed");
  if (hipMemset(p, 0, kFlagBytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    (void)hipFree(p);
    return fail(HH_EHIP, "flag buffer initialisation failed");
  }
  ctx->flags = (uint32_t *)p;
  return HH_OK;
}

// The decode launch structure of a context: hh_ctx_decode_fused's value, or for -1 the
// environment's HH_DECODE_FUSED (0, 1 or 2), else 2.
int decode_mode(const hh_ctx *ctx) {
  static const int env_mode = [] {
    const char *v = std::getenv("HH_DECODE_FUSED");
    return (v && v[0] >= '0' && v[0] <= '2' && v[1] == 0) ? v[0] - '0' : 2;
  }();
  return ctx->decode_fused < 0 ? env_mode : ctx->decode_fused;
}

// Whether a decode call takes the one-launch kernel (mode 1; it is not faster than the
// two-launch decode).
bool use_fused(const hh_ctx *ctx, const hh_moe_desc &d, int T) {
  const bool enabled = decode_mode(ctx) == 1;
  // Under capture the fused kernel's per-call flag epoch would be frozen into the graph.
  return enabled && !ctx->capturing && d.quant == HH_QUANT_MXFP4 && T <= kSmallT &&
         hh::decode_fused_fits(d.hidden, d.intermediate, d.experts, d.top_k, d.shared_intermediate) &&
         sizeof(uint32_t) * ((size_t)hh::decode_fused_flags(kSmallT, d.experts, d.top_k, d.intermediate) + 128) <= kFlagBytes;
}

int check_desc(const hh_moe_desc *d) {
  if (!d) return fail(HH_EINVAL, "desc is NULL");
  if (d->hidden <= 0 || d->intermediate <= 0 || d->experts <= 0)
    return fail(HH_EINVAL, "hidden, intermediate and experts must be positive");
  if (d->experts > hh::kMaxExperts) return fail(HH_EINVAL, "at most 512 experts");
  if (d->top_k < 1 || d->top_k > hh::kMaxTopK || d->top_k > d->experts)
    return fail(HH_ETOPK, "top_k must be in 1..8 and at most the expert count");
  if (d->quant < HH_QUANT_MXFP4 || d->quant > HH_QUANT_BF16) return fail(HH_EINVAL, "unknown quant");
  if (d->activation < HH_ACT_SWIGLU_OAI || d->activation > HH_ACT_GELU_TANH)
    return fail(HH_EINVAL, "unknown activation");
  if (d->router < HH_ROUTER_TOPK_SOFTMAX || d->router > HH_ROUTER_GEMMA)
    return fail(HH_EINVAL, "unknown router");
  if (d->shared_intermediate < 0) return fail(HH_EINVAL, "negative shared_intermediate");
  if (d->hidden % 64 || d->intermediate % 64 || d->shared_intermediate % 64)
    return fail(HH_ESHAPE, "hidden, intermediate and shared_intermediate must be multiples of 64");
  if ((d->quant == HH_QUANT_MLX4 || d->quant == HH_QUANT_MLX8) && d->group_size != 64)
    return fail(HH_ESHAPE, "MLX affine layers must use group_size 64");
  return HH_OK;
}

hh::RouteArgs route_args(const hh_moe_desc &d, const hh_moe_weights *w, uint8_t *base,
                         const Scratch &s, const uint16_t *x, const uint16_t *xr, int T) {
  hh::RouteArgs r{};
  r.x = x;
  r.xr = xr ? xr : x;
  r.router_w = w ? w->router_weight : nullptr;
  r.router_b = w ? w->router_bias : nullptr;
  r.router_scale = w ? w->router_scale : nullptr;
  r.router_pes = w ? w->router_expert_scale : nullptr;
  r.shared_gate = (w && d.shared_intermediate > 0) ? w->shared_gate : nullptr;
  if (w && w->router_bits) {
    r.router_bits = w->router_bits;
    r.rq_words = w->router_words;
    r.rq_scales = w->router_scales;
    r.rq_biases = w->router_biases;
    if (d.shared_intermediate > 0) {
      r.sg_words = w->shared_gate_words;
      r.sg_scales = w->shared_gate_scales;
      r.sg_biases = w->shared_gate_biases;
      // shared_gate marks "a shared expert is present" for the selection and dispatch code;
      // the MLX kernels read the sg_* tensors, never it.
      r.shared_gate = (const uint16_t *)w->shared_gate_words;
    }
  }
  r.tokens = T;
  r.hidden = d.hidden;
  r.experts = d.experts;
  r.top_k = d.top_k;
  r.slots = s.slots;
  r.router = d.router;
  r.tile_tokens = s.tile_tokens;
  r.want_dispatch = 1;
  r.eps = d.router_eps;
  r.logits = nullptr;
  r.lg64 = (double *)(base + (T > kSmallT && w && w->router_bits ? s.slot_out : s.lg64));
  r.lg32 = (float *)(base + s.lg32);
  r.wn = (float *)(base + s.wn);
  r.topk_idx = (int32_t *)(base + s.topk_idx);
  r.topk_w = (float *)(base + s.topk_w);
  r.slot_w = (float *)(base + s.slot_w);
  r.shared_w = nullptr;
  r.seg = (int32_t *)(base + s.seg);
  r.order = (int32_t *)(base + s.order);
  r.work = (int4 *)(base + s.work);
  r.n_work = (int32_t *)(base + s.n_work);
  r.dcount = (size_t)T * d.top_k >= (size_t)hh::DB_MIN_ASSIGN ? (int32_t *)(base + s.dcount) : nullptr;
  r.max_work = s.max_work;
  r.work_half = s.half_down ? (int4 *)(base + s.work_half) : nullptr;
  r.n_work_half = s.half_down ? (int32_t *)(base + s.n_work_half) : nullptr;
  r.max_work_half = s.max_work_half;
  if (d.quant == HH_QUANT_MXFP4 && x) {
    r.xq = base + s.xq;
    r.xs = base + s.xs;
    r.xld = s.xld;
  }
  return r;
}

void fill_group(hh::ExpertGroup &g, const hh_moe_desc &d, const void *blobs, size_t stride,
                int inter) {
  hh_blob_layout lay;
  hh_expert_blob_layout(&d, inter, &lay);
  g.blobs = (const uint8_t *)blobs;
  g.stride = stride ? stride : lay.stride_bytes;
  g.inter = inter;
  for (int i = 0; i < 9; ++i) g.off[i] = i < lay.slot_count ? lay.offset[i] : 0;
}

// The timing events of the next phase when profiling is on (none otherwise).
int phase_timing(hh_ctx *ctx, hh::Timing *tm, bool off = false) {
  *tm = hh::Timing{};
  if (!ctx->profile || off) return HH_OK;
  while (ctx->events_used + 2 > ctx->events.size()) {
    hipEvent_t ev;
    HH_HIP(hipEventCreate(&ev));
    ctx->events.push_back(ev);
  }
  tm->start = ctx->events[ctx->events_used++];
  tm->stop = ctx->events[ctx->events_used++];
  return HH_OK;
}

// The router tensors: bf16 router_weight (+ shared_gate), or an MLX-affine router.
int check_router(const hh_moe_desc *d, const hh_moe_weights *w, const uint16_t *x,
                 const uint16_t *x_router) {
  if (w->router_bits == 0) {
    if (!w->router_weight) return fail(HH_EINVAL, "router_weight is required");
    if ((uintptr_t)w->router_weight & 15) return fail(HH_EALIGN, "router_weight must be 16-byte aligned");
    if (d->shared_intermediate > 0 && !w->shared_gate)
      return fail(HH_EINVAL, "a shared expert needs shared_gate");
    return HH_OK;
  }
  if (w->router_bits != 4 && w->router_bits != 8) return fail(HH_EINVAL, "router_bits must be 0, 4 or 8");
  if (!w->router_words || !w->router_scales || !w->router_biases)
    return fail(HH_EINVAL, "an MLX router needs router_words, router_scales and router_biases");
  if (d->router == HH_ROUTER_GEMMA) return fail(HH_EINVAL, "the GEMMA router takes a bf16 projection");
  if (((uintptr_t)w->router_words | (uintptr_t)w->shared_gate_words) & 15)
    return fail(HH_EALIGN, "router_words and shared_gate_words must be 16-byte aligned");
  if (d->shared_intermediate > 0) {
    if (!w->shared_gate_words || !w->shared_gate_scales || !w->shared_gate_biases)
      return fail(HH_EINVAL, "a shared expert with an MLX router needs shared_gate_words/scales/biases");
    if (x_router && x_router != x)
      return fail(HH_EINVAL, "an MLX router with a shared expert routes on x (x_router NULL or x)");
  }
  return HH_OK;
}

// The FFN block's scratch after the layer's: the bf16 layer input, the GEMMA router's bf16
// residual, and (Gemma branches) the expert branch's fp32 output.
struct BlockScratch {
  size_t xn, xr, mix, total;
};
BlockScratch block_plan(const hh_moe_desc &d, const Scratch &s, int T, bool gemma) {
  const size_t row16 = align_up(sizeof(uint16_t) * (size_t)T * d.hidden, 256);
  const size_t row32 = align_up(sizeof(float) * (size_t)T * d.hidden, 256);
  BlockScratch b;
  b.xn = s.total;
  b.xr = b.xn + row16;
  b.mix = b.xr + (d.router == HH_ROUTER_GEMMA ? row16 : 0);
  b.total = b.mix + (gemma ? row32 : 0);
  return b;
}

// Argument checks shared by the layer entry points (HH_OK or the error code).
int check_forward(const hh_ctx *ctx, const hh_moe_desc *d, const hh_moe_weights *w,
                  const uint16_t *x, const uint16_t *x_router, int32_t T, const float *y) {
  if (!ctx) return fail(HH_EINVAL, "ctx is NULL");
  int rc = check_desc(d);
  if (rc) return rc;
  if (!w || !w->experts || !x || !y) return fail(HH_EINVAL, "experts, x and y are required");
  if (int rc = check_router(d, w, x, x_router)) return rc;
  if (d->router == HH_ROUTER_GEMMA && (!w->router_scale || !w->router_expert_scale))
    return fail(HH_EINVAL, "the GEMMA router needs router_scale and router_expert_scale");
  if (d->shared_intermediate > 0 && !w->shared_expert)
    return fail(HH_EINVAL, "a shared expert needs shared_expert");
  if (T < 0 || T > kMaxTokens) return fail(HH_EINVAL, "token count outside 0..65536");
  if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)w->experts | (uintptr_t)(x_router ? x_router : x)) & 15)
    return fail(HH_EALIGN, "x, x_router, y and experts must be 16-byte aligned");
  if (w->expert_stride % 256) return fail(HH_EALIGN, "expert_stride must be a multiple of 256");
  if (w->shared_expert && ((uintptr_t)w->shared_expert & 255))
    return fail(HH_EALIGN, "shared_expert must be 256-byte aligned");
  if ((uintptr_t)w->experts & 255) return fail(HH_EALIGN, "experts must be 256-byte aligned");

  return HH_OK;
}

// One layer over T ≥ 1 tokens with its scratch at `base` (laid out by plan(*d, T)). With
// `noalloc` the call takes neither the one-launch decode (its flag buffer is allocated on first
// use) nor profiling events.
// The FFN block's norm when the small-batch router kernel forms the layer input itself.
struct BlockIn {
  const float *hidden;
  const uint16_t *norm_w;
  float eps;
  int pow_form;
};

int forward_layer(hh_ctx *ctx, const hh_moe_desc *d, const hh_moe_weights *w, const uint16_t *x,
                  const uint16_t *x_router, int32_t T, float *y, int32_t *topk_idx, float *topk_w,
                  uint8_t *base, const Scratch &s, bool noalloc, const float *resid = nullptr,
                  const BlockIn *bin = nullptr) {
  int rc;

  hh::RouteArgs r = route_args(*d, w, base, s, x, x_router, T);
  if (topk_idx) r.topk_idx = topk_idx;
  if (topk_w) r.topk_w = topk_w;
  if (bin) {
    r.resid = bin->hidden;
    r.norm_w = bin->norm_w;
    r.norm_eps = bin->eps;
    r.norm_pow = bin->pow_form;
    r.xn_out = d->quant == HH_QUANT_MXFP4 ? nullptr : const_cast<uint16_t *>(x);
  }
  hh::Timing tm;
  rc = phase_timing(ctx, &tm, noalloc);
  if (rc) return rc;

  hh::GemmArgs g{};
  fill_group(g.grp[0], *d, w->experts, w->expert_stride, d->intermediate);
  if (d->shared_intermediate > 0) fill_group(g.grp[1], *d, w->shared_expert, 0, d->shared_intermediate);
  else g.grp[1] = g.grp[0];
  g.hidden = d->hidden;
  g.experts = d->experts;
  g.top_k = d->top_k;
  g.slots = s.slots;
  g.quant = d->quant;
  g.act = d->activation;
  g.expert_bias = d->expert_bias;
  g.group = d->group_size;
  g.alpha = d->swiglu_alpha;
  g.limit = d->swiglu_limit;
  g.ldh = s.ldh;
  g.max_work = s.max_work;
  g.x = x;
  g.order = r.order;
  g.work = r.work;
  g.n_work = r.n_work;
  g.h_hi = (uint16_t *)(base + s.h_hi);
  g.h_lo = (uint16_t *)(base + s.h_lo);
  g.slot_w = r.slot_w;
  g.slot_out = (float *)(base + s.slot_out);
  g.y = y;
  g.resid = resid;
  g.xq = r.xq;
  g.xs = r.xs;
  g.xld = s.xld;
  g.hq = base + s.hq;
  g.hs = base + s.hs;
  g.hld = s.hld;

  if (!noalloc && !resid && w->router_bits == 0 && use_fused(ctx, *d, T)) {
    // Decode in one launch (decode_mx): logits and h terms in the arena, flags in the
    // context's flag buffer.
    if ((rc = ensure_flags(ctx))) return rc;
    hh::FuseArgs f{};
    f.flags = ctx->flags;
    f.status = (uint32_t *)(base + s.status);
    if (++ctx->epoch == 0) ++ctx->epoch;   // flags start at 0
    f.epoch = ctx->epoch;
    f.seq = ctx->fused_calls++;
    f.ctr = ctx->flags + kFlagBytes / sizeof(uint32_t) - 128;   // the last 2·64 words
    HH_HIP(hh::launch_decode_fused(d->router == HH_ROUTER_GEMMA, g, r, f, ctx->stream, tm));
    for (int p = 1; p < 4; ++p) {   // the other phases are empty: keep the record aligned
      hh::Timing te;
      if ((rc = phase_timing(ctx, &te, noalloc))) return rc;
      if (te.start) {
        HH_HIP(hipEventRecord(te.start, ctx->stream));
        HH_HIP(hipEventRecord(te.stop, ctx->stream));
      }
    }
    ctx->dispatches += 1;
    return HH_OK;
  }
  // MXFP4 decode in two launches: the router runs as the first workgroups of the gate-up
  // launch (flags in the context's flag buffer; not under capture, whose graph would freeze the
  // call's flag epoch, and not for the allocation-free entry, which owns no flag buffer). In the
  // FFN block (bin) those workgroups, and the gate-up workgroups' x terms, form x from the
  // residual rows themselves.
  const bool fr = T <= kSmallT && !noalloc && (!resid || bin) && !ctx->capturing && w->router_bits == 0 &&
                  decode_mode(ctx) == 2 && hh::fused_router_fits(d->quant, d->hidden, d->experts, d->router, T) &&
                  sizeof(uint32_t) * (size_t)hh::fused_router_flags(T, d->experts) <= kFlagBytes;
  if (fr) {
    if ((rc = ensure_flags(ctx))) return rc;
    if (tm.start) {   // the routing phase is inside the gate-up launch: an empty profiled phase
      HH_HIP(hipEventRecord(tm.start, ctx->stream));
      HH_HIP(hipEventRecord(tm.stop, ctx->stream));
    }
  } else {
    HH_HIP(hh::launch_route(r, ctx->stream, tm));
  }

  if (T <= kSmallT) {
    // Decode: exact logits → gate-up (selects the top-k itself) → down with the rank-ordered
    // combine in its epilogue.
    hh::Timing tm_down, tm_comb;
    if ((rc = phase_timing(ctx, &tm, noalloc))) return rc;
    if ((rc = phase_timing(ctx, &tm_down, noalloc))) return rc;
    if ((rc = phase_timing(ctx, &tm_comb, noalloc))) return rc;
    hh::FuseArgs f{};
    if (fr) {
      f.flags = ctx->flags;
      f.status = (uint32_t *)(base + s.status);
      if (++ctx->epoch == 0) ++ctx->epoch;   // flags start at 0
      f.epoch = ctx->epoch;
    }
    HH_HIP(hh::launch_small(d->quant, g, r, ctx->stream, tm, tm_down, fr ? &f : nullptr));
    if (tm_comb.start) {   // no combine launch: an empty profiled phase keeps the record aligned
      HH_HIP(hipEventRecord(tm_comb.start, ctx->stream));
      HH_HIP(hipEventRecord(tm_comb.stop, ctx->stream));
    }
    ctx->dispatches += fr ? 2 : 3;
    return HH_OK;
  }
  int rows = hh::gemm_rows_per_block(d->quant, 0);
  g.row_tiles = (s.ldh + rows - 1) / rows;
  if ((rc = phase_timing(ctx, &tm, noalloc))) return rc;
  HH_HIP(hh::launch_gemm(0, d->quant, s.nt, g, ctx->stream, tm));
  rows = hh::gemm_rows_per_block(d->quant, 1);
  g.row_tiles = (d->hidden + rows - 1) / rows;
  if ((rc = phase_timing(ctx, &tm, noalloc))) return rc;
  if (s.half_down) {
    hh::GemmArgs gd = g;
    gd.work = r.work_half;
    gd.n_work = r.n_work_half;
    gd.max_work = s.max_work_half;
    HH_HIP(hh::launch_gemm(1, d->quant, s.nt / 2, gd, ctx->stream, tm));
  } else {
    HH_HIP(hh::launch_gemm(1, d->quant, s.nt, g, ctx->stream, tm));
  }
  if ((rc = phase_timing(ctx, &tm, noalloc))) return rc;
  HH_HIP(hh::launch_combine(g.slot_out, s.slots, d->hidden, T, y, resid, ctx->stream, tm));
  ctx->dispatches += 6;   // route logits, select, dispatch, gate-up, down, combine
  return HH_OK;
}


}  // namespace

extern "C" {

const char *hh_last_error(void) { return g_error.c_str(); }

int hh_ctx_create(hh_ctx **out, int32_t device) {
  if (!out) return fail(HH_EINVAL, "out is NULL");
  *out = nullptr;
  int n = 0;
  HH_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(HH_EINVAL, "no such device");
  HH_HIP(hipSetDevice(device));
  hh_ctx *c = new hh_ctx();
  c->device = device;
  c->scratch = static_scratch(device, &c->scratch_error);   // device is current
  // Default priority, non-blocking with respect to the legacy default stream.
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipStreamCreateWithFlags");
  }
  *out = c;
  return HH_OK;
}

int hh_ctx_destroy(hh_ctx *ctx) {
  if (!ctx) return HH_OK;
  // Teardown is best effort: every resource is released whatever an earlier release returned.
  (void)hipSetDevice(ctx->device);
  if (ctx->capturing) {   // abandon an unfinished capture
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(ctx->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
    ctx->capturing = false;
  }
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->arena) (void)hipFree(ctx->arena);
  if (ctx->attn) (void)hipFree(ctx->attn);
  if (ctx->flags) (void)hipFree(ctx->flags);
  for (hipEvent_t ev : ctx->events) (void)hipEventDestroy(ev);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return HH_OK;
}

void *hh_ctx_stream(hh_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int hh_ctx_synchronize(hh_ctx *ctx) {
  if (!ctx) return fail(HH_EINVAL, "ctx is NULL");
  if (ctx->capturing) return fail(HH_EINVAL, "the context is capturing a graph");
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hipStreamSynchronize(ctx->stream));
  return HH_OK;
}

int64_t hh_dispatch_count(const hh_ctx *ctx) { return ctx ? ctx->dispatches : 0; }

int hh_ctx_profile(hh_ctx *ctx, int32_t enable) {
  if (!ctx) return fail(HH_EINVAL, "ctx is NULL");
  if (ctx->capturing) return fail(HH_EINVAL, "the context is capturing a graph");
  ctx->profile = enable != 0;
  return HH_OK;
}

int hh_ctx_profile_read(hh_ctx *ctx, double *phase_ms, int64_t *calls) {
  if (!ctx || !phase_ms || !calls) return fail(HH_EINVAL, "NULL argument");
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hipStreamSynchronize(ctx->stream));
  for (int p = 0; p < 4; ++p) phase_ms[p] = 0.0;
  const size_t n = ctx->events_used / 8;
  for (size_t c = 0; c < n; ++c)
    for (int p = 0; p < 4; ++p) {
      float ms = 0.f;
      HH_HIP(hipEventElapsedTime(&ms, ctx->events[8 * c + 2 * p], ctx->events[8 * c + 2 * p + 1]));
      phase_ms[p] += ms;
    }
  *calls = (int64_t)n;
  ctx->events_used = 0;
  return HH_OK;
}

int hh_ctx_decode_fused(hh_ctx *ctx, int32_t enable) {
  if (!ctx) return fail(HH_EINVAL, "ctx is NULL");
  if (enable < -1 || enable > 2) return fail(HH_EINVAL, "enable must be -1, 0, 1 or 2");
  ctx->decode_fused = enable;
  return HH_OK;
}

int hh_desc_check(const hh_moe_desc *desc) { return check_desc(desc); }

int hh_expert_blob_layout(const hh_moe_desc *d, int32_t inter, hh_blob_layout *out) {
  if (!d || !out) return fail(HH_EINVAL, "NULL argument");
  const size_t H = (size_t)d->hidden, I = (size_t)inter;
  size_t sizes[9];
  int n;
  // ExpertBlobLayout.swift:78-103 (MXFP4), :127-143 (BF16), :193-223 (MLX), with the
  // MLXAffineLayout byte counts (MLXAffineLayout.swift:51-54).
  if (d->quant == HH_QUANT_MXFP4) {
    n = 6;
    sizes[0] = 2 * I * (H / 32) * 16; sizes[1] = 2 * I * (H / 32); sizes[2] = 2 * I * 2;
    sizes[3] = H * (I / 32) * 16;     sizes[4] = H * (I / 32);     sizes[5] = H * 2;
  } else if (d->quant == HH_QUANT_BF16) {
    n = 2;
    sizes[0] = 2 * I * H * 2; sizes[1] = H * I * 2;
  } else if (d->quant == HH_QUANT_MLX4 || d->quant == HH_QUANT_MLX8) {
    const size_t bits = d->quant == HH_QUANT_MLX4 ? 4 : 8, g = (size_t)d->group_size;
    if (g == 0) return fail(HH_EINVAL, "group_size is 0");
    n = 9;
    const size_t gw = I * H * bits / 8, gs = I * (H / g) * 2, dw = H * I * bits / 8, ds = H * (I / g) * 2;
    sizes[0] = gw; sizes[1] = gs; sizes[2] = gs;
    sizes[3] = gw; sizes[4] = gs; sizes[5] = gs;
    sizes[6] = dw; sizes[7] = ds; sizes[8] = ds;
  } else {
    return fail(HH_EINVAL, "unknown quant");
  }
  size_t cursor = 0;
  out->slot_count = n;
  for (int i = 0; i < 9; ++i) {
    if (i < n) {
      cursor = align_up(cursor, 256);
      out->offset[i] = cursor;
      out->bytes[i] = sizes[i];
      cursor += sizes[i];
    } else {
      out->offset[i] = out->bytes[i] = 0;
    }
  }
  out->payload_bytes = cursor;
  out->stride_bytes = align_up(cursor, 16384);
  return HH_OK;
}

int hh_ctx_reserve(hh_ctx *ctx, const hh_moe_desc *d, int32_t max_tokens) {
  if (!ctx) return fail(HH_EINVAL, "ctx is NULL");
  int rc = check_desc(d);
  if (rc) return rc;
  if (max_tokens <= 0 || max_tokens > kMaxTokens) return fail(HH_EINVAL, "max_tokens outside 1..65536");
  // The plan for a batch that switches to 64-token tiles can be smaller than for a batch just
  // below the switch; reserve the larger of the two.
  size_t need = 0;
  // Plans just below a token-tile switch can exceed the one for max_tokens.
  for (int t : {max_tokens, std::min(max_tokens, 63), std::min(max_tokens, 127)})
    need = std::max(need, plan(*d, t).total);
  return ensure_arena(ctx, need);
}

int hh_moe_forward(hh_ctx *ctx, const hh_moe_desc *d, const hh_moe_weights *w,
                   const uint16_t *x, const uint16_t *x_router, int32_t T, float *y,
                   int32_t *topk_idx, float *topk_w) {
  int rc = check_forward(ctx, d, w, x, x_router, T, y);
  if (rc) return rc;
  if (T == 0) return HH_OK;
  HH_HIP(hipSetDevice(ctx->device));
  const Scratch s = plan(*d, T);
  if ((rc = ensure_arena(ctx, s.total))) return rc;
  return forward_layer(ctx, d, w, x, x_router, T, y, topk_idx, topk_w, ctx->arena, s, false);
}

int hh_moe_block_forward(hh_ctx *ctx, const hh_moe_desc *d, const hh_moe_weights *w,
                         const hh_block_norms *nm, float *hidden, const float *dense_out,
                         int32_t T, int32_t *topk_idx, float *topk_w) {
  if (!nm || !nm->pre_norm) return fail(HH_EINVAL, "norms and norms->pre_norm are required");
  const bool gemma = nm->post_expert_norm != nullptr;
  if (gemma && (!nm->post_dense_norm || !nm->post_norm || !dense_out))
    return fail(HH_EINVAL, "Gemma branches need post_dense_norm, post_norm and dense_out");
  if (!hidden) return fail(HH_EINVAL, "hidden is NULL");
  // The layer's checks, with the bf16 input the block writes standing in for x.
  int rc = check_forward(ctx, d, w, (const uint16_t *)hidden, nullptr, T, hidden);
  if (rc) return rc;
  if (d->hidden > 8192) return fail(HH_ESHAPE, "the block entry takes hidden <= 8192");
  if (dense_out && ((uintptr_t)dense_out & 15)) return fail(HH_EALIGN, "dense_out must be 16-byte aligned");
  if (T == 0) return HH_OK;
  HH_HIP(hipSetDevice(ctx->device));
  const Scratch s = plan(*d, T);
  const BlockScratch bs = block_plan(*d, s, T, gemma);
  const bool router_resid = d->router == HH_ROUTER_GEMMA;
  const size_t o_xn = bs.xn, o_xr = bs.xr, o_mix = bs.mix;
  if ((rc = ensure_arena(ctx, bs.total))) return rc;
  uint8_t *base = ctx->arena;
  uint16_t *xn = (uint16_t *)(base + o_xn);
  uint16_t *xr = router_resid ? (uint16_t *)(base + o_xr) : nullptr;
  // Up to 16 tokens with a bf16 (non-GEMMA) router and H ≤ 4096, the router kernel forms the layer
  // input itself (one launch fewer); otherwise a norm kernel writes it first. Both round the same
  // fp64 values (row_sumsq's canonical sum).
  const BlockIn bin{hidden, nm->pre_norm, nm->eps, router_resid ? 1 : 0};
  const bool fused = T <= kSmallT && w->router_bits == 0 && !router_resid && d->hidden <= 4096;
  if (!fused) {
    HH_HIP(hh::launch_block_norm(hidden, nm->pre_norm, d->hidden, nm->eps, router_resid ? 1 : 0, T,
                                 xn, xr, ctx->stream));
    ctx->dispatches += 1;
  }
  if (!gemma)
    return forward_layer(ctx, d, w, xn, xr, T, hidden, topk_idx, topk_w, base, s, false, hidden,
                         fused ? &bin : nullptr);
  float *mix = (float *)(base + o_mix);
  if ((rc = forward_layer(ctx, d, w, xn, xr, T, mix, topk_idx, topk_w, base, s, false, nullptr,
                          fused ? &bin : nullptr)))
    return rc;
  HH_HIP(hh::launch_block_gemma_finish(hidden, mix, dense_out, nm->post_dense_norm,
                                       nm->post_expert_norm, nm->post_norm, nm->layer_scalar,
                                       d->hidden, nm->eps, T, ctx->stream));
  ctx->dispatches += 1;
  return HH_OK;
}

int hh_moe_forward_noalloc(hh_ctx *ctx, const hh_moe_desc *d, const hh_moe_weights *w,
                           const uint16_t *x, const uint16_t *x_router, int32_t T, float *y,
                           int32_t *topk_idx, float *topk_w) {
  int rc = check_forward(ctx, d, w, x, x_router, T, y);
  if (rc) return rc;
  if (T == 0) return HH_OK;
  if (!ctx->scratch) return fail(HH_EHIP, "static scratch unavailable: " + ctx->scratch_error);
  const Scratch s = plan(*d, T);
  if (s.total > HH_NOALLOC_SCRATCH_BYTES)
    return fail(HH_ENOMEM, "the call needs " + std::to_string(s.total) +
                               " bytes of scratch; the allocation-free entry point has " +
                               std::to_string((size_t)HH_NOALLOC_SCRATCH_BYTES) + " (use fewer tokens)");
  HH_HIP(hipSetDevice(ctx->device));
  return forward_layer(ctx, d, w, x, x_router, T, y, topk_idx, topk_w, ctx->scratch, s, true);
}

int hh_ctx_capture_begin(hh_ctx *ctx) {
  if (!ctx) return fail(HH_EINVAL, "ctx is NULL");
  if (ctx->capturing) return fail(HH_EINVAL, "the context is already capturing");
  if (ctx->profile) return fail(HH_EINVAL, "profiling is on: turn it off before capture");
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
  ctx->capturing = true;
  ctx->capture_base = ctx->dispatches;
  return HH_OK;
}

int hh_ctx_capture_end(hh_ctx *ctx, hh_graph **out) {
  if (!ctx || !out) return fail(HH_EINVAL, "NULL argument");
  *out = nullptr;
  if (!ctx->capturing) return fail(HH_EINVAL, "the context is not capturing");
  HH_HIP(hipSetDevice(ctx->device));
  ctx->capturing = false;
  const int64_t recorded = ctx->dispatches - ctx->capture_base;
  ctx->dispatches = ctx->capture_base;
  hipGraph_t graph = nullptr;
  HH_HIP(hipStreamEndCapture(ctx->stream, &graph));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return hip_fail(e, "hipGraphInstantiate");
  }
  hh_graph *g = new hh_graph;
  g->ctx = ctx;
  g->graph = graph;
  g->exec = exec;
  g->dispatches = recorded;
  ctx->live_graphs += 1;
  *out = g;
  return HH_OK;
}

int hh_graph_launch(hh_graph *g) {
  if (!g) return fail(HH_EINVAL, "graph is NULL");
  if (g->ctx->capturing) return fail(HH_EINVAL, "the context is capturing a graph");
  HH_HIP(hipSetDevice(g->ctx->device));
  HH_HIP(hipGraphLaunch(g->exec, g->ctx->stream));
  g->ctx->dispatches += g->dispatches;
  return HH_OK;
}

int hh_graph_destroy(hh_graph *g) {
  if (!g) return HH_OK;
  (void)hipSetDevice(g->ctx->device);   // best effort, as hh_ctx_destroy
  (void)hipStreamSynchronize(g->ctx->stream);
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  g->ctx->live_graphs -= 1;
  delete g;
  return HH_OK;
}

int hh_scatter_expert_tensor(hh_ctx *ctx, const hh_moe_desc *d, int32_t inter, int32_t slot,
                             int32_t experts, const void *src, int64_t src_bytes, void *blobs,
                             uint64_t stride) {
  if (!ctx || !d || !src || !blobs) return fail(HH_EINVAL, "NULL argument");
  if (ctx->capturing) return fail(HH_EINVAL, "the context is capturing a graph");
  int rc = check_desc(d);
  if (rc) return rc;
  hh_blob_layout lay;
  if ((rc = hh_expert_blob_layout(d, inter, &lay))) return rc;
  if (slot < 0 || slot >= lay.slot_count) return fail(HH_EINVAL, "slot outside the format's blob slots");
  if (experts <= 0) return fail(HH_EINVAL, "experts must be positive");
  if (stride == 0) stride = lay.stride_bytes;
  if (stride < lay.payload_bytes) return fail(HH_ESHAPE, "expert_stride is smaller than one blob");
  if (stride % 256 || ((uintptr_t)blobs & 255)) return fail(HH_EALIGN, "blobs and expert_stride must be 256-byte aligned");
  const size_t bytes = lay.bytes[slot];
  if (src_bytes != (int64_t)bytes * experts)
    return fail(HH_ESHAPE, "src_bytes is not experts x the slot's byte count");
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hipMemcpy2DAsync((uint8_t *)blobs + lay.offset[slot], stride, src, bytes, bytes, experts,
                          hipMemcpyDefault, ctx->stream));
  // Loading is off the hot path: return with the copy complete, so a host source can be
  // released at once.
  HH_HIP(hipStreamSynchronize(ctx->stream));
  ctx->dispatches += 1;
  return HH_OK;
}

int hh_attention_decode(hh_ctx *ctx, const float *q, const uint16_t *k_cache,
                        const uint16_t *v_cache, const uint16_t *sinks, int32_t q_heads,
                        int32_t kv_heads, int32_t head_dim, int32_t key_count, int32_t ring_size,
                        int32_t start_position, float sm_scale, float *out) {
  if (!ctx || !q || !k_cache || !v_cache || !sinks || !out) return fail(HH_EINVAL, "NULL argument");
  if (head_dim != 64 && head_dim != 128) return fail(HH_ESHAPE, "head_dim must be 64 or 128");
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || q_heads / kv_heads > hh::kAttnQM)
    return fail(HH_ESHAPE, "q_heads must be kv_heads x 1..8");
  if (key_count < 0 || ring_size < 0 || start_position < 0 || (ring_size > 0 && key_count > ring_size))
    return fail(HH_EINVAL, "key_count, ring_size and start_position must be >= 0, keys within the ring");
  if (((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)q) & 15)
    return fail(HH_EALIGN, "q and the caches must be 16-byte aligned");
  // The key count and ring position are kernel arguments: a recorded graph would replay them
  // unchanged at every later step.
  if (ctx->capturing)
    return fail(HH_EINVAL, "hh_attention_decode cannot be recorded in a graph (its key count and "
                           "ring position change every step); call it eagerly");
  // Chunks of at least 256 keys (one 64-key tile per wave), up to ~1024 workgroups.
  const int chunks = std::max(1, std::min(key_count / 256, std::max(1, hh::kAttnMaxChunks / kv_heads)));
  const int per_chunk = std::max(1, (key_count + chunks - 1) / chunks);
  const size_t slots = (size_t)q_heads * chunks;
  const size_t need = sizeof(float) * slots * (2 + (size_t)head_dim);
  HH_HIP(hipSetDevice(ctx->device));
  if (ctx->attn_bytes < need) {
    if (ctx->live_graphs > 0)
      return fail(HH_EINVAL, "the call needs larger attention partials, but graphs of this context "
                             "still use the current ones (destroy the graphs first)");
    if (ctx->attn) {
      HH_HIP(hipStreamSynchronize(ctx->stream));
      HH_HIP(hipFree(ctx->attn));
      ctx->attn = nullptr;
      ctx->attn_bytes = 0;
    }
    void *p = nullptr;
    if (hipMalloc(&p, need) != hipSuccess) return fail(HH_ENOMEM, "attention partials allocation failed");
    ctx->attn = (float *)p;
    ctx->attn_bytes = need;
  }
  hh::AttnArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.sinks = sinks;
  a.qh = q_heads;
  a.kvh = kv_heads;
  a.d = head_dim;
  a.keys = key_count;
  a.ring = ring_size;
  a.start = start_position;
  a.chunks = chunks;
  a.per_chunk = per_chunk;
  a.scale = sm_scale;
  a.pmax = ctx->attn;
  a.pden = ctx->attn + slots;
  a.pout = ctx->attn + 2 * slots;
  a.out = out;
  HH_HIP(hh::launch_attention_decode(a, ctx->stream));
  ctx->dispatches += 2;
  return HH_OK;
}

int hh_mxfp4_dequant(hh_ctx *ctx, const uint8_t *blocks, const uint8_t *scales, int64_t n,
                     float *out) {
  if (!ctx || !blocks || !scales || !out) return fail(HH_EINVAL, "NULL argument");
  if (n < 0) return fail(HH_EINVAL, "negative block count");
  if (((uintptr_t)blocks | (uintptr_t)out) & 15) return fail(HH_EALIGN, "blocks and out must be 16-byte aligned");
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hh::launch_mxfp4_dequant(blocks, scales, n, out, ctx->stream));
  ctx->dispatches += 1;
  return HH_OK;
}

int hh_mlx_dequant(hh_ctx *ctx, const uint32_t *words, const uint16_t *scales,
                   const uint16_t *biases, int32_t rows, int32_t cols, int32_t bits,
                   int32_t group, float *out) {
  if (!ctx || !words || !scales || !biases || !out) return fail(HH_EINVAL, "NULL argument");
  if (bits != 4 && bits != 8) return fail(HH_EINVAL, "bits must be 4 or 8");
  if (rows < 0 || cols < 0 || group <= 0 || cols % group || group % (32 / bits))
    return fail(HH_ESHAPE, "cols must divide into groups and groups into words");
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hh::launch_mlx_dequant(words, scales, biases, rows, cols, bits, group, out, ctx->stream));
  ctx->dispatches += 1;
  return HH_OK;
}

int hh_router_topk(hh_ctx *ctx, const hh_moe_desc *d, const hh_moe_weights *w,
                   const uint16_t *x_router, int32_t T, double *logits, int32_t *topk_idx,
                   float *topk_w, float *shared_w) {
  if (!ctx) return fail(HH_EINVAL, "ctx is NULL");
  int rc = check_desc(d);
  if (rc) return rc;
  if (!w || !x_router || !topk_idx || !topk_w)
    return fail(HH_EINVAL, "the weights, x_router, topk_idx and topk_w are required");
  if (d->router == HH_ROUTER_GEMMA && (!w->router_scale || !w->router_expert_scale))
    return fail(HH_EINVAL, "the GEMMA router needs router_scale and router_expert_scale");
  if ((uintptr_t)x_router & 15) return fail(HH_EALIGN, "x_router must be 16-byte aligned");
  if (w->router_bits == 0 && !w->router_weight) return fail(HH_EINVAL, "router_weight is required");
  if (w->router_bits == 0 && ((uintptr_t)w->router_weight & 15))
    return fail(HH_EALIGN, "router_weight must be 16-byte aligned");
  if (w->router_bits) {
    hh_moe_desc dd = *d;
    if (!shared_w) dd.shared_intermediate = 0;   // no shared gate wanted
    if (int rc2 = check_router(&dd, w, x_router, x_router)) return rc2;
  }
  if (T < 0 || T > kMaxTokens) return fail(HH_EINVAL, "token count outside 0..65536");
  if (T == 0) return HH_OK;
  HH_HIP(hipSetDevice(ctx->device));
  const Scratch s = plan(*d, T);
  rc = ensure_arena(ctx, s.total);
  if (rc) return rc;
  hh::RouteArgs r = route_args(*d, w, ctx->arena, s, x_router, x_router, T);
  r.want_dispatch = 0;
  r.xq = nullptr;   // no expert products follow
  r.logits = logits;
  r.topk_idx = topk_idx;
  r.topk_w = topk_w;
  r.shared_w = shared_w;
  if (d->shared_intermediate > 0 &&
      (w->router_bits ? (!shared_w || !w->shared_gate_words) : !w->shared_gate))
    r.shared_gate = nullptr;
  HH_HIP(hh::launch_route(r, ctx->stream));
  ctx->dispatches += 2;
  return HH_OK;
}

int hh_activation(hh_ctx *ctx, const hh_moe_desc *d, const float *gate, const float *up,
                  int64_t n, float *out) {
  if (!ctx || !d || !gate || !up || !out) return fail(HH_EINVAL, "NULL argument");
  if (d->activation < HH_ACT_SWIGLU_OAI || d->activation > HH_ACT_GELU_TANH)
    return fail(HH_EINVAL, "unknown activation");
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hh::launch_activation(d->activation, d->swiglu_alpha, d->swiglu_limit, gate, up, n,
                               out, ctx->stream));
  ctx->dispatches += 1;
  return HH_OK;
}

int hh_permute(hh_ctx *ctx, const int32_t *topk_idx, int32_t T, int32_t K, int32_t E,
               int32_t *seg_offsets, int32_t *order) {
  if (!ctx || !topk_idx || !seg_offsets || !order) return fail(HH_EINVAL, "NULL argument");
  if (E <= 0 || E > hh::kMaxExperts) return fail(HH_EINVAL, "experts must be in 1..512");
  if (K < 1 || K > hh::kMaxTopK || K > E) return fail(HH_ETOPK, "top_k must be in 1..8");
  if (T < 0 || T > kMaxTokens) return fail(HH_EINVAL, "token count outside 0..65536");
  HH_HIP(hipSetDevice(ctx->device));
  hh_moe_desc d{};
  d.hidden = 64; d.intermediate = 64; d.experts = E; d.top_k = K;
  const Scratch s = plan(d, std::max(T, 1));
  int rc = ensure_arena(ctx, s.total);
  if (rc) return rc;
  hh::RouteArgs r = route_args(d, nullptr, ctx->arena, s, nullptr, nullptr, T);
  r.topk_idx = const_cast<int32_t *>(topk_idx);
  r.order = order;
  HH_HIP(hh::launch_permute(r, ctx->stream));
  ctx->dispatches += 1;
  HH_HIP(hipMemcpyAsync(seg_offsets, r.seg, sizeof(int32_t) * (E + 1), hipMemcpyDeviceToDevice,
                        ctx->stream));
  return HH_OK;
}

int hh_expert_gemm(hh_ctx *ctx, const hh_matrix *m, const float *x, int32_t T, float *y) {
  if (!ctx || !m || !x || !y || !m->weights) return fail(HH_EINVAL, "NULL argument");
  const int R = m->rows, Kc = m->cols, q = m->quant;
  if (q < HH_QUANT_MXFP4 || q > HH_QUANT_BF16) return fail(HH_EINVAL, "unknown quant");
  if (R <= 0 || Kc <= 0 || R % 64 || Kc % 64) return fail(HH_ESHAPE, "rows and cols must be positive multiples of 64");
  if (T < 0 || T > kMaxTokens) return fail(HH_EINVAL, "token count outside 0..65536");
  const bool mlx = q == HH_QUANT_MLX4 || q == HH_QUANT_MLX8;
  if (q != HH_QUANT_BF16 && !m->scales) return fail(HH_EINVAL, "MXFP4 and MLX matrices need scales");
  if (mlx && (!m->biases || m->group_size != 64)) return fail(HH_ESHAPE, "MLX matrices need biases and group_size 64");
  if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)m->weights) & 15)
    return fail(HH_EALIGN, "x, y and weights must be 16-byte aligned");
  // The down kernels stage scales (and MLX biases) with 16-byte loads and read the MXFP4 row
  // bias as part of the same one-expert blob.
  if (((uintptr_t)m->scales | (uintptr_t)m->biases | (uintptr_t)m->bias) & 15)
    return fail(HH_EALIGN, "scales, biases and bias must be 16-byte aligned");
  if (q == HH_QUANT_MXFP4 && (size_t)R * Kc / 2 > 0x7FFFFFF0u) return fail(HH_ESHAPE, "MXFP4 matrix above 2 GiB");
  if (T == 0) return HH_OK;
  HH_HIP(hipSetDevice(ctx->device));
  // Scratch: the activation operand of T rows, routing (topk, weights, order) and the work list.
  const int tile = 32;
  const size_t ldh = align_up((size_t)Kc, 64), hld = align_up(ldh, 512);
  const bool mx = q == HH_QUANT_MXFP4;
  const int items = (T + tile - 1) / tile;
  size_t c = 0;
  auto take = [&](size_t bytes) { size_t o = c; c = align_up(c + bytes, 256); return o; };
  const size_t o_hi = take(mx ? 0 : 2 * (size_t)T * ldh), o_lo = take(mx ? 0 : 2 * (size_t)T * ldh);
  const size_t o_hq = take(mx ? (size_t)T * hh::NTH * hld : 0), o_hs = take(mx ? (size_t)T * hh::NTH * (hld / 32) : 0);
  const size_t o_w = take(4 * (size_t)T), o_k = take(4 * (size_t)T), o_ord = take(4 * (size_t)T);
  const size_t o_work = take(sizeof(int4) * (size_t)items), o_nw = take(4);
  int rc = ensure_arena(ctx, c);
  if (rc) return rc;
  uint8_t *base = ctx->arena;
  // The matrix as the down tensors of a one-expert blob: offsets from the lowest pointer.
  const uint8_t *p[3] = {(const uint8_t *)m->weights, (const uint8_t *)m->scales,
                         (const uint8_t *)(mx ? m->bias : m->biases)};
  const uint8_t *lo = p[0];
  for (const uint8_t *v : p)
    if (v && v < lo) lo = v;
  hh::GemmArgs g{};
  hh::ExpertGroup &e = g.grp[0];
  e.blobs = lo;
  e.stride = 0;
  e.inter = Kc;
  auto off = [&](const uint8_t *v) { return (uint64_t)(v ? v - lo : 0); };
  if (mx) {
    e.off[3] = off(p[0]); e.off[4] = off(p[1]); e.off[5] = off(p[2]);
    e.down_bytes = (uint32_t)((size_t)R * Kc / 2);
  } else if (q == HH_QUANT_BF16) {
    e.off[1] = off(p[0]);
  } else {
    e.off[6] = off(p[0]); e.off[7] = off(p[1]); e.off[8] = off(p[2]);
  }
  g.grp[1] = g.grp[0];
  g.hidden = R;
  g.experts = 1;
  g.top_k = 1;
  g.slots = 1;
  g.quant = q;
  g.act = HH_ACT_SILU;
  g.expert_bias = (mx && m->bias) ? 1 : 0;
  g.group = m->group_size;
  g.ldh = (int)ldh;
  g.hld = (int)hld;
  g.xld = (int)hld;
  g.h_hi = (uint16_t *)(base + o_hi);
  g.h_lo = (uint16_t *)(base + o_lo);
  g.hq = base + o_hq;
  g.hs = base + o_hs;
  g.slot_w = (const float *)(base + o_w);
  g.order = (const int32_t *)(base + o_ord);
  g.work = (const int4 *)(base + o_work);
  g.n_work = (const int32_t *)(base + o_nw);
  g.y = y;
  g.slot_out = y;   // one slot per token: the slot rows are the output rows
  int32_t *topk = (int32_t *)(base + o_k);
  HH_HIP(hh::launch_proj_prepare(g, x, T, Kc, topk, (int32_t *)(base + o_ord), tile, ctx->stream));
  if (T <= kSmallT) {
    HH_HIP(hh::launch_down_small(q, g, topk, T, ctx->stream, hh::Timing{}));
  } else {
    const int rows = hh::gemm_rows_per_block(q, 1);
    g.row_tiles = (R + rows - 1) / rows;
    g.max_work = items;
    HH_HIP(hh::launch_gemm(1, q, 2, g, ctx->stream, hh::Timing{}));
  }
  ctx->dispatches += 2;
  return HH_OK;
}

#ifdef HH_TRACE
// Development build only: the decode kernels' timeline of the last call (hh_gemm.hip).
// [kernel][block][point]: kernel 0 the small-batch router (hh_route.hip), 1 gate-up, 2 down.
int hh_debug_trace_read(void *out, size_t bytes) {
  if (hh::trace_read(out, bytes) != hipSuccess) return HH_EHIP;
  return hh::trace_read_route(out, bytes) == hipSuccess ? HH_OK : HH_EHIP;
}
int hh_debug_trace_clear(void) {
  return hh::trace_clear() == hipSuccess && hh::trace_clear_route() == hipSuccess ? HH_OK : HH_EHIP;
}
#endif

int hh_expert_gemv(hh_ctx *ctx, const hh_matrix *m, const float *x, float *y) {
  return hh_expert_gemm(ctx, m, x, 1, y);
}

int hh_combine(hh_ctx *ctx, const float *slots, const float *weights, int32_t T, int32_t count,
               int32_t size, float *y) {
  if (!ctx || !slots || !y) return fail(HH_EINVAL, "NULL argument");
  if (T < 0 || count < 1 || size < 0) return fail(HH_EINVAL, "tokens, count and size must be non-negative (count ≥ 1)");
  if ((int64_t)T * size == 0) return HH_OK;
  HH_HIP(hipSetDevice(ctx->device));
  HH_HIP(hh::launch_combine_weighted(slots, weights, T, count, size, y, ctx->stream));
  ctx->dispatches += 1;
  return HH_OK;
}

// ---- the model's MoE halves as one runner ----------------------------------------------------

}  // extern "C"

struct hh_runner {
  hh_ctx *ctx = nullptr;
  struct Layer {
    bool set = false;
    hh_moe_desc desc{};
    hh_moe_weights w{};
    hh_block_norms norms{};
    const float *dense_out = nullptr;
  };
  std::vector<Layer> layers;
};

extern "C" {

int hh_runner_create(hh_ctx *ctx, int32_t layers, hh_runner **out) {
  if (!ctx || !out) return fail(HH_EINVAL, "NULL argument");
  *out = nullptr;
  if (layers <= 0 || layers > 4096) return fail(HH_EINVAL, "layers outside 1..4096");
  hh_runner *r = new hh_runner;
  r->ctx = ctx;
  r->layers.resize((size_t)layers);
  *out = r;
  return HH_OK;
}

int hh_runner_destroy(hh_runner *r) {
  delete r;
  return HH_OK;
}

int hh_runner_set_layer(hh_runner *r, int32_t layer, const hh_moe_desc *d, const hh_moe_weights *w,
                        const hh_block_norms *norms, const float *dense_out) {
  if (!r || !d || !w || !norms) return fail(HH_EINVAL, "NULL argument");
  if (layer < 0 || layer >= (int32_t)r->layers.size()) return fail(HH_EINVAL, "no such layer");
  int rc = check_desc(d);
  if (rc) return rc;
  if (!norms->pre_norm) return fail(HH_EINVAL, "norms->pre_norm is required");
  if (norms->post_expert_norm && (!norms->post_dense_norm || !norms->post_norm || !dense_out))
    return fail(HH_EINVAL, "Gemma branches need post_dense_norm, post_norm and dense_out");
  hh_runner::Layer &L = r->layers[(size_t)layer];
  L.set = true;
  L.desc = *d;
  L.w = *w;
  L.norms = *norms;
  L.dense_out = dense_out;
  return HH_OK;
}

int hh_runner_reserve(hh_runner *r, int32_t max_tokens) {
  if (!r) return fail(HH_EINVAL, "runner is NULL");
  if (max_tokens <= 0 || max_tokens > kMaxTokens) return fail(HH_EINVAL, "max_tokens outside 1..65536");
  size_t need = 0;
  for (const hh_runner::Layer &L : r->layers) {
    if (!L.set) return fail(HH_EINVAL, "a layer of the runner is not set");
    const bool gemma = L.norms.post_expert_norm != nullptr;
    for (int t : {max_tokens, std::min(max_tokens, 63), std::min(max_tokens, 127)})
      need = std::max(need, block_plan(L.desc, plan(L.desc, t), t, gemma).total);
  }
  return ensure_arena(r->ctx, need);
}

int hh_runner_forward(hh_runner *r, float *hidden, int32_t T, hh_layer_hook hook, void *user) {
  if (!r || !hidden) return fail(HH_EINVAL, "NULL argument");
  for (size_t l = 0; l < r->layers.size(); ++l) {
    const hh_runner::Layer &L = r->layers[l];
    if (!L.set) return fail(HH_EINVAL, "layer " + std::to_string(l) + " of the runner is not set");
    if (hook) {
      const int hrc = hook(user, (int32_t)l, (void *)r->ctx->stream);
      if (hrc) return fail(hrc, "the layer hook failed at layer " + std::to_string(l));
    }
    const int rc = hh_moe_block_forward(r->ctx, &L.desc, &L.w, &L.norms, hidden, L.dense_out, T,
                                        nullptr, nullptr);
    if (rc) return rc;
  }
  return HH_OK;
}

int hh_runner_capture(hh_runner *r, float *hidden, int32_t T, hh_layer_hook hook, void *user,
                      hh_graph **out) {
  if (!r || !out) return fail(HH_EINVAL, "NULL argument");
  int rc = hh_ctx_capture_begin(r->ctx);
  if (rc) return rc;
  const int frc = hh_runner_forward(r, hidden, T, hook, user);
  const std::string ferr = g_error;
  rc = hh_ctx_capture_end(r->ctx, out);
  if (frc) {
    if (*out) { hh_graph_destroy(*out); *out = nullptr; }
    return fail(frc, ferr);
  }
  return rc;
}

}  // extern "C"
