/*
 * hydra_hip.h — C ABI of HydraHIP, the MI355X (gfx950) mixture-of-experts layer.
 *
 * This header is the drop-in boundary that replaces the Metal MoE passes of Hydra's
 * HydraMetal module behind the HydraCore layer interface. Plain C: no C++ types, no torch
 * types, caller-owned device pointers, int status codes.
 *
 * Conventions
 *   - Every function returns HH_OK (0) or a negative HH_E* code, and never aborts.
 *     hh_last_error() returns a human-readable message for the calling thread.
 *   - Tensors are device pointers from hipMalloc (or any allocation the HIP device can read).
 *     Weight blobs follow the reference's expert blob layout byte for byte
 *     (Sources/HydraCore/ExpertBlobLayout.swift:78-103 MXFP4, :127-143 BF16, :193-223 MLX);
 *     hh_expert_blob_layout() returns the sub-tensor offsets.
 *   - One hh_ctx owns one HIP stream (the "serial encoder" of the reference,
 *     Sources/HydraMetal/MetalContext.swift:139-178). Work is enqueued in call order and no
 *     entry point synchronises the host except hh_ctx_synchronize().
 *   - bf16 values are passed as uint16_t bit patterns (little endian), fp32 as float.
 *
 * Enumerations keep the same numeric values in the fp64 oracle under oracle/.
 */
#ifndef HYDRA_HIP_H
#define HYDRA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------------- */
#define HH_OK        0
#define HH_EINVAL   -1  /* a dimension or enum is out of range, or a required pointer is NULL */
#define HH_EALIGN   -2  /* a pointer or dimension breaks an alignment the kernels rely on */
#define HH_ETOPK    -3  /* top_k outside 1..8 or above the expert count */
#define HH_EHIP     -4  /* a HIP runtime call failed; hh_last_error() has the HIP message */
#define HH_ENOMEM   -5  /* the context could not allocate its scratch arena */
#define HH_ESHAPE   -6  /* a dimension is not a multiple the format requires */

/* ---- enumerations ---------------------------------------------------------------------- */
/* Expert weight format. Also fixes how gate and up are stored:
 *   MXFP4: one fused gate_up matrix [2I][H], rows interleaved gate0, up0, gate1, ...
 *          (Sources/HydraReference/ReferenceLayer.swift:11; ReferenceOps.swift:81-82)
 *   BF16 : one fused gate_up matrix [2I][H], gate = rows 0..I-1, up = rows I..2I-1
 *          (Sources/HydraMetal/Gemma4Weights.swift:107-112)
 *   MLX4/MLX8: separate gate [I][H], up [I][H] and down [H][I] affine matrices
 *          (Sources/HydraCore/ExpertBlobLayout.swift:163-224)                                   */
typedef enum { HH_QUANT_MXFP4 = 0, HH_QUANT_MLX4 = 1, HH_QUANT_MLX8 = 2, HH_QUANT_BF16 = 3 } hh_quant;

/* Gated activation applied to (gate, up):
 *   SWIGLU_OAI: g=min(g,limit), u=clamp(u,±limit), g·σ(alpha·g)·(u+1)  (ReferenceOps.swift:87-99)
 *   SILU      : g·σ(g)·u                                              (QwenReferenceOps.swift:149-151)
 *   GELU_TANH : 0.5·g·(1+tanh(√(2/π)(g+0.044715g³)))·u               (Gemma4ReferenceOps.swift:37-45) */
typedef enum { HH_ACT_SWIGLU_OAI = 0, HH_ACT_SILU = 1, HH_ACT_GELU_TANH = 2 } hh_act;

/* Router convention:
 *   TOPK_SOFTMAX        : top-k of the logits, softmax over the k      (ReferenceOps.swift:173-183)
 *   SOFTMAX_TOPK_RENORM : softmax over all, top-k, renormalise        (QwenReferenceOps.swift:159-179)
 *   GEMMA               : unscaled RMSNorm·scale·H^-½ → logits → softmax → top-k → renormalise
 *                         → × per-expert scale                          (Gemma4ReferenceOps.swift:131-156)
 * Ties select the smaller expert index in every convention.                                 */
typedef enum { HH_ROUTER_TOPK_SOFTMAX = 0, HH_ROUTER_SOFTMAX_TOPK_RENORM = 1, HH_ROUTER_GEMMA = 2 } hh_router;

/* ---- layer description ----------------------------------------------------------------- */
/* Mirrors the hot-path fields of HydraCore's GptOssConfig (GptOssConfig.swift:60-86),
 * Qwen35MoeConfig (Qwen35MoeConfig.swift:73-128) and Gemma4Config (Gemma4Config.swift:73-77). */
typedef struct hh_moe_desc {
    int32_t hidden;              /* H: multiple of 64                                          */
    int32_t intermediate;        /* I: expert intermediate, multiple of 64                      */
    int32_t experts;             /* E: 1..512                                                   */
    int32_t top_k;               /* K: 1..8 (the reference's maxRouterTopK, ForwardEncoder.swift:133) */
    int32_t shared_intermediate; /* 0 = no shared expert; else the shared expert's I            */
    int32_t quant;               /* hh_quant                                                    */
    int32_t group_size;          /* MLX affine group (64); ignored otherwise                   */
    int32_t activation;          /* hh_act                                                      */
    int32_t router;              /* hh_router                                                   */
    int32_t expert_bias;         /* 1: MXFP4 blobs carry bf16 gate_up and down biases (GPT-OSS) */
    float   swiglu_alpha;        /* 1.702 for GPT-OSS                                           */
    float   swiglu_limit;        /* 7.0 for GPT-OSS                                             */
    float   router_eps;          /* RMSNorm epsilon of the GEMMA router (1e-6)                  */
} hh_moe_desc;

/* Device pointers to the layer's weights. */
typedef struct hh_moe_weights {
    const void *experts;             /* E expert blobs, reference blob layout for desc->quant  */
    size_t      expert_stride;       /* bytes between blobs; 0 = the reference stride (16 KiB aligned) */
    const void *shared_expert;       /* one blob of shared_intermediate, same format, or NULL   */
    const uint16_t *router_weight;   /* bf16 [E][H] (NULL with an MLX router, below)            */
    const uint16_t *router_bias;     /* bf16 [E] or NULL (GPT-OSS router bias)                  */
    const uint16_t *router_scale;    /* bf16 [H], GEMMA router only                             */
    const uint16_t *router_expert_scale; /* bf16 [E], GEMMA router only                         */
    const uint16_t *shared_gate;     /* bf16 [H]: the shared expert's sigmoid gate row          */
    /* MLX-affine router (Qwen's published builds quantise mlp.gate and
     * mlp.shared_expert_gate to 8 bits: Qwen35MoeConfig.swift:340-342; applied by
     * QwenMixtureBlock.encodeRouterAndShared, QwenMixtureBlock.swift:153-177). router_bits 0:
     * the bf16 router_weight / shared_gate above are used. 4 or 8: router_words uint32
     * [E][H·bits/32], router_scales / router_biases bf16 [E][H/64] (group 64) replace
     * router_weight, and, for a shared expert, shared_gate_words/scales/biases ([1][H] in the
     * same format) replace shared_gate. Logits are exact: every weight q·s + b and every
     * product with the bf16 input is formed exactly in fp64 (Gemma4ReferenceOps.swift:210-239),
     * so top-k indices equal the fp64 reference's. Not with the GEMMA router; the router input
     * must be x (x_router NULL or equal to x) when a shared expert is present.               */
    int32_t         router_bits;
    const uint32_t *router_words;
    const uint16_t *router_scales;
    const uint16_t *router_biases;
    const uint32_t *shared_gate_words;
    const uint16_t *shared_gate_scales;
    const uint16_t *shared_gate_biases;
} hh_moe_weights;

/* Byte layout of one expert blob (offsets from the blob start). Slots in consumption order:
 *   MXFP4: gate_up blocks, gate_up scales, gate_up bias, down blocks, down scales, down bias
 *   BF16 : gate_up, down
 *   MLX  : gate words, gate scales, gate biases, up words/scales/biases, down words/scales/biases */
typedef struct hh_blob_layout {
    int32_t slot_count;
    size_t  offset[9];
    size_t  bytes[9];
    size_t  payload_bytes;   /* end of the last slot                                            */
    size_t  stride_bytes;    /* payload rounded up to 16 KiB                                     */
} hh_blob_layout;

typedef struct hh_ctx hh_ctx;

/* ---- context ----------------------------------------------------------------------------- */
/* Replaces MetalContext (Sources/HydraMetal/MetalContext.swift:44-70): binds device `device`
 * and creates one default-priority stream owned by the context.                              */
int hh_ctx_create(hh_ctx **out, int32_t device);
int hh_ctx_destroy(hh_ctx *ctx);
/* The context's stream as a hipStream_t (opaque here). */
void *hh_ctx_stream(hh_ctx *ctx);
/* Waits for every enqueued call; the analogue of MetalContext.wait (MetalContext.swift:191-202),
 * which reports a failed command buffer instead of returning silent zeros.                   */
int hh_ctx_synchronize(hh_ctx *ctx);
/* Pre-sizes the scratch arena for up to max_tokens tokens of layers shaped like `desc`, so
 * that later hh_moe_forward calls within that bound allocate nothing (the reference's
 * preallocated scratch, LayerRunner.swift:6-10).                                             */
int hh_ctx_reserve(hh_ctx *ctx, const hh_moe_desc *desc, int32_t max_tokens);
/* Kernel launches issued through this context since creation (the DispatchCounter analogue,
 * ForwardEncoder.swift:34-68).                                                               */
int64_t hh_dispatch_count(const hh_ctx *ctx);
const char *hh_last_error(void);
/* Per-phase GPU timing with HIP events recorded on the context's stream around each kernel of
 * hh_moe_forward (phase 0 route, 1 gate-up product, 2 down product, 3 combine): the
 * reference's GPU start/end timing (Qwen35MoeRunner.swift:281) per pass. Off by default.
 * hh_ctx_profile_read synchronises the stream, returns the summed milliseconds of each phase
 * and the number of profiled forward calls, and clears the record.                           */
int hh_ctx_profile(hh_ctx *ctx, int32_t enable);
int hh_ctx_profile_read(hh_ctx *ctx, double *phase_ms /* [4] */, int64_t *calls);
/* The launch structure of MXFP4 decode calls (at most 16 tokens), with the same results bit
 * for bit in every mode; hh_moe_block_forward follows it too. 0: three launches (router,
 * gate-up, down). 2: two launches, the router as the first workgroups of the gate-up launch
 * (1 or 2 tokens, bf16 non-GEMMA routers, H <= 4096, E <= 128; other calls, calls under capture
 * and the allocation-free entry take three); the profile then records the routing phase as
 * empty. 1: one launch (router, gate-up and down roles; no shared
 * expert, top_k <= 4, E <= 128), whose profile records the whole layer as phase 0. -1: the
 * default, the environment variable HH_DECODE_FUSED (0, 1 or 2) or else 2. No counterpart in
 * the reference: a scheduling choice of this implementation.                               */
int hh_ctx_decode_fused(hh_ctx *ctx, int32_t enable);

/* ---- description helpers ------------------------------------------------------------------ */
/* Validates a description; HH_OK or the code hh_moe_forward would return for it.             */
int hh_desc_check(const hh_moe_desc *desc);
/* Blob layout for an expert of `intermediate` rows under desc's format (pass desc->intermediate
 * for routed experts, desc->shared_intermediate for the shared one).                          */
int hh_expert_blob_layout(const hh_moe_desc *desc, int32_t intermediate, hh_blob_layout *out);

/* ---- the layer ----------------------------------------------------------------------------- */
/* One MoE layer over T tokens, entirely on device with no host synchronisation:
 * router logits → top-k weights → dispatch/permutation → gate-up product + activation →
 * down product → rank-ordered weighted combine (+ sigmoid-gated shared expert).
 *
 * Replaces, as one call, LayerRunner.encodeAttentionAndRouter's router half, selectedExperts,
 * encodeSingleExpert ×K and encodeCombineSlices (LayerRunner.swift:130-301) for decode, and
 * PrefillRunner.encodeExpert (PrefillRunner.swift:252-302), QwenMixtureBlock
 * .encodeRouterAndShared/encodeExperts/encodeCombine (QwenMixtureBlock.swift:122-263) and
 * Gemma4LayerRunner.encodeSingleExpert/encodeExpertGroup (Gemma4LayerRunner.swift:579-677)
 * for the other families. Semantics follow ReferenceLayer.swift:189-204,
 * QwenReferenceLayer.swift:387-405 and Gemma4ReferenceLayer.swift:188-204.
 *
 *   x        bf16 [T][H]   the expert (and, unless x_router is given, router) input
 *   x_router bf16 [T][H]   router input, or NULL for x (Gemma routes on the residual)
 *   y        fp32 [T][H]   the mixture's contribution; the caller adds the residual
 *   topk_idx int32 [T][K]  selected experts in rank order, or NULL
 *   topk_w   fp32 [T][K]   their weights, or NULL
 *
 * A token's result does not depend on T or on the other tokens in the call: a T-token call
 * equals T one-token calls bit for bit.                                                      */
int hh_moe_forward(hh_ctx *ctx, const hh_moe_desc *desc, const hh_moe_weights *w,
                   const uint16_t *x, const uint16_t *x_router, int32_t tokens,
                   float *y, int32_t *topk_idx, float *topk_w);

/* The whole FFN block around the MoE layer, on the fp32 residual stream `hidden` [T][H]
 * (updated in place), with the RMSNorms and residual adds fused around hh_moe_forward's
 * kernels. Two structures, chosen by norms->post_expert_norm:
 *
 *   pre-norm (post_expert_norm NULL; GPT-OSS, Qwen):
 *       x = bf16(rmsnorm(hidden, pre_norm));  hidden += moe(x)
 *     ReferenceLayer.decode (ReferenceLayer.swift:189-202), QwenLayerRunner
 *     (QwenLayerRunner.swift:11-14); the GPU sequence rmsNorm → router → experts → addInPlace
 *     of LayerRunner.swift:202-216 and :279-301. rmsnorm(v, w) = v·(mean v² + eps)^-½·w
 *     (ReferenceOps.swift:20-25). The residual add is done by the layer's last kernel.
 *   Gemma's parallel branches (post_expert_norm set; dense_out, post_dense_norm, post_norm
 *   required): the expert branch reads x = bf16(rmsnorm(hidden, pre_norm)) (the
 *   pre_feedforward_layernorm_2), the GEMMA router reads bf16(hidden) (the residual), and
 *       hidden = (hidden + rmsnorm(rmsnorm(dense_out, post_dense_norm)
 *                                  + rmsnorm(moe(x), post_expert_norm), post_norm)) · scalar
 *     Gemma4ReferenceLayer.forward (Gemma4ReferenceLayer.swift:175-214),
 *     Gemma4LayerRunner.encodeCombineBranches (Gemma4LayerRunner.swift:683-723). dense_out is
 *     the dense MLP's output before its post-norm (post_feedforward_layernorm_1).
 *
 * Norms and sums are computed in fp64 and x is rounded once to bf16 (the layer's input format,
 * as for hh_moe_forward). H ≤ 8192. Norm weights are bf16 [H]; layer_scalar bf16 [1] or NULL
 * (1). The pow form (mean + eps)^-½ of Gemma4ReferenceOps.swift:28 is used for the GEMMA
 * router's layers, 1/√(mean + eps) otherwise.                                                */
typedef struct hh_block_norms {
    const uint16_t *pre_norm;          /* the expert input's RMSNorm weight (required)          */
    const uint16_t *post_expert_norm;  /* Gemma post_feedforward_layernorm_2, or NULL          */
    const uint16_t *post_dense_norm;   /* Gemma post_feedforward_layernorm_1                   */
    const uint16_t *post_norm;         /* Gemma post_feedforward_layernorm                     */
    const uint16_t *layer_scalar;      /* Gemma layer_scalar (bf16 [1]) or NULL                */
    float eps;                         /* the model's rms_norm_eps                             */
} hh_block_norms;
int hh_moe_block_forward(hh_ctx *ctx, const hh_moe_desc *desc, const hh_moe_weights *w,
                         const hh_block_norms *norms, float *hidden, const float *dense_out,
                         int32_t tokens, int32_t *topk_idx, float *topk_w);

/* Allocation-free variant of hh_moe_forward, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has
 * no counterpart in the reference; this entry needs no reservation at all. Same arguments, results
 * bit for bit equal to hh_moe_forward's. Its scratch is a fixed array of
 * HH_NOALLOC_SCRATCH_BYTES in each device's memory, held from library load until the process
 * ends, instead of the context's arena; the call makes no hipMalloc/hipFree, never takes the
 * one-launch decode and records no profiling events. A call whose scratch plan exceeds the
 * array returns HH_ENOMEM before enqueuing anything (decode of every family fits; prefill fits
 * while T·(K+shared)·H·4 bytes of slot outputs and the routing tables stay under the limit,
 * e.g. up to a few hundred tokens of a GPT-OSS layer). Every call on a device shares that
 * device's array, so calls that overlap on one device (from two contexts or streams) race:
 * serialise them on one stream. The array keeps the last call's contents; no kernel reads
 * scratch it has not written in the same call, so nothing needs clearing between calls.    */
#define HH_NOALLOC_SCRATCH_BYTES (16u << 20)
int hh_moe_forward_noalloc(hh_ctx *ctx, const hh_moe_desc *desc, const hh_moe_weights *w,
                           const uint16_t *x, const uint16_t *x_router, int32_t tokens,
                           float *y, int32_t *topk_idx, float *topk_w);

/* Decode attention with per-head sinks over an fp16 key/value history (the step before the
 * router in every layer): ForwardEncoder.attention (ForwardEncoder.swift:1107-1160) with
 * attention_decode_split/attention_decode_merge (attention.metal:307-450); semantics of
 * ReferenceLayer.decode (ReferenceLayer.swift:150-180).
 *   q        fp32 [q_heads][head_dim]
 *   k_cache, v_cache  fp16 bits [rows][kv_heads][head_dim]; key position p is row p % ring_size
 *            (ring_size 0: row p); keys start_position .. start_position + key_count - 1
 *   sinks    bf16 [q_heads], in the softmax denominator only
 *   out      fp32 [q_heads][head_dim]
 * head_dim 64 or 128, q_heads = kv_heads × 1..8 (HH_ESHAPE otherwise). Refused (HH_EINVAL)
 * while the context captures a graph: key_count and start_position change every decode step,
 * and a graph would replay the recorded values.                                             */
int hh_attention_decode(hh_ctx *ctx, const float *q, const uint16_t *k_cache,
                        const uint16_t *v_cache, const uint16_t *sinks, int32_t q_heads,
                        int32_t kv_heads, int32_t head_dim, int32_t key_count, int32_t ring_size,
                        int32_t start_position, float sm_scale, float *out);

/* A layer stack as one HIP graph (the per-layer-stack graphs a HIP-backed
 * ModelRunner.forward / TextModelRunner would replay in place of encoding every layer's passes
 * per token, ModelRunner.swift:110-230): between hh_ctx_capture_begin and hh_ctx_capture_end
 * the context's hh_moe_forward calls are recorded, not run, with the buffers they were given;
 * hh_graph_launch replays them on the context's stream. The scratch arena must already cover
 * every recorded call (hh_ctx_reserve; a call that would grow it fails), profiling must be off,
 * and while recording the context accepts no call that synchronises (hh_ctx_synchronize,
 * hh_scatter_expert_tensor); the one-launch decode (hh_ctx_decode_fused) is not used for
 * recorded calls. A graph's calls share the context's arena, so replays of graphs of one
 * context are ordered by its stream, like eager calls.                                      */
typedef struct hh_graph hh_graph;
int hh_ctx_capture_begin(hh_ctx *ctx);
int hh_ctx_capture_end(hh_ctx *ctx, hh_graph **out);
int hh_graph_launch(hh_graph *graph);
int hh_graph_destroy(hh_graph *graph);

/* The MoE halves of a whole model behind a HIP-backed ModelRunner (ModelRunner.forward /
 * prefill, ModelRunner.swift:110-230, 418-547; QwenLayerRunner.swift:11-14): per layer the
 * caller's token mixer (attention), enqueued by `hook` on the context's stream, then the
 * layer's FFN block (hh_moe_block_forward) — router, experts and residual on the device with no
 * host synchronisation between layers (the reference waits for a router readback before it can
 * fetch each layer's experts, ModelRunner.swift:164-170). hh_runner_capture records the whole
 * stack, hooks included, as one HIP graph for a fixed token count (the hooks must only enqueue
 * work on the stream they are given). Layers are set once with their description, weights,
 * norms and, for Gemma's parallel branches, the buffer the hook fills with the dense MLP's
 * output. hh_runner_reserve sizes the context's scratch for every layer up to max_tokens
 * (required before capture).                                                                 */
typedef struct hh_runner hh_runner;
typedef int (*hh_layer_hook)(void *user, int32_t layer, void *stream);
int hh_runner_create(hh_ctx *ctx, int32_t layers, hh_runner **out);
int hh_runner_destroy(hh_runner *runner);
int hh_runner_set_layer(hh_runner *runner, int32_t layer, const hh_moe_desc *desc,
                        const hh_moe_weights *w, const hh_block_norms *norms,
                        const float *dense_out);
int hh_runner_reserve(hh_runner *runner, int32_t max_tokens);
int hh_runner_forward(hh_runner *runner, float *hidden, int32_t tokens, hh_layer_hook hook,
                      void *user);
int hh_runner_capture(hh_runner *runner, float *hidden, int32_t tokens, hh_layer_hook hook,
                      void *user, hh_graph **out);

/* Checkpoint expert tensors straight into HBM: copies one stacked checkpoint tensor, the E
 * experts' copies of blob slot `slot` back to back (E × bytes[slot] bytes, e.g. GPT-OSS's
 * model.layers.L.mlp.experts.gate_up_proj_blocks [E][2I][H/32][16]), into the E blobs at
 * `blobs`: blob e's bytes offset[slot] .. + bytes[slot] (offsets and sizes of
 * hh_expert_blob_layout(desc, intermediate)) = src[e·bytes[slot] ..]. One strided copy on the
 * context's stream, complete when the call returns; `src` may be host or device memory. Replaces the installer's expert ScatterCopy operations (RepackPlan.swift:198-230,
 * GemmaRepackPlan.swift:137-155, QwenRepackPlan.swift:97-126), writing the blob layout the
 * kernels read in place of a .hydra file. HH_ESHAPE if src_bytes ≠ experts × bytes[slot].    */
int hh_scatter_expert_tensor(hh_ctx *ctx, const hh_moe_desc *desc, int32_t intermediate,
                             int32_t slot, int32_t experts, const void *src, int64_t src_bytes,
                             void *blobs, uint64_t expert_stride);

/* ---- operator-level entry points (parity tests mirror the encoder passes) ----------------- */
/* MXFP4 → fp32 (MXFP4.swift:67-99; GPU mxfp4_dequantize, mxfp4.metal:25). `blocks` is
 * nblocks×16 bytes, `scales` nblocks bytes, `out` nblocks×32 floats. Uses the same decode
 * the expert products use.                                                                    */
int hh_mxfp4_dequant(hh_ctx *ctx, const uint8_t *blocks, const uint8_t *scales,
                     int64_t nblocks, float *out);
/* MLX affine → fp32, value = fma(q, scale, bias) (Gemma4ReferenceOps.swift:196-221).
 * words uint32 [rows][cols/(32/bits)], scales/biases bf16 [rows][cols/group].               */
int hh_mlx_dequant(hh_ctx *ctx, const uint32_t *words, const uint16_t *scales,
                   const uint16_t *biases, int32_t rows, int32_t cols, int32_t bits,
                   int32_t group_size, float *out);
/* Router only: logits → top-k → weights, per desc->router, with top-k indices equal to those
 * of fp64 logits. Replaces routerTopK / routerTopKBatched / gemmaRouterTopK(Batched)
 * (ForwardEncoder.swift:1183-1200, 1283-1323). logits (fp64 [T][K], the selected experts'
 * logits in rank order), and shared_w (fp32 [T], the shared expert's sigmoid gate) may be
 * NULL. SOFTMAX_TOPK_RENORM and GEMMA rank by fp64 probability as the reference does: experts
 * whose exp(logit − max) is 0 tie and are taken by increasing index (weight 0, logit −inf in
 * `logits`), QwenReferenceOps.swift:164-173, Gemma4ReferenceOps.swift:146-149.               */
int hh_router_topk(hh_ctx *ctx, const hh_moe_desc *desc, const hh_moe_weights *w,
                   const uint16_t *x_router, int32_t tokens, double *logits,
                   int32_t *topk_idx, float *topk_w, float *shared_w);
/* Gated activation on fp32 pairs (swiglu/qwen_silu_multiply/gelu_mul, attention.metal:81,
 * qwen.metal:279, gemma.metal:77): out[i] = act(gate[i], up[i]) with the same device
 * function the fused gate-up epilogue uses.                                                   */
int hh_activation(hh_ctx *ctx, const hh_moe_desc *desc, const float *gate, const float *up,
                  int64_t n, float *out);
/* Token→expert permutation (PrefillRunner.assignments, PrefillRunner.swift:224-246, done on
 * device): for topk_idx [T][K], writes seg_offsets int32 [E+1] and order int32 [T·K], the
 * assignment ids t·K+r grouped by expert in ascending expert order, stable in (t, r).       */
int hh_permute(hh_ctx *ctx, const int32_t *topk_idx, int32_t tokens, int32_t top_k,
               int32_t experts, int32_t *seg_offsets, int32_t *order);

/* One weight matrix in an expert format, for the projection entries below. All pointers are
 * device memory; rows and cols are multiples of 64.
 *   MXFP4: weights = blocks [rows][cols/32][16] (low nibble = even column), scales = e8m0 bytes
 *          [rows][cols/32], bias = bf16 [rows] or NULL (MXFP4.swift:67-99)
 *   BF16 : weights = bf16 [rows][cols]
 *   MLX4/MLX8: weights = words [rows][cols·bits/32] (low-order value first), scales and biases
 *          bf16 [rows][cols/group_size] (MLXAffineLayout.swift:22-66), group_size 64           */
/* A weight matrix for the operator-level projections. Every pointer (weights, scales, biases,
 * bias) must be 16-byte aligned (HH_EALIGN otherwise), as the tensors of a blob are.          */
typedef struct hh_matrix {
    int32_t quant;            /* hh_quant                                                       */
    int32_t rows, cols;
    int32_t group_size;       /* MLX: 64                                                        */
    const void *weights;
    const void *scales;       /* MXFP4 / MLX; NULL for BF16                                     */
    const uint16_t *biases;   /* MLX group biases; NULL otherwise                               */
    const uint16_t *bias;     /* MXFP4: per-row bf16 bias added to y, or NULL                   */
} hh_matrix;

/* y = W·x (+ bias) for one fp32 input vector x [cols] → y fp32 [rows]: the operator-level
 * expert projection of ForwardEncoder.expertProjection (ForwardEncoder.swift:947-972, MXFP4
 * with bias), mlxAffineProjection (:328-365) and encodeProjection(.bf16) (:300-313), run on
 * the layer's own down-product kernels (the input in the layer's activation operand: MXFP4 as
 * three fp8 terms per 32-column block, ~2^-13 relative; BF16/MLX as a bf16 hi + lo pair).   */
int hh_expert_gemv(hh_ctx *ctx, const hh_matrix *m, const float *x, float *y);
/* The same for `tokens` input rows x [tokens][cols] → y [tokens][rows] (BatchEncoder
 * .expertProjection, BatchEncoder.swift:147-173; mlxAffineBatchedProjection,
 * ForwardEncoder.swift:456-487): the layer's decode down kernel up to 16 tokens, its prefill
 * kernels above. Row t equals hh_expert_gemv of x[t] bit for bit.                           */
int hh_expert_gemm(hh_ctx *ctx, const hh_matrix *m, const float *x, int32_t tokens, float *y);
/* Weighted combine in rank order: y[t][j] = Σ_{r<count} weights[t][r]·slots[t][r][j], each
 * product rounded to fp32 and the sum taken from r = 0 (write_expert_scaled then
 * sum_expert_slices, dense.metal:131-158, as LayerRunner.encodeCombineSlices,
 * LayerRunner.swift:279-301, encodes them). slots fp32 [tokens][count][size]; weights fp32
 * [tokens][count], or NULL for a plain sum of the slots.                                     */
int hh_combine(hh_ctx *ctx, const float *slots, const float *weights, int32_t tokens,
               int32_t count, int32_t size, float *y);

#ifdef __cplusplus
}
#endif
#endif /* HYDRA_HIP_H */
