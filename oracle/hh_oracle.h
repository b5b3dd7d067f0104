/*
 * hh_oracle.h — fp64 CPU restatement of Hydra's HydraReference MoE path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (hydra_amd/, include/) links, loads or
 * calls this. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker / the timed CPU baseline.
 *
 * Enumerations use the numeric values of include/hydra_hip.h so a description can be handed
 * to both sides unchanged.
 */
#ifndef HH_ORACLE_H
#define HH_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hho_desc {
    int32_t hidden, intermediate, experts, top_k, shared_intermediate;
    int32_t quant;        /* 0 MXFP4, 1 MLX4, 2 MLX8, 3 BF16 */
    int32_t group_size;
    int32_t activation;   /* 0 SWIGLU_OAI, 1 SILU, 2 GELU_TANH */
    int32_t router;       /* 0 TOPK_SOFTMAX, 1 SOFTMAX_TOPK_RENORM, 2 GEMMA */
    int32_t expert_bias;
    double swiglu_alpha, swiglu_limit, router_eps;
} hho_desc;

/* Test-only format: fp64 gate [I][H], up [I][H], down [H][I] (for fp64 reference fixtures). */
#define HHO_QUANT_F64 100

typedef struct hho_weights {
    const uint8_t *experts; size_t expert_stride;
    const uint8_t *shared_expert;
    const uint16_t *router_weight, *router_bias, *router_scale, *router_expert_scale, *shared_gate;
    /* MLX-affine router (router_bits 4 or 8, group 64): replaces router_weight / shared_gate,
     * dequantised to fp64 q·scale + bias (Gemma4ReferenceOps.swift:210-221). */
    int32_t router_bits;
    const uint32_t *router_words; const uint16_t *router_scales, *router_biases;
    const uint32_t *shared_gate_words; const uint16_t *shared_gate_scales, *shared_gate_biases;
} hho_weights;

typedef struct hho_weights_f64 {
    const uint8_t *experts; size_t expert_stride;
    const uint8_t *shared_expert;
    const double *router_weight, *router_bias, *router_scale, *router_expert_scale, *shared_gate;
} hho_weights_f64;

float    hho_bf16_to_f32(uint16_t bits);
uint16_t hho_f32_to_bf16(float value);
void     hho_bf16_to_f32_array(const uint16_t *in, float *out, size_t n);
void     hho_f32_to_bf16_array(const float *in, uint16_t *out, size_t n);

void hho_mxfp4_decode(const uint8_t *packed, const uint8_t *scales, size_t nblocks, float *out);
void hho_mlx_unpack(const uint32_t *words, size_t nwords, int bits, int32_t *out);
void hho_mlx_dequant(const uint32_t *words, const double *scales, const double *biases,
                     int cols, int bits, int group, double *out);

void   hho_swiglu(const double *row, int pairs, double alpha, double limit, double *out);
double hho_silu(double x);
double hho_sigmoid(double x);
double hho_gelu_tanh(double x);

void hho_router_topk_softmax(const double *logits, int experts, int k, int32_t *idx, double *w);
void hho_router_softmax_topk_renorm(const double *logits, int experts, int k, int32_t *idx, double *w);
void hho_router_gemma(const double *hidden, int h, const double *projection /*[E][H]*/,
                      const double *scale, const double *per_expert_scale, int experts, int k,
                      double eps, int32_t *idx, double *w);

int  hho_blob_layout(const hho_desc *d, int intermediate, size_t offset[9], size_t bytes[9],
                     size_t *payload, size_t *stride);

/* One expert's feed-forward for one token: down(act(gate x, up x)) (+ biases for MXFP4 with
 * expert_bias). x double [H] → out double [H]. */
void hho_expert_ffn(const hho_desc *d, const uint8_t *blob, int intermediate, const double *x,
                    double *out);

/* The router logits of one token, fp64, for the GEMMA router after its normalisation. */
void hho_router_logits(const hho_desc *d, const hho_weights *w, const double *x, double *logits);

/* Whole layer. x bf16 [T][H]; x_router NULL or bf16 [T][H]; y double [T][H];
 * idx int32 [T][K]; wts double [T][K]; shared_w double [T] or NULL.
 * nthreads > 1 parallelises each matrix-vector product over rows (OpenMP). */
int hho_moe_forward_f64(const hho_desc *d, const hho_weights_f64 *w, const double *x,
                        const double *x_router, int tokens, double *y, int32_t *idx,
                        double *wts, double *shared_w, int nthreads);
void hho_router_logits_f64(const hho_desc *d, const hho_weights_f64 *w, const double *x,
                           double *logits);
int hho_moe_forward(const hho_desc *d, const hho_weights *w, const uint16_t *x,
                    const uint16_t *x_router, int tokens, double *y, int32_t *idx,
                    double *wts, double *shared_w, int nthreads);

#ifdef __cplusplus
}
#endif
void hho_attention_decode(const double *q, const double *k_cache, const double *v_cache,
                          const double *sinks, int q_heads, int kv_heads, int head_dim,
                          int key_count, int ring_size, int start_position, double sm_scale,
                          double *out);

#endif
