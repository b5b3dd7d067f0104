/*
 * hh_oracle.c — fp64 CPU restatement of Hydra's HydraReference MoE path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the timed CPU baseline.
 * The product never links or loads this file.
 *
 * Every function follows a reference routine, cited file:line relative to the Hydra
 * repository root. It is written as plain loops, in the same order as the reference, so that
 * a divergence reads as a GPU bug and not as an ambiguity here.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   hho_mxfp4_decode          committed golden vector (64 blocks, all 256 bytes) + known answers
 *   hho_bf16_*                exhaustive 2^16 round trip + RNE closed form
 *   hho_mlx_unpack/dequant    known answers of the reference tests; numpy dequant-then-dot
 *   hho_swiglu                reference fixture reference_ops.json["swiglu"] + clamp traps
 *   hho_gelu_tanh             reference fixture gemma4_operators.json["gelu_tanh"]
 *   hho_silu / hho_sigmoid    closed form (math.exp), special points
 *   hho_router_topk_softmax   reference fixture reference_ops.json["router"]
 *   hho_router_softmax_topk_renorm  identity with topk_softmax (QwenMixtureTests.swift:34-65)
 *                                   + brute force over permutations on tiny E
 *   hho_router_gemma          reference fixture gemma4_operators.json["router"] and ["layer"]
 *   hho_expert_ffn / hho_moe_forward  numpy dense formulation (dequantise whole matrices,
 *                             matmul) on tiny shapes for every format; Gemma MoE branch inside
 *                             the reference's full-layer fixture gemma4_operators.json["layer"]
 *   hho_blob_layout           the reference's own byte counts (MXFP4Tests.swift:106-119) and
 *                             closed-form alignment rules
 *   hho_attention_decode      reference fixtures reference_ops.json["sdpa_full"],
 *                             ["sdpa_sliding"] (every query row as one decode step), a sink of
 *                             -inf against plain softmax attention, one key = its value row
 */
#include "hh_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- BF16 (Sources/HydraFormat/BF16.swift:20-33) ------------------------------------------ */

float hho_bf16_to_f32(uint16_t bits) {
    /* BF16.toFloat: the 16 bits become the top half of a Float32. */
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t hho_f32_to_bf16(float value) {
    /* BF16.fromFloat: NaN quieted by setting bit 6, else round to nearest even. */
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if (value != value) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t rounding = 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + rounding) >> 16);
}

void hho_bf16_to_f32_array(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = hho_bf16_to_f32(in[i]);
}

void hho_f32_to_bf16_array(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = hho_f32_to_bf16(in[i]);
}

static double bf(uint16_t b) { return (double)hho_bf16_to_f32(b); }

/* ---- MXFP4 (Sources/HydraFormat/MXFP4.swift:29-42, 67-99) ---------------------------------- */

static const float kE2M1[16] = {
    +0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f, +4.0f, +6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

void hho_mxfp4_decode(const uint8_t *packed, const uint8_t *scales, size_t nblocks, float *out) {
    for (size_t b = 0; b < nblocks; ++b) {
        /* scaleFactor: exp2(Float(Int(scale) - 127)), in float (MXFP4.swift:37-42). */
        float factor = exp2f((float)((int)scales[b] - 127));
        for (int i = 0; i < 16; ++i) {
            uint8_t byte = packed[b * 16 + i];
            /* Low nibble → even index, high nibble → odd index (MXFP4.swift:91-96). */
            out[b * 32 + 2 * i] = kE2M1[byte & 0x0F] * factor;
            out[b * 32 + 2 * i + 1] = kE2M1[byte >> 4] * factor;
        }
    }
}

/* ---- MLX affine (Sources/HydraReference/Gemma4ReferenceOps.swift:196-240) ------------------- */

void hho_mlx_unpack(const uint32_t *words, size_t nwords, int bits, int32_t *out) {
    /* MLXAffine.unpack: the first value occupies the least significant bits (:196-207). */
    int per_word = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    for (size_t w = 0; w < nwords; ++w)
        for (int s = 0; s < per_word; ++s)
            out[w * per_word + s] = (int32_t)((words[w] >> (s * bits)) & mask);
}

void hho_mlx_dequant(const uint32_t *words, const double *scales, const double *biases,
                     int cols, int bits, int group, double *out) {
    /* MLXAffine.dequantize: q · scale + bias, one scale and bias per group (:210-221). */
    int per_word = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    for (int i = 0; i < cols; ++i) {
        uint32_t q = (words[i / per_word] >> ((i % per_word) * bits)) & mask;
        int g = i / group;
        out[i] = (double)q * scales[g] + biases[g];
    }
}

/* ---- activations ------------------------------------------------------------------------- */

double hho_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); } /* QwenReferenceOps.swift:34 */
double hho_silu(double x) { return x * hho_sigmoid(x); }         /* QwenReferenceOps.swift:36 */

double hho_gelu_tanh(double x) {
    /* Gemma4ReferenceOps.gelu (:37-40). */
    double inner = sqrt(2.0 / M_PI) * (x + 0.044715 * x * x * x);
    return 0.5 * x * (1.0 + tanh(inner));
}

void hho_swiglu(const double *row, int pairs, double alpha, double limit, double *out) {
    /* ReferenceOps.swiglu (:87-99): even = gate, odd = linear; the gate is clamped from above
     * only, the linear branch on both sides and gets +1; swish is x·σ(alpha·x). */
    for (int i = 0; i < pairs; ++i) {
        double gate = fmin(row[2 * i], limit);
        double linear = fmin(fmax(row[2 * i + 1], -limit), limit);
        double activated = gate * (1.0 / (1.0 + exp(-alpha * gate)));
        out[i] = activated * (linear + 1.0);
    }
}

static double act_pair(const hho_desc *d, double gate, double up) {
    switch (d->activation) {
    case 0: {
        double row[2] = {gate, up}, out;
        hho_swiglu(row, 1, d->swiglu_alpha, d->swiglu_limit, &out);
        return out;
    }
    case 1: return hho_silu(gate) * up;       /* QwenReferenceOps.siluMultiply (:149-152) */
    default: return hho_gelu_tanh(gate) * up; /* Gemma4ReferenceOps.mlp (:43-45) */
    }
}

/* ---- routers -------------------------------------------------------------------------------- */

/* Descending by value, ties to the smaller index: the order the reference's sorts produce. */
static void order_desc(const double *v, int n, int k, int32_t *idx) {
    /* A selection of the k best with an explicit (value desc, index asc) order; equal to the
     * prefix of `indices.sorted { v[a] == v[b] ? a < b : v[a] > v[b] }`. */
    char *taken = (char *)calloc((size_t)n, 1);
    for (int r = 0; r < k; ++r) {
        int best = -1;
        for (int e = 0; e < n; ++e) {
            if (taken[e]) continue;
            if (best < 0 || v[e] > v[best]) best = e; /* strict: the smaller index stays */
        }
        idx[r] = best;
        taken[best] = 1;
    }
    free(taken);
}

void hho_router_topk_softmax(const double *logits, int experts, int k, int32_t *idx, double *w) {
    /* ReferenceOps.router (:173-183): top-k first, softmax over the k selected logits. */
    order_desc(logits, experts, k, idx);
    double peak = -INFINITY;
    for (int r = 0; r < k; ++r) peak = fmax(peak, logits[idx[r]]);
    double total = 0.0;
    for (int r = 0; r < k; ++r) { w[r] = exp(logits[idx[r]] - peak); total += w[r]; }
    for (int r = 0; r < k; ++r) w[r] /= total;
}

static void softmax(const double *v, int n, double *out) {
    /* Gemma4ReferenceOps.softmax (:113-118) and the first half of QwenReferenceOps.router. */
    double peak = -INFINITY;
    for (int i = 0; i < n; ++i) peak = fmax(peak, v[i]);
    double total = 0.0;
    for (int i = 0; i < n; ++i) { out[i] = exp(v[i] - peak); total += out[i]; }
    for (int i = 0; i < n; ++i) out[i] /= total;
}

void hho_router_softmax_topk_renorm(const double *logits, int experts, int k, int32_t *idx,
                                    double *w) {
    /* QwenReferenceOps.router (:159-179): softmax over every expert, iterative arg-max with a
     * strict `>` over the probabilities, then renormalise the selected ones. */
    double *p = (double *)malloc(sizeof(double) * (size_t)experts);
    softmax(logits, experts, p);
    order_desc(p, experts, k, idx);
    double sum = 0.0;
    for (int r = 0; r < k; ++r) sum += p[idx[r]];
    for (int r = 0; r < k; ++r) w[r] = p[idx[r]] / sum;
    free(p);
}

void hho_router_gemma(const double *hidden, int h, const double *projection, const double *scale,
                      const double *per_expert_scale, int experts, int k, double eps,
                      int32_t *idx, double *w) {
    /* Gemma4ReferenceOps.router (:131-156) with rmsNorm(weight: nil) (:25-31). */
    double sum = 0.0;
    for (int i = 0; i < h; ++i) sum += hidden[i] * hidden[i];
    double s = pow(sum / (double)h + eps, -0.5);
    double root = pow((double)h, -0.5);
    double *scaled = (double *)malloc(sizeof(double) * (size_t)h);
    for (int i = 0; i < h; ++i) scaled[i] = hidden[i] * s * scale[i] * root;
    double *logits = (double *)malloc(sizeof(double) * (size_t)experts);
    for (int e = 0; e < experts; ++e) {
        double dot = 0.0;
        for (int i = 0; i < h; ++i) dot += scaled[i] * projection[(size_t)e * h + i];
        logits[e] = dot;
    }
    double *p = (double *)malloc(sizeof(double) * (size_t)experts);
    softmax(logits, experts, p);
    order_desc(p, experts, k, idx);
    double total = 0.0;
    for (int r = 0; r < k; ++r) total += p[idx[r]];
    for (int r = 0; r < k; ++r) w[r] = p[idx[r]] / total * per_expert_scale[idx[r]];
    free(scaled); free(logits); free(p);
}

/* ---- blob layouts (Sources/HydraCore/ExpertBlobLayout.swift) -------------------------------- */

static size_t align_up(size_t v, size_t a) { size_t r = v % a; return r ? v + (a - r) : v; }

int hho_blob_layout(const hho_desc *d, int inter, size_t offset[9], size_t bytes[9],
                    size_t *payload, size_t *stride) {
    size_t H = (size_t)d->hidden, I = (size_t)inter;
    size_t sizes[9];
    int n;
    if (d->quant == 0) {
        /* ExpertBlobLayout.init (:78-103): gate_up blocks/scales/bias, down blocks/scales/bias. */
        n = 6;
        sizes[0] = 2 * I * (H / 32) * 16; sizes[1] = 2 * I * (H / 32); sizes[2] = 2 * I * 2;
        sizes[3] = H * (I / 32) * 16;     sizes[4] = H * (I / 32);     sizes[5] = H * 2;
    } else if (d->quant == HHO_QUANT_F64) {
        /* Test-only fp64 matrices, gate [I][H], up [I][H], down [H][I], for the reference's
         * fp64 fixtures (not a reference format). */
        n = 3;
        sizes[0] = I * H * 8; sizes[1] = I * H * 8; sizes[2] = H * I * 8;
    } else if (d->quant == 3) {
        /* GemmaExpertBlobLayout.init (:127-143): fused gate_up [2I][H] bf16, down [H][I]. */
        n = 2;
        sizes[0] = 2 * I * H * 2; sizes[1] = H * I * 2;
    } else {
        /* MLXExpertBlobLayout.init (:193-223) with MLXAffineLayout byte counts
         * (Sources/HydraCore/MLXAffineLayout.swift:51-54). */
        int bits = d->quant == 1 ? 4 : 8;
        size_t vpw = (size_t)(32 / bits), g = (size_t)d->group_size;
        n = 9;
        size_t gw = I * (H / vpw) * 4, gs = I * (H / g) * 2;
        size_t dw = H * (I / vpw) * 4, ds = H * (I / g) * 2;
        sizes[0] = gw; sizes[1] = gs; sizes[2] = gs;
        sizes[3] = gw; sizes[4] = gs; sizes[5] = gs;
        sizes[6] = dw; sizes[7] = ds; sizes[8] = ds;
    }
    size_t cursor = 0;
    for (int i = 0; i < n; ++i) {
        cursor = align_up(cursor, 256); /* tensorAlignment (:48) */
        offset[i] = cursor;
        bytes[i] = sizes[i];
        cursor += sizes[i];
    }
    *payload = cursor;
    *stride = align_up(cursor, 16384); /* pageAlignment (:38) */
    return n;
}

/* ---- matrices inside a blob ---------------------------------------------------------------- */

typedef struct {
    int quant, rows, cols, group;
    const uint8_t *w;     /* MXFP4 blocks / bf16 / MLX words */
    const uint8_t *s;     /* MXFP4 scales / MLX bf16 scales */
    const uint8_t *b;     /* MLX bf16 biases */
} matref;

static void decode_row(const matref *m, int row, double *out, float *ftmp) {
    int cols = m->cols;
    if (m->quant == 0) {
        size_t nb = (size_t)cols / 32;
        hho_mxfp4_decode(m->w + (size_t)row * nb * 16, m->s + (size_t)row * nb, nb, ftmp);
        for (int i = 0; i < cols; ++i) out[i] = (double)ftmp[i];
    } else if (m->quant == 3) {
        const uint16_t *r = (const uint16_t *)m->w + (size_t)row * cols;
        for (int i = 0; i < cols; ++i) out[i] = bf(r[i]);
    } else if (m->quant == HHO_QUANT_F64) {
        memcpy(out, (const double *)m->w + (size_t)row * cols, sizeof(double) * (size_t)cols);
    } else {
        int bits = m->quant == 1 ? 4 : 8;
        int vpw = 32 / bits, ng = cols / m->group;
        const uint32_t *words = (const uint32_t *)m->w + (size_t)row * (cols / vpw);
        const uint16_t *sc = (const uint16_t *)m->s + (size_t)row * ng;
        const uint16_t *bi = (const uint16_t *)m->b + (size_t)row * ng;
        double sd[1024], bd[1024]; /* ng ≤ 1024 is checked by the caller's shapes */
        for (int g = 0; g < ng; ++g) { sd[g] = bf(sc[g]); bd[g] = bf(bi[g]); }
        hho_mlx_dequant(words, sd, bd, cols, bits, m->group, out);
    }
}

/* y[r] = Σ_i W[r][i]·x[i] (+ bias[r]) for r in [r0, r0+nrows) with row stride `rstep`
 * (ReferenceLayer.matVec, ReferenceLayer.swift:288-297: sum in column order, bias last). */
static void matvec(const matref *m, const double *x, const uint16_t *bias, int r0, int rstep,
                   int nrows, double *y, int nthreads) {
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) if (nthreads > 1)
#endif
    {
        double *row = (double *)malloc(sizeof(double) * (size_t)m->cols);
        float *ftmp = (float *)malloc(sizeof(float) * (size_t)m->cols);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int j = 0; j < nrows; ++j) {
            int r = r0 + j * rstep;
            decode_row(m, r, row, ftmp);
            double sum = 0.0;
            for (int i = 0; i < m->cols; ++i) sum += row[i] * x[i];
            y[j] = bias ? sum + bf(bias[r]) : sum;
        }
        free(row);
        free(ftmp);
    }
    (void)nthreads;
}

static void expert_ffn_threads(const hho_desc *d, const uint8_t *blob, int I, const double *x,
                               double *out, int nthreads) {
    size_t off[9], by[9], payload, stride;
    hho_blob_layout(d, I, off, by, &payload, &stride);
    int H = d->hidden;
    double *gate = (double *)malloc(sizeof(double) * (size_t)I);
    double *up = (double *)malloc(sizeof(double) * (size_t)I);
    double *act = (double *)malloc(sizeof(double) * (size_t)I);
    matref gu, dn;
    const uint16_t *gu_bias = NULL, *dn_bias = NULL;
    if (d->quant == 0) {
        gu = (matref){0, 2 * I, H, 32, blob + off[0], blob + off[1], NULL};
        dn = (matref){0, H, I, 32, blob + off[3], blob + off[4], NULL};
        if (d->expert_bias) {
            gu_bias = (const uint16_t *)(blob + off[2]);
            dn_bias = (const uint16_t *)(blob + off[5]);
        }
        /* Interleaved rows [gate0, up0, gate1, ...] (ReferenceLayer.swift:195-196). */
        matvec(&gu, x, gu_bias, 0, 2, I, gate, nthreads);
        matvec(&gu, x, gu_bias, 1, 2, I, up, nthreads);
    } else if (d->quant == HHO_QUANT_F64) {
        matref g = {HHO_QUANT_F64, I, H, 0, blob + off[0], NULL, NULL};
        matref u = {HHO_QUANT_F64, I, H, 0, blob + off[1], NULL, NULL};
        dn = (matref){HHO_QUANT_F64, H, I, 0, blob + off[2], NULL, NULL};
        matvec(&g, x, NULL, 0, 1, I, gate, nthreads);
        matvec(&u, x, NULL, 0, 1, I, up, nthreads);
    } else if (d->quant == 3) {
        gu = (matref){3, 2 * I, H, 0, blob + off[0], NULL, NULL};
        dn = (matref){3, H, I, 0, blob + off[1], NULL, NULL};
        /* Halves: gate = rows 0..I-1, up = rows I..2I-1 (Gemma4Weights.swift:107-112). */
        matvec(&gu, x, NULL, 0, 1, I, gate, nthreads);
        matvec(&gu, x, NULL, I, 1, I, up, nthreads);
    } else {
        matref g = {d->quant, I, H, d->group_size, blob + off[0], blob + off[1], blob + off[2]};
        matref u = {d->quant, I, H, d->group_size, blob + off[3], blob + off[4], blob + off[5]};
        dn = (matref){d->quant, H, I, d->group_size, blob + off[6], blob + off[7], blob + off[8]};
        matvec(&g, x, NULL, 0, 1, I, gate, nthreads);
        matvec(&u, x, NULL, 0, 1, I, up, nthreads);
    }
    for (int i = 0; i < I; ++i) act[i] = act_pair(d, gate[i], up[i]);
    matvec(&dn, act, dn_bias, 0, 1, H, out, nthreads);
    free(gate); free(up); free(act);
}

void hho_expert_ffn(const hho_desc *d, const uint8_t *blob, int I, const double *x, double *out) {
    expert_ffn_threads(d, blob, I, x, out, 1);
}

void hho_router_logits_f64(const hho_desc *d, const hho_weights_f64 *w, const double *x,
                           double *logits) {
    int H = d->hidden, E = d->experts;
    if (d->router == 2) {
        /* Gemma: the normalisation and both scales come before the projection (:135-144). */
        double sum = 0.0;
        for (int i = 0; i < H; ++i) sum += x[i] * x[i];
        double s = pow(sum / (double)H + d->router_eps, -0.5);
        double root = pow((double)H, -0.5);
        for (int e = 0; e < E; ++e) {
            double dot = 0.0;
            for (int i = 0; i < H; ++i)
                dot += x[i] * s * w->router_scale[i] * root * w->router_weight[(size_t)e * H + i];
            logits[e] = dot;
        }
        return;
    }
    /* ReferenceLayer.matVec (:288-297) / QwenReferenceMixture.project (:375-377). */
    for (int e = 0; e < E; ++e) {
        double sum = 0.0;
        for (int i = 0; i < H; ++i) sum += w->router_weight[(size_t)e * H + i] * x[i];
        logits[e] = w->router_bias ? sum + w->router_bias[e] : sum;
    }
}

int hho_moe_forward_f64(const hho_desc *d, const hho_weights_f64 *w, const double *x,
                        const double *x_router, int tokens, double *y, int32_t *idx,
                        double *wts, double *shared_w, int nthreads) {
    int H = d->hidden, E = d->experts, K = d->top_k;
    if (K < 1 || K > 8 || K > E) return -3;
    size_t off[9], by[9], payload, stride;
    hho_blob_layout(d, d->intermediate, off, by, &payload, &stride);
    size_t es = w->expert_stride ? w->expert_stride : stride;
    double *logits = (double *)malloc(sizeof(double) * (size_t)E);
    double *out = (double *)malloc(sizeof(double) * (size_t)H);
    for (int t = 0; t < tokens; ++t) {
        const double *xd = x + (size_t)t * H;
        const double *xr = x_router ? x_router + (size_t)t * H : xd;
        int32_t *ti = idx + (size_t)t * K;
        double *tw = wts + (size_t)t * K;
        if (d->router == 2) {
            hho_router_gemma(xr, H, w->router_weight, w->router_scale, w->router_expert_scale,
                             E, K, d->router_eps, ti, tw);
        } else {
            hho_router_logits_f64(d, w, xr, logits);
            if (d->router == 0) hho_router_topk_softmax(logits, E, K, ti, tw);
            else hho_router_softmax_topk_renorm(logits, E, K, ti, tw);
        }
        double *yt = y + (size_t)t * H;
        for (int i = 0; i < H; ++i) yt[i] = 0.0;
        /* Weighted sum in rank order (ReferenceLayer.swift:378-385,
         * QwenReferenceLayer.swift:391-397, Gemma4ReferenceLayer.swift:196-204). */
        for (int r = 0; r < K; ++r) {
            expert_ffn_threads(d, w->experts + (size_t)ti[r] * es, d->intermediate, xd, out,
                               nthreads);
            for (int i = 0; i < H; ++i) yt[i] += tw[r] * out[i];
        }
        if (d->shared_intermediate > 0 && w->shared_expert) {
            /* Shared expert gated by σ of its own row, applied to its output
             * (QwenReferenceLayer.swift:399-404). */
            double logit = 0.0;
            for (int i = 0; i < H; ++i) logit += w->shared_gate[i] * xd[i];
            double sc = hho_sigmoid(logit);
            if (shared_w) shared_w[t] = sc;
            expert_ffn_threads(d, w->shared_expert, d->shared_intermediate, xd, out, nthreads);
            for (int i = 0; i < H; ++i) yt[i] += sc * out[i];
        }
    }
    free(logits); free(out);
    return 0;
}

static double *widen(const uint16_t *b, size_t n) {
    if (!b) return NULL;
    double *o = (double *)malloc(sizeof(double) * n);
    for (size_t i = 0; i < n; ++i) o[i] = bf(b[i]);
    return o;
}

/* The router (rows = E) or shared gate (rows = 1) as fp64 [rows][H]: bf16 values widened, or an
 * MLX-affine matrix (group 64) dequantised row by row as QwenReferenceMixture receives it. */
static double *widen_router(const hho_weights *w, int shared_gate, size_t rows, size_t H) {
    const uint32_t *words = shared_gate ? w->shared_gate_words : w->router_words;
    const uint16_t *sc = shared_gate ? w->shared_gate_scales : w->router_scales;
    const uint16_t *bi = shared_gate ? w->shared_gate_biases : w->router_biases;
    if (!w->router_bits || !words) return widen(shared_gate ? w->shared_gate : w->router_weight, rows * H);
    const size_t wpr = H * (size_t)w->router_bits / 32, gpr = H / 64;
    double *o = (double *)malloc(sizeof(double) * rows * H);
    double *sd = (double *)malloc(sizeof(double) * gpr), *bd = (double *)malloc(sizeof(double) * gpr);
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < gpr; ++g) { sd[g] = bf(sc[r * gpr + g]); bd[g] = bf(bi[r * gpr + g]); }
        hho_mlx_dequant(words + r * wpr, sd, bd, (int)H, w->router_bits, 64, o + r * H);
    }
    free(sd); free(bd);
    return o;
}

int hho_moe_forward(const hho_desc *d, const hho_weights *w, const uint16_t *x,
                    const uint16_t *x_router, int tokens, double *y, int32_t *idx, double *wts,
                    double *shared_w, int nthreads) {
    size_t H = (size_t)d->hidden, E = (size_t)d->experts, T = (size_t)tokens;
    hho_weights_f64 w64 = {w->experts, w->expert_stride, w->shared_expert,
                           widen_router(w, 0, E, H), widen(w->router_bias, E),
                           widen(w->router_scale, H), widen(w->router_expert_scale, E),
                           widen_router(w, 1, 1, H)};
    double *xd = widen(x, T * H);
    double *xr = widen(x_router, T * H);
    int rc = hho_moe_forward_f64(d, &w64, xd, xr, tokens, y, idx, wts, shared_w, nthreads);
    free((void *)w64.router_weight); free((void *)w64.router_bias);
    free((void *)w64.router_scale); free((void *)w64.router_expert_scale);
    free((void *)w64.shared_gate); free(xd); free(xr);
    return rc;
}

void hho_router_logits(const hho_desc *d, const hho_weights *w, const double *x, double *logits) {
    size_t H = (size_t)d->hidden, E = (size_t)d->experts;
    hho_weights_f64 w64 = {w->experts, w->expert_stride, w->shared_expert,
                           widen_router(w, 0, E, H), widen(w->router_bias, E),
                           widen(w->router_scale, H), widen(w->router_expert_scale, E),
                           widen_router(w, 1, 1, H)};
    hho_router_logits_f64(d, &w64, x, logits);
    free((void *)w64.router_weight); free((void *)w64.router_bias);
    free((void *)w64.router_scale); free((void *)w64.router_expert_scale);
    free((void *)w64.shared_gate);
}

/* Decode attention over a key/value history with per-head sinks (ReferenceLayer.swift:150-180;
 * GPU attention_decode_split + attention_decode_merge, attention.metal:307-450). Keys
 * start_position .. start_position + key_count - 1 are visible; a key at position p lives in
 * cache row p % ring_size (ring_size 0: row p). Caches are [rows][kv_heads][head_dim], query and
 * out [q_heads][head_dim]; query head h reads kv head h / (q_heads / kv_heads). The sink enters
 * the softmax denominator only. */
void hho_attention_decode(const double *q, const double *k_cache, const double *v_cache,
                          const double *sinks, int q_heads, int kv_heads, int head_dim,
                          int key_count, int ring_size, int start_position, double sm_scale,
                          double *out) {
    const int q_mult = q_heads / kv_heads;
    double *logits = (double *)malloc(sizeof(double) * (size_t)(key_count > 0 ? key_count : 1));
    for (int h = 0; h < q_heads; ++h) {
        const int kvh = h / q_mult;
        const double sink = sinks[h];
        double peak = sink;
        for (int j = 0; j < key_count; ++j) {
            const long pos = (long)start_position + j;
            const long row = ring_size > 0 ? pos % ring_size : pos;
            const double *kr = k_cache + ((size_t)row * kv_heads + kvh) * head_dim;
            double dot = 0.0;
            for (int i = 0; i < head_dim; ++i) dot += q[(size_t)h * head_dim + i] * kr[i];
            logits[j] = dot * sm_scale;
            if (logits[j] > peak) peak = logits[j];
        }
        double den = exp(sink - peak);
        for (int j = 0; j < key_count; ++j) den += exp(logits[j] - peak);
        for (int i = 0; i < head_dim; ++i) out[(size_t)h * head_dim + i] = 0.0;
        for (int j = 0; j < key_count; ++j) {
            const long pos = (long)start_position + j;
            const long row = ring_size > 0 ? pos % ring_size : pos;
            const double *vr = v_cache + ((size_t)row * kv_heads + kvh) * head_dim;
            const double w = exp(logits[j] - peak) / den;
            for (int i = 0; i < head_dim; ++i) out[(size_t)h * head_dim + i] += w * vr[i];
        }
    }
    free(logits);
}
