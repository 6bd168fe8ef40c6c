/*
 * CPU oracle of the dense decoder step — TEST INFRASTRUCTURE ONLY.
 *
 * Restates qwn_decoder_forward / qwn_decoder_generate
 * (c/qwanto_decode.c:1566-2032, 2085-2125) for a dense Qwen2/Qwen3-style
 * model -- optional q/k/v/o projection biases (add_bias, :926-929, applied
 * at :1649-1651 and :1722) and per-head q/k RMSNorm (:1652-1655) -- with
 * `--kv-cache q8` and greedy sampling,
 * using the oracle's kernels for every matmul (qo_matmul_q4_0 /
 * qo_matmul_hvsq2 = qwn_matmul_*_f32, qo_matmul_f16 = the F16 path of
 * qwn_matmul_f32) and the Q8 KV cache (qo_q8_*).  The element-wise steps
 * follow the reference's AVX2 code paths operation for operation:
 *   rmsnorm      c/qwanto_decode.c:627-652 (n % 8 == 0: eight fma lanes)
 *   RoPE table   :601-625 (glibc powf/cosf/sinf), rotation :686-729 (fma)
 *   SwiGLU       :1946-1949, residual vec_add, greedy argmax :2043-2065
 * The embedding is F16 or BF16 (:561); the LM head is lm_head.weight when
 * present (F16, BF16, Q4_0 or HyperVSQ-2), else the embedding (:1074-1076).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "qwn_oracle.h"

struct qo_decoder {
    qo_model m;
    int threads;
    int position;
    uint32_t perturb;                  /* 0, or the seed of the rounding perturbation */
    uint32_t calls;                    /* matmul calls (perturbation stream) */
    float *x, *xb, *q, *k, *v, *ctx, *gate, *up, *hidden, *logits;
    float *rope_cos, *rope_sin;        /* [max_ctx][head_dim/2] */
    int8_t **kcache, **vcache;         /* per layer [max_ctx][kv_channels] */
    float **kscale, **vscale;          /* per layer [max_ctx][groups] */
};

void qo_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    if (n % 8 == 0) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < n; i += 8)
            for (int j = 0; j < 8; j++) acc[j] = fmaf(x[i + j], x[i + j], acc[j]);
        const float ss = acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
        const float inv = 1.0f / sqrtf((ss / (float)n) + eps);
        for (int i = 0; i < n; i++) out[i] = (x[i] * inv) * w[i];
        return;
    }
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float inv = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

void qo_rope_table(float *cos_t, float *sin_t, int max_ctx, int half, float theta) {
    for (int pos = 0; pos < max_ctx; pos++)
        for (int i = 0; i < half; i++) {
            const float angle = (float)pos * powf(theta, -2.0f * i / (2 * half));
            cos_t[(size_t)pos * half + i] = cosf(angle);
            sin_t[(size_t)pos * half + i] = sinf(angle);
        }
}

/* c/qwanto_decode.c:703-716: row[i] = a*c - b*s and row[i+half] = a*s + b*c
 * as fmsub/fmadd over a rounded product. */
void qo_rope_apply(float *v, int heads, int dim, const float *ct, const float *st) {
    const int half = dim / 2;
    for (int h = 0; h < heads; h++) {
        float *row = v + (size_t)h * dim;
        for (int i = 0; i < half; i++) {
            const float a = row[i], b = row[i + half];
            row[i] = fmaf(a, ct[i], -(b * st[i]));
            row[i + half] = fmaf(a, st[i], b * ct[i]);
        }
    }
}

int qo_argmax(const float *logits, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (logits[i] > logits[best]) best = i;
    return best;
}

/* add_bias (c/qwanto_decode.c:926-929): x[i] += b[i]; b may be NULL */
static void add_bias(float *x, const float *b, int n) {
    if (!b) return;
    for (int i = 0; i < n; i++) x[i] += b[i];
}

static const float *bias_of(const qo_decoder *d, int layer, int which) {
    return d->m.biases ? d->m.biases[4 * layer + which] : NULL;
}

/* Calibration only (qo_decoder_set_perturbation): rounding-sized changes
 * at every stage where a GPU step rounds differently, on a pseudo-random
 * half of each vector's elements.  Element-wise stages (the RMSNorm,
 * attention and SwiGLU outputs): one ulp of the element.  Sums (the
 * projection outputs and the logits): 2^-23 of the vector's largest
 * magnitude, the size of the differences another fp32 order of the same
 * exact integer dot products gives (the error of a sum scales with its
 * largest terms, not with the result).  Running the oracle with and
 * without it measures how far such differences -- and the int8 rounding
 * flips they cause -- travel through the layers. */
static uint32_t perturb_hash(const qo_decoder *d, uint32_t call, int i) {
    uint32_t h = d->perturb * 0x9E3779B1u ^ call * 0x85EBCA77u ^ (uint32_t)i * 0xC2B2AE3Du;
    h ^= h >> 15;
    h *= 0x2C1B3C6Du;
    h ^= h >> 12;
    return h;
}

static void perturb_outputs(qo_decoder *d, float *y, int n) {
    if (!d->perturb) return;
    const uint32_t call = d->calls++;
    for (int i = 0; i < n; i++) {
        const uint32_t h = perturb_hash(d, call, i);
        if (h & 1u) y[i] = nextafterf(y[i], (h & 2u) ? INFINITY : -INFINITY);
    }
}

static void perturb_sums(qo_decoder *d, float *y, int n) {
    if (!d->perturb) return;
    const uint32_t call = d->calls++;
    float m = 0.0f;
    for (int i = 0; i < n; i++) m = fmaxf(m, fabsf(y[i]));
    const float delta = ldexpf(m, -23);
    for (int i = 0; i < n; i++) {
        const uint32_t h = perturb_hash(d, call, i);
        if (h & 1u) y[i] += (h & 2u) ? delta : -delta;
    }
}

static int matmul(qo_decoder *d, const uint8_t *w, const float *x, int in, int out, float *y) {
    const int rc = d->m.cfg.proj_dtype == QO_PROJ_Q4_0 ? qo_matmul_q4_0(w, x, 1, in, out, y, d->threads)
                                                       : qo_matmul_hvsq2(w, x, 1, in, out, y, d->threads, -1);
    if (rc == 0) perturb_sums(d, y, out);
    return rc;
}

/* The LM head (c/qwanto_decode.c:2007): lm_head.weight when the model has
 * one, else the embedding (:1074-1076), through the matmul of its dtype
 * (qwn_matmul_f32, c/qwanto_kernels.c:1531-1616: Q4_0 and HyperVSQ-2
 * quantize the activation per call, F16 and BF16 decode rows). */
static int lm_head(qo_decoder *d, const float *x, float *logits) {
    const qo_model_config *c = &d->m.cfg;
    const void *w = d->m.lm_head ? d->m.lm_head : (const void *)d->m.embed;
    const int dt = d->m.lm_head ? d->m.lm_head_dtype : (d->m.embed_dtype ? d->m.embed_dtype : QO_DT_F16);
    switch (dt) {
    case QO_DT_F16: qo_matmul_f16((const uint16_t *)w, x, 1, c->hidden, c->vocab, logits, d->threads); return 0;
    case QO_DT_BF16: qo_matmul_bf16((const uint16_t *)w, x, 1, c->hidden, c->vocab, logits, d->threads); return 0;
    case QO_DT_Q4_0: return qo_matmul_q4_0((const uint8_t *)w, x, 1, c->hidden, c->vocab, logits, d->threads);
    case QO_DT_HVSQ2:
        return qo_matmul_hvsq2((const uint8_t *)w, x, 1, c->hidden, c->vocab, logits, d->threads, -1);
    default: return -1;
    }
}

void qo_decoder_set_perturbation(qo_decoder *d, uint32_t seed) {
    d->perturb = seed;
    d->calls = 0;
}

void qo_decoder_free(qo_decoder *d) {
    if (!d) return;
    const int L = d->m.cfg.layers;
    for (int l = 0; l < L; l++) {
        if (d->kcache) free(d->kcache[l]);
        if (d->vcache) free(d->vcache[l]);
        if (d->kscale) free(d->kscale[l]);
        if (d->vscale) free(d->vscale[l]);
    }
    free(d->kcache); free(d->vcache); free(d->kscale); free(d->vscale);
    free(d->x); free(d->xb); free(d->q); free(d->k); free(d->v); free(d->ctx);
    free(d->gate); free(d->up); free(d->hidden); free(d->logits);
    free(d->rope_cos); free(d->rope_sin);
    free(d);
}

qo_decoder *qo_decoder_create(const qo_model *m, int threads) {
    const qo_model_config *c = &m->cfg;
    if (c->head_dim % 2 || c->heads % c->kv_heads) return NULL;
    qo_decoder *d = (qo_decoder *)calloc(1, sizeof(*d));
    if (!d) return NULL;
    d->m = *m;
    d->threads = threads;
    const int D = c->hidden, Q = c->heads * c->head_dim, KV = c->kv_heads * c->head_dim;
    const int I = c->intermediate, groups = (KV + 63) / 64, half = c->head_dim / 2;
    d->x = malloc(D * 4); d->xb = malloc((D > Q ? D : Q) * 4);
    d->q = malloc(Q * 4); d->k = malloc(KV * 4); d->v = malloc(KV * 4); d->ctx = malloc(Q * 4);
    d->gate = malloc(I * 4); d->up = malloc(I * 4); d->hidden = malloc(I * 4);
    d->logits = malloc((size_t)c->vocab * 4);
    d->rope_cos = malloc((size_t)c->max_ctx * half * 4);
    d->rope_sin = malloc((size_t)c->max_ctx * half * 4);
    d->kcache = calloc(c->layers, sizeof(void *)); d->vcache = calloc(c->layers, sizeof(void *));
    d->kscale = calloc(c->layers, sizeof(void *)); d->vscale = calloc(c->layers, sizeof(void *));
    if (!d->x || !d->xb || !d->q || !d->k || !d->v || !d->ctx || !d->gate || !d->up || !d->hidden ||
        !d->logits || !d->rope_cos || !d->rope_sin || !d->kcache || !d->vcache || !d->kscale || !d->vscale) {
        qo_decoder_free(d);
        return NULL;
    }
    for (int l = 0; l < c->layers; l++) {
        d->kcache[l] = calloc((size_t)c->max_ctx * KV, 1);
        d->vcache[l] = calloc((size_t)c->max_ctx * KV, 1);
        d->kscale[l] = calloc((size_t)c->max_ctx * groups, 4);
        d->vscale[l] = calloc((size_t)c->max_ctx * groups, 4);
        if (!d->kcache[l] || !d->vcache[l] || !d->kscale[l] || !d->vscale[l]) {
            qo_decoder_free(d);
            return NULL;
        }
    }
    qo_rope_table(d->rope_cos, d->rope_sin, c->max_ctx, half, c->rope_theta);
    return d;
}

int qo_decoder_position(const qo_decoder *d) { return d->position; }

int qo_decoder_forward(qo_decoder *d, int token, float *logits_out) {
    const qo_model_config *c = &d->m.cfg;
    const int D = c->hidden, H = c->heads, HK = c->kv_heads, HD = c->head_dim;
    const int Q = H * HD, KV = HK * HD, I = c->intermediate, groups = (KV + 63) / 64;
    const int pos = d->position, half = HD / 2;
    if (token < 0 || token >= c->vocab || pos >= c->max_ctx) return -1;
    /* embedding row: F16 or BF16 (qwn_row_f32, c/qwanto_kernels.c:1508-1527) */
    const uint16_t *erow = d->m.embed + (size_t)token * D;
    if (d->m.embed_dtype == QO_DT_BF16)
        for (int i = 0; i < D; i++) d->x[i] = qo_bf16_to_float(erow[i]);
    else
        for (int i = 0; i < D; i++) d->x[i] = qo_half_to_float(erow[i]);
    const float *ct = d->rope_cos + (size_t)pos * half, *st = d->rope_sin + (size_t)pos * half;
    for (int l = 0; l < c->layers; l++) {
        const uint8_t *const *w = d->m.proj + (size_t)l * 7;
        qo_rmsnorm(d->xb, d->x, d->m.norms[2 * l], D, c->rms_eps);
        perturb_outputs(d, d->xb, D);
        if (matmul(d, w[0], d->xb, D, Q, d->q) || matmul(d, w[1], d->xb, D, KV, d->k) ||
            matmul(d, w[2], d->xb, D, KV, d->v))
            return -1;
        add_bias(d->q, bias_of(d, l, 0), Q);
        add_bias(d->k, bias_of(d, l, 1), KV);
        add_bias(d->v, bias_of(d, l, 2), KV);
        if (d->m.qk_norms) {
            /* head_rmsnorm (c/qwanto_decode.c:654-684, 1652-1655): per head, in place,
             * the same arithmetic as rmsnorm */
            for (int h = 0; h < H; h++)
                qo_rmsnorm(d->q + (size_t)h * HD, d->q + (size_t)h * HD, d->m.qk_norms[2 * l], HD, c->rms_eps);
            for (int h = 0; h < HK; h++)
                qo_rmsnorm(d->k + (size_t)h * HD, d->k + (size_t)h * HD, d->m.qk_norms[2 * l + 1], HD,
                           c->rms_eps);
        }
        qo_rope_apply(d->q, H, HD, ct, st);
        qo_rope_apply(d->k, HK, HD, ct, st);
        qo_q8_quantize_vector(d->k, d->kcache[l] + (size_t)pos * KV, d->kscale[l] + (size_t)pos * groups, KV);
        qo_q8_quantize_vector(d->v, d->vcache[l] + (size_t)pos * KV, d->vscale[l] + (size_t)pos * groups, KV);
        qo_q8_attention(d->q, d->kcache[l], d->vcache[l], d->kscale[l], d->vscale[l], H, HK, HD, pos,
                        1.0f / sqrtf((float)HD), d->ctx, d->threads);
        perturb_outputs(d, d->ctx, Q);
        if (matmul(d, w[3], d->ctx, Q, D, d->xb)) return -1;
        add_bias(d->xb, bias_of(d, l, 3), D);
        for (int i = 0; i < D; i++) d->x[i] += d->xb[i];
        qo_rmsnorm(d->xb, d->x, d->m.norms[2 * l + 1], D, c->rms_eps);
        perturb_outputs(d, d->xb, D);
        if (matmul(d, w[4], d->xb, D, I, d->gate) || matmul(d, w[5], d->xb, D, I, d->up)) return -1;
        for (int i = 0; i < I; i++) {
            const float g = d->gate[i];
            d->hidden[i] = (g / (1.0f + expf(-g))) * d->up[i];
        }
        perturb_outputs(d, d->hidden, I);
        if (matmul(d, w[6], d->hidden, I, D, d->xb)) return -1;
        for (int i = 0; i < D; i++) d->x[i] += d->xb[i];
    }
    qo_rmsnorm(d->xb, d->x, d->m.final_norm, D, c->rms_eps);
    perturb_outputs(d, d->xb, D);
    if (lm_head(d, d->xb, d->logits)) return -1;
    perturb_sums(d, d->logits, c->vocab);
    d->position++;
    if (logits_out) memcpy(logits_out, d->logits, (size_t)c->vocab * 4);
    return 0;
}

/* Greedy generation: forward the prompt, then max_new times pick the first
 * maximum of the logits and forward it.  tokens[s] is the s-th generated id,
 * margins[s] the gap between the best and second-best logit it was chosen
 * from (may be NULL). */
int qo_decoder_generate(qo_decoder *d, const int *prompt, int prompt_count, int max_new, int *tokens,
                        float *margins) {
    for (int i = 0; i < prompt_count; i++)
        if (qo_decoder_forward(d, prompt[i], NULL)) return -1;
    const int V = d->m.cfg.vocab;
    for (int s = 0; s < max_new; s++) {
        const int t = qo_argmax(d->logits, V);
        tokens[s] = t;
        if (margins) {
            float second = -INFINITY;
            for (int i = 0; i < V; i++)
                if (i != t && d->logits[i] > second) second = d->logits[i];
            margins[s] = d->logits[t] - second;
        }
        if (qo_decoder_forward(d, t, NULL)) return -1;
    }
    return max_new;
}
