#ifndef QWN_ORACLE_H
#define QWN_ORACLE_H

/*
 * CPU oracle for the quantized decode path — TEST INFRASTRUCTURE ONLY.
 *
 * A C restatement of the reference's CPU kernels, used to check the qwn_hip
 * GPU library (tests/, __graft_entry__.smoke()) and as the timed CPU
 * baseline in bench.py.  Nothing in the product links or calls this code.
 *
 * Every function names the reference lines it follows.  How each one is
 * pinned (reference build, known-answer tests, closed forms) is listed in
 * tests/test_oracle_*.py.
 */

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Exact binary16 -> binary32, subnormals included
 * (c/qwanto_kernels.c:264-285). */
float qo_half_to_float(uint16_t h);

/* Per-token symmetric int8 activation quantization
 * (c/qwanto_kernels.c:354-433): scale = amax/127 (1 when amax == 0),
 * q = rint(clamp(x * (1/scale), -127, 127)), zero padding up to padded_k,
 * act_sums[t][b] = sum of q over 32-element block b (blocks past K sum 0).
 * act_sums may be NULL. */
void qo_quantize_tokens(const float *x, int M, int K, int padded_k,
                        int8_t *q8, float *scales, int32_t *act_sums,
                        int sum_blocks);

/* ---- Q4_0 ---------------------------------------------------------- */

/* Integer part of dot_q4_q8_block (c/qwanto_kernels.c:503-534):
 * sum over the block of (nibble - 8) * a. */
int32_t qo_q4_0_block_raw(const uint8_t *blk, const int8_t *q8, int valid);

/* y[n] = sum_b fma(float(raw_b) * d_b, x_scale, .) in block order, the
 * per-token inner loop of qwn_matmul_q4_0_f32 (c/qwanto_kernels.c:1271-1319).
 * q8 is one quantized token. Rows are parallel over `threads` OpenMP threads
 * (0 = library default). */
void qo_gemv_q4_0_q8(const uint8_t *w, const int8_t *q8, float x_scale,
                     int K, int N, float *y, int threads);

/* Full qwn_matmul_q4_0_f32 (c/qwanto_kernels.c:1178-1322): quantize each
 * token, then qo_gemv_q4_0_q8 per token. */
int qo_matmul_q4_0(const uint8_t *w, const float *x, int M, int K, int N,
                   float *y, int threads);

/* Per-block int32 raw sums [N][ceil(K/32)] for bit-exact checks. */
void qo_q4_0_block_sums(const uint8_t *w, const int8_t *q8, int K, int N,
                        int32_t *raw);

/* ---- HyperVSQ-2 ---------------------------------------------------- */

/* Scalar golden GEMV (c/qwanto_kernels.c:619-667). */
void qo_gemv_hvsq2_scalar(const uint8_t *w, const int8_t *q8,
                          const int32_t *act_sums, float x_scale, int K,
                          int N, size_t row_bytes, float *out);

/* Delayed-reduction GEMV, the reference's production CPU kernel
 * (c/qwanto_kernels.c:841-918): eight fp32 lanes per row, each fed by the
 * int32 sum of four adjacent products of every full octant, one offset
 * accumulator, one final horizontal sum.  Variant 0 = plain C restatement,
 * 1 = AVX2 (maddubs), 2 = AVX-VNNI (VEX dpbusd), 3 = AVX512-VNNI+VL (EVEX
 * dpbusd), -1 = best available.  All variants are bit-identical. */
void qo_gemv_hvsq2_delayed(const uint8_t *w, const int8_t *q8,
                           const int32_t *act_sums, float x_scale, int K,
                           int N, size_t row_bytes, float *out, int variant);

/* qwn_matmul_hypervsq2_f32 (c/qwanto_kernels.c:998-1176): quantize, then per
 * token an OpenMP loop over 64-row chunks of the delayed kernel
 * (variant as above; variant == -2 selects the scalar golden). */
int qo_matmul_hvsq2(const uint8_t *w, const float *x, int M, int K, int N,
                    float *y, int threads, int variant);

/* Per-octant int32 sums for bit-exact checks: sum_q[N][nb*8] =
 * sum (code-1)*a, sum_a[nb*8] = sum a (octants past K are 0). */
void qo_hvsq2_octant_sums(const uint8_t *w, const int8_t *q8, int K, int N,
                          int32_t *sum_q, int32_t *sum_a);

/* Best delayed variant this CPU runs (see qo_gemv_hvsq2_delayed). */
int qo_hvsq2_best_variant(void);
const char *qo_variant_name(int variant);

/* ---- F16 ----------------------------------------------------------- */

/* Generic F16 matmul of qwn_matmul_f32 (c/qwanto_kernels.c:1503-1527,
 * 1605-1614): decode a row to fp32, then sum += x[k]*row[k] in k order.
 * The reference runs it on one thread; `threads` > 1 splits rows only. */
void qo_matmul_f16(const uint16_t *w, const float *x, int M, int K, int N,
                   float *y, int threads);

/* Exact bfloat16 -> binary32: the 16 bits become the high half
 * (c/qwanto_kernels.c:287-290). */
float qo_bf16_to_float(uint16_t h);

/* The BF16 case of the same matmul: qwn_row_f32 decodes a BF16 row
 * (c/qwanto_kernels.c:1508-1527), then the same loop as F16
 * (:1605-1614). */
void qo_matmul_bf16(const uint16_t *w, const float *x, int M, int K, int N,
                    float *y, int threads);

/* ---- Q8 KV cache --------------------------------------------------- */

/* qwn_q8_quantize_vector (c/qwanto_turboquant.c:555-586): per 64-channel
 * group scale = amax(finite)/127 (1 when 0), q = lrintf(clamp(v/scale)),
 * non-finite -> 0. */
void qo_q8_quantize_vector(const float *src, int8_t *dst, float *scales,
                           int n_channels);

/* qwn_q8_cache_attention_head (c/qwanto_turboquant.c:648-702) over a
 * token-major cache: keys/values [tokens][n_channels] int8, scales
 * [tokens][ceil(n_channels/64)] fp32. scores needs pos+1 floats. */
void qo_q8_attention_head(const float *query, const int8_t *keys,
                          const int8_t *values, const float *key_scales,
                          const float *value_scales, int n_channels,
                          int head_dim, int kv_head, int pos, float scale,
                          float *scores, float *ctx);

/* All query heads with the decoder's GQA mapping kv = h / (H / HK)
 * (c/qwanto_decode.c:1742-1754); OpenMP over heads. */
void qo_q8_attention(const float *query, const int8_t *keys,
                     const int8_t *values, const float *key_scales,
                     const float *value_scales, int query_heads, int kv_heads,
                     int head_dim, int pos, float scale, float *out,
                     int threads);

/* The same over the GPU ABI's mapping kv = h * HK / H, any head ratio
 * (c/cuda/qwn_hypervsq2_cuda_abi.cu:184); one thread. */
void qo_q8_attention_abi(const float *query, const int8_t *keys,
                         const int8_t *values, const float *key_scales,
                         const float *value_scales, int query_heads, int kv_heads,
                         int head_dim, int pos, float scale, float *out);

/* ---- dense decoder (qwn_oracle_decoder.c) ------------------------------ */

#define QO_PROJ_HVSQ2 1
#define QO_PROJ_Q4_0 2

typedef struct {
    int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab, max_ctx;
    float rope_theta, rms_eps;
    int proj_dtype; /* QO_PROJ_* */
} qo_model_config;

/* dtypes of the embedding and of an untied LM head */
#define QO_DT_F16 1
#define QO_DT_BF16 4
#define QO_DT_Q4_0 2
#define QO_DT_HVSQ2 9

typedef struct {
    qo_model_config cfg;
    const uint16_t *embed;          /* [vocab][hidden], F16 or BF16 (embed_dtype); the LM head when
                                       lm_head is NULL (tied) */
    const float *final_norm;        /* [hidden] */
    const uint8_t *const *proj;     /* [layers * 7]: q k v o gate up down blocks */
    const float *const *norms;      /* [layers * 2]: input, post attention */
    const float *const *qk_norms;   /* NULL, or [layers * 2]: per-head q and k norm weights
                                       [head_dim] (Qwen3 self_attn.q_norm / k_norm) */
    const float *const *biases;     /* NULL, or [layers * 4]: q, k, v, o projection biases
                                       (self_attn.{q,k,v,o}_proj.bias), each NULL or
                                       [that projection's rows] */
    int embed_dtype;                /* QO_DT_F16 or QO_DT_BF16 (0 = F16) */
    const void *lm_head;            /* NULL (tied), or lm_head.weight [vocab][hidden] in lm_head_dtype
                                       (c/qwanto_decode.c:1074-1076) */
    int lm_head_dtype;              /* QO_DT_F16 / QO_DT_BF16 / QO_DT_Q4_0 / QO_DT_HVSQ2 */
} qo_model;

typedef struct qo_decoder qo_decoder;

/* rmsnorm (c/qwanto_decode.c:627-652). */
void qo_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
/* RoPE tables [max_ctx][half] (c/qwanto_decode.c:601-625). */
void qo_rope_table(float *cos_t, float *sin_t, int max_ctx, int half, float theta);
/* NeoX half-split rotation of `heads` rows (c/qwanto_decode.c:686-729). */
void qo_rope_apply(float *v, int heads, int dim, const float *ct, const float *st);
/* First index of the maximum (c/qwanto_decode.c:2043-2065). */
int qo_argmax(const float *logits, int n);

qo_decoder *qo_decoder_create(const qo_model *m, int threads);
void qo_decoder_free(qo_decoder *d);
int qo_decoder_position(const qo_decoder *d);
/* One forward step (c/qwanto_decode.c:1566-2032); logits_out may be NULL. */
int qo_decoder_forward(qo_decoder *d, int token, float *logits_out);
/* Calibration mode (seed 0 = off, the default): after every RMSNorm,
 * attention and SwiGLU a pseudo-random half of the outputs moves by one ulp,
 * after every projection and the LM head by 2^-23 of the largest output.
 * Not the reference's arithmetic: it measures how far rounding-sized
 * differences travel through the model's layers. */
void qo_decoder_set_perturbation(qo_decoder *d, uint32_t seed);
/* Greedy generate (c/qwanto_decode.c:2085-2125). */
int qo_decoder_generate(qo_decoder *d, const int *prompt, int prompt_count, int max_new, int *tokens,
                        float *margins);

#ifdef __cplusplus
}
#endif

#endif /* QWN_ORACLE_H */
