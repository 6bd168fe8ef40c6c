/*
 * Plain-pointer wrappers around the reference CPU kernels — TEST
 * INFRASTRUCTURE ONLY.
 *
 * Compiled by oracle/Makefile together with the reference's own sources
 * (c/qwanto_kernels.c, c/qwanto_native.c, c/qwanto_turboquant.c, read in
 * place under /root/reference) into oracle/_ref/libqwn_ref.so.  The tests use
 * it to pin the oracle restatement bit for bit; nothing in the product or
 * on the GPU path loads it.  The reference entry points take a mapped model
 * and a tensor descriptor, so each wrapper describes a caller buffer as a
 * one-tensor model whose payload starts at offset 0.
 */
#include "qwanto_kernels.h"
#include "qwanto_native.h"
#include "qwanto_turboquant.h"

#include <stdlib.h>
#include <string.h>

static void describe(QwnModel *m, QwnTensorDesc *d, const void *data,
                     uint64_t bytes, uint32_t dtype, int K, int N) {
    memset(m, 0, sizeof(*m));
    memset(d, 0, sizeof(*d));
    m->base = (uint8_t *)data;
    m->file_size = (size_t)bytes;
    strcpy(d->name, "w");
    d->name_len = 1;
    d->dtype = dtype;
    d->n_dims = 2;
    d->shape[0] = (uint64_t)K;
    d->shape[1] = (uint64_t)N;
    d->numel = (uint64_t)K * (uint64_t)N;
    d->byte_offset = 0;
    d->byte_size = bytes;
}

static int run_matmul(uint32_t dtype, const void *w, uint64_t bytes,
                      const float *x, int M, int K, int N, float *y) {
    QwnModel m;
    QwnTensorDesc d;
    QwnScratch s;
    describe(&m, &d, w, bytes, dtype, K, N);
    if (qwn_scratch_init(&s, M, K) != 0) return -1;
    int rc = qwn_matmul_f32(&m, &d, x, M, K, N, &s, y);
    qwn_scratch_destroy(&s);
    return rc;
}

int ref_matmul_q4_0(const void *w, uint64_t bytes, const float *x, int M,
                    int K, int N, float *y) {
    return run_matmul(QWN_DT_Q4_0, w, bytes, x, M, K, N, y);
}

int ref_matmul_hvsq2(const void *w, uint64_t bytes, const float *x, int M,
                     int K, int N, float *y) {
    return run_matmul(QWN_DT_HYPER_VSQ2, w, bytes, x, M, K, N, y);
}

int ref_matmul_f16(const void *w, uint64_t bytes, const float *x, int M,
                   int K, int N, float *y) {
    return run_matmul(QWN_DT_F16, w, bytes, x, M, K, N, y);
}

int ref_matmul_bf16(const void *w, uint64_t bytes, const float *x, int M,
                    int K, int N, float *y) {
    return run_matmul(QWN_DT_BF16, w, bytes, x, M, K, N, y);
}

/* Quantize one token as the decoder does before a GPU call
 * (qwn_prepare_cuda_activation) and expose the block sums too. */
int ref_quantize_token(const float *x, int K, int8_t *q8_out,
                       float *scale_out, int32_t *sums_out) {
    QwnScratch s;
    if (qwn_scratch_init(&s, 1, K) != 0) return -1;
    const int8_t *q8 = NULL;
    float scale = 0.0f;
    int rc = qwn_prepare_cuda_activation(x, K, &s, &q8, &scale);
    if (rc == 0) {
        memcpy(q8_out, q8, (size_t)s.padded_k);
        *scale_out = scale;
        if (sums_out)
            memcpy(sums_out, s.activation_sums,
                   (size_t)s.activation_sum_blocks * sizeof(int32_t));
    }
    qwn_scratch_destroy(&s);
    return rc;
}

const char *ref_cpu_kernel_name(void) { return qwn_cpu_kernel_name(); }

/* Build a Q8 cache from `tokens` rows of fp32 K/V and run every query head
 * through qwn_q8_cache_attention_head with the decoder's GQA mapping
 * (c/qwanto_decode.c:1741-1754). Also returns the cache contents. */
int ref_q8_attention(const float *keys, const float *values, int tokens,
                     int kv_heads, int head_dim, const float *query,
                     int query_heads, int pos, float scale, float *out,
                     int8_t *k_q, int8_t *v_q, float *k_s, float *v_s) {
    QwnQ8Cache c;
    const int channels = kv_heads * head_dim;
    /* qwn_q8_quantize_vector zero-fills every 64-wide group to its end,
     * past n_channels when n_channels % 64 != 0 (c/qwanto_turboquant.c:584),
     * so the last token would write beyond the cache; 64 spare tokens give
     * that overrun room. */
    if (qwn_q8_cache_init(&c, tokens + 64, kv_heads, head_dim) != 0) return -1;
    for (int t = 0; t < tokens; t++)
        if (qwn_q8_cache_append(&c, keys + (size_t)t * channels,
                                values + (size_t)t * channels, channels) != 0) {
            qwn_q8_cache_free(&c);
            return -1;
        }
    float *scores = (float *)malloc((size_t)tokens * sizeof(float));
    if (!scores) {
        qwn_q8_cache_free(&c);
        return -1;
    }
    const float ratio = (float)query_heads / (float)kv_heads;
    for (int h = 0; h < query_heads; h++) {
        const int kh = (int)((float)h / ratio);
        qwn_q8_cache_attention_head(query + (size_t)h * head_dim, &c, kh, pos,
                                    scale, scores, out + (size_t)h * head_dim);
    }
    if (k_q) memcpy(k_q, c.packed_k, (size_t)tokens * c.token_stride);
    if (v_q) memcpy(v_q, c.packed_v, (size_t)tokens * c.token_stride);
    if (k_s) memcpy(k_s, c.scales_k, (size_t)tokens * c.scale_stride * sizeof(float));
    if (v_s) memcpy(v_s, c.scales_v, (size_t)tokens * c.scale_stride * sizeof(float));
    free(scores);
    qwn_q8_cache_free(&c);
    return 0;
}

/* The reference's placement plan (qwn_plan_residency,
 * c/qwanto_native.c:400-435) of a .qwn file: items[capacity] in plan order
 * and totals[3] (GPU, RAM, file-backed bytes); returns the tensor count, or
 * -1 when the file does not open or the plan fails. */
int qrh_plan_residency(const char *path, uint64_t gpu_budget, uint64_t ram_budget, QwnPlacement *items,
                       uint32_t capacity, uint64_t *totals) {
    QwnModel m;
    const char *err = NULL;
    if (qwn_open(path, &m, &err) != 0) return -1;
    QwnResidencyPlan plan;
    memset(&plan, 0, sizeof(plan));
    plan.items = items;
    plan.capacity = capacity;
    const int rc = qwn_plan_residency(&m, gpu_budget, ram_budget, &plan);
    totals[0] = plan.gpu_bytes;
    totals[1] = plan.ram_bytes;
    totals[2] = plan.nvme_bytes;
    qwn_close(&m);
    return rc == 0 ? (int)plan.count : -1;
}
