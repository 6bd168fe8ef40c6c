/*
 * A CPU-only stand-in for qwn_cuda.so -- TEST INFRASTRUCTURE ONLY.
 *
 * Exports the versioned qwn_cuda_abi_* set (include/qwn_cuda_abi.h) with no
 * device behind it, so the host decoder's loader (the reference's
 * qwn_cuda_load, c/qwanto_decode.c:267-462) can be driven through each of
 * its refusal branches on a machine without a GPU.  One compile-time switch
 * per branch (tests/test_loader_branches.py builds every variant):
 *
 *   FAKE_OMIT_GEMM        no qwn_cuda_abi_hypervsq2_gemm export (a legacy library)
 *   FAKE_ABI_VERSION=n    query() reports ABI version n
 *   FAKE_INFO_SIZE=n      query() reports struct_size n
 *   FAKE_BLOCK_BYTES=n    query() reports n-byte HyperVSQ-2 blocks
 *   FAKE_NO_Q8_CAP        no Q8 KV capability bit
 *   FAKE_OMIT_KV_RESET    no qwn_cuda_abi_kv_cache_reset export
 *   FAKE_CAPS_FAIL        get_capabilities() fails while query() succeeds
 *   FAKE_DEVICES=n        enumerate_devices() reports n devices
 *   FAKE_CONTEXT_FAIL     context_create() fails
 *   FAKE_NO_Q4_CAP        no Q4_0 capability bit (the build's extension)
 *   FAKE_GEMV_ZERO_COUNT  gemv returns OK without counting a matmul
 *   FAKE_COMPUTE          a working CPU library: uploads are copied, every
 *                         projection and Q8 KV call is computed by the
 *                         oracle (link with oracle/liboracle.so), so the host
 *                         decoder runs end to end without a device
 *
 * Without FAKE_COMPUTE every accepted call returns OK and does nothing else;
 * gemv refuses (UNSUPPORTED) unless FAKE_GEMV_ZERO_COUNT.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qwn_cuda_abi.h"
#ifdef FAKE_COMPUTE
#include "qwn_oracle.h"

typedef struct {
    uint8_t *data;
    uint32_t dtype, rows, cols;
} FakeTensor;

typedef struct {
    uint32_t max_tokens, channels, groups;
    int8_t *keys, *values;
    float *key_scales, *value_scales;
} FakeCache;
#endif

#ifndef FAKE_ABI_VERSION
#define FAKE_ABI_VERSION QWN_CUDA_ABI_VERSION
#endif
#ifndef FAKE_INFO_SIZE
#define FAKE_INFO_SIZE sizeof(QwnCudaAbiInfo)
#endif
#ifndef FAKE_BLOCK_BYTES
#define FAKE_BLOCK_BYTES QWN_CUDA_HYPERVSQ2_BLOCK_BYTES
#endif
#ifndef FAKE_DEVICES
#define FAKE_DEVICES 1
#endif

static char g_error[128] = "";
static QwnCudaTelemetry g_telemetry;
static int g_context_token;
#ifndef FAKE_COMPUTE
static int g_tensor_token, g_cache_token;
#endif

static void fill_info(QwnCudaAbiInfo *info, uint32_t version) {
    memset(info, 0, sizeof(*info));
    info->header.struct_size = (uint32_t)(FAKE_INFO_SIZE);
    info->header.abi_version = version;
    uint64_t caps = QWN_CUDA_CAP_HYPERVSQ2_GEMV | QWN_CUDA_CAP_HYPERVSQ2_GEMM | QWN_CUDA_CAP_RESIDENT_WEIGHTS |
                    QWN_CUDA_CAP_TELEMETRY | QWN_CUDA_CAP_DEVICE_ENUMERATION | QWN_CUDA_CAP_Q8_KV |
                    QWN_CUDA_CAP_Q4_0_GEMV | QWN_CUDA_CAP_F16_GEMV | QWN_CUDA_CAP_BF16_GEMV;
#ifdef FAKE_NO_Q8_CAP
    caps &= ~(uint64_t)QWN_CUDA_CAP_Q8_KV;
#endif
#ifdef FAKE_NO_Q4_CAP
    caps &= ~(uint64_t)QWN_CUDA_CAP_Q4_0_GEMV;
#endif
    info->capability_bits = caps;
    info->max_devices = 1;
    info->max_resident_tensors = 1024;
    info->hypervsq2_block_bytes = FAKE_BLOCK_BYTES;
    info->hypervsq2_block_elements = QWN_CUDA_HYPERVSQ2_BLOCK_ELEMENTS;
    snprintf(info->abi_name, sizeof(info->abi_name), "fake-cpu-abi");
}

QWN_CUDA_ABI_API int qwn_cuda_abi_query(QwnCudaAbiInfo *info) {
    if (!info) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    fill_info(info, FAKE_ABI_VERSION);
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_get_capabilities(QwnCudaAbiInfo *info) {
    if (!info) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
#ifdef FAKE_CAPS_FAIL
    snprintf(g_error, sizeof(g_error), "fake: capability query refused");
    return QWN_CUDA_STATUS_UNAVAILABLE;
#else
    fill_info(info, FAKE_ABI_VERSION);
    return QWN_CUDA_STATUS_OK;
#endif
}

QWN_CUDA_ABI_API int qwn_cuda_abi_enumerate_devices(QwnCudaDeviceInfo *devices, uint32_t capacity,
                                                     uint32_t *count) {
    if (!count) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    *count = FAKE_DEVICES;
    for (uint32_t i = 0; devices && i < capacity && i < (uint32_t)FAKE_DEVICES; i++) {
        memset(&devices[i], 0, sizeof(devices[i]));
        devices[i].header.struct_size = sizeof(devices[i]);
        devices[i].header.abi_version = QWN_CUDA_ABI_VERSION;
        devices[i].device_id = (int32_t)i;
        snprintf(devices[i].name, sizeof(devices[i].name), "fake device %u", i);
    }
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_context_create(const QwnCudaContextOptions *options,
                                                 QwnCudaContextHandle *context) {
    if (!options || !context) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
#ifdef FAKE_CONTEXT_FAIL
    snprintf(g_error, sizeof(g_error), "fake: no context on device %d", options->device_id);
    return QWN_CUDA_STATUS_UNAVAILABLE;
#else
    context->opaque = &g_context_token;
    memset(&g_telemetry, 0, sizeof(g_telemetry));
    g_telemetry.header.struct_size = sizeof(g_telemetry);
    g_telemetry.header.abi_version = QWN_CUDA_ABI_VERSION;
    return QWN_CUDA_STATUS_OK;
#endif
}

QWN_CUDA_ABI_API int qwn_cuda_abi_context_destroy(QwnCudaContextHandle *context) {
    if (context) context->opaque = NULL;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_upload_tensor(QwnCudaContextHandle *context, const QwnCudaTensorUpload *upload,
                                                QwnCudaTensorHandle *tensor) {
    if (!context || !upload || !tensor) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
#ifdef FAKE_COMPUTE
    FakeTensor *t = (FakeTensor *)calloc(1, sizeof(FakeTensor));
    if (!t || !(t->data = (uint8_t *)malloc(upload->data_bytes))) {
        free(t);
        return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    }
    memcpy(t->data, upload->host_data, upload->data_bytes);
    t->dtype = upload->dtype;
    t->rows = upload->rows;
    t->cols = upload->cols;
    tensor->opaque = t;
#else
    tensor->opaque = &g_tensor_token;
#endif
    g_telemetry.gpu_upload_count++;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_release_tensor(QwnCudaContextHandle *context, QwnCudaTensorHandle *tensor) {
    (void)context;
#ifdef FAKE_COMPUTE
    if (tensor && tensor->opaque) {
        free(((FakeTensor *)tensor->opaque)->data);
        free(tensor->opaque);
    }
#endif
    if (tensor) tensor->opaque = NULL;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_create(QwnCudaContextHandle *context, const QwnCudaKvCacheOptions *options,
                                                  QwnCudaKvCacheHandle *cache) {
    if (!context || !options || !cache) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
#ifdef FAKE_COMPUTE
    FakeCache *c = (FakeCache *)calloc(1, sizeof(FakeCache));
    if (!c) return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    c->max_tokens = options->max_tokens;
    c->channels = options->kv_heads * options->head_dim;
    c->groups = (c->channels + 63) / 64;
    const size_t n = (size_t)c->max_tokens * c->channels, g = (size_t)c->max_tokens * c->groups;
    c->keys = (int8_t *)calloc(n, 1);
    c->values = (int8_t *)calloc(n, 1);
    c->key_scales = (float *)calloc(g, sizeof(float));
    c->value_scales = (float *)calloc(g, sizeof(float));
    cache->opaque = c;
    if (!c->keys || !c->values || !c->key_scales || !c->value_scales) {
        qwn_cuda_abi_kv_cache_destroy(context, cache);
        return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    }
#else
    cache->opaque = &g_cache_token;
#endif
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_destroy(QwnCudaContextHandle *context, QwnCudaKvCacheHandle *cache) {
    (void)context;
#ifdef FAKE_COMPUTE
    if (cache && cache->opaque) {
        FakeCache *c = (FakeCache *)cache->opaque;
        free(c->keys);
        free(c->values);
        free(c->key_scales);
        free(c->value_scales);
        free(c);
    }
#endif
    if (cache) cache->opaque = NULL;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_append(QwnCudaContextHandle *context,
                                                  const QwnCudaKvAppendRequest *request,
                                                  QwnCudaTelemetry *telemetry) {
    (void)context;
#ifdef FAKE_COMPUTE
    if (!request || !request->cache.opaque) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    FakeCache *c = (FakeCache *)request->cache.opaque;
    if (request->token >= c->max_tokens || request->n_channels != c->channels) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    const size_t t = request->token;
    qo_q8_quantize_vector(request->host_key, c->keys + t * c->channels, c->key_scales + t * c->groups,
                          (int)c->channels);
    qo_q8_quantize_vector(request->host_value, c->values + t * c->channels, c->value_scales + t * c->groups,
                          (int)c->channels);
    g_telemetry.kv_cache_kernel_count++;
#else
    (void)request;
#endif
    if (telemetry) *telemetry = g_telemetry;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_attention(QwnCudaContextHandle *context,
                                                     const QwnCudaKvAttentionRequest *request,
                                                     QwnCudaTelemetry *telemetry) {
    (void)context;
#ifdef FAKE_COMPUTE
    if (!request || !request->cache.opaque) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    FakeCache *c = (FakeCache *)request->cache.opaque;
    if (request->position >= c->max_tokens || request->kv_heads * request->head_dim != c->channels)
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    qo_q8_attention_abi(request->host_query, c->keys, c->values, c->key_scales, c->value_scales,
                        (int)request->query_heads, (int)request->kv_heads, (int)request->head_dim,
                        (int)request->position, request->scale, request->host_output);
    g_telemetry.kv_cache_kernel_count++;
#else
    (void)request;
#endif
    if (telemetry) *telemetry = g_telemetry;
    return QWN_CUDA_STATUS_OK;
}

#ifndef FAKE_OMIT_KV_RESET
QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_reset(QwnCudaContextHandle *context, QwnCudaKvCacheHandle *cache) {
    (void)context;
    (void)cache;
    return QWN_CUDA_STATUS_OK;
}
#endif

#ifdef FAKE_COMPUTE
/* One token per request row, as the host decoder sends them: Q4_0 and
 * HyperVSQ-2 take int8 tokens with one scale, F16 and BF16 take fp32. */
static int fake_matmul(const QwnCudaGemmRequest *request, QwnCudaTelemetry *telemetry) {
    if (!request || !request->tensor.opaque || !request->input_q8 || !request->output)
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    const FakeTensor *t = (const FakeTensor *)request->tensor.opaque;
    const int K = (int)t->cols, N = (int)t->rows;
    if (request->rows != t->rows || request->cols != t->cols) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    for (uint32_t b = 0; b < request->batch; b++) {
        float *y = request->output + (size_t)b * request->output_stride;
        if (t->dtype == QWN_CUDA_TENSOR_F16 && request->input_mode == QWN_CUDA_INPUT_F32) {
            const float *x = (const float *)request->input_q8 + (size_t)b * request->input_stride;
            qo_matmul_f16((const uint16_t *)t->data, x, 1, K, N, y, 1);
        } else if (t->dtype == QWN_CUDA_TENSOR_BF16 && request->input_mode == QWN_CUDA_INPUT_F32) {
            const float *x = (const float *)request->input_q8 + (size_t)b * request->input_stride;
            qo_matmul_bf16((const uint16_t *)t->data, x, 1, K, N, y, 1);
        } else if (request->input_mode == QWN_CUDA_INPUT_Q8 && t->dtype == QWN_CUDA_TENSOR_Q4_0_18) {
            const int8_t *q = request->input_q8 + (size_t)b * request->input_stride;
            const float s = request->input_scales ? request->input_scales[b] : request->input_scale;
            qo_gemv_q4_0_q8(t->data, q, s, K, N, y, 1);
        } else if (request->input_mode == QWN_CUDA_INPUT_Q8 && t->dtype == QWN_CUDA_TENSOR_HYPERVSQ2_74) {
            const int padded = (K + 255) & ~255;
            int8_t *q = (int8_t *)calloc((size_t)padded, 1);
            int32_t *sums = (int32_t *)calloc((size_t)padded / 32, sizeof(int32_t));
            if (!q || !sums) {
                free(q);
                free(sums);
                return QWN_CUDA_STATUS_OUT_OF_MEMORY;
            }
            memcpy(q, request->input_q8 + (size_t)b * request->input_stride, (size_t)K);
            for (int i = 0; i < padded; i++) sums[i / 32] += q[i];
            const float s = request->input_scales ? request->input_scales[b] : request->input_scale;
            qo_gemv_hvsq2_delayed(t->data, q, sums, s, K, N, (size_t)(K + 255) / 256 * 74, y, 0);
            free(q);
            free(sums);
        } else {
            snprintf(g_error, sizeof(g_error), "fake: dtype %u with input mode %u", t->dtype, request->input_mode);
            return QWN_CUDA_STATUS_UNSUPPORTED;
        }
    }
    g_telemetry.gpu_matmul_count++;
    if (telemetry) *telemetry = g_telemetry;
    return QWN_CUDA_STATUS_OK;
}
#else
static int fake_matmul(const QwnCudaGemmRequest *request, QwnCudaTelemetry *telemetry) {
    (void)request;
#ifdef FAKE_GEMV_ZERO_COUNT
    if (telemetry) *telemetry = g_telemetry; /* OK, but no matmul counted */
    return QWN_CUDA_STATUS_OK;
#else
    if (telemetry) *telemetry = g_telemetry;
    snprintf(g_error, sizeof(g_error), "fake: no device to run a projection on");
    return QWN_CUDA_STATUS_UNSUPPORTED;
#endif
}
#endif

QWN_CUDA_ABI_API int qwn_cuda_abi_hypervsq2_gemv(QwnCudaContextHandle *context, const QwnCudaGemmRequest *request,
                                                 QwnCudaTelemetry *telemetry) {
    (void)context;
    return fake_matmul(request, telemetry);
}

#ifndef FAKE_OMIT_GEMM
QWN_CUDA_ABI_API int qwn_cuda_abi_hypervsq2_gemm(QwnCudaContextHandle *context, const QwnCudaGemmRequest *request,
                                                 QwnCudaTelemetry *telemetry) {
    (void)context;
    return fake_matmul(request, telemetry);
}
#endif

QWN_CUDA_ABI_API int qwn_cuda_abi_synchronize(QwnCudaContextHandle *context) {
    (void)context;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_get_telemetry(QwnCudaContextHandle *context, QwnCudaTelemetry *telemetry) {
    (void)context;
    if (telemetry) *telemetry = g_telemetry;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_cuda_abi_last_error(char *buffer, uint32_t buffer_size) {
    if (!buffer || buffer_size == 0) return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    snprintf(buffer, buffer_size, "%s", g_error);
    return QWN_CUDA_STATUS_OK;
}
