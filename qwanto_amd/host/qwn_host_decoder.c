/*
 * Host-side dense decoder over the qwn_cuda ABI (declared in
 * include/qwn_host_decoder.h).
 *
 * Follows the reference host step for step where its semantics are fixed:
 *   ABI bring-up            c/qwanto_decode.c:267-462
 *   matmul dispatch         c/qwanto_decode.c:776-924 (+ Q4_0 / F16 routing)
 *   activation quantize     c/qwanto_kernels.c:354-445 (host side, per call)
 *   rmsnorm                 c/qwanto_decode.c:627-652
 *   RoPE table / rotation   c/qwanto_decode.c:601-625, 686-729
 *   Q8 KV append/attention  c/qwanto_decode.c:1657-1724
 *   SwiGLU, residual        c/qwanto_decode.c:1946-1951
 *   forward / generate      c/qwanto_decode.c:1566-2032, 2085-2125
 * Arithmetic is written with explicit fused multiply-adds where the
 * reference's AVX2 paths fuse, and the file is compiled without
 * contraction, so the host-side values are the reference's bit for bit.
 */
#define _GNU_SOURCE
#include "qwn_host_decoder.h"

#include <dlfcn.h>
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "qwn_cuda_abi.h"

enum { PROJ_Q, PROJ_K, PROJ_V, PROJ_O, PROJ_GATE, PROJ_UP, PROJ_DOWN, PROJ_COUNT };

typedef struct {
    void *handle;
    QwnCudaAbiQueryFn query;
    QwnCudaCapabilityQueryFn get_capabilities;
    QwnCudaEnumerateDevicesFn enumerate_devices;
    QwnCudaContextCreateFn context_create;
    QwnCudaContextDestroyFn context_destroy;
    QwnCudaTensorUploadFn upload_tensor;
    QwnCudaTensorReleaseFn release_tensor;
    QwnCudaKvCreateFn kv_cache_create;
    QwnCudaKvDestroyFn kv_cache_destroy;
    QwnCudaKvAppendFn kv_cache_append;
    QwnCudaKvAttentionFn kv_cache_attention;
    QwnCudaKvResetFn kv_cache_reset;
    QwnCudaGemvFn gemv;
    QwnCudaGemmFn gemm;
    QwnCudaSynchronizeFn synchronize;
    QwnCudaTelemetryFn get_telemetry;
    QwnCudaLastErrorFn last_error;
    QwnCudaAbiInfo caps;
    QwnCudaContextHandle context;
} Abi;

typedef struct {
    const void *host;        /* host tensor this slot caches */
    QwnCudaTensorHandle tensor;
} Resident;

struct QhdDecoder {
    QhdModel m;
    Abi abi;
    int position;
    int padded_k;
    float *x, *xb, *q, *k, *v, *ctx, *gate, *up, *hidden, *logits;
    int8_t *q8;
    float *rope_cos, *rope_sin;
    Resident *resident;      /* lazily uploaded tensors, one per projection + LM head */
    int resident_count, resident_cap;
    QwnCudaKvCacheHandle *kv;
    QhdMetrics metrics;
    char error[256];
};

static void fail(QhdDecoder *d, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(d->error, sizeof(d->error), fmt, ap);
    va_end(ap);
    if (d->abi.last_error) {
        char buf[160];
        buf[0] = 0;
        d->abi.last_error(buf, sizeof(buf));
        if (buf[0]) {
            size_t n = strlen(d->error);
            snprintf(d->error + n, sizeof(d->error) - n, " (library: %s)", buf);
        }
    }
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + ts.tv_nsec * 1e-9;
}

static float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            exp = 127 - 15 + 1;
            while (!(mant & 0x400u)) {
                mant <<= 1;
                exp--;
            }
            bits = sign | (exp << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof(f));
    return f;
}

/* ---- ABI bring-up (c/qwanto_decode.c:267-462) ---------------------------- */

static void set_reason(QhdDecoder *d, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(d->metrics.backend_reason, sizeof(d->metrics.backend_reason), fmt, ap);
    va_end(ap);
}

/* A capability block the host accepts (c/qwanto_decode.c:365-370, 408-413). */
static int caps_ok(const QwnCudaAbiInfo *c) {
    return c->header.abi_version == QWN_CUDA_ABI_VERSION && c->header.struct_size >= sizeof(QwnCudaAbiInfo) &&
           (c->capability_bits & QWN_CUDA_CAP_HYPERVSQ2_GEMV) &&
           c->hypervsq2_block_bytes == QWN_CUDA_HYPERVSQ2_BLOCK_BYTES &&
           c->hypervsq2_block_elements == QWN_CUDA_HYPERVSQ2_BLOCK_ELEMENTS;
}

/* The reference loader's checks in its order, each refusal with its
 * reason string: library present; the twelve versioned exports; query()
 * (ABI version, struct size, HyperVSQ-2 74-byte layout); Q8 KV capability
 * and the five KV exports (this decoder always uses the Q8 cache, the
 * reference's --kv-cache q8); get_capabilities() with the same checks; the
 * device enumerated; context creation.  Then this decoder's own need: the
 * Q4_0 / F16 capabilities it routes through the ABI. */
static int load_abi(QhdDecoder *d, const char *path, int device) {
    char candidate[PATH_MAX];
    if (!path) {
        Dl_info info;
        memset(&info, 0, sizeof(info));
        if (!dladdr((void *)&load_abi, &info) || !info.dli_fname) {
            fail(d, "cannot locate the decoder library's directory");
            set_reason(d, "qwn_cuda_dll_absent_from_runtime_directory");
            return -1;
        }
        snprintf(candidate, sizeof(candidate), "%s", info.dli_fname);
        char *slash = strrchr(candidate, '/');
        if (slash) slash[1] = '\0';
        else candidate[0] = '\0';
        strncat(candidate, "qwn_cuda.so", sizeof(candidate) - strlen(candidate) - 1);
        char canonical[PATH_MAX];
        if (realpath(candidate, canonical)) snprintf(candidate, sizeof(candidate), "%s", canonical);
        path = candidate;
    }
    Abi *a = &d->abi;
    a->handle = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!a->handle) {
        fail(d, "cannot load %s: %s", path, dlerror());
        set_reason(d, "qwn_cuda_dll_absent_from_runtime_directory");
        return -1;
    }
#define RESOLVE(field, name) (*(void **)&a->field = dlsym(a->handle, name))
    RESOLVE(query, "qwn_cuda_abi_query");
    RESOLVE(get_capabilities, "qwn_cuda_abi_get_capabilities");
    RESOLVE(enumerate_devices, "qwn_cuda_abi_enumerate_devices");
    RESOLVE(context_create, "qwn_cuda_abi_context_create");
    RESOLVE(context_destroy, "qwn_cuda_abi_context_destroy");
    RESOLVE(upload_tensor, "qwn_cuda_abi_upload_tensor");
    RESOLVE(release_tensor, "qwn_cuda_abi_release_tensor");
    RESOLVE(kv_cache_create, "qwn_cuda_abi_kv_cache_create");
    RESOLVE(kv_cache_destroy, "qwn_cuda_abi_kv_cache_destroy");
    RESOLVE(kv_cache_append, "qwn_cuda_abi_kv_cache_append");
    RESOLVE(kv_cache_attention, "qwn_cuda_abi_kv_cache_attention");
    RESOLVE(kv_cache_reset, "qwn_cuda_abi_kv_cache_reset");
    RESOLVE(gemv, "qwn_cuda_abi_hypervsq2_gemv");
    RESOLVE(gemm, "qwn_cuda_abi_hypervsq2_gemm");
    RESOLVE(synchronize, "qwn_cuda_abi_synchronize");
    RESOLVE(get_telemetry, "qwn_cuda_abi_get_telemetry");
    RESOLVE(last_error, "qwn_cuda_abi_last_error");
#undef RESOLVE
    if (!a->query || !a->get_capabilities || !a->enumerate_devices || !a->context_create || !a->context_destroy ||
        !a->upload_tensor || !a->release_tensor || !a->gemv || !a->gemm || !a->synchronize || !a->get_telemetry ||
        !a->last_error) {
        a->last_error = NULL;
        fail(d, "%s lacks the versioned qwnrun ABI", path);
        set_reason(d, "qwn_cuda_dll_missing_versioned_abi_%u", QWN_CUDA_ABI_VERSION);
        return -1;
    }
    qwn_cuda_abi_header_init(&a->caps.header, sizeof(a->caps));
    if (a->query(&a->caps) != QWN_CUDA_STATUS_OK || !caps_ok(&a->caps)) {
        fail(d, "ABI or HyperVSQ-2 74-byte capability check failed");
        set_reason(d, "abi_capability_or_hypervsq2_layout_rejected");
        return -1;
    }
    if (!(a->caps.capability_bits & QWN_CUDA_CAP_Q8_KV) || !a->kv_cache_create || !a->kv_cache_destroy ||
        !a->kv_cache_append || !a->kv_cache_attention || !a->kv_cache_reset) {
        fail(d, "Q8 KV-cache capability is unavailable");
        set_reason(d, "cuda_q8_kv_capability_unavailable");
        return -1;
    }
    qwn_cuda_abi_header_init(&a->caps.header, sizeof(a->caps));
    if (a->get_capabilities(&a->caps) != QWN_CUDA_STATUS_OK || !caps_ok(&a->caps)) {
        fail(d, "capability query failed");
        set_reason(d, "cuda_capability_query_failed");
        return -1;
    }
    QwnCudaDeviceInfo devices[16];
    memset(devices, 0, sizeof(devices));
    uint32_t device_count = 0;
    if (a->enumerate_devices(devices, 16, &device_count) != QWN_CUDA_STATUS_OK || device_count == 0 ||
        device < 0 || (uint32_t)device >= device_count || device >= 16) {
        fail(d, "device %d is unavailable", device);
        set_reason(d, "cuda_device_index_%d_not_enumerated", device);
        return -1;
    }
    QwnCudaContextOptions opts;
    memset(&opts, 0, sizeof(opts));
    qwn_cuda_abi_header_init(&opts.header, sizeof(opts));
    opts.device_id = device;
    opts.context_size = (uint64_t)d->m.cfg.max_ctx;
    qwn_cuda_abi_header_init(&a->context.header, sizeof(a->context));
    if (a->context_create(&opts, &a->context) != QWN_CUDA_STATUS_OK) {
        a->context.opaque = NULL;
        fail(d, "context creation failed");
        set_reason(d, "cuda_context_creation_failed_device_%d", device);
        return -1;
    }
    const int head_dt = d->m.lm_head ? d->m.lm_head_dtype : (d->m.embed_dtype ? d->m.embed_dtype : QHD_DT_F16);
    const uint64_t need = (head_dt == QHD_DT_F16 ? QWN_CUDA_CAP_F16_GEMV : 0) |
                          (head_dt == QHD_DT_BF16 ? QWN_CUDA_CAP_BF16_GEMV : 0) |
                          (d->m.cfg.proj_dtype == QHD_PROJ_Q4_0 || head_dt == QHD_DT_Q4_0 ? QWN_CUDA_CAP_Q4_0_GEMV : 0);
    if ((a->caps.capability_bits & need) != need) {
        fail(d, "the ABI library lacks F16 / BF16 / Q4_0 support (capabilities 0x%llx)",
             (unsigned long long)a->caps.capability_bits);
        set_reason(d, "qwn_hip_q4_0_f16_capability_unavailable");
        return -1;
    }
    set_reason(d, "versioned_abi_%u_loaded_device_%d", QWN_CUDA_ABI_VERSION, device);
    return 0;
}

static void mirror_telemetry(QhdDecoder *d, const QwnCudaTelemetry *t) {
    QhdMetrics *m = &d->metrics;
    m->gpu_matmul_count = t->gpu_matmul_count;
    m->gpu_kernel_launch_count = t->gpu_kernel_launch_count;
    m->gpu_upload_bytes = t->gpu_upload_bytes;
    m->gpu_resident_bytes = t->gpu_resident_bytes;
    m->kv_cache_kernel_count = t->kv_cache_kernel_count;
    m->gpu_kernel_ms = t->gpu_kernel_ms;
    m->gpu_transfer_ms = t->gpu_transfer_ms;
    m->gpu_sync_ms = t->gpu_sync_ms;
    snprintf(m->kernel_type, sizeof(m->kernel_type), "%s", t->kernel_type);
}

/* ---- element-wise host steps ------------------------------------------------ */

/* c/qwanto_decode.c:627-652: eight fused lanes, left-to-right lane sum. */
static void rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
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

/* add_bias (c/qwanto_decode.c:926-929): x[i] += b[i]; b may be NULL */
static void add_bias(float *x, const float *b, int n) {
    if (!b) return;
    for (int i = 0; i < n; i++) x[i] += b[i];
}

static const float *bias_of(const QhdDecoder *d, int layer, int which) {
    return d->m.biases ? d->m.biases[4 * layer + which] : NULL;
}

static void rope(float *v, int heads, int dim, const float *ct, const float *st) {
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

/* c/qwanto_kernels.c:354-433 for one token: scale = amax/127 (1 if 0),
 * q = rint(clamp(x * (1/scale), +-127)), zero padding. */
static float quantize_activation(const float *x, int K, int padded, int8_t *q8) {
    float amax = 0.0f;
    for (int i = 0; i < K; i++) {
        const float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    for (int i = 0; i < K; i++) {
        float v = x[i] * inv;
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        q8[i] = (int8_t)lrintf(v);
    }
    memset(q8 + K, 0, (size_t)(padded - K));
    return scale;
}

/* ---- matmul dispatch (c/qwanto_decode.c:776-924) ------------------------------ */

static int resident_slot(QhdDecoder *d, const void *host, uint32_t dtype, uint32_t block_bytes, uint64_t bytes,
                         int out, int in) {
    for (int i = 0; i < d->resident_count; i++)
        if (d->resident[i].host == host) return i;
    if (d->resident_count == d->resident_cap) {
        fail(d, "resident tensor table full");
        return -1;
    }
    QwnCudaTensorUpload up;
    memset(&up, 0, sizeof(up));
    qwn_cuda_abi_header_init(&up.header, sizeof(up));
    up.host_data = host;
    up.data_bytes = bytes;
    up.dtype = dtype;
    up.rows = (uint32_t)out;
    up.cols = (uint32_t)in;
    up.block_bytes = block_bytes;
    Resident *r = &d->resident[d->resident_count];
    qwn_cuda_abi_header_init(&r->tensor.header, sizeof(r->tensor));
    d->metrics.abi_calls++;
    if (d->abi.upload_tensor(&d->abi.context, &up, &r->tensor) != QWN_CUDA_STATUS_OK) {
        fail(d, "upload of a %dx%d tensor failed", out, in);
        return -1;
    }
    r->host = host;
    return d->resident_count++;
}

static int gemv(QhdDecoder *d, int slot, const void *input, float scale, uint32_t mode, int in, int out,
                float *y) {
    QwnCudaGemmRequest req;
    memset(&req, 0, sizeof(req));
    qwn_cuda_abi_header_init(&req.header, sizeof(req));
    req.tensor = d->resident[slot].tensor;
    req.input_q8 = (const int8_t *)input;
    req.input_scale = scale;
    req.output = y;
    req.batch = 1;
    req.rows = (uint32_t)out;
    req.cols = (uint32_t)in;
    req.input_stride = (uint32_t)in;
    req.output_stride = (uint32_t)out;
    req.input_mode = mode;
    QwnCudaTelemetry tm;
    memset(&tm, 0, sizeof(tm));
    qwn_cuda_abi_header_init(&tm.header, sizeof(tm));
    d->metrics.abi_calls++;
    if (d->abi.gemv(&d->abi.context, &req, &tm) != QWN_CUDA_STATUS_OK || tm.gpu_matmul_count == 0) {
        fail(d, "GPU projection %dx%d failed", out, in);
        return -1;
    }
    mirror_telemetry(d, &tm);
    return 0;
}

/* A quantized matmul (Q4_0 or HyperVSQ-2 blocks): the activation quantized
 * on the host, one GEMV call (c/qwanto_decode.c:776-924). */
static int matmul_q(QhdDecoder *d, const uint8_t *w, int q4, const float *x, int in, int out, float *y) {
    const uint64_t row_bytes = q4 ? (uint64_t)(in + 31) / 32 * 18 : (uint64_t)(in + 255) / 256 * 74;
    const int slot = resident_slot(d, w, q4 ? QWN_CUDA_TENSOR_Q4_0_18 : QWN_CUDA_TENSOR_HYPERVSQ2_74,
                                   q4 ? 18 : 74, row_bytes * (uint64_t)out, out, in);
    if (slot < 0) return -1;
    const float scale = quantize_activation(x, in, d->padded_k, d->q8);
    return gemv(d, slot, d->q8, scale, QWN_CUDA_INPUT_Q8, in, out, y);
}

static int matmul(QhdDecoder *d, const uint8_t *w, const float *x, int in, int out, float *y) {
    return matmul_q(d, w, d->m.cfg.proj_dtype == QHD_PROJ_Q4_0, x, in, out, y);
}

/* The LM head (c/qwanto_decode.c:2007): lm_head.weight when the model has
 * one, else the embedding (:1074-1076).  F16 / BF16 rows take the fp32
 * activation; Q4_0 / HyperVSQ-2 blocks quantize it as every projection. */
static int lm_head(QhdDecoder *d, const float *x, float *logits) {
    const QhdConfig *c = &d->m.cfg;
    const void *w = d->m.lm_head ? d->m.lm_head : (const void *)d->m.embed;
    const int dt = d->m.lm_head ? d->m.lm_head_dtype : (d->m.embed_dtype ? d->m.embed_dtype : QHD_DT_F16);
    if (dt == QHD_DT_Q4_0 || dt == QHD_DT_HVSQ2)
        return matmul_q(d, (const uint8_t *)w, dt == QHD_DT_Q4_0, x, c->hidden, c->vocab, logits);
    const int slot = resident_slot(d, w, dt == QHD_DT_BF16 ? QWN_CUDA_TENSOR_BF16 : QWN_CUDA_TENSOR_F16, 2,
                                   (uint64_t)c->vocab * c->hidden * 2, c->vocab, c->hidden);
    if (slot < 0) return -1;
    return gemv(d, slot, x, 0.0f, QWN_CUDA_INPUT_F32, c->hidden, c->vocab, logits);
}

/* ---- lifecycle ------------------------------------------------------------------- */

void qhd_close(QhdDecoder *d) {
    if (!d) return;
    Abi *a = &d->abi;
    if (a->handle && a->context.opaque && a->context_destroy) {
        for (int i = 0; i < d->resident_count; i++) a->release_tensor(&a->context, &d->resident[i].tensor);
        if (d->kv)
            for (int l = 0; l < d->m.cfg.layers; l++)
                if (d->kv[l].opaque) a->kv_cache_destroy(&a->context, &d->kv[l]);
        a->context_destroy(&a->context);
    }
    if (a->handle) dlclose(a->handle);
    free(d->x); free(d->xb); free(d->q); free(d->k); free(d->v); free(d->ctx);
    free(d->gate); free(d->up); free(d->hidden); free(d->logits); free(d->q8);
    free(d->rope_cos); free(d->rope_sin); free(d->resident); free(d->kv);
    free(d);
}

QhdDecoder *qhd_open(const QhdModel *model, const char *abi_path, int device, char *error, int error_len,
                     char *reason) {
    QhdDecoder *d = (QhdDecoder *)calloc(1, sizeof(*d));
    if (!d) return NULL;
    d->m = *model;
    const QhdConfig *c = &d->m.cfg;
    if (c->hidden <= 0 || c->heads <= 0 || c->kv_heads <= 0 || c->heads % c->kv_heads || c->head_dim % 2 ||
        c->layers <= 0 || c->vocab <= 0 || c->max_ctx <= 0 ||
        (c->proj_dtype != QHD_PROJ_Q4_0 && c->proj_dtype != QHD_PROJ_HVSQ2)) {
        snprintf(d->error, sizeof(d->error), "invalid model configuration");
        goto out_fail;
    }
    const int D = c->hidden, Q = c->heads * c->head_dim, KV = c->kv_heads * c->head_dim;
    const int I = c->intermediate, half = c->head_dim / 2;
    int maxk = D > Q ? D : Q;
    if (I > maxk) maxk = I;
    d->padded_k = (maxk + 255) & ~255;
    d->x = malloc(D * 4); d->xb = malloc((size_t)maxk * 4); d->q = malloc(Q * 4); d->k = malloc(KV * 4);
    d->v = malloc(KV * 4); d->ctx = malloc(Q * 4); d->gate = malloc(I * 4); d->up = malloc(I * 4);
    d->hidden = malloc(I * 4); d->logits = malloc((size_t)c->vocab * 4); d->q8 = malloc(d->padded_k);
    d->rope_cos = malloc((size_t)c->max_ctx * half * 4); d->rope_sin = malloc((size_t)c->max_ctx * half * 4);
    d->resident_cap = c->layers * PROJ_COUNT + 1;
    d->resident = calloc(d->resident_cap, sizeof(Resident));
    d->kv = calloc(c->layers, sizeof(QwnCudaKvCacheHandle));
    if (!d->x || !d->xb || !d->q || !d->k || !d->v || !d->ctx || !d->gate || !d->up || !d->hidden || !d->logits ||
        !d->q8 || !d->rope_cos || !d->rope_sin || !d->resident || !d->kv) {
        snprintf(d->error, sizeof(d->error), "host allocation failed");
        goto out_fail;
    }
    /* c/qwanto_decode.c:601-625 */
    for (int pos = 0; pos < c->max_ctx; pos++)
        for (int i = 0; i < half; i++) {
            const float angle = (float)pos * powf(c->rope_theta, -2.0f * i / (2 * half));
            d->rope_cos[(size_t)pos * half + i] = cosf(angle);
            d->rope_sin[(size_t)pos * half + i] = sinf(angle);
        }
    if (load_abi(d, abi_path, device) != 0) goto out_fail;
    for (int l = 0; l < c->layers; l++) {
        QwnCudaKvCacheOptions o;
        memset(&o, 0, sizeof(o));
        qwn_cuda_abi_header_init(&o.header, sizeof(o));
        o.max_tokens = (uint32_t)c->max_ctx;
        o.kv_heads = (uint32_t)c->kv_heads;
        o.head_dim = (uint32_t)c->head_dim;
        qwn_cuda_abi_header_init(&d->kv[l].header, sizeof(d->kv[l]));
        if (d->abi.kv_cache_create(&d->abi.context, &o, &d->kv[l]) != QWN_CUDA_STATUS_OK) {
            fail(d, "Q8 KV cache creation failed for layer %d", l);
            goto out_fail;
        }
    }
    return d;
out_fail:
    if (error && error_len > 0) snprintf(error, (size_t)error_len, "%s", d->error);
    if (reason) snprintf(reason, sizeof(d->metrics.backend_reason), "%s", d->metrics.backend_reason);
    qhd_close(d);
    return NULL;
}

const char *qhd_last_error(const QhdDecoder *d) { return d ? d->error : "no decoder"; }

int qhd_metrics(const QhdDecoder *d, QhdMetrics *out) {
    if (!d || !out) return -1;
    *out = d->metrics;
    return 0;
}

/* ---- forward / generate ---------------------------------------------------------- */

static int kv_step(QhdDecoder *d, int l, int pos) {
    const QhdConfig *c = &d->m.cfg;
    QwnCudaTelemetry tm;
    memset(&tm, 0, sizeof(tm));
    qwn_cuda_abi_header_init(&tm.header, sizeof(tm));
    QwnCudaKvAppendRequest ap;
    memset(&ap, 0, sizeof(ap));
    qwn_cuda_abi_header_init(&ap.header, sizeof(ap));
    ap.cache = d->kv[l];
    ap.host_key = d->k;
    ap.host_value = d->v;
    ap.n_channels = (uint32_t)(c->kv_heads * c->head_dim);
    ap.token = (uint32_t)pos;
    d->metrics.abi_calls++;
    if (d->abi.kv_cache_append(&d->abi.context, &ap, &tm) != QWN_CUDA_STATUS_OK) {
        fail(d, "layer %d Q8 KV append failed", l);
        return -1;
    }
    QwnCudaKvAttentionRequest at;
    memset(&at, 0, sizeof(at));
    qwn_cuda_abi_header_init(&at.header, sizeof(at));
    at.cache = d->kv[l];
    at.host_query = d->q;
    at.host_output = d->ctx;
    at.query_heads = (uint32_t)c->heads;
    at.kv_heads = (uint32_t)c->kv_heads;
    at.head_dim = (uint32_t)c->head_dim;
    at.position = (uint32_t)pos;
    at.scale = 1.0f / sqrtf((float)c->head_dim);
    d->metrics.abi_calls++;
    if (d->abi.kv_cache_attention(&d->abi.context, &at, &tm) != QWN_CUDA_STATUS_OK) {
        fail(d, "layer %d Q8 KV attention failed", l);
        return -1;
    }
    d->metrics.kv_cache_kernel_count = tm.kv_cache_kernel_count;
    return 0;
}

int qhd_forward(QhdDecoder *d, int token, float *logits_out) {
    const QhdConfig *c = &d->m.cfg;
    const int D = c->hidden, HD = c->head_dim, Q = c->heads * HD, KV = c->kv_heads * HD, I = c->intermediate;
    const int pos = d->position, half = HD / 2;
    if (token < 0 || token >= c->vocab || pos >= c->max_ctx) {
        fail(d, "token %d or position %d out of range", token, pos);
        return -1;
    }
    /* embedding row: F16 or BF16 (qwn_row_f32, c/qwanto_kernels.c:1508-1527) */
    const uint16_t *erow = d->m.embed + (size_t)token * D;
    if (d->m.embed_dtype == QHD_DT_BF16) {
        for (int i = 0; i < D; i++) {
            const uint32_t bits = (uint32_t)erow[i] << 16;
            memcpy(&d->x[i], &bits, sizeof(float));
        }
    } else {
        for (int i = 0; i < D; i++) d->x[i] = half_to_float(erow[i]);
    }
    const float *ct = d->rope_cos + (size_t)pos * half, *st = d->rope_sin + (size_t)pos * half;
    for (int l = 0; l < c->layers; l++) {
        const uint8_t *const *w = d->m.proj + (size_t)l * PROJ_COUNT;
        rmsnorm(d->xb, d->x, d->m.norms[2 * l], D, c->rms_eps);
        if (matmul(d, w[PROJ_Q], d->xb, D, Q, d->q) || matmul(d, w[PROJ_K], d->xb, D, KV, d->k) ||
            matmul(d, w[PROJ_V], d->xb, D, KV, d->v))
            return -1;
        add_bias(d->q, bias_of(d, l, PROJ_Q), Q);
        add_bias(d->k, bias_of(d, l, PROJ_K), KV);
        add_bias(d->v, bias_of(d, l, PROJ_V), KV);
        if (d->m.qk_norms) {
            /* head_rmsnorm (c/qwanto_decode.c:654-684): each head in place */
            for (int h = 0; h < c->heads; h++)
                rmsnorm(d->q + (size_t)h * HD, d->q + (size_t)h * HD, d->m.qk_norms[2 * l], HD, c->rms_eps);
            for (int h = 0; h < c->kv_heads; h++)
                rmsnorm(d->k + (size_t)h * HD, d->k + (size_t)h * HD, d->m.qk_norms[2 * l + 1], HD, c->rms_eps);
        }
        rope(d->q, c->heads, HD, ct, st);
        rope(d->k, c->kv_heads, HD, ct, st);
        if (kv_step(d, l, pos)) return -1;
        if (matmul(d, w[PROJ_O], d->ctx, Q, D, d->xb)) return -1;
        add_bias(d->xb, bias_of(d, l, PROJ_O), D);
        for (int i = 0; i < D; i++) d->x[i] += d->xb[i];
        rmsnorm(d->xb, d->x, d->m.norms[2 * l + 1], D, c->rms_eps);
        if (matmul(d, w[PROJ_GATE], d->xb, D, I, d->gate) || matmul(d, w[PROJ_UP], d->xb, D, I, d->up)) return -1;
        for (int i = 0; i < I; i++) {
            const float g = d->gate[i];
            d->hidden[i] = (g / (1.0f + expf(-g))) * d->up[i];
        }
        if (matmul(d, w[PROJ_DOWN], d->hidden, I, D, d->xb)) return -1;
        for (int i = 0; i < D; i++) d->x[i] += d->xb[i];
    }
    rmsnorm(d->xb, d->x, d->m.final_norm, D, c->rms_eps);
    if (lm_head(d, d->xb, d->logits)) return -1;
    d->position++;
    if (logits_out) memcpy(logits_out, d->logits, (size_t)c->vocab * 4);
    return 0;
}

static int argmax(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

int qhd_generate(QhdDecoder *d, const int *prompt, int prompt_count, int max_new, int *tokens, float *margins) {
    const double t0 = now_s();
    d->metrics.prompt_tokens = prompt_count;
    for (int i = 0; i < prompt_count; i++)
        if (qhd_forward(d, prompt[i], NULL)) return -1;
    const double t1 = now_s();
    d->metrics.prefill_ms = (t1 - t0) * 1e3;
    const int V = d->m.cfg.vocab;
    int generated = 0;
    for (int s = 0; s < max_new; s++) {
        const int t = argmax(d->logits, V);
        tokens[s] = t;
        if (margins) {
            float second = -INFINITY;
            for (int i = 0; i < V; i++)
                if (i != t && d->logits[i] > second) second = d->logits[i];
            margins[s] = d->logits[t] - second;
        }
        generated++;
        if (qhd_forward(d, t, NULL)) return -1;
    }
    d->metrics.generated_tokens = generated;
    d->metrics.decode_wall_ms = (now_s() - t1) * 1e3;
    return generated;
}
