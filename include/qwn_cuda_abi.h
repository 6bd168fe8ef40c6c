#ifndef QWN_CUDA_ABI_H
#define QWN_CUDA_ABI_H

/*
 * qwn_hip: the versioned qwnrun GPU ABI, implemented for one AMD Instinct
 * MI355X (gfx950).
 *
 * This is the contract that qwnrun resolves from "<exe dir>/qwn_cuda.so"
 * (reference: c/cuda/qwn_cuda_abi.h, loaded by c/qwanto_decode.c:267-462).
 * Every struct, enum value and exported symbol of ABI version 1 keeps the
 * reference's binary layout, because an unmodified qwnrun dlopen()s this
 * library and passes its own structs: the layout is the interface, so it
 * cannot be redesigned. tests/test_abi.py checks every size and field
 * offset against a fixture generated from the reference header.
 *
 * Extensions (marked EXT below) only append enum values and capability bits;
 * the ABI version stays 1 because the reference host rejects any other
 * (c/qwanto_decode.c:366).  A v1 host that only knows HyperVSQ-2 never sees
 * them.
 *
 * No GPU runtime types appear here: a host can validate and load the
 * library without linking HIP.
 */

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define QWN_CUDA_ABI_API __attribute__((visibility("default")))
#else
#define QWN_CUDA_ABI_API
#endif

#define QWN_CUDA_ABI_VERSION 1u
#define QWN_CUDA_ABI_NAME "qwn_cuda_hypervsq2"
#define QWN_CUDA_HYPERVSQ2_BLOCK_BYTES 74u
#define QWN_CUDA_HYPERVSQ2_BLOCK_ELEMENTS 256u
#define QWN_CUDA_MAX_RESIDENT_TENSORS 512u
#define QWN_CUDA_MAX_RESIDENT_KV_CACHES 128u

/* EXT: Q4_0 blocks are an fp16 scale followed by 32 nibbles
 * (c/qwanto_native.h:35, element 2j = low nibble of byte j). */
#define QWN_CUDA_Q4_0_BLOCK_BYTES 18u
#define QWN_CUDA_Q4_0_BLOCK_ELEMENTS 32u

/* Leading member of every public struct.  The callee accepts a struct when
 * abi_version matches and struct_size is at least the size it was built
 * with, so later versions may append fields. */
typedef struct {
    uint32_t struct_size;
    uint32_t abi_version;
    uint32_t reserved[4];
} QwnCudaAbiHeader;

static inline void qwn_cuda_abi_header_init(QwnCudaAbiHeader *header,
                                             uint32_t struct_size) {
    if (!header) return;
    header->struct_size = struct_size;
    header->abi_version = QWN_CUDA_ABI_VERSION;
    header->reserved[0] = 0;
    header->reserved[1] = 0;
    header->reserved[2] = 0;
    header->reserved[3] = 0;
}

enum {
    QWN_CUDA_CAP_HYPERVSQ2_GEMV = 1ull << 0,
    QWN_CUDA_CAP_HYPERVSQ2_GEMM = 1ull << 1,
    QWN_CUDA_CAP_RESIDENT_WEIGHTS = 1ull << 2,
    QWN_CUDA_CAP_TELEMETRY = 1ull << 3,
    QWN_CUDA_CAP_DEVICE_ENUMERATION = 1ull << 4,
    QWN_CUDA_CAP_Q8_KV = 1ull << 5,
    /* EXT: Q4_0 (18-byte block) tensors through hypervsq2_gemv/gemm. */
    QWN_CUDA_CAP_Q4_0_GEMV = 1ull << 6,
    /* EXT: F16 row-major tensors with QWN_CUDA_INPUT_F32 activations. */
    QWN_CUDA_CAP_F16_GEMV = 1ull << 7,
    /* EXT: the qwn_hip_ext_* device-pointer entry points (qwn_hip_ext.h). */
    QWN_CUDA_CAP_DEVICE_POINTERS = 1ull << 8,
    /* EXT: BF16 row-major tensors with QWN_CUDA_INPUT_F32 activations. */
    QWN_CUDA_CAP_BF16_GEMV = 1ull << 9
};

typedef enum {
    QWN_CUDA_STATUS_OK = 0,
    QWN_CUDA_STATUS_INVALID_ARGUMENT = -1,
    QWN_CUDA_STATUS_ABI_MISMATCH = -2,
    QWN_CUDA_STATUS_UNAVAILABLE = -3,
    QWN_CUDA_STATUS_OUT_OF_MEMORY = -4,
    QWN_CUDA_STATUS_UNSUPPORTED = -5,
    QWN_CUDA_STATUS_RUNTIME_ERROR = -6
} QwnCudaStatus;

typedef enum {
    QWN_CUDA_TENSOR_HYPERVSQ2_74 = 1,
    /* EXT */
    QWN_CUDA_TENSOR_Q4_0_18 = 2,
    /* EXT: IEEE binary16, rows x cols row-major (cols fastest). */
    QWN_CUDA_TENSOR_F16 = 3,
    /* EXT: bfloat16 (the high half of a binary32), rows x cols row-major. */
    QWN_CUDA_TENSOR_BF16 = 4
} QwnCudaTensorDType;

typedef enum {
    QWN_CUDA_INPUT_Q8 = 1,
    /* EXT: input_q8 points at fp32 activations [batch x input_stride];
     * F16 and BF16 tensors take them as is, quantized tensors quantize them per
     * token on the device (the reference's host-side arithmetic). */
    QWN_CUDA_INPUT_F32 = 2
} QwnCudaInputMode;

typedef struct {
    QwnCudaAbiHeader header;
    uint64_t capability_bits;
    uint32_t max_devices;
    uint32_t max_resident_tensors;
    uint32_t hypervsq2_block_bytes;
    uint32_t hypervsq2_block_elements;
    char abi_name[32];
} QwnCudaAbiInfo;

typedef struct {
    QwnCudaAbiHeader header;
    int32_t device_id;
    int32_t compute_major;
    int32_t compute_minor;
    uint64_t total_vram_bytes;
    uint64_t free_vram_bytes;
    char name[128];
    char driver[64];
} QwnCudaDeviceInfo;

typedef struct {
    QwnCudaAbiHeader header;
    int32_t device_id;
    uint32_t flags;
    uint64_t memory_budget_bytes;
    uint64_t context_size;
} QwnCudaContextOptions;

typedef struct {
    QwnCudaAbiHeader header;
    void *opaque;
} QwnCudaContextHandle;

typedef struct {
    QwnCudaAbiHeader header;
    void *opaque;
} QwnCudaTensorHandle;

typedef struct {
    QwnCudaAbiHeader header;
    void *opaque;
} QwnCudaKvCacheHandle;

typedef struct {
    QwnCudaAbiHeader header;
    uint32_t max_tokens;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t reserved;
} QwnCudaKvCacheOptions;

typedef struct {
    QwnCudaAbiHeader header;
    QwnCudaKvCacheHandle cache;
    const float *host_key;
    const float *host_value;
    uint32_t n_channels;
    uint32_t token;
} QwnCudaKvAppendRequest;

typedef struct {
    QwnCudaAbiHeader header;
    QwnCudaKvCacheHandle cache;
    const float *host_query;
    float *host_output;
    uint32_t query_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t position;
    float scale;
} QwnCudaKvAttentionRequest;

typedef struct {
    QwnCudaAbiHeader header;
    const void *host_data;
    uint64_t data_bytes;
    uint32_t dtype;
    uint32_t rows;
    uint32_t cols;
    uint32_t block_bytes;
} QwnCudaTensorUpload;

typedef struct {
    QwnCudaAbiHeader header;
    QwnCudaTensorHandle tensor;
    const int8_t *input_q8;
    float input_scale;
    const float *input_scales;
    float *output;
    uint32_t batch;
    uint32_t rows;
    uint32_t cols;
    uint32_t input_stride;
    uint32_t output_stride;
    uint32_t input_mode;
} QwnCudaGemmRequest;

/* Cumulative per-context counters; every call that takes a telemetry
 * pointer copies the whole struct out. */
typedef struct {
    QwnCudaAbiHeader header;
    uint64_t gpu_matmul_count;
    uint64_t gpu_kernel_launch_count;
    uint64_t gpu_projection_count;
    uint64_t gpu_upload_count;
    uint64_t gpu_upload_bytes;
    uint64_t gpu_resident_bytes;
    uint64_t cpu_matmul_fallback_count;
    uint64_t unsupported_projection_count;
    double gpu_kernel_ms;
    double gpu_transfer_ms;
    double gpu_sync_ms;
    int32_t device_id;
    uint32_t reserved_device;
    char device_name[128];
    char kernel_type[32];
    char dll_hash[65];
    uint64_t kv_cache_kernel_count;
    uint64_t kv_cache_upload_bytes;
    uint64_t kv_cache_resident_bytes;
    double kv_cache_kernel_ms;
    double kv_cache_transfer_ms;
    char kv_cache_kernel_type[32];
} QwnCudaTelemetry;

typedef int (*QwnCudaAbiQueryFn)(QwnCudaAbiInfo *info);
typedef int (*QwnCudaCapabilityQueryFn)(QwnCudaAbiInfo *info);
typedef int (*QwnCudaEnumerateDevicesFn)(QwnCudaDeviceInfo *devices,
                                         uint32_t capacity,
                                         uint32_t *count);
typedef int (*QwnCudaContextCreateFn)(const QwnCudaContextOptions *options,
                                      QwnCudaContextHandle *context);
typedef int (*QwnCudaContextDestroyFn)(QwnCudaContextHandle *context);
typedef int (*QwnCudaTensorUploadFn)(QwnCudaContextHandle *context,
                                     const QwnCudaTensorUpload *upload,
                                     QwnCudaTensorHandle *tensor);
typedef int (*QwnCudaTensorReleaseFn)(QwnCudaContextHandle *context,
                                      QwnCudaTensorHandle *tensor);
typedef int (*QwnCudaKvCreateFn)(QwnCudaContextHandle *context,
                                  const QwnCudaKvCacheOptions *options,
                                  QwnCudaKvCacheHandle *cache);
typedef int (*QwnCudaKvDestroyFn)(QwnCudaContextHandle *context,
                                  QwnCudaKvCacheHandle *cache);
typedef int (*QwnCudaKvAppendFn)(QwnCudaContextHandle *context,
                                 const QwnCudaKvAppendRequest *request,
                                 QwnCudaTelemetry *telemetry);
typedef int (*QwnCudaKvAttentionFn)(QwnCudaContextHandle *context,
                                    const QwnCudaKvAttentionRequest *request,
                                    QwnCudaTelemetry *telemetry);
typedef int (*QwnCudaKvResetFn)(QwnCudaContextHandle *context,
                                QwnCudaKvCacheHandle *cache);
typedef int (*QwnCudaGemvFn)(QwnCudaContextHandle *context,
                             const QwnCudaGemmRequest *request,
                             QwnCudaTelemetry *telemetry);
typedef int (*QwnCudaGemmFn)(QwnCudaContextHandle *context,
                             const QwnCudaGemmRequest *request,
                             QwnCudaTelemetry *telemetry);
typedef int (*QwnCudaSynchronizeFn)(QwnCudaContextHandle *context);
typedef int (*QwnCudaTelemetryFn)(QwnCudaContextHandle *context,
                                  QwnCudaTelemetry *telemetry);
typedef int (*QwnCudaLastErrorFn)(char *buffer, uint32_t buffer_size);

/* Replaces c/cuda/qwn_hypervsq2_cuda_abi.cu:417 (abi query + capability bits). */
QWN_CUDA_ABI_API int qwn_cuda_abi_query(QwnCudaAbiInfo *info);
/* Replaces :438; same answer as query. */
QWN_CUDA_ABI_API int qwn_cuda_abi_get_capabilities(QwnCudaAbiInfo *info);
/* Replaces :442; real HIP enumeration (name, gcnArchName, VRAM). */
QWN_CUDA_ABI_API int qwn_cuda_abi_enumerate_devices(QwnCudaDeviceInfo *devices,
                                                     uint32_t capacity,
                                                     uint32_t *count);
/* Replaces :477; one HIP stream + staging per context. */
QWN_CUDA_ABI_API int qwn_cuda_abi_context_create(
    const QwnCudaContextOptions *options, QwnCudaContextHandle *context);
/* Replaces :504. */
QWN_CUDA_ABI_API int qwn_cuda_abi_context_destroy(QwnCudaContextHandle *context);
/* Replaces :537; repacks to the device layout after the copy. */
QWN_CUDA_ABI_API int qwn_cuda_abi_upload_tensor(QwnCudaContextHandle *context,
                                                const QwnCudaTensorUpload *upload,
                                                QwnCudaTensorHandle *tensor);
/* Replaces :587. */
QWN_CUDA_ABI_API int qwn_cuda_abi_release_tensor(QwnCudaContextHandle *context,
                                                 QwnCudaTensorHandle *tensor);
/* Replaces :604; 16-token pages of int8 K/V plus fp32 group scales. */
QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_create(
    QwnCudaContextHandle *context, const QwnCudaKvCacheOptions *options,
    QwnCudaKvCacheHandle *cache);
/* Replaces :812. */
QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_destroy(
    QwnCudaContextHandle *context, QwnCudaKvCacheHandle *cache);
/* Replaces :692 (Q8 quantize of one token's K and V). */
QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_append(
    QwnCudaContextHandle *context, const QwnCudaKvAppendRequest *request,
    QwnCudaTelemetry *telemetry);
/* Replaces :749 (split-T flash-decode attention over the Q8 cache). */
QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_attention(
    QwnCudaContextHandle *context, const QwnCudaKvAttentionRequest *request,
    QwnCudaTelemetry *telemetry);
/* Replaces :803. */
QWN_CUDA_ABI_API int qwn_cuda_abi_kv_cache_reset(
    QwnCudaContextHandle *context, QwnCudaKvCacheHandle *cache);
/* Replaces :835 (batch must be 1). */
QWN_CUDA_ABI_API int qwn_cuda_abi_hypervsq2_gemv(QwnCudaContextHandle *context,
                                                const QwnCudaGemmRequest *request,
                                                QwnCudaTelemetry *telemetry);
/* Replaces :845 (any batch; weights read once for all tokens). */
QWN_CUDA_ABI_API int qwn_cuda_abi_hypervsq2_gemm(QwnCudaContextHandle *context,
                                                const QwnCudaGemmRequest *request,
                                                QwnCudaTelemetry *telemetry);
/* Replaces :854. */
QWN_CUDA_ABI_API int qwn_cuda_abi_synchronize(QwnCudaContextHandle *context);
/* Replaces :865. */
QWN_CUDA_ABI_API int qwn_cuda_abi_get_telemetry(QwnCudaContextHandle *context,
                                                QwnCudaTelemetry *telemetry);
/* Replaces :874 (process-wide last error string). */
QWN_CUDA_ABI_API int qwn_cuda_abi_last_error(char *buffer, uint32_t buffer_size);

#ifdef __cplusplus
}
#endif

#endif /* QWN_CUDA_ABI_H */
