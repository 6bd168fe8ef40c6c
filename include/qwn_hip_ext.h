#ifndef QWN_HIP_EXT_H
#define QWN_HIP_EXT_H

/*
 * qwn_hip extensions beyond the reference's qwnrun ABI.
 *
 * None of these has a counterpart in c/cuda/qwn_cuda_abi.h.  They exist for
 * callers that keep activations on the device: a resident decode loop, a
 * benchmark that times kernels with inputs already in HBM, HIP graph
 * capture.  They take DEVICE pointers, enqueue on the caller's stream
 * (a hipStream_t passed as void*; NULL = the context's own stream, a
 * blocking stream, so ordered with work on the null stream), never
 * synchronise and never allocate, so they are safe to record into a graph.
 * The library advertises them with QWN_CUDA_CAP_DEVICE_POINTERS.
 *
 * Contexts, tensors and KV caches are the handles of qwn_cuda_abi.h.
 * Device pointer alignment: int8 activation rows and fp32 activation rows
 * must start on 16-byte boundaries (pointer and row stride).
 */

#include "qwn_cuda_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    QwnCudaAbiHeader header;
    uint32_t dtype;          /* QwnCudaTensorDType */
    uint32_t rows;
    uint32_t cols;
    uint32_t units_per_row;  /* lane work units: HyperVSQ-2 block, 4 Q4_0 blocks, 8 halves */
    uint64_t logical_bytes;  /* bytes in the on-disk format (what the ABI was given) */
    uint64_t device_bytes;   /* bytes resident in the device layout */
    uint32_t lanes_per_row;  /* launch plan for batch 1 */
    uint32_t units_per_lane;
    uint32_t rows_per_wave;
    uint32_t grid;
    uint64_t mfma_copy_bytes; /* the batched GEMM's MFMA-order copy (0: none), charged to the
                                 context's budget and gpu_resident_bytes with logical_bytes */
} QwnHipTensorInfo;

/* Shape, byte counts and batch-1 launch plan of a resident tensor. */
QWN_CUDA_ABI_API int qwn_hip_ext_tensor_info(const QwnCudaTensorHandle *tensor,
                                             QwnHipTensorInfo *info);

/* Activation images.  The GEMV reads activations from an "image": per token
 * the exact LDS layout its dot products use (int8 values split into signed
 * high and unsigned low nibbles in the order the weight unpack produces,
 * plus per-32 correction sums; fp32 for F16 tensors).  Images depend only
 * on the tensor's dtype and column count, so one image serves every tensor
 * with the same input (q/k/v, gate/up).  Image strides and pointers must be
 * 16-byte aligned. */
QWN_CUDA_ABI_API uint64_t qwn_hip_ext_activation_image_bytes(const QwnCudaTensorHandle *tensor);

/* Image from int8 tokens (HyperVSQ-2, Q4_0 tensors) or fp32 tokens (F16
 * tensors): x [batch][x_stride elements] -> image [batch][image_stride]. */
QWN_CUDA_ABI_API int qwn_hip_ext_prepare_image_device(QwnCudaContextHandle *context,
                                                      const QwnCudaTensorHandle *tensor,
                                                      const void *x, uint32_t batch,
                                                      uint32_t x_stride, void *image,
                                                      uint32_t image_stride, void *stream);

/* Per-token int8 quantization of fp32 x (the activation step of
 * c/qwanto_kernels.c:354-433) fused with the image build: writes scales
 * [batch], the images and, if q8 is not NULL, the int8 tokens
 * [batch][q8_stride] zero padded. */
QWN_CUDA_ABI_API int qwn_hip_ext_quantize_image_device(QwnCudaContextHandle *context,
                                                       const QwnCudaTensorHandle *tensor,
                                                       const float *x, uint32_t batch,
                                                       uint32_t x_stride, void *image,
                                                       uint32_t image_stride, float *scales,
                                                       int8_t *q8, uint32_t q8_stride,
                                                       void *stream);

/* GEMV/GEMM on images: output [batch][output_stride] = W x_t * scale_t
 * (scales[t], or `scale` when scales is NULL; ignored for F16).  Weights
 * are read once per 16 tokens. */
QWN_CUDA_ABI_API int qwn_hip_ext_gemm_image_device(QwnCudaContextHandle *context,
                                                   const QwnCudaTensorHandle *tensor,
                                                   const void *image, uint32_t image_stride,
                                                   const float *scales, float scale,
                                                   float *output, uint32_t batch,
                                                   uint32_t output_stride, void *stream);

/* Grouped GEMV: up to 4 tensors of one dtype and column count that share
 * one input (q/k/v, gate/up) in a single launch.  Input modes:
 *   IMAGE    prebuilt activation images [batch][image_stride], scales
 *   F32      one fp32 token x [cols] (cols a multiple of 32); every
 *            workgroup quantizes it per token itself (c/qwanto_kernels.c:
 *            354-433) into its LDS image -- no separate quantize launch
 *   RMSNORM  y = (x * 1/sqrt(mean(x^2) + eps)) * norm, then as F32
 *            (c/qwanto_decode.c:627-652)
 *   SWIGLU   y = (x / (1 + exp(-x))) * x2, then as F32
 *            (c/qwanto_decode.c:1946-1949)
 * Output modes: STORE; ADD (outputs += result, one token: the residual
 * stream); ARGMAX (store, and one packed key per workgroup in
 * argmax_partials -- qwn_hip_ext_gemv_group_partials() of them -- reduced
 * by qwn_hip_ext_argmax_device to the first index of the largest output);
 * SWIGLU (two tensors of one shape, gate and up, one token: outputs[0] =
 * (g / (1 + exp(-g))) * u per row, c/qwanto_decode.c:1946-1949; outputs[1]
 * is not written).
 * Device pointers, caller's stream, no allocation. */
#define QWN_HIP_GEMV_INPUT_IMAGE 0u
#define QWN_HIP_GEMV_INPUT_F32 1u
#define QWN_HIP_GEMV_INPUT_RMSNORM 2u
#define QWN_HIP_GEMV_INPUT_SWIGLU 3u
#define QWN_HIP_GEMV_OUTPUT_STORE 0u
#define QWN_HIP_GEMV_OUTPUT_ADD 1u
#define QWN_HIP_GEMV_OUTPUT_ARGMAX 2u
#define QWN_HIP_GEMV_OUTPUT_SWIGLU 3u
#define QWN_HIP_GEMV_MAX_GROUP 4u

typedef struct {
    QwnCudaAbiHeader header;
    uint32_t count;                       /* tensors, 1..4 */
    uint32_t input_mode;                  /* QWN_HIP_GEMV_INPUT_* */
    uint32_t output_mode;                 /* QWN_HIP_GEMV_OUTPUT_* */
    uint32_t batch;                       /* tokens (image input); 1 otherwise */
    const QwnCudaTensorHandle *tensors;   /* [count] */
    float *const *outputs;                /* [count] device fp32 [batch][output_stride] */
    uint32_t output_stride;               /* 0: rows of each tensor */
    uint32_t image_stride;
    const void *image;
    const float *scales;                  /* image input: per-token scales or NULL */
    float scale;                          /* image input without scales */
    float eps;                            /* RMSNORM */
    const float *x;                       /* fp32 input [cols] */
    const float *x2;                      /* SWIGLU: the up projection [cols] */
    const float *norm;                    /* RMSNORM weights [cols] */
    float *scale_out;                     /* optional: the activation scale (one float) */
    uint64_t *argmax_partials;            /* ARGMAX */
} QwnHipGemvGroupRequest;

QWN_CUDA_ABI_API uint32_t qwn_hip_ext_gemv_group_partials(QwnCudaContextHandle *context,
                                                          const QwnHipGemvGroupRequest *request);
QWN_CUDA_ABI_API int qwn_hip_ext_gemv_group_device(QwnCudaContextHandle *context,
                                                   const QwnHipGemvGroupRequest *request, void *stream);
QWN_CUDA_ABI_API int qwn_hip_ext_argmax_device(QwnCudaContextHandle *context, const uint64_t *partials,
                                               uint32_t count, int32_t *index, void *stream);

/* int8 MFMA batch GEMM of a HyperVSQ-2 or Q4_0 tensor, 1..16 tokens per
 * call (the ABI's GEMM uses it by itself from 2 HyperVSQ-2 / 3 Q4_0
 * tokens on the MFMA-order copy, from 3 / 6 without it): HyperVSQ-2 blocks are exact int8 dot products with the octant
 * multipliers folded into the weights (v_mfma_i32_16x16x64_i8), Q4_0 blocks
 * one v_mfma_i32_16x16x32_i8 each on the signed codes n - 8, on tiles of 16
 * rows x 16 tokens.  The activations are read from an "MFMA image" of the
 * int8 tokens (qwn_hip_ext_mfma_image_bytes() bytes, 16-byte aligned;
 * 0 for F16 tensors), built by qwn_hip_ext_mfma_image_device from q8
 * [batch][q8_stride].  output [batch][output_stride] = W x_t * scales[t]. */
QWN_CUDA_ABI_API uint64_t qwn_hip_ext_mfma_image_bytes(const QwnCudaTensorHandle *tensor);
QWN_CUDA_ABI_API int qwn_hip_ext_mfma_image_device(QwnCudaContextHandle *context,
                                                   const QwnCudaTensorHandle *tensor, const int8_t *q8,
                                                   uint32_t batch, uint32_t q8_stride, void *image,
                                                   void *stream);
QWN_CUDA_ABI_API int qwn_hip_ext_gemm_mfma_device(QwnCudaContextHandle *context,
                                                  const QwnCudaTensorHandle *tensor, const void *image,
                                                  const float *scales, float *output, uint32_t batch,
                                                  uint32_t output_stride, void *stream);
/* The same GEMM over `count` (1..4) tensors of one kind with the same
 * column count that share one MFMA image (q/k/v, gate/up), in one launch:
 * outputs[i] [batch][output_stride or the tensor's rows]; accumulate != 0
 * adds the product to the outputs (a residual stream) instead. */
QWN_CUDA_ABI_API int qwn_hip_ext_gemm_mfma_group_device(QwnCudaContextHandle *context,
                                                        const QwnCudaTensorHandle *tensors, uint32_t count,
                                                        const void *image, const float *scales,
                                                        float *const *outputs, uint32_t batch,
                                                        uint32_t output_stride, uint32_t accumulate,
                                                        void *stream);

/* Upload `count` tensors, each as qwn_cuda_abi_upload_tensor
 * (c/cuda/qwn_cuda_abi.h:244-246), through one pipeline: whole-row chunks
 * of each host buffer (an mmap'd .qwn payload, say) are copied into one of
 * two pinned staging slots while the other slot's DMA and repack run; the
 * call synchronises once for the batch.  out[i] receives tensor i's handle;
 * on failure nothing of the batch stays resident.  (No counterpart in the
 * reference: its host uploads tensor by tensor, c/qwanto_decode.c:790-830.) */
QWN_CUDA_ABI_API int qwn_hip_ext_upload_batch(QwnCudaContextHandle *context,
                                              const QwnCudaTensorUpload *uploads, uint32_t count,
                                              QwnCudaTensorHandle *out);

/* Tensor placement with a GPU tier, as the reference's qwn_plan_residency
 * (c/qwanto_native.c:379-435, replaced here): tensors in the order of their
 * name's priority (embedding / LM head 255, norms 245, attention 230, dense
 * gate 210, other 160, experts 80), then smaller first, then index; each
 * goes to the GPU while the GPU budget has room, else to RAM while the RAM
 * budget has room, else stays file-backed.  items[count] receive the plan
 * in that order (the reference's QwnPlacement layout), totals[3] the GPU,
 * RAM and file bytes.  gpu_budget QWN_HIP_GPU_BUDGET_AUTO: 90% of the free
 * memory of the context's device (context required), as the reference host
 * sizes its GPU tier (c/qwanto_decode.c:202-216); otherwise context may be
 * NULL. */
#define QWN_HIP_TIER_GPU 0u
#define QWN_HIP_TIER_RAM 1u
#define QWN_HIP_TIER_FILE 2u
#define QWN_HIP_GPU_BUDGET_AUTO UINT64_MAX
typedef struct {
    uint64_t name_hash;       /* FNV-1a 64 of the name (the .qwn index hash) */
    uint64_t byte_offset;
    uint64_t byte_size;
    uint32_t tensor_index;
    uint8_t tier;             /* QWN_HIP_TIER_* */
    uint8_t priority;
    uint16_t reserved;
} QwnHipPlacement;
QWN_CUDA_ABI_API int qwn_hip_ext_plan_residency(QwnCudaContextHandle *context, const char *const *names,
                                                const uint64_t *byte_offsets, const uint64_t *byte_sizes,
                                                uint32_t count, uint64_t gpu_budget, uint64_t ram_budget,
                                                QwnHipPlacement *items, uint64_t *totals);

/* Per-token int8 quantization on the device without an image:
 * x fp32 [batch][x_stride] -> q8 [batch][q8_stride] (zero padded past
 * cols), scales [batch]. */
QWN_CUDA_ABI_API int qwn_hip_ext_quantize_device(QwnCudaContextHandle *context,
                                                 const float *x, uint32_t batch,
                                                 uint32_t cols, uint32_t x_stride,
                                                 int8_t *q8, uint32_t q8_stride,
                                                 float *scales, void *stream);

/* Append `count` tokens of fp32 K and V ([count][n_channels], device) at
 * position cache.tokens; synchronous bookkeeping, asynchronous kernels. */
QWN_CUDA_ABI_API int qwn_hip_ext_kv_append_device(QwnCudaContextHandle *context,
                                                  QwnCudaKvCacheHandle *cache,
                                                  const float *keys,
                                                  const float *values,
                                                  uint32_t count, void *stream);

/* Attention over tokens [0, position] with a device query and output
 * ([query_heads][head_dim] fp32).  `workspace` is a device buffer of at
 * least qwn_hip_ext_attention_workspace_bytes() bytes. */
QWN_CUDA_ABI_API uint64_t qwn_hip_ext_attention_workspace_bytes(
    QwnCudaKvCacheHandle *cache, uint32_t query_heads, uint32_t position);
QWN_CUDA_ABI_API int qwn_hip_ext_kv_attention_device(QwnCudaContextHandle *context,
                                                     QwnCudaKvCacheHandle *cache,
                                                     const float *query, float *output,
                                                     uint32_t query_heads,
                                                     uint32_t position, float scale,
                                                     void *workspace, void *stream);

/* The same attention with no workspace argument and no allocation: the
 * split partials live in a file-scope device array of 4 MiB per GPU (its
 * address looked up once per device at context creation).  No counterpart
 * in the reference; for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid hipMalloc).  A request whose partials
 * exceed the array (qwn_hip_ext_attention_workspace_bytes() > 4 MiB) is
 * refused with QWN_CUDA_STATUS_INVALID_ARGUMENT.  Every call on one GPU
 * shares that GPU's array, so calls must not run at the same time on one
 * GPU: a call is refused with QWN_CUDA_STATUS_UNAVAILABLE while the
 * previous call on that GPU, enqueued on a different stream (another
 * stream of the caller, another context's stream), has not finished.
 * Calls on one stream are ordered and always accepted.  Calls recorded
 * into a HIP graph are not tracked: a graph that replays them on two
 * streams at once races. */
QWN_CUDA_ABI_API int qwn_hip_ext_kv_attention_device_noalloc(QwnCudaContextHandle *context,
                                                             QwnCudaKvCacheHandle *cache,
                                                             const float *query, float *output,
                                                             uint32_t query_heads, uint32_t position,
                                                             float scale, void *stream);

/* Debug: the integer sums of the GEMV for one token, computed by the same
 * device code as the GEMV (host pointers, synchronous).  HyperVSQ-2:
 * out[row][block*8 + octant] = sum (code-1)*a; Q4_0: out[row][block] =
 * sum (nibble-8)*a.  out_capacity counts int32 elements. */
QWN_CUDA_ABI_API int qwn_hip_ext_debug_int_sums(QwnCudaContextHandle *context,
                                                const QwnCudaTensorHandle *tensor,
                                                const int8_t *host_q8,
                                                int32_t *host_out,
                                                uint64_t out_capacity);

/* Debug: the exact int32 block dot products of the int8 MFMA GEMM
 * (qwn_hip_ext_gemm_mfma_device's kernel, the same plan and operand code)
 * for batch (1..16) int8 tokens host_q8 [batch][cols] (host pointers,
 * synchronous).  out[token][row][block]: HyperVSQ-2 per 256-weight block
 * sum over octants of multiplier * sum (code-1)*a; Q4_0 per 32-weight block
 * sum (nibble-8)*a.  out_capacity counts int32 elements. */
QWN_CUDA_ABI_API int qwn_hip_ext_debug_mfma_int_sums(QwnCudaContextHandle *context,
                                                     const QwnCudaTensorHandle *tensor,
                                                     const int8_t *host_q8, uint32_t batch,
                                                     int32_t *host_out, uint64_t out_capacity);

/* Debug: cached tokens [first, first + count) of a Q8 KV cache in the CPU
 * cache's token-major layout (c/qwanto_turboquant.h:78-94): keys/values
 * [count][kv_heads*head_dim] int8, scales [count][ceil(channels/64)] fp32
 * (host pointers, synchronous). */
QWN_CUDA_ABI_API int qwn_hip_ext_debug_kv_read(QwnCudaContextHandle *context,
                                               const QwnCudaKvCacheHandle *cache, uint32_t first,
                                               uint32_t count, int8_t *host_keys, int8_t *host_values,
                                               float *host_key_scales, float *host_value_scales);

#ifdef __cplusplus
}
#endif

#endif /* QWN_HIP_EXT_H */
