#ifndef QWN_HIP_EXT_H
#define QWN_HIP_EXT_H

/*
 * qwn_hip extensions beyond the reference's qwnrun ABI.
 *
 * None of these has a counterpart in c/cuda/qwn_cuda_abi.h.  They exist for
 * callers that keep activations on the device: a resident decode loop, a
 * benchmark that times kernels with inputs already in HBM, HIP graph
 * capture.  They take DEVICE pointers, enqueue on the caller's stream
 * (a hipStream_t passed as void*; NULL = the context's own stream), never
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
} QwnHipTensorInfo;

/* Shape, byte counts and batch-1 launch plan of a resident tensor. */
QWN_CUDA_ABI_API int qwn_hip_ext_tensor_info(const QwnCudaTensorHandle *tensor,
                                             QwnHipTensorInfo *info);

/* GEMV/GEMM with device pointers: request->input_q8 / input_scales /
 * output are device addresses (input_q8 is fp32 for F16 tensors with
 * QWN_CUDA_INPUT_F32).  Any batch; weights are read once per 16 tokens. */
QWN_CUDA_ABI_API int qwn_hip_ext_gemm_device(QwnCudaContextHandle *context,
                                             const QwnCudaGemmRequest *request,
                                             void *stream);

/* Per-token int8 quantization on the device, the activation step of
 * c/qwanto_kernels.c:354-433: x fp32 [batch][x_stride] -> q8
 * [batch][q8_stride] (zero padded past cols), scales [batch]. */
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

/* Debug: the integer sums of the GEMV for one token, computed by the same
 * device code as the GEMV (host pointers, synchronous).  HyperVSQ-2:
 * out[row][block*8 + octant] = sum (code-1)*a; Q4_0: out[row][block] =
 * sum (nibble-8)*a.  out_capacity counts int32 elements. */
QWN_CUDA_ABI_API int qwn_hip_ext_debug_int_sums(QwnCudaContextHandle *context,
                                                const QwnCudaTensorHandle *tensor,
                                                const int8_t *host_q8,
                                                int32_t *host_out,
                                                uint64_t out_capacity);

#ifdef __cplusplus
}
#endif

#endif /* QWN_HIP_EXT_H */
