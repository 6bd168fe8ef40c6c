#ifndef QWN_HOST_DECODER_H
#define QWN_HOST_DECODER_H

/*
 * Host-side dense decoder over the qwn_cuda ABI (libqwn_host_decoder.so).
 *
 * The host half of qwnrun's GPU decode path, restated: ABI bring-up
 * (c/qwanto_decode.c:267-462: dlopen of qwn_cuda.so next to this library,
 * symbol resolution, version/capability checks, context creation), the
 * matmul dispatch (:776-924: lazy upload cached per tensor, host-side int8
 * activation quantization, one synchronous ABI call per projection,
 * telemetry mirrored into metrics, fail-closed), the Q8 KV calls
 * (:1657-1724) and the forward / greedy generate semantics
 * (:1566-2032, :2085-2125) of a dense Qwen2-style model.  Q4_0, F16 and
 * BF16 tensors are routed through the ABI too (the library's extra dtypes),
 * so every projection and the LM head (tied, or lm_head.weight in any of
 * those dtypes) run on the GPU.
 *
 * There is no CPU fallback: if the ABI library is missing or refuses a
 * call, the call fails and last_error says why.
 */

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QHD_PROJ_HVSQ2 1 /* 74-byte HyperVSQ-2 blocks */
#define QHD_PROJ_Q4_0 2  /* 18-byte Q4_0 blocks */

/* dtypes of the embedding (F16, BF16) and of an untied LM head (any) */
#define QHD_DT_F16 1
#define QHD_DT_Q4_0 2
#define QHD_DT_BF16 4
#define QHD_DT_HVSQ2 9

typedef struct {
    int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab, max_ctx;
    float rope_theta, rms_eps;
    int proj_dtype; /* QHD_PROJ_* */
} QhdConfig;

/* Host weights (row-major [out][in] blocks; kept alive by the caller). */
typedef struct {
    QhdConfig cfg;
    const uint16_t *embed;      /* [vocab][hidden] in embed_dtype; the LM head when lm_head is NULL */
    const float *final_norm;    /* [hidden] */
    const uint8_t *const *proj; /* [layers * 7]: q k v o gate up down */
    const float *const *norms;  /* [layers * 2]: input, post-attention */
    const float *const *qk_norms; /* NULL, or [layers * 2]: per-head q and k RMSNorm weights
                                     [head_dim] (self_attn.q_norm / k_norm,
                                     c/qwanto_decode.c:654-684, 1652-1655) */
    const float *const *biases;   /* NULL, or [layers * 4]: q, k, v, o projection biases
                                     (self_attn.*_proj.bias), each NULL or [rows]
                                     (c/qwanto_decode.c:926-929, 1649-1651, 1722) */
    int embed_dtype;              /* QHD_DT_F16 (also 0) or QHD_DT_BF16 (c/qwanto_decode.c:561) */
    const void *lm_head;          /* NULL (tied), or lm_head.weight [vocab][hidden] in lm_head_dtype
                                     (c/qwanto_decode.c:1074-1076) */
    int lm_head_dtype;            /* QHD_DT_F16 / QHD_DT_BF16 / QHD_DT_Q4_0 / QHD_DT_HVSQ2 */
} QhdModel;

typedef struct {
    uint64_t gpu_matmul_count;    /* telemetry.gpu_matmul_count */
    uint64_t cpu_fallback_count;  /* always 0: no fallback exists */
    uint64_t gpu_kernel_launch_count;
    uint64_t gpu_upload_bytes;
    uint64_t gpu_resident_bytes;
    uint64_t kv_cache_kernel_count;
    uint64_t abi_calls;           /* synchronous ABI round trips */
    double gpu_kernel_ms, gpu_transfer_ms, gpu_sync_ms;
    double prefill_ms, decode_wall_ms;
    int prompt_tokens, generated_tokens;
    char kernel_type[32];
    /* why the ABI library was accepted or refused: the reference loader's
     * cuda_backend_reason strings (c/qwanto_decode.c:323-461), e.g.
     * "qwn_cuda_dll_absent_from_runtime_directory",
     * "qwn_cuda_dll_missing_versioned_abi_1",
     * "abi_capability_or_hypervsq2_layout_rejected",
     * "cuda_q8_kv_capability_unavailable", "cuda_capability_query_failed",
     * "cuda_device_index_<n>_not_enumerated",
     * "cuda_context_creation_failed_device_<n>",
     * "versioned_abi_1_loaded_device_<n>"; plus this decoder's own
     * "qwn_hip_q4_0_f16_capability_unavailable" (it routes Q4_0 and F16
     * tensors through the ABI) */
    char backend_reason[96];
} QhdMetrics;

typedef struct QhdDecoder QhdDecoder;

/* abi_path: the ABI library to load; NULL = "qwn_cuda.so" in the directory
 * of this library (the reference loader's rule).  On failure returns NULL
 * with the message in `error` and, when `reason` is not NULL, the
 * backend_reason string in `reason` (96 bytes). */
QhdDecoder *qhd_open(const QhdModel *model, const char *abi_path, int device, char *error,
                     int error_len, char *reason);
void qhd_close(QhdDecoder *d);
/* One forward step; logits_out (vocab floats) may be NULL. */
int qhd_forward(QhdDecoder *d, int token, float *logits_out);
/* Greedy generation: tokens[max_new], margins[max_new] (best minus
 * second-best logit; may be NULL).  Returns the number generated. */
int qhd_generate(QhdDecoder *d, const int *prompt, int prompt_count, int max_new, int *tokens,
                 float *margins);
int qhd_metrics(const QhdDecoder *d, QhdMetrics *out);
const char *qhd_last_error(const QhdDecoder *d);

#ifdef __cplusplus
}
#endif

#endif /* QWN_HOST_DECODER_H */
