#ifndef QWN_HIP_DECODER_H
#define QWN_HIP_DECODER_H

/*
 * Resident greedy decoder on one MI355X (extension; no counterpart in
 * c/cuda/qwn_cuda_abi.h).
 *
 * The reference host runs the dense decoder step on the CPU and calls the
 * GPU ABI once per projection and KV operation, synchronously, with host
 * buffers (c/qwanto_decode.c:776-924, :1657-1724).  This decoder keeps the
 * whole step on the device: the residual stream, RMSNorm, RoPE, the Q8 KV
 * cache, SwiGLU, the tied F16 LM head and the greedy argmax, with the same
 * semantics as the reference forward/generate (c/qwanto_decode.c:1566-2032,
 * 2043-2125).  One step is a fixed sequence of kernels that read the token
 * and position from device memory, captured once as a HIP graph; a greedy
 * generation replays it without host synchronisation between tokens.
 *
 * Weights are the tensors of qwn_cuda_abi.h, already uploaded to the same
 * context (qwn_cuda_abi_upload_tensor): seven projections per layer
 * (HyperVSQ-2 or Q4_0, one dtype per decoder), the F16 or BF16 embedding
 * (c/qwanto_decode.c:561), which is also the LM head unless an untied
 * lm_head tensor is given.  Norm weights are copied from the host at
 * creation, and so are the optional per-head q/k norm weights of Qwen3
 * layers and the optional q/k/v/o projection biases.
 */

#include "qwn_cuda_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    QwnCudaAbiHeader header;
    uint32_t hidden;
    uint32_t intermediate;
    uint32_t layers;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t vocab;
    uint32_t max_ctx;         /* KV-cache capacity in tokens */
    float rope_theta;
    float rms_eps;
    const QwnCudaTensorHandle *projections; /* [layers * 7]: q, k, v, o, gate, up, down */
    const QwnCudaTensorHandle *embedding;   /* F16 or BF16 [vocab][hidden] */
    const float *input_norms;               /* host [layers][hidden] */
    const float *post_norms;                /* host [layers][hidden] */
    const float *final_norm;                /* host [hidden] */
    const float *q_norms;                   /* NULL, or host [layers][head_dim]: Qwen3 per-head q norm */
    const float *k_norms;                   /* NULL, or host [layers][head_dim]: Qwen3 per-head k norm
                                               (self_attn.q_norm / k_norm, c/qwanto_decode.c:975-976,
                                               1652-1655; both or neither) */
    /* Optional projection biases (self_attn.{q,k,v,o}_proj.bias; Qwen2
     * checkpoints carry q/k/v biases), each NULL or host [layers][rows of
     * that projection]: added to the projection's output as the reference's
     * add_bias (c/qwanto_decode.c:926-929, 1649-1651, 1722). */
    const float *q_biases;                  /* [layers][heads * head_dim] */
    const float *k_biases;                  /* [layers][kv_heads * head_dim] */
    const float *v_biases;                  /* [layers][kv_heads * head_dim] */
    const float *o_biases;                  /* [layers][hidden] */
    /* Optional untied LM head (lm_head.weight / output.weight,
     * c/qwanto_decode.c:1074-1076): NULL, the embedding is the head; else a
     * [vocab][hidden] tensor in F16, BF16, Q4_0 or HyperVSQ-2 (the quantized
     * kinds quantize the final-norm output per token, as every quantized
     * projection does, c/qwanto_decode.c:2007). */
    const QwnCudaTensorHandle *lm_head;
} QwnHipDecoderDesc;

typedef struct {
    QwnCudaAbiHeader header;
    void *opaque;
} QwnHipDecoderHandle;

typedef struct {
    QwnCudaAbiHeader header;
    uint32_t prompt_tokens;
    uint32_t generated_tokens;
    uint32_t position;            /* tokens in the KV cache */
    uint32_t launches_per_step;   /* kernels in one step */
    double prefill_ms;            /* wall clock, prompt steps */
    double decode_ms;             /* wall clock, generated steps */
    uint64_t weight_bytes_per_step; /* algorithmic weight bytes one step reads */
    uint32_t graph;               /* 1 if steps replay a captured HIP graph */
    uint32_t prefill_block_tokens; /* prompt tokens per prefill block */
} QwnHipDecoderStats;

QWN_CUDA_ABI_API int qwn_hip_decoder_create(QwnCudaContextHandle *context, const QwnHipDecoderDesc *desc,
                                            QwnHipDecoderHandle *out);
QWN_CUDA_ABI_API int qwn_hip_decoder_destroy(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder);
/* Empties the KV cache (position 0). */
QWN_CUDA_ABI_API int qwn_hip_decoder_reset(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder);
/* One step on `token` at the current position (synchronous).  `logits`
 * (vocab floats) and `next_token` (the greedy choice) may be NULL. */
QWN_CUDA_ABI_API int qwn_hip_decoder_forward(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                             int32_t token, float *logits, int32_t *next_token);
/* `count` prompt tokens at the current position in prefill blocks of up to
 * 16 tokens: each projection of a block is one batched GEMV (the weights
 * are read once per block instead of once per token), then RoPE, the Q8
 * append and causal attention per token.  Same cache contents and, up to
 * the fp32 summation order of the norms, the same logits as `count`
 * forward() calls (c/qwanto_decode.c:2093 steps the prompt token by token).
 * `logits` / `next_token`: those of the last token (may be NULL). */
QWN_CUDA_ABI_API int qwn_hip_decoder_prefill(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                             const int32_t *tokens, uint32_t count, float *logits,
                                             int32_t *next_token);
/* Speculative-decoding verification: `count` (1..16) draft tokens at the
 * current position as one block (as qwn_hip_decoder_prefill), with the tied
 * LM head run on EVERY token of the block in one batched F16 GEMV:
 * logits [count][vocab] (host, may be NULL) are the logits after each
 * token, next_tokens[count] (may be NULL) the greedy choice after each --
 * the [nodes x vocab] scores a draft-tree verifier consumes
 * (c/qwanto_jetspec.c:160-205), where the reference steps its target model
 * token by token (c/qwn_speculative.c:389-433).  The cache then holds all
 * `count` tokens; qwn_hip_decoder_truncate drops the rejected ones. */
QWN_CUDA_ABI_API int qwn_hip_decoder_verify(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                            const int32_t *tokens, uint32_t count, float *logits,
                                            int32_t *next_tokens);
/* Speculative verification of a draft TREE (c/qwanto_jetspec.h:17-33):
 * `count` (1..64) nodes after the cached prefix of P tokens, node i =
 * (tokens[i], parents[i]) with parents[i] an earlier node or -1 (a root,
 * attached to the prefix).  One forward over the nodes in index order (one
 * block of up to 64 on the int8-MFMA path, else blocks of 16): node i is
 * rotated for position P + depth(i), its K/V held
 * at cache slot P + i, and it attends to the prefix, its ancestors and
 * itself (the ancestor mask of qwn_jetspec_build_tree_mask,
 * c/qwanto_jetspec.c:33-49).  logits [count][vocab] (host, may be NULL) are
 * the target's logits after each node -- the prediction for its children --
 * and next_tokens[count] (may be NULL) their first maxima.  The rows
 * qwn_jetspec_verify_tree reads (c/qwanto_jetspec.c:160-205: row i is the
 * target's prediction FOR node i) are the logits of node i's parent, or,
 * for a root, the logits after the prefix's last token.  The position stays
 * at P: qwn_hip_decoder_commit_path keeps an accepted path, and any other
 * call drops the tree. */
QWN_CUDA_ABI_API int qwn_hip_decoder_verify_tree(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                                 const int32_t *tokens, const int32_t *parents, uint32_t count,
                                                 float *logits, int32_t *next_tokens);
/* After qwn_hip_decoder_verify_tree: keeps the root-to-node path
 * nodes[0..length) (nodes[0] a root, nodes[k] a child of nodes[k-1]) --
 * their K/V, as the tree forward computed them, move to cache slots
 * P .. P + length - 1 -- drops the other nodes, and moves the position to
 * P + length. */
QWN_CUDA_ABI_API int qwn_hip_decoder_commit_path(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                                 const uint32_t *nodes, uint32_t length);
/* Keep the first `position` cached tokens (position <= the current one):
 * the next step writes at `position`. */
QWN_CUDA_ABI_API int qwn_hip_decoder_truncate(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                              uint32_t position);
/* Greedy generation as c/qwanto_decode.c:2085-2125: the prompt (in prefill
 * blocks, as qwn_hip_decoder_prefill), then max_new times: tokens[s] =
 * argmax of the last logits, one step on it.  Synchronises once after the
 * prompt and once at the end. */
QWN_CUDA_ABI_API int qwn_hip_decoder_generate(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                              const int32_t *prompt, uint32_t prompt_count, uint32_t max_new,
                                              int32_t *tokens, QwnHipDecoderStats *stats);

/* Debug: cached tokens [first, first + count) of layer `layer`'s Q8 KV cache
 * in the CPU cache's token-major layout (c/qwanto_turboquant.h:78-94):
 * keys/values [count][kv_heads*head_dim] int8, scales [count][groups] fp32
 * (host pointers, synchronous). */
QWN_CUDA_ABI_API int qwn_hip_decoder_debug_kv_read(QwnCudaContextHandle *context, QwnHipDecoderHandle *decoder,
                                                   uint32_t layer, uint32_t first, uint32_t count, int8_t *keys,
                                                   int8_t *values, float *key_scales, float *value_scales);

#ifdef __cplusplus
}
#endif

#endif /* QWN_HIP_DECODER_H */
