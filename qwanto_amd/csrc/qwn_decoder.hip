// Resident greedy decoder (include/qwn_hip_decoder.h).
//
// One decode step is a fixed kernel sequence that reads the input token and
// the position from device memory, so it is captured once as a HIP graph and
// replayed for every token.  Per layer (dense Qwen2-style, semantics of
// c/qwanto_decode.c:1566-2032):
//
//   q,k,v   = W_qkv rmsnorm(x)        one grouped GEMV: every workgroup
//                                     normalizes and int8-quantizes x itself
//   RoPE(q, k); Q8 append of k, v     one workgroup
//   ctx     = attention over the Q8 cache (split-T partials + merge)
//   x      += W_o ctx                 GEMV quantizing ctx in its prologue,
//                                     residual added in its epilogue
//   h       = silu(W_g rmsnorm(x)) * W_u rmsnorm(x)
//                                     grouped GEMV, gate and up rows paired
//                                     in each workgroup, SwiGLU in the epilogue
//   x      += W_down h                GEMV quantizing h in its prologue
//
// then logits = E rmsnorm(x) (F16 tied LM head, per-workgroup argmax
// partials in the epilogue) and one kernel that picks the greedy token,
// records it and advances the position.  Nothing crosses PCIe per token.
#include "qwn_context.h"
#include "qwn_device.h"
#include "qwn_hip_decoder.h"
#include "qwn_internal.h"

#include <chrono>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

namespace qwn {

namespace {

constexpr int kProj = 7;
constexpr uint32_t kPrefillTokens = 16;  // tokens of a chain verify block (the GEMV's widest launch)
constexpr uint32_t kBlockTokens = 64;    // tokens of a prompt / draft-tree block (MFMA GEMMs of 16-token groups)
constexpr uint32_t kTreeNodes = 64;      // draft-tree nodes per verify (c/qwanto_jetspec.h:17)
constexpr uint32_t kTreeBlocks = kTreeNodes / kPrefillTokens;  // blocks of the narrowest block size
enum { P_Q, P_K, P_V, P_O, P_GATE, P_UP, P_DOWN };

// x = embedding row of the step's token (feed[pos] when the host supplied
// one, else the previous step's greedy choice): F16 or BF16 -> fp32 straight
// from the embedding's wave-tile layout.  One thread per 8 values.
struct EmbedArgs {
    const uint8_t *payload;
    size_t tile_payload;
    uint32_t lanes, rows_per_wave, units, hidden, vocab, max_ctx;
    uint32_t bf16;  // BF16 rows (c/qwanto_decode.c:561): the 16 bits are the high half
    const int32_t *feed;
    const int32_t *state;  // [0] = last greedy token, [1] = position
    float *x;
    // RoPE: the table rows of the step's position copied to rope_row
    // ([cos | sin], 2 * half floats) for the attention kernels to read at a
    // fixed address
    const float *cos_tab, *sin_tab;
    uint32_t half;
    float *rope_row;
};

__device__ __forceinline__ float embed_value(uint32_t raw, uint32_t bf16) {
    return bf16 ? __builtin_bit_cast(float, raw << 16) : half_to_float(raw);
}

__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int32_t pos = a.state[1];
    if (idx < 2 * a.half) {
        const uint32_t row = (pos >= 0 && static_cast<uint32_t>(pos) < a.max_ctx) ? static_cast<uint32_t>(pos) : 0u;
        const float *tab = idx < a.half ? a.cos_tab : a.sin_tab;
        a.rope_row[idx] = tab[static_cast<size_t>(row) * a.half + idx % a.half];
    }
    if (idx >= a.units * 4) return;
    int32_t token = (pos >= 0 && static_cast<uint32_t>(pos) < a.max_ctx) ? a.feed[pos] : -1;
    if (token < 0) token = a.state[0];
    if (token < 0 || static_cast<uint32_t>(token) >= a.vocab) token = 0;
    const uint32_t u = idx / 4, q = idx % 4;
    const UnitAddr ad = unit_addr(static_cast<uint32_t>(token), u, q, a.lanes, a.rows_per_wave, a.units,
                                  a.tile_payload, 0);
    const uint4 h = *reinterpret_cast<const uint4 *>(a.payload + ad.payload);
    const uint32_t w[4] = {h.x, h.y, h.z, h.w};
    const uint32_t k0 = u * 32 + q * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (k0 + e < a.hidden) a.x[k0 + e] = embed_value((w[e >> 1] >> (16 * (e & 1))) & 0xffffu, a.bf16);
}

// Prefill block: x[i] = embedding row of feed[p0 + i] for the block's
// tokens i < count (p0 = the device position), and the positions p0 + i
// recorded for the block's kernels.  grid (ceil(units*4 / 256), count).
__global__ __launch_bounds__(256) void prefill_embed_kernel(EmbedArgs a, uint32_t count, float *x,
                                                            int32_t *positions) {
    const uint32_t i = blockIdx.y;
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int32_t pos = a.state[1] + static_cast<int32_t>(i);
    if (idx == 0) positions[i] = pos;
    if (idx >= a.units * 4) return;
    int32_t token = (pos >= 0 && static_cast<uint32_t>(pos) < a.max_ctx) ? a.feed[pos] : -1;
    if (token < 0 || static_cast<uint32_t>(token) >= a.vocab) token = 0;
    const uint32_t u = idx / 4, q = idx % 4;
    const UnitAddr ad = unit_addr(static_cast<uint32_t>(token), u, q, a.lanes, a.rows_per_wave, a.units,
                                  a.tile_payload, 0);
    const uint4 h = *reinterpret_cast<const uint4 *>(a.payload + ad.payload);
    const uint32_t w[4] = {h.x, h.y, h.z, h.w};
    const uint32_t k0 = u * 32 + q * 8;
    float *xi = x + static_cast<size_t>(i) * a.hidden;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (k0 + e < a.hidden) xi[k0 + e] = embed_value((w[e >> 1] >> (16 * (e & 1))) & 0xffffu, a.bf16);
}

// End of a prefill block: the device position moves past the block, or, in
// the block that ends the prompt, to its last token, which the greedy step
// end then records and passes.
__global__ void prefill_advance_kernel(int32_t *state, const int32_t *positions, uint32_t count, uint32_t last) {
    if (blockIdx.x == 0 && threadIdx.x == 0) state[1] = positions[count - 1] + (last ? 0 : 1);
}

// Greedy token of the step (largest logit, first index on ties), recorded
// at out_tokens[pos]; the position advances.  One workgroup.
__global__ __launch_bounds__(1024) void step_end_kernel(const uint64_t *__restrict__ partials, uint32_t n,
                                                        int32_t *state, int32_t *out_tokens, uint32_t max_ctx) {
    __shared__ uint64_t red[1024 / kWaveSize];
    uint64_t key = 0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) key = partials[i] > key ? partials[i] : key;
    for (int off = kWaveSize / 2; off > 0; off >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(key), off);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(key >> 32), off);
        const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
        key = o > key ? o : key;
    }
    if (threadIdx.x % kWaveSize == 0) red[threadIdx.x / kWaveSize] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t best = red[0];
        for (uint32_t w = 1; w < blockDim.x / kWaveSize; ++w) best = red[w] > best ? red[w] : best;
        const int32_t token = best ? static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(best)) : 0;
        const int32_t pos = state[1];
        if (pos >= 0 && static_cast<uint32_t>(pos) < max_ctx) out_tokens[pos] = token;
        state[0] = token;
        state[1] = pos + 1;
    }
}

}  // namespace

struct Decoder {
    Context *ctx = nullptr;
    uint32_t hidden = 0, inter = 0, layers = 0, heads = 0, kv_heads = 0, head_dim = 0, vocab = 0, max_ctx = 0;
    float eps = 0.0f, attn_scale = 0.0f;
    std::vector<const DeviceTensor *> proj;
    const DeviceTensor *embed = nullptr;
    const DeviceTensor *head = nullptr;  // the LM head: an untied lm_head tensor, or embed
    void *allocation = nullptr;
    float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *gate = nullptr,
          *up = nullptr, *logits = nullptr, *partials = nullptr;
    float *norms_in = nullptr, *norms_post = nullptr, *final_norm = nullptr, *cos_tab = nullptr,
          *sin_tab = nullptr, *rope_row = nullptr;
    float *q_norms = nullptr, *k_norms = nullptr;  // [layers][head_dim] or null
    float *bias[4] = {};                           // q, k, v, o: [layers][rows] or null
    uint64_t *argmax = nullptr;
    uint32_t argmax_n = 0;
    int32_t *state = nullptr, *feed = nullptr, *out_tokens = nullptr;
    std::vector<KvCache> caches;
    hipGraphExec_t exec = nullptr;
    bool graph_tried = false;
    // prefill: blocks of up to block_tokens prompt tokens (kBlockTokens on
    // the MFMA path, else kPrefillTokens) through the GEMMs ([token][...]
    // buffers), one graph per (block size, ends the prompt)
    float *px = nullptr, *pq = nullptr, *pk = nullptr, *pv = nullptr, *pattn = nullptr, *pgate = nullptr,
          *pup = nullptr, *pscales = nullptr;
    uint8_t *pimg = nullptr;
    uint32_t pimg_stride = 0;
    // blocks that mfma_batch() sends through the int8 MFMA GEMM: the MFMA
    // image of the widest input, written by the quantize step
    uint8_t *pmimg = nullptr;
    int32_t *ppos = nullptr;
    // verify blocks: the LM head on every token of the block
    float *vlogits = nullptr;       // [kTreeNodes][vocab]
    int32_t *vids = nullptr;        // [kTreeNodes] greedy id after each token
    uint64_t *row_keys = nullptr;   // [kBlockTokens][rows_argmax_parts(vocab)] argmax workspace
    uint8_t *vimg = nullptr;        // [kBlockTokens][vimg_stride] fp32 LM-head images
    uint8_t *hpieces = nullptr;     // F16/BF16 head on the matrix cores: the block's activation pieces
    float *hunscale = nullptr;      // [kBlockTokens] their per-token unscale factors
    uint32_t vimg_stride = 0;
    // one graph per (block size, block kind: inner / ends the prompt / verify)
    uint32_t block_tokens = kPrefillTokens;
    hipGraphExec_t prefill_exec[kBlockTokens + 1][3] = {};
    bool prefill_tried[kBlockTokens + 1][3] = {};
    // draft trees: per node its ancestor-or-self mask and rotation position
    // (prefix length + depth), the prefix length, an accepted path; one
    // graph per (block of the tree, block size)
    uint64_t *tree_mask = nullptr;  // [kTreeNodes]
    int32_t *tree_pos = nullptr;    // [kTreeNodes]
    int32_t *tree_base = nullptr;   // [1]
    int32_t *tree_path = nullptr;   // [kTreeNodes]
    hipGraphExec_t tree_exec[kTreeBlocks][kBlockTokens + 1] = {};
    bool tree_tried[kTreeBlocks][kBlockTokens + 1] = {};
    uint32_t tree_nodes = 0;        // nodes of the verified tree awaiting commit (0: none)
    std::vector<int32_t> tree_parents, tree_tokens;
    uint32_t position = 0;
    uint32_t launches = 0;
    uint32_t layer_launches = 0;  // kernels per layer
    bool fused_attention = false; // RoPE + append + attention in one kernel
    uint64_t weight_bytes = 0;
};

void destroy_decoder(Decoder *d) {
    if (!d) return;
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    for (auto &row : d->prefill_exec)
        for (hipGraphExec_t x : row)
            if (x) (void)hipGraphExecDestroy(x);
    for (auto &row : d->tree_exec)
        for (hipGraphExec_t x : row)
            if (x) (void)hipGraphExecDestroy(x);
    if (d->allocation) (void)hipFree(d->allocation);
    delete d;
}

namespace {

Decoder *decoder_of(Context *ctx, const QwnHipDecoderHandle *h) {
    if (!h || !header_ok(*h) || !h->opaque) return nullptr;
    auto *d = static_cast<Decoder *>(h->opaque);
    return std::find(ctx->decoders.begin(), ctx->decoders.end(), d) != ctx->decoders.end() ? d : nullptr;
}

// Bias of projection p (P_Q .. P_O) in layer l, or null.
const float *layer_bias(const Decoder *d, uint32_t l, int p) {
    if (!d->bias[p]) return nullptr;
    const uint32_t rows = p == P_O ? d->hidden : (p == P_Q ? d->heads : d->kv_heads) * d->head_dim;
    return d->bias[p] + static_cast<size_t>(l) * rows;
}

GemvGroupLaunch group(std::initializer_list<const DeviceTensor *> ts, std::initializer_list<float *> outs) {
    GemvGroupLaunch g;
    for (const DeviceTensor *t : ts) g.tensors[g.njobs++] = t;
    int i = 0;
    for (float *o : outs) g.outputs[i++] = o;
    return g;
}

EmbedArgs embed_args(const Decoder *d) {
    EmbedArgs ea{};
    ea.payload = d->embed->payload;
    ea.tile_payload = d->embed->tile_payload_bytes;
    ea.lanes = d->embed->lanes;
    ea.rows_per_wave = d->embed->rows_per_wave;
    ea.units = d->embed->units;
    ea.hidden = d->hidden;
    ea.vocab = d->vocab;
    ea.max_ctx = d->max_ctx;
    ea.feed = d->feed;
    ea.state = d->state;
    ea.x = d->x;
    ea.cos_tab = d->cos_tab;
    ea.sin_tab = d->sin_tab;
    ea.half = d->head_dim / 2;
    ea.rope_row = d->rope_row;
    ea.bf16 = d->embed->bf16 ? 1u : 0u;
    return ea;
}

// The LM head launch of one token, with per-workgroup argmax partials.  The
// final RMSNorm runs in the head's own prologue in every workgroup (F16 and
// BF16 heads keep the normalized values in fp32, Q4_0 and HyperVSQ-2 heads
// quantize them, as the projections do): one launch fewer per token than a
// separate norm kernel writing an fp32 image, 1211 -> 1217 tok/s on the
// Qwen2-1.5B-shaped F16-head decode.
GemvGroupLaunch head_launch(const Decoder *d, const float *x) {
    GemvGroupLaunch head = group({d->head}, {d->logits});
    head.input_mode = kInNorm;
    head.x = x;
    head.norm = d->final_norm;
    head.eps = d->eps;
    head.output_mode = kOutArgmax;
    head.argmax_partials = d->argmax;
    return head;
}

// The LM head on the fp32 residual x (c/qwanto_decode.c:2000-2007) and the
// step end that records the greedy token at the device position and
// advances it.
hipError_t enqueue_head(Decoder *d, const float *x, hipStream_t s) {
    hipError_t e;
    if ((e = launch_gemv_group(head_launch(d, x), s)) != hipSuccess) return e;
    hipLaunchKernelGGL(step_end_kernel, dim3(1), dim3(1024), 0, s, d->argmax, d->argmax_n, d->state,
                       d->out_tokens, d->max_ctx);
    return hipGetLastError();
}

// What follows the layers of a prefill block.  kBlockTree: 16 nodes of a
// draft tree (block `block` of it), the LM head on each as kBlockVerify.
enum BlockKind : uint32_t { kBlockInner = 0, kBlockLast = 1, kBlockVerify = 2, kBlockTree = 3 };

// One prefill block of `m` prompt tokens at the device position (their ids
// in feed): per layer the projections of all m tokens in one batched GEMV
// each (weights read once per launch), RoPE and the Q8 append of the m
// keys/values, causal attention of every token over the cache up to its
// own position, residual adds in the GEMV epilogues.  kBlockLast: the block
// ends the prompt, so the LM head runs on its last token and the greedy
// token is recorded as a decode step would.  kBlockVerify: the LM head runs
// on every token of the block (one batched F16 GEMV, the head's weights
// read once), logits [m][vocab] and each token's greedy successor; the
// device position moves past the block and the last token's greedy id is
// recorded as the step's.  kBlockTree: nodes 16 * block + i of a draft tree
// (their ids in feed at the device position, which is the tree's base slot
// plus 16 * block): each rotated for its position (prefix length + depth,
// tree_pos), appended at its slot, attending to the prefix and its
// ancestor-or-self slots (tree_mask); the head as kBlockVerify, into rows
// 16 * block + i of vlogits / vids; the device position moves past the block.
hipError_t enqueue_prefill(Decoder *d, uint32_t m, uint32_t kind, hipStream_t s, uint32_t block = 0) {
    const bool last = kind == kBlockLast;
    const bool tree = kind == kBlockTree;
    const uint32_t row0 = tree ? block * d->block_tokens : 0;
    hipError_t e;
    const EmbedArgs ea = embed_args(d);
    hipLaunchKernelGGL(prefill_embed_kernel, dim3((ea.units * 4 + 255) / 256, m), dim3(256), 0, s, ea, m, d->px,
                       d->ppos);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const uint32_t D = d->hidden, Q = d->heads * d->head_dim, I = d->inter;
    // one projection group of the block: its input prepared per token
    // (mode: fp32 / RMSNorm / SwiGLU of x), then the batched dot8 GEMV on
    // activation images, or where mfma_batch() says so the int8 MFMA GEMM
    // on the MFMA image; add: residual stream
    const bool mfma = d->pmimg && mfma_batch(d->proj[P_Q]->kind, m, d->proj[P_Q]->mfma_payload != nullptr);
    // swiglu (MFMA, gate/up with the MFMA-order copy): outs[0] = silu(gate) * up
    auto project = [&](std::initializer_list<const DeviceTensor *> ts, std::initializer_list<float *> outs,
                       uint32_t mode, const float *x, const float *x2, const float *norm, uint32_t x_stride,
                       bool add, std::initializer_list<const float *> biases, bool swiglu = false) {
        const float *bv[kMaxGroup] = {};
        {
            uint32_t n = 0;
            for (const float *b : biases) bv[n++] = b;
        }
        const DeviceTensor &t0 = **ts.begin();
        hipError_t e2;
        if (mfma) {
            if ((e2 = launch_prepare_image(t0, mode, x, x2, norm, d->eps, m, x_stride, nullptr, 0, d->pscales,
                                           nullptr, 0, s, d->pmimg)) != hipSuccess)
                return e2;
            const DeviceTensor *tv[kMaxGroup];
            float *ov[kMaxGroup];
            uint32_t n = 0;
            for (const DeviceTensor *t : ts) tv[n++] = t;
            n = 0;
            for (float *o : outs) ov[n++] = o;
            return launch_gemm_mfma_group(tv, ov, n, d->pmimg, d->pscales, m, nullptr, s, add, nullptr, bv, swiglu);
        }
        if ((e2 = launch_prepare_image(t0, mode, x, x2, norm, d->eps, m, x_stride, d->pimg, d->pimg_stride,
                                       d->pscales, nullptr, 0, s)) != hipSuccess)
            return e2;
        GemvGroupLaunch g = group(ts, outs);
        g.input_mode = kInImage;
        g.output_mode = add ? kOutAdd : kOutStore;
        g.image = d->pimg;
        g.image_stride = d->pimg_stride;
        g.scales = d->pscales;
        g.batch = m;
        for (int i = 0; i < kMaxGroup; ++i) g.bias[i] = bv[i];
        return launch_gemv_group(g, s);
    };
    for (uint32_t l = 0; l < d->layers; ++l) {
        const DeviceTensor *const *w = d->proj.data() + static_cast<size_t>(l) * kProj;
        const float *nin = d->norms_in + static_cast<size_t>(l) * D;
        const float *npost = d->norms_post + static_cast<size_t>(l) * D;
        const float *qn = d->q_norms ? d->q_norms + static_cast<size_t>(l) * d->head_dim : nullptr;
        const float *kn = d->k_norms ? d->k_norms + static_cast<size_t>(l) * d->head_dim : nullptr;
        if ((e = project({w[P_Q], w[P_K], w[P_V]}, {d->pq, d->pk, d->pv}, kInNorm, d->px, nullptr, nin, D, false,
                         {layer_bias(d, l, P_Q), layer_bias(d, l, P_K), layer_bias(d, l, P_V)})) != hipSuccess ||
            (e = launch_rope_append(d->caches[l], d->pq, d->heads, d->pk, d->pv, d->cos_tab, d->sin_tab, d->ppos, s,
                                    m, qn, kn, d->eps, tree ? d->tree_pos + row0 : nullptr)) != hipSuccess)
            return e;
        if (d->fused_attention) {
            DecodeAttentionLaunch at;
            at.cache = &d->caches[l];
            at.query = d->pq;
            at.output = d->pattn;
            at.partials = d->partials;
            at.query_heads = d->heads;
            at.position_ptr = d->ppos;
            at.span_tokens = d->max_ctx;
            at.scale = d->attn_scale;
            at.count = m;
            if (tree) {
                at.tree_mask = d->tree_mask + row0;
                at.tree_base = d->tree_base;
            }
            if ((e = launch_decode_attention(at, s)) != hipSuccess) return e;
        } else {
            for (uint32_t i = 0; i < m; ++i)
                if ((e = launch_attention_at(d->caches[l], d->pq + static_cast<size_t>(i) * Q,
                                             d->pattn + static_cast<size_t>(i) * Q, d->heads, d->ppos + i,
                                             d->attn_scale, d->partials, s, tree ? d->tree_mask + row0 + i : nullptr,
                                             tree ? d->tree_base : nullptr)) != hipSuccess)
                    return e;
        }
        // on the MFMA path with the MFMA-order copy the gate/up launch stores
        // silu(gate) * up itself, and the down input is quantized as is
        const bool pair = mfma && w[P_GATE]->mfma_payload && w[P_GATE]->mfma_meta && w[P_UP]->mfma_payload &&
                          w[P_UP]->mfma_meta;
        if ((e = project({w[P_O]}, {d->px}, kInF32, d->pattn, nullptr, nullptr, Q, true,
                         {layer_bias(d, l, P_O)})) != hipSuccess ||
            (e = project({w[P_GATE], w[P_UP]}, {d->pgate, d->pup}, kInNorm, d->px, nullptr, npost, D, false, {},
                         pair)) != hipSuccess ||
            (e = project({w[P_DOWN]}, {d->px}, pair ? kInF32 : kInSwiglu, d->pgate, pair ? nullptr : d->pup, nullptr,
                         I, true, {})) != hipSuccess)
            return e;
    }
    hipLaunchKernelGGL(prefill_advance_kernel, dim3(1), dim3(64), 0, s, d->state, d->ppos, m, last ? 1u : 0u);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (last) return enqueue_head(d, d->px + static_cast<size_t>(m - 1) * D, s);
    if (kind == kBlockVerify || tree) {
        // the head on every token: F16/BF16 rows on the matrix cores (the
        // normed tokens as narrow pieces, the head read once for the block)
        // where the pieces fit, else fp32 images (F16/BF16) or per-token int8
        // images of the normalized tokens (Q4_0/HyperVSQ-2), one batched GEMV
        float *vl = d->vlogits + static_cast<size_t>(row0) * d->vocab;
        if (d->hpieces) {
            // up to 32 tokens per head launch (the head read once per launch)
            for (uint32_t t0 = 0; t0 < m; t0 += 2 * kPrefillTokens) {
                const uint32_t mg = std::min(2 * kPrefillTokens, m - t0);
                if ((e = launch_head_pieces(*d->head, d->px + static_cast<size_t>(t0) * D, D, d->final_norm, d->eps,
                                            mg, d->hpieces, d->hunscale + t0, s)) != hipSuccess ||
                    (e = launch_mfma_head(*d->head, d->hpieces, d->hunscale + t0, mg,
                                          vl + static_cast<size_t>(t0) * d->vocab, d->vocab, s)) != hipSuccess)
                    return e;
            }
            return launch_rows_argmax(vl, m, d->vocab, d->vocab, d->vids + row0, d->state, d->row_keys, s);
        }
        if (d->head->kind == kF16)
            e = launch_norm_image(*d->head, d->px, d->final_norm, d->eps, d->vimg, s, m, D, d->vimg_stride);
        else
            e = launch_prepare_image(*d->head, kInNorm, d->px, nullptr, d->final_norm, d->eps, m, D, d->vimg,
                                     d->vimg_stride, d->pscales, nullptr, 0, s);
        if (e != hipSuccess) return e;
        GemvGroupLaunch head = group({d->head}, {d->vlogits + static_cast<size_t>(row0) * d->vocab});
        head.image = d->vimg;
        head.image_stride = d->vimg_stride;
        if (d->head->kind != kF16) head.scales = d->pscales;
        head.batch = m;
        head.output_stride[0] = d->vocab;
        if ((e = launch_gemv_group(head, s)) != hipSuccess) return e;
        return launch_rows_argmax(d->vlogits + static_cast<size_t>(row0) * d->vocab, m, d->vocab, d->vocab,
                                  d->vids + row0, d->state, d->row_keys, s);
    }
    return hipSuccess;
}

// The launches of one step, in order; `count` only counts them.
hipError_t enqueue_step(Decoder *d, hipStream_t s, uint32_t *count) {
    uint32_t n = 0;
    hipError_t e;
    const EmbedArgs ea = embed_args(d);
    hipLaunchKernelGGL(embed_kernel, dim3((std::max(ea.units * 4, 2 * ea.half) + 255) / 256), dim3(256), 0, s, ea);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    ++n;
    int32_t *pos = d->state + 1;
    for (uint32_t l = 0; l < d->layers; ++l) {
        const DeviceTensor *const *w = d->proj.data() + static_cast<size_t>(l) * kProj;
        const float *qn = d->q_norms ? d->q_norms + static_cast<size_t>(l) * d->head_dim : nullptr;
        const float *kn = d->k_norms ? d->k_norms + static_cast<size_t>(l) * d->head_dim : nullptr;
        GemvGroupLaunch qkv = group({w[P_Q], w[P_K], w[P_V]}, {d->q, d->k, d->v});
        qkv.input_mode = kInNorm;
        for (int p = P_Q; p <= P_V; ++p) qkv.bias[p] = layer_bias(d, l, p);
        qkv.x = d->x;
        qkv.norm = d->norms_in + static_cast<size_t>(l) * d->hidden;
        qkv.eps = d->eps;
        if ((e = launch_gemv_group(qkv, s)) != hipSuccess) return e;
        if (d->fused_attention) {
            DecodeAttentionLaunch at;
            at.cache = &d->caches[l];
            at.query = d->q;
            at.output = d->attn;
            at.partials = d->partials;
            at.query_heads = d->heads;
            at.position_ptr = pos;
            at.span_tokens = d->max_ctx;
            at.scale = d->attn_scale;
            at.key = d->k;
            at.value = d->v;
            at.cos_tab = d->rope_row;
            at.sin_tab = d->rope_row + d->head_dim / 2;
            at.rope_row_only = true;
            at.q_norm = qn;
            at.k_norm = kn;
            at.eps = d->eps;
            if ((e = launch_decode_attention(at, s)) != hipSuccess) return e;
        } else {
            if ((e = launch_rope_append(d->caches[l], d->q, d->heads, d->k, d->v, d->cos_tab, d->sin_tab, pos, s, 1,
                                        qn, kn, d->eps)) != hipSuccess)
                return e;
            if ((e = launch_attention_at(d->caches[l], d->q, d->attn, d->heads, pos, d->attn_scale, d->partials,
                                         s)) != hipSuccess)
                return e;
        }
        GemvGroupLaunch o = group({w[P_O]}, {d->x});
        o.input_mode = kInF32;
        o.output_mode = kOutAdd;
        o.bias[0] = layer_bias(d, l, P_O);
        o.x = d->attn;
        if ((e = launch_gemv_group(o, s)) != hipSuccess) return e;
        // gate and up rows paired in each workgroup: the epilogue writes
        // silu(gate) * up, so the down projection only quantizes it
        GemvGroupLaunch gu = group({w[P_GATE], w[P_UP]}, {d->gate, d->up});
        gu.input_mode = kInNorm;
        gu.output_mode = kOutSwiglu;
        gu.x = d->x;
        gu.norm = d->norms_post + static_cast<size_t>(l) * d->hidden;
        gu.eps = d->eps;
        if ((e = launch_gemv_group(gu, s)) != hipSuccess) return e;
        GemvGroupLaunch down = group({w[P_DOWN]}, {d->x});
        down.input_mode = kInF32;
        down.output_mode = kOutAdd;
        down.x = d->gate;
        if ((e = launch_gemv_group(down, s)) != hipSuccess) return e;
        n += d->layer_launches;
    }
    if ((e = enqueue_head(d, d->x, s)) != hipSuccess) return e;
    n += 2;
    if (count) *count = n;
    return hipSuccess;
}

// Captures `enqueue` once into *exec (left null when capture fails, so the
// caller launches the kernels directly) and launches it.
template <typename F>
hipError_t run_captured(hipStream_t s, hipGraphExec_t *exec, bool *tried, F enqueue) {
    if (!*tried) {
        *tried = true;
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            const hipError_t le = enqueue();
            e = hipStreamEndCapture(s, &g);
            if (le != hipSuccess) e = le;
        }
        if (e == hipSuccess && g) e = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
        if (g) (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            *exec = nullptr;
            (void)hipGetLastError();
        }
    }
    if (*exec) return hipGraphLaunch(*exec, s);
    return enqueue();
}

// The prompt, already in feed at the device position, in prefill blocks.
hipError_t run_prefill(Decoder *d, uint32_t count) {
    hipStream_t s = d->ctx->stream;
    for (uint32_t i = 0; i < count; i += d->block_tokens) {
        const uint32_t m = std::min(d->block_tokens, count - i);
        const uint32_t kind = i + m == count ? kBlockLast : kBlockInner;
        const hipError_t e = run_captured(s, &d->prefill_exec[m][kind], &d->prefill_tried[m][kind],
                                          [&] { return enqueue_prefill(d, m, kind, s); });
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// One verify block of m <= kPrefillTokens tokens, already in feed.
hipError_t run_verify(Decoder *d, uint32_t m) {
    hipStream_t s = d->ctx->stream;
    return run_captured(s, &d->prefill_exec[m][kBlockVerify], &d->prefill_tried[m][kBlockVerify],
                        [&] { return enqueue_prefill(d, m, kBlockVerify, s); });
}

// The nodes of a draft tree, already in feed at the device position (the
// tree's base slot), in blocks of up to block_tokens nodes (one block for a
// tree of 64 on the MFMA path): a node's ancestors come before it, so every
// block finds them in the cache.
hipError_t run_tree(Decoder *d, uint32_t count) {
    hipStream_t s = d->ctx->stream;
    for (uint32_t b = 0; b * d->block_tokens < count; ++b) {
        const uint32_t m = std::min(d->block_tokens, count - b * d->block_tokens);
        const hipError_t e = run_captured(s, &d->tree_exec[b][m], &d->tree_tried[b][m],
                                          [&] { return enqueue_prefill(d, m, kBlockTree, s, b); });
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Runs one step: the captured graph when capture worked, else the kernels.
hipError_t run_step(Decoder *d) {
    hipStream_t s = d->ctx->stream;
    if (!d->graph_tried) {
        d->graph_tried = true;
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            const hipError_t le = enqueue_step(d, s, nullptr);
            e = hipStreamEndCapture(s, &g);
            if (le != hipSuccess) e = le;
        }
        if (e == hipSuccess && g) e = hipGraphInstantiate(&d->exec, g, nullptr, nullptr, 0);
        if (g) (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            d->exec = nullptr;
            (void)hipGetLastError();
        }
    }
    if (d->exec) return hipGraphLaunch(d->exec, s);
    return enqueue_step(d, s, nullptr);
}

const DeviceTensor *check_shape(Context *ctx, const QwnCudaTensorHandle &h, int kind, uint32_t rows, uint32_t cols) {
    ResidentTensor *rt = tensor_of(ctx, h);
    if (!rt || rt->t.kind != kind || rt->t.rows != rows || rt->t.cols != cols) return nullptr;
    return &rt->t;
}

uint64_t logical_bytes(const DeviceTensor &t) { return t.logical_bytes; }

}  // namespace

}  // namespace qwn

using namespace qwn;

extern "C" {

QWN_CUDA_ABI_API int qwn_hip_decoder_create(QwnCudaContextHandle *handle, const QwnHipDecoderDesc *desc,
                                            QwnHipDecoderHandle *out) {
    Context *ctx = context_of(handle);
    if (!ctx || !desc || !out || !header_ok(*desc) || !header_ok(*out) || !desc->projections ||
        !desc->embedding || !desc->input_norms || !desc->post_norms || !desc->final_norm || desc->hidden == 0 ||
        desc->layers == 0 || desc->heads == 0 || desc->kv_heads == 0 || desc->heads % desc->kv_heads ||
        desc->head_dim == 0 || desc->head_dim % 2 || desc->vocab == 0 || desc->max_ctx == 0 ||
        desc->intermediate == 0 || (!desc->q_norms) != (!desc->k_norms) ||
        (desc->q_norms && desc->heads + desc->kv_heads > static_cast<uint32_t>(kMaxNormHeads))) {
        set_error("invalid decoder description");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    auto *d = new (std::nothrow) Decoder();
    if (!d) return QWN_CUDA_STATUS_OUT_OF_MEMORY;
    d->ctx = ctx;
    d->hidden = desc->hidden;
    d->inter = desc->intermediate;
    d->layers = desc->layers;
    d->heads = desc->heads;
    d->kv_heads = desc->kv_heads;
    d->head_dim = desc->head_dim;
    d->vocab = desc->vocab;
    d->max_ctx = desc->max_ctx;
    d->eps = desc->rms_eps;
    d->attn_scale = 1.0f / sqrtf(static_cast<float>(desc->head_dim));
    const uint32_t D = d->hidden, Q = d->heads * d->head_dim, KV = d->kv_heads * d->head_dim, I = d->inter;
    // weights: one quantized dtype for every projection, shapes of the config
    ResidentTensor *first = tensor_of(ctx, desc->projections[0]);
    const int kind = first ? first->t.kind : 0;
    bool ok = kind == kHvsq2 || kind == kQ4_0;
    const uint32_t shapes[kProj][2] = {{Q, D}, {KV, D}, {KV, D}, {D, Q}, {I, D}, {I, D}, {D, I}};
    for (uint32_t l = 0; ok && l < d->layers; ++l)
        for (int p = 0; ok && p < kProj; ++p) {
            const DeviceTensor *t = check_shape(ctx, desc->projections[l * kProj + p], kind, shapes[p][0],
                                                shapes[p][1]);
            ok = t != nullptr;
            d->proj.push_back(t);
            if (t) d->weight_bytes += logical_bytes(*t);
        }
    d->embed = ok ? check_shape(ctx, *desc->embedding, kF16, d->vocab, D) : nullptr;
    d->head = d->embed;
    if (ok && desc->lm_head) {
        ResidentTensor *rh = tensor_of(ctx, *desc->lm_head);
        d->head = rh && rh->t.rows == d->vocab && rh->t.cols == D ? &rh->t : nullptr;
    }
    if (!ok || !d->embed || !d->head) {
        delete d;
        set_error("decoder weights do not match the configuration (one quantized dtype for all projections, "
                  "F16/BF16 [vocab][hidden] embedding, lm_head [vocab][hidden] if given)");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    // per step the LM head is read whole; the embedding only one row
    d->weight_bytes += d->head->logical_bytes;

    // device memory: activations, tables, caches, state
    std::vector<std::pair<void **, size_t>> parts;
    auto part = [&](void **p, size_t bytes) { parts.push_back({p, (bytes + 255) & ~static_cast<size_t>(255)}); };
    part(reinterpret_cast<void **>(&d->x), D * 4);
    part(reinterpret_cast<void **>(&d->q), Q * 4);
    part(reinterpret_cast<void **>(&d->k), KV * 4);
    part(reinterpret_cast<void **>(&d->v), KV * 4);
    part(reinterpret_cast<void **>(&d->attn), Q * 4);
    part(reinterpret_cast<void **>(&d->gate), static_cast<size_t>(I) * 4);
    part(reinterpret_cast<void **>(&d->up), static_cast<size_t>(I) * 4);
    part(reinterpret_cast<void **>(&d->logits), static_cast<size_t>(d->vocab) * 4);
    part(reinterpret_cast<void **>(&d->norms_in), static_cast<size_t>(d->layers) * D * 4);
    part(reinterpret_cast<void **>(&d->norms_post), static_cast<size_t>(d->layers) * D * 4);
    part(reinterpret_cast<void **>(&d->final_norm), D * 4);
    if (desc->q_norms) {
        part(reinterpret_cast<void **>(&d->q_norms), static_cast<size_t>(d->layers) * d->head_dim * 4);
        part(reinterpret_cast<void **>(&d->k_norms), static_cast<size_t>(d->layers) * d->head_dim * 4);
    }
    const float *const host_bias[4] = {desc->q_biases, desc->k_biases, desc->v_biases, desc->o_biases};
    const uint32_t bias_rows[4] = {Q, KV, KV, D};
    for (int p = 0; p < 4; ++p)
        if (host_bias[p]) part(reinterpret_cast<void **>(&d->bias[p]), static_cast<size_t>(d->layers) * bias_rows[p] * 4);
    const uint32_t half = d->head_dim / 2;
    part(reinterpret_cast<void **>(&d->cos_tab), static_cast<size_t>(d->max_ctx) * half * 4);
    part(reinterpret_cast<void **>(&d->sin_tab), static_cast<size_t>(d->max_ctx) * half * 4);
    part(reinterpret_cast<void **>(&d->rope_row), static_cast<size_t>(half) * 2 * 4);
    part(reinterpret_cast<void **>(&d->state), 2 * 4);
    part(reinterpret_cast<void **>(&d->feed), static_cast<size_t>(d->max_ctx) * 4);
    part(reinterpret_cast<void **>(&d->out_tokens), static_cast<size_t>(d->max_ctx) * 4);
    // prefill blocks: [token][...] activations, images of the widest input
    {
        const size_t P = kBlockTokens;
        part(reinterpret_cast<void **>(&d->px), P * D * 4);
        part(reinterpret_cast<void **>(&d->pq), P * Q * 4);
        part(reinterpret_cast<void **>(&d->pk), P * KV * 4);
        part(reinterpret_cast<void **>(&d->pv), P * KV * 4);
        part(reinterpret_cast<void **>(&d->pattn), P * Q * 4);
        part(reinterpret_cast<void **>(&d->pgate), P * I * 4);
        part(reinterpret_cast<void **>(&d->pup), P * I * 4);
        part(reinterpret_cast<void **>(&d->pscales), P * 4);
        part(reinterpret_cast<void **>(&d->ppos), P * 4);
        size_t stride = 0;
        for (int p : {P_Q, P_O, P_DOWN}) stride = std::max(stride, image_bytes(kind, d->proj[p]->units));
        d->pimg_stride = static_cast<uint32_t>((stride + 15) & ~static_cast<size_t>(15));
        // dot8 images: blocks of up to kPrefillTokens tokens take that path
        part(reinterpret_cast<void **>(&d->pimg), kPrefillTokens * d->pimg_stride);
        // MFMA images: one per 16-token group of a block
        if (kind == kHvsq2 || kind == kQ4_0) {
            part(reinterpret_cast<void **>(&d->pmimg),
                 (kBlockTokens / 16) * std::max({mfma_image_bytes(*d->proj[P_DOWN]), mfma_image_bytes(*d->proj[P_Q]),
                                                 mfma_image_bytes(*d->proj[P_O])}));
            d->block_tokens = kBlockTokens;
        }
        d->vimg_stride =
            static_cast<uint32_t>((image_bytes(d->head->kind, d->head->units) + 15) & ~static_cast<size_t>(15));
        part(reinterpret_cast<void **>(&d->vimg), P * d->vimg_stride);
        if (mfma_head_supported(*d->head)) {
            part(reinterpret_cast<void **>(&d->hpieces), head_pieces_bytes_32(*d->head));
            part(reinterpret_cast<void **>(&d->hunscale), P * 4);
        }
        part(reinterpret_cast<void **>(&d->vlogits), static_cast<size_t>(kTreeNodes) * d->vocab * 4);
        part(reinterpret_cast<void **>(&d->vids), kTreeNodes * 4);
        part(reinterpret_cast<void **>(&d->row_keys), P * rows_argmax_parts(d->vocab) * 8);
        part(reinterpret_cast<void **>(&d->tree_mask), kTreeNodes * 8);
        part(reinterpret_cast<void **>(&d->tree_pos), kTreeNodes * 4);
        part(reinterpret_cast<void **>(&d->tree_base), 4);
        part(reinterpret_cast<void **>(&d->tree_path), kTreeNodes * 4);
    }
    // attention partials of the device-position kernels
    KvCache proto;
    proto.max_tokens = d->max_ctx;
    proto.kv_heads = d->kv_heads;
    proto.head_dim = d->head_dim;
    const size_t cache_bytes = (kv_cache_layout(proto, nullptr) + 255) & ~static_cast<size_t>(255);
    // contexts of one split: RoPE, append and attention in one kernel; longer
    // ones: the RoPE/append kernel, then the split attention (MFMA where the
    // shape allows) and its merge
    d->fused_attention = decode_attention_supported(proto, d->heads) && d->head_dim % 64 == 0 &&
                         decode_split_tokens(proto, d->max_ctx) >= d->max_ctx;
    part(reinterpret_cast<void **>(&d->partials),
         std::max<size_t>(d->fused_attention ? decode_attention_workspace_floats(proto, d->heads, d->max_ctx)
                                             : attention_at_workspace_floats(proto, d->heads),
                          1) * 4);
    {
        // the head launch's shape; its buffers are not placed yet, so
        // non-null placeholders stand in for them (validity only)
        GemvGroupLaunch head = head_launch(d, reinterpret_cast<const float *>(16));
        head.outputs[0] = reinterpret_cast<float *>(16);
        head.argmax_partials = reinterpret_cast<uint64_t *>(16);
        if (head.input_mode == kInImage) head.image = reinterpret_cast<const void *>(16);
        else head.norm = reinterpret_cast<const float *>(16);
        d->argmax_n = gemv_group_grid(head);
    }
    part(reinterpret_cast<void **>(&d->argmax), static_cast<size_t>(d->argmax_n) * 8);
    // every grouped launch of the step must accept its fused input
    bool fits = d->argmax_n > 0;
    {
        auto probe = [&](std::initializer_list<const DeviceTensor *> ts, uint32_t mode) {
            GemvGroupLaunch g = group(ts, {});
            for (int i = 0; i < g.njobs; ++i) g.outputs[i] = reinterpret_cast<float *>(16);
            g.input_mode = mode;
            g.x = g.x2 = g.norm = reinterpret_cast<const float *>(16);
            return gemv_group_grid(g) > 0;
        };
        const DeviceTensor *const *w = d->proj.data();
        GemvGroupLaunch gu = group({w[P_GATE], w[P_UP]}, {});
        gu.outputs[0] = gu.outputs[1] = reinterpret_cast<float *>(16);
        gu.input_mode = kInNorm;
        gu.output_mode = kOutSwiglu;
        gu.x = gu.norm = reinterpret_cast<const float *>(16);
        fits = fits && probe({w[P_Q], w[P_K], w[P_V]}, kInNorm) && probe({w[P_O]}, kInF32) &&
               gemv_group_grid(gu) > 0 && probe({w[P_DOWN]}, kInF32);
    }
    if (!fits || KV > 8192) {
        delete d;
        set_error("decoder shapes exceed the fused GEMV limits (columns a multiple of 32, at most 16384)");
        return QWN_CUDA_STATUS_UNSUPPORTED;
    }
    size_t total = 0;
    for (auto &p : parts) total += p.second;
    const size_t act_bytes = total;
    total += cache_bytes * d->layers;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc(&d->allocation, total);
    if (e != hipSuccess) {
        delete d;
        return hip_fail("decoder allocation", e, QWN_CUDA_STATUS_OUT_OF_MEMORY);
    }
    uint8_t *base = static_cast<uint8_t *>(d->allocation);
    size_t off = 0;
    for (auto &p : parts) {
        *p.first = base + off;
        off += p.second;
    }
    for (uint32_t l = 0; l < d->layers; ++l) {
        KvCache c;
        c.max_tokens = d->max_ctx;
        c.kv_heads = d->kv_heads;
        c.head_dim = d->head_dim;
        kv_cache_layout(c, base + act_bytes + static_cast<size_t>(l) * cache_bytes);
        d->caches.push_back(c);
    }
    // host tables: norms, RoPE (c/qwanto_decode.c:601-625), empty feed
    std::vector<float> cs(static_cast<size_t>(d->max_ctx) * half), sn(cs.size());
    for (uint32_t p = 0; p < d->max_ctx; ++p)
        for (uint32_t i = 0; i < half; ++i) {
            const float angle = static_cast<float>(p) *
                                powf(desc->rope_theta, -2.0f * static_cast<float>(i) / static_cast<float>(2 * half));
            cs[static_cast<size_t>(p) * half + i] = cosf(angle);
            sn[static_cast<size_t>(p) * half + i] = sinf(angle);
        }
    std::vector<int32_t> feed(d->max_ctx, -1);
    const int32_t state0[2] = {0, 0};
    hipStream_t s = ctx->stream;
    if (e == hipSuccess) e = hipMemsetAsync(base, 0, total, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->norms_in, desc->input_norms, static_cast<size_t>(d->layers) * D * 4,
                           hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->norms_post, desc->post_norms, static_cast<size_t>(d->layers) * D * 4,
                           hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->final_norm, desc->final_norm, D * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && desc->q_norms)
        e = hipMemcpyAsync(d->q_norms, desc->q_norms, static_cast<size_t>(d->layers) * d->head_dim * 4,
                           hipMemcpyHostToDevice, s);
    if (e == hipSuccess && desc->k_norms)
        e = hipMemcpyAsync(d->k_norms, desc->k_norms, static_cast<size_t>(d->layers) * d->head_dim * 4,
                           hipMemcpyHostToDevice, s);
    for (int p = 0; p < 4; ++p)
        if (e == hipSuccess && host_bias[p])
            e = hipMemcpyAsync(d->bias[p], host_bias[p], static_cast<size_t>(d->layers) * bias_rows[p] * 4,
                               hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->cos_tab, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->sin_tab, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->feed, feed.data(), feed.size() * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->state, state0, sizeof(state0), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        destroy_decoder(d);
        return hip_fail("decoder set-up", e);
    }
    // qkv, attention (+ merge past one split; RoPE/append and split + merge
    // as three kernels without the fused kernel), o, gate/up, down
    const uint32_t attention_launches =
        d->fused_attention ? 1
                           : 1 + (mfma_attention_supported(proto, d->heads) ? mfma_attention_launches(proto, d->heads, d->max_ctx)
                                                                           : 2);
    d->layer_launches = 4 + attention_launches;
    // + embed, LM head (final RMSNorm in its prologue), step end
    d->launches = d->layer_launches * d->layers + 3;
    ctx->decoders.push_back(d);
    std::memset(out, 0, sizeof(*out));
    qwn_cuda_abi_header_init(&out->header, sizeof(*out));
    out->opaque = d;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_destroy(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d) {
        set_error("invalid decoder handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    ctx->decoders.erase(std::find(ctx->decoders.begin(), ctx->decoders.end(), d));
    destroy_decoder(d);
    h->opaque = nullptr;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_reset(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d) {
        set_error("invalid decoder handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    d->tree_nodes = 0;
    const int32_t state0[2] = {0, 0};
    std::vector<int32_t> feed(d->max_ctx, -1);
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMemcpyAsync(d->state, state0, sizeof(state0), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->feed, feed.data(), feed.size() * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail("decoder reset", e);
    d->position = 0;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_debug_kv_read(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h,
                                                   uint32_t layer, uint32_t first, uint32_t count, int8_t *keys,
                                                   int8_t *values, float *key_scales, float *value_scales) {
    Context *ctx = context_of(handle);
    if (!ctx || !keys || !values || !key_scales || !value_scales || count == 0) {
        set_error("invalid decoder KV read");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || layer >= d->layers || first > d->position || count > d->position - first) {
        set_error("decoder KV read beyond the decoder's layers or position");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    KvCache c = d->caches[layer];
    c.tokens = d->position;
    const size_t vb = static_cast<size_t>(count) * c.channels, sb = static_cast<size_t>(count) * c.groups * 4;
    hipError_t e = hipSetDevice(ctx->device);
    void *buf = nullptr;
    if (e == hipSuccess) e = hipMalloc(&buf, 2 * vb + 2 * sb + 256);
    uint8_t *b = static_cast<uint8_t *>(buf);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess)
        e = launch_kv_gather(c, first, count, reinterpret_cast<int8_t *>(b), reinterpret_cast<int8_t *>(b + vb),
                             reinterpret_cast<float *>(b + 2 * vb), reinterpret_cast<float *>(b + 2 * vb + sb),
                             ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(keys, b, vb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(values, b + vb, vb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(key_scales, b + 2 * vb, sb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(value_scales, b + 2 * vb + sb, sb, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (buf) (void)hipFree(buf);
    return e == hipSuccess ? QWN_CUDA_STATUS_OK : hip_fail("decoder KV read", e);
}

QWN_CUDA_ABI_API int qwn_hip_decoder_forward(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h, int32_t token,
                                             float *logits, int32_t *next_token) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || token < 0 || static_cast<uint32_t>(token) >= d->vocab || d->position >= d->max_ctx) {
        set_error("invalid decoder step (token out of range or context full)");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    d->tree_nodes = 0;
    hipStream_t s = ctx->stream;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMemcpyAsync(d->feed + d->position, &token, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = run_step(d);
    if (e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, d->logits, static_cast<size_t>(d->vocab) * 4, hipMemcpyDeviceToHost, s);
    int32_t st[2] = {0, 0};
    if (e == hipSuccess) e = hipMemcpyAsync(st, d->state, sizeof(st), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail("decoder step", e);
    d->position++;
    if (next_token) *next_token = st[0];
    ctx->telemetry.gpu_matmul_count += 4ull * d->layers + 1;
    ctx->telemetry.gpu_kernel_launch_count += d->launches;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_prefill(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h,
                                             const int32_t *tokens, uint32_t count, float *logits,
                                             int32_t *next_token) {
    Context *ctx = context_of(handle);
    if (!ctx || !tokens || count == 0) {
        set_error("invalid prefill request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || static_cast<uint64_t>(d->position) + count > d->max_ctx) {
        set_error("prefill does not fit the decoder's context");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < count; ++i)
        if (tokens[i] < 0 || static_cast<uint32_t>(tokens[i]) >= d->vocab) {
            set_error("prefill token %u out of range", i);
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
    d->tree_nodes = 0;
    hipStream_t s = ctx->stream;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->feed + d->position, tokens, static_cast<size_t>(count) * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = run_prefill(d, count);
    if (e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, d->logits, static_cast<size_t>(d->vocab) * 4, hipMemcpyDeviceToHost, s);
    int32_t st[2] = {0, 0};
    if (e == hipSuccess) e = hipMemcpyAsync(st, d->state, sizeof(st), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail("decoder prefill", e);
    d->position += count;
    if (next_token) *next_token = st[0];
    const uint64_t blocks = (count + d->block_tokens - 1) / d->block_tokens;
    ctx->telemetry.gpu_matmul_count += blocks * 4ull * d->layers + 1;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_verify(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h,
                                            const int32_t *tokens, uint32_t count, float *logits,
                                            int32_t *next_tokens) {
    Context *ctx = context_of(handle);
    if (!ctx || !tokens || count == 0 || count > kPrefillTokens) {
        set_error("invalid verify request (1..%u tokens)", kPrefillTokens);
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || static_cast<uint64_t>(d->position) + count > d->max_ctx) {
        set_error("verify block does not fit the decoder's context");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < count; ++i)
        if (tokens[i] < 0 || static_cast<uint32_t>(tokens[i]) >= d->vocab) {
            set_error("verify token %u out of range", i);
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
    d->tree_nodes = 0;
    hipStream_t s = ctx->stream;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->feed + d->position, tokens, static_cast<size_t>(count) * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = run_verify(d, count);
    if (e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, d->vlogits, static_cast<size_t>(count) * d->vocab * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && next_tokens)
        e = hipMemcpyAsync(next_tokens, d->vids, static_cast<size_t>(count) * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail("decoder verify", e);
    d->position += count;
    ctx->telemetry.gpu_matmul_count += 4ull * d->layers + 1;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_truncate(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h,
                                              uint32_t position) {
    Context *ctx = context_of(handle);
    if (!ctx) {
        set_error("invalid context handle");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || position > d->position) {
        set_error("truncate position beyond the decoder's tokens");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    // the cache slots past `position` are overwritten by the next tokens;
    // only the device position and the host mirror move
    d->tree_nodes = 0;
    const int32_t pos = static_cast<int32_t>(position);
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMemcpyAsync(d->state + 1, &pos, 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail("decoder truncate", e);
    d->position = position;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_verify_tree(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h,
                                                 const int32_t *tokens, const int32_t *parents, uint32_t count,
                                                 float *logits, int32_t *next_tokens) {
    Context *ctx = context_of(handle);
    if (!ctx || !tokens || !parents || count == 0 || count > kTreeNodes) {
        set_error("invalid tree verify request (1..%u nodes)", kTreeNodes);
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || static_cast<uint64_t>(d->position) + count > d->max_ctx) {
        set_error("draft tree does not fit the decoder's context");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    // depth and ancestor-or-self mask of every node (c/qwanto_jetspec.c:33-49)
    std::vector<uint64_t> mask(count);
    std::vector<int32_t> pos(count);
    std::vector<uint32_t> depth(count);
    for (uint32_t i = 0; i < count; ++i) {
        const int32_t p = parents[i];
        if (tokens[i] < 0 || static_cast<uint32_t>(tokens[i]) >= d->vocab || p < -1 || p >= static_cast<int32_t>(i)) {
            set_error("tree node %u: token out of range or parent not an earlier node (or -1)", i);
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
        depth[i] = p < 0 ? 0 : depth[p] + 1;
        mask[i] = (p < 0 ? 0ull : mask[p]) | (1ull << i);
        pos[i] = static_cast<int32_t>(d->position + depth[i]);
    }
    // the masked attention runs in the one-split decode kernel or the MFMA kernel
    if (!d->fused_attention && !mfma_attention_supported(d->caches[0], d->heads)) {
        set_error("tree verify needs the decode or MFMA attention for this head shape");
        return QWN_CUDA_STATUS_UNSUPPORTED;
    }
    d->tree_nodes = 0;
    hipStream_t s = ctx->stream;
    const int32_t base = static_cast<int32_t>(d->position);
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->feed + d->position, tokens, static_cast<size_t>(count) * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->tree_mask, mask.data(), count * 8, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->tree_pos, pos.data(), count * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->tree_base, &base, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = run_tree(d, count);
    // the nodes stay in slots base .. base + count - 1 until a path is
    // committed; the position stays at the prefix
    if (e == hipSuccess) e = hipMemcpyAsync(d->state + 1, &base, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, d->vlogits, static_cast<size_t>(count) * d->vocab * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && next_tokens)
        e = hipMemcpyAsync(next_tokens, d->vids, static_cast<size_t>(count) * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail("decoder tree verify", e);
    d->tree_nodes = count;
    d->tree_parents.assign(parents, parents + count);
    d->tree_tokens.assign(tokens, tokens + count);
    const uint64_t blocks = (count + d->block_tokens - 1) / d->block_tokens;
    ctx->telemetry.gpu_matmul_count += blocks * (4ull * d->layers + 1);
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_commit_path(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h,
                                                 const uint32_t *nodes, uint32_t length) {
    Context *ctx = context_of(handle);
    if (!ctx || !nodes || length == 0) {
        set_error("invalid path commit request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || d->tree_nodes == 0 || length > d->tree_nodes) {
        set_error("no verified draft tree to commit from (or the path is longer than the tree)");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::vector<int32_t> path(length), toks(length);
    for (uint32_t k = 0; k < length; ++k) {
        const int32_t want = k == 0 ? -1 : static_cast<int32_t>(nodes[k - 1]);
        if (nodes[k] >= d->tree_nodes || d->tree_parents[nodes[k]] != want) {
            set_error("path node %u is not %s", k, k == 0 ? "a root of the tree" : "a child of the previous node");
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
        path[k] = static_cast<int32_t>(nodes[k]);
        toks[k] = d->tree_tokens[nodes[k]];
    }
    hipStream_t s = ctx->stream;
    const int32_t next = static_cast<int32_t>(d->position + length);
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMemcpyAsync(d->tree_path, path.data(), length * 4, hipMemcpyHostToDevice, s);
    for (uint32_t l = 0; e == hipSuccess && l < d->layers; ++l)
        e = launch_kv_commit_path(d->caches[l], d->tree_base, d->tree_path, length, s);
    // the accepted tokens as the cache's history, and the position past them
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->feed + d->position, toks.data(), length * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d->state + 1, &next, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail("decoder path commit", e);
    d->position += length;
    d->tree_nodes = 0;
    ctx->telemetry.kv_cache_kernel_count += d->layers;
    return QWN_CUDA_STATUS_OK;
}

QWN_CUDA_ABI_API int qwn_hip_decoder_generate(QwnCudaContextHandle *handle, QwnHipDecoderHandle *h,
                                              const int32_t *prompt, uint32_t prompt_count, uint32_t max_new,
                                              int32_t *tokens, QwnHipDecoderStats *stats) {
    Context *ctx = context_of(handle);
    if (!ctx || !prompt || prompt_count == 0 || (max_new && !tokens) || (stats && !header_ok(*stats))) {
        set_error("invalid generate request");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(ctx->mutex);
    Decoder *d = decoder_of(ctx, h);
    if (!d || static_cast<uint64_t>(d->position) + prompt_count + max_new > d->max_ctx) {
        set_error("generation does not fit the decoder's context");
        return QWN_CUDA_STATUS_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < prompt_count; ++i)
        if (prompt[i] < 0 || static_cast<uint32_t>(prompt[i]) >= d->vocab) {
            set_error("prompt token %u out of range", i);
            return QWN_CUDA_STATUS_INVALID_ARGUMENT;
        }
    d->tree_nodes = 0;
    hipStream_t s = ctx->stream;
    const uint32_t p0 = d->position;
    std::vector<int32_t> feed(d->max_ctx - p0, -1);
    std::memcpy(feed.data(), prompt, static_cast<size_t>(prompt_count) * 4);
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMemcpyAsync(d->feed + p0, feed.data(), feed.size() * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    const auto t0 = std::chrono::steady_clock::now();
    if (e == hipSuccess) e = run_prefill(d, prompt_count);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    const auto t1 = std::chrono::steady_clock::now();
    for (uint32_t i = 0; e == hipSuccess && i < max_new; ++i) e = run_step(d);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    const auto t2 = std::chrono::steady_clock::now();
    if (e == hipSuccess && max_new)
        e = hipMemcpy(tokens, d->out_tokens + p0 + prompt_count - 1, static_cast<size_t>(max_new) * 4,
                      hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail("decoder generate", e);
    d->position = p0 + prompt_count + max_new;
    const uint64_t steps = prompt_count + max_new;
    ctx->telemetry.gpu_matmul_count += steps * (4ull * d->layers + 1);
    ctx->telemetry.gpu_kernel_launch_count += steps * d->launches;
    if (stats) {
        std::memset(stats, 0, sizeof(*stats));
        qwn_cuda_abi_header_init(&stats->header, sizeof(*stats));
        stats->prompt_tokens = prompt_count;
        stats->generated_tokens = max_new;
        stats->position = d->position;
        stats->launches_per_step = d->launches;
        stats->prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        stats->decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
        stats->weight_bytes_per_step = d->weight_bytes;
        stats->graph = d->exec ? 1u : 0u;
        stats->prefill_block_tokens = d->block_tokens;
    }
    return QWN_CUDA_STATUS_OK;
}

}  // extern "C"
