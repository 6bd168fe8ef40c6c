// Internal declarations shared by the qwn_hip translation units.
//
// Device layouts (chosen at upload; the ABI keeps them private).
//
// Every GEMV launch maps a matrix onto waves the same way: a row is split
// across `lanes` lanes L (a power of two, so the row sum is a DPP reduction),
// each lane owning up to `upl` units (strided by L), and a wave holds
// R = 64/L rows.  A "unit" is one HyperVSQ-2 block (256 weights), four Q4_0
// blocks (128 weights) or 32 F16 weights -- 64 payload bytes in four
// 16-byte chunks for every kind.
// Weights are stored wave tile by wave tile in exactly the order the lanes
// load them, and only real units are stored, so every load instruction of a
// wave reads one contiguous span with no padding:
//
//   tile t = rows t*R .. t*R+R-1; unit slot i holds units i*L + j (j < L),
//   n_i = min(L, units - i*L) of them (the last slots may be partial/empty)
//   payload: [tile][slot i][chunk q < 4][row g < R][j < n_i][16 B]
//   meta:    [tile][slot i][row g < R][j < n_i][8 B]
//
//   HyperVSQ-2: chunk q = codes of octants 2q, 2q+1 (16 B); meta = fp16
//               d_base, fp16 m_base, four bytes of octant multipliers (the
//               two reserved bytes of the 74-byte block are dropped: the
//               reference kernels never read them either)
//   Q4_0:       chunk q = the 16 nibble bytes of block 4u+q; meta = the
//               four fp16 block scales (zero for padding blocks)
//   F16:        chunk q = halves 8q..8q+7 of the unit, no meta (BF16
//               tensors use the same layout, flagged DeviceTensor::bf16)
// Rows past the matrix end (the last tile) are stored as zeros.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qwn {

enum WeightKind : int { kHvsq2 = 1, kQ4_0 = 2, kF16 = 3 };

constexpr int kWaveSize = 64;
constexpr int kGemvWaves = 4;                     // waves per workgroup (default launch)
constexpr int kGemvThreads = kWaveSize * kGemvWaves;
constexpr int kGemvMaxWaves = 8;                  // waves per workgroup (largest launch)
constexpr int kGemvMaxThreads = kWaveSize * kGemvMaxWaves;
constexpr int kTilePad = 16;                      // tiles are stored in multiples of this
constexpr uint32_t kChipCus = 256;                // compute units of one MI355X
constexpr int kMaxTokensPerLaunch = 16;
constexpr int kMfmaMaxBatch = 64;                 // tokens of one MFMA GEMM launch (16-token groups)
constexpr size_t kGemvLdsLimit = 64 * 1024;
constexpr int kMaxGroup = 4;                      // tensors sharing one input in one launch

// Elements covered by one unit, and LDS bytes one token's unit occupies
// (activation bytes plus 16 bytes of padding so that lanes reading
// consecutive units hit different LDS banks).
__host__ __device__ constexpr int unit_elems(int kind) {
    return kind == kHvsq2 ? 256 : (kind == kQ4_0 ? 128 : 32);
}
__host__ __device__ constexpr int unit_lds_bytes(int kind) {
    return kind == kHvsq2 ? 272 : 144;
}

struct DeviceTensor {
    int kind = 0;
    uint32_t rows = 0;
    uint32_t cols = 0;
    uint32_t units = 0;          // units per row
    // lane plan, fixed at upload because it defines the layout
    uint32_t lanes = 0;
    uint32_t upl = 0;
    uint32_t rows_per_wave = 0;
    uint32_t chunks = 0;         // 16-byte payload chunks per unit
    uint32_t tiles = 0;
    size_t tile_payload_bytes = 0;
    size_t tile_meta_bytes = 0;
    uint8_t *payload = nullptr;
    uint8_t *meta = nullptr;     // null for F16
    bool bf16 = false;           // kF16 layout holding bfloat16 weights (the high halves of fp32)
    uint64_t device_bytes = 0;   // bytes allocated on the device
    uint64_t logical_bytes = 0;  // algorithmic (on-disk) bytes
    // HyperVSQ-2 MFMA staging: gaps (16-byte pieces after every 64) of the
    // payload and meta copies in LDS, chosen for the tile shape
    uint32_t stage_pad_p = 0;
    uint32_t stage_pad_m = 0;
    // HyperVSQ-2: optional second copy in the MFMA GEMM's operand order,
    // payload [16-row group][unit][chunk g][row m][16 B], meta [16-row
    // group][unit][row m][8 B] (rows past the matrix zero); null if absent
    uint8_t *mfma_payload = nullptr;
    uint8_t *mfma_meta = nullptr;
};

// Bytes of a HyperVSQ-2 tensor's MFMA-order copy (0 for other kinds).
size_t mfma_copy_bytes(const DeviceTensor &t);
// Fills t.mfma_payload / t.mfma_meta (a block of mfma_copy_bytes at
// mfma_payload) from the wave-tile layout, on `stream` after its upload.
hipError_t launch_mfma_copy(const DeviceTensor &t, hipStream_t stream);

// Launch shape of one GEMV call.
struct GemvPlan {
    int tokens = 0;        // tokens per launch (template width)
    int grid = 0;
    size_t lds_bytes = 0;
};

// Fills units/lanes/upl/rows_per_wave/chunks/tiles and the tile sizes
// of a tensor whose kind/rows/cols are set; false if no plan fits.
bool layout_tensor(DeviceTensor &t);
// Same with a forced lane plan (lanes a power of two <= 64, upl one of the
// compiled widths, lanes * upl >= units); false if it does not fit.
bool layout_tensor_with(DeviceTensor &t, uint32_t lanes, uint32_t upl);

GemvPlan plan_gemv(const DeviceTensor &t, int batch);

// Repack one tensor from its on-disk bytes (already copied to `staging`
// on the device) into the device layout of `t`.
hipError_t repack_tensor(const DeviceTensor &t, const uint8_t *staging,
                         hipStream_t stream);
// The same in pieces: zero the device layout (padding slots stay zero),
// then repack rows [row0, row0 + nrows) from their on-disk bytes at `src`.
hipError_t clear_tensor(const DeviceTensor &t, hipStream_t stream);
hipError_t repack_rows(const DeviceTensor &t, const uint8_t *src, uint32_t row0, uint32_t nrows,
                       hipStream_t stream);

// Bytes of one token's activation image for a tensor kind / unit count
// (the LDS layout the GEMV reads, padded to 16 bytes).
size_t image_bytes(int kind, uint32_t units);

// Build images from int8 tokens (HyperVSQ-2, Q4_0) or fp32 tokens (F16):
// x [batch][x_stride] elements -> image [batch][image_stride bytes].
hipError_t launch_image(const DeviceTensor &t, const void *x, uint32_t batch, uint32_t x_stride,
                        uint8_t *image, uint32_t image_stride, hipStream_t stream);

// Per-token int8 quantization (c/qwanto_kernels.c:354-433) fused with the
// image build: fp32 x [batch][x_stride] -> scales [batch], image, and the
// int8 tokens q8 [batch][q8_stride] when q8 is not null.  With a null
// image only the int8 tokens are produced (t gives the padding width).
hipError_t launch_quantize_image(const DeviceTensor &t, const float *x, uint32_t batch, uint32_t x_stride,
                                 uint8_t *image, uint32_t image_stride, float *scales, int8_t *q8,
                                 uint32_t q8_stride, hipStream_t stream);

struct GemvLaunch {
    const DeviceTensor *tensor;
    const void *image;        // activation images [batch][image_stride]
    uint32_t image_stride;    // bytes
    const float *scales;      // per-token scales (null -> scalar `scale`)
    float scale;
    float *output;            // fp32 [batch][output_stride]
    uint32_t batch;
    uint32_t output_stride;   // elements
    int32_t *debug_sums;      // non-null: dump integer sums of token 0 instead
};

hipError_t launch_gemv(const GemvLaunch &g, hipStream_t stream);

// ---- grouped GEMV ---------------------------------------------------------
// One launch over up to kMaxGroup tensors that share an input (same kind and
// column count, hence the same lane plan): q/k/v, gate/up.  The input is
// either prebuilt activation images or, for one token, an fp32 vector that
// every workgroup turns into its own LDS image (optionally after an RMSNorm
// or a SwiGLU), so no separate quantization launch is needed.
enum GemvInput : uint32_t {
    kInImage = 0,    // images [ntok][image_stride], scales per token
    kInF32 = 1,      // y = x
    kInNorm = 2,     // y = (x * 1/sqrt(mean(x^2) + eps)) * norm
    kInSwiglu = 3,   // y = (x / (1 + exp(-x))) * x2
};
enum GemvOutput : uint32_t {
    kOutStore = 0,   // out = W y * scale
    kOutAdd = 1,     // out += W y * scale (residual stream)
    kOutArgmax = 2,  // store, plus per-workgroup (value, first index) maxima
    kOutSwiglu = 3,  // two jobs of one shape (gate, up) paired row by row in
                     // each workgroup: outputs[0] = silu(gate) * up
                     // (c/qwanto_decode.c:1946-1949), outputs[1] unused
};

struct GemvGroupLaunch {
    int njobs = 0;
    const DeviceTensor *tensors[kMaxGroup] = {};
    float *outputs[kMaxGroup] = {};
    uint32_t input_mode = kInImage;
    uint32_t output_mode = kOutStore;
    // kInImage
    const void *image = nullptr;
    uint32_t image_stride = 0;
    const float *scales = nullptr;
    float scale = 1.0f;
    uint32_t batch = 1;
    // fp32 modes (one token, cols % 32 == 0)
    const float *x = nullptr;
    const float *x2 = nullptr;
    const float *norm = nullptr;
    float eps = 0.0f;
    float *scale_out = nullptr;           // workgroup 0 stores its activation scale here
    uint64_t *argmax_partials = nullptr;  // kOutArgmax: [grid] packed keys
    uint32_t output_stride[kMaxGroup] = {};  // elements between tokens per job (0: its rows)
    int waves = 0;                        // workgroup size in waves (0: chosen here)
    const float *bias[kMaxGroup] = {};    // per job: null, or [rows] added to the stored product
                                          // (STORE / ADD: before the residual add)
};

// Workgroups a grouped launch uses (the argmax partial count).
uint32_t gemv_group_grid(const GemvGroupLaunch &g);
hipError_t launch_gemv_group(const GemvGroupLaunch &g, hipStream_t stream);
// Images of a block of fp32 tokens after the input transform of `mode`
// (kInF32, kInNorm with `norm` and eps, kInSwiglu with x2 at the same
// stride), quantized per token as launch_quantize_image; with mfma_image
// (batch <= 16) the tokens' columns of the MFMA image are written as well.
hipError_t launch_prepare_image(const DeviceTensor &t, uint32_t mode, const float *x, const float *x2,
                                const float *norm, float eps, uint32_t batch, uint32_t x_stride, uint8_t *image,
                                uint32_t image_stride, float *scales, int8_t *q8, uint32_t q8_stride,
                                hipStream_t stream, uint8_t *mfma_image = nullptr);
// int8 MFMA batch GEMM of a HyperVSQ-2 tensor for 1..16 tokens (used from 8
// tokens up): the activation layout its tiles read (the "MFMA image"), built
// from int8 tokens [batch][q8_stride] (values past cols ignored), and the
// GEMM on it: output [batch][output_stride] = W x_t * scales[t].
size_t mfma_image_bytes(const DeviceTensor &t);
hipError_t launch_mfma_image(const DeviceTensor &t, const int8_t *q8, uint32_t batch, uint32_t q8_stride,
                             uint8_t *image, hipStream_t stream);
hipError_t launch_gemm_mfma(const DeviceTensor &t, const uint8_t *image, const float *scales, float *output,
                            uint32_t batch, uint32_t output_stride, hipStream_t stream);
// The same over up to kMaxGroup tensors of equal K sharing one image (one
// launch); output_strides may be null (0 entries: each tensor's rows);
// accumulate: outputs += W x_t * scales[t] (the residual stream).  Up to
// kMfmaMaxBatch tokens: token group g (tokens 16g .. 16g+15) reads its own
// MFMA image at image + g * mfma_image_bytes(t) (dump: at most 16 tokens).
// swiglu: tensors[0] / [1] are a gate / up pair of equal rows, both with
// the MFMA-order copy, no bias, no accumulate: outputs[0] = silu(gate) * up
// per token (outputs[1] untouched).
hipError_t launch_gemm_mfma_group(const DeviceTensor *const *tensors, float *const *outputs, uint32_t count,
                                  const uint8_t *image, const float *scales, uint32_t batch,
                                  const uint32_t *output_strides, hipStream_t stream, bool accumulate = false,
                                  int32_t *dump = nullptr, const float *const *biases = nullptr,
                                  bool swiglu = false);
constexpr uint32_t kMfmaMinTokens = 3;
constexpr uint32_t kMfmaMinTokensQ4 = 6;
// LDS per workgroup the MFMA GEMM plans its staging against: gfx950's
// 160 KB (context creation refuses a device that reports less).
constexpr uint64_t kMfmaLdsLimit = 160 * 1024;
// Batches that take the int8 MFMA GEMM instead of the batched dot8 GEMV
// (per-layer times with the weights rotated through HBM).  With the
// MFMA-order copy (`copy`): HyperVSQ-2 from 2 tokens (Qwen3-4B layers: the
// MFMA GEMM 20.5 / 20.9 / 21.0 us at 1 / 2 / 3 tokens, the dot8 GEMV 18.1 /
// 23.3 / 33.3), Q4_0 from 3 (Qwen2-1.5B layers: the MFMA GEMM 20.4 / 20.7 /
// 21.6 us, the dot8 GEMV 16.3 / 18.8 / 24.5).  Without it, staged in LDS:
// HyperVSQ-2 from 3 tokens (about 24-26 us whatever the token count),
// Q4_0 from 6 (about 31 us).
inline bool mfma_batch(uint32_t kind, uint32_t batch, bool copy) {
    return (kind == kHvsq2 && batch >= (copy ? 2u : kMfmaMinTokens)) ||
           (kind == kQ4_0 && batch >= (copy ? kMfmaMinTokens : kMfmaMinTokensQ4));
}

// RMSNorm of `count` fp32 tokens ([count][x_stride]) into fp32 images of an
// F16 tensor ([count][image_stride]).
hipError_t launch_norm_image(const DeviceTensor &t, const float *x, const float *norm, float eps, uint8_t *image,
                             hipStream_t stream, uint32_t count = 1, uint32_t x_stride = 0,
                             uint32_t image_stride = 0);
// First index of the largest value of every row of [rows][cols] fp32 into
// ids[rows]; the last row's also into *last_out when given.  keys: device
// workspace of rows * rows_argmax_parts(cols) u64 (each row is split over
// that many workgroups, then reduced).
// LM head of a block of up to 32 tokens on the matrix cores (F16 / BF16
// heads whose activation pieces fit the LDS limit): launch_head_pieces
// RMSNorms each token of x [ntok][x_stride] with `norm` and writes its
// narrow pieces (head_pieces_bytes for up to 16 tokens, head_pieces_bytes_32
// beyond) and per-token unscale factors [ntok]; launch_mfma_head writes out
// [ntok][out_stride] = the logits (beyond 16 tokens: the rows cleared, then
// the two halves of the K range added in).
constexpr size_t kHeadLdsLimit = 144 * 1024;
size_t head_pieces_bytes(const DeviceTensor &t);
size_t head_pieces_bytes_32(const DeviceTensor &t);
bool mfma_head_supported(const DeviceTensor &t);
hipError_t launch_head_pieces(const DeviceTensor &t, const float *x, uint32_t x_stride, const float *norm, float eps,
                              uint32_t ntok, uint8_t *pieces, float *unscale, hipStream_t stream);
hipError_t launch_mfma_head(const DeviceTensor &t, const uint8_t *pieces, const float *unscale, uint32_t ntok,
                            float *out, uint32_t out_stride, hipStream_t stream);

constexpr uint32_t kRowsArgmaxMaxParts = 32;
uint32_t rows_argmax_parts(uint32_t cols);
hipError_t launch_rows_argmax(const float *v, uint32_t rows, uint32_t cols, uint32_t stride, int32_t *ids,
                              int32_t *last_out, uint64_t *keys, hipStream_t stream);
// Reduce argmax partials [n] to the winning row index (first index on ties).
hipError_t launch_argmax_finish(const uint64_t *partials, uint32_t n, int32_t *index_out, hipStream_t stream);

// ---- Q8 KV cache ------------------------------------------------------
struct KvCache {
    uint32_t max_tokens = 0;
    uint32_t kv_heads = 0;
    uint32_t head_dim = 0;
    uint32_t channels = 0;
    uint32_t groups = 0;       // ceil(channels / 64) scale groups per token
    uint32_t pages = 0;        // ceil(max_tokens / 16)
    uint32_t quads = 0;        // ceil(pages / 4): 64-token groups of pages
    uint32_t tokens = 0;
    int8_t *keys = nullptr;    // [kv_heads][pages][head_dim/16][16 tokens][16 channels]
    int8_t *values = nullptr;  // [kv_heads][pages][head_dim][16 tokens]
    float *key_scales = nullptr;    // [groups][quads][16 slots][4 pages]
    float *value_scales = nullptr;
    uint64_t bytes = 0;
};

constexpr int kKvPageTokens = 16;

// Geometry of a cache whose max_tokens/kv_heads/head_dim are set: fills
// channels/groups/pages and, when base is given, the four arrays inside one
// allocation of the returned size.
size_t kv_cache_layout(KvCache &c, uint8_t *base);

// RoPE (c/qwanto_decode.c:686-729) on q [query_heads][head_dim] in place and
// on key [channels], then the Q8 append of the rotated key and of value at
// slot *pos_ptr (one workgroup per token; cos/sin tables
// [max_tokens][head_dim/2]).  count > 1: a block of tokens, q/key/value
// [count][...] back to back, token i at slot pos_ptr[i].
// q_norm/k_norm (both or neither, [head_dim]): per-head RMSNorm with eps
// before the rotation (Qwen3, c/qwanto_decode.c:654-684), at most
// kMaxNormHeads query + KV heads.  rope_pos_ptr (optional, [count]): the
// positions the tokens are rotated for when they differ from their slots
// (a draft tree's node at slot P + index has position P + depth).
constexpr int kMaxNormHeads = 128;
hipError_t launch_rope_append(const KvCache &c, float *query, uint32_t query_heads, const float *key,
                              const float *value, const float *cos_tab, const float *sin_tab,
                              const int32_t *pos_ptr, hipStream_t stream, uint32_t count = 1,
                              const float *q_norm = nullptr, const float *k_norm = nullptr, float eps = 0.0f,
                              const int32_t *rope_pos_ptr = nullptr);

// Quantize `count` consecutive tokens' fp32 K and V ([count][channels])
// into slots token .. token + count - 1 (one launch per 32768 tokens).
hipError_t launch_kv_append(const KvCache &c, const float *key,
                            const float *value, uint32_t token,
                            hipStream_t stream, uint32_t count = 1);

// Looks up, once per device (which must be current), the device address of
// the allocation-free attention's file-scope partials array
// (qwn_noalloc.hip).
hipError_t noalloc_init_device(int device);

// Token-major copy of cached tokens [first, first + count) (debug readback):
// keys/values [count][channels], scales [count][groups].
hipError_t launch_kv_gather(const KvCache &c, uint32_t first, uint32_t count, int8_t *keys, int8_t *values,
                            float *key_scales, float *value_scales, hipStream_t stream);

struct AttentionLaunch {
    const KvCache *cache;
    const float *query;     // [query_heads][head_dim]
    float *output;          // [query_heads][head_dim]
    uint32_t query_heads;
    uint32_t position;      // attend over tokens [0, position]
    float scale;
    float *partials;        // workspace, attention_workspace_floats()
};

size_t attention_workspace_floats(const KvCache &c, uint32_t query_heads,
                                  uint32_t position);
hipError_t launch_attention(const AttentionLaunch &a, hipStream_t stream);

// Decode attention (one workgroup per KV head and split, online softmax,
// no merge pass while one split covers the context): attends q [query_heads]
// [head_dim] to tokens [0, position] (position read from position_ptr when
// given).  With key/value/cos/sin it is the decode step: RoPE on q and on
// the current key, Q8 append of key and value at the position, attention
// including them.  span_tokens fixes the split plan: the context length for
// a host-known position, max_tokens for a device position.  head_dim 64,
// 128 or 256, at most 8 query heads per KV head.
struct DecodeAttentionLaunch {
    const KvCache *cache = nullptr;
    const float *query = nullptr;
    float *output = nullptr;
    float *partials = nullptr;   // decode_attention_workspace_floats()
    uint32_t query_heads = 0;
    uint32_t position = 0;
    const int32_t *position_ptr = nullptr;
    uint32_t span_tokens = 0;
    float scale = 1.0f;
    const float *key = nullptr;
    const float *value = nullptr;
    const float *cos_tab = nullptr;   // [max_tokens][head_dim / 2], or the position's row only:
    const float *sin_tab = nullptr;
    bool rope_row_only = false;       // cos_tab / sin_tab hold just the current position's row
    uint32_t count = 1;               // > 1: a block of query tokens (no key/value): query and
                                      // output [count][query_heads][head_dim], positions
                                      // position_ptr[count], one split
    const float *q_norm = nullptr;    // with key: per-head q/k RMSNorm weights [head_dim]
    const float *k_norm = nullptr;    // before RoPE (both or neither)
    float eps = 0.0f;
    // a block of draft-tree nodes (no key/value, position_ptr their slots):
    // tree_mask[count] ancestor-or-self bits over slots *tree_base + a;
    // slots below *tree_base (the prefix) are always attended
    const uint64_t *tree_mask = nullptr;
    const int32_t *tree_base = nullptr;
};
// int8 MFMA attention (no RoPE/append) over span tokens of the cache: the
// position from position_ptr when non-null; partials of
// mfma_attention_workspace_floats floats when the span needs more than one
// split, merged into output by a second kernel (mfma_attention_launches).
bool mfma_attention_supported(const KvCache &c, uint32_t query_heads);
size_t mfma_attention_workspace_floats(const KvCache &c, uint32_t query_heads, uint32_t span);
uint32_t mfma_attention_launches(const KvCache &c, uint32_t query_heads, uint32_t span);
hipError_t launch_mfma_attention(const KvCache &c, const float *query, float *output, float *partials,
                                 uint32_t query_heads, uint32_t position, const int32_t *position_ptr,
                                 uint32_t span, float scale, hipStream_t stream,
                                 const uint64_t *tree_mask = nullptr, const int32_t *tree_base = nullptr);
bool decode_attention_supported(const KvCache &c, uint32_t query_heads);
uint32_t decode_split_tokens(const KvCache &c, uint32_t tokens);
size_t decode_attention_workspace_floats(const KvCache &c, uint32_t query_heads, uint32_t tokens);
hipError_t launch_decode_attention(const DecodeAttentionLaunch &l, hipStream_t stream);

// Device-position variants for graph replay: the token index / position is
// read from device memory when the kernels run; attention uses a fixed grid
// of kDevicePositionSplit-token splits over the whole cache, splits past
// the position writing empty partials.
constexpr uint32_t kDevicePositionSplit = 64;
hipError_t launch_kv_append_at(const KvCache &c, const float *key, const float *value,
                               const int32_t *token_ptr, hipStream_t stream);
size_t attention_at_workspace_floats(const KvCache &c, uint32_t query_heads);
// tree_mask / tree_base: a draft-tree node's ancestor mask (as in
// DecodeAttentionLaunch; needs the MFMA attention, mfma_attention_supported).
hipError_t launch_attention_at(const KvCache &c, const float *query, float *output,
                               uint32_t query_heads, const int32_t *position_ptr, float scale,
                               float *partials, hipStream_t stream, const uint64_t *tree_mask = nullptr,
                               const int32_t *tree_base = nullptr);

// Keeps a draft tree's accepted path: for k < len, the K/V and scales of
// slot base + path[k] move to slot base + k (path strictly increasing from
// a node at index >= 0, each path[k] >= k, so an in-order copy never reads
// a slot it has already overwritten).  path: device [len], len <= 64.
hipError_t launch_kv_commit_path(const KvCache &c, const int32_t *base, const int32_t *path, uint32_t len,
                                 hipStream_t stream);

}  // namespace qwn
