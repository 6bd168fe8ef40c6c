// Internal declarations shared by the qwn_hip translation units.
//
// Device layouts (chosen at upload; the ABI keeps them private):
//
//  HyperVSQ-2 (74-byte blocks of 256 weights, c/qwanto_native.h:96-103)
//    codes plane  [rows][nb][64 B]   the 2-bit codes, 16-byte aligned
//    meta  plane  [rows][nb][8 B]    {fp16 d_base, fp16 m_base, 4 bytes of
//                                     octant multipliers}; the two reserved
//                                     bytes are dropped (never read by the
//                                     reference kernels either)
//  Q4_0 (18-byte blocks of 32 weights, c/qwanto_native.h:35)
//    nibble plane [rows][nu*4][16 B] nibbles, rows padded to a multiple of
//                                     four blocks with zero blocks
//    scale  plane [rows][nu*4] fp16  zero for padding blocks
//  F16: [rows][cols] binary16, row stride padded to 16 bytes
//
// A "unit" is what one lane consumes per step: one HyperVSQ-2 block (256
// weights), four Q4_0 blocks (128 weights) or eight F16 weights.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qwn {

enum WeightKind : int { kHvsq2 = 1, kQ4_0 = 2, kF16 = 3 };

constexpr int kWaveSize = 64;
constexpr int kGemvWaves = 4;                     // waves per workgroup
constexpr int kGemvThreads = kWaveSize * kGemvWaves;
constexpr int kMaxTokensPerLaunch = 16;
constexpr size_t kGemvLdsLimit = 64 * 1024;

// Elements covered by one unit, and LDS bytes one token's unit occupies
// (activation bytes plus 16 bytes of padding so that lanes reading
// consecutive units hit different LDS banks).
__host__ __device__ constexpr int unit_elems(int kind) {
    return kind == kHvsq2 ? 256 : (kind == kQ4_0 ? 128 : 8);
}
__host__ __device__ constexpr int unit_lds_bytes(int kind) {
    return kind == kHvsq2 ? 272 : (kind == kQ4_0 ? 144 : 32);
}

struct DeviceTensor {
    int kind = 0;
    uint32_t rows = 0;
    uint32_t cols = 0;
    uint32_t units = 0;          // units per row
    uint8_t *payload = nullptr;  // codes / nibbles / halves plane
    uint8_t *meta = nullptr;     // meta / scale plane (null for F16)
    size_t payload_row_bytes = 0;
    size_t meta_row_bytes = 0;
    uint64_t device_bytes = 0;   // bytes allocated on the device
    uint64_t logical_bytes = 0;  // algorithmic (on-disk) bytes
};

// Lane mapping of one GEMV launch: each row is split across `lanes` lanes
// of a wave, each lane handling `upl` units strided by `lanes`, and a wave
// holds `rows_per_wave` such row groups.
struct GemvPlan {
    int lanes = 0;
    int upl = 0;
    int rows_per_wave = 0;
    int tokens = 0;        // tokens per launch (template width)
    int grid = 0;
    size_t lds_bytes = 0;
};

GemvPlan plan_gemv(const DeviceTensor &t, int batch);

// Repack one tensor from its on-disk bytes (already copied to `staging`
// on the device) into the device layout of `t`.
hipError_t repack_tensor(const DeviceTensor &t, const uint8_t *staging,
                         hipStream_t stream);

struct GemvLaunch {
    const DeviceTensor *tensor;
    const void *input;        // int8 [batch][input_stride] or fp32 for F16
    const float *scales;      // per-token scales (null -> scalar `scale`)
    float scale;
    float *output;            // fp32 [batch][output_stride]
    uint32_t batch;
    uint32_t input_stride;    // elements
    uint32_t output_stride;   // elements
    int32_t *debug_sums;      // non-null: dump integer sums instead
};

hipError_t launch_gemv(const GemvLaunch &g, hipStream_t stream);

// Per-token quantization on the device (c/qwanto_kernels.c:354-433):
// x fp32 [M][K] -> q8 [M][out_stride] zero padded, scales [M].
hipError_t launch_quantize_tokens(const float *x, int M, int K, int x_stride,
                                  int8_t *q8, int out_stride, float *scales,
                                  hipStream_t stream);

// ---- Q8 KV cache ------------------------------------------------------
struct KvCache {
    uint32_t max_tokens = 0;
    uint32_t kv_heads = 0;
    uint32_t head_dim = 0;
    uint32_t channels = 0;
    uint32_t groups = 0;       // ceil(channels / 64) scale groups per token
    uint32_t pages = 0;        // ceil(max_tokens / 16)
    uint32_t tokens = 0;
    int8_t *keys = nullptr;    // [pages][kv_heads][16][head_dim]
    int8_t *values = nullptr;
    float *key_scales = nullptr;    // [pages][16][groups]
    float *value_scales = nullptr;
    uint64_t bytes = 0;
};

constexpr int kKvPageTokens = 16;

// Quantize one token's fp32 K and V [channels] into slot `token`.
hipError_t launch_kv_append(const KvCache &c, const float *key,
                            const float *value, uint32_t token,
                            hipStream_t stream);

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

}  // namespace qwn
