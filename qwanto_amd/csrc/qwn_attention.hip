// Q8 KV cache: append (quantize) and split-T decode attention for gfx950.
//
// Numerics follow the CPU Q8 cache (c/qwanto_turboquant.c:555-702):
//   append:    per 64-channel group scale = amax(finite)/127 (1 if 0),
//              q = rint(clamp(v / scale, -127, 127)), non-finite -> 0
//   attention: s_t = scale * sum_c q_c * (k_c * ks), softmax over t <= pos,
//              ctx = sum_t p_t * (v_t * vs)
// The reference GPU kernel walks tokens serially with every score in
// shared memory (c/cuda/qwn_hypervsq2_cuda_abi.cu:175-223); here the token
// range is split across workgroups (flash-decoding), every K/V row is
// loaded once per KV head and reused by all query heads of its group, and a
// second pass merges the per-split (max, sum, output) triples.
//
// Layout: 16-token pages, each laid out for the MFMA operands:
//   K int8 [page][kv_head][head_dim/16][16 tokens][16 channels]: 16 channels
//     of one token are one 16-byte word and the 16 tokens of a chunk are
//     256 contiguous bytes (head_dim padded to a multiple of 16);
//   V int8 [page][kv_head][head_dim][16 tokens]: the 16 tokens of one
//     channel are one 16-byte word;
//   scales fp32 [page][group][16 tokens], groups of 64 channels over the
//     flattened kv_head*head_dim channels (the reference's grouping).
#include "qwn_device.h"
#include "qwn_internal.h"

#include <algorithm>

namespace qwn {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kMaxSplitTokens = 256;

// Each KV head's pages are contiguous, so a workgroup streaming one head's
// span of the context reads one contiguous run of keys and one of values.
// key byte of (token, head, channel); channels 16q .. 16q + 15 of a token
// are the 16 bytes at k_index(token, head, 16q)
__device__ __forceinline__ size_t k_index(const KvCache &c, uint32_t token, uint32_t head, uint32_t dim) {
    const uint32_t page = token / kKvPageTokens, slot = token % kKvPageTokens;
    const uint32_t chunks = (c.head_dim + 15) / 16;
    return (((static_cast<size_t>(head) * c.pages + page) * chunks + dim / 16) * kKvPageTokens + slot) * 16 +
           dim % 16;
}

// value byte of (token, head, channel)
__device__ __forceinline__ size_t v_offset(const KvCache &c, uint32_t token, uint32_t head, uint32_t dim) {
    const uint32_t page = token / kKvPageTokens, slot = token % kKvPageTokens;
    return ((static_cast<size_t>(head) * c.pages + page) * c.head_dim + dim) * kKvPageTokens + slot;
}

// the 16 value bytes of (page, head, channel)
__device__ __forceinline__ size_t v_page_offset(const KvCache &c, uint32_t page, uint32_t head, uint32_t dim) {
    return ((static_cast<size_t>(head) * c.pages + page) * c.head_dim + dim) * kKvPageTokens;
}

__device__ __forceinline__ void store_q8(const KvCache &c, bool is_v, uint32_t token, uint32_t head, uint32_t dim,
                                         int8_t q) {
    if (is_v) c.values[v_offset(c, token, head, dim)] = q;
    else c.keys[k_index(c, token, head, dim)] = q;
}

// scale of (token, group): [group][64-token quad][slot 0..15][page of the
// quad 0..3], so the four floats at scale_index(64q + slot, g) are the
// scales of tokens slot, 16 + slot, 32 + slot, 48 + slot of quad q
__device__ __forceinline__ size_t scale_index(const KvCache &c, uint32_t token, uint32_t group) {
    return ((static_cast<size_t>(group) * c.quads + token / (4 * kKvPageTokens)) * kKvPageTokens +
            token % kKvPageTokens) * 4 + (token / kKvPageTokens) % 4;
}

// grid (groups, 2, tokens): y = 0 quantizes K, y = 1 quantizes V; z is the
// token of a block of consecutive tokens (key/value [z][channels], slot
// token + z).  64 threads, one per channel of the group.
__global__ __launch_bounds__(64) void kv_append_kernel(KvCache c, const float *__restrict__ key,
                                                       const float *__restrict__ value, uint32_t token,
                                                       const int32_t *__restrict__ token_ptr) {
    if (token_ptr) token = static_cast<uint32_t>(*token_ptr);
    token += blockIdx.z;
    if (token >= c.max_tokens) return;
    const uint32_t g = blockIdx.x;
    const bool is_v = blockIdx.y == 1;
    const float *src = (is_v ? value : key) + static_cast<size_t>(blockIdx.z) * c.channels;
    const uint32_t ch = g * 64 + threadIdx.x;
    const bool valid = ch < c.channels;
    const float v = valid ? src[ch] : 0.0f;
    float amax = (valid && isfinite(v)) ? fabsf(v) : 0.0f;
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    if (threadIdx.x == 0) (is_v ? c.value_scales : c.key_scales)[scale_index(c, token, g)] = scale;
    if (valid) {
        int8_t q = 0;
        if (isfinite(v)) {
            const float s = v / scale;  // IEEE division, like the CPU path
            q = s >= 127.0f ? 127 : (s <= -127.0f ? -127 : static_cast<int8_t>(__builtin_rintf(s)));
        }
        store_q8(c, is_v, token, ch / c.head_dim, ch % c.head_dim, q);
    }
}

// Token-major copy of tokens [first, first + count): keys/values
// [count][channels] int8 and scales [count][groups] fp32, the CPU cache's
// layout (c/qwanto_turboquant.h:78-94), read through the same index
// functions the attention kernels use.
__global__ __launch_bounds__(256) void kv_gather_kernel(KvCache c, uint32_t first, uint32_t count,
                                                        int8_t *__restrict__ keys, int8_t *__restrict__ values,
                                                        float *__restrict__ key_scales,
                                                        float *__restrict__ value_scales) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx < static_cast<uint64_t>(count) * c.channels) {
        const uint32_t t = static_cast<uint32_t>(idx / c.channels), ch = static_cast<uint32_t>(idx % c.channels);
        const uint32_t head = ch / c.head_dim, dim = ch % c.head_dim;
        keys[idx] = c.keys[k_index(c, first + t, head, dim)];
        values[idx] = c.values[v_offset(c, first + t, head, dim)];
    }
    if (idx < static_cast<uint64_t>(count) * c.groups) {
        const uint32_t t = static_cast<uint32_t>(idx / c.groups), g = static_cast<uint32_t>(idx % c.groups);
        key_scales[idx] = c.key_scales[scale_index(c, first + t, g)];
        value_scales[idx] = c.value_scales[scale_index(c, first + t, g)];
    }
}

// A draft tree's accepted path into consecutive slots: thread i < channels
// moves channel i's key and value bytes, thread i < groups the group's two
// scales, for k = 0, 1, ... in order (slot base + path[k] -> base + k; the
// path is strictly increasing with path[k] >= k, so no source slot is read
// after this thread overwrote it, and no two threads touch one byte).
__global__ __launch_bounds__(256) void kv_commit_path_kernel(KvCache c, const int32_t *__restrict__ base_ptr,
                                                             const int32_t *__restrict__ path, uint32_t len) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t base = static_cast<uint32_t>(*base_ptr);
    if (idx < c.channels) {
        const uint32_t head = idx / c.head_dim, dim = idx % c.head_dim;
        for (uint32_t k = 0; k < len; ++k) {
            const uint32_t src = base + static_cast<uint32_t>(path[k]), dst = base + k;
            if (src >= c.max_tokens) break;
            c.keys[k_index(c, dst, head, dim)] = c.keys[k_index(c, src, head, dim)];
            c.values[v_offset(c, dst, head, dim)] = c.values[v_offset(c, src, head, dim)];
        }
    }
    if (idx < c.groups) {
        for (uint32_t k = 0; k < len; ++k) {
            const uint32_t src = base + static_cast<uint32_t>(path[k]), dst = base + k;
            if (src >= c.max_tokens) break;
            c.key_scales[scale_index(c, dst, idx)] = c.key_scales[scale_index(c, src, idx)];
            c.value_scales[scale_index(c, dst, idx)] = c.value_scales[scale_index(c, src, idx)];
        }
    }
}

struct AttnArgs {
    KvCache c;
    const float *query;
    float *partials;  // [query_heads][nsplit][head_dim + 2]
    uint32_t query_heads;
    uint32_t group;   // query heads per kv head
    uint32_t tokens;  // position + 1
    uint32_t split;   // tokens per split
    uint32_t nsplit;
    float scale;
    const int32_t *position_ptr;  // non-null: tokens = *position_ptr + 1 (fixed split grid)
    uint32_t head_mapped;         // 1: blockIdx.y is a query head (group 1), its KV head
                                  // head * kv_heads / query_heads (any head ratio)
};

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float i8(uint32_t w, int i) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * i)) & 0xffu));
}

// One workgroup = one KV head x one split of <= 256 tokens.
// FAST: head_dim % 16 == 0 and head_dim <= 256 (16-byte row loads, one
// scale per 16-channel chunk); otherwise channel-by-channel.
template <int GMAX, bool FAST>
__global__ __launch_bounds__(kAttnThreads) void attention_split_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float sm[];
    const KvCache &c = a.c;
    const uint32_t D = c.head_dim;
    // query heads hbase .. hbase + G - 1 read KV head kvh
    const uint32_t kvh = a.head_mapped ? blockIdx.y * c.kv_heads / a.query_heads : blockIdx.y;
    const uint32_t G = a.group;
    const uint32_t hbase = a.head_mapped ? blockIdx.y : blockIdx.y * G;
    const uint32_t split = blockIdx.x;
    const uint32_t t0 = split * a.split;
    const uint32_t tokens = a.position_ptr ? static_cast<uint32_t>(*a.position_ptr) + 1u : a.tokens;
    if (t0 >= tokens) {
        // a split past the current position (fixed grid): an empty partial
        for (uint32_t i = threadIdx.x; i < G * D; i += blockDim.x) {
            const uint32_t g = i / D, d = i % D;
            float *dst = a.partials + (static_cast<size_t>(hbase + g) * a.nsplit + split) * (D + 2);
            dst[2 + d] = 0.0f;
            if (d == 0) {
                dst[0] = -INFINITY;
                dst[1] = 0.0f;
            }
        }
        return;
    }
    const uint32_t n = min(a.split, tokens - t0);
    float *q = sm;                              // [GMAX][D]
    float *p = q + GMAX * D;                    // [split][GMAX]
    float *wred = p + kMaxSplitTokens * GMAX;   // [4 waves][GMAX]
    float *pv = wred + 4 * GMAX;                // PV reduction [phases][GMAX][D]

    for (uint32_t i = threadIdx.x; i < GMAX * D; i += blockDim.x) {
        const uint32_t g = i / D, d = i % D;
        q[i] = g < G ? a.query[(static_cast<size_t>(hbase) + g) * D + d] : 0.0f;
    }
    __syncthreads();

    // ---- scores: one thread per token, all query heads of the group ----
    const uint32_t t = threadIdx.x;
    float s[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) s[g] = -INFINITY;
    if (t < n) {
        const uint32_t tok = t0 + t;
        float dot[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) dot[g] = 0.0f;
        if (FAST) {
            for (uint32_t c0 = 0; c0 < D; c0 += 16) {
                const uint4 kw = *reinterpret_cast<const uint4 *>(c.keys + k_index(c, tok, kvh, c0));
                const float sc = c.key_scales[scale_index(c, tok, (kvh * D + c0) / 64)];
                const uint32_t w[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    float kf[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) kf[i] = i8(w[qd], i) * sc;
#pragma unroll
                    for (int g = 0; g < GMAX; ++g) {
                        if (g >= static_cast<int>(G)) break;
                        const float4 qq = *reinterpret_cast<const float4 *>(q + g * D + c0 + qd * 4);
                        dot[g] = fmaf(qq.x, kf[0], dot[g]);
                        dot[g] = fmaf(qq.y, kf[1], dot[g]);
                        dot[g] = fmaf(qq.z, kf[2], dot[g]);
                        dot[g] = fmaf(qq.w, kf[3], dot[g]);
                    }
                }
            }
        } else {
            for (uint32_t d = 0; d < D; ++d) {
                const float kf = static_cast<float>(c.keys[k_index(c, tok, kvh, d)]) *
                                 c.key_scales[scale_index(c, tok, (kvh * D + d) / 64)];
#pragma unroll
                for (int g = 0; g < GMAX; ++g)
                    if (g < static_cast<int>(G)) dot[g] = fmaf(q[g * D + d], kf, dot[g]);
            }
        }
#pragma unroll
        for (int g = 0; g < GMAX; ++g) s[g] = g < static_cast<int>(G) ? dot[g] * a.scale : -INFINITY;
    }

    // ---- split-local softmax statistics ----
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    float m[GMAX], l[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        const float wm = wave_max(s[g]);
        if (lane == 0) wred[wave * GMAX + g] = wm;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
        m[g] = fmaxf(fmaxf(wred[g], wred[GMAX + g]), fmaxf(wred[2 * GMAX + g], wred[3 * GMAX + g]));
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        const float e = (t < n && g < static_cast<int>(G)) ? expf(s[g] - m[g]) : 0.0f;
        if (t < kMaxSplitTokens) p[t * GMAX + g] = e;
        const float ws = wave_sum(e);
        if (lane == 0) wred[wave * GMAX + g] = ws;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GMAX; ++g) l[g] = (wred[g] + wred[GMAX + g]) + (wred[2 * GMAX + g] + wred[3 * GMAX + g]);

    // ---- P.V: thread = (channel quad, token phase), all heads of the group ----
    const uint32_t quads = (D + 3) / 4;
    const uint32_t phases = blockDim.x / quads;  // >= 1 since D <= 1024
    const uint32_t quad = threadIdx.x % quads, phase = threadIdx.x / quads;
    float acc[GMAX][4];
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[g][i] = 0.0f;
    if (phase < phases) {
        for (uint32_t tt = phase; tt < n; tt += phases) {
            const uint32_t tok = t0 + tt;
            float vf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t d = quad * 4 + i;
                vf[i] = d < D ? static_cast<float>(c.values[v_offset(c, tok, kvh, d)]) *
                                    c.value_scales[scale_index(c, tok, (kvh * D + d) / 64)]
                              : 0.0f;
            }
#pragma unroll
            for (int g = 0; g < GMAX; ++g) {
                if (g >= static_cast<int>(G)) break;
                const float pg = p[tt * GMAX + g];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(pg, vf[i], acc[g][i]);
            }
        }
    }
    // reduce the phases through LDS
    for (uint32_t i = threadIdx.x; i < phases * GMAX * D; i += blockDim.x) pv[i] = 0.0f;
    __syncthreads();
    if (phase < phases) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t d = quad * 4 + i;
                if (g < static_cast<int>(G) && d < D) pv[(phase * GMAX + g) * D + d] = acc[g][i];
            }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < G * D; i += blockDim.x) {
        const uint32_t g = i / D, d = i % D;
        float o = 0.0f;
        for (uint32_t ph = 0; ph < phases; ++ph) o += pv[(ph * GMAX + g) * D + d];
        const uint32_t head = hbase + g;
        float *dst = a.partials + (static_cast<size_t>(head) * a.nsplit + split) * (D + 2);
        dst[2 + d] = o;
        if (d == 0) {
            dst[0] = m[g];
            dst[1] = l[g];
        }
    }
}

// grid (query_heads): merge the split partials of one head (empty splits
// carry m = -inf, l = 0 and drop out).
__global__ __launch_bounds__(256) void attention_merge_kernel(const float *__restrict__ partials,
                                                              float *out, uint32_t nsplit, uint32_t D) {
    const uint32_t head = blockIdx.x;
    const float *base = partials + static_cast<size_t>(head) * nsplit * (D + 2);
    float mx = -INFINITY;
    for (uint32_t sidx = 0; sidx < nsplit; ++sidx) mx = fmaxf(mx, base[sidx * (D + 2)]);
    float total = 0.0f;
    for (uint32_t sidx = 0; sidx < nsplit; ++sidx)
        total += base[sidx * (D + 2) + 1] * expf(base[sidx * (D + 2)] - mx);
    const float inv = total > 0.0f ? 1.0f / total : 0.0f;
    for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
        float o = 0.0f;
        for (uint32_t sidx = 0; sidx < nsplit; ++sidx)
            o = fmaf(base[sidx * (D + 2) + 2 + d], expf(base[sidx * (D + 2)] - mx), o);
        out[static_cast<size_t>(head) * D + d] = o * inv;
    }
}

uint32_t split_tokens(const KvCache &c, uint32_t tokens) {
    // aim for >= 1024 workgroups over the KV heads, 16..256 tokens each
    uint32_t s = (tokens * c.kv_heads + 1023) / 1024;
    s = (s + 15) / 16 * 16;
    return std::min<uint32_t>(std::max<uint32_t>(s, 16), kMaxSplitTokens);
}

template <int GMAX, bool FAST>
hipError_t launch_split(const AttnArgs &args, hipStream_t stream) {
    const uint32_t D = args.c.head_dim;
    const uint32_t quads = (D + 3) / 4;
    const uint32_t phases = kAttnThreads / quads;
    const size_t lds = (static_cast<size_t>(GMAX) * D + kMaxSplitTokens * GMAX + 4 * GMAX +
                        static_cast<size_t>(phases) * GMAX * D) * sizeof(float);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const uint32_t rows = args.head_mapped ? args.query_heads : args.c.kv_heads;
    hipLaunchKernelGGL((attention_split_kernel<GMAX, FAST>), dim3(args.nsplit, rows),
                       dim3(kAttnThreads), lds, stream, args);
    return hipGetLastError();
}

template <int GMAX>
hipError_t launch_fast_or_not(const AttnArgs &args, hipStream_t stream) {
    const uint32_t D = args.c.head_dim;
    if (D % 16 == 0 && D <= 256) return launch_split<GMAX, true>(args, stream);
    return launch_split<GMAX, false>(args, stream);
}

}  // namespace

namespace {

// One workgroup: RoPE on the query heads (in place) and on the key, then the
// Q8 append of the rotated key and of the value at slot *pos_ptr.  The
// rotation is the reference's NeoX half split with its fused multiply-adds
// (c/qwanto_decode.c:686-729):
//   r[i] = fma(a, cos_i, -(b * sin_i)),  r[i + half] = fma(a, sin_i, b * cos_i)
// with a = x[i], b = x[i + half] and the cos/sin table row of the position;
// the append quantizes per 64-channel group as kv_append_kernel.  grid (n):
// workgroup i takes token i of a block -- q + i*q_stride, k/v + i*kv_stride,
// cache slot pos_ptr[i], rotated for position rope_pos_ptr[i] (the slot
// when null; a draft tree's node sits at slot P + index but position
// P + depth).
__global__ __launch_bounds__(1024) void rope_append_kernel(KvCache c, float *__restrict__ q, uint32_t q_heads,
                                                           const float *__restrict__ k,
                                                           const float *__restrict__ v,
                                                           const float *__restrict__ cos_tab,
                                                           const float *__restrict__ sin_tab,
                                                           const int32_t *__restrict__ pos_ptr, uint32_t q_stride,
                                                           uint32_t kv_stride, const float *__restrict__ q_norm,
                                                           const float *__restrict__ k_norm, float eps,
                                                           const int32_t *__restrict__ rope_pos_ptr) {
    extern __shared__ float kr[];  // [channels] rotated key
    __shared__ float inv_s[kMaxNormHeads];
    q += static_cast<size_t>(blockIdx.x) * q_stride;
    k += static_cast<size_t>(blockIdx.x) * kv_stride;
    v += static_cast<size_t>(blockIdx.x) * kv_stride;
    const uint32_t pos = static_cast<uint32_t>(pos_ptr[blockIdx.x]);
    const uint32_t rpos = rope_pos_ptr ? static_cast<uint32_t>(rope_pos_ptr[blockIdx.x]) : pos;
    const uint32_t D = c.head_dim, half = D / 2;
    const uint32_t row = rpos < c.max_tokens ? rpos : 0;
    const float *ct = cos_tab + static_cast<size_t>(row) * half;
    const float *st = sin_tab + static_cast<size_t>(row) * half;
    // the value this thread quantizes first (group gi = wave of the quantize
    // loop below), loaded with the rotation's inputs rather than after the
    // barrier
    const uint32_t gi0 = threadIdx.x / 64, ch0 = (gi0 - c.groups) * 64 + threadIdx.x % 64;
    const bool v0 = gi0 >= c.groups && gi0 < 2 * c.groups && ch0 < c.channels;
    const float vpre = v[v0 ? ch0 : 0];
    // per-head q/k RMSNorm ahead of the rotation (c/qwanto_decode.c:654-684,
    // 1652-1655): one wave per head for its 1/rms, applied as (x * inv) * w
    const bool qk = q_norm != nullptr;
    if (qk) {
        const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64, nwaves = blockDim.x / 64;
        for (uint32_t hh = wave; hh < q_heads + c.kv_heads; hh += nwaves) {
            const float *x = hh < q_heads ? q + static_cast<size_t>(hh) * D : k + static_cast<size_t>(hh - q_heads) * D;
            float ss = 0.0f;
            for (uint32_t d = lane; d < D; d += 64) ss = fmaf(x[d], x[d], ss);
            ss = wave_sum_all(ss);
            if (lane == 0) inv_s[hh] = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
        }
        lds_barrier();
    }
    for (uint32_t p = threadIdx.x; p < q_heads * half; p += blockDim.x) {
        const uint32_t h = p / half, i = p % half;
        float *r = q + static_cast<size_t>(h) * D;
        float a = r[i], b = r[i + half];
        if (qk) {
            a = (a * inv_s[h]) * q_norm[i];
            b = (b * inv_s[h]) * q_norm[i + half];
        }
        r[i] = fmaf(a, ct[i], -(b * st[i]));
        r[i + half] = fmaf(a, st[i], b * ct[i]);
    }
    for (uint32_t p = threadIdx.x; p < c.kv_heads * half; p += blockDim.x) {
        const uint32_t h = p / half, i = p % half;
        float a = k[h * D + i], b = k[h * D + i + half];
        if (qk) {
            a = (a * inv_s[q_heads + h]) * k_norm[i];
            b = (b * inv_s[q_heads + h]) * k_norm[i + half];
        }
        kr[h * D + i] = fmaf(a, ct[i], -(b * st[i]));
        kr[h * D + i + half] = fmaf(a, st[i], b * ct[i]);
    }
    lds_barrier();   // the rotated keys; the rotated queries go to memory, read by a later launch
    if (pos >= c.max_tokens) return;
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64, nwaves = blockDim.x / 64;
    for (uint32_t gi = wave; gi < 2 * c.groups; gi += nwaves) {
        const bool is_v = gi >= c.groups;
        const uint32_t g = is_v ? gi - c.groups : gi;
        const uint32_t ch = g * 64 + lane;
        const bool valid = ch < c.channels;
        const float x = valid ? (is_v ? (gi == gi0 ? vpre : v[ch]) : kr[ch]) : 0.0f;
        float amax = (valid && isfinite(x)) ? fabsf(x) : 0.0f;
        for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        if (lane == 0) (is_v ? c.value_scales : c.key_scales)[scale_index(c, pos, g)] = scale;
        if (valid) {
            int8_t qv = 0;
            if (isfinite(x)) {
                const float sq = x / scale;  // IEEE division, like the CPU path
                qv = sq >= 127.0f ? 127 : (sq <= -127.0f ? -127 : static_cast<int8_t>(__builtin_rintf(sq)));
            }
            store_q8(c, is_v, pos, ch / D, ch % D, qv);
        }
    }
}

// ---- decode attention -------------------------------------------------------
//
// One workgroup of 256 x TPT threads per query head, the whole context (up
// to 1024 tokens) in one split: the short-context decode step, bound by
// memory latency, the rate one CU pulls a chunk in (~70 KB for 256 tokens)
// and the per-token arithmetic, not by bytes (a KV head's query heads read
// its rows from L2).  Online softmax over chunks of 256 tokens; every load
// of a chunk is one round trip, the first chunk's issued with the query's
// before anything waits.
//   scores: TPT adjacent lanes per token, each D/TPT channels of its key
//           row, scaled per 64-channel group, summed by lane swaps
//   P.V:    thread = (channel, phase of 4-token groups); the chunk's value
//           words (16 tokens of one channel) staged in LDS in the cache's
//           own channel-major page order; phases summed through LDS at the
//           end
//
// Decode mode (key != null): RoPE on the query head (c/qwanto_decode.c:
// 686-729), optionally after a per-head RMSNorm of query and key (654-684),
// and the current key (rotated) and value Q8-quantized (c/qwanto_turboquant.c:
// 555-600), stored in the cache for later steps and attended to from LDS.
// Prefill mode (key == null): grid z is the query token of a block, its
// query already rotated and its key/value already in the cache.
struct DecodeAttnArgs {
    KvCache c;
    const float *query;      // [H][D]
    float *output;           // [H][D]
    uint32_t group;          // query heads per KV head
    uint32_t span;           // attends to tokens [0, min(position + 1, span))
    float scale;
    uint32_t position;
    const int32_t *position_ptr;
    const float *key;        // decode mode: current token fp32 [channels]
    const float *value;
    const float *cos_tab;    // [max_tokens][D/2], or [D/2] for the current position (rope_row_only)
    const float *sin_tab;
    uint32_t rope_row_only;
    uint32_t token_stride;   // floats between the query (and output) rows of a token block
    uint32_t count;          // query tokens (grid z)
    const float *q_norm;     // decode mode, optional: per-head q/k RMSNorm weights [head_dim]
    const float *k_norm;
    float eps;
    // prefill mode, optional: a draft tree's ancestor masks, one per query
    // token; slot *tree_base + a is attended only where bit a is set (slots
    // below *tree_base, the prefix, always)
    const uint64_t *tree_mask;
    const int32_t *tree_base;
};

// Whether slot t is attended under a tree mask relative to slot `base`
// (no tree: tree_bits() gives all ones).  The 64-bit test is a lookup of
// the mask's two halves by the slot's offset, written without any shift by
// a wrapped offset: an earlier form, t < base || (mask >> min(t - base,
// 63)) & 1, was compiled into the shift alone (the t < base test dropped),
// which masked every token.
__device__ __forceinline__ bool tree_attends(uint32_t t, uint32_t base, uint64_t mask) {
    const uint32_t off = t - base;  // the slot's tree index when t >= base
    const uint32_t half = off < 32u ? static_cast<uint32_t>(mask) : static_cast<uint32_t>(mask >> 32);
    const bool bit = ((half >> (off & 31u)) & 1u) != 0u;
    return t < base || (off < 64u && bit);
}

__device__ __forceinline__ int8_t q8_of(float x, float scale) {
    if (!isfinite(x)) return 0;
    const float s = x / scale;  // IEEE division, like the CPU path
    return s >= 127.0f ? 127 : (s <= -127.0f ? -127 : static_cast<int8_t>(__builtin_rintf(s)));
}

__device__ __forceinline__ float i8f(uint32_t w, int i) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * i)) & 0xffu));
}

template <int D, int TPT>
__global__ __launch_bounds__(256 * TPT) void decode_attention_kernel(DecodeAttnArgs a) {
    constexpr int NT = 256 * TPT, NW = NT / 64;
    constexpr int LW = NW / 2;                 // loader waves: the upper half of the workgroup
    constexpr int NG = D / 64;                 // Q8 scale groups per head
    constexpr int CH = 256;                    // tokens per chunk, TPT lanes each in the scores
    constexpr int KCH = D / 16;                // 16-channel key chunks per token
    constexpr int CPT = D / TPT;               // key channels per lane
    constexpr int KWT = CPT / 16;              // 16-byte key words per lane
    constexpr int KGL = CPT >= 64 ? CPT / 64 : 1;    // key scale groups per lane
    constexpr int WPG = KWT / KGL;                   // key words per lane and group
    constexpr int VGL = (NG + TPT - 1) / TPT;        // value scale groups per lane
    constexpr int PH = NT / D;                 // P.V: phases of 4-token groups
    constexpr int TSTEP = 4 * PH;              // P.V: token stride of a thread
    constexpr int NIT = CH / TSTEP;            // P.V: a thread's 4-token groups per chunk
    constexpr int KBLK = CH * D / 1024;        // 1 KB blocks of the chunk's keys (and of its values)
    constexpr uint32_t half = D / 2;
    static_assert(NT / TPT == CH && (CPT >= 64 ? CPT % 64 == 0 : 64 % CPT == 0) && PH >= 1 && NIT % 4 == 0 &&
                      D % 64 == 0 && NG <= LW && KBLK % LW == 0,
                  "decode attention geometry");
    // the chunk as the cache holds it (16 pages from a page boundary)
    __shared__ __align__(16) int8_t k_l[CH * D];       // keys [page][16-channel chunk][slot][16]
    __shared__ __align__(16) int8_t v_l[CH * D];       // values [page][channel][slot]
    __shared__ __align__(16) float ksc_l[NG][CH];      // scales per group [quad][slot][page of the quad]
    __shared__ __align__(16) float vsc_l[NG][CH];
    __shared__ __align__(16) int8_t qp_s[3][D];        // the query as three int8 pieces
    __shared__ float qs_s[NG];                         // the first piece's scale per group
    __shared__ __align__(16) float pw_s[NG][CH];       // softmax weight x value scale, per group and slot
    __shared__ float red[2][NW];
    __shared__ __align__(16) float pv_s[PH * D];
    __shared__ __align__(16) int8_t kcur[D];
    __shared__ __align__(16) int8_t vcur[D];
    __shared__ float kcur_s[NG], vcur_s[NG];
    __shared__ float nrm_s[8];
    const KvCache &c = a.c;
    const uint32_t head = blockIdx.y, kvh = head / a.group;
    const bool writer = head % a.group == 0;  // appends the current token
    const uint32_t tid = threadIdx.x, lane = tid % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / 64);
    // a wave's 64 / TPT slots, each in lanes l, l + 64 / TPT, ...: the
    // lanes of one part read consecutive 16-byte key words of LDS (no bank
    // conflicts), the parts of a slot are combined with one lane swizzle
    constexpr uint32_t SPW = 64 / TPT;        // slots per wave
    const uint32_t slot = wave * SPW + lane % SPW, part = lane / SPW;
    const uint32_t kgrp = part * CPT / 64;     // first scale group of this lane's key channels
    const float *query = a.query + static_cast<size_t>(blockIdx.z) * a.token_stride + static_cast<size_t>(head) * D;
    float *out = a.output + static_cast<size_t>(blockIdx.z) * a.token_stride + static_cast<size_t>(head) * D;
    const bool rope = a.key != nullptr;
    const bool qk = rope && a.q_norm != nullptr;
    const bool row_only = rope && a.rope_row_only;
    // Pin the argument fields of every early load: one batch of scalar
    // loads and one wait ahead of the vector loads (a field read first at
    // its use puts a dependent scalar round trip in front of the loads).
    {
        const uint64_t pk = reinterpret_cast<uint64_t>(c.keys), pv = reinterpret_cast<uint64_t>(c.values);
        const uint64_t pks = reinterpret_cast<uint64_t>(c.key_scales);
        const uint64_t pvs = reinterpret_cast<uint64_t>(c.value_scales);
        const uint64_t pq = reinterpret_cast<uint64_t>(a.query), pkey = reinterpret_cast<uint64_t>(a.key);
        const uint64_t pval = reinterpret_cast<uint64_t>(a.value), pct = reinterpret_cast<uint64_t>(a.cos_tab);
        const uint64_t pst = reinterpret_cast<uint64_t>(a.sin_tab), pqn = reinterpret_cast<uint64_t>(a.q_norm);
        const uint64_t pkn = reinterpret_cast<uint64_t>(a.k_norm), ppos = reinterpret_cast<uint64_t>(a.position_ptr);
        asm volatile("" ::"s"(pk), "s"(pv), "s"(pks), "s"(pvs), "s"(pq), "s"(pkey), "s"(pval), "s"(pct), "s"(pst),
                     "s"(pqn), "s"(pkn), "s"(ppos), "s"(c.pages), "s"(c.quads), "s"(c.max_tokens), "s"(a.group),
                     "s"(a.token_stride), "s"(a.rope_row_only));
    }

    // The loader waves copy a chunk of 256 tokens (pages p0 .. p0 + 15,
    // clamped to the cache's last page / quad) straight into LDS: one 1 KB
    // block per wave instruction, keys and values each a contiguous run of
    // the KV head's pages, then each group's key and value scales (four
    // 64-token quads, 1 KB).  Tokens past the readable ones are masked later.
    auto issue_chunk = [&](uint32_t c0) {
        const uint32_t lw = wave - LW;
        const uint32_t p0 = c0 / kKvPageTokens, pmax = c.pages - 1, qmax = c.quads - 1;
#pragma unroll
        for (int jj = 0; jj < KBLK / LW; ++jj) {
            const uint32_t j = jj * LW + lw, off = j * 1024 + lane * 16;
            const uint32_t pg = min(p0 + off / (D * 16), pmax);
            const size_t src = (static_cast<size_t>(kvh) * c.pages + pg) * (D * 16) + off % (D * 16);
            __builtin_amdgcn_global_load_lds(c.keys + src, (lds_void *)(k_l + j * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(c.values + src, (lds_void *)(v_l + j * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int bb = 0; bb < (2 * NG + LW - 1) / LW; ++bb) {
            const uint32_t b = bb * LW + lw;
            if (b < 2u * NG) {
                const uint32_t g = b % NG;
                const uint32_t q = min(c0 / (4 * kKvPageTokens) + lane / 16, qmax);
                const size_t src = (static_cast<size_t>(kvh * NG + g) * c.quads + q) * 64 + (lane % 16) * 4;
                if (b < static_cast<uint32_t>(NG))
                    __builtin_amdgcn_global_load_lds(c.key_scales + src, (lds_void *)(&ksc_l[g][0]), 16, 0, 0);
                else
                    __builtin_amdgcn_global_load_lds(c.value_scales + src, (lds_void *)(&vsc_l[g][0]), 16, 0, 0);
            }
        }
    };

    // 0. The loads.  Loader waves: the first chunk (it does not depend on
    //    the position: its tokens past the position are masked).  Waves
    //    w < NG, the prologue's: channel d = tid of the query with its RoPE
    //    partner, of the current key and value, the norm weights and
    //    cos/sin (a wave's loads return in issue order, so the prologue
    //    never waits behind the chunk).  Only a RoPE table indexed by the
    //    position waits for the position.
    // the current value's quantization takes waves NG .. 2NG-1 where they
    // are not loaders (head_dim <= 128), else it joins the query's waves
    constexpr bool VSEP = 2 * NG <= LW;
    const bool loader = wave >= static_cast<uint32_t>(LW);
    const bool prep = wave < static_cast<uint32_t>(NG);
    const bool vprep = VSEP ? (wave >= static_cast<uint32_t>(NG) && wave < 2u * NG) : prep;
    const uint32_t vwave = VSEP ? wave - NG : wave;   // value group of a vprep wave
    const uint32_t qd = tid % D, qi = qd < half ? qd : qd - half;
    float qa = 0.0f, qb = 0.0f, ka = 0.0f, kb = 0.0f, va = 0.0f;
    float qwa = 0.0f, qwb = 0.0f, kwa = 0.0f, kwb = 0.0f, cs = 0.0f, sn = 0.0f;
    const float *ct = a.cos_tab, *st = a.sin_tab;
    if (loader) {
        issue_chunk(0);
    } else if (prep) {
        qa = query[rope ? qi : qd];
        qb = query[qi + half];
        if (rope) {
            const float *kh = a.key + static_cast<size_t>(kvh) * D;
            ka = kh[qi];
            kb = kh[qi + half];
            if (!VSEP) va = a.value[static_cast<size_t>(kvh) * D + qd];
            if (row_only) {
                cs = ct[qi];
                sn = st[qi];
            }
            if (qk) {
                qwa = a.q_norm[qi];
                qwb = a.q_norm[qi + half];
                kwa = a.k_norm[qi];
                kwb = a.k_norm[qi + half];
            }
        }
    } else if (VSEP && vprep && rope) {
        va = a.value[static_cast<size_t>(kvh) * D + qd];
    }
    const uint32_t pos = a.position_ptr ? static_cast<uint32_t>(a.position_ptr[blockIdx.z]) : a.position;
    const bool ok = pos < c.max_tokens;   // else the workgroup writes nothing and ends
    if (prep && rope && !row_only && ok) {
        // a full RoPE table: the position's row
        cs = ct[static_cast<size_t>(pos) * half + qi];
        sn = st[static_cast<size_t>(pos) * half + qi];
    }
    const uint32_t t1 = min(pos + 1, a.span);
    const bool cur = ok && rope && pos < t1;
    const uint64_t tmask = a.tree_mask ? a.tree_mask[blockIdx.z] : 0ull;
    const uint32_t tbase = a.tree_mask ? static_cast<uint32_t>(*a.tree_base) : 0xffffffffu;

    // 1. q/k norms: 1/rms of the query head and of the current key head
    //    from the prologue waves' sums of squares
    float qinv = 1.0f, kinv = 1.0f;
    if (qk) {
        if (prep) {
            const float qs2 = wave_sum_all((qd < half ? qa : qb) * (qd < half ? qa : qb));
            const float ks2 = wave_sum_all((qd < half ? ka : kb) * (qd < half ? ka : kb));
            if (lane == 0) {
                nrm_s[wave] = qs2;
                nrm_s[4 + wave] = ks2;
            }
        }
        lds_barrier();
        float sq = 0.0f, sk = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            sq += nrm_s[g];
            sk += nrm_s[4 + g];
        }
        qinv = 1.0f / sqrtf(sq / static_cast<float>(D) + a.eps);
        kinv = 1.0f / sqrtf(sk / static_cast<float>(D) + a.eps);
    }

    // 2. Wave w < NG: query group w (normed and rotated in decode mode) as
    //    three int8 pieces, q = s (q1 + q2 / 128 + q3 / 16384) with
    //    s = max|q| / 127, each piece the rounded remainder of the ones
    //    before: the scores are exact integer dot products with the int8
    //    keys and the representation error is at most s / 32768 per channel
    //    (below the fp32 rounding of max|q|); a non-finite query makes s NaN,
    //    and so its scores.  Then the current token's key group w (normed,
    //    rotated), Q8-quantized; its value groups in the vprep waves.
    if (prep) {
        float v = qa;
        float xk = 0.0f;
        if (rope) {
            float x0 = qa, x1 = qb, y0 = ka, y1 = kb;
            if (qk) {
                x0 = (x0 * qinv) * qwa;
                x1 = (x1 * qinv) * qwb;
                y0 = (y0 * kinv) * kwa;
                y1 = (y1 * kinv) * kwb;
            }
            v = qd < half ? fmaf(x0, cs, -(x1 * sn)) : fmaf(x0, sn, x1 * cs);
            xk = qd < half ? fmaf(y0, cs, -(y1 * sn)) : fmaf(y0, sn, y1 * cs);
        }
        const bool fin = isfinite(v);
        const float amax = wave_max_all(fin ? fabsf(v) : 0.0f);
        const float bad = wave_max_all(fin ? 0.0f : 1.0f);
        const float s1 = amax > 0.0f ? amax / 127.0f : 0.0f;
        const float inv1 = amax > 0.0f ? 127.0f / amax : 0.0f;
        const float x = fin ? v : 0.0f;
        const float p1 = fminf(127.0f, fmaxf(-127.0f, __builtin_rintf(x * inv1)));
        const float r1 = fmaf(-p1, s1, x);
        const float p2 = fminf(127.0f, fmaxf(-127.0f, __builtin_rintf(r1 * (inv1 * 128.0f))));
        const float r2 = fmaf(-p2, s1 * 0x1p-7f, r1);
        const float p3 = fminf(127.0f, fmaxf(-127.0f, __builtin_rintf(r2 * (inv1 * 16384.0f))));
        qp_s[0][qd] = static_cast<int8_t>(p1);
        qp_s[1][qd] = static_cast<int8_t>(p2);
        qp_s[2][qd] = static_cast<int8_t>(p3);
        if (lane == 0) qs_s[wave] = bad > 0.0f ? __builtin_nanf("") : s1;
        if (cur) {
            const float kmax = wave_max_all(isfinite(xk) ? fabsf(xk) : 0.0f);
            const float ksc = kmax > 0.0f ? kmax / 127.0f : 1.0f;
            const int8_t kq = q8_of(xk, ksc);
            kcur[qd] = kq;
            if (writer) store_q8(c, false, pos, kvh, qd, kq);
            if (lane == 0) {
                kcur_s[wave] = ksc;
                if (writer) c.key_scales[scale_index(c, pos, kvh * NG + wave)] = ksc;
            }
        }
    }
    if (vprep && cur) {
        const float vmax = wave_max_all(isfinite(va) ? fabsf(va) : 0.0f);
        const float vsc = vmax > 0.0f ? vmax / 127.0f : 1.0f;
        const int8_t vq = q8_of(va, vsc);
        vcur[qd] = vq;
        if (writer) store_q8(c, true, pos, kvh, qd, vq);
        if (lane == 0) {
            vcur_s[vwave] = vsc;
            if (writer) c.value_scales[scale_index(c, pos, kvh * NG + vwave)] = vsc;
        }
    }
    if (loader) wait_vmcnt<0>();   // the chunk is in LDS
    lds_barrier();
    if (!ok) return;

    const uint32_t vch = tid % D, ph = tid / D;   // P.V channel and phase
    const uint32_t vgrp = vch / 64;
    const uint32_t pl = slot / kKvPageTokens, s16 = slot % kKvPageTokens;
    const uint32_t sidx = ((slot / (4 * kKvPageTokens)) * kKvPageTokens + s16) * 4 + pl % 4;   // in ksc_l/vsc_l
    float m_run = -INFINITY, l_run = 0.0f, acc = 0.0f;
    for (uint32_t c0 = 0; c0 < t1; c0 += CH) {
        const uint32_t n = min(static_cast<uint32_t>(CH), t1 - c0);
        // 3. a later chunk: the previous one is consumed (barrier at the
        //    end of its pass), the loader waves copy this one
        if (c0 != 0) {
            if (loader) {
                issue_chunk(c0);
                wait_vmcnt<0>();
            }
            lds_barrier();
        }
        const bool has = slot < n && tree_attends(c0 + slot, tbase, tmask);
        // the current token's slot is being written by this launch: its key,
        // scales and value byte come from kcur / vcur
        const bool is_cur = cur && has && c0 + slot == pos;
        // 4. the score of this lane's token: per scale group, the exact int8
        //    dot products of its key channels with the three query pieces,
        //    scaled by the key scale and the piece scale, summed over the
        //    token's TPT lanes
        float sc = 0.0f;
        // waves whose slots all lie past the chunk's tokens skip the
        // products (their LDS reads are most of the phase's traffic)
        const bool wave_has = wave * SPW < n;
#pragma unroll
        for (int g = 0; g < KGL; ++g) {
            if (!wave_has) break;
            int d1 = 0, d2 = 0, d3 = 0;
#pragma unroll
            for (int w = g * WPG; w < (g + 1) * WPG; ++w) {
                const uint32_t kc = part * (CPT / 16) + w;   // 16-channel chunk of this word
                const int8_t *kp = is_cur ? kcur + kc * 16 : k_l + ((pl * KCH + kc) * kKvPageTokens + s16) * 16;
                const uint4 kw = *reinterpret_cast<const uint4 *>(kp);
                const uint4 a1 = *reinterpret_cast<const uint4 *>(&qp_s[0][kc * 16]);
                const uint4 a2 = *reinterpret_cast<const uint4 *>(&qp_s[1][kc * 16]);
                const uint4 a3 = *reinterpret_cast<const uint4 *>(&qp_s[2][kc * 16]);
                d1 = sdot4(kw.x, a1.x, d1); d1 = sdot4(kw.y, a1.y, d1);
                d1 = sdot4(kw.z, a1.z, d1); d1 = sdot4(kw.w, a1.w, d1);
                d2 = sdot4(kw.x, a2.x, d2); d2 = sdot4(kw.y, a2.y, d2);
                d2 = sdot4(kw.z, a2.z, d2); d2 = sdot4(kw.w, a2.w, d2);
                d3 = sdot4(kw.x, a3.x, d3); d3 = sdot4(kw.y, a3.y, d3);
                d3 = sdot4(kw.z, a3.z, d3); d3 = sdot4(kw.w, a3.w, d3);
            }
            const float f = fmaf(static_cast<float>(d3), 0x1p-14f,
                                 fmaf(static_cast<float>(d2), 0x1p-7f, static_cast<float>(d1)));
            const uint32_t gk = kgrp + g;
            const float ks = is_cur ? kcur_s[gk] : ksc_l[gk][sidx];
            sc = fmaf(ks * qs_s[gk], f, sc);
        }
#pragma unroll
        for (int off = SPW; off < 64; off <<= 1) sc += __shfl_xor(sc, off);
        // 5. chunk softmax, running max and sum
        sc = has ? sc * a.scale : -INFINITY;
        {
            const float m = wave_max_all(sc);
            if (lane == 0) red[0][wave] = m;
        }
        lds_barrier();
        float mc = red[0][0];
#pragma unroll
        for (int w = 1; w < NW; ++w) mc = fmaxf(mc, red[0][w]);
        const float mn = fmaxf(m_run, mc);
        const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - mn);
        m_run = mn;
        const float p = has ? expf(sc - mn) : 0.0f;
        // the weight of each value group of the slot: p times the token's
        // value scale (masked slots 0: their scales may be any bits)
#pragma unroll
        for (int g = 0; g < VGL; ++g) {
            const uint32_t gg = part * VGL + g;
            if (gg < static_cast<uint32_t>(NG)) {
                const float vs = is_cur ? vcur_s[gg] : vsc_l[gg][sidx];
                pw_s[gg][slot] = has ? p * vs : 0.0f;
            }
        }
        {
            const float ps = wave_sum_all(part == 0 ? p : 0.0f);
            if (lane == 0) red[1][wave] = ps;
        }
        lds_barrier();
        float lc = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) lc += red[1][w];
        l_run = l_run * alpha + lc;
        acc *= alpha;
        // 6. P.V of this thread's channel over its 4-token groups (from LDS),
        //    four groups' loads at a time; the first token of a batch decides
        //    (per wave) whether it runs, masked slots carry weight 0.  The
        //    current token's byte replaces the cache's in its group.
        const uint32_t ctl = cur && pos >= c0 && pos - c0 < static_cast<uint32_t>(CH) ? pos - c0 : 0xffffffffu;
        const uint32_t cshift = 8 * (ctl % 4), cbyte = static_cast<uint32_t>(static_cast<uint8_t>(vcur[vch])) << cshift;
        const uint32_t *v_u32 = reinterpret_cast<const uint32_t *>(v_l);
        const float *pw = pw_s[vgrp];
#pragma unroll
        for (int q4 = 0; q4 < NIT / 4; ++q4) {
            if (4 * ph + TSTEP * 4 * q4 >= n) break;
            uint32_t vw[4];
            float4 pp[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t tl = 4 * ph + TSTEP * (4 * q4 + i);
                vw[i] = v_u32[((tl / kKvPageTokens) * D + vch) * 4 + (tl % kKvPageTokens) / 4];
                pp[i] = *reinterpret_cast<const float4 *>(pw + tl);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t tl = 4 * ph + TSTEP * (4 * q4 + i);
                const uint32_t w4 = tl == (ctl & ~3u) ? (vw[i] & ~(0xffu << cshift)) | cbyte : vw[i];
                acc = fmaf(pp[i].x, i8f(w4, 0), acc);
                acc = fmaf(pp[i].y, i8f(w4, 1), acc);
                acc = fmaf(pp[i].z, i8f(w4, 2), acc);
                acc = fmaf(pp[i].w, i8f(w4, 3), acc);
            }
        }
        // the next chunk overwrites the chunk and the weights
        if (c0 + CH < t1) lds_barrier();
    }

    // 7. sum the token phases; the output
    pv_s[ph * D + vch] = acc;
    lds_barrier();
    if (tid < static_cast<uint32_t>(D)) {
        float o = 0.0f;
#pragma unroll
        for (int p = 0; p < PH; ++p) o += pv_s[p * D + tid];
        out[tid] = o / l_run;
    }
}

// grid (query heads): the split partials of one head, weighted by
// exp(m_s - max m) (empty splits carry m = -inf, l = 0 and drop out).  The
// split statistics are staged in LDS and reduced by the whole workgroup;
// each output channel is summed over the splits by 256 / D threads.
// PRE > 0: the merge kernel loads up to PRE splits per thread up front
// (the smallest of 8 and 16 that covers the launch): one memory round
// instead of two.  32 query heads of 128 channels: 9.54 -> 9.02 us per
// call at 4096 tokens (16 splits, PRE 8; PRE 16 there reloads split 0 into
// the spare slots and gives the gain back), 21.3 -> 21.0 at 32768 (32
// splits, PRE 16).
template <uint32_t PRE>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float *__restrict__ partials, float *out,
                                                           uint32_t nsplit, uint32_t D) {
    __shared__ float w_s[1024];
    __shared__ float l_s[1024];
    __shared__ float red_s[2][4];
    __shared__ float part_s[256];
    const uint32_t head = blockIdx.x, tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const float *base = partials + static_cast<size_t>(head) * nsplit * (D + 2);
    // channel d = tid % D, splits part, part + parts, ...
    const uint32_t parts = D <= 256 ? 256 / D : 1;
    // PRE (D <= 256: one channel pass, at most PRE splits per thread): the
    // thread's partial values are loaded with the maxima
    // and sums below, in one memory round, and combined in the same order as
    // the loop further down (so the result is the same to the bit).
    constexpr uint32_t kMergePre = PRE;
    float pv[PRE ? PRE : 1];
    if constexpr (PRE > 0) {
        const uint32_t d = tid % D, part = tid / D;
#pragma unroll
        for (uint32_t j = 0; j < kMergePre; ++j) {
            const uint32_t sidx = part + j * parts;
            pv[j] = base[(sidx < nsplit ? sidx : 0u) * (D + 2) + 2 + d];  // split 0 always exists
        }
    }
    float mx = -INFINITY;
    for (uint32_t sidx = tid; sidx < nsplit; sidx += blockDim.x) {
        const float m = base[sidx * (D + 2)];
        w_s[sidx] = m;
        l_s[sidx] = base[sidx * (D + 2) + 1];
        mx = fmaxf(mx, m);
    }
    mx = wave_max_all(mx);
    if (lane == 0) red_s[0][wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red_s[0][0], red_s[0][1]), fmaxf(red_s[0][2], red_s[0][3]));
    float total = 0.0f;
    for (uint32_t sidx = tid; sidx < nsplit; sidx += blockDim.x) {
        const float m = w_s[sidx];
        const float w = m == -INFINITY ? 0.0f : expf(m - mx);
        w_s[sidx] = w;
        total = fmaf(l_s[sidx], w, total);
    }
    total = wave_sum_all(total);
    if (lane == 0) red_s[1][wave] = total;
    __syncthreads();
    total = (red_s[1][0] + red_s[1][1]) + (red_s[1][2] + red_s[1][3]);
    const float inv = total > 0.0f ? 1.0f / total : 0.0f;
    if constexpr (PRE > 0) {
        const uint32_t d = tid % D, part = tid / D;
        float o = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < kMergePre; ++j) {
            const uint32_t sidx = part + j * parts;
            if (sidx < nsplit) o = fmaf(pv[j], w_s[sidx], o);
        }
        part_s[tid] = o;
        __syncthreads();
        if (part == 0) {
            float sum = 0.0f;
            for (uint32_t pi = 0; pi < parts; ++pi) sum += part_s[pi * D + d];
            out[static_cast<size_t>(head) * D + d] = sum * inv;
        }
        return;
    }
    for (uint32_t d0 = 0; d0 < D; d0 += 256 / parts) {
        const uint32_t d = d0 + tid % D, part = tid / D;
        float o = 0.0f;
        if (part < parts && d < D) {
            uint32_t sidx = part;
            for (; sidx + 3 * parts < nsplit; sidx += 4 * parts) {
                const float p0 = base[sidx * (D + 2) + 2 + d], p1 = base[(sidx + parts) * (D + 2) + 2 + d];
                const float p2 = base[(sidx + 2 * parts) * (D + 2) + 2 + d];
                const float p3 = base[(sidx + 3 * parts) * (D + 2) + 2 + d];
                o = fmaf(p0, w_s[sidx], o);
                o = fmaf(p1, w_s[sidx + parts], o);
                o = fmaf(p2, w_s[sidx + 2 * parts], o);
                o = fmaf(p3, w_s[sidx + 3 * parts], o);
            }
            for (; sidx < nsplit; sidx += parts) o = fmaf(base[sidx * (D + 2) + 2 + d], w_s[sidx], o);
        }
        __syncthreads();
        part_s[tid] = o;
        __syncthreads();
        if (part == 0 && d < D) {
            float sum = 0.0f;
            for (uint32_t pi = 0; pi < parts; ++pi) sum += part_s[pi * D + tid % D];
            out[static_cast<size_t>(head) * D + d] = sum * inv;
        }
    }
}

// ---- int8 MFMA attention (no RoPE/append; any context length) --------------
//
// Both products run on v_mfma_i32_16x16x64_i8 (lane l holds A row l%16 and
// B column l%16 for k-bytes 16*(l/16)..+15; C[4*(l/16)+r][l%16]):
//   scores  A = query pieces [head*4 + piece][64 channels of one scale group],
//           B = keys [64 channels][16 tokens of one page] (key rows are
//           contiguous), C = [head, piece][token]
//   P.V     A = probability pieces [head*4 + piece][64 tokens],
//           B = values [64 tokens][16 channels] (the channel-major page word),
//           C = [head, piece][channel]
// A float operand x is split into three int8 pieces with one scale per
// (head, 64-group): x ~= s1*q1 + s2*q2 + s3*q3, s1 = amax/127,
// s2 = s1/254, s3 = s2/254, each residual taken exactly with an fma, so
// |x - sum| <= amax * 6e-8; the integer dots are exact and are combined in
// fp32.  The fourth piece row is zero.  The value scale of each token is
// folded into its probability before the split (p' = p * vs).
//
// A workgroup = one KV head x `split` tokens, NW waves; wave w takes the
// 64-token blocks w, w+NW, ... with its own online softmax (per query head:
// max, sum, output), and the waves merge through LDS.
// With one split the workgroup writes the output, else (max, sum, output)
// partials for decode_merge_kernel.
typedef int att_v4i __attribute__((ext_vector_type(4)));

struct MfmaAttnArgs {
    KvCache c;
    const float *query;       // [H][D]
    float *output;            // [H][D] (nsplit == 1)
    float *partials;          // [H][nsplit][D + 2] (nsplit > 1)
    uint32_t group;           // query heads per KV head (<= 4 * RT)
    uint32_t split;           // tokens per workgroup, a multiple of 64 * waves
    uint32_t nsplit;
    float scale;
    uint32_t position;
    const int32_t *position_ptr;
    const uint64_t *tree_mask;  // optional: the query token's ancestor mask over slots *tree_base + a
    const int32_t *tree_base;
};

__device__ __forceinline__ int piece_round(float v) {
    return static_cast<int>(fminf(fmaxf(__builtin_rintf(v), -127.0f), 127.0f));
}

// the three pieces of x for scale s1 (inv1 = 1/s1), packed one byte each
__device__ __forceinline__ uint32_t three_pieces(float x, float s1, float inv1) {
    const float s2 = s1 * (1.0f / 254.0f), s3 = s2 * (1.0f / 254.0f);
    const int q1 = piece_round(x * inv1);
    const float r1 = fmaf(-static_cast<float>(q1), s1, x);
    const int q2 = piece_round(r1 * (inv1 * 254.0f));
    const float r2 = fmaf(-static_cast<float>(q2), s2, r1);
    const int q3 = piece_round(r2 * (inv1 * 64516.0f));
    (void)s3;
    return (static_cast<uint32_t>(q1) & 0xffu) | ((static_cast<uint32_t>(q2) & 0xffu) << 8) |
           ((static_cast<uint32_t>(q3) & 0xffu) << 16);
}

__device__ __forceinline__ float pieces_dot(att_v4i cacc, float s1) {
    const float s2 = s1 * (1.0f / 254.0f), s3 = s2 * (1.0f / 254.0f);
    return fmaf(s3, static_cast<float>(cacc[2]), fmaf(s2, static_cast<float>(cacc[1]), s1 * static_cast<float>(cacc[0])));
}

// Reductions over each 16-lane row by DPP row rotations (row_ror 8, 4, 2,
// 1): every lane of the row ends with the row's max / sum (the sum's
// association differs between lanes; callers read one lane).
template <int CTRL>
__device__ __forceinline__ float dpp_rot(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_rot<0x128>(v));
    v = fmaxf(v, dpp_rot<0x124>(v));
    v = fmaxf(v, dpp_rot<0x122>(v));
    return fmaxf(v, dpp_rot<0x121>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_rot<0x128>(v);
    v += dpp_rot<0x124>(v);
    v += dpp_rot<0x122>(v);
    return v + dpp_rot<0x121>(v);
}

// DPP quad permutations: quad_perm<ctrl> moves within each 4-lane quad
// (0xb1: lane ^ 1, 0x4e: lane ^ 2); quad_bcast_u32(v, q) gives every lane of
// the quad lane q's v.
template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ uint32_t quad_bcast_u32(uint32_t v, int q) {
    const int x = static_cast<int>(v);
    switch (q) {
    case 0: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x00, 0xf, 0xf, false));
    case 1: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x55, 0xf, 0xf, false));
    case 2: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0xaa, 0xf, 0xf, false));
    default: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0xff, 0xf, 0xf, false));
    }
}

__device__ __forceinline__ float f4_at(const float4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ void lds_wave_sync() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

constexpr uint32_t kMfmaMaxSplits = 512;

// NW waves per workgroup (mfma_attn_plan; eight, two per SIMD, measured
// slower at 4K and 32K-token contexts)
template <int D, int RT, int NW>
__global__ __launch_bounds__(64 * NW) void mfma_attention_kernel(MfmaAttnArgs a) {
    constexpr int NG = D / 64;   // scale groups per head = MFMA k-steps
    constexpr int NT = 4;        // pages (16-token tiles) per 64-token block
    constexpr int HR = 4 * RT;   // query-head rows
    __shared__ __align__(16) int8_t pp_s[NW][RT][NG][4][3][64];  // per wave: p' pieces [head][piece][token]
    __shared__ float ml_s[NW][HR][2];
    __shared__ __align__(16) float o_s[NW][HR][D];
    const KvCache &c = a.c;
    const uint32_t tid = threadIdx.x, lane = tid % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const uint32_t kvh = blockIdx.y, split = blockIdx.x, G = a.group;
    const uint32_t pos = a.position_ptr ? static_cast<uint32_t>(*a.position_ptr) : a.position;
    if (pos >= c.max_tokens) return;
    const uint32_t tokens = pos + 1;
    const uint32_t t0 = split * a.split;
    if (t0 >= tokens) {
        // a split past the position (fixed grid): an empty partial
        for (uint32_t i = tid; i < G * D; i += blockDim.x) {
            const uint32_t g = i / D, d = i % D;
            float *dst = a.partials + (static_cast<size_t>(kvh * G + g) * a.nsplit + split) * (D + 2);
            dst[2 + d] = 0.0f;
            if (d == 0) {
                dst[0] = -INFINITY;
                dst[1] = 0.0f;
            }
        }
        return;
    }
    const uint32_t t1 = min(tokens, t0 + a.split);
    const uint32_t col = lane % 16, kq = lane / 16;   // MFMA column / k-quarter of this lane
    const uint64_t tmask = a.tree_mask ? *a.tree_mask : 0ull;
    const uint32_t tbase = a.tree_mask ? static_cast<uint32_t>(*a.tree_base) : 0xffffffffu;

    // 1. query pieces (A of the scores), this lane: head (col / 4) of row
    //    tile rt, piece col % 4, channels 64g + 16kq .. +15.  Where the
    //    registers allow (kEarly), the query loads are issued first, then the
    //    first block's keys and values, and the pieces are computed while
    //    those are in flight (loads retire in order, so a query load issued
    //    after them would wait for them).
    constexpr bool kEarly = D <= 128 && RT * NG <= 4;
    att_v4i qa[RT][NG];
    float qs1[RT][NG];   // s1 of head kq (+ 4rt): the C-layout head of this lane
    float4 xq[kEarly ? RT : 1][kEarly ? NG : 1];
    // The four lanes of a quad (piece col % 4) share a head and 16
    // channels: lane p loads and splits channels 4p .. 4p + 3, and the
    // quad exchanges the pieces.  Rows past the group load head 0's
    // channels (no branch around the loads, so the waits that follow can
    // count them exactly) and are zeroed where the pieces are made.
    auto load_query = [&](int rt, int g) -> float4 {
        const uint32_t hl = rt * 4 + col / 4;
        return *reinterpret_cast<const float4 *>(a.query + static_cast<size_t>(kvh * G + (hl < G ? hl : 0u)) * D +
                                                 64 * g + 16 * kq + 4 * (col % 4));
    };
    auto make_pieces = [&](int rt, int g, float4 xin) {
        const uint32_t piece = col % 4;
        const bool row_ok = rt * 4 + col / 4 < G;
        const float x[4] = {row_ok ? xin.x : 0.0f, row_ok ? xin.y : 0.0f, row_ok ? xin.z : 0.0f,
                            row_ok ? xin.w : 0.0f};
        float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        amax = fmaxf(amax, quad_perm<0xb1>(amax));   // lanes p ^ 1
        amax = fmaxf(amax, quad_perm<0x4e>(amax));   // lanes p ^ 2
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const float s1 = amax > 0.0f ? amax * (1.0f / 127.0f) : 1.0f;
        const float inv1 = amax > 0.0f ? 127.0f / amax : 1.0f;
        // mine[j]: piece j of my four channels, one byte each
        uint32_t mine[3] = {0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t pc = three_pieces(x[e], s1, inv1);
#pragma unroll
            for (int j = 0; j < 3; ++j) mine[j] |= ((pc >> (8 * j)) & 0xffu) << (8 * e);
        }
        // word q of my operand: piece `piece` of lane q's channels
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t b0 = quad_bcast_u32(mine[0], q), b1 = quad_bcast_u32(mine[1], q);
            const uint32_t b2 = quad_bcast_u32(mine[2], q);
            w[q] = piece == 0 ? b0 : piece == 1 ? b1 : piece == 2 ? b2 : 0u;
        }
        qa[rt][g] = att_v4i{static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]),
                            static_cast<int>(w[3])};
        // head h's scale sits in lane 4h (kq 0, piece 0)
        qs1[rt][g] = __shfl(s1, 4 * kq);
    };
    if constexpr (kEarly) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int g = 0; g < NG; ++g) xq[rt][g] = load_query(rt, g);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. loads of a block: keys (B of the scores) for token b0 + 16i + col
    //    and its scales; value words (B of P.V) of page b0/16 + kq, channel
    //    64g + 16n + col.  Tokens past t1 read a valid token (t0) and are
    //    masked.  The next block's loads are issued before this block's
    //    arithmetic.
    struct BlockLoads {
        att_v4i kb[NG][NT], vb[NG][4];
        float4 ks[NG], vs[NG];   // .x .. .w: scales of tokens b0 + col, + 16, + 32, + 48
    };
    auto load_block = [&](uint32_t b0, BlockLoads &L) {
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const uint32_t t = b0 + 16 * i + col;
            const uint32_t tl = t < t1 ? t : t0;
#pragma unroll
            for (int g = 0; g < NG; ++g)
                L.kb[g][i] = *reinterpret_cast<const att_v4i *>(c.keys + k_index(c, tl, kvh, 64 * g + 16 * kq));
        }
        // b0 starts a 64-token quad: one 16-byte load per scale group gives
        // this lane's token in each of the four pages (masked tokens read
        // slots of the same quad, which hold finite values)
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            L.ks[g] = *reinterpret_cast<const float4 *>(c.key_scales + scale_index(c, b0 + col, kvh * NG + g));
            L.vs[g] = *reinterpret_cast<const float4 *>(c.value_scales + scale_index(c, b0 + col, kvh * NG + g));
        }
        const uint32_t pt = b0 + 16 * kq;
        const uint32_t pg = (pt < t1 ? pt : t0) / kKvPageTokens;
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int n = 0; n < 4; ++n)
                L.vb[g][n] = *reinterpret_cast<const att_v4i *>(c.values + v_page_offset(c, pg, kvh, 64 * g + 16 * n + col));
    };
    // blocks of this wave: b0, b0 + step, ... below t1 (wave-uniform)
    const uint32_t step = 64 * NW;
    uint32_t b0 = t0 + 64 * wave;
    const uint32_t nblk = b0 < t1 ? (t1 - b0 + step - 1) / step : 0u;
    const uint32_t last = b0 + (nblk ? nblk - 1 : 0u) * step;
    BlockLoads buf0;
    if constexpr (kEarly) {
        // unconditional (a wave without blocks loads the split's first
        // block and never uses it): no branch for the waits to merge over
        load_block(nblk ? b0 : t0, buf0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int g = 0; g < NG; ++g) make_pieces(rt, g, xq[rt][g]);
    } else {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int g = 0; g < NG; ++g) make_pieces(rt, g, load_query(rt, g));
        __builtin_amdgcn_sched_barrier(0);
        if (D <= 128 && nblk) load_block(b0, buf0);
    }

    float m_run[RT], l_run[RT], o_acc[RT][NG][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m_run[rt] = -INFINITY;
        l_run[rt] = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int n = 0; n < 4; ++n) o_acc[rt][g][n] = 0.0f;
    }

    auto process_block = [&](const BlockLoads &cur, uint32_t b0) {
        const att_v4i (&kb)[NG][NT] = cur.kb;
        const att_v4i (&vb)[NG][4] = cur.vb;
        const float4 (&ks)[NG] = cur.ks;
        const float4 (&vs)[NG] = cur.vs;
        bool valid[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const uint32_t t = b0 + 16 * i + col;
            valid[i] = t < t1 && tree_attends(t, tbase, tmask);
        }

#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            // 3. scores of head kq (+4rt) for token b0 + 16i + col
            float sc[NT];
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                float dot = 0.0f;
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    const att_v4i cacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[rt][g], kb[g][i],
                                                                               att_v4i{0, 0, 0, 0}, 0, 0, 0);
                    dot = fmaf(pieces_dot(cacc, qs1[rt][g]), f4_at(ks[g], i), dot);
                }
                sc[i] = valid[i] ? dot * a.scale : -INFINITY;
            }
            // 4. online softmax of the block (per head: one 16-lane row)
            float cm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            cm = row16_max(cm);
            const float mn = fmaxf(m_run[rt], cm);
            const float alpha = m_run[rt] == -INFINITY ? 0.0f : expf(m_run[rt] - mn);
            m_run[rt] = mn;
            float p[NT], ps = 0.0f;
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                p[i] = valid[i] ? expf(sc[i] - mn) : 0.0f;
                ps += p[i];
            }
            l_run[rt] = fmaf(l_run[rt], alpha, row16_sum(ps));
            // 5. p' = p * vs per scale group, split into pieces -> LDS
            float ps1[NG];
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                float pv[NT], am = 0.0f;
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    pv[i] = p[i] * f4_at(vs[g], i);
                    am = fmaxf(am, pv[i]);
                }
                am = row16_max(am);
                const float s1 = am > 0.0f ? am * (1.0f / 127.0f) : 1.0f;
                const float inv1 = am > 0.0f ? 127.0f / am : 1.0f;
                ps1[g] = s1;
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    const uint32_t pc = three_pieces(pv[i], s1, inv1);
                    int8_t *dst = &pp_s[wave][rt][g][kq][0][16 * i + col];
                    dst[0] = static_cast<int8_t>(pc & 0xffu);
                    dst[64] = static_cast<int8_t>((pc >> 8) & 0xffu);
                    dst[128] = static_cast<int8_t>((pc >> 16) & 0xffu);
                }
            }
            lds_wave_sync();
            // 6. P.V: A lane = head col/4, piece col%4, tokens 16kq .. +15
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                att_v4i pa = {0, 0, 0, 0};
                if (col % 4 < 3)
                    pa = *reinterpret_cast<const att_v4i *>(&pp_s[wave][rt][g][col / 4][col % 4][16 * kq]);
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    const att_v4i cacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb[g][n], att_v4i{0, 0, 0, 0},
                                                                               0, 0, 0);
                    o_acc[rt][g][n] = fmaf(o_acc[rt][g][n], alpha, pieces_dot(cacc, ps1[g]));
                }
            }
            lds_wave_sync();
        }
    };
    // Two load buffers used in turn (no register copy between them, so the
    // wait before a block covers that block's loads only and the next
    // block's stay in flight).  The last prefetch of a wave re-reads its
    // current block (an L2 hit) so every load is unconditional.  At head_dim
    // 256 two buffers do not fit the registers: load, then compute.
    if constexpr (D <= 128) {
        BlockLoads buf1;
        for (uint32_t k = 1; k < nblk; k += 2) {
            load_block(b0 + step, buf1);
            process_block(buf0, b0);
            load_block(min(b0 + 2 * step, last), buf0);
            process_block(buf1, b0 + step);
            b0 += 2 * step;
        }
        if (nblk % 2) process_block(buf0, b0);
    } else {
        for (; b0 < t1; b0 += step) {
            load_block(b0, buf0);
            process_block(buf0, b0);
        }
    }

    // 7. merge the four waves: lane (kq, col) holds head kq (+4rt), channel
    //    64g + 16n + col
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        if (col == 0) {
            ml_s[wave][rt * 4 + kq][0] = m_run[rt];
            ml_s[wave][rt * 4 + kq][1] = l_run[rt];
        }
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int n = 0; n < 4; ++n) o_s[wave][rt * 4 + kq][64 * g + 16 * n + col] = o_acc[rt][g][n];
    }
    __syncthreads();
    for (uint32_t i = tid; i < G * D; i += blockDim.x) {
        const uint32_t hl = i / D, d = i % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, ml_s[w][hl][0]);
        float l = 0.0f, o = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float m = ml_s[w][hl][0];
            const float f = m == -INFINITY ? 0.0f : expf(m - mx);
            l = fmaf(ml_s[w][hl][1], f, l);
            o = fmaf(o_s[w][hl][d], f, o);
        }
        const uint32_t head = kvh * G + hl;
        if (a.nsplit == 1) {
            a.output[static_cast<size_t>(head) * D + d] = o / l;
        } else {
            float *dst = a.partials + (static_cast<size_t>(head) * a.nsplit + split) * (D + 2);
            dst[2 + d] = o;
            if (d == 0) {
                dst[0] = mx;
                dst[1] = l;
            }
        }
    }
}

template <int D, int RT, int NW>
hipError_t launch_mfma_attention_kernel(const MfmaAttnArgs &args, hipStream_t stream) {
    hipLaunchKernelGGL((mfma_attention_kernel<D, RT, NW>), dim3(args.nsplit, args.c.kv_heads), dim3(64 * NW), 0,
                       stream, args);
    return hipGetLastError();
}

template <int D, int RT>
hipError_t launch_mfma_attention_nw(const MfmaAttnArgs &args, uint32_t waves, hipStream_t stream) {
    if (waves != 4) return hipErrorInvalidValue;
    return launch_mfma_attention_kernel<D, RT, 4>(args, stream);
}

template <int D>
hipError_t launch_mfma_attention_rt(const MfmaAttnArgs &args, uint32_t waves, hipStream_t stream) {
    return args.group <= 4 ? launch_mfma_attention_nw<D, 1>(args, waves, stream)
                           : launch_mfma_attention_nw<D, 2>(args, waves, stream);
}

// Two lanes per token (512 threads): measured on MI355X at 12 query / 2 KV
// heads, position 100, graph of back-to-back launches: 5.5 us per launch
// against 6.2 with four lanes (16 waves: the softmax's wave reductions and
// barriers cost more than the shorter scores save) and 6.1 with one (the
// per-token chains get longer)
constexpr int kDecodeTpt = 2;

template <int D>
hipError_t launch_decode_kernel(const DecodeAttnArgs &args, hipStream_t stream) {
    hipLaunchKernelGGL((decode_attention_kernel<D, kDecodeTpt>),
                       dim3(1, args.c.kv_heads * args.group, std::max(args.count, 1u)), dim3(256 * kDecodeTpt), 0,
                       stream, args);
    return hipGetLastError();
}

}  // namespace

size_t kv_cache_layout(KvCache &c, uint8_t *base) {
    c.channels = c.kv_heads * c.head_dim;
    c.groups = (c.channels + 63u) / 64u;
    c.pages = (c.max_tokens + kKvPageTokens - 1) / kKvPageTokens;
    c.quads = (c.pages + 3) / 4;
    const size_t slots = static_cast<size_t>(c.pages) * kKvPageTokens;
    const size_t padded_dim = (c.head_dim + 15u) / 16u * 16u;
    const size_t key_bytes = (slots * c.kv_heads * padded_dim + 255) & ~static_cast<size_t>(255);
    const size_t value_bytes = (slots * c.channels + 255) & ~static_cast<size_t>(255);
    const size_t scale_bytes =
        (static_cast<size_t>(c.quads) * 4 * kKvPageTokens * c.groups * sizeof(float) + 255) & ~static_cast<size_t>(255);
    if (base) {
        c.keys = reinterpret_cast<int8_t *>(base);
        c.values = reinterpret_cast<int8_t *>(base + key_bytes);
        c.key_scales = reinterpret_cast<float *>(base + key_bytes + value_bytes);
        c.value_scales = reinterpret_cast<float *>(base + key_bytes + value_bytes + scale_bytes);
    }
    return key_bytes + value_bytes + 2 * scale_bytes;
}

hipError_t launch_rope_append(const KvCache &c, float *query, uint32_t query_heads, const float *key,
                              const float *value, const float *cos_tab, const float *sin_tab,
                              const int32_t *pos_ptr, hipStream_t stream, uint32_t count, const float *q_norm,
                              const float *k_norm, float eps, const int32_t *rope_pos_ptr) {
    if (c.head_dim % 2 || c.channels > 8192 || count == 0 || (!q_norm) != (!k_norm) ||
        (q_norm && query_heads + c.kv_heads > static_cast<uint32_t>(kMaxNormHeads)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_append_kernel, dim3(count), dim3(1024), c.channels * sizeof(float), stream, c, query,
                       query_heads, key, value, cos_tab, sin_tab, pos_ptr, query_heads * c.head_dim, c.channels,
                       q_norm, k_norm, eps, rope_pos_ptr);
    return hipGetLastError();
}

bool decode_attention_supported(const KvCache &c, uint32_t query_heads) {
    return (c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256) && query_heads % c.kv_heads == 0 &&
           query_heads / c.kv_heads <= 8;
}

// Tokens per workgroup: the whole context up to 1024 tokens (one workgroup
// per KV head, no merge); beyond that, splits sized for ~512 workgroups.
uint32_t decode_split_tokens(const KvCache &c, uint32_t tokens) {
    if (tokens <= 1024) return std::max<uint32_t>(tokens, 1);
    uint32_t s = 64;
    while (s < 8192 && static_cast<uint64_t>(tokens) * c.kv_heads > static_cast<uint64_t>(s) * 512) s *= 2;
    return s;
}

size_t decode_attention_workspace_floats(const KvCache &c, uint32_t query_heads, uint32_t tokens) {
    const uint32_t s = decode_split_tokens(c, tokens);
    const uint32_t nsplit = (tokens + s - 1) / s;
    return nsplit > 1 ? static_cast<size_t>(query_heads) * nsplit * (c.head_dim + 2) : 0;
}

bool mfma_attention_supported(const KvCache &c, uint32_t query_heads) {
    return (c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256) && query_heads >= c.kv_heads &&
           query_heads % c.kv_heads == 0 && query_heads / c.kv_heads <= 8;
}

// Launch plan over `span` tokens: four waves per workgroup, each streaming
// 64-token blocks with the next block's loads in flight; tokens per
// workgroup one block per wave, doubled while the grid would exceed 256
// workgroups (one per CU, every workgroup resident in one round) or a KV
// head kMfmaMaxSplits splits.  Measured on MI355X at 32 query / 8 KV heads,
// 4096 and 32768 tokens: one, two or eight waves per workgroup and grids of
// 512 or 1024 workgroups all ran slower (at 32768 tokens the 256-workgroup
// kernel already streams the cache at about 5 TB/s).
struct MfmaAttnPlan {
    uint32_t waves, split, nsplit;
};

constexpr uint32_t kMfmaAttnWaves = 4;
constexpr uint32_t kMfmaAttnMaxWgs = 256;

MfmaAttnPlan mfma_attn_plan(const KvCache &c, uint32_t span) {
    MfmaAttnPlan p;
    p.waves = kMfmaAttnWaves;
    uint64_t s = 64u * p.waves;
    // stops at one split (s >= span) whatever the KV head count
    while (s < span && ((span + s - 1) / s * c.kv_heads > kMfmaAttnMaxWgs || (span + s - 1) / s > kMfmaMaxSplits))
        s *= 2;
    p.split = static_cast<uint32_t>(std::min<uint64_t>(s, 0x80000000u));
    p.nsplit = static_cast<uint32_t>((static_cast<uint64_t>(span) + p.split - 1) / p.split);
    return p;
}

uint32_t mfma_attention_launches(const KvCache &c, uint32_t, uint32_t span) {
    return mfma_attn_plan(c, span).nsplit > 1 ? 2 : 1;
}

size_t mfma_attention_workspace_floats(const KvCache &c, uint32_t query_heads, uint32_t span) {
    const uint32_t nsplit = mfma_attn_plan(c, span).nsplit;
    return nsplit > 1 ? static_cast<size_t>(query_heads) * nsplit * (c.head_dim + 2) : 0;
}

hipError_t launch_mfma_attention(const KvCache &c, const float *query, float *output, float *partials,
                                 uint32_t query_heads, uint32_t position, const int32_t *position_ptr,
                                 uint32_t span, float scale, hipStream_t stream, const uint64_t *tree_mask,
                                 const int32_t *tree_base) {
    if (!mfma_attention_supported(c, query_heads) || span == 0 || span > c.max_tokens ||
        (!tree_mask) != (!tree_base))
        return hipErrorInvalidValue;
    MfmaAttnArgs args{};
    args.tree_mask = tree_mask;
    args.tree_base = tree_base;
    args.c = c;
    args.query = query;
    args.output = output;
    args.partials = partials;
    args.group = query_heads / c.kv_heads;
    const MfmaAttnPlan plan = mfma_attn_plan(c, span);
    args.split = plan.split;
    args.nsplit = plan.nsplit;
    if ((args.nsplit > 1 && !partials) || args.nsplit > kMfmaMaxSplits) return hipErrorInvalidValue;
    args.scale = scale;
    args.position = position;
    args.position_ptr = position_ptr;
    hipError_t e;
    switch (c.head_dim) {
    case 64: e = launch_mfma_attention_rt<64>(args, plan.waves, stream); break;
    case 128: e = launch_mfma_attention_rt<128>(args, plan.waves, stream); break;
    default: e = launch_mfma_attention_rt<256>(args, plan.waves, stream); break;
    }
    if (e != hipSuccess || args.nsplit == 1) return e;
    const uint32_t D = c.head_dim;
    const uint32_t parts = D <= 256 ? 256 / D : 0;
    if (args.nsplit <= 8 * parts)
        hipLaunchKernelGGL(decode_merge_kernel<8>, dim3(query_heads), dim3(256), 0, stream, partials, output,
                           args.nsplit, D);
    else if (args.nsplit <= 16 * parts)
        hipLaunchKernelGGL(decode_merge_kernel<16>, dim3(query_heads), dim3(256), 0, stream, partials, output,
                           args.nsplit, D);
    else
        hipLaunchKernelGGL(decode_merge_kernel<0>, dim3(query_heads), dim3(256), 0, stream, partials, output,
                           args.nsplit, D);
    return hipGetLastError();
}

hipError_t launch_decode_attention(const DecodeAttentionLaunch &l, hipStream_t stream) {
    const KvCache &c = *l.cache;
    if (!decode_attention_supported(c, l.query_heads) || (l.key && (c.head_dim % 64 || !l.value || !l.cos_tab ||
                                                                    !l.sin_tab)) ||
        l.count == 0 || (l.count > 1 && (l.key || !l.position_ptr)) || (!l.tree_mask) != (!l.tree_base) ||
        (l.tree_mask && (l.key || !l.position_ptr)))
        return hipErrorInvalidValue;
    // the whole context in one split (K/V rows are re-read per query head
    // from L2: the latency case); longer contexts take the RoPE/append
    // kernel and the MFMA attention
    if (l.span_tokens == 0 || decode_split_tokens(c, l.span_tokens) < l.span_tokens) return hipErrorInvalidValue;
    if ((!l.q_norm) != (!l.k_norm) || (l.q_norm && !l.key)) return hipErrorInvalidValue;
    DecodeAttnArgs args{};
    args.c = c;
    args.query = l.query;
    args.output = l.output;
    args.group = l.query_heads / c.kv_heads;
    args.span = l.span_tokens;
    args.scale = l.scale;
    args.position = l.position;
    args.position_ptr = l.position_ptr;
    args.key = l.key;
    args.value = l.value;
    args.cos_tab = l.cos_tab;
    args.sin_tab = l.sin_tab;
    args.rope_row_only = l.rope_row_only ? 1u : 0u;
    args.count = l.count;
    args.token_stride = l.query_heads * c.head_dim;
    args.q_norm = l.q_norm;
    args.k_norm = l.k_norm;
    args.eps = l.eps;
    args.tree_mask = l.tree_mask;
    args.tree_base = l.tree_base;
    switch (c.head_dim) {
    case 64: return launch_decode_kernel<64>(args, stream);
    case 128: return launch_decode_kernel<128>(args, stream);
    default: return launch_decode_kernel<256>(args, stream);
    }
}

hipError_t launch_kv_commit_path(const KvCache &c, const int32_t *base, const int32_t *path, uint32_t len,
                                 hipStream_t stream) {
    if (!base || !path || len == 0 || len > 64) return hipErrorInvalidValue;
    const uint32_t n = std::max(c.channels, c.groups);
    hipLaunchKernelGGL(kv_commit_path_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, c, base, path, len);
    return hipGetLastError();
}

hipError_t launch_kv_append(const KvCache &c, const float *key, const float *value, uint32_t token,
                            hipStream_t stream, uint32_t count) {
    if (count == 0 || token >= c.max_tokens || count > c.max_tokens - token) return hipErrorInvalidValue;
    for (uint32_t done = 0; done < count;) {
        const uint32_t n = std::min<uint32_t>(count - done, 32768u);
        hipLaunchKernelGGL(kv_append_kernel, dim3(c.groups, 2, n), dim3(64), 0, stream, c,
                           key + static_cast<size_t>(done) * c.channels, value + static_cast<size_t>(done) * c.channels,
                           token + done, static_cast<const int32_t *>(nullptr));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        done += n;
    }
    return hipSuccess;
}

hipError_t launch_kv_gather(const KvCache &c, uint32_t first, uint32_t count, int8_t *keys, int8_t *values,
                            float *key_scales, float *value_scales, hipStream_t stream) {
    if (count == 0 || first > c.tokens || count > c.tokens - first) return hipErrorInvalidValue;
    const uint64_t n = static_cast<uint64_t>(count) * c.channels;  // channels >= groups
    hipLaunchKernelGGL(kv_gather_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream, c, first,
                       count, keys, values, key_scales, value_scales);
    return hipGetLastError();
}

hipError_t launch_kv_append_at(const KvCache &c, const float *key, const float *value, const int32_t *token_ptr,
                               hipStream_t stream) {
    hipLaunchKernelGGL(kv_append_kernel, dim3(c.groups, 2), dim3(64), 0, stream, c, key, value, 0u, token_ptr);
    return hipGetLastError();
}

size_t attention_workspace_floats(const KvCache &c, uint32_t query_heads, uint32_t position) {
    const uint32_t tokens = position + 1;
    if (mfma_attention_supported(c, query_heads)) return mfma_attention_workspace_floats(c, query_heads, tokens);
    const uint32_t s = split_tokens(c, tokens);
    const uint32_t nsplit = (tokens + s - 1) / s;
    return static_cast<size_t>(query_heads) * nsplit * (c.head_dim + 2);
}

namespace {
// Query heads share a workgroup per KV head when they divide evenly into
// groups of at most 8; any other ratio (query heads not a multiple of the
// KV heads, fewer query than KV heads, or more than 8 per KV head) takes one
// workgroup per query head with the reference's mapping
// kv_head = head * kv_heads / query_heads (c/cuda/qwn_hypervsq2_cuda_abi.cu:184).
void set_head_plan(AttnArgs &args, const KvCache &c, uint32_t query_heads) {
    args.query_heads = query_heads;
    const bool grouped = query_heads >= c.kv_heads && query_heads % c.kv_heads == 0 && query_heads / c.kv_heads <= 8;
    args.head_mapped = grouped ? 0u : 1u;
    args.group = grouped ? query_heads / c.kv_heads : 1u;
}

hipError_t launch_split_and_merge(AttnArgs &args, float *output, hipStream_t stream) {
    hipError_t e;
    if (args.head_mapped || args.group <= 1) e = launch_fast_or_not<1>(args, stream);
    else if (args.group <= 2) e = launch_fast_or_not<2>(args, stream);
    else if (args.group <= 4) e = launch_fast_or_not<4>(args, stream);
    else if (args.group <= 8) e = launch_fast_or_not<8>(args, stream);
    else return hipErrorInvalidValue;
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_merge_kernel, dim3(args.query_heads), dim3(256), 0, stream, args.partials, output,
                       args.nsplit, args.c.head_dim);
    return hipGetLastError();
}
}  // namespace

size_t attention_at_workspace_floats(const KvCache &c, uint32_t query_heads) {
    if (mfma_attention_supported(c, query_heads))
        return mfma_attention_workspace_floats(c, query_heads, c.max_tokens);
    const uint32_t nsplit = (c.max_tokens + kDevicePositionSplit - 1) / kDevicePositionSplit;
    return static_cast<size_t>(query_heads) * nsplit * (c.head_dim + 2);
}

hipError_t launch_attention_at(const KvCache &c, const float *query, float *output, uint32_t query_heads,
                               const int32_t *position_ptr, float scale, float *partials, hipStream_t stream,
                               const uint64_t *tree_mask, const int32_t *tree_base) {
    if (query_heads == 0 || c.head_dim > 1024) return hipErrorInvalidValue;
    if (mfma_attention_supported(c, query_heads))
        return launch_mfma_attention(c, query, output, partials, query_heads, 0, position_ptr, c.max_tokens, scale,
                                     stream, tree_mask, tree_base);
    if (tree_mask) return hipErrorInvalidValue;  // tree masks: the MFMA and decode kernels only
    AttnArgs args{};
    args.c = c;
    args.query = query;
    args.partials = partials;
    set_head_plan(args, c, query_heads);
    args.split = kDevicePositionSplit;
    args.nsplit = (c.max_tokens + kDevicePositionSplit - 1) / kDevicePositionSplit;
    args.scale = scale;
    args.position_ptr = position_ptr;
    return launch_split_and_merge(args, output, stream);
}

hipError_t launch_attention(const AttentionLaunch &a, hipStream_t stream) {
    const KvCache &c = *a.cache;
    if (a.position >= c.tokens || a.query_heads == 0 || c.head_dim > 1024) return hipErrorInvalidValue;
    if (mfma_attention_supported(c, a.query_heads))
        return launch_mfma_attention(c, a.query, a.output, a.partials, a.query_heads, a.position, nullptr,
                                     a.position + 1, a.scale, stream);
    AttnArgs args{};
    args.c = c;
    args.query = a.query;
    args.partials = a.partials;
    set_head_plan(args, c, a.query_heads);
    args.tokens = a.position + 1;
    args.split = split_tokens(c, args.tokens);
    args.nsplit = (args.tokens + args.split - 1) / args.split;
    args.scale = a.scale;
    args.position_ptr = nullptr;
    return launch_split_and_merge(args, a.output, stream);
}

}  // namespace qwn
