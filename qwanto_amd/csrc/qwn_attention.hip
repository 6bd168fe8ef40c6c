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
// Layout: 16-token pages, K/V int8 [page][kv_head][16][head_dim], scales
// fp32 [page][16][groups] with groups over the flattened kv_head*head_dim
// channels (the reference's token-major grouping).
#include "qwn_device.h"
#include "qwn_internal.h"

#include <algorithm>

namespace qwn {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kMaxSplitTokens = 256;

__device__ __forceinline__ size_t kv_offset(const KvCache &c, uint32_t token, uint32_t head) {
    const uint32_t page = token / kKvPageTokens, slot = token % kKvPageTokens;
    return ((static_cast<size_t>(page) * c.kv_heads + head) * kKvPageTokens + slot) * c.head_dim;
}

__device__ __forceinline__ size_t scale_offset(const KvCache &c, uint32_t token) {
    return static_cast<size_t>(token) * c.groups;  // pages are contiguous: [page][16][groups]
}

// grid (groups, 2): y = 0 quantizes K, y = 1 quantizes V.  64 threads, one
// per channel of the group.
__global__ __launch_bounds__(64) void kv_append_kernel(KvCache c, const float *__restrict__ key,
                                                       const float *__restrict__ value, uint32_t token,
                                                       const int32_t *__restrict__ token_ptr) {
    if (token_ptr) token = static_cast<uint32_t>(*token_ptr);
    if (token >= c.max_tokens) return;
    const uint32_t g = blockIdx.x;
    const bool is_v = blockIdx.y == 1;
    const float *src = is_v ? value : key;
    const uint32_t ch = g * 64 + threadIdx.x;
    const bool valid = ch < c.channels;
    const float v = valid ? src[ch] : 0.0f;
    float amax = (valid && isfinite(v)) ? fabsf(v) : 0.0f;
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    if (threadIdx.x == 0) (is_v ? c.value_scales : c.key_scales)[scale_offset(c, token) + g] = scale;
    if (valid) {
        int8_t q = 0;
        if (isfinite(v)) {
            const float s = v / scale;  // IEEE division, like the CPU path
            q = s >= 127.0f ? 127 : (s <= -127.0f ? -127 : static_cast<int8_t>(__builtin_rintf(s)));
        }
        const uint32_t head = ch / c.head_dim, dim = ch % c.head_dim;
        (is_v ? c.values : c.keys)[kv_offset(c, token, head) + dim] = q;
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
    const uint32_t kvh = blockIdx.y;
    const uint32_t split = blockIdx.x;
    const uint32_t t0 = split * a.split;
    const uint32_t tokens = a.position_ptr ? static_cast<uint32_t>(*a.position_ptr) + 1u : a.tokens;
    const uint32_t G = a.group;
    if (t0 >= tokens) {
        // a split past the current position (fixed grid): an empty partial
        for (uint32_t i = threadIdx.x; i < G * D; i += blockDim.x) {
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
    const uint32_t n = min(a.split, tokens - t0);
    float *q = sm;                              // [GMAX][D]
    float *p = q + GMAX * D;                    // [split][GMAX]
    float *wred = p + kMaxSplitTokens * GMAX;   // [4 waves][GMAX]
    float *pv = wred + 4 * GMAX;                // PV reduction [phases][GMAX][D]

    for (uint32_t i = threadIdx.x; i < GMAX * D; i += blockDim.x) {
        const uint32_t g = i / D, d = i % D;
        q[i] = g < G ? a.query[(static_cast<size_t>(kvh) * G + g) * D + d] : 0.0f;
    }
    __syncthreads();

    // ---- scores: one thread per token, all query heads of the group ----
    const uint32_t t = threadIdx.x;
    float s[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) s[g] = -INFINITY;
    if (t < n) {
        const uint32_t tok = t0 + t;
        const int8_t *krow = c.keys + kv_offset(c, tok, kvh);
        const float *ks = c.key_scales + scale_offset(c, tok);
        float dot[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) dot[g] = 0.0f;
        if (FAST) {
            for (uint32_t c0 = 0; c0 < D; c0 += 16) {
                const uint4 kw = *reinterpret_cast<const uint4 *>(krow + c0);
                const float sc = ks[(kvh * D + c0) / 64];
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
                const float kf = static_cast<float>(krow[d]) * ks[(kvh * D + d) / 64];
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
            const int8_t *vrow = c.values + kv_offset(c, tok, kvh);
            const float *vs = c.value_scales + scale_offset(c, tok);
            float vf[4];
            if (FAST) {
                const uint32_t w = *reinterpret_cast<const uint32_t *>(vrow + quad * 4);
                const float sc = vs[(kvh * D + quad * 4) / 64];
#pragma unroll
                for (int i = 0; i < 4; ++i) vf[i] = i8(w, i) * sc;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t d = quad * 4 + i;
                    vf[i] = d < D ? static_cast<float>(vrow[d]) * vs[(kvh * D + d) / 64] : 0.0f;
                }
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
        const uint32_t head = kvh * G + g;
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
    hipLaunchKernelGGL((attention_split_kernel<GMAX, FAST>), dim3(args.nsplit, args.c.kv_heads),
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
// the append quantizes per 64-channel group as kv_append_kernel.
__global__ __launch_bounds__(1024) void rope_append_kernel(KvCache c, float *__restrict__ q, uint32_t q_heads,
                                                           const float *__restrict__ k,
                                                           const float *__restrict__ v,
                                                           const float *__restrict__ cos_tab,
                                                           const float *__restrict__ sin_tab,
                                                           const int32_t *__restrict__ pos_ptr) {
    extern __shared__ float kr[];  // [channels] rotated key
    const uint32_t pos = static_cast<uint32_t>(*pos_ptr);
    const uint32_t D = c.head_dim, half = D / 2;
    const uint32_t row = pos < c.max_tokens ? pos : 0;
    const float *ct = cos_tab + static_cast<size_t>(row) * half;
    const float *st = sin_tab + static_cast<size_t>(row) * half;
    for (uint32_t p = threadIdx.x; p < q_heads * half; p += blockDim.x) {
        const uint32_t h = p / half, i = p % half;
        float *r = q + static_cast<size_t>(h) * D;
        const float a = r[i], b = r[i + half];
        r[i] = fmaf(a, ct[i], -(b * st[i]));
        r[i + half] = fmaf(a, st[i], b * ct[i]);
    }
    for (uint32_t p = threadIdx.x; p < c.kv_heads * half; p += blockDim.x) {
        const uint32_t h = p / half, i = p % half;
        const float a = k[h * D + i], b = k[h * D + i + half];
        kr[h * D + i] = fmaf(a, ct[i], -(b * st[i]));
        kr[h * D + i + half] = fmaf(a, st[i], b * ct[i]);
    }
    __syncthreads();
    if (pos >= c.max_tokens) return;
    const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64, nwaves = blockDim.x / 64;
    for (uint32_t gi = wave; gi < 2 * c.groups; gi += nwaves) {
        const bool is_v = gi >= c.groups;
        const uint32_t g = is_v ? gi - c.groups : gi;
        const uint32_t ch = g * 64 + lane;
        const bool valid = ch < c.channels;
        const float x = valid ? (is_v ? v[ch] : kr[ch]) : 0.0f;
        float amax = (valid && isfinite(x)) ? fabsf(x) : 0.0f;
        for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        if (lane == 0) (is_v ? c.value_scales : c.key_scales)[scale_offset(c, pos) + g] = scale;
        if (valid) {
            int8_t qv = 0;
            if (isfinite(x)) {
                const float sq = x / scale;  // IEEE division, like the CPU path
                qv = sq >= 127.0f ? 127 : (sq <= -127.0f ? -127 : static_cast<int8_t>(__builtin_rintf(sq)));
            }
            (is_v ? c.values : c.keys)[kv_offset(c, pos, ch / D) + ch % D] = qv;
        }
    }
}

// ---- decode attention -------------------------------------------------------
//
// One workgroup per (query head or KV head, split of `split` tokens), 256
// threads: while one split spans the context (<= 1024 tokens) a workgroup
// serves one query head (short contexts are latency-bound; the K/V rows are
// re-read per query head from L2), past that all G query heads of the KV
// head share each K/V load (long contexts are bandwidth-bound); online softmax over chunks of 256
// tokens, so one split covers contexts up to 1024 tokens and no merge pass
// is needed (nsplit == 1 writes the output).  Each chunk is one memory round
// trip: a thread loads one token's whole key row (scores) and, at the same
// time, the value bytes it needs later; nothing waits on a cross-lane
// reduction per token.
//   scores: thread = token, s_g = sum over 64-channel groups of
//           k_scale * sum q_g,c * k_c (the group scale factored out)
//   P.V:    thread = (4-channel quad, token phase), V prefetched, phases
//           summed through LDS at the end
//
// Decode mode (key != null): the workgroup also applies RoPE to its query
// heads (c/qwanto_decode.c:686-729) and, for the split holding the current
// position, rotates and Q8-quantizes the current key and value
// (c/qwanto_turboquant.c:555-600), stores them in the cache for later steps
// and attends to them from LDS.
struct DecodeAttnArgs {
    KvCache c;
    const float *query;      // [H][D]
    float *output;           // [H][D] (nsplit == 1)
    float *partials;         // [H][nsplit][D + 2] (nsplit > 1)
    uint32_t group;          // query heads per KV head
    uint32_t heads_per_wg;   // query heads one workgroup handles (divides group)
    uint32_t split;
    uint32_t nsplit;
    float scale;
    uint32_t position;
    const int32_t *position_ptr;
    const float *key;        // decode mode: current token fp32 [channels]
    const float *value;
    const float *cos_tab;    // [max_tokens][D/2]
    const float *sin_tab;
};

__device__ __forceinline__ float rope_at(const float *x, uint32_t d, uint32_t half, const float *ct, const float *st) {
    const uint32_t i = d < half ? d : d - half;
    const float a = x[i], b = x[i + half];
    return d < half ? fmaf(a, ct[i], -(b * st[i])) : fmaf(a, st[i], b * ct[i]);
}

__device__ __forceinline__ int8_t q8_of(float x, float scale) {
    if (!isfinite(x)) return 0;
    const float s = x / scale;  // IEEE division, like the CPU path
    return s >= 127.0f ? 127 : (s <= -127.0f ? -127 : static_cast<int8_t>(__builtin_rintf(s)));
}

__device__ __forceinline__ float i8f(uint32_t w, int i) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * i)) & 0xffu));
}

template <int D, int GMAX>
__global__ __launch_bounds__(256) void decode_attention_kernel(DecodeAttnArgs a) {
    constexpr int NG = D / 64;                 // Q8 scale groups per head
    constexpr int KW = D / 16;                 // uint4 words of one K or V row
    constexpr int CH = D <= 128 ? 256 : 128;   // tokens per chunk (V rows staged in LDS)
    constexpr int QUADS = D / 4;               // P.V: 4-channel quads
    constexpr int PH = 256 / QUADS;            // P.V: token phases
    __shared__ __align__(16) float q_s[GMAX * D];
    __shared__ float s_s[GMAX * CH];
    __shared__ float red[2][4][GMAX];
    __shared__ __align__(16) float pv_s[PH * GMAX * D];
    __shared__ __align__(16) uint4 v_s[CH * KW];   // the chunk's V rows
    __shared__ float vsc_s[CH * NG];               // and their scales
    __shared__ __align__(16) int8_t kcur[D];
    __shared__ __align__(16) int8_t vcur[D];
    __shared__ float kcur_s[NG], vcur_s[NG];
    const KvCache &c = a.c;
    // this workgroup: KV head kvh, its query heads h0 .. h0 + G - 1
    const uint32_t G = a.heads_per_wg, wgs_per_kv = a.group / G;
    const uint32_t kvh = blockIdx.y / wgs_per_kv, split = blockIdx.x;
    const uint32_t h0 = kvh * a.group + (blockIdx.y % wgs_per_kv) * G;
    const bool writer = blockIdx.y % wgs_per_kv == 0;  // appends the current token
    const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const uint32_t pos = a.position_ptr ? static_cast<uint32_t>(*a.position_ptr) : a.position;
    if (pos >= c.max_tokens) return;
    const uint32_t tokens = pos + 1;
    const uint32_t t0 = split * a.split;
    if (t0 >= tokens) {
        // a split past the position (fixed grid): an empty partial
        for (uint32_t i = tid; i < G * D; i += blockDim.x) {
            const uint32_t g = i / D, d = i % D;
            float *dst = a.partials + (static_cast<size_t>(h0 + g) * a.nsplit + split) * (D + 2);
            dst[2 + d] = 0.0f;
            if (d == 0) {
                dst[0] = -INFINITY;
                dst[1] = 0.0f;
            }
        }
        return;
    }
    const uint32_t t1 = min(tokens, t0 + a.split);
    const bool rope = a.key != nullptr;
    const bool cur = rope && pos >= t0 && pos < t1;
    constexpr uint32_t half = D / 2;
    const float *ct = rope ? a.cos_tab + static_cast<size_t>(pos) * half : nullptr;
    const float *st = rope ? a.sin_tab + static_cast<size_t>(pos) * half : nullptr;

    // 1. query heads of this KV head (rotated in decode mode) -> LDS
    for (uint32_t i = tid; i < GMAX * D; i += blockDim.x) {
        const uint32_t g = i / D, d = i % D;
        float v = 0.0f;
        if (g < G) {
            const float *qh = a.query + static_cast<size_t>(h0 + g) * D;
            v = rope ? rope_at(qh, d, half, ct, st) : qh[d];
        }
        q_s[i] = v;
    }
    // the current token's key (rotated) and value: one wave per 64-channel group
    if (cur) {
        for (uint32_t gi = wave; gi < 2 * NG; gi += 4) {
            const bool is_v = gi >= NG;
            const uint32_t grp = is_v ? gi - NG : gi;
            const uint32_t d = grp * 64 + lane;
            const float *src = (is_v ? a.value : a.key) + static_cast<size_t>(kvh) * D;
            const float x = is_v ? src[d] : rope_at(src, d, half, ct, st);
            const float amax = wave_max_all(isfinite(x) ? fabsf(x) : 0.0f);
            const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const int8_t qv = q8_of(x, scale);
            (is_v ? vcur : kcur)[d] = qv;
            if (writer) (is_v ? c.values : c.keys)[kv_offset(c, pos, kvh) + d] = qv;
            if (lane == 0) {
                (is_v ? vcur_s : kcur_s)[grp] = scale;
                if (writer) (is_v ? c.value_scales : c.key_scales)[scale_offset(c, pos) + kvh * NG + grp] = scale;
            }
        }
    }
    __syncthreads();

    const uint32_t quad = tid % QUADS, ph = tid / QUADS;
    const uint32_t vgrp = (quad * 4) / 64;
    float m_run[GMAX], l_run[GMAX], acc[GMAX][4];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[g][i] = 0.0f;
    }

    for (uint32_t c0 = t0; c0 < t1; c0 += CH) {
        const uint32_t n = min(static_cast<uint32_t>(CH), t1 - c0);
        // 2. one round trip: thread tid takes token c0 + tid -- its key row,
        //    value row and scales (global loads; the current token from LDS)
        const bool has = tid < n;
        const uint32_t tk = has ? c0 + tid : t0;
        const bool is_cur = cur && has && tk == pos;
        uint4 kr[KW], vr[KW];
        float ks[NG], vsc[NG];
        {
            // the current token's slot is being written by this launch: load
            // any written row instead and take the token from LDS below
            const uint32_t tl = is_cur ? t0 : tk;
            const uint4 *kp = reinterpret_cast<const uint4 *>(c.keys + kv_offset(c, tl, kvh));
            const uint4 *vp = reinterpret_cast<const uint4 *>(c.values + kv_offset(c, tl, kvh));
#pragma unroll
            for (int w = 0; w < KW; ++w) {
                kr[w] = kp[w];
                vr[w] = vp[w];
            }
            const size_t so = scale_offset(c, tl) + kvh * NG;
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                ks[g] = c.key_scales[so + g];
                vsc[g] = c.value_scales[so + g];
            }
        }
        if (cur) {
#pragma unroll
            for (int w = 0; w < KW; ++w) {
                // component selects (a select of the uint4 struct goes through scratch)
                const uint4 kc = reinterpret_cast<const uint4 *>(kcur)[w];
                const uint4 vc = reinterpret_cast<const uint4 *>(vcur)[w];
                kr[w].x = is_cur ? kc.x : kr[w].x;
                kr[w].y = is_cur ? kc.y : kr[w].y;
                kr[w].z = is_cur ? kc.z : kr[w].z;
                kr[w].w = is_cur ? kc.w : kr[w].w;
                vr[w].x = is_cur ? vc.x : vr[w].x;
                vr[w].y = is_cur ? vc.y : vr[w].y;
                vr[w].z = is_cur ? vc.z : vr[w].z;
                vr[w].w = is_cur ? vc.w : vr[w].w;
            }
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                ks[g] = is_cur ? kcur_s[g] : ks[g];
                vsc[g] = is_cur ? vcur_s[g] : vsc[g];
            }
        }
        // the value row and its scales -> LDS for the P.V phase
#pragma unroll
        for (int w = 0; w < KW; ++w) v_s[tid % CH * KW + w] = vr[w];
#pragma unroll
        for (int g = 0; g < NG; ++g) vsc_s[tid % CH * NG + g] = has ? vsc[g] : 0.0f;
        // 3. scores of this thread's token
        float sc[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) sc[g] = 0.0f;
#pragma unroll
        for (int grp = 0; grp < NG; ++grp) {
            float part[GMAX];
#pragma unroll
            for (int g = 0; g < GMAX; ++g) part[g] = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint4 kw = kr[grp * 4 + w];
                const uint32_t k4[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float k0 = i8f(k4[e], 0), k1 = i8f(k4[e], 1), k2 = i8f(k4[e], 2), k3 = i8f(k4[e], 3);
                    const uint32_t d0 = grp * 64 + w * 16 + e * 4;
#pragma unroll
                    for (int g = 0; g < GMAX; ++g) {
                        if (static_cast<uint32_t>(g) >= G) break;
                        const float4 qq = *reinterpret_cast<const float4 *>(q_s + g * D + d0);
                        part[g] = fmaf(qq.x, k0, part[g]);
                        part[g] = fmaf(qq.y, k1, part[g]);
                        part[g] = fmaf(qq.z, k2, part[g]);
                        part[g] = fmaf(qq.w, k3, part[g]);
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < GMAX; ++g) sc[g] = fmaf(part[g], ks[grp], sc[g]);
        }
        // 4. chunk softmax, running max and sum
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            sc[g] = (has && static_cast<uint32_t>(g) < G) ? sc[g] * a.scale : -INFINITY;
            const float m = wave_max_all(sc[g]);
            if (lane == 0) red[0][wave][g] = m;
        }
        __syncthreads();
        float alpha[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            const float mc = fmaxf(fmaxf(red[0][0][g], red[0][1][g]), fmaxf(red[0][2][g], red[0][3][g]));
            const float mn = fmaxf(m_run[g], mc);
            alpha[g] = m_run[g] == -INFINITY ? 0.0f : expf(m_run[g] - mn);
            m_run[g] = mn;
            const float p = (has && static_cast<uint32_t>(g) < G) ? expf(sc[g] - mn) : 0.0f;
            if (tid < CH) s_s[g * CH + tid] = p;
            const float ps = wave_sum_all(p);
            if (lane == 0) red[1][wave][g] = ps;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            l_run[g] = l_run[g] * alpha[g] + ((red[1][0][g] + red[1][1][g]) + (red[1][2][g] + red[1][3][g]));
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] *= alpha[g];
        }
        // 5. P.V of this thread's quad over its tokens (from LDS)
        for (uint32_t tl = ph; tl < n; tl += PH) {
            const uint32_t vw = reinterpret_cast<const uint32_t *>(v_s + tl * KW)[quad];
            const float vs = vsc_s[tl * NG + vgrp];
            const float v0 = i8f(vw, 0) * vs, v1 = i8f(vw, 1) * vs, v2 = i8f(vw, 2) * vs, v3 = i8f(vw, 3) * vs;
#pragma unroll
            for (int g = 0; g < GMAX; ++g) {
                if (static_cast<uint32_t>(g) >= G) break;
                const float p = s_s[g * CH + tl];
                acc[g][0] = fmaf(p, v0, acc[g][0]);
                acc[g][1] = fmaf(p, v1, acc[g][1]);
                acc[g][2] = fmaf(p, v2, acc[g][2]);
                acc[g][3] = fmaf(p, v3, acc[g][3]);
            }
        }
        __syncthreads();
    }

    // 6. sum the token phases; output or partial
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
        if (static_cast<uint32_t>(g) < G)
            *reinterpret_cast<float4 *>(pv_s + (ph * GMAX + g) * D + quad * 4) =
                make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
    __syncthreads();
    for (uint32_t i = tid; i < G * D; i += blockDim.x) {
        const uint32_t g = i / D, d = i % D;
        float o = 0.0f;
#pragma unroll
        for (int p = 0; p < PH; ++p) o += pv_s[(p * GMAX + g) * D + d];
        const uint32_t head = h0 + g;
        if (a.nsplit == 1) {
            a.output[static_cast<size_t>(head) * D + d] = o / l_run[g];
        } else {
            float *dst = a.partials + (static_cast<size_t>(head) * a.nsplit + split) * (D + 2);
            dst[2 + d] = o;
            if (d == 0) {
                dst[0] = m_run[g];
                dst[1] = l_run[g];
            }
        }
    }
}

// grid (query heads): the split partials of one head, weighted by
// exp(m_s - max m) (empty splits carry m = -inf, l = 0 and drop out).
__global__ __launch_bounds__(256) void decode_merge_kernel(const float *__restrict__ partials, float *out,
                                                           uint32_t nsplit, uint32_t D) {
    __shared__ float w_s[1024];
    __shared__ float total_s;
    const uint32_t head = blockIdx.x;
    const float *base = partials + static_cast<size_t>(head) * nsplit * (D + 2);
    for (uint32_t sidx = threadIdx.x; sidx < nsplit; sidx += blockDim.x) w_s[sidx] = base[sidx * (D + 2)];
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t sidx = 0; sidx < nsplit; ++sidx) mx = fmaxf(mx, w_s[sidx]);
    __syncthreads();
    for (uint32_t sidx = threadIdx.x; sidx < nsplit; sidx += blockDim.x) {
        const float m = base[sidx * (D + 2)];
        w_s[sidx] = m == -INFINITY ? 0.0f : expf(m - mx);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        for (uint32_t sidx = 0; sidx < nsplit; ++sidx) total = fmaf(base[sidx * (D + 2) + 1], w_s[sidx], total);
        total_s = total;
    }
    __syncthreads();
    const float inv = total_s > 0.0f ? 1.0f / total_s : 0.0f;
    for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
        float o = 0.0f;
        for (uint32_t sidx = 0; sidx < nsplit; ++sidx) o = fmaf(base[sidx * (D + 2) + 2 + d], w_s[sidx], o);
        out[static_cast<size_t>(head) * D + d] = o * inv;
    }
}

template <int D, int GMAX>
hipError_t launch_decode_kernel(const DecodeAttnArgs &args, hipStream_t stream) {
    const uint32_t wgs_per_kv = args.group / args.heads_per_wg;
    hipLaunchKernelGGL((decode_attention_kernel<D, GMAX>), dim3(args.nsplit, args.c.kv_heads * wgs_per_kv),
                       dim3(256), 0, stream, args);
    return hipGetLastError();
}

template <int D>
hipError_t launch_decode_g(const DecodeAttnArgs &args, hipStream_t stream) {
    if (args.heads_per_wg <= 1) return launch_decode_kernel<D, 1>(args, stream);
    if (args.heads_per_wg <= 2) return launch_decode_kernel<D, 2>(args, stream);
    if (args.heads_per_wg <= 4) return launch_decode_kernel<D, 4>(args, stream);
    return launch_decode_kernel<D, 8>(args, stream);
}

hipError_t launch_decode_attention_args(const DecodeAttnArgs &args, float *output, hipStream_t stream) {
    hipError_t e;
    switch (args.c.head_dim) {
    case 64: e = launch_decode_g<64>(args, stream); break;
    case 128: e = launch_decode_g<128>(args, stream); break;
    case 256: e = launch_decode_g<256>(args, stream); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || args.nsplit == 1) return e;
    hipLaunchKernelGGL(decode_merge_kernel, dim3(args.c.kv_heads * args.group), dim3(256), 0, stream, args.partials,
                       output, args.nsplit, args.c.head_dim);
    return hipGetLastError();
}

}  // namespace

size_t kv_cache_layout(KvCache &c, uint8_t *base) {
    c.channels = c.kv_heads * c.head_dim;
    c.groups = (c.channels + 63u) / 64u;
    c.pages = (c.max_tokens + kKvPageTokens - 1) / kKvPageTokens;
    const size_t slots = static_cast<size_t>(c.pages) * kKvPageTokens;
    const size_t value_bytes = (slots * c.channels + 255) & ~static_cast<size_t>(255);
    const size_t scale_bytes = (slots * c.groups * sizeof(float) + 255) & ~static_cast<size_t>(255);
    if (base) {
        c.keys = reinterpret_cast<int8_t *>(base);
        c.values = reinterpret_cast<int8_t *>(base + value_bytes);
        c.key_scales = reinterpret_cast<float *>(base + 2 * value_bytes);
        c.value_scales = reinterpret_cast<float *>(base + 2 * value_bytes + scale_bytes);
    }
    return 2 * value_bytes + 2 * scale_bytes;
}

hipError_t launch_rope_append(const KvCache &c, float *query, uint32_t query_heads, const float *key,
                              const float *value, const float *cos_tab, const float *sin_tab,
                              const int32_t *pos_ptr, hipStream_t stream) {
    if (c.head_dim % 2 || c.channels > 8192) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_append_kernel, dim3(1), dim3(1024), c.channels * sizeof(float), stream, c, query,
                       query_heads, key, value, cos_tab, sin_tab, pos_ptr);
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

hipError_t launch_decode_attention(const DecodeAttentionLaunch &l, hipStream_t stream) {
    const KvCache &c = *l.cache;
    if (!decode_attention_supported(c, l.query_heads) || (l.key && (c.head_dim % 64 || !l.value || !l.cos_tab ||
                                                                    !l.sin_tab)))
        return hipErrorInvalidValue;
    DecodeAttnArgs args{};
    args.c = c;
    args.query = l.query;
    args.output = l.output;
    args.partials = l.partials;
    args.group = l.query_heads / c.kv_heads;
    args.split = decode_split_tokens(c, l.span_tokens);
    args.nsplit = (l.span_tokens + args.split - 1) / args.split;
    // one query head per workgroup while a workgroup spans the context (the
    // latency case: K/V are re-read per head from L2); all heads of a KV
    // head together once the context is split (the bandwidth case)
    args.heads_per_wg = args.nsplit == 1 ? 1 : args.group;
    if (args.nsplit > 1 && !l.partials) return hipErrorInvalidValue;
    if (args.nsplit > 1024) return hipErrorInvalidValue;
    args.scale = l.scale;
    args.position = l.position;
    args.position_ptr = l.position_ptr;
    args.key = l.key;
    args.value = l.value;
    args.cos_tab = l.cos_tab;
    args.sin_tab = l.sin_tab;
    return launch_decode_attention_args(args, l.output, stream);
}

hipError_t launch_kv_append(const KvCache &c, const float *key, const float *value, uint32_t token,
                            hipStream_t stream) {
    if (token >= c.max_tokens) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_append_kernel, dim3(c.groups, 2), dim3(64), 0, stream, c, key, value, token,
                       static_cast<const int32_t *>(nullptr));
    return hipGetLastError();
}

hipError_t launch_kv_append_at(const KvCache &c, const float *key, const float *value, const int32_t *token_ptr,
                               hipStream_t stream) {
    hipLaunchKernelGGL(kv_append_kernel, dim3(c.groups, 2), dim3(64), 0, stream, c, key, value, 0u, token_ptr);
    return hipGetLastError();
}

size_t attention_workspace_floats(const KvCache &c, uint32_t query_heads, uint32_t position) {
    const uint32_t tokens = position + 1;
    const uint32_t s = split_tokens(c, tokens);
    const uint32_t nsplit = (tokens + s - 1) / s;
    return std::max(static_cast<size_t>(query_heads) * nsplit * (c.head_dim + 2),
                    decode_attention_workspace_floats(c, query_heads, tokens));
}

namespace {
hipError_t launch_split_and_merge(AttnArgs &args, float *output, hipStream_t stream) {
    hipError_t e;
    if (args.group <= 1) e = launch_fast_or_not<1>(args, stream);
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
    const uint32_t nsplit = (c.max_tokens + kDevicePositionSplit - 1) / kDevicePositionSplit;
    return static_cast<size_t>(query_heads) * nsplit * (c.head_dim + 2);
}

hipError_t launch_attention_at(const KvCache &c, const float *query, float *output, uint32_t query_heads,
                               const int32_t *position_ptr, float scale, float *partials, hipStream_t stream) {
    if (query_heads % c.kv_heads != 0 || c.head_dim > 1024) return hipErrorInvalidValue;
    AttnArgs args{};
    args.c = c;
    args.query = query;
    args.partials = partials;
    args.query_heads = query_heads;
    args.group = query_heads / c.kv_heads;
    args.split = kDevicePositionSplit;
    args.nsplit = (c.max_tokens + kDevicePositionSplit - 1) / kDevicePositionSplit;
    args.scale = scale;
    args.position_ptr = position_ptr;
    return launch_split_and_merge(args, output, stream);
}

hipError_t launch_attention(const AttentionLaunch &a, hipStream_t stream) {
    const KvCache &c = *a.cache;
    if (a.position >= c.tokens || a.query_heads % c.kv_heads != 0 || c.head_dim > 1024)
        return hipErrorInvalidValue;
    if (decode_attention_supported(c, a.query_heads)) {
        DecodeAttentionLaunch l;
        l.cache = &c;
        l.query = a.query;
        l.output = a.output;
        l.partials = a.partials;
        l.query_heads = a.query_heads;
        l.position = a.position;
        l.span_tokens = a.position + 1;
        l.scale = a.scale;
        return launch_decode_attention(l, stream);
    }
    AttnArgs args{};
    args.c = c;
    args.query = a.query;
    args.partials = a.partials;
    args.query_heads = a.query_heads;
    args.group = a.query_heads / c.kv_heads;
    args.tokens = a.position + 1;
    args.split = split_tokens(c, args.tokens);
    args.nsplit = (args.tokens + args.split - 1) / args.split;
    args.scale = a.scale;
    args.position_ptr = nullptr;
    return launch_split_and_merge(args, a.output, stream);
}

}  // namespace qwn
