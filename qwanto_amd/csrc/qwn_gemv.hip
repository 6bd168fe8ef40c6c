// Quantized GEMV / small-batch GEMM kernels for gfx950 (CDNA4).
//
// Decode at batch 1 reads every weight exactly once, so the kernel is an
// HBM stream: each lane loads whole 64-byte units with 128-bit loads (all
// of its loads issued before it touches the activations), the int8
// activations are staged once per workgroup in LDS in the byte order the
// unpack produces, the 2-/4-bit codes are widened with shift+mask and fed
// to v_dot4_i32_i8, and per-row partial sums are combined through LDS.
//
// Semantics follow the reference CPU kernels:
//   HyperVSQ-2  y = xs * sum_blocks (d/8 * sum_oct s_oct*(sum code*a - sum a)
//                                    + m * sum a)        c/qwanto_kernels.c:619-667
//   Q4_0        y = xs * sum_blocks d * (sum nibble*a - 8 * sum a)
//                                                         c/qwanto_kernels.c:503-534,1178-1322
//   F16         y = sum_k x[k] * w[k]                    c/qwanto_kernels.c:1531-1616
// The integer parts are exact; only the fp32 combination order differs
// from the CPU's.
#include "qwn_internal.h"

#include <algorithm>

namespace qwn {
namespace {

constexpr uint32_t kMask2 = 0x03030303u;
constexpr uint32_t kMask4 = 0x0f0f0f0fu;

__device__ __forceinline__ float half_to_float(uint32_t bits) {
    // v_cvt_f32_f16 keeps fp16 subnormals (the default f16 denormal mode),
    // matching the CPU's exact conversion (c/qwanto_kernels.c:264-285).
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// ---- activation staging ------------------------------------------------
//
// HyperVSQ-2: a code dword holds 16 consecutive weights, weight 4j+i in
// bits 2i of byte j, so (w >> 2i) & 0x03030303 holds weights {i, 4+i, 8+i,
// 12+i}.  Each 16-activation group is stored transposed to match:
// dword i = bytes {a_i, a_{4+i}, a_{8+i}, a_{12+i}}.
// Q4_0: a nibble dword holds 8 weights, low nibbles = even elements, so
// each 8-activation group is stored as {a0,a2,a4,a6},{a1,a3,a5,a7}.

template <int KIND>
__device__ __forceinline__ void store_block32(uint8_t *act_token, uint32_t e0,
                                              const uint32_t w[8]) {
    if (KIND == kHvsq2) {
        const uint32_t u = e0 / 256, off = e0 % 256;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            uint32_t p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                p[i] = byte_of(w[4 * g + 0], i) | (byte_of(w[4 * g + 1], i) << 8) |
                       (byte_of(w[4 * g + 2], i) << 16) | (byte_of(w[4 * g + 3], i) << 24);
            *reinterpret_cast<uint4 *>(act_token + u * 272 + (off / 16 + g) * 16) =
                make_uint4(p[0], p[1], p[2], p[3]);
        }
    } else {
        const uint32_t u = e0 / 128, off = e0 % 128;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t a = w[2 * g], b = w[2 * g + 1];
            const uint32_t lo = byte_of(a, 0) | (byte_of(a, 2) << 8) | (byte_of(b, 0) << 16) |
                                (byte_of(b, 2) << 24);
            const uint32_t hi = byte_of(a, 1) | (byte_of(a, 3) << 8) | (byte_of(b, 1) << 16) |
                                (byte_of(b, 3) << 24);
            *reinterpret_cast<uint2 *>(act_token + u * 144 + (off / 8 + g) * 8) = make_uint2(lo, hi);
        }
    }
}

// Stage `ntok` int8 tokens (row stride `stride` bytes, 16-byte aligned) of
// K valid activations, zero padded to units*unit_elems, plus the sum of
// every 32-activation block.
template <int KIND, int MT>
__device__ void stage_int8(const int8_t *__restrict__ x, uint32_t stride, uint32_t K,
                           uint32_t units, uint32_t ntok, uint8_t *act, int32_t *sums) {
    const uint32_t nblk = units * unit_elems(KIND) / 32;
    const uint32_t token_bytes = units * unit_lds_bytes(KIND);
    for (uint32_t idx = threadIdx.x; idx < MT * nblk; idx += blockDim.x) {
        const uint32_t t = idx / nblk, b = idx % nblk, e0 = b * 32;
        uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (t < ntok && e0 < K) {
            const int8_t *src = x + static_cast<size_t>(t) * stride + e0;
            if (e0 + 32 <= K) {
                const uint4 v0 = *reinterpret_cast<const uint4 *>(src);
                const uint4 v1 = *reinterpret_cast<const uint4 *>(src + 16);
                w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
                w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
            } else {
                for (uint32_t i = 0; i < K - e0; ++i)
                    w[i >> 2] |= (static_cast<uint32_t>(static_cast<uint8_t>(src[i]))) << (8 * (i & 3));
            }
        }
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = dot4(w[i], 0x01010101u, s);
        sums[t * nblk + b] = s;
        store_block32<KIND>(act + t * token_bytes, e0, w);
    }
}

// fp32 activations for F16 weights: unit = 8 floats, zero padded.
template <int MT>
__device__ void stage_f32(const float *__restrict__ x, uint32_t stride, uint32_t K,
                          uint32_t units, uint32_t ntok, float *act) {
    for (uint32_t idx = threadIdx.x; idx < MT * units; idx += blockDim.x) {
        const uint32_t t = idx / units, u = idx % units, e0 = u * 8;
        float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
        if (t < ntok && e0 < K) {
            const float *src = x + static_cast<size_t>(t) * stride + e0;
            if (e0 + 8 <= K) {
                v0 = *reinterpret_cast<const float4 *>(src);
                v1 = *reinterpret_cast<const float4 *>(src + 4);
            } else {
                float tmp[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                for (uint32_t i = 0; i < K - e0; ++i) tmp[i] = src[i];
                v0 = make_float4(tmp[0], tmp[1], tmp[2], tmp[3]);
                v1 = make_float4(tmp[4], tmp[5], tmp[6], tmp[7]);
            }
        }
        float4 *dst = reinterpret_cast<float4 *>(act + (static_cast<size_t>(t) * units + u) * 8);
        dst[0] = v0;
        dst[1] = v1;
    }
}

// ---- per-unit integer cores (shared by the GEMV and the dump kernel) ----

// sum over one octant of code*a (codes 0..3), octant = two code dwords.
__device__ __forceinline__ int hv_octant_dot(uint32_t w0, uint32_t w1, uint4 a0, uint4 a1) {
    int d = dot4(w0 & kMask2, a0.x, 0);
    d = dot4((w0 >> 2) & kMask2, a0.y, d);
    d = dot4((w0 >> 4) & kMask2, a0.z, d);
    d = dot4((w0 >> 6) & kMask2, a0.w, d);
    d = dot4(w1 & kMask2, a1.x, d);
    d = dot4((w1 >> 2) & kMask2, a1.y, d);
    d = dot4((w1 >> 4) & kMask2, a1.z, d);
    d = dot4((w1 >> 6) & kMask2, a1.w, d);
    return d;
}

// sum over one Q4_0 block of nibble*a; a0/a1 hold the staged activations
// of nibble dwords (0,1) and (2,3).
__device__ __forceinline__ int q4_block_dot(uint4 n, uint4 a0, uint4 a1) {
    int d = dot4(n.x & kMask4, a0.x, 0);
    d = dot4((n.x >> 4) & kMask4, a0.y, d);
    d = dot4(n.y & kMask4, a0.z, d);
    d = dot4((n.y >> 4) & kMask4, a0.w, d);
    d = dot4(n.z & kMask4, a1.x, d);
    d = dot4((n.z >> 4) & kMask4, a1.y, d);
    d = dot4(n.w & kMask4, a1.z, d);
    d = dot4((n.w >> 4) & kMask4, a1.w, d);
    return d;
}

struct GemvArgs {
    const uint8_t *payload;
    const uint8_t *meta;
    size_t payload_row_bytes;
    size_t meta_row_bytes;
    const void *input;
    const float *scales;
    float scale;
    float *output;
    uint32_t rows;
    uint32_t cols;
    uint32_t units;
    uint32_t lanes;
    uint32_t rows_per_wave;
    uint32_t ntok;
    uint32_t input_stride;
    uint32_t output_stride;
};

template <int KIND, int MT, int UPL>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = threadIdx.x % kWaveSize;
    const uint32_t wave = threadIdx.x / kWaveSize;
    const uint32_t L = a.lanes;
    const uint32_t grp = lane / L;
    const uint32_t j = lane - grp * L;
    const uint32_t row = (blockIdx.x * kGemvWaves + wave) * a.rows_per_wave + grp;
    const bool active = grp < a.rows_per_wave && row < a.rows;

    // 1. Issue every weight load of this lane before anything else.
    uint4 pay[UPL][KIND == kF16 ? 1 : 4];
    uint2 met[UPL];
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        const uint32_t u = j + i * L;
        const bool ok = active && u < a.units;
        if (KIND == kF16) {
            pay[i][0] = ok ? *reinterpret_cast<const uint4 *>(
                                 a.payload + row * a.payload_row_bytes + u * 16)
                           : make_uint4(0, 0, 0, 0);
        } else {
            const uint4 *src = reinterpret_cast<const uint4 *>(
                a.payload + row * a.payload_row_bytes + static_cast<size_t>(u) * 64);
#pragma unroll
            for (int q = 0; q < 4; ++q) pay[i][q] = ok ? src[q] : make_uint4(0, 0, 0, 0);
            met[i] = ok ? *reinterpret_cast<const uint2 *>(a.meta + row * a.meta_row_bytes +
                                                           static_cast<size_t>(u) * 8)
                        : make_uint2(0, 0);
        }
    }

    // 2. Stage the activations of all tokens in LDS.
    const uint32_t nblk = a.units * unit_elems(KIND) / 32;
    uint8_t *act = smem;
    int32_t *sums = reinterpret_cast<int32_t *>(smem + MT * a.units * unit_lds_bytes(KIND));
    float *red = reinterpret_cast<float *>(
        smem + MT * a.units * unit_lds_bytes(KIND) + (KIND == kF16 ? 0 : MT * nblk * 4));
    if (KIND == kF16)
        stage_f32<MT>(static_cast<const float *>(a.input), a.input_stride, a.cols, a.units,
                      a.ntok, reinterpret_cast<float *>(act));
    else
        stage_int8<KIND, MT>(static_cast<const int8_t *>(a.input), a.input_stride, a.cols,
                             a.units, a.ntok, act, sums);
    __syncthreads();

    // 3. Dot products.
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        const uint32_t u = j + i * L;
        if (!(active && u < a.units)) continue;
        if (KIND == kHvsq2) {
            const uint32_t *cw = reinterpret_cast<const uint32_t *>(pay[i]);
            const float d = half_to_float(met[i].x & 0xffffu);
            const float m = half_to_float(met[i].x >> 16);
            const uint32_t subs = met[i].y;
            int s1[MT], sa[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) s1[t] = sa[t] = 0;
#pragma unroll
            for (int o = 0; o < 8; ++o) {
                const int s = static_cast<int>((subs >> (4 * o)) & 15u);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const uint8_t *at = act + (t * a.units + u) * 272 + o * 32;
                    const uint4 a0 = *reinterpret_cast<const uint4 *>(at);
                    const uint4 a1 = *reinterpret_cast<const uint4 *>(at + 16);
                    const int so = sums[t * nblk + u * 8 + o];
                    s1[t] += s * (hv_octant_dot(cw[2 * o], cw[2 * o + 1], a0, a1) - so);
                    sa[t] += so;
                }
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                acc[t] = fmaf(d, static_cast<float>(s1[t]) * 0.125f, acc[t]);
                acc[t] = fmaf(m, static_cast<float>(sa[t]), acc[t]);
            }
        } else if (KIND == kQ4_0) {
            const uint32_t sc[2] = {met[i].x, met[i].y};
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float d = half_to_float(sc[b >> 1] >> (16 * (b & 1)));
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const uint8_t *at = act + (t * a.units + u) * 144 + b * 32;
                    const uint4 a0 = *reinterpret_cast<const uint4 *>(at);
                    const uint4 a1 = *reinterpret_cast<const uint4 *>(at + 16);
                    const int raw = q4_block_dot(pay[i][b], a0, a1) - 8 * sums[t * nblk + u * 4 + b];
                    acc[t] = fmaf(static_cast<float>(raw), d, acc[t]);
                }
            }
        } else {
            const uint32_t h[4] = {pay[i][0].x, pay[i][0].y, pay[i][0].z, pay[i][0].w};
            float wf[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                wf[2 * q] = half_to_float(h[q] & 0xffffu);
                wf[2 * q + 1] = half_to_float(h[q] >> 16);
            }
            const float *xa = reinterpret_cast<const float *>(act);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const float4 x0 = *reinterpret_cast<const float4 *>(xa + (t * a.units + u) * 8);
                const float4 x1 = *reinterpret_cast<const float4 *>(xa + (t * a.units + u) * 8 + 4);
                float s = acc[t];
                s = fmaf(wf[0], x0.x, s); s = fmaf(wf[1], x0.y, s);
                s = fmaf(wf[2], x0.z, s); s = fmaf(wf[3], x0.w, s);
                s = fmaf(wf[4], x1.x, s); s = fmaf(wf[5], x1.y, s);
                s = fmaf(wf[6], x1.z, s); s = fmaf(wf[7], x1.w, s);
                acc[t] = s;
            }
        }
    }

    // 4. Combine the L partials of each row through LDS.
    float *my = red + threadIdx.x * MT;
#pragma unroll
    for (int t = 0; t < MT; ++t) my[t] = acc[t];
    __syncthreads();
    if (active) {
        const float *base = red + (wave * kWaveSize + grp * L) * MT;
        for (uint32_t t = j; t < a.ntok && t < MT; t += L) {
            float s = 0.0f;
            for (uint32_t l = 0; l < L; ++l) s += base[l * MT + t];
            if (KIND != kF16) s *= a.scales ? a.scales[t] : a.scale;
            a.output[static_cast<size_t>(t) * a.output_stride + row] = s;
        }
    }
}

// Integer dump: one thread per (row, unit), token 0 only.  Same staging
// and per-unit cores as gemv_kernel; used by the bit-exactness tests.
//   HyperVSQ-2: out[row][unit*8 + oct] = sum (code-1)*a
//   Q4_0:       out[row][block]       = sum (nibble-8)*a
template <int KIND>
__global__ __launch_bounds__(kGemvThreads) void dump_kernel(GemvArgs a, int32_t *out,
                                                            uint32_t out_row) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t nblk = a.units * unit_elems(KIND) / 32;
    uint8_t *act = smem;
    int32_t *sums = reinterpret_cast<int32_t *>(smem + a.units * unit_lds_bytes(KIND));
    stage_int8<KIND, 1>(static_cast<const int8_t *>(a.input), a.input_stride, a.cols, a.units,
                        1, act, sums);
    __syncthreads();
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.rows * a.units) return;
    const uint32_t row = idx / a.units, u = idx % a.units;
    const uint4 *src = reinterpret_cast<const uint4 *>(a.payload + row * a.payload_row_bytes +
                                                       static_cast<size_t>(u) * 64);
    uint4 pay[4] = {src[0], src[1], src[2], src[3]};
    if (KIND == kHvsq2) {
        const uint32_t *cw = reinterpret_cast<const uint32_t *>(pay);
        for (int o = 0; o < 8; ++o) {
            const uint8_t *at = act + u * 272 + o * 32;
            const int v = hv_octant_dot(cw[2 * o], cw[2 * o + 1], *reinterpret_cast<const uint4 *>(at),
                                        *reinterpret_cast<const uint4 *>(at + 16)) -
                          sums[u * 8 + o];
            out[static_cast<size_t>(row) * out_row + u * 8 + o] = v;
        }
    } else {
        for (int b = 0; b < 4; ++b) {
            if (u * 4 + b >= out_row) break;
            const uint8_t *at = act + u * 144 + b * 32;
            out[static_cast<size_t>(row) * out_row + u * 4 + b] =
                q4_block_dot(pay[b], *reinterpret_cast<const uint4 *>(at),
                             *reinterpret_cast<const uint4 *>(at + 16)) -
                8 * sums[u * 4 + b];
        }
    }
    (void)nblk;
}

// ---- repack --------------------------------------------------------------

__global__ void repack_hvsq2(const uint8_t *__restrict__ src, uint8_t *codes, uint8_t *meta,
                             uint32_t rows, uint32_t nb, size_t codes_row, size_t meta_row) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<size_t>(rows) * nb) return;
    const uint32_t r = idx / nb, b = idx % nb;
    const uint8_t *blk = src + idx * 74;
    uint8_t *dc = codes + r * codes_row + static_cast<size_t>(b) * 64;
    for (int i = 0; i < 64; i += 4) {
        const uint32_t v = blk[10 + i] | (blk[11 + i] << 8) | (blk[12 + i] << 16) |
                           (static_cast<uint32_t>(blk[13 + i]) << 24);
        *reinterpret_cast<uint32_t *>(dc + i) = v;
    }
    const uint32_t m0 = blk[0] | (blk[1] << 8) | (blk[2] << 16) | (static_cast<uint32_t>(blk[3]) << 24);
    const uint32_t m1 = blk[4] | (blk[5] << 8) | (blk[6] << 16) | (static_cast<uint32_t>(blk[7]) << 24);
    *reinterpret_cast<uint2 *>(meta + r * meta_row + static_cast<size_t>(b) * 8) = make_uint2(m0, m1);
}

__global__ void repack_q4_0(const uint8_t *__restrict__ src, uint8_t *nibbles, uint8_t *scales,
                            uint32_t rows, uint32_t nb, size_t nib_row, size_t scale_row) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<size_t>(rows) * nb) return;
    const uint32_t r = idx / nb, b = idx % nb;
    const uint8_t *blk = src + idx * 18;
    uint8_t *dn = nibbles + r * nib_row + static_cast<size_t>(b) * 16;
    for (int i = 0; i < 16; i += 4) {
        const uint32_t v = blk[2 + i] | (blk[3 + i] << 8) | (blk[4 + i] << 16) |
                           (static_cast<uint32_t>(blk[5 + i]) << 24);
        *reinterpret_cast<uint32_t *>(dn + i) = v;
    }
    *reinterpret_cast<uint16_t *>(scales + r * scale_row + static_cast<size_t>(b) * 2) =
        static_cast<uint16_t>(blk[0] | (blk[1] << 8));
}

// ---- per-token quantization ---------------------------------------------

__global__ __launch_bounds__(256) void quantize_tokens_kernel(const float *__restrict__ x, int K,
                                                              int x_stride, int8_t *q8,
                                                              int out_stride, float *scales) {
    __shared__ float wave_max[256 / kWaveSize];
    const int t = blockIdx.x;
    const float *row = x + static_cast<size_t>(t) * x_stride;
    float amax = 0.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) amax = fmaxf(amax, fabsf(row[k]));
    for (int off = kWaveSize / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (threadIdx.x % kWaveSize == 0) wave_max[threadIdx.x / kWaveSize] = amax;
    __syncthreads();
    amax = wave_max[0];
    for (int w = 1; w < static_cast<int>(blockDim.x / kWaveSize); ++w) amax = fmaxf(amax, wave_max[w]);
    // IEEE division and reciprocal, as the CPU path (c/qwanto_kernels.c:385-386)
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) scales[t] = scale;
    int8_t *out = q8 + static_cast<size_t>(t) * out_stride;
    for (int k = threadIdx.x; k < out_stride; k += blockDim.x) {
        int8_t q = 0;
        if (k < K) {
            const float v = fminf(127.0f, fmaxf(-127.0f, row[k] * inv));
            q = static_cast<int8_t>(__builtin_rintf(v));
        }
        out[k] = q;
    }
}

template <int KIND, int MT, int UPL>
hipError_t launch_one(const GemvPlan &p, const GemvArgs &args, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_kernel<KIND, MT, UPL>), dim3(p.grid), dim3(kGemvThreads), p.lds_bytes,
                       stream, args);
    return hipGetLastError();
}

template <int KIND, int MT>
hipError_t dispatch_upl(const GemvPlan &p, const GemvArgs &args, hipStream_t stream) {
    switch (p.upl) {
    case 1: return launch_one<KIND, MT, 1>(p, args, stream);
    case 2: return launch_one<KIND, MT, 2>(p, args, stream);
    case 3: return launch_one<KIND, MT, 3>(p, args, stream);
    case 4: return launch_one<KIND, MT, 4>(p, args, stream);
    case 6: return launch_one<KIND, MT, 6>(p, args, stream);
    case 8: return launch_one<KIND, MT, 8>(p, args, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int KIND>
hipError_t dispatch_mt(const GemvPlan &p, const GemvArgs &args, hipStream_t stream) {
    switch (p.tokens) {
    case 1: return dispatch_upl<KIND, 1>(p, args, stream);
    case 2: return dispatch_upl<KIND, 2>(p, args, stream);
    case 4: return dispatch_upl<KIND, 4>(p, args, stream);
    case 8: return dispatch_upl<KIND, 8>(p, args, stream);
    case 16: return dispatch_upl<KIND, 16>(p, args, stream);
    default: return hipErrorInvalidValue;
    }
}

size_t lds_for(int kind, uint32_t units, int mt) {
    const size_t act = static_cast<size_t>(mt) * units * unit_lds_bytes(kind);
    const size_t sums = kind == kF16 ? 0 : static_cast<size_t>(mt) * units * unit_elems(kind) / 32 * 4;
    const size_t red = static_cast<size_t>(kGemvThreads) * mt * 4;
    return act + sums + red;
}

}  // namespace

GemvPlan plan_gemv(const DeviceTensor &t, int batch) {
    GemvPlan p;
    static const int kUpl[] = {1, 2, 3, 4, 6, 8};
    double best = -1.0;
    for (int upl : kUpl) {
        const int L = static_cast<int>((t.units + upl - 1) / upl);
        if (L > kWaveSize) continue;
        const int rpw = kWaveSize / L;
        // fraction of lane-unit slots doing real work
        const double eff = static_cast<double>(t.units) / (static_cast<double>(L) * upl) *
                           (static_cast<double>(rpw) * L) / kWaveSize;
        if (eff > best + 0.04) {
            best = eff;
            p.upl = upl;
            p.lanes = L;
            p.rows_per_wave = rpw;
        }
    }
    if (p.upl == 0) return p;  // too many units per row
    int mt = 1;
    const int want = std::min(batch, kMaxTokensPerLaunch);
    while (mt < want) mt *= 2;
    while (mt > 1 && lds_for(t.kind, t.units, mt) > kGemvLdsLimit) mt /= 2;
    p.tokens = mt;
    p.lds_bytes = lds_for(t.kind, t.units, mt);
    const int rows_per_wg = p.rows_per_wave * kGemvWaves;
    p.grid = static_cast<int>((t.rows + rows_per_wg - 1) / rows_per_wg);
    return p;
}

hipError_t repack_tensor(const DeviceTensor &t, const uint8_t *staging, hipStream_t stream) {
    if (t.kind == kHvsq2) {
        const uint32_t nb = t.units;
        const size_t n = static_cast<size_t>(t.rows) * nb;
        hipLaunchKernelGGL(repack_hvsq2, dim3((n + 255) / 256), dim3(256), 0, stream, staging,
                           t.payload, t.meta, t.rows, nb, t.payload_row_bytes, t.meta_row_bytes);
        return hipGetLastError();
    }
    if (t.kind == kQ4_0) {
        const uint32_t nb = (t.cols + 31) / 32;
        const size_t n = static_cast<size_t>(t.rows) * nb;
        hipError_t e = hipMemsetAsync(t.payload, 0, t.payload_row_bytes * t.rows, stream);
        if (e == hipSuccess) e = hipMemsetAsync(t.meta, 0, t.meta_row_bytes * t.rows, stream);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(repack_q4_0, dim3((n + 255) / 256), dim3(256), 0, stream, staging,
                           t.payload, t.meta, t.rows, nb, t.payload_row_bytes, t.meta_row_bytes);
        return hipGetLastError();
    }
    if (t.kind == kF16) {
        hipError_t e = hipMemsetAsync(t.payload, 0, t.payload_row_bytes * t.rows, stream);
        if (e != hipSuccess) return e;
        return hipMemcpy2DAsync(t.payload, t.payload_row_bytes, staging,
                                static_cast<size_t>(t.cols) * 2, static_cast<size_t>(t.cols) * 2,
                                t.rows, hipMemcpyDeviceToDevice, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(const GemvLaunch &g, hipStream_t stream) {
    const DeviceTensor &t = *g.tensor;
    GemvArgs args{};
    args.payload = t.payload;
    args.meta = t.meta;
    args.payload_row_bytes = t.payload_row_bytes;
    args.meta_row_bytes = t.meta_row_bytes;
    args.rows = t.rows;
    args.cols = t.cols;
    args.units = t.units;
    args.input_stride = g.input_stride;
    args.output_stride = g.output_stride;

    if (g.debug_sums) {
        if (t.kind == kF16) return hipErrorInvalidValue;
        args.input = g.input;
        const size_t lds = static_cast<size_t>(t.units) * unit_lds_bytes(t.kind) +
                           static_cast<size_t>(t.units) * unit_elems(t.kind) / 32 * 4;
        if (lds > kGemvLdsLimit) return hipErrorInvalidValue;
        const size_t n = static_cast<size_t>(t.rows) * t.units;
        const uint32_t out_row = t.kind == kHvsq2 ? t.units * 8 : (t.cols + 31) / 32;
        if (t.kind == kHvsq2)
            hipLaunchKernelGGL(dump_kernel<kHvsq2>, dim3((n + kGemvThreads - 1) / kGemvThreads),
                               dim3(kGemvThreads), lds, stream, args, g.debug_sums, out_row);
        else
            hipLaunchKernelGGL(dump_kernel<kQ4_0>, dim3((n + kGemvThreads - 1) / kGemvThreads),
                               dim3(kGemvThreads), lds, stream, args, g.debug_sums, out_row);
        return hipGetLastError();
    }

    const GemvPlan p = plan_gemv(t, static_cast<int>(g.batch));
    if (p.upl == 0 || p.tokens == 0 || p.lds_bytes > kGemvLdsLimit) return hipErrorInvalidValue;
    args.lanes = p.lanes;
    args.rows_per_wave = p.rows_per_wave;
    const size_t elem = t.kind == kF16 ? 4 : 1;
    for (uint32_t t0 = 0; t0 < g.batch; t0 += p.tokens) {
        args.ntok = std::min<uint32_t>(p.tokens, g.batch - t0);
        args.input = static_cast<const uint8_t *>(g.input) + static_cast<size_t>(t0) * g.input_stride * elem;
        args.scales = g.scales ? g.scales + t0 : nullptr;
        args.scale = g.scale;
        args.output = g.output + static_cast<size_t>(t0) * g.output_stride;
        hipError_t e;
        if (t.kind == kHvsq2) e = dispatch_mt<kHvsq2>(p, args, stream);
        else if (t.kind == kQ4_0) e = dispatch_mt<kQ4_0>(p, args, stream);
        else e = dispatch_mt<kF16>(p, args, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_quantize_tokens(const float *x, int M, int K, int x_stride, int8_t *q8,
                                  int out_stride, float *scales, hipStream_t stream) {
    hipLaunchKernelGGL(quantize_tokens_kernel, dim3(M), dim3(256), 0, stream, x, K, x_stride, q8,
                       out_stride, scales);
    return hipGetLastError();
}

}  // namespace qwn
