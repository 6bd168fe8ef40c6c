// Quantized GEMV / small-batch GEMM kernels for gfx950 (CDNA4).
//
// Decode at batch 1 reads every weight exactly once, so the kernel is an
// HBM stream.  Each wave owns a tile of rows stored contiguously in the
// order its lanes load it (qwn_internal.h), so every 128-bit load
// instruction of the wave reads one contiguous span.
//
// Activations arrive as an "activation image": the exact LDS byte layout
// the dot products read (below), built once per token by a producer kernel
// (from int8, from fp32, or fused with the int8 quantization).  A workgroup
// copies the image into LDS with direct global->LDS loads issued before its
// weight loads, waits only for those, and reduces each row's lane partials
// with DPP adds.
//
// Integer core.  An int8 activation is written a = 16*h + l with h = a >> 4
// in [-8, 7] (signed nibble) and l = a & 15 in [0, 15] (unsigned nibble), so
//   sum c*a = 16 * sdot8(c, h) + udot8(c, l)          (v_dot8_i32_i4 / v_dot8_u32_u4)
// exactly, for any 4-bit weight field c.
//   HyperVSQ-2: a code dword holds weights 4j+i at bits 8j+2i; masking with
//     0x33333333 leaves weights {0,2,..,14} in nibbles 0..7 and
//     (w >> 2) & 0x33333333 the odd ones, so two masks feed four dot8s
//     (16 weights).  sum (c-1)*a = that - sum a.
//   Q4_0: the nibble dword already holds weights 0..7 in nibbles 0..7;
//     (n - 8) is n ^ 8 as a signed nibble, and
//     sum (n-8)*a = 16*sdot8(n^0x88888888, h) + udot8(n, l) - 8*sum l.
//
// Image layout per token (padded to 16 bytes):
//   HyperVSQ-2: per unit 16 groups x {h even, l even, h odd, l odd} nibble
//               words (256 B) + 16 B pad; then sum a per 32 activations
//   Q4_0:       per unit 16 groups x {h, l} nibble words (128 B) + 16 B pad;
//               then 8 * sum l per 32 activations
//   F16:        per unit 32 floats (128 B) + 16 B pad
//
// Semantics follow the reference CPU kernels:
//   HyperVSQ-2  y = xs * sum_blocks (d/8 * sum_oct s_oct*(sum code*a - sum a)
//                                    + m * sum a)        c/qwanto_kernels.c:619-667
//   Q4_0        y = xs * sum_blocks d * (sum nibble*a - 8 * sum a)
//                                                         c/qwanto_kernels.c:503-534,1178-1322
//   F16         y = sum_k x[k] * w[k]                    c/qwanto_kernels.c:1531-1616
// The integer parts are exact; only the fp32 combination order differs
// from the CPU's.
#include "qwn_device.h"
#include "qwn_internal.h"

#include <algorithm>
#include <type_traits>

namespace qwn {

size_t image_act_bytes(int kind, uint32_t units) {
    return static_cast<size_t>(units) * unit_lds_bytes(kind);
}

size_t image_bytes(int kind, uint32_t units) {
    const size_t sums = kind == kF16 ? 0 : static_cast<size_t>(units) * unit_elems(kind) / 32 * 4;
    return (image_act_bytes(kind, units) + sums + 15) & ~static_cast<size_t>(15);
}

namespace {

constexpr uint32_t kMask33 = 0x33333333u;
constexpr uint32_t kFlip8 = 0x88888888u;


__device__ __forceinline__ int sdot8(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot8(static_cast<int>(a), static_cast<int>(b), c, false);
}
__device__ __forceinline__ int udot8(uint32_t a, uint32_t b, int c) {
    return static_cast<int>(__builtin_amdgcn_udot8(a, b, static_cast<uint32_t>(c), false));
}

// int8 tokens [M][stride] (K valid, zero padded) -> images.  grid (blocks, M).
template <int KIND>
__global__ __launch_bounds__(256) void image_from_int8_kernel(const int8_t *__restrict__ x, uint32_t stride,
                                                              uint32_t K, uint32_t units, uint8_t *image,
                                                              uint32_t image_stride) {
    const uint32_t nblk = units * unit_elems(KIND) / 32;
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t t = blockIdx.y;
    if (b >= nblk) return;
    const uint32_t e0 = b * 32;
    uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int8_t *src = x + static_cast<size_t>(t) * stride + e0;
    if (e0 + 32 <= K && (reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
        const uint4 v0 = *reinterpret_cast<const uint4 *>(src);
        const uint4 v1 = *reinterpret_cast<const uint4 *>(src + 16);
        w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
        w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
    } else {
        for (uint32_t i = 0; i < 32 && e0 + i < K; ++i)
            w[i >> 2] |= (static_cast<uint32_t>(static_cast<uint8_t>(src[i]))) << (8 * (i & 3));
    }
    put_block32<KIND>(image + static_cast<size_t>(t) * image_stride, units, b, w);
}

// fp32 tokens [M][stride] (K valid) -> F16 images.  grid (groups of 8, M).
__global__ __launch_bounds__(256) void image_from_f32_kernel(const float *__restrict__ x, uint32_t stride,
                                                             uint32_t K, uint32_t units, uint8_t *image,
                                                             uint32_t image_stride) {
    const uint32_t gi = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t t = blockIdx.y;
    if (gi >= units * 4) return;
    const uint32_t e0 = gi * 8;
    float v[8];
    const float *src = x + static_cast<size_t>(t) * stride + e0;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = e0 + i < K ? src[i] : 0.0f;
    float4 *dst = reinterpret_cast<float4 *>(image + static_cast<size_t>(t) * image_stride + (gi / 4) * 144 +
                                             (gi % 4) * 32);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// RMSNorm of a token into an F16 tensor's fp32 image (the tied LM head
// input): y = (x * 1/sqrt(mean(x^2) + eps)) * w (c/qwanto_decode.c:627-652).
// One workgroup of 1024 threads per token: token blockIdx.x reads
// x + blockIdx.x * x_stride and writes image + blockIdx.x * image_stride.
__global__ __launch_bounds__(1024) void norm_image_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                          uint32_t K, uint32_t units, float eps, uint8_t *image,
                                                          uint32_t x_stride, uint32_t image_stride) {
    __shared__ float red[1024 / kWaveSize];
    x += static_cast<size_t>(blockIdx.x) * x_stride;
    image += static_cast<size_t>(blockIdx.x) * image_stride;
    float ss = 0.0f;
    for (uint32_t k = threadIdx.x; k < K; k += blockDim.x) ss = fmaf(x[k], x[k], ss);
    ss = wave_sum_all(ss);
    if (threadIdx.x % kWaveSize == 0) red[threadIdx.x / kWaveSize] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (uint32_t i = 0; i < blockDim.x / kWaveSize; ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
    for (uint32_t k = threadIdx.x; k < units * 32; k += blockDim.x) {
        const float v = k < K ? (x[k] * inv) * w[k] : 0.0f;
        *reinterpret_cast<float *>(image + (k / 32) * 144 + (k % 32) * 4) = v;
    }
}

// Elements per image sub-block written by one lane (a quarter or half of a
// 32-block: the per-32 sums are combined across adjacent lanes).
__host__ __device__ constexpr int fused_sub_elems(int kind) { return kind == kHvsq2 ? 16 : 8; }

// Per-token int8 quantization (c/qwanto_kernels.c:354-433) fused with the
// image: x fp32 [M][x_stride] -> scales [M], image [M][image_stride] and,
// when q8 is given, the int8 token [M][q8_stride] zero padded.  grid (M),
// one workgroup per token.  The quantized value is the input (kInF32), its
// RMSNorm with weights `norm` (kInNorm, c/qwanto_decode.c:627-652) or
// silu(x) * x2 (kInSwiglu, c/qwanto_decode.c:1946-1949): the arithmetic of
// the fused one-token GEMV prologue for a block of tokens.  The values are
// staged in LDS (dynamic, K floats) with coalesced loads where they fit
// (`staged`), else recomputed from global memory; the image is written in
// E-element sub-blocks by adjacent lanes, as the prologue does.  With
// `mimg`, token t's columns of the int8-MFMA image of up to 16 tokens are
// written instead of q8 (one sub-block is one 8- or 16-byte slot of that
// image; HyperVSQ-2's block sums are reduced over the adjacent lanes
// holding the block); tokens >= M of the image are left as they are (the GEMM neither
// mixes token columns nor stores those tokens).  NT threads per token;
// EPT > 0 (K <= NT EPT, the row staged): thread t loads elements t + NT e of
// the input (and of the norm weights or the SwiGLU up half) into registers
// in one batch of loads before anything waits, and the two reductions meet
// at LDS-only barriers.  EPT = 0 (NT 1024): a strided loop that re-reads the
// row from global memory.
template <int KIND, int EPT, int NT>
__global__ __launch_bounds__(NT) void quantize_image_kernel(const float *__restrict__ x, uint32_t K,
                                                              uint32_t x_stride, uint32_t units, uint8_t *image,
                                                              uint32_t image_stride, float *scales, int8_t *q8,
                                                              uint32_t q8_stride, uint32_t mode,
                                                              const float *__restrict__ x2,
                                                              const float *__restrict__ norm, float eps,
                                                              uint32_t staged, uint8_t *mimg, size_t mimg_group) {
    extern __shared__ float vals[];  // [K] when staged
    __shared__ float wave_red[2][1024 / kWaveSize];
    constexpr uint32_t E = fused_sub_elems(KIND);
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t W = blockDim.x / kWaveSize;
    const float *row = x + static_cast<size_t>(t) * x_stride;
    // the MFMA image of the token's 16-token group, its column tc there
    const uint32_t tc = t % 16;
    if (mimg) mimg += (t / 16) * mimg_group;
    float inv_rms = 1.0f;
    auto value = [&](uint32_t k) {
        const float v = row[k];
        if (mode == kInNorm) return (v * inv_rms) * norm[k];
        if (mode == kInSwiglu) return (v / (1.0f + expf(-v))) * x2[static_cast<size_t>(t) * x_stride + k];
        return v;
    };
    float amax = 0.0f;
    if constexpr (EPT > 0) {
        const float *ysrc = mode == kInNorm ? norm : mode == kInSwiglu ? x2 + static_cast<size_t>(t) * x_stride : row;
        float xv[EPT], yv[EPT];
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const uint32_t k = tid + static_cast<uint32_t>(NT) * e, kk = k < K ? k : 0u;
            xv[e] = row[kk];
            yv[e] = ysrc[kk];
        }
        if (mode == kInNorm) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < EPT; ++e)
                if (tid + static_cast<uint32_t>(NT) * e < K) ss = fmaf(xv[e], xv[e], ss);
            ss = wave_sum_all(ss);
            if (tid % kWaveSize == 0) wave_red[0][tid / kWaveSize] = ss;
            lds_barrier();
            float tot = wave_red[0][0];
            for (uint32_t w = 1; w < W; ++w) tot += wave_red[0][w];
            inv_rms = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
        }
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const uint32_t k = tid + static_cast<uint32_t>(NT) * e;
            if (k < K) {
                const float xe = xv[e];
                const float v = mode == kInNorm     ? (xe * inv_rms) * yv[e]
                                : mode == kInSwiglu ? (xe / (1.0f + expf(-xe))) * yv[e]
                                                    : xe;
                vals[k] = v;
                amax = fmaxf(amax, fabsf(v));
            }
        }
        amax = wave_max_all(amax);
        if (tid % kWaveSize == 0) wave_red[1][tid / kWaveSize] = amax;
        lds_barrier();
        amax = wave_red[1][0];
        for (uint32_t w = 1; w < W; ++w) amax = fmaxf(amax, wave_red[1][w]);
    } else {
        if (mode == kInNorm) {
            float ss = 0.0f;
            for (uint32_t k = tid; k < K; k += blockDim.x) ss = fmaf(row[k], row[k], ss);
            ss = wave_sum_all(ss);
            if (tid % kWaveSize == 0) wave_red[0][tid / kWaveSize] = ss;
            __syncthreads();
            float tot = wave_red[0][0];
            for (uint32_t w = 1; w < W; ++w) tot += wave_red[0][w];
            inv_rms = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
        }
        for (uint32_t k = tid; k < K; k += blockDim.x) {
            const float v = value(k);
            if (staged) vals[k] = v;
            amax = fmaxf(amax, fabsf(v));
        }
        amax = wave_max_all(amax);
        if (tid % kWaveSize == 0) wave_red[1][tid / kWaveSize] = amax;
        __syncthreads();
        amax = wave_red[1][0];
        for (uint32_t w = 1; w < W; ++w) amax = fmaxf(amax, wave_red[1][w]);
    }
    // IEEE division and reciprocal, as the CPU path (c/qwanto_kernels.c:385-386)
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    if (tid == 0) scales[t] = scale;
    const uint32_t nsub = units * unit_elems(KIND) / E;
    uint8_t *img = image ? image + static_cast<size_t>(t) * image_stride : nullptr;
    int8_t *q8row = q8 ? q8 + static_cast<size_t>(t) * q8_stride : nullptr;
    // every lane runs the sub-block step (its cross-lane sums), those past
    // the image write nothing
    for (uint32_t base = 0; base < nsub; base += blockDim.x) {
        const uint32_t sb = base + tid;
        uint32_t w[E / 4];
        uint32_t qb[E];
#pragma unroll
        for (uint32_t i = 0; i < E; ++i) {
            const uint32_t k = sb * E + i;
            qb[i] = 0;
            if (sb < nsub && k < K) {
                const float c = fminf(127.0f, fmaxf(-127.0f, (staged ? vals[k] : value(k)) * inv));
                qb[i] = q8_low_byte(c);
            }
        }
#pragma unroll
        for (uint32_t i = 0; i < E / 4; ++i) w[i] = pack_low_bytes(qb[4 * i], qb[4 * i + 1], qb[4 * i + 2], qb[4 * i + 3]);
        if (img) put_sub_block<KIND>(img, units, sb, nsub, w);
        if (mimg) {
            if constexpr (KIND == kQ4_0) {
                // slot (block sb/4, group sb%4): elements {0,2,4,6} then {1,3,5,7}
                const uint32_t nblk = (K + 31) / 32;
                if (sb < nblk * 4) {
                    // bytes 0, 2 / 1, 3 of each word (v_perm_b32: bytes 0-3 of
                    // the second operand, 4-7 of the first)
                    const uint32_t lo = __builtin_amdgcn_perm(w[1], w[0], 0x06040200u);
                    const uint32_t hi = __builtin_amdgcn_perm(w[1], w[0], 0x07050301u);
                    *reinterpret_cast<uint2 *>(mimg + (static_cast<size_t>(sb) * 16 + tc) * 8) = make_uint2(lo, hi);
                }
            } else {
                // elements 16 sb .. 16 sb + 15 are slice sl = sb % 4 of group
                // g = (sb / 4) % 4 of block sb / 16, image slot
                // (block * 16 + sl * 4 + g); word k = byte k of w[0..3]
                int s = 0;
#pragma unroll
                for (uint32_t i = 0; i < E; ++i) s += static_cast<int8_t>((w[i >> 2] >> (8 * (i & 3))) & 0xffu);
                // the 16 lanes' sum into the first lane of each 16-lane row
                // (DPP row shifts toward lane 0; lanes past the row add 0)
                s += __builtin_amdgcn_update_dpp(0, s, 0x101, 0xf, 0xf, false);
                s += __builtin_amdgcn_update_dpp(0, s, 0x102, 0xf, 0xf, false);
                s += __builtin_amdgcn_update_dpp(0, s, 0x104, 0xf, 0xf, false);
                s += __builtin_amdgcn_update_dpp(0, s, 0x108, 0xf, 0xf, false);
                if (sb < nsub) {
                    // byte k of w[0..3] -> word k: a 4x4 byte transpose in
                    // two rounds of byte permutes
                    const uint32_t p01l = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);
                    const uint32_t p01h = __builtin_amdgcn_perm(w[1], w[0], 0x07030602u);
                    const uint32_t p23l = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
                    const uint32_t p23h = __builtin_amdgcn_perm(w[3], w[2], 0x07030602u);
                    const uint32_t o[4] = {__builtin_amdgcn_perm(p23l, p01l, 0x05040100u),
                                           __builtin_amdgcn_perm(p23l, p01l, 0x07060302u),
                                           __builtin_amdgcn_perm(p23h, p01h, 0x05040100u),
                                           __builtin_amdgcn_perm(p23h, p01h, 0x07060302u)};
                    const uint32_t slot = (sb & ~15u) | ((sb & 3u) << 2) | ((sb >> 2) & 3u);
                    *reinterpret_cast<uint4 *>(mimg + (static_cast<size_t>(slot) * 16 + tc) * 16) =
                        make_uint4(o[0], o[1], o[2], o[3]);
                    if ((sb & 15u) == 0)
                        reinterpret_cast<float *>(mimg + static_cast<size_t>(units) * 4096)[(sb >> 4) * 16 + tc] =
                            static_cast<float>(s);
                }
            }
        }
        if (q8row && sb < nsub)
#pragma unroll
            for (uint32_t i = 0; i < E; ++i)
                if (sb * E + i < q8_stride) q8row[sb * E + i] = static_cast<int8_t>((w[i >> 2] >> (8 * (i & 3))) & 0xffu);
    }
    if (q8row)
        for (uint32_t k = nsub * E + tid; k < q8_stride; k += blockDim.x) q8row[k] = 0;
}

// Copy `ntok` token images (global stride `stride`, `bytes` each, a
// multiple of 16) into LDS back to back, one 16-byte direct load per lane;
// returns after issuing (the caller waits).
template <int MT>
__device__ __forceinline__ void issue_image_copy(const uint8_t *__restrict__ image, uint32_t stride,
                                                 uint32_t bytes, uint32_t ntok, uint8_t *lds) {
    const uint32_t per_tok = bytes / 16;
    const uint32_t total = MT == 1 ? per_tok : per_tok * ntok;
    const uint32_t lane = threadIdx.x % kWaveSize;
    for (uint32_t c0 = (threadIdx.x / kWaveSize) * kWaveSize; c0 < total; c0 += blockDim.x) {
        const uint32_t c = c0 + lane;
        if (c < total) {
            const uint32_t t = MT == 1 ? 0 : c / per_tok, r = c - t * per_tok;
            __builtin_amdgcn_global_load_lds(image + static_cast<size_t>(t) * stride + r * 16,
                                             (lds_void *)(lds + c0 * 16), 16, 0, 0);
        }
    }
}


// ---- per-unit integer cores (shared by the GEMV and the dump kernel) ----

// sum over one octant of code*a: w0/w1 = the octant's code dwords, a0/a1 =
// the image words of its two 16-element groups.
__device__ __forceinline__ int hv_octant_dot(uint32_t w0, uint32_t w1, uint4 a0, uint4 a1) {
    const uint32_t e0 = w0 & kMask33, o0 = (w0 >> 2) & kMask33;
    const uint32_t e1 = w1 & kMask33, o1 = (w1 >> 2) & kMask33;
    int hi = sdot8(e0, a0.x, 0);
    hi = sdot8(o0, a0.z, hi);
    hi = sdot8(e1, a1.x, hi);
    hi = sdot8(o1, a1.z, hi);
    int lo = udot8(e0, a0.y, 0);
    lo = udot8(o0, a0.w, lo);
    lo = udot8(e1, a1.y, lo);
    lo = udot8(o1, a1.w, lo);
    return hi * 16 + lo;
}

// sum over one Q4_0 block of (nibble-8)*a + 8*sum l, i.e. before the
// image's correction; a0 = (h,l) of nibble dwords 0,1, a1 = of dwords 2,3.
__device__ __forceinline__ int q4_block_dot(uint4 n, uint4 a0, uint4 a1) {
    int hi = sdot8(n.x ^ kFlip8, a0.x, 0);
    hi = sdot8(n.y ^ kFlip8, a0.z, hi);
    hi = sdot8(n.z ^ kFlip8, a1.x, hi);
    hi = sdot8(n.w ^ kFlip8, a1.z, hi);
    int lo = udot8(n.x, a0.y, 0);
    lo = udot8(n.y, a0.w, lo);
    lo = udot8(n.z, a1.y, lo);
    lo = udot8(n.w, a1.w, lo);
    return hi * 16 + lo;
}

struct GemvArgs {
    // jobs (tensors sharing the input); job i owns workgroups
    // [job_block[i], job_block[i+1]), job_block[njobs] = grid
    const uint8_t *payload[kMaxGroup];
    const uint8_t *meta[kMaxGroup];
    float *output[kMaxGroup];
    uint32_t rows[kMaxGroup];
    uint32_t job_block[kMaxGroup + 1];
    uint32_t njobs;
    // lane plan shared by the jobs
    size_t tile_payload_bytes;
    size_t tile_meta_bytes;
    uint32_t units;
    uint32_t lanes;
    uint32_t lanes_log2;
    uint32_t rows_per_wave;
    uint32_t input_mode;
    uint32_t output_mode;
    // image input
    const uint8_t *image;
    const float *scales;
    float scale;
    uint32_t ntok;
    uint32_t image_stride;
    uint32_t image_bytes;
    // fp32 input
    const float *x;
    const float *x2;
    const float *norm;
    float eps;
    uint32_t cols;
    float *scale_out;
    // output
    uint32_t output_stride[kMaxGroup];  // elements between tokens, per job
    uint64_t *argmax_partials;
    const float *bias[kMaxGroup];       // per job: null, or [rows] added to the product
    uint32_t bf16;                      // kF16 layout holding bfloat16 weights
};

// Separately rounded product and sum (never contracted into an fma).
__device__ __forceinline__ float mul_rounded(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_rounded(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}

// Workgroup reductions for the fused prologue: every thread gets the same
// result, combined in wave order (identical in every workgroup).
__device__ __forceinline__ float wg_sum(float v, float *red, uint32_t waves) {
    v = wave_sum_all(v);
    if (threadIdx.x % kWaveSize == 0) red[threadIdx.x / kWaveSize] = v;
    lds_barrier();
    float s = red[0];
    for (uint32_t w = 1; w < waves; ++w) s += red[w];
    return s;
}
__device__ __forceinline__ float wg_max(float v, float *red, uint32_t waves) {
    v = wave_max_all(v);
    if (threadIdx.x % kWaveSize == 0) red[threadIdx.x / kWaveSize] = v;
    lds_barrier();
    float s = red[0];
    for (uint32_t w = 1; w < waves; ++w) s = fmaxf(s, red[w]);
    return s;
}

// Argmax key: larger value wins, then the smaller row (the CPU's
// first-maximum rule, c/qwanto_decode.c:2048-2065); NaN never wins.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t row) {
    if (v != v) return 0;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<uint64_t>(ord) << 32) | (0xffffffffu - row);
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int off) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), off);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), off);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// FR (fused, one token only): the input is an fp32 vector turned into the
// LDS image by every workgroup, in sub-blocks of E elements (16 for
// HyperVSQ-2, 8 otherwise), FR (1 .. 32/E) sub-blocks per thread: the fewer,
// the shorter each thread's chain.  FR 0: prebuilt images are copied to LDS.
// Workgroups of up to kGemvMaxWaves waves where a lane's registers allow it
// (UPL <= 4), else kGemvWaves.
__host__ __device__ constexpr int max_waves_for(int upl) { return upl <= 4 ? kGemvMaxWaves : kGemvWaves; }


// PAIRED_TILES: the tensor is stored one unit per lane (lanes >= 2) and the
// launch runs it two units per lane: a wave takes two adjacent tiles, half
// the lanes per row (lane j of a row holds its units j and j + L/2) and
// twice the rows, so each workgroup's prologue serves as many rows as on a
// two-units-per-lane layout.  Fused one-token launches whose one-tile grid
// would hold more workgroups than the chip has CUs use it.
template <int KIND, int MT, int UPL, int FR, bool PAIRED_TILES = false>
__global__ __launch_bounds__(kWaveSize * max_waves_for(UPL)) void gemv_kernel(GemvArgs a) {
    constexpr bool FUSED = FR != 0;
    static_assert(!PAIRED_TILES || (UPL == 2 && MT == 1), "paired tiles: two units per lane, one token");
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[2][kGemvMaxWaves];
    __shared__ uint64_t red_key[kGemvMaxWaves];
    __shared__ float up_s[kGemvMaxWaves / 2 * kWaveSize];
    constexpr int CH = 4;
    // Wave-uniform values are kept in scalar registers (readfirstlane): a
    // per-lane job index would turn the pointer selection below into vector
    // loads of the kernel arguments and a full memory round trip ahead of the
    // weight stream.
    const uint32_t W = blockDim.x / kWaveSize;
    const uint32_t lane = threadIdx.x % kWaveSize;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
    const uint32_t L = PAIRED_TILES ? a.lanes >> 1 : a.lanes;  // lanes per row of this launch
    const uint32_t grp = lane >> (PAIRED_TILES ? a.lanes_log2 - 1 : a.lanes_log2);
    const uint32_t j = lane & (L - 1);

    // Job of this workgroup.  Every job field is read unconditionally and
    // chosen by selects, so all kernel-argument loads issue in one batch
    // (a field loaded only once the job is known would add a dependent
    // scalar round trip ahead of the weight stream).  Paired jobs (SwiGLU):
    // the first half of the waves takes a tile of job 0, the second half the
    // same tile of job 1.
    // Pin the argument fields the prologue needs: one batch of scalar loads
    // and a single wait, instead of loads issued one by one at first use.
    {
        const uint64_t p0 = reinterpret_cast<uint64_t>(a.payload[0]), p1 = reinterpret_cast<uint64_t>(a.payload[1]);
        const uint64_t p2 = reinterpret_cast<uint64_t>(a.payload[2]), p3 = reinterpret_cast<uint64_t>(a.payload[3]);
        const uint64_t m0 = reinterpret_cast<uint64_t>(a.meta[0]), m1 = reinterpret_cast<uint64_t>(a.meta[1]);
        const uint64_t m2 = reinterpret_cast<uint64_t>(a.meta[2]), m3 = reinterpret_cast<uint64_t>(a.meta[3]);
        const uint64_t img = reinterpret_cast<uint64_t>(FUSED ? static_cast<const void *>(a.x)
                                                              : static_cast<const void *>(a.image));
        if constexpr (FUSED) {
            const uint64_t x2 = reinterpret_cast<uint64_t>(a.x2), nrm = reinterpret_cast<uint64_t>(a.norm);
            asm volatile("" ::"s"(p0), "s"(p1), "s"(p2), "s"(p3), "s"(m0), "s"(m1), "s"(m2), "s"(m3), "s"(img),
                         "s"(a.job_block[1]), "s"(a.job_block[2]), "s"(a.job_block[3]), "s"(a.rows[0]),
                         "s"(a.tile_payload_bytes), "s"(a.tile_meta_bytes), "s"(a.units), "s"(a.lanes_log2),
                         "s"(a.rows_per_wave), "s"(a.output_mode), "s"(W), "s"(x2), "s"(nrm), "s"(a.cols),
                         "s"(a.input_mode), "s"(a.eps));
        } else {
            asm volatile("" ::"s"(p0), "s"(p1), "s"(p2), "s"(p3), "s"(m0), "s"(m1), "s"(m2), "s"(m3), "s"(img),
                         "s"(a.job_block[1]), "s"(a.job_block[2]), "s"(a.job_block[3]), "s"(a.rows[0]),
                         "s"(a.tile_payload_bytes), "s"(a.tile_meta_bytes), "s"(a.units), "s"(a.lanes_log2),
                         "s"(a.rows_per_wave), "s"(a.output_mode), "s"(a.image_bytes), "s"(W));
        }
    }
    const bool paired = MT == 1 && a.output_mode == kOutSwiglu;
    const uint32_t half_w = W / 2;
    const uint32_t b1 = a.job_block[1], b2 = a.job_block[2], b3 = a.job_block[3];
    uint32_t job = (blockIdx.x >= b1 ? 1u : 0u) + (blockIdx.x >= b2 ? 1u : 0u) + (blockIdx.x >= b3 ? 1u : 0u);
    if (paired) job = wave >= half_w ? 1u : 0u;
    job = __builtin_amdgcn_readfirstlane(job);
    const uint8_t *payload = job == 0 ? a.payload[0] : job == 1 ? a.payload[1] : job == 2 ? a.payload[2] : a.payload[3];
    const uint8_t *meta = job == 0 ? a.meta[0] : job == 1 ? a.meta[1] : job == 2 ? a.meta[2] : a.meta[3];
    float *output = job == 0 ? a.output[0] : job == 1 ? a.output[1] : job == 2 ? a.output[2] : a.output[3];
    const uint32_t rows = job == 0 ? a.rows[0] : job == 1 ? a.rows[1] : job == 2 ? a.rows[2] : a.rows[3];
    const uint32_t out_stride = job == 0   ? a.output_stride[0]
                                : job == 1 ? a.output_stride[1]
                                : job == 2 ? a.output_stride[2]
                                           : a.output_stride[3];
    const uint32_t first = paired ? 0u : (job == 0 ? 0u : job == 1 ? b1 : job == 2 ? b2 : b3);
    const uint32_t tile = (PAIRED_TILES ? 2 : 1) *
                          (paired ? blockIdx.x * half_w + wave % half_w : (blockIdx.x - first) * W + wave);
    const uint32_t row = tile * a.rows_per_wave + grp;
    const bool active = grp < (PAIRED_TILES ? 2 : 1) * a.rows_per_wave && row < rows;
    const bool writer = active && j == L - 1;
    constexpr bool fused = FUSED && MT == 1;

    // 0. The input: image -> LDS by direct loads, or the fp32 vector(s) into
    //    registers: thread t takes the E-element sub-blocks t, t + blockDim,
    //    ... (the 32/E sub-blocks of a 32-block sit in adjacent lanes).
    constexpr int E = fused_sub_elems(KIND);
    constexpr int SR = FR > 0 ? FR : 1;                      // sub-blocks per thread
    constexpr int EW = E / 4;                                // float4 / int8 words per sub-block
    const uint32_t nblk = a.units * unit_elems(KIND) / 32;  // 32-blocks in the image
    const uint32_t nsub = nblk * (32 / E);                   // sub-blocks in the image
    const uint32_t nvalid = a.cols / E;                      // sub-blocks holding input values
    float4 xv[SR][EW], x2v[SR][EW];
    if constexpr (fused) {
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const uint32_t sb = threadIdx.x + r * blockDim.x;
            const float4 *src = reinterpret_cast<const float4 *>(a.x + (sb < nvalid ? sb * E : 0));
#pragma unroll
            for (int i = 0; i < EW; ++i) xv[r][i] = src[i];
        }
        if (a.input_mode != kInF32) {
            const float *p2 = a.input_mode == kInNorm ? a.norm : a.x2;
#pragma unroll
            for (int r = 0; r < SR; ++r) {
                const uint32_t sb = threadIdx.x + r * blockDim.x;
                const float4 *src2 = reinterpret_cast<const float4 *>(p2 + (sb < nvalid ? sb * E : 0));
#pragma unroll
                for (int i = 0; i < EW; ++i) x2v[r][i] = src2[i];
            }
        }
    } else {
        issue_image_copy<MT>(a.image, a.image_stride, a.image_bytes, a.ntok, smem);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 1. Every weight load of this lane, metadata before codes.  Lanes
    //    without a unit load from the tile start instead of branching, so
    //    the loads stay one unconditional burst.
    const size_t R = a.rows_per_wave;
    uint2 met[UPL];
    uint4 pay[UPL][CH];
    if constexpr (PAIRED_TILES) {
        // row grp of the pair: tile tile + grp / R, row grp % R; the tile's
        // one slot holds all n = units units of a row
        const uint32_t n = a.units, g = grp & (a.rows_per_wave - 1);
        const bool second = grp >= a.rows_per_wave;
        const uint8_t *tile_p = payload + tile * a.tile_payload_bytes + (second ? a.tile_payload_bytes : 0);
        const uint8_t *tile_m = meta + tile * a.tile_meta_bytes + (second ? a.tile_meta_bytes : 0);
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const uint32_t u = j + i * L;
            met[i] = *reinterpret_cast<const uint2 *>(active && u < n ? tile_m + (g * n + u) * 8 : tile_m);
        }
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const uint32_t u = j + i * L;
            const uint8_t *base = tile_p + (g * n + u) * 16;
#pragma unroll
            for (int q = 0; q < CH; ++q)
                pay[i][q] = *reinterpret_cast<const uint4 *>(active && u < n ? base + q * R * n * 16 : tile_p);
        }
    } else {
        const uint8_t *tile_p = payload + tile * a.tile_payload_bytes;
        const uint8_t *tile_m = meta + tile * a.tile_meta_bytes;
        // Unit slot i holds units i*L + j, n = min(L, units - i*L) of them,
        // stored compactly (qwn_internal.h).
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const uint32_t n = min(L, a.units > i * L ? a.units - i * L : 0u);
            const bool ok = active && j < n;
            if (KIND != kF16)
                met[i] = *reinterpret_cast<const uint2 *>(
                    ok ? tile_m + 8 * R * L * i + (grp * n + j) * 8 : tile_m);
        }
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const uint32_t n = min(L, a.units > i * L ? a.units - i * L : 0u);
            const bool ok = active && j < n;
            const uint8_t *base = tile_p + 64 * R * L * i + (grp * n + j) * 16;
#pragma unroll
            for (int q = 0; q < CH; ++q)
                pay[i][q] = *reinterpret_cast<const uint4 *>(ok ? base + q * R * n * 16 : tile_p);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // Loads whose results are needed only at the end: token scales (a
    // dependent scalar load, issued after the weight burst) and the residual.
    float tok_scale[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) tok_scale[t] = a.scale;
    if (a.scales) {
#pragma unroll
        for (int t = 0; t < MT; ++t) tok_scale[t] = a.scales[t < static_cast<int>(a.ntok) ? t : 0];
    }
    float resid = 0.0f;
    if (a.output_mode == kOutAdd && writer) resid = output[row];
    const float *bias = job == 0 ? a.bias[0] : job == 1 ? a.bias[1] : job == 2 ? a.bias[2] : a.bias[3];
    float bias_v = 0.0f;
    if (bias && writer) bias_v = bias[row];

    // 2. The LDS image.  Fused: this thread's block after the norm/SwiGLU,
    //    quantized with the workgroup-wide scale (c/qwanto_kernels.c:354-433)
    //    while the weight loads are in flight.  Image: wait for this wave's
    //    direct loads only (vector loads retire in issue order), then for
    //    every wave's share.
    if constexpr (fused) {
        float v[SR][E];
#pragma unroll
        for (int r = 0; r < SR; ++r)
#pragma unroll
            for (int i = 0; i < EW; ++i) {
                v[r][4 * i] = xv[r][i].x; v[r][4 * i + 1] = xv[r][i].y;
                v[r][4 * i + 2] = xv[r][i].z; v[r][4 * i + 3] = xv[r][i].w;
            }
        bool has[SR];
#pragma unroll
        for (int r = 0; r < SR; ++r) has[r] = threadIdx.x + r * blockDim.x < nvalid;
        if (a.input_mode == kInNorm) {
            float ss = 0.0f;
#pragma unroll
            for (int r = 0; r < SR; ++r) {
                float sr = 0.0f;
#pragma unroll
                for (int i = 0; i < E; ++i) sr = fmaf(v[r][i], v[r][i], sr);
                ss += has[r] ? sr : 0.0f;
            }
            ss = wg_sum(ss, red[0], W);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(a.cols) + a.eps);
#pragma unroll
            for (int r = 0; r < SR; ++r)
#pragma unroll
                for (int i = 0; i < EW; ++i) {
                    v[r][4 * i] = (v[r][4 * i] * inv) * x2v[r][i].x;
                    v[r][4 * i + 1] = (v[r][4 * i + 1] * inv) * x2v[r][i].y;
                    v[r][4 * i + 2] = (v[r][4 * i + 2] * inv) * x2v[r][i].z;
                    v[r][4 * i + 3] = (v[r][4 * i + 3] * inv) * x2v[r][i].w;
                }
        } else if (a.input_mode == kInSwiglu) {
#pragma unroll
            for (int r = 0; r < SR; ++r)
#pragma unroll
                for (int i = 0; i < EW; ++i) {
                    const float u[4] = {x2v[r][i].x, x2v[r][i].y, x2v[r][i].z, x2v[r][i].w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const float g = v[r][4 * i + k];
                        v[r][4 * i + k] = (g / (1.0f + expf(-g))) * u[k];
                    }
                }
        }
#pragma unroll
        for (int r = 0; r < SR; ++r)
            if (!has[r]) {
#pragma unroll
                for (int i = 0; i < E; ++i) v[r][i] = 0.0f;
            }
        if (KIND == kF16) {
#pragma unroll
            for (int r = 0; r < SR; ++r) {
                const uint32_t sb = threadIdx.x + r * blockDim.x;
                if (sb < nsub) {
                    const uint32_t e0 = sb * E;
                    float4 *dst = reinterpret_cast<float4 *>(smem + (e0 / 32) * 144 + (e0 % 32) * 4);
#pragma unroll
                    for (int i = 0; i < EW; ++i)
                        dst[i] = make_float4(v[r][4 * i], v[r][4 * i + 1], v[r][4 * i + 2], v[r][4 * i + 3]);
                }
            }
        } else {
            float amax = 0.0f;
#pragma unroll
            for (int r = 0; r < SR; ++r)
#pragma unroll
                for (int i = 0; i < E; ++i) amax = fmaxf(amax, fabsf(v[r][i]));
            amax = wg_max(amax, red[1], W);
            // IEEE division and reciprocal, as the CPU path (c/qwanto_kernels.c:385-386)
            const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / scale;
            tok_scale[0] = scale;
            if (a.scale_out && blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = scale;
#pragma unroll
            for (int r = 0; r < SR; ++r) {
                uint32_t w[EW], qb[E];
#pragma unroll
                for (int i = 0; i < E; ++i) qb[i] = q8_low_byte(fminf(127.0f, fmaxf(-127.0f, v[r][i] * inv)));
#pragma unroll
                for (int i = 0; i < EW; ++i) w[i] = pack_low_bytes(qb[4 * i], qb[4 * i + 1], qb[4 * i + 2], qb[4 * i + 3]);
                put_sub_block<KIND>(smem, a.units, threadIdx.x + r * blockDim.x, nsub, w);
            }
        }
        lds_barrier();
    } else {
        wait_vmcnt<(KIND == kF16 ? 4 : 5) * UPL>();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }

    // 3. Dot products.
    const uint32_t ib = a.image_bytes;
    const uint32_t act_bytes = a.units * unit_lds_bytes(KIND);
    // Paired tiles keep one sum per unit slot: the row total is then the
    // upper half's lane sum plus the lower half's, the order the one-unit
    // launch's lane reduction adds them in, so both launches of a tensor
    // round alike.
    constexpr int NS = PAIRED_TILES ? UPL : 1;
    float accs[NS][MT];
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) accs[i][t] = 0.0f;
#pragma unroll
    for (int i = 0; i < UPL; ++i) {
        const uint32_t u = j + i * L;
        if (!(active && u < a.units)) continue;
        float(&acc)[MT] = accs[PAIRED_TILES ? i : 0];
        if (KIND == kHvsq2) {
            const uint32_t *cw = reinterpret_cast<const uint32_t *>(pay[i]);
            const float d = half_to_float(met[i].x & 0xffffu);
            const float m = half_to_float(met[i].x >> 16);
            const uint32_t subs = met[i].y;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const uint8_t *img = smem + t * ib;
                const uint4 *at = reinterpret_cast<const uint4 *>(img + u * 272);
                uint4 av[16];
#pragma unroll
                for (int g = 0; g < 16; ++g) av[g] = at[g];
                const int4 *sp = reinterpret_cast<const int4 *>(img + act_bytes + u * 32);
                const int4 sv0 = sp[0], sv1 = sp[1];
                const int so[8] = {sv0.x, sv0.y, sv0.z, sv0.w, sv1.x, sv1.y, sv1.z, sv1.w};
                int s1 = 0, sa = 0;
#pragma unroll
                for (int o = 0; o < 8; ++o) {
                    const int s = static_cast<int>((subs >> (4 * o)) & 15u);
                    s1 += s * (hv_octant_dot(cw[2 * o], cw[2 * o + 1], av[2 * o], av[2 * o + 1]) - so[o]);
                    sa += so[o];
                }
                acc[t] = fmaf(d, static_cast<float>(s1) * 0.125f, acc[t]);
                acc[t] = fmaf(m, static_cast<float>(sa), acc[t]);
            }
        } else if (KIND == kQ4_0) {
            const uint32_t sc[2] = {met[i].x, met[i].y};
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const uint8_t *img = smem + t * ib;
                const uint4 *at = reinterpret_cast<const uint4 *>(img + u * 144);
                const int4 corr = *reinterpret_cast<const int4 *>(img + act_bytes + u * 16);
                const int cb[4] = {corr.x, corr.y, corr.z, corr.w};
#pragma unroll
                for (int b4 = 0; b4 < 4; ++b4) {
                    const float d = half_to_float(sc[b4 >> 1] >> (16 * (b4 & 1)));
                    const int raw = q4_block_dot(pay[i][b4], at[2 * b4], at[2 * b4 + 1]) - cb[b4];
                    acc[t] = fmaf(static_cast<float>(raw), d, acc[t]);
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t h[4] = {pay[i][q].x, pay[i][q].y, pay[i][q].z, pay[i][q].w};
                float wf[8];
                if (a.bf16) {
                    // bfloat16: the 16 bits are the high half of the fp32 value
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        wf[2 * k] = __builtin_bit_cast(float, h[k] << 16);
                        wf[2 * k + 1] = __builtin_bit_cast(float, h[k] & 0xffff0000u);
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        wf[2 * k] = half_to_float(h[k] & 0xffffu);
                        wf[2 * k + 1] = half_to_float(h[k] >> 16);
                    }
                }
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const float4 *xa = reinterpret_cast<const float4 *>(smem + t * ib + u * 144 + q * 32);
                    const float4 x0 = xa[0], x1 = xa[1];
                    float s = acc[t];
                    s = fmaf(wf[0], x0.x, s); s = fmaf(wf[1], x0.y, s);
                    s = fmaf(wf[2], x0.z, s); s = fmaf(wf[3], x0.w, s);
                    s = fmaf(wf[4], x1.x, s); s = fmaf(wf[5], x1.y, s);
                    s = fmaf(wf[6], x1.z, s); s = fmaf(wf[7], x1.w, s);
                    acc[t] = s;
                }
            }
        }
    }

    // 4. Combine the L partials of each row with DPP; the group's last lane
    //    holds the row total and writes it.
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        acc[t] = group_sum(accs[0][t], L);
        if constexpr (PAIRED_TILES) acc[t] = group_sum(accs[1][t], L) + acc[t];
    }
    float first_out = 0.0f;
    if (paired) {
        // up rows -> LDS; the gate lane of the same row forms the SwiGLU
        const float sv = mul_rounded(acc[0], tok_scale[0]);
        if (job == 1 && writer) up_s[(wave - half_w) * kWaveSize + lane] = sv;
        lds_barrier();
        if (job == 0 && writer) {
            const float u = up_s[wave * kWaveSize + lane];
            output[row] = mul_rounded(sv / (1.0f + expf(-sv)), u);
        }
    } else if (writer) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (static_cast<uint32_t>(t) >= a.ntok) break;
            float s = acc[t];
            // rounded product, then the residual add: the CPU stores the
            // projection before vec_add(x, y) (c/qwanto_decode.c:1925, 1955), so no
            // contraction into one fused multiply-add here
            if (KIND != kF16) s = mul_rounded(s, tok_scale[t]);
            // the projection's bias, added to the stored product as the CPU's
            // add_bias (c/qwanto_decode.c:926-929, 1649-1651, 1722)
            if (bias) s = add_rounded(s, bias_v);
            if (a.output_mode == kOutAdd)
                s = add_rounded(t == 0 ? resid : output[static_cast<size_t>(t) * out_stride + row], s);
            if (t == 0) first_out = s;
            output[static_cast<size_t>(t) * out_stride + row] = s;
        }
    }
    if (MT == 1 && a.output_mode == kOutArgmax) {
        uint64_t key = writer ? argmax_key(first_out, row) : 0;
        for (int off = kWaveSize / 2; off > 0; off >>= 1) {
            const uint64_t o = shfl_xor_u64(key, off);
            key = o > key ? o : key;
        }
        if (lane == 0) red_key[wave] = key;
        lds_barrier();
        if (threadIdx.x == 0) {
            uint64_t best = red_key[0];
            for (uint32_t w = 1; w < W; ++w) best = red_key[w] > best ? red_key[w] : best;
            a.argmax_partials[blockIdx.x] = best;
        }
    }
}

// ---- int8 MFMA batch GEMM (HyperVSQ-2, 8..16 tokens) ----------------------
//
// With the octant multiplier folded into the weight, w = s_oct * (code - 1)
// lies in [-15, 30], so a whole 256-weight block is one exact int8 dot
// product per (row, token):
//   y[t][n] = xs_t * sum_blocks (d/8 * sum_i w_i a_t,i + m * sum_i a_t,i)
// (the same combination as the dot8 path).  A 16-row x 16-token tile takes
// four v_mfma_i32_16x16x64_i8 per block: lane l holds A row l%16 and B
// column (token) l%16 for k-bytes 16*(l/16)..+15, and C[4*(l/16)+r][l%16].
// Lane group g = l/16 takes the block's code chunk g (octants 2g, 2g+1);
// instruction s takes its code dword s.  The A bytes come out of the code
// dword through a byte permute over the table [-s, 0, s, 2s]: output dword
// k holds the weights of code fields k of bytes 0..3, i.e. elements
// 4*byte + k, so the MFMA image stores each 16-element group of activations
// in that transposed order:
//   image [block][s][g][token 0..15][16 B] (byte 4k+b = element 16s+4b+k of
//   the group 64g..64g+63), then the blocks' activation sums as floats
//   [block][token 0..15] (|sum| <= 256 * 127: exact).
// The weights stay in the GEMV wave-tile layout (one resident copy).  A
// workgroup owns a 16-row group and its waves split the K blocks, combining
// their partial tiles through LDS in wave order.  Where the group fits LDS
// its tiles are copied there whole (mfma_chunk_hv: the weights are then the
// B operand, so a lane applies its own row's scales); longer rows read the
// weights straight from HBM (mfma_chunk: weights as the A operand).
constexpr int kMfmaTokens = 16;

__host__ __device__ constexpr size_t mfma_image_block_bytes() { return 16 * 256 + 16 * 4; }

__global__ __launch_bounds__(256) void mfma_image_kernel(const int8_t *__restrict__ q8, uint32_t q8_stride,
                                                         uint32_t K, uint32_t M, uint32_t units, uint8_t *img) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < units * 256) {
        const uint32_t m = idx % 16, g = (idx / 16) % 4, sl = (idx / 64) % 4, b = idx / 256;
        uint32_t w[4] = {0, 0, 0, 0};
        if (m < M) {
            const uint32_t e0 = b * 256 + 64 * g + 16 * sl;
            const int8_t *src = q8 + static_cast<size_t>(m) * q8_stride;
#pragma unroll
            for (int bi = 0; bi < 4; ++bi)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t e = e0 + 4 * bi + k;
                    const uint32_t v = e < K ? static_cast<uint8_t>(src[e]) : 0u;
                    w[k] |= v << (8 * bi);
                }
        }
        *reinterpret_cast<uint4 *>(img + static_cast<size_t>(idx) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (idx < units * 16) {
        const uint32_t b = idx / 16, m = idx % 16;
        int sum = 0;
        if (m < M) {
            const int8_t *src = q8 + static_cast<size_t>(m) * q8_stride;
            for (uint32_t i = 0; i < 256; ++i) {
                const uint32_t e = b * 256 + i;
                if (e < K) sum += src[e];
            }
        }
        reinterpret_cast<float *>(img + static_cast<size_t>(units) * 4096)[idx] = static_cast<float>(sum);
    }
}

// Q4_0: one v_mfma_i32_16x16x32_i8 per 32-weight block.  A lane's weight
// operand is the 4 nibble bytes of weights 8g..8g+7 of its row (g = lane /
// 16) as two words, low nibbles then high nibbles (turned into the signed
// weights n - 8), so each 8-byte group of the image holds elements
// 8g + {0,2,4,6,1,3,5,7} of the block:
//   image [block][g][token 0..15][8 B]  (no activation sums: the signed
//   weights need no correction).
__host__ __device__ constexpr size_t mfma_q4_image_block_bytes() { return 4 * 16 * 8; }

__global__ __launch_bounds__(256) void mfma_q4_image_kernel(const int8_t *__restrict__ q8, uint32_t q8_stride,
                                                            uint32_t K, uint32_t M, uint32_t nblk, uint8_t *img) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < nblk * 64) {
        const uint32_t m = idx % 16, g = (idx / 16) % 4, b = idx / 64;
        uint32_t w[2] = {0, 0};
        if (m < M) {
            const int8_t *src = q8 + static_cast<size_t>(m) * q8_stride;
            const uint32_t e0 = b * 32 + 8 * g;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t e = e0 + (i < 4 ? 2 * i : 2 * (i - 4) + 1);
                const uint32_t v = e < K ? static_cast<uint8_t>(src[e]) : 0u;
                w[i >> 2] |= v << (8 * (i & 3));
            }
        }
        *reinterpret_cast<uint2 *>(img + static_cast<size_t>(idx) * 8) = make_uint2(w[0], w[1]);
    }
}

typedef int mfma_v4i __attribute__((ext_vector_type(4)));

// One launch over up to kMaxGroup HyperVSQ-2 tensors that share the image
// (same K, so the same wave-tile plan).  Job i owns workgroups
// [job_block[i], job_block[i+1]).  A workgroup computes one row group of
// 16*RT rows; its 2^ks_log2 waves split the K blocks (wave ks takes blocks
// [ks*nb, ks*nb + nb)).
struct MfmaArgs {
    const uint8_t *payload[kMaxGroup];
    const uint8_t *meta[kMaxGroup];
    float *output[kMaxGroup];
    uint32_t rows[kMaxGroup];
    uint32_t tiles[kMaxGroup];  // wave tiles allocated per job
    uint32_t output_stride[kMaxGroup];
    uint32_t job_block[kMaxGroup + 1];
    size_t tile_payload_bytes;
    size_t tile_meta_bytes;
    uint32_t units, lanes_log2, rows_per_wave_log2;
    uint32_t nblk;         // K blocks of a row (HyperVSQ-2: units; Q4_0: 32-weight blocks)
    uint32_t ks_log2;      // waves per workgroup (log2)
    uint32_t nb;           // K blocks per wave
    uint32_t stage_bytes;  // LDS bytes of the staged weight region (STAGE)
    const uint8_t *image;  // mfma images of up to 64 tokens, one per 16-token group (blockIdx.y)
    size_t group_image_bytes;
    const float *scales;   // [ntok]
    uint32_t ntok;
    uint32_t vec_out;      // bit i: job i's rows may be stored 4 at a time (16-byte aligned)
    uint32_t accumulate;   // out += W x (residual add) instead of out = W x
    int32_t *dump;         // DUMP kernels: exact int32 block dots [token][row][nblk] of job 0
    const float *bias[kMaxGroup];  // per job: null, or [rows] added to each token's product
    uint32_t pad_p, pad_m;         // HyperVSQ-2 staging gaps (hv_lds_pieces)
};

constexpr int kMfmaMaxWaves = 8;
constexpr int kMfmaSplitMaxWaves = 16;  // the Q4_0 K-split kernel

// Byte offsets of (row, unit, chunk g) in the wave-tile layout:
//   payload tile * tile_payload + 64*R*L*slot + (g*R*n + grp*n + jj) * 16
//   meta    tile * tile_meta    +  8*R*L*slot + (grp*n + jj) * 8
// with slot = unit / L, jj = unit % L, n = units in the slot.
// The 16-token group of a launch over more tokens (blockIdx.y): its image
// (groups of 16 tokens stored one after another), scales, token count and
// first token.
struct MfmaTok {
    const uint8_t *image;
    const float *scales;
    uint32_t ntok, tok0;
};
__device__ __forceinline__ MfmaTok mfma_tok(const MfmaArgs &a) {
    MfmaTok t;
    t.tok0 = 16 * blockIdx.y;
    t.image = a.image + blockIdx.y * a.group_image_bytes;
    t.scales = a.scales + t.tok0;
    t.ntok = min(16u, a.ntok - t.tok0);
    return t;
}

struct MfmaUnit {
    size_t payload, meta;
};
__device__ __forceinline__ MfmaUnit mfma_unit(const MfmaArgs &a, uint32_t row, uint32_t b, uint32_t g) {
    const uint32_t L = 1u << a.lanes_log2, R = 1u << a.rows_per_wave_log2;
    const uint32_t slot = b >> a.lanes_log2, jj = b & (L - 1);
    const uint32_t n = min(L, a.units - slot * L);
    const uint32_t tile = row >> a.rows_per_wave_log2, grp = row & (R - 1);
    MfmaUnit u;
    u.payload = tile * a.tile_payload_bytes + static_cast<size_t>(64) * R * L * slot +
                (static_cast<size_t>(g) * R * n + grp * n + jj) * 16;
    u.meta = tile * a.tile_meta_bytes + static_cast<size_t>(8) * R * L * slot + (grp * n + jj) * 8;
    return u;
}

// One chunk of up to NB blocks of a row group read straight from the
// wave-tile layout (rows too long to stage in LDS): the weight and image
// loads of the whole chunk are issued before the first MFMA.  The weights
// are the MFMA's A operand here, so lane (g, m) holds rows 4g .. 4g+3 of
// token m and takes those rows' d and m from the lanes that loaded them.
template <int NB, int RT, bool DUMP>
__device__ __forceinline__ void mfma_chunk(const MfmaArgs &a, const MfmaTok &tk, const uint8_t *payload, const uint8_t *meta,
                                           uint32_t rows, uint32_t r0, uint32_t b0, uint32_t nblk, uint32_t lane,
                                           float (&acc)[RT][4]) {
    const uint32_t g = lane >> 4, m = lane & 15;
    const float *sums = reinterpret_cast<const float *>(tk.image + static_cast<size_t>(a.units) * 4096);
    uint4 A[NB][RT];
    uint2 Mt[NB][RT];
    mfma_v4i B[NB][4];
    float SA[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t b = b0 + (static_cast<uint32_t>(i) < nblk ? i : 0);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t row = r0 + 16 * t + m;
            const MfmaUnit u = mfma_unit(a, row < rows ? row : 0, b, g);
            A[i][t] = *reinterpret_cast<const uint4 *>(payload + u.payload);
            Mt[i][t] = *reinterpret_cast<const uint2 *>(meta + u.meta);
        }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t b = b0 + (static_cast<uint32_t>(i) < nblk ? i : 0);
        const uint8_t *ib = tk.image + static_cast<size_t>(b) * 4096 + lane * 16;
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) B[i][sl] = *reinterpret_cast<const mfma_v4i *>(ib + sl * 1024);
        SA[i] = sums[b * 16 + m];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int t = 0; t < RT; ++t)
            if (r0 + 16 * t + m >= rows) Mt[i][t] = make_uint2(0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (static_cast<uint32_t>(i) >= nblk) break;
        const float sa = SA[i];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t subs = (Mt[i][t].y >> (8 * g)) & 0xffu;
            const uint32_t cw[4] = {A[i][t].x, A[i][t].y, A[i][t].z, A[i][t].w};
            mfma_v4i ci = {0, 0, 0, 0};
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) {
                const uint32_t sub = (subs >> (4 * (sl >> 1))) & 15u;
                // table bytes: code 0 -> -s, 1 -> 0, 2 -> s, 3 -> 2s
                const uint32_t lut = ((0u - sub) & 0xffu) | (sub << 16) | ((2u * sub) << 24);
                const uint32_t c = cw[sl];
                mfma_v4i av;
                av.x = static_cast<int>(__builtin_amdgcn_perm(0u, lut, c & 0x03030303u));
                av.y = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 2) & 0x03030303u));
                av.z = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 4) & 0x03030303u));
                av.w = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 6) & 0x03030303u));
                ci = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, B[i][sl], ci, 0, 0, 0);
            }
            if constexpr (DUMP) {
                // sum over the block's octants of multiplier * sum (code-1)*a
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t row = r0 + 16 * t + 4 * g + r;
                    if (row < rows && m < tk.ntok)
                        a.dump[(static_cast<size_t>(m) * rows + row) * a.nblk + b0 + i] = ci[r];
                }
            }
            // C element r of this lane is row 4g + r of the tile: its
            // d_base / m_base were loaded by lane 4g + r
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t dm = static_cast<uint32_t>(__shfl(static_cast<int>(Mt[i][t].x), 4 * g + r));
                const float dsc = half_to_float(dm & 0xffffu) * 0.125f;
                const float msc = half_to_float(dm >> 16);
                acc[t][r] = fmaf(static_cast<float>(ci[r]), dsc, fmaf(msc, sa, acc[t][r]));
            }
        }
    }
}

// Staged HyperVSQ-2 row groups keep their tiles' wave-tile layout (copied
// whole, every load instruction one contiguous 1 KB span), with a gap of
// `pad` 16-byte pieces after every 64 pieces (each copy instruction's LDS
// destination moves on by 64 + pad pieces): piece q of the copy sits at LDS
// piece q + (q / 64) * pad.  The gaps (payload and meta separately, chosen
// per tile shape at upload: hv_stage_pads) spread a wave's operand reads of
// one block over the LDS banks, which the plain layout folds onto two of
// sixteen 16-byte bank groups for the common shapes.
__host__ __device__ constexpr uint32_t hv_lds_pieces(uint32_t pieces, uint32_t pad) {
    return pieces + (pieces + 63) / 64 * pad;
}
__host__ __device__ constexpr uint32_t hv_stage_bytes(uint32_t units, uint32_t pad_p, uint32_t pad_m) {
    return 16 * hv_lds_pieces(64 * units, pad_p) + 16 * hv_lds_pieces(8 * units, pad_m);
}

// Per-lane operand offsets of a staged group for lane (g, m): the payload
// piece and meta byte of row m's unit 0 in a full slot and in the last
// slot (whose width differs); a unit adds a wave-uniform slot and lane offset.
struct HvLane {
    uint32_t qf, ql, mf, ml, last_slot;
};

__device__ __forceinline__ HvLane hv_lane(const MfmaArgs &a, const MfmaTok &tk, uint32_t lane) {
    const uint32_t L = 1u << a.lanes_log2, R = 1u << a.rows_per_wave_log2;
    const uint32_t g = lane >> 4, m = lane & 15;
    const uint32_t tl = m >> a.rows_per_wave_log2, grp = m & (R - 1);
    HvLane h;
    h.last_slot = (a.units - 1) >> a.lanes_log2;
    const uint32_t nlast = a.units - h.last_slot * L;
    const uint32_t tq = tl * static_cast<uint32_t>(a.tile_payload_bytes / 16);
    const uint32_t tmb = tl * static_cast<uint32_t>(a.tile_meta_bytes);
    h.qf = tq + (g * R + grp) * L;
    h.ql = tq + (g * R + grp) * nlast;
    h.mf = tmb + 8 * grp * L;
    h.ml = tmb + 8 * grp * nlast;
    return h;
}

// The image operands of up to NB HyperVSQ-2 blocks from b0 (nv of them real,
// the rest repeat b0): per block four 16-byte MFMA operands (tokens m, chunk
// g of each slice) and the activation sums of tokens 4g .. 4g+3.  Bounded
// buffer loads: the columns of tokens past tk.ntok read as zero with no
// memory access (their products are never stored), so a 4-token batch moves
// a quarter of the image.  Always 5 * NB loads, so a caller can wait for
// older loads with vmcnt(5 * NB).
template <int NB>
struct HvImage {
    mfma_v4i B[NB][4];
    float4 SA[NB];
};

template <int NB>
__device__ __forceinline__ void hv_image_loads(const MfmaArgs &a, const MfmaTok &tk, uint32_t b0, uint32_t nv, uint32_t lane,
                                               HvImage<NB> &im) {
    const uint32_t bytes = a.units * static_cast<uint32_t>(mfma_image_block_bytes());
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(tk.image), 0, static_cast<int>(bytes), 0x00020000);
    const uint32_t m = lane & 15, g = lane >> 4;
    const uint32_t skip = m < tk.ntok ? 0u : 0x80000000u, sskip = 4 * g < tk.ntok ? 0u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t b = b0 + (static_cast<uint32_t>(i) < nv ? i : 0);
        const uint32_t off = (b * 4096 + lane * 16) | skip;
#pragma unroll
        for (int sl = 0; sl < 4; ++sl)
            im.B[i][sl] =
                __builtin_bit_cast(mfma_v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off + sl * 1024, 0, 0));
        im.SA[i] = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(rs, (a.units * 4096 + (b * 16 + 4 * g) * 4) | sskip, 0, 0));
    }
}

// One chunk of up to NB HyperVSQ-2 blocks b0 .. b0 + nv - 1 of a staged
// group (`im` their image operands, `meta_lds` the staged meta).  The tokens
// are the MFMA's A operand and the weight rows its B operand, so lane (g, m)
// accumulates tokens 4g .. 4g+3 of row m and applies the d and m of its own
// row (no exchange between lanes).  `live`: row m exists (else its scales
// count as 0).
template <int NB, bool DUMP>
__device__ __forceinline__ void mfma_chunk_hv(const MfmaArgs &a, const MfmaTok &tk, const uint8_t *lds, uint32_t meta_lds,
                                              const HvLane &hl, uint32_t b0, uint32_t nv, bool live, uint32_t rows,
                                              uint32_t r0, uint32_t lane, const HvImage<NB> &im, float (&acc)[4]) {
    const uint32_t g = lane >> 4, m = lane & 15;
    const uint32_t R = 1u << a.rows_per_wave_log2, L = 1u << a.lanes_log2;
    uint4 A[NB];
    uint2 Mt[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t b = b0 + (static_cast<uint32_t>(i) < nv ? i : 0);
        const uint32_t slot = b >> a.lanes_log2, jj = b & (L - 1);
        const bool last = slot == hl.last_slot;
        const uint32_t q = (last ? hl.ql : hl.qf) + 4 * R * L * slot + jj;
        A[i] = *reinterpret_cast<const uint4 *>(lds + 16 * (q + (q >> 6) * a.pad_p));
        const uint32_t mb = (last ? hl.ml : hl.mf) + 8 * R * L * slot + 8 * jj, mq = mb >> 4;
        Mt[i] = *reinterpret_cast<const uint2 *>(lds + meta_lds + 16 * (mq + (mq >> 6) * a.pad_m) + (mb & 8u));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (static_cast<uint32_t>(i) >= nv) break;
        const uint32_t subs = (Mt[i].y >> (8 * g)) & 0xffu;
        const uint32_t cw[4] = {A[i].x, A[i].y, A[i].z, A[i].w};
        mfma_v4i ci = {0, 0, 0, 0};
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
            const uint32_t sub = (subs >> (4 * (sl >> 1))) & 15u;
            // table bytes: code 0 -> -s, 1 -> 0, 2 -> s, 3 -> 2s
            const uint32_t lut = ((0u - sub) & 0xffu) | (sub << 16) | ((2u * sub) << 24);
            const uint32_t c = cw[sl];
            mfma_v4i wv;
            wv.x = static_cast<int>(__builtin_amdgcn_perm(0u, lut, c & 0x03030303u));
            wv.y = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 2) & 0x03030303u));
            wv.z = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 4) & 0x03030303u));
            wv.w = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 6) & 0x03030303u));
            // C[token][row]: element r is token 4g + r of row m
            ci = __builtin_amdgcn_mfma_i32_16x16x64_i8(im.B[i][sl], wv, ci, 0, 0, 0);
        }
        if constexpr (DUMP) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t row = r0 + m, tok = 4 * g + r;
                if (row < rows && tok < tk.ntok)
                    a.dump[(static_cast<size_t>(tok) * rows + row) * a.nblk + b0 + i] = ci[r];
            }
        }
        const uint32_t dm = live ? Mt[i].x : 0u;
        const float dsc = half_to_float(dm & 0xffffu) * 0.125f;
        const float msc = half_to_float(dm >> 16);
        const float sa[4] = {im.SA[i].x, im.SA[i].y, im.SA[i].z, im.SA[i].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(static_cast<float>(ci[r]), dsc, fmaf(msc, sa[r], acc[r]));
    }
}

// Staged Q4_0 row groups are laid out row-major in LDS: payload
// [16 rows][q4_pay_stride(units) 16-byte pieces] (piece b of a row = chunk
// b % 4 of unit b / 4, i.e. 32-weight block b), then meta [16 rows]
// [q4_meta_stride(units) dwords] (unit u's four fp16 scales at dwords 2u,
// 2u + 1).  The odd piece stride (and odd pair stride of the meta) spreads
// a wave's 16 rows over the LDS banks, and a block's address is a per-lane
// base plus the block index, with no per-block layout arithmetic.
__host__ __device__ constexpr uint32_t q4_pay_stride(uint32_t units) { return 4 * units + 1; }
__host__ __device__ constexpr uint32_t q4_meta_stride(uint32_t units) { return 2 * (units | 1u); }
__host__ __device__ constexpr uint32_t q4_stage_bytes(uint32_t units) {
    return 16 * 16 * q4_pay_stride(units) + 16 * 4 * q4_meta_stride(units);
}

// Q4_0 codes n of four bytes, low or high nibbles, as the signed int8
// weights n - 8: per byte (0x80 | n) - 8 stays within the byte (no borrow),
// and flipping its top bit gives n - 8 in two's complement.
__device__ __forceinline__ uint32_t q4_signed(uint32_t nibbles) {
    return ((nibbles | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

// The image words of up to NB Q4_0 blocks from b0 (each lane's 8 bytes of
// a block: tokens m, elements 8g .. 8g+7); blocks past kb1 are not loaded.
template <int NB>
__device__ __forceinline__ void q4_image_loads(const MfmaArgs &a, const MfmaTok &tk, uint32_t b0, uint32_t kb1, uint32_t lane,
                                               uint2 (&B)[NB]) {
    if (b0 >= kb1) return;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t b = b0 + i < kb1 ? b0 + i : b0;
        B[i] = *reinterpret_cast<const uint2 *>(tk.image + static_cast<size_t>(b) * 512 + lane * 8);
    }
}

// One chunk of up to NB Q4_0 blocks (32 weights each; unit u = b / 4 holds
// blocks 4u .. 4u+3 as its four 16-byte payload chunks and their fp16
// scales as its meta), one v_mfma_i32_16x16x32_i8 per block on the signed
// weights n - 8 (so a block's product is its exact integer dot, no
// correction).  The tokens are the MFMA's A operand and the weight rows its
// B operand, so lane (g, m) accumulates tokens 4g .. 4g+3 of weight row m
// and applies the block scale it loaded itself.  `B` holds the chunk's
// image words, loaded by the caller ahead of time (STAGE: one chunk ahead,
// so the next chunk's image loads are in flight while this one computes).
// STAGE: the row group is in LDS in the row-major layout, `ppieces` and
// `mpieces` its payload and meta strides.
template <int NB, int RT, bool STAGE, bool DUMP>
__device__ __forceinline__ void mfma_chunk_q4(const MfmaArgs &a, const MfmaTok &tk, const uint8_t *payload, const uint8_t *meta,
                                              const uint8_t *lds, uint32_t meta_lds, uint32_t rows,
                                              uint32_t r0, uint32_t b0, uint32_t nblk, uint32_t lane,
                                              uint32_t ppieces, uint32_t mpieces, const uint2 (&B)[NB],
                                              float (&acc)[RT][4]) {
    const uint32_t g = lane >> 4, m = lane & 15;
    // the four fp16 block scales of a unit as two plain words (a select of
    // a uint2's fields by the block's position went through scratch memory)
    uint32_t A[NB][RT], Ml[NB][RT], Mh[NB][RT];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t b = b0 + (static_cast<uint32_t>(i) < nblk ? i : 0);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t row = r0 + 16 * t + m;
            const MfmaUnit u = STAGE ? MfmaUnit{} : mfma_unit(a, row < rows ? row : 0u, b >> 2, b & 3);
            if constexpr (STAGE) {
                // row 16t + m of the staged group (rows past the tensor read
                // the group's row 0 and get scale 0)
                const uint32_t rr = row < rows ? 16 * t + m : 0u;
                A[i][t] = *reinterpret_cast<const uint32_t *>(lds + 16 * (rr * ppieces + b) + 4 * g);
                const uint2 mt = *reinterpret_cast<const uint2 *>(lds + meta_lds + 4 * (rr * mpieces + 2 * (b >> 2)));
                Ml[i][t] = mt.x;
                Mh[i][t] = mt.y;
            } else {
                A[i][t] = *reinterpret_cast<const uint32_t *>(payload + u.payload + 4 * g);
                const uint2 mt = *reinterpret_cast<const uint2 *>(meta + u.meta);
                Ml[i][t] = mt.x;
                Mh[i][t] = mt.y;
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (static_cast<uint32_t>(i) >= nblk) break;
        const uint32_t q = (b0 + i) & 3;
        const long xv = static_cast<long>((static_cast<uint64_t>(B[i].y) << 32) | B[i].x);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t lo = q4_signed(A[i][t] & 0x0f0f0f0fu), hi = q4_signed((A[i][t] >> 4) & 0x0f0f0f0fu);
            const long wv = static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
            mfma_v4i ci = {0, 0, 0, 0};
            // C[token][row]: element r is token 4g + r of row m
            ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(xv, wv, ci, 0, 0, 0);
            if constexpr (DUMP) {
                // sum (nibble-8)*a of the block for token 4g + r, row m
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t row = r0 + 16 * t + m, tok = 4 * g + r;
                    if (row < rows && tok < tk.ntok)
                        a.dump[(static_cast<size_t>(tok) * rows + row) * a.nblk + b0 + i] = ci[r];
                }
            }
            // rows past the tensor contribute nothing (scale 0)
            const uint64_t w64 = (static_cast<uint64_t>(Mh[i][t]) << 32) | Ml[i][t];
            const uint32_t h = r0 + 16 * t + m < rows ? static_cast<uint32_t>(w64 >> (16 * q)) & 0xffffu : 0u;
            const float d = half_to_float(h);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(static_cast<float>(ci[r]), d, acc[t][r]);
        }
    }
}

template <int KIND, int NB, int RT, bool STAGE, bool DUMP>
__global__ __launch_bounds__(kWaveSize * kMfmaMaxWaves) void mfma_gemm_kernel(MfmaArgs a) {
    const MfmaTok tk = mfma_tok(a);
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = threadIdx.x % kWaveSize;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
    const uint32_t KS = 1u << a.ks_log2;
    const uint32_t ks = wave;
    const uint32_t b1 = a.job_block[1], b2 = a.job_block[2], b3 = a.job_block[3];
    uint32_t job = (blockIdx.x >= b1 ? 1u : 0u) + (blockIdx.x >= b2 ? 1u : 0u) + (blockIdx.x >= b3 ? 1u : 0u);
    job = __builtin_amdgcn_readfirstlane(job);
    const uint8_t *payload = job == 0 ? a.payload[0] : job == 1 ? a.payload[1] : job == 2 ? a.payload[2] : a.payload[3];
    const uint8_t *meta = job == 0 ? a.meta[0] : job == 1 ? a.meta[1] : job == 2 ? a.meta[2] : a.meta[3];
    float *output = job == 0 ? a.output[0] : job == 1 ? a.output[1] : job == 2 ? a.output[2] : a.output[3];
    const uint32_t rows = job == 0 ? a.rows[0] : job == 1 ? a.rows[1] : job == 2 ? a.rows[2] : a.rows[3];
    const uint32_t tiles = job == 0 ? a.tiles[0] : job == 1 ? a.tiles[1] : job == 2 ? a.tiles[2] : a.tiles[3];
    const uint32_t stride = job == 0   ? a.output_stride[0]
                            : job == 1 ? a.output_stride[1]
                            : job == 2 ? a.output_stride[2]
                                       : a.output_stride[3];
    output += static_cast<size_t>(tk.tok0) * stride;  // this launch's token group
    const uint32_t first = job == 0 ? 0u : job == 1 ? b1 : job == 2 ? b2 : b3;
    const float *bias = job == 0 ? a.bias[0] : job == 1 ? a.bias[1] : job == 2 ? a.bias[2] : a.bias[3];
    const uint32_t r0 = (blockIdx.x - first) * (16 * RT);
    const uint32_t kb0 = ks * a.nb;
    const uint32_t kb1 = min(a.nblk, kb0 + a.nb);
    // token-major epilogue (lane (g, m): tokens 4g .. 4g+3 of row m): its
    // token scales and, adding into the output, the prior outputs, loaded
    // now so the epilogue does not wait a memory round trip
    float xs_pre[4], res_pre[RT][4];
    if constexpr (KIND == kQ4_0 || STAGE) {
        const uint32_t g = lane >> 4, m = lane & 15;
#pragma unroll
        for (int r = 0; r < 4; ++r) xs_pre[r] = tk.scales[min(4 * g + r, tk.ntok - 1)];
        if (a.accumulate && ks == 0) {
#pragma unroll
            for (int t = 0; t < RT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t tok = 4 * g + r, row = r0 + 16 * t + m;
                    res_pre[t][r] = tok < tk.ntok && row < rows ? output[static_cast<size_t>(tok) * stride + row] : 0.0f;
                }
        }
    }

    // STAGE: the row group's wave tiles (16*RT rows = a whole number of
    // tiles) are copied into LDS row-major with direct loads
    const uint32_t t0 = r0 >> a.rows_per_wave_log2;
    uint32_t meta_lds = 0, ppieces = 0, mpieces = 0;
    HvImage<NB> him;
    uint2 Bx[NB], By[NB];
    if constexpr (STAGE) {
        const uint32_t ntile = min((16u * RT) >> a.rows_per_wave_log2, tiles - t0);
        if constexpr (KIND == kQ4_0) {
            const uint8_t *psrc = payload + static_cast<size_t>(t0) * a.tile_payload_bytes;
            const uint8_t *msrc = meta + static_cast<size_t>(t0) * a.tile_meta_bytes;
            // row-major layout (q4_pay_stride): LDS piece p of the copy is
            // (row p / stride, block p % stride); the lane order fixes the
            // destination, so each lane computes its piece's source in the
            // wave-tile layout, in 32-bit arithmetic, its (row, block)
            // advanced by the workgroup's width each step (one division up
            // front).  A padding piece copies its row's last block again
            // (same cache line); rows past the tensor's tiles copy the tile
            // start (read with scale 0).
            const uint32_t L = 1u << a.lanes_log2, R = 1u << a.rows_per_wave_log2, step = blockDim.x;
            const uint32_t tp = static_cast<uint32_t>(a.tile_payload_bytes);
            const uint32_t tm = static_cast<uint32_t>(a.tile_meta_bytes);
            ppieces = q4_pay_stride(a.units);
            mpieces = q4_meta_stride(a.units);
            meta_lds = 16 * 16 * ppieces;
            {
                const uint32_t dq = step / ppieces, dr = step - dq * ppieces;
                uint32_t pc = wave * kWaveSize + lane, rr = pc / ppieces, b = pc - rr * ppieces;
                for (uint32_t c0 = wave * kWaveSize; c0 < 16 * ppieces; c0 += step) {
                    const uint32_t tl = rr >> a.rows_per_wave_log2, bb = min(b, 4 * a.units - 1);
                    const uint32_t u = bb >> 2, slot = u >> a.lanes_log2, n = min(L, a.units - slot * L);
                    const uint32_t src =
                        tl < ntile ? tl * tp + 64 * R * L * slot + 16 * (((bb & 3) * R + (rr & (R - 1))) * n + (u & (L - 1)))
                                   : 0u;
                    if (pc < 16 * ppieces)
                        __builtin_amdgcn_global_load_lds(psrc + src, (lds_void *)(smem + c0 * 16), 16, 0, 0);
                    pc += step;
                    b += dr;
                    rr += dq;
                    if (b >= ppieces) {
                        b -= ppieces;
                        ++rr;
                    }
                }
            }
            {
                const uint32_t dq = step / mpieces, dr = step - dq * mpieces;
                uint32_t dw = wave * kWaveSize + lane, rr = dw / mpieces, w = dw - rr * mpieces;
                for (uint32_t c0 = wave * kWaveSize; c0 < 16 * mpieces; c0 += step) {
                    const uint32_t tl = rr >> a.rows_per_wave_log2, u = min(w >> 1, a.units - 1);
                    const uint32_t slot = u >> a.lanes_log2, n = min(L, a.units - slot * L);
                    const uint32_t src =
                        tl < ntile ? tl * tm + 8 * R * L * slot + 8 * ((rr & (R - 1)) * n + (u & (L - 1))) + 4 * (w & 1)
                                   : 0u;
                    if (dw < 16 * mpieces)
                        __builtin_amdgcn_global_load_lds(msrc + src, (lds_void *)(smem + meta_lds + c0 * 4), 4, 0, 0);
                    dw += step;
                    w += dr;
                    rr += dq;
                    if (w >= mpieces) {
                        w -= mpieces;
                        ++rr;
                    }
                }
            }
            // the first chunk's image words go out behind the copies
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_sched_barrier(0);
            q4_image_loads<NB>(a, tk, kb0, kb1, lane, Bx);
        } else {
            static_assert(RT == 1, "the staged HyperVSQ-2 group is 16 rows");
            const uint8_t *psrc = payload + static_cast<size_t>(t0) * a.tile_payload_bytes;
            const uint8_t *msrc = meta + static_cast<size_t>(t0) * a.tile_meta_bytes;
            const uint32_t np = ntile * static_cast<uint32_t>(a.tile_payload_bytes / 16);
            const uint32_t nm = (ntile * static_cast<uint32_t>(a.tile_meta_bytes) + 15) / 16;
            meta_lds = 16 * hv_lds_pieces(64 * a.units, a.pad_p);
            for (uint32_t c0 = wave * kWaveSize; c0 < np; c0 += blockDim.x)
                if (c0 + lane < np)
                    __builtin_amdgcn_global_load_lds(psrc + 16 * static_cast<size_t>(c0 + lane),
                                                     (lds_void *)(smem + 16 * (c0 + (c0 >> 6) * a.pad_p)), 16, 0, 0);
            for (uint32_t c0 = wave * kWaveSize; c0 < nm; c0 += blockDim.x)
                if (c0 + lane < nm)
                    __builtin_amdgcn_global_load_lds(msrc + 16 * static_cast<size_t>(c0 + lane),
                                                     (lds_void *)(smem + meta_lds + 16 * (c0 + (c0 >> 6) * a.pad_m)),
                                                     16, 0, 0);
            // the first chunk's image loads go out behind the copies
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_sched_barrier(0);
            if (kb0 < kb1) hv_image_loads<NB>(a, tk, kb0, min(static_cast<uint32_t>(NB), kb1 - kb0), lane, him);
        }
        // this wave's copies landed (all but its first image loads, which
        // retire after them)
        if (kb0 < kb1) wait_vmcnt<KIND == kHvsq2 ? 5 * NB : NB>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();  // ... and every wave's
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }

    float acc[RT][4];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;
    if constexpr (KIND == kHvsq2 && STAGE) {
        const bool live = r0 + (lane & 15) < rows;
        const HvLane hl = hv_lane(a, tk, lane);
        for (uint32_t b0 = kb0; b0 < kb1; b0 += NB) {
            const uint32_t nv = min(static_cast<uint32_t>(NB), kb1 - b0);
            if (b0 != kb0) hv_image_loads<NB>(a, tk, b0, nv, lane, him);
            mfma_chunk_hv<NB, DUMP>(a, tk, smem, meta_lds, hl, b0, nv, live, rows, r0, lane, him, acc[0]);
        }
    } else if constexpr (KIND == kHvsq2) {
        for (uint32_t b0 = kb0; b0 < kb1; b0 += NB)
            mfma_chunk<NB, RT, DUMP>(a, tk, payload, meta, rows, r0, b0, min(static_cast<uint32_t>(NB), kb1 - b0), lane,
                                     acc);
    } else if constexpr (STAGE) {
        // the weights are in LDS: each chunk's image words are loaded one
        // chunk ahead (two register sets used in turn, the first chunk's
        // behind the staging copies), so a chunk's products run while the
        // next chunk's image is on its way
        for (uint32_t b0 = kb0; b0 < kb1; b0 += 2 * NB) {
            const uint32_t b1 = b0 + NB;
            q4_image_loads<NB>(a, tk, b1, kb1, lane, By);
            mfma_chunk_q4<NB, RT, STAGE, DUMP>(a, tk, payload, meta, smem, meta_lds, rows, r0, b0,
                                               min(static_cast<uint32_t>(NB), kb1 - b0), lane, ppieces, mpieces,
                                               Bx, acc);
            if (b1 >= kb1) break;
            q4_image_loads<NB>(a, tk, b1 + NB, kb1, lane, Bx);
            mfma_chunk_q4<NB, RT, STAGE, DUMP>(a, tk, payload, meta, smem, meta_lds, rows, r0, b1,
                                               min(static_cast<uint32_t>(NB), kb1 - b1), lane, ppieces, mpieces,
                                               By, acc);
        }
    } else {
        for (uint32_t b0 = kb0; b0 < kb1; b0 += NB) {
            q4_image_loads<NB>(a, tk, b0, kb1, lane, Bx);
            mfma_chunk_q4<NB, RT, STAGE, DUMP>(a, tk, payload, meta, smem, meta_lds, rows, r0, b0,
                                               min(static_cast<uint32_t>(NB), kb1 - b0), lane, ppieces, mpieces,
                                               Bx, acc);
        }
    }

    // the K-split partials, summed in wave order (LDS after the staged tiles)
    if (KS > 1) {
        float *part_s = reinterpret_cast<float *>(smem + a.stage_bytes);
        if (ks > 0) {
            float *dst = part_s + ((ks - 1) * kWaveSize + lane) * 4 * RT;
#pragma unroll
            for (int t = 0; t < RT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) dst[4 * t + r] = acc[t][r];
        }
        __syncthreads();
        if (ks == 0)
            for (uint32_t k = 1; k < KS; ++k) {
                const float *src = part_s + ((k - 1) * kWaveSize + lane) * 4 * RT;
#pragma unroll
                for (int t = 0; t < RT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][r] += src[4 * t + r];
            }
    }
    // lane (g, m) holds rows 4g .. 4g+3 of each tile for token m: one
    // 16-byte store where the rows are whole and the output row aligned
    // accumulate: out += the rounded product (the residual stream), in two
    // roundings as the dot8 epilogue
    const uint32_t g = lane >> 4, m = lane & 15;
    if constexpr (KIND == kQ4_0 || STAGE) {
        // lane (g, m) holds tokens 4g .. 4g+3 of row m of each tile: rows
        // are contiguous per token, so 16 lanes store one 64-byte span
        if (ks == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tok = 4 * g + r;
                if (tok >= tk.ntok) continue;
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    const uint32_t row = r0 + 16 * t + m;
                    if (row >= rows) continue;
                    float v = mul_rounded(acc[t][r], xs_pre[r]);
                    if (bias) v = add_rounded(v, bias[row]);
                    output[static_cast<size_t>(tok) * stride + row] = a.accumulate ? add_rounded(res_pre[t][r], v) : v;
                }
            }
        }
        return;
    }
    if (ks == 0 && m < tk.ntok) {
        const float xs = tk.scales[m];
        const bool vec = (a.vec_out >> job) & 1u;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t n0 = r0 + 16 * t + 4 * g;
            float *dst = output + static_cast<size_t>(m) * stride + n0;
            if (vec && n0 + 4 <= rows) {
                float4 v = make_float4(mul_rounded(acc[t][0], xs), mul_rounded(acc[t][1], xs),
                                       mul_rounded(acc[t][2], xs), mul_rounded(acc[t][3], xs));
                if (bias) {
                    const float4 bv = *reinterpret_cast<const float4 *>(bias + n0);
                    v = make_float4(add_rounded(v.x, bv.x), add_rounded(v.y, bv.y), add_rounded(v.z, bv.z),
                                    add_rounded(v.w, bv.w));
                }
                if (a.accumulate) {
                    const float4 o = *reinterpret_cast<const float4 *>(dst);
                    v = make_float4(add_rounded(o.x, v.x), add_rounded(o.y, v.y), add_rounded(o.z, v.z),
                                    add_rounded(o.w, v.w));
                }
                *reinterpret_cast<float4 *>(dst) = v;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (n0 + r < rows) {
                        float v = mul_rounded(acc[t][r], xs);
                        if (bias) v = add_rounded(v, bias[n0 + r]);
                        dst[r] = a.accumulate ? add_rounded(dst[r], v) : v;
                    }
            }
        }
    }
}

// HyperVSQ-2 tensors with an MFMA-order copy: each wave loads its operands
// straight from HBM (a unit's 16 rows x 4 chunks are one contiguous 1 KB,
// lane (g, m) taking chunk g of row m; its meta one 128-byte span), so a
// workgroup has no staging copy, no barrier before its products and no LDS
// bank gaps; the products are mfma_chunk_hv's, the K-split sum and the
// token-major epilogue mfma_gemm_kernel's.  SPLIT: the residual adds over
// few row groups, each row group split four ways by unit range, the
// partials added with float atomics (in no fixed order).  payload[i] /
// meta[i] of the arguments are the copies.
template <int NB, bool SPLIT, bool DUMP, bool PAIR = false>
__global__ __launch_bounds__(kWaveSize * kMfmaMaxWaves) void mfma_direct_kernel(MfmaArgs a) {
    const MfmaTok tk = mfma_tok(a);
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = threadIdx.x % kWaveSize;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
    const uint32_t KS = 1u << a.ks_log2;
    static_assert(!PAIR || (!SPLIT && !DUMP), "gate/up pairs: plain stores");
    // PAIR (the SwiGLU of a gate/up pair): waves [0, KS) take the gate rows
    // of the row group, waves [KS, 2 KS) the same up rows; wj is a wave's
    // index within its job
    const uint32_t wj = PAIR && wave >= KS ? wave - KS : wave;
    const uint32_t b1 = a.job_block[1], b2 = a.job_block[2], b3 = a.job_block[3];
    uint32_t job = (blockIdx.x >= b1 ? 1u : 0u) + (blockIdx.x >= b2 ? 1u : 0u) + (blockIdx.x >= b3 ? 1u : 0u);
    job = __builtin_amdgcn_readfirstlane(job);
    if constexpr (PAIR) job = wave >= KS ? 1u : 0u;
    const uint8_t *payload = job == 0 ? a.payload[0] : job == 1 ? a.payload[1] : job == 2 ? a.payload[2] : a.payload[3];
    const uint8_t *meta = job == 0 ? a.meta[0] : job == 1 ? a.meta[1] : job == 2 ? a.meta[2] : a.meta[3];
    float *output = job == 0 ? a.output[0] : job == 1 ? a.output[1] : job == 2 ? a.output[2] : a.output[3];
    const uint32_t rows = job == 0 ? a.rows[0] : job == 1 ? a.rows[1] : job == 2 ? a.rows[2] : a.rows[3];
    const uint32_t stride = job == 0   ? a.output_stride[0]
                            : job == 1 ? a.output_stride[1]
                            : job == 2 ? a.output_stride[2]
                                       : a.output_stride[3];
    output += static_cast<size_t>(tk.tok0) * stride;  // this launch's token group
    const uint32_t first = job == 0 ? 0u : job == 1 ? b1 : job == 2 ? b2 : b3;
    const float *bias = job == 0 ? a.bias[0] : job == 1 ? a.bias[1] : job == 2 ? a.bias[2] : a.bias[3];
    const uint32_t local = PAIR ? blockIdx.x : blockIdx.x - first;
    const uint32_t qs = SPLIT ? (local & 3u) : 0u, rg = SPLIT ? (local >> 2) : local, r0 = rg * 16;
    const uint32_t g = lane >> 4, m = lane & 15;
    // this workgroup's units (SPLIT: quarter qs of the row's), then the wave's
    const uint32_t per_split = SPLIT ? (a.nblk + 3) / 4 : a.nblk;
    const uint32_t s0 = min(a.nblk, qs * per_split), s1 = min(a.nblk, s0 + per_split);
    const uint32_t kb0 = min(s1, s0 + wj * a.nb), kb1 = min(s1, kb0 + a.nb);
    // the epilogue's token scales and prior outputs, loaded ahead
    float xs_pre[4], res_pre[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) xs_pre[r] = tk.scales[min(4 * g + r, tk.ntok - 1)];
    if (!SPLIT && a.accumulate && wj == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = 4 * g + r, row = r0 + m;
            res_pre[r] = tok < tk.ntok && row < rows ? output[static_cast<size_t>(tok) * stride + row] : 0.0f;
        }
    }
    const uint8_t *pbase = payload + (static_cast<size_t>(rg) * a.units) * 1024 + lane * 16;
    const uint8_t *mbase = meta + (static_cast<size_t>(rg) * a.units) * 128 + m * 8;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    HvImage<NB> im;
    // the image as bounded buffer loads that skip absent tokens' columns
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(tk.image), 0, static_cast<int>(a.units * static_cast<uint32_t>(mfma_image_block_bytes())),
        0x00020000);
    const uint32_t skip = m < tk.ntok ? 0u : 0x80000000u, sskip = 4 * g < tk.ntok ? 0u : 0x80000000u;
    // one chunk of the wave's units from b0; the first is issued outside the
    // loop, so the loop header's wait for every load in flight does not
    // hold the first weight loads behind the epilogue's early loads
    auto chunk = [&](uint32_t b0) {
        const uint32_t nv = min(static_cast<uint32_t>(NB), kb1 - b0);
        uint4 A[NB];
        uint2 Mt[NB];
        // unit by unit (weights, meta, image), so a unit's products wait
        // only for its own loads and the later units' arrive meanwhile
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const uint32_t u = b0 + (static_cast<uint32_t>(i) < nv ? i : 0);
            A[i] = *reinterpret_cast<const uint4 *>(pbase + static_cast<size_t>(u) * 1024);
            Mt[i] = *reinterpret_cast<const uint2 *>(mbase + static_cast<size_t>(u) * 128);
            const uint32_t off = (u * 4096 + lane * 16) | skip;
#pragma unroll
            for (int sl = 0; sl < 4; ++sl)
                im.B[i][sl] =
                    __builtin_bit_cast(mfma_v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off + sl * 1024, 0, 0));
            im.SA[i] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(rs, (a.units * 4096 + (u * 16 + 4 * g) * 4) | sskip, 0, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (static_cast<uint32_t>(i) >= nv) break;
            const uint32_t subs = (Mt[i].y >> (8 * g)) & 0xffu;
            const uint32_t cw[4] = {A[i].x, A[i].y, A[i].z, A[i].w};
            mfma_v4i ci = {0, 0, 0, 0};
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) {
                const uint32_t sub = (subs >> (4 * (sl >> 1))) & 15u;
                // table bytes: code 0 -> -s, 1 -> 0, 2 -> s, 3 -> 2s
                const uint32_t lut = ((0u - sub) & 0xffu) | (sub << 16) | ((2u * sub) << 24);
                const uint32_t c = cw[sl];
                mfma_v4i wv;
                wv.x = static_cast<int>(__builtin_amdgcn_perm(0u, lut, c & 0x03030303u));
                wv.y = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 2) & 0x03030303u));
                wv.z = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 4) & 0x03030303u));
                wv.w = static_cast<int>(__builtin_amdgcn_perm(0u, lut, (c >> 6) & 0x03030303u));
                // C[token][row]: element r is token 4g + r of row m
                ci = __builtin_amdgcn_mfma_i32_16x16x64_i8(im.B[i][sl], wv, ci, 0, 0, 0);
            }
            if constexpr (DUMP) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t row = r0 + m, tok = 4 * g + r;
                    if (row < rows && tok < tk.ntok)
                        a.dump[(static_cast<size_t>(tok) * rows + row) * a.nblk + b0 + i] = ci[r];
                }
            }
            // rows past the matrix are zero in the copy: d = m = 0
            const uint32_t dm = Mt[i].x;
            const float dsc = half_to_float(dm & 0xffffu) * 0.125f;
            const float msc = half_to_float(dm >> 16);
            const float sa[4] = {im.SA[i].x, im.SA[i].y, im.SA[i].z, im.SA[i].w};
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = fmaf(static_cast<float>(ci[r]), dsc, fmaf(msc, sa[r], acc[r]));
        }
    };
    if (kb0 < kb1) chunk(kb0);
    for (uint32_t b0 = kb0 + NB; b0 < kb1; b0 += NB) chunk(b0);
    // the K-split partials, summed in wave order
    if (KS > 1) {
        // PAIR: each job's partials in its own region (a grouped launch's
        // other jobs are other workgroups)
        float *part_s = reinterpret_cast<float *>(smem) + (PAIR ? job : 0u) * (KS - 1) * kWaveSize * 4;
        if (wj > 0) {
            float *dst = part_s + ((wj - 1) * kWaveSize + lane) * 4;
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r] = acc[r];
        }
        __syncthreads();
        if (wj == 0)
            for (uint32_t k = 1; k < KS; ++k) {
                const float *src = part_s + ((k - 1) * kWaveSize + lane) * 4;
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] += src[r];
            }
    }
    // lane (g, m) holds tokens 4g .. 4g+3 of row m; accumulate: out += the
    // rounded product, in two roundings as the dot8 epilogue
    if constexpr (PAIR) {
        // the up wave hands its rounded products over; the gate wave stores
        // silu(gate) * up, the arithmetic of the SwiGLU input transform
        float *up_s = reinterpret_cast<float *>(smem) + 2 * (KS - 1) * kWaveSize * 4;
        if (job == 1 && wj == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) up_s[lane * 4 + r] = mul_rounded(acc[r], xs_pre[r]);
        }
        __syncthreads();
        if (job == 0 && wj == 0 && r0 + m < rows) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tok = 4 * g + r;
                if (tok >= tk.ntok) continue;
                const float gv = mul_rounded(acc[r], xs_pre[r]), uv = up_s[lane * 4 + r];
                output[static_cast<size_t>(tok) * stride + r0 + m] = mul_rounded(gv / (1.0f + expf(-gv)), uv);
            }
        }
        return;
    }
    const uint32_t row = r0 + m;
    if (wave == 0 && row < rows) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = 4 * g + r;
            if (tok >= tk.ntok) continue;
            float v = mul_rounded(acc[r], xs_pre[r]);
            if constexpr (SPLIT) {
                if (bias && qs == 0) v = add_rounded(v, bias[row]);
                unsafeAtomicAdd(output + static_cast<size_t>(tok) * stride + row, v);
            } else {
                if (bias) v = add_rounded(v, bias[row]);
                output[static_cast<size_t>(tok) * stride + row] = a.accumulate ? add_rounded(res_pre[r], v) : v;
            }
        }
    }
}

// The MFMA-order copy of a HyperVSQ-2 or Q4_0 tensor from its wave-tile
// layout: one thread per 16-byte payload piece and per 8-byte meta entry of
// the copy.
struct MfmaCopyArgs {
    const uint8_t *payload, *meta;
    uint8_t *dst_payload, *dst_meta;
    size_t tile_payload, tile_meta;
    uint32_t units, lanes_log2, rows_per_wave_log2, tiles, groups, q4;
};

__global__ __launch_bounds__(256) void mfma_copy_kernel(MfmaCopyArgs a) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t L = 1u << a.lanes_log2, R = 1u << a.rows_per_wave_log2;
    const size_t npay = static_cast<size_t>(a.groups) * a.units * 64;
    if (idx < npay) {
        const uint32_t piece = static_cast<uint32_t>(idx % 64), gu = static_cast<uint32_t>(idx / 64);
        const uint32_t rg = gu / a.units, u = gu - rg * a.units, g = piece >> 4, row = rg * 16 + (piece & 15);
        uint4 v = make_uint4(0, 0, 0, 0);
        if ((row >> a.rows_per_wave_log2) < a.tiles) {
            const uint32_t tile = row >> a.rows_per_wave_log2, grp = row & (R - 1);
            const uint32_t slot = u >> a.lanes_log2, n = min(L, a.units - slot * L);
            const uint8_t *src = a.payload + tile * a.tile_payload + static_cast<size_t>(64) * R * L * slot;
            if (a.q4) {
                // Q4_0: word q of piece (g, m) is word g of block 4u + q
                // (chunk q) of row m
                uint32_t w[4];
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q)
                    w[q] = *reinterpret_cast<const uint32_t *>(
                        src + 16 * (static_cast<size_t>(q) * R * n + grp * n + (u & (L - 1))) + 4 * g);
                v = make_uint4(w[0], w[1], w[2], w[3]);
            } else {
                v = *reinterpret_cast<const uint4 *>(src + 16 * (static_cast<size_t>(g) * R * n + grp * n + (u & (L - 1))));
            }
        }
        reinterpret_cast<uint4 *>(a.dst_payload)[idx] = v;
    }
    const size_t nmeta = static_cast<size_t>(a.groups) * a.units * 16;
    if (idx < nmeta) {
        const uint32_t gu = static_cast<uint32_t>(idx / 16), rg = gu / a.units, u = gu - rg * a.units;
        const uint32_t row = rg * 16 + static_cast<uint32_t>(idx % 16);
        uint2 v = make_uint2(0, 0);
        if ((row >> a.rows_per_wave_log2) < a.tiles) {
            const uint32_t tile = row >> a.rows_per_wave_log2, grp = row & (R - 1);
            const uint32_t slot = u >> a.lanes_log2, n = min(L, a.units - slot * L);
            v = *reinterpret_cast<const uint2 *>(a.meta + tile * a.tile_meta + static_cast<size_t>(8) * R * L * slot +
                                                 8 * (static_cast<size_t>(grp) * n + (u & (L - 1))));
        }
        reinterpret_cast<uint2 *>(a.dst_meta)[idx] = v;
    }
}

// Q4_0 launches of few row groups in accumulate mode (the residual adds of
// the o and down projections: 96-160 row groups leave most of the 256 CUs
// idle, and a CU's vector ALU bounds the per-block work): each row group is
// split four ways along K by a block's position in its unit (split s takes
// blocks 4u + s, i.e. chunk s of every unit, which in the wave-tile layout
// is one contiguous span per tile and slot), so a split stages a quarter of
// the row group's payload (and its whole meta), its waves divide the units,
// and the four partial products are added to the output with float atomics
// (their order is not fixed: the last bits of the residual can differ from
// run to run).
struct Q4Split {
    uint32_t qs, pst, mst, meta_lds;
};

// One chunk of the split's units v0 .. v0 + nv - 1 (block 4v + qs of each),
// operands read from the split's row-major staging: payload [16 rows][pst
// pieces] (piece v = chunk qs of unit v), meta [16 rows][mst dwords].
template <int NB>
__device__ __forceinline__ void mfma_chunk_q4s(const MfmaArgs &a, const MfmaTok &tk, const uint8_t *lds, const Q4Split &sp,
                                               uint32_t rows, uint32_t r0, uint32_t v0, uint32_t nv, uint32_t lane,
                                               float (&acc)[4]) {
    const uint32_t g = lane >> 4, m = lane & 15;
    const uint32_t row = r0 + m;
    const uint32_t rr = row < rows ? m : 0u;
    uint32_t A[NB], Ml[NB], Mh[NB];
    uint2 B[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint32_t v = v0 + (static_cast<uint32_t>(i) < nv ? i : 0);
        A[i] = *reinterpret_cast<const uint32_t *>(lds + 16 * (rr * sp.pst + v) + 4 * g);
        const uint2 mt = *reinterpret_cast<const uint2 *>(lds + sp.meta_lds + 4 * (rr * sp.mst + 2 * v));
        Ml[i] = mt.x;
        Mh[i] = mt.y;
        const uint32_t b = min(4 * v + sp.qs, a.nblk - 1);
        B[i] = *reinterpret_cast<const uint2 *>(tk.image + static_cast<size_t>(b) * 512 + lane * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
    const bool live = row < rows;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (static_cast<uint32_t>(i) >= nv) break;
        const bool has = live && 4 * (v0 + i) + sp.qs < a.nblk;
        const long xv = static_cast<long>((static_cast<uint64_t>(B[i].y) << 32) | B[i].x);
        const uint32_t lo = q4_signed(A[i] & 0x0f0f0f0fu), hi = q4_signed((A[i] >> 4) & 0x0f0f0f0fu);
        const long wv = static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
        mfma_v4i ci = {0, 0, 0, 0};
        ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(xv, wv, ci, 0, 0, 0);
        const uint64_t w64 = (static_cast<uint64_t>(Mh[i]) << 32) | Ml[i];
        const uint32_t h = has ? static_cast<uint32_t>(w64 >> (16 * sp.qs)) & 0xffffu : 0u;
        const float d = half_to_float(h);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(static_cast<float>(ci[r]), d, acc[r]);
    }
}

template <int NB>
__global__ __launch_bounds__(kWaveSize * kMfmaSplitMaxWaves) void mfma_q4_split_kernel(MfmaArgs a) {
    const MfmaTok tk = mfma_tok(a);
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = threadIdx.x % kWaveSize;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
    const uint32_t KS = 1u << a.ks_log2;
    const uint32_t b1 = a.job_block[1], b2 = a.job_block[2], b3 = a.job_block[3];
    uint32_t job = (blockIdx.x >= b1 ? 1u : 0u) + (blockIdx.x >= b2 ? 1u : 0u) + (blockIdx.x >= b3 ? 1u : 0u);
    job = __builtin_amdgcn_readfirstlane(job);
    const uint8_t *payload = job == 0 ? a.payload[0] : job == 1 ? a.payload[1] : job == 2 ? a.payload[2] : a.payload[3];
    const uint8_t *meta = job == 0 ? a.meta[0] : job == 1 ? a.meta[1] : job == 2 ? a.meta[2] : a.meta[3];
    float *output = job == 0 ? a.output[0] : job == 1 ? a.output[1] : job == 2 ? a.output[2] : a.output[3];
    const uint32_t rows = job == 0 ? a.rows[0] : job == 1 ? a.rows[1] : job == 2 ? a.rows[2] : a.rows[3];
    const uint32_t tiles = job == 0 ? a.tiles[0] : job == 1 ? a.tiles[1] : job == 2 ? a.tiles[2] : a.tiles[3];
    const uint32_t stride = job == 0   ? a.output_stride[0]
                            : job == 1 ? a.output_stride[1]
                            : job == 2 ? a.output_stride[2]
                                       : a.output_stride[3];
    output += static_cast<size_t>(tk.tok0) * stride;  // this launch's token group
    const uint32_t first = job == 0 ? 0u : job == 1 ? b1 : job == 2 ? b2 : b3;
    const float *bias = job == 0 ? a.bias[0] : job == 1 ? a.bias[1] : job == 2 ? a.bias[2] : a.bias[3];
    const uint32_t local = blockIdx.x - first;
    const uint32_t R = 1u << a.rows_per_wave_log2, L = 1u << a.lanes_log2;
    Q4Split sp;
    sp.qs = local & 3u;
    const uint32_t r0 = (local >> 2) * 16;
    const uint32_t t0 = r0 >> a.rows_per_wave_log2;
    // the row group's chunk qs of every unit, row-major, then its meta; the
    // lane order fixes the LDS destination, so each lane computes its
    // piece's source (padding pieces and rows past the tensor's tiles copy
    // the tile start: never read, or read with scale 0)
    const uint32_t ntile = min(16u >> a.rows_per_wave_log2, tiles - t0);
    sp.pst = a.units | 1u;
    sp.mst = q4_meta_stride(a.units);
    sp.meta_lds = 16 * 16 * sp.pst;
    const uint8_t *psrc = payload + static_cast<size_t>(t0) * a.tile_payload_bytes;
    const uint8_t *msrc = meta + static_cast<size_t>(t0) * a.tile_meta_bytes;
    for (uint32_t c0 = wave * kWaveSize; c0 < 16 * sp.pst; c0 += blockDim.x) {
        const uint32_t pc = c0 + lane, rr = pc / sp.pst, v = pc - rr * sp.pst;
        const uint32_t tl = rr >> a.rows_per_wave_log2, grp = rr & (R - 1);
        size_t src = 0;
        if (rr < 16 && v < a.units && tl < ntile) {
            const uint32_t slot = v >> a.lanes_log2, n = min(L, a.units - slot * L);
            src = static_cast<size_t>(tl) * a.tile_payload_bytes + static_cast<size_t>(64) * R * L * slot +
                  16 * (sp.qs * R * n + grp * n + (v & (L - 1)));
        }
        if (pc < 16 * sp.pst) __builtin_amdgcn_global_load_lds(psrc + src, (lds_void *)(smem + c0 * 16), 16, 0, 0);
    }
    for (uint32_t c0 = wave * kWaveSize; c0 < 16 * sp.mst; c0 += blockDim.x) {
        const uint32_t dw = c0 + lane, rr = dw / sp.mst, w = dw - rr * sp.mst;
        const uint32_t tl = rr >> a.rows_per_wave_log2, grp = rr & (R - 1), v = w >> 1;
        size_t src = 0;
        if (rr < 16 && v < a.units && tl < ntile) {
            const uint32_t slot = v >> a.lanes_log2, n = min(L, a.units - slot * L);
            src = static_cast<size_t>(tl) * a.tile_meta_bytes + static_cast<size_t>(8) * R * L * slot +
                  8 * (grp * n + (v & (L - 1))) + 4 * (w & 1);
        }
        if (dw < 16 * sp.mst)
            __builtin_amdgcn_global_load_lds(msrc + src, (lds_void *)(smem + sp.meta_lds + c0 * 4), 4, 0, 0);
    }
    wait_vmcnt<0>();               // this wave's copies landed
    __builtin_amdgcn_s_barrier();  // ... and every wave's
    __atomic_signal_fence(__ATOMIC_SEQ_CST);

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t v0 = wave * a.nb, v1 = min(a.units, v0 + a.nb);
    for (uint32_t v = v0; v < v1; v += NB)
        mfma_chunk_q4s<NB>(a, tk, smem, sp, rows, r0, v, min(static_cast<uint32_t>(NB), v1 - v), lane, acc);

    // the waves' partials, summed in wave order (LDS after the staged tiles)
    if (KS > 1) {
        float *part_s = reinterpret_cast<float *>(smem + a.stage_bytes);
        if (wave > 0) {
            float *dst = part_s + ((wave - 1) * kWaveSize + lane) * 4;
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r] = acc[r];
        }
        __syncthreads();
        if (wave == 0)
            for (uint32_t k = 1; k < KS; ++k) {
                const float *src = part_s + ((k - 1) * kWaveSize + lane) * 4;
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] += src[r];
            }
    }
    // lane (g, m) holds tokens 4g .. 4g+3 of row m: the split's rounded
    // partial product (and, split 0, the bias) added to the output
    const uint32_t g = lane >> 4, m = lane & 15, row = r0 + m;
    if (wave == 0 && row < rows) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = 4 * g + r;
            if (tok >= tk.ntok) continue;
            float v = mul_rounded(acc[r], tk.scales[tok]);
            if (bias && sp.qs == 0) v = add_rounded(v, bias[row]);
            unsafeAtomicAdd(output + static_cast<size_t>(tok) * stride + row, v);
        }
    }
}

// Q4_0 tensors with an MFMA-order copy: a unit (four 32-weight blocks) of
// 16 rows is one contiguous 1 KB, 16 bytes per lane (g, m): word q holds
// lane g's four bytes of row m's block 4u + q (its eight K positions: low
// nibbles 4g .. 4g+3, high 16+4g .. 16+4g+3), so one load feeds the unit's
// four MFMAs; the row's four block scales are one 8-byte load.  Each wave
// loads a chunk of units straight from HBM, then multiplies.  SPLIT: the
// residual adds over few row groups, each row group split four ways by
// unit range, the partials added with float atomics (in no fixed order);
// otherwise mfma_gemm_kernel's single pass, the waves' partials summed in
// wave order.  payload[i] / meta[i] of the arguments are the copies; a.nb
// is units per wave.
template <int NB, bool SPLIT, bool DUMP, bool PAIR = false>
__global__ __launch_bounds__(kWaveSize * kMfmaMaxWaves) void mfma_q4_direct_kernel(MfmaArgs a) {
    const MfmaTok tk = mfma_tok(a);
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = threadIdx.x % kWaveSize;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
    const uint32_t KS = 1u << a.ks_log2;
    static_assert(!PAIR || (!SPLIT && !DUMP), "gate/up pairs: plain stores");
    // PAIR (the SwiGLU of a gate/up pair): waves [0, KS) take the gate rows
    // of the row group, waves [KS, 2 KS) the same up rows; wj is a wave's
    // index within its job
    const uint32_t wj = PAIR && wave >= KS ? wave - KS : wave;
    const uint32_t b1 = a.job_block[1], b2 = a.job_block[2], b3 = a.job_block[3];
    uint32_t job = (blockIdx.x >= b1 ? 1u : 0u) + (blockIdx.x >= b2 ? 1u : 0u) + (blockIdx.x >= b3 ? 1u : 0u);
    job = __builtin_amdgcn_readfirstlane(job);
    if constexpr (PAIR) job = wave >= KS ? 1u : 0u;
    const uint8_t *payload = job == 0 ? a.payload[0] : job == 1 ? a.payload[1] : job == 2 ? a.payload[2] : a.payload[3];
    const uint8_t *meta = job == 0 ? a.meta[0] : job == 1 ? a.meta[1] : job == 2 ? a.meta[2] : a.meta[3];
    float *output = job == 0 ? a.output[0] : job == 1 ? a.output[1] : job == 2 ? a.output[2] : a.output[3];
    const uint32_t rows = job == 0 ? a.rows[0] : job == 1 ? a.rows[1] : job == 2 ? a.rows[2] : a.rows[3];
    const uint32_t stride = job == 0   ? a.output_stride[0]
                            : job == 1 ? a.output_stride[1]
                            : job == 2 ? a.output_stride[2]
                                       : a.output_stride[3];
    output += static_cast<size_t>(tk.tok0) * stride;  // this launch's token group
    const uint32_t first = job == 0 ? 0u : job == 1 ? b1 : job == 2 ? b2 : b3;
    const float *bias = job == 0 ? a.bias[0] : job == 1 ? a.bias[1] : job == 2 ? a.bias[2] : a.bias[3];
    const uint32_t local = PAIR ? blockIdx.x : blockIdx.x - first;
    const uint32_t qs = SPLIT ? (local & 3u) : 0u, rg = SPLIT ? (local >> 2) : local, r0 = rg * 16;
    const uint32_t g = lane >> 4, m = lane & 15, row = r0 + m;
    // this workgroup's units (SPLIT: quarter qs of the row's), then the wave's
    const uint32_t per_split = SPLIT ? (a.units + 3) / 4 : a.units;
    const uint32_t s0 = min(a.units, qs * per_split), s1 = min(a.units, s0 + per_split);
    const uint32_t v0 = min(s1, s0 + wj * a.nb), v1 = min(s1, v0 + a.nb);
    float xs_pre[4], res_pre[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) xs_pre[r] = tk.scales[min(4 * g + r, tk.ntok - 1)];
    if (!SPLIT && a.accumulate && wj == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = 4 * g + r;
            res_pre[r] = tok < tk.ntok && row < rows ? output[static_cast<size_t>(tok) * stride + row] : 0.0f;
        }
    }
    const uint8_t *pbase = payload + static_cast<size_t>(rg) * a.units * 1024 + lane * 16;
    const uint8_t *mbase = meta + static_cast<size_t>(rg) * a.units * 128 + m * 8;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // one chunk of the wave's units from c0; the first is issued outside the
    // loop, so the loop header's wait for every load in flight does not
    // hold the first weight loads behind the epilogue's early loads
    auto chunk = [&](uint32_t c0) {
        const uint32_t nv = min(static_cast<uint32_t>(NB), v1 - c0);
        uint4 A[NB];
        uint2 Mt[NB], X[NB][4];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const uint32_t u = c0 + (static_cast<uint32_t>(i) < nv ? i : 0);
            A[i] = *reinterpret_cast<const uint4 *>(pbase + static_cast<size_t>(u) * 1024);
            Mt[i] = *reinterpret_cast<const uint2 *>(mbase + static_cast<size_t>(u) * 128);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // blocks past K (the last unit's padding) read the last block
                // and are skipped below
                const uint32_t b = min(4 * u + q, a.nblk - 1);
                X[i][q] = *reinterpret_cast<const uint2 *>(tk.image + static_cast<size_t>(b) * 512 + lane * 8);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (static_cast<uint32_t>(i) >= nv) break;
            const uint32_t u = c0 + i;
            const uint32_t cw[4] = {A[i].x, A[i].y, A[i].z, A[i].w};
            const uint32_t dw[2] = {Mt[i].x, Mt[i].y};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t b = 4 * u + q;
                if (b >= a.nblk) break;
                const long xv = static_cast<long>((static_cast<uint64_t>(X[i][q].y) << 32) | X[i][q].x);
                const uint32_t lo = q4_signed(cw[q] & 0x0f0f0f0fu), hi = q4_signed((cw[q] >> 4) & 0x0f0f0f0fu);
                const long wv = static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
                mfma_v4i ci = {0, 0, 0, 0};
                // C[token][row]: element r is token 4g + r of row m
                ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(xv, wv, ci, 0, 0, 0);
                if constexpr (DUMP) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t tok = 4 * g + r;
                        if (row < rows && tok < tk.ntok) a.dump[(static_cast<size_t>(tok) * rows + row) * a.nblk + b] = ci[r];
                    }
                }
                // rows past the matrix are zero in the copy: scale 0
                const float d = half_to_float((dw[q >> 1] >> (16 * (q & 1))) & 0xffffu);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] = fmaf(static_cast<float>(ci[r]), d, acc[r]);
            }
        }
    };
    if (v0 < v1) chunk(v0);
    for (uint32_t c0 = v0 + NB; c0 < v1; c0 += NB) chunk(c0);
    // the K-split partials, summed in wave order
    if (KS > 1) {
        // PAIR: each job's partials in its own region (a grouped launch's
        // other jobs are other workgroups)
        float *part_s = reinterpret_cast<float *>(smem) + (PAIR ? job : 0u) * (KS - 1) * kWaveSize * 4;
        if (wj > 0) {
            float *dst = part_s + ((wj - 1) * kWaveSize + lane) * 4;
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r] = acc[r];
        }
        __syncthreads();
        if (wj == 0)
            for (uint32_t k = 1; k < KS; ++k) {
                const float *src = part_s + ((k - 1) * kWaveSize + lane) * 4;
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] += src[r];
            }
    }
    if constexpr (PAIR) {
        // the up wave hands its rounded products over; the gate wave stores
        // silu(gate) * up, the arithmetic of the SwiGLU input transform
        float *up_s = reinterpret_cast<float *>(smem) + 2 * (KS - 1) * kWaveSize * 4;
        if (job == 1 && wj == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) up_s[lane * 4 + r] = mul_rounded(acc[r], xs_pre[r]);
        }
        __syncthreads();
        if (job == 0 && wj == 0 && r0 + m < rows) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tok = 4 * g + r;
                if (tok >= tk.ntok) continue;
                const float gv = mul_rounded(acc[r], xs_pre[r]), uv = up_s[lane * 4 + r];
                output[static_cast<size_t>(tok) * stride + r0 + m] = mul_rounded(gv / (1.0f + expf(-gv)), uv);
            }
        }
        return;
    }
    // lane (g, m) holds tokens 4g .. 4g+3 of row m
    if (wave == 0 && row < rows) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = 4 * g + r;
            if (tok >= tk.ntok) continue;
            float v = mul_rounded(acc[r], xs_pre[r]);
            if constexpr (SPLIT) {
                if (bias && qs == 0) v = add_rounded(v, bias[row]);
                unsafeAtomicAdd(output + static_cast<size_t>(tok) * stride + row, v);
            } else {
                if (bias) v = add_rounded(v, bias[row]);
                output[static_cast<size_t>(tok) * stride + row] = a.accumulate ? add_rounded(res_pre[r], v) : v;
            }
        }
    }
}

// Winner of the argmax partials: one workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void argmax_finish_kernel(const uint64_t *__restrict__ partials, uint32_t n,
                                                             int32_t *index_out) {
    __shared__ uint64_t red_key[1024 / kWaveSize];
    uint64_t key = 0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) key = partials[i] > key ? partials[i] : key;
    for (int off = kWaveSize / 2; off > 0; off >>= 1) {
        const uint64_t o = shfl_xor_u64(key, off);
        key = o > key ? o : key;
    }
    if (threadIdx.x % kWaveSize == 0) red_key[threadIdx.x / kWaveSize] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t best = red_key[0];
        for (uint32_t w = 1; w < blockDim.x / kWaveSize; ++w) best = red_key[w] > best ? red_key[w] : best;
        *index_out = best ? static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(best)) : 0;
    }
}

// Integer dump: one thread per (row, unit), token 0 only.  Same image and
// per-unit cores as gemv_kernel; used by the bit-exactness tests.
//   HyperVSQ-2: out[row][unit*8 + oct] = sum (code-1)*a
//   Q4_0:       out[row][block]       = sum (nibble-8)*a
template <int KIND>
__global__ __launch_bounds__(kGemvThreads) void dump_kernel(GemvArgs a, int32_t *out, uint32_t out_row) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.rows[0] * a.units) return;
    const uint32_t row = idx / a.units, u = idx % a.units;
    uint4 pay[4];
    for (uint32_t q = 0; q < 4; ++q) {
        const UnitAddr ad = unit_addr(row, u, q, a.lanes, a.rows_per_wave, a.units, a.tile_payload_bytes,
                                      a.tile_meta_bytes);
        pay[q] = *reinterpret_cast<const uint4 *>(a.payload[0] + ad.payload);
    }
    const uint8_t *img = a.image;
    const int32_t *sums = reinterpret_cast<const int32_t *>(img + a.units * unit_lds_bytes(KIND));
    if (KIND == kHvsq2) {
        const uint32_t *cw = reinterpret_cast<const uint32_t *>(pay);
        for (int o = 0; o < 8; ++o) {
            const uint4 *at = reinterpret_cast<const uint4 *>(img + u * 272 + o * 32);
            out[static_cast<size_t>(row) * out_row + u * 8 + o] =
                hv_octant_dot(cw[2 * o], cw[2 * o + 1], at[0], at[1]) - sums[u * 8 + o];
        }
    } else {
        for (int b = 0; b < 4; ++b) {
            if (u * 4 + b >= out_row) break;
            const uint4 *at = reinterpret_cast<const uint4 *>(img + u * 144 + b * 32);
            out[static_cast<size_t>(row) * out_row + u * 4 + b] =
                q4_block_dot(pay[b], at[0], at[1]) - sums[u * 4 + b];
        }
    }
}

// ---- repack: on-disk blocks -> wave-tile layout -----------------------------
// One thread per (row, unit); the destination was zero filled.

struct RepackArgs {
    const uint8_t *src;  // the on-disk blocks of rows [row0, row0 + rows)
    uint8_t *payload;
    uint8_t *meta;
    uint32_t row0, rows, cols, units, lanes, rows_per_wave;
    size_t tile_payload, tile_meta;
};

__device__ inline uint32_t load_u32_unaligned(const uint8_t *p) {
    return p[0] | (p[1] << 8) | (p[2] << 16) | (static_cast<uint32_t>(p[3]) << 24);
}

template <int KIND>
__global__ void repack_kernel(RepackArgs r) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<size_t>(r.rows) * r.units) return;
    const uint32_t lrow = idx / r.units, u = idx % r.units, row = r.row0 + lrow;
    UnitAddr ad[4];
    for (uint32_t q = 0; q < 4; ++q)
        ad[q] = unit_addr(row, u, q, r.lanes, r.rows_per_wave, r.units, r.tile_payload, r.tile_meta);
    if (KIND == kHvsq2) {
        const uint8_t *blk = r.src + idx * 74;  // [row][unit] blocks, unit == block
        for (uint32_t q = 0; q < 4; ++q) {
            uint4 v;
            v.x = load_u32_unaligned(blk + 10 + 16 * q);
            v.y = load_u32_unaligned(blk + 14 + 16 * q);
            v.z = load_u32_unaligned(blk + 18 + 16 * q);
            v.w = load_u32_unaligned(blk + 22 + 16 * q);
            *reinterpret_cast<uint4 *>(r.payload + ad[q].payload) = v;
        }
        *reinterpret_cast<uint2 *>(r.meta + ad[0].meta) =
            make_uint2(load_u32_unaligned(blk), load_u32_unaligned(blk + 4));
    } else if (KIND == kQ4_0) {
        const uint32_t nb = (r.cols + 31) / 32;
        uint32_t sc[2] = {0, 0};
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t b = u * 4 + q;
            if (b >= nb) break;
            const uint8_t *blk = r.src + (static_cast<size_t>(lrow) * nb + b) * 18;
            uint4 v;
            v.x = load_u32_unaligned(blk + 2);
            v.y = load_u32_unaligned(blk + 6);
            v.z = load_u32_unaligned(blk + 10);
            v.w = load_u32_unaligned(blk + 14);
            *reinterpret_cast<uint4 *>(r.payload + ad[q].payload) = v;
            sc[q >> 1] |= static_cast<uint32_t>(blk[0] | (blk[1] << 8)) << (16 * (q & 1));
        }
        *reinterpret_cast<uint2 *>(r.meta + ad[0].meta) = make_uint2(sc[0], sc[1]);
    } else {
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t k0 = u * 32 + q * 8;
            uint32_t h[4] = {0, 0, 0, 0};
            if (k0 < r.cols) {
                const uint8_t *src = r.src + (static_cast<size_t>(lrow) * r.cols + k0) * 2;
                const uint32_t n = min(8u, r.cols - k0);
                for (uint32_t i = 0; i < n; ++i)
                    h[i >> 1] |= static_cast<uint32_t>(src[2 * i] | (src[2 * i + 1] << 8)) << (16 * (i & 1));
            }
            *reinterpret_cast<uint4 *>(r.payload + ad[q].payload) = make_uint4(h[0], h[1], h[2], h[3]);
        }
    }
}

template <int KIND, int UPL, bool PT>
hipError_t launch_fused(uint32_t grid, uint32_t threads, size_t lds, const GemvArgs &args, hipStream_t stream) {
    // as few sub-blocks per thread as the workgroup allows
    const uint32_t nsub = args.units * unit_elems(KIND) / fused_sub_elems(KIND);
    const uint32_t per_thread = (nsub + threads - 1) / threads;
    if (per_thread <= 1)
        hipLaunchKernelGGL((gemv_kernel<KIND, 1, UPL, 1, PT>), dim3(grid), dim3(threads), lds, stream, args);
    else if (per_thread <= 2)
        hipLaunchKernelGGL((gemv_kernel<KIND, 1, UPL, 2, PT>), dim3(grid), dim3(threads), lds, stream, args);
    else if constexpr (fused_sub_elems(KIND) == 8) {
        if (per_thread <= 3)
            hipLaunchKernelGGL((gemv_kernel<KIND, 1, UPL, 3, PT>), dim3(grid), dim3(threads), lds, stream, args);
        else
            hipLaunchKernelGGL((gemv_kernel<KIND, 1, UPL, 4, PT>), dim3(grid), dim3(threads), lds, stream, args);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int KIND, int MT, int UPL>
hipError_t launch_one(uint32_t grid, uint32_t threads, size_t lds, const GemvArgs &args, int tpw,
                      hipStream_t stream) {
    if constexpr (MT == 1) {
        if (args.input_mode != kInImage) {
            // two tiles per wave: the one-unit layout run two units per lane
            if constexpr (UPL == 1 && KIND != kF16)
                if (tpw == 2) return launch_fused<KIND, 2, true>(grid, threads, lds, args, stream);
            if (tpw != 1) return hipErrorInvalidValue;
            return launch_fused<KIND, UPL, false>(grid, threads, lds, args, stream);
        }
    }
    if (tpw != 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_kernel<KIND, MT, UPL, 0>), dim3(grid), dim3(threads), lds, stream, args);
    return hipGetLastError();
}

template <int KIND, int MT>
hipError_t dispatch_upl(uint32_t grid, uint32_t threads, size_t lds, const GemvArgs &args, int upl, int tpw,
                        hipStream_t stream) {
    switch (upl) {
    case 1: return launch_one<KIND, MT, 1>(grid, threads, lds, args, tpw, stream);
    case 2: return launch_one<KIND, MT, 2>(grid, threads, lds, args, tpw, stream);
    case 3: return launch_one<KIND, MT, 3>(grid, threads, lds, args, tpw, stream);
    case 4: return launch_one<KIND, MT, 4>(grid, threads, lds, args, tpw, stream);
    case 5: return launch_one<KIND, MT, 5>(grid, threads, lds, args, tpw, stream);
    case 6: return launch_one<KIND, MT, 6>(grid, threads, lds, args, tpw, stream);
    case 8: return launch_one<KIND, MT, 8>(grid, threads, lds, args, tpw, stream);
    case 10: return launch_one<KIND, MT, 10>(grid, threads, lds, args, tpw, stream);
    case 12: return launch_one<KIND, MT, 12>(grid, threads, lds, args, tpw, stream);
    case 16: return launch_one<KIND, MT, 16>(grid, threads, lds, args, tpw, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int KIND>
hipError_t dispatch_mt(int mt, uint32_t grid, uint32_t threads, size_t lds, const GemvArgs &args, int upl,
                       hipStream_t stream, int tpw = 1) {
    switch (mt) {
    case 1: return dispatch_upl<KIND, 1>(grid, threads, lds, args, upl, tpw, stream);
    case 2: return dispatch_upl<KIND, 2>(grid, threads, lds, args, upl, tpw, stream);
    case 4: return dispatch_upl<KIND, 4>(grid, threads, lds, args, upl, tpw, stream);
    case 8: return dispatch_upl<KIND, 8>(grid, threads, lds, args, upl, tpw, stream);
    case 16: return dispatch_upl<KIND, 16>(grid, threads, lds, args, upl, tpw, stream);
    default: return hipErrorInvalidValue;
    }
}

GemvArgs args_of(const DeviceTensor &t) {
    GemvArgs a{};
    a.payload[0] = t.payload;
    a.meta[0] = t.meta;
    a.rows[0] = t.rows;
    a.njobs = 1;
    a.tile_payload_bytes = t.tile_payload_bytes;
    a.tile_meta_bytes = t.tile_meta_bytes;
    a.units = t.units;
    a.lanes = t.lanes;
    a.lanes_log2 = static_cast<uint32_t>(__builtin_ctz(t.lanes));
    a.rows_per_wave = t.rows_per_wave;
    a.image_bytes = static_cast<uint32_t>(image_bytes(t.kind, t.units));
    a.cols = t.cols;
    a.scale = 1.0f;
    a.bf16 = t.bf16 ? 1u : 0u;
    return a;
}

constexpr int kUplWidths[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16};

bool set_units(DeviceTensor &t) {
    if (t.kind == kHvsq2) t.units = (t.cols + 255u) / 256u;
    else if (t.kind == kQ4_0) t.units = ((t.cols + 31u) / 32u + 3u) / 4u;
    else if (t.kind == kF16) t.units = (t.cols + 31u) / 32u;
    else return false;
    t.chunks = 4;
    return true;
}

}  // namespace

// The gaps of the staged HyperVSQ-2 layout (hv_lds_pieces) for a tile
// shape, found by laying out a wave's operand reads of every unit of a row
// group: the payload gap with the fewest 16-byte reads per 16-byte bank
// group (ds_read_b128 over 64 lanes: 4 at best), summed over the units, and
// the meta gap with the fewest distinct 8-byte words per 8-byte bank pair
// (16 rows, the four lane groups reading the same words).
static void hv_stage_pads(DeviceTensor &t) {
    t.stage_pad_p = t.stage_pad_m = 0;
    const uint32_t L = t.lanes, R = t.rows_per_wave, units = t.units;
    if (t.kind != kHvsq2 || R == 0 || 16 % R != 0) return;
    const uint32_t last = (units - 1) / L, nlast = units - last * L;
    const uint32_t tq = static_cast<uint32_t>(t.tile_payload_bytes / 16), tmb = static_cast<uint32_t>(t.tile_meta_bytes);
    uint64_t best_p = ~0ull, best_m = ~0ull;
    for (uint32_t pad = 0; pad < 16; ++pad) {
        uint64_t cost_p = 0, cost_m = 0;
        for (uint32_t b = 0; b < units; ++b) {
            const uint32_t slot = b / L, jj = b % L, n = slot == last ? nlast : L;
            uint32_t cnt[16] = {};
            uint32_t words[16], nwords = 0;
            for (uint32_t lane = 0; lane < 64; ++lane) {
                const uint32_t g = lane >> 4, m = lane & 15, tl = m / R, grp = m % R;
                const uint32_t q = tl * tq + (g * R + grp) * n + 4 * R * L * slot + jj;
                ++cnt[(q + (q >> 6) * pad) & 15u];
                if (g == 0) {
                    const uint32_t mb = tl * tmb + 8 * R * L * slot + 8 * (grp * n + jj), mq = mb >> 4;
                    words[nwords++] = (16 * (mq + (mq >> 6) * pad) + (mb & 8u)) / 8;
                }
            }
            uint32_t worst = 0;
            for (uint32_t c : cnt) worst = std::max(worst, c);
            cost_p += worst;
            uint32_t per[32] = {};
            for (uint32_t i = 0; i < nwords; ++i) {
                bool seen = false;
                for (uint32_t j = 0; j < i; ++j) seen |= words[j] == words[i];
                if (!seen) ++per[words[i] & 31u];
            }
            uint32_t wm = 0;
            for (uint32_t c : per) wm = std::max(wm, c);
            cost_m += wm;
        }
        if (cost_p < best_p) best_p = cost_p, t.stage_pad_p = pad;
        if (cost_m < best_m) best_m = cost_m, t.stage_pad_m = pad;
    }
}

bool layout_tensor_with(DeviceTensor &t, uint32_t lanes, uint32_t upl) {
    if (!set_units(t)) return false;
    bool upl_ok = false;
    for (int w : kUplWidths) upl_ok |= static_cast<uint32_t>(w) == upl;
    if (!upl_ok || lanes == 0 || lanes > 64 || (lanes & (lanes - 1)) || lanes * upl < t.units) return false;
    t.lanes = lanes;
    t.upl = upl;
    t.rows_per_wave = kWaveSize / lanes;
    t.tiles = (t.rows + t.rows_per_wave - 1) / t.rows_per_wave;
    // whole workgroups of tiles for every launch width, so a workgroup
    // never reads past the end
    t.tiles = (t.tiles + kTilePad - 1) / kTilePad * kTilePad;
    // compact tiles: only real units are stored (idle lanes load nothing new)
    t.tile_payload_bytes = static_cast<size_t>(t.rows_per_wave) * t.units * t.chunks * 16;
    t.tile_meta_bytes = t.kind == kF16 ? 0 : static_cast<size_t>(t.rows_per_wave) * t.units * 8;
    const size_t payload = t.tile_payload_bytes * t.tiles;
    const size_t meta = t.tile_meta_bytes * t.tiles;
    t.device_bytes = ((payload + 255) & ~static_cast<size_t>(255)) + meta;
    hv_stage_pads(t);
    return true;
}

// Lane plan: L lanes per row (a power of two, at most 64), one unit per
// lane for the quantized kinds, two for the FFN's expanding projections
// (gate and up: rows >= 3x columns, 8 units or more), about four for F16
// rows (the LM head).  A wave's dot products are one serial chain of about
// 160 VALU instructions per HyperVSQ-2 unit (60 per Q4_0 unit) that at
// decode grid sizes no other wave shares its SIMD with, so one unit per lane
// halves the chain of two: launches from a prebuilt image gain (Qwen3-4B
// HyperVSQ-2 q/k/v 3.54 -> 3.48 us, o 3.37 -> 3.14, down 4.59 -> 4.13).
// Fused one-token launches whose one-unit grid would exceed a workgroup per
// CU run such a tensor two units per lane over two tiles (paired tiles:
// q/k/v 4.81 -> 4.79 us, o at one unit 4.28 -> 3.99; down 6.81 -> 7.19, its
// row segments no longer line up with the cache lines).  Gate and up keep
// two units per lane: their paired-tile launches lost 0.12 (Qwen3-4B) and
// 0.38 us (Qwen2-1.5B) against the compact two-unit tiles.  Idle lanes cost
// VALU slots but no memory traffic (compact tiles).  q, k and v share the
// columns and have fewer rows than 3x the columns, so a grouped launch's
// tensors agree.
bool layout_tensor(DeviceTensor &t) {
    if (!set_units(t)) return false;
    const bool expanding = t.rows >= 3 * t.cols;
    const uint32_t per_lane = t.kind == kF16 ? 4 : (t.units >= 8 && expanding ? 2 : 1);
    const uint32_t target = (t.units + per_lane - 1) / per_lane;
    uint32_t L = 1;
    while (L < target && L < static_cast<uint32_t>(kWaveSize)) L *= 2;
    const uint32_t need = (t.units + L - 1) / L;
    for (int w : kUplWidths)
        if (static_cast<uint32_t>(w) >= need) return layout_tensor_with(t, L, static_cast<uint32_t>(w));
    return false;
}

GemvPlan plan_gemv(const DeviceTensor &t, int batch) {
    GemvPlan p;
    int mt = 1;
    const int want = std::min(batch, kMaxTokensPerLaunch);
    while (mt < want) mt *= 2;
    const size_t ib = image_bytes(t.kind, t.units);
    while (mt > 1 && ib * mt > kGemvLdsLimit) mt /= 2;
    p.tokens = mt;
    p.lds_bytes = ib * mt;
    p.grid = static_cast<int>(t.tiles / kGemvWaves);
    return p;
}

hipError_t clear_tensor(const DeviceTensor &t, hipStream_t stream) {
    return hipMemsetAsync(t.payload, 0, t.device_bytes, stream);
}

hipError_t repack_rows(const DeviceTensor &t, const uint8_t *src, uint32_t row0, uint32_t nrows,
                       hipStream_t stream) {
    if (row0 + nrows > t.rows || nrows == 0) return hipErrorInvalidValue;
    RepackArgs r{};
    r.src = src;
    r.payload = t.payload;
    r.meta = t.meta;
    r.row0 = row0;
    r.rows = nrows;
    r.cols = t.cols;
    r.units = t.units;
    r.lanes = t.lanes;
    r.rows_per_wave = t.rows_per_wave;
    r.tile_payload = t.tile_payload_bytes;
    r.tile_meta = t.tile_meta_bytes;
    const size_t n = static_cast<size_t>(nrows) * t.units;
    const dim3 grid((n + 255) / 256);
    if (t.kind == kHvsq2) hipLaunchKernelGGL(repack_kernel<kHvsq2>, grid, dim3(256), 0, stream, r);
    else if (t.kind == kQ4_0) hipLaunchKernelGGL(repack_kernel<kQ4_0>, grid, dim3(256), 0, stream, r);
    else hipLaunchKernelGGL(repack_kernel<kF16>, grid, dim3(256), 0, stream, r);
    return hipGetLastError();
}

hipError_t repack_tensor(const DeviceTensor &t, const uint8_t *staging, hipStream_t stream) {
    hipError_t e = clear_tensor(t, stream);
    if (e != hipSuccess) return e;
    return repack_rows(t, staging, 0, t.rows, stream);
}

hipError_t launch_image(const DeviceTensor &t, const void *x, uint32_t batch, uint32_t x_stride,
                        uint8_t *image, uint32_t image_stride, hipStream_t stream) {
    if (t.kind == kF16) {
        const dim3 grid((t.units * 4 + 255) / 256, batch);
        hipLaunchKernelGGL(image_from_f32_kernel, grid, dim3(256), 0, stream, static_cast<const float *>(x),
                           x_stride, t.cols, t.units, image, image_stride);
    } else {
        const uint32_t nblk = t.units * unit_elems(t.kind) / 32;
        const dim3 grid((nblk + 255) / 256, batch);
        if (t.kind == kHvsq2)
            hipLaunchKernelGGL(image_from_int8_kernel<kHvsq2>, grid, dim3(256), 0, stream,
                               static_cast<const int8_t *>(x), x_stride, t.cols, t.units, image, image_stride);
        else
            hipLaunchKernelGGL(image_from_int8_kernel<kQ4_0>, grid, dim3(256), 0, stream,
                               static_cast<const int8_t *>(x), x_stride, t.cols, t.units, image, image_stride);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_image(const DeviceTensor &t, const float *x, uint32_t batch, uint32_t x_stride,
                                 uint8_t *image, uint32_t image_stride, float *scales, int8_t *q8,
                                 uint32_t q8_stride, hipStream_t stream) {
    return launch_prepare_image(t, kInF32, x, nullptr, nullptr, 0.0f, batch, x_stride, image, image_stride, scales,
                                q8, q8_stride, stream);
}

hipError_t launch_prepare_image(const DeviceTensor &t, uint32_t mode, const float *x, const float *x2,
                                const float *norm, float eps, uint32_t batch, uint32_t x_stride, uint8_t *image,
                                uint32_t image_stride, float *scales, int8_t *q8, uint32_t q8_stride,
                                hipStream_t stream, uint8_t *mfma_image) {
    if (batch == 0 || mode > kInSwiglu || mode == kInImage || (mode == kInNorm && !norm) ||
        (mode == kInSwiglu && !x2) || (mfma_image && batch > static_cast<uint32_t>(kMfmaMaxBatch)))
        return hipErrorInvalidValue;
    const size_t mgroup = mfma_image ? mfma_image_bytes(t) : 0;
    const uint32_t staged = static_cast<size_t>(t.cols) * sizeof(float) <= kGemvLdsLimit ? 1u : 0u;
    const size_t lds = staged ? static_cast<size_t>(t.cols) * sizeof(float) : 0;
    if (t.kind != kHvsq2 && t.kind != kQ4_0) return hipErrorInvalidValue;
    // rows up to 4096 wide: 256 threads (the two reductions' barriers
    // synchronise four waves), else 1024
    const bool narrow = staged && t.cols <= 4096;
    const uint32_t nt = narrow ? 256u : 1024u;
    const uint32_t per = (t.cols + nt - 1) / nt;   // elements per thread (staged rows: at most 16)
    auto go = [&](auto kind_c, auto ept_c) {
        constexpr int KD = decltype(kind_c)::value, EP = decltype(ept_c)::value;
        if (narrow)
            hipLaunchKernelGGL((quantize_image_kernel<KD, EP, 256>), dim3(batch), dim3(256), lds, stream, x, t.cols,
                               x_stride, t.units, image, image_stride, scales, q8, q8_stride, mode, x2, norm, eps,
                               staged, mfma_image, mgroup);
        else
            hipLaunchKernelGGL((quantize_image_kernel<KD, EP, 1024>), dim3(batch), dim3(1024), lds, stream, x,
                               t.cols, x_stride, t.units, image, image_stride, scales, q8, q8_stride, mode, x2, norm,
                               eps, staged, mfma_image, mgroup);
    };
    auto by_ept = [&](auto kind_c) {
        if (!staged) go(kind_c, std::integral_constant<int, 0>{});
        else if (per <= 1) go(kind_c, std::integral_constant<int, 1>{});
        else if (per <= 2) go(kind_c, std::integral_constant<int, 2>{});
        else if (per <= 4) go(kind_c, std::integral_constant<int, 4>{});
        else if (per <= 6) go(kind_c, std::integral_constant<int, 6>{});
        else if (per <= 8) go(kind_c, std::integral_constant<int, 8>{});
        else if (per <= 10) go(kind_c, std::integral_constant<int, 10>{});
        else go(kind_c, std::integral_constant<int, 16>{});
    };
    if (t.kind == kHvsq2) by_ept(std::integral_constant<int, kHvsq2>{});
    else by_ept(std::integral_constant<int, kQ4_0>{});
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvLaunch &g, hipStream_t stream) {
    const DeviceTensor &t = *g.tensor;
    if (g.debug_sums) {
        if (t.kind == kF16) return hipErrorInvalidValue;
        GemvArgs args = args_of(t);
        args.image = static_cast<const uint8_t *>(g.image);
        args.image_stride = g.image_stride;
        const size_t n = static_cast<size_t>(t.rows) * t.units;
        const uint32_t out_row = t.kind == kHvsq2 ? t.units * 8 : (t.cols + 31) / 32;
        if (t.kind == kHvsq2)
            hipLaunchKernelGGL(dump_kernel<kHvsq2>, dim3((n + kGemvThreads - 1) / kGemvThreads),
                               dim3(kGemvThreads), 0, stream, args, g.debug_sums, out_row);
        else
            hipLaunchKernelGGL(dump_kernel<kQ4_0>, dim3((n + kGemvThreads - 1) / kGemvThreads),
                               dim3(kGemvThreads), 0, stream, args, g.debug_sums, out_row);
        return hipGetLastError();
    }
    GemvGroupLaunch gg;
    gg.njobs = 1;
    gg.tensors[0] = g.tensor;
    gg.outputs[0] = g.output;
    gg.image = g.image;
    gg.image_stride = g.image_stride;
    gg.scales = g.scales;
    gg.scale = g.scale;
    gg.batch = g.batch;
    gg.output_stride[0] = g.output_stride;
    return launch_gemv_group(gg, stream);
}

namespace {

// Tiles per wave: 2 (paired tiles) for a one-token fused launch on a
// one-unit-per-lane layout whose one-tile-per-wave grid would hold more
// workgroups than the chip has CUs (each workgroup repeats the
// RMSNorm/quantize prologue, so the extra workgroups cost more than the
// shorter dot chain saves: Qwen3-4B q/k/v 5.24 us at one tile per wave,
// 4.79 paired), else 1.
int choose_tpw(const GemvGroupLaunch &g, uint32_t total_tiles) {
    const DeviceTensor &t = *g.tensors[0];
    if (g.waves || g.input_mode == kInImage || g.batch != 1 || t.upl != 1 || t.lanes < 2 || t.kind == kF16)
        return 1;
    const int wmax = max_waves_for(1);
    const uint32_t nsub = t.units * unit_elems(t.kind) / fused_sub_elems(t.kind);
    int w = kGemvWaves;
    while (static_cast<uint32_t>(w) * kWaveSize < nsub && w < wmax) w *= 2;
    while (w < wmax && total_tiles / (2 * w) >= 512) w *= 2;
    return total_tiles / static_cast<uint32_t>(w) > kChipCus ? 2 : 1;
}

// Workgroup width: the fused prologue needs a thread per 32-block of the
// input (and runs shortest with a thread per sub-block); otherwise wider
// workgroups only when the grid stays >= 2 per CU.
int choose_waves(const GemvGroupLaunch &g, uint32_t total_tiles) {
    const DeviceTensor &t = *g.tensors[0];
    if (g.waves) return g.waves;
    total_tiles /= static_cast<uint32_t>(choose_tpw(g, total_tiles));
    const int wmax = max_waves_for(static_cast<int>(t.upl));
    const uint32_t nsub = t.units * unit_elems(t.kind) / fused_sub_elems(t.kind);
    int w = kGemvWaves;
    if (g.input_mode != kInImage)
        while (static_cast<uint32_t>(w) * kWaveSize < nsub && w < wmax) w *= 2;
    while (w < wmax && total_tiles / (2 * w) >= 512) w *= 2;
    return w;
}

bool group_valid(const GemvGroupLaunch &g) {
    if (g.njobs < 1 || g.njobs > kMaxGroup) return false;
    const DeviceTensor &t0 = *g.tensors[0];
    for (int i = 0; i < g.njobs; ++i) {
        if (!g.tensors[i] || !g.outputs[i]) return false;
        const DeviceTensor &t = *g.tensors[i];
        if (t.kind != t0.kind || t.bf16 != t0.bf16 || t.cols != t0.cols || t.units != t0.units ||
            t.lanes != t0.lanes || t.upl != t0.upl || t.rows_per_wave != t0.rows_per_wave)
            return false;
    }
    if (g.input_mode != kInImage) {
        if (g.batch != 1 || !g.x || t0.cols % 32 != 0) return false;
        if (g.input_mode == kInNorm && !g.norm) return false;
        if (g.input_mode == kInSwiglu && !g.x2) return false;
        if (t0.units * unit_elems(t0.kind) / 32 >
            static_cast<uint32_t>(kWaveSize * max_waves_for(static_cast<int>(t0.upl))))
            return false;
    } else if (!g.image) {
        return false;
    }
    if (g.output_mode == kOutArgmax && (g.batch != 1 || !g.argmax_partials || g.njobs != 1)) return false;
    if (g.output_mode == kOutArgmax || g.output_mode == kOutSwiglu)
        for (int i = 0; i < g.njobs; ++i)
            if (g.bias[i]) return false;
    if (g.output_mode == kOutSwiglu &&
        (g.batch != 1 || g.njobs != 2 || g.tensors[0]->rows != g.tensors[1]->rows))
        return false;
    return true;
}

}  // namespace

uint32_t gemv_group_grid(const GemvGroupLaunch &g) {
    if (!group_valid(g)) return 0;
    uint32_t tiles = 0;
    for (int i = 0; i < g.njobs; ++i) tiles += g.tensors[i]->tiles;
    const int w = choose_waves(g, tiles);
    return tiles / (w * choose_tpw(g, tiles));  // paired jobs: tiles of one job / (w / 2), the same
}

hipError_t launch_gemv_group(const GemvGroupLaunch &g, hipStream_t stream) {
    if (!group_valid(g)) return hipErrorInvalidValue;
    const DeviceTensor &t = *g.tensors[0];
    GemvArgs args = args_of(t);
    uint32_t tiles = 0;
    for (int i = 0; i < g.njobs; ++i) tiles += g.tensors[i]->tiles;
    const int w = choose_waves(g, tiles);
    const int tpw = choose_tpw(g, tiles);
    if ((w != 4 && w != 8) || w > max_waves_for(static_cast<int>(t.upl) * tpw)) return hipErrorInvalidValue;
    args.njobs = static_cast<uint32_t>(g.njobs);
    uint32_t blk = 0;
    for (int i = 0; i < g.njobs; ++i) {
        const DeviceTensor &ti = *g.tensors[i];
        if (ti.tiles % (w * tpw)) return hipErrorInvalidValue;
        args.payload[i] = ti.payload;
        args.meta[i] = ti.meta;
        args.output[i] = g.outputs[i];
        args.rows[i] = ti.rows;
        args.output_stride[i] = g.output_stride[i] ? g.output_stride[i] : ti.rows;
        args.bias[i] = g.bias[i];
        args.job_block[i] = blk;
        blk += ti.tiles / (w * tpw);
    }
    for (int i = g.njobs; i <= kMaxGroup; ++i) args.job_block[i] = blk;
    const uint32_t grid = blk;
    const uint32_t threads = static_cast<uint32_t>(w) * kWaveSize;
    args.input_mode = g.input_mode;
    args.output_mode = g.output_mode;
    args.argmax_partials = g.argmax_partials;
    if (g.input_mode != kInImage) {
        args.x = g.x;
        args.x2 = g.x2;
        args.norm = g.norm;
        args.eps = g.eps;
        args.scale_out = g.scale_out;
        args.ntok = 1;
        const size_t lds = image_bytes(t.kind, t.units);
        if (lds > kGemvLdsLimit) return hipErrorInvalidValue;
        if (t.kind == kHvsq2) return dispatch_mt<kHvsq2>(1, grid, threads, lds, args, t.upl, stream, tpw);
        if (t.kind == kQ4_0) return dispatch_mt<kQ4_0>(1, grid, threads, lds, args, t.upl, stream, tpw);
        return dispatch_mt<kF16>(1, grid, threads, lds, args, t.upl, stream, tpw);
    }
    const GemvPlan p = plan_gemv(t, static_cast<int>(g.batch));
    if (p.tokens == 0 || p.lds_bytes > kGemvLdsLimit) return hipErrorInvalidValue;
    for (uint32_t t0 = 0; t0 < g.batch; t0 += p.tokens) {
        args.ntok = std::min<uint32_t>(p.tokens, g.batch - t0);
        args.image = static_cast<const uint8_t *>(g.image) + static_cast<size_t>(t0) * g.image_stride;
        args.image_stride = g.image_stride;
        args.scales = g.scales ? g.scales + t0 : nullptr;
        args.scale = g.scale;
        for (int i = 0; i < g.njobs; ++i) args.output[i] = g.outputs[i] + static_cast<size_t>(t0) * args.output_stride[i];
        hipError_t e;
        if (t.kind == kHvsq2) e = dispatch_mt<kHvsq2>(p.tokens, grid, threads, p.lds_bytes, args, t.upl, stream);
        else if (t.kind == kQ4_0) e = dispatch_mt<kQ4_0>(p.tokens, grid, threads, p.lds_bytes, args, t.upl, stream);
        else e = dispatch_mt<kF16>(p.tokens, grid, threads, p.lds_bytes, args, t.upl, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// K steps of one MFMA block: HyperVSQ-2 256-weight blocks, Q4_0 32-weight blocks.
uint32_t mfma_steps(const DeviceTensor &t) { return t.kind == kQ4_0 ? (t.cols + 31) / 32 : t.units; }

size_t mfma_image_bytes(const DeviceTensor &t) {
    if (t.kind == kQ4_0) return static_cast<size_t>(mfma_steps(t)) * mfma_q4_image_block_bytes();
    return t.kind == kHvsq2 ? static_cast<size_t>(t.units) * mfma_image_block_bytes() : 0;
}

hipError_t launch_mfma_image(const DeviceTensor &t, const int8_t *q8, uint32_t batch, uint32_t q8_stride,
                             uint8_t *image, hipStream_t stream) {
    if ((t.kind != kHvsq2 && t.kind != kQ4_0) || batch == 0 || batch > static_cast<uint32_t>(kMfmaTokens))
        return hipErrorInvalidValue;
    if (t.kind == kQ4_0) {
        const uint32_t n = mfma_steps(t) * 64;
        hipLaunchKernelGGL(mfma_q4_image_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, q8, q8_stride, t.cols,
                           batch, mfma_steps(t), image);
        return hipGetLastError();
    }
    const uint32_t n = t.units * 256;
    hipLaunchKernelGGL(mfma_image_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, q8, q8_stride, t.cols, batch,
                       t.units, image);
    return hipGetLastError();
}

namespace {

// Launch shape of an MFMA GEMM over `total_rows` rows of K = units blocks:
// a workgroup per 16-row group (one row tile per wave measured faster than
// two or four sharing the image loads: more waves, shorter chains), its
// waves splitting the K blocks -- the fewest that keep a wave's blocks
// within the unrolled chunk of 5, then more (up to 8) while the launch has
// fewer than 4096 waves (Q4_0: 8192) and every wave keeps two blocks or
// more (the four-way K-split kernel of Q4_0 residual adds, up to 16).  STAGE
// where the row group is a whole number of wave tiles and they fit in LDS
// (kMfmaLdsLimit with the partial tiles).
struct MfmaPlan {
    int nbt = 0, rt = 1;
    bool stage = false;
    uint32_t ks_log2 = 0, nb = 0, waves = 0, stage_bytes = 0, lds_bytes = 0;
};

MfmaPlan mfma_plan(const DeviceTensor &t, uint64_t total_rows) {
    MfmaPlan p;
    // K steps, and the unrolled chunk: 5 HyperVSQ-2 blocks (four MFMAs
    // each), 8 Q4_0 blocks (one MFMA each)
    const uint32_t units = mfma_steps(t);
    const uint32_t chunk = t.kind == kQ4_0 ? 8 : 5;
    const uint64_t groups = (total_rows + 16 * p.rt - 1) / (16 * p.rt);
    auto per_wave = [&](uint32_t ks) { return (units + (1u << ks) - 1) >> ks; };
    if (t.kind == kQ4_0) {
        // as many K-split waves as keep the whole launch within one round of
        // resident waves (256 CUs x 32)
        while (p.ks_log2 < 3 && (groups << (p.ks_log2 + 1)) <= 8192 && per_wave(p.ks_log2 + 1) >= 2) ++p.ks_log2;
    } else {
        while (p.ks_log2 < 3 && per_wave(p.ks_log2) > chunk) ++p.ks_log2;
        while (p.ks_log2 < 3 && (groups << p.ks_log2) < 4096 && per_wave(p.ks_log2 + 1) >= 2) ++p.ks_log2;
    }
    p.nb = per_wave(p.ks_log2);
    p.nbt = p.nb <= 2 ? 2 : p.nb <= 3 ? 3 : (p.nb <= 5 || chunk == 5) ? 5 : 8;
    p.waves = 1u << p.ks_log2;
    const uint32_t part = (p.waves - 1) * kWaveSize * 4 * p.rt * 4;
    const uint32_t rows_grp = 16u * p.rt;
    // staging needs whole tiles in the row group (tiles of 32 or 64 rows
    // are never staged) and fits gfx950's 160 KB of LDS per workgroup
    // (HyperVSQ-2 meta copied in whole 16-byte pieces: an even number of
    // 8-byte entries per tile)
    const bool whole = rows_grp % t.rows_per_wave == 0 && (t.kind != kHvsq2 || t.tile_meta_bytes % 16 == 0);
    const uint64_t stage = !whole                ? 0
                           : t.kind == kQ4_0 ? q4_stage_bytes(t.units)
                                             : hv_stage_bytes(t.units, t.stage_pad_p, t.stage_pad_m);
    p.stage = whole && stage + part <= kMfmaLdsLimit;
    p.stage_bytes = p.stage ? static_cast<uint32_t>(stage) : 0;
    p.lds_bytes = p.stage_bytes + part;
    return p;
}

// 16-token groups of a launch (grid.y; each group its own MFMA image)
uint32_t mfma_groups(const MfmaArgs &a) { return (a.ntok + 15) / 16; }

template <int KIND, int NB, int RT>
hipError_t launch_mfma_rt(bool stage, uint32_t grid, uint32_t threads, size_t lds, const MfmaArgs &a,
                          hipStream_t stream) {
    if (a.dump) {
        if (stage)
            hipLaunchKernelGGL((mfma_gemm_kernel<KIND, NB, RT, true, true>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream, a);
        else
            hipLaunchKernelGGL((mfma_gemm_kernel<KIND, NB, RT, false, true>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream,
                               a);
    } else if (stage) {
        hipLaunchKernelGGL((mfma_gemm_kernel<KIND, NB, RT, true, false>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream, a);
    } else {
        hipLaunchKernelGGL((mfma_gemm_kernel<KIND, NB, RT, false, false>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream, a);
    }
    return hipGetLastError();
}

template <int KIND, int NB>
hipError_t launch_mfma_nb(const MfmaPlan &p, uint32_t grid, const MfmaArgs &a, hipStream_t stream) {
    return launch_mfma_rt<KIND, NB, 1>(p.stage, grid, p.waves * kWaveSize, p.lds_bytes, a, stream);
}

}  // namespace

size_t mfma_copy_bytes(const DeviceTensor &t) {
    if (t.kind != kHvsq2 && t.kind != kQ4_0) return 0;
    const size_t groups = (t.rows + 15) / 16;
    return groups * t.units * 1024 + groups * t.units * 128;
}

hipError_t launch_mfma_copy(const DeviceTensor &t, hipStream_t stream) {
    if ((t.kind != kHvsq2 && t.kind != kQ4_0) || !t.mfma_payload || !t.mfma_meta || !t.payload || !t.meta)
        return hipErrorInvalidValue;
    MfmaCopyArgs c{};
    c.payload = t.payload;
    c.meta = t.meta;
    c.dst_payload = t.mfma_payload;
    c.dst_meta = t.mfma_meta;
    c.tile_payload = t.tile_payload_bytes;
    c.tile_meta = t.tile_meta_bytes;
    c.units = t.units;
    c.lanes_log2 = static_cast<uint32_t>(__builtin_ctz(t.lanes));
    c.rows_per_wave_log2 = static_cast<uint32_t>(__builtin_ctz(t.rows_per_wave));
    c.tiles = t.tiles;
    c.groups = (t.rows + 15) / 16;
    c.q4 = t.kind == kQ4_0 ? 1u : 0u;
    const size_t n = static_cast<size_t>(c.groups) * t.units * 64;
    hipLaunchKernelGGL(mfma_copy_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream, c);
    return hipGetLastError();
}

hipError_t launch_gemm_mfma_group(const DeviceTensor *const *tensors, float *const *outputs, uint32_t count,
                                  const uint8_t *image, const float *scales, uint32_t batch,
                                  const uint32_t *output_strides, hipStream_t stream, bool accumulate,
                                  int32_t *dump, const float *const *biases, bool swiglu) {
    if ((dump && (count != 1 || batch > static_cast<uint32_t>(kMfmaTokens))) || count == 0 ||
        count > static_cast<uint32_t>(kMaxGroup) || !image || !scales || batch == 0 ||
        batch > static_cast<uint32_t>(kMfmaMaxBatch))
        return hipErrorInvalidValue;
    const DeviceTensor &t0 = *tensors[0];
    uint64_t total_rows = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const DeviceTensor &t = *tensors[i];
        if ((t.kind != kHvsq2 && t.kind != kQ4_0) || t.kind != t0.kind || t.cols != t0.cols ||
            t.units != t0.units || t.lanes != t0.lanes ||
            t.rows_per_wave != t0.rows_per_wave || t.tile_payload_bytes != t0.tile_payload_bytes ||
            t.tile_meta_bytes != t0.tile_meta_bytes || !outputs[i])
            return hipErrorInvalidValue;
        total_rows += t.rows;
    }
    MfmaPlan p = mfma_plan(t0, total_rows);
    // tensors that all carry the MFMA-order copy: direct loads
    bool direct = true;
    for (uint32_t i = 0; i < count; ++i) direct = direct && tensors[i]->mfma_payload && tensors[i]->mfma_meta;
    // a gate/up pair stored as silu(gate) * up into outputs[0]: direct
    // loads, plain stores, two tensors of equal rows
    if (swiglu && (!direct || count != 2 || accumulate || dump || tensors[1]->rows != t0.rows ||
                   (biases && (biases[0] || biases[1]))))
        return hipErrorInvalidValue;
    // residual adds over few row groups: the four-way K split
    const uint64_t groups = (total_rows + 15) / 16;
    const bool split = accumulate && !dump && groups < 256 && (direct || (t0.kind == kQ4_0 && p.stage));
    if (split && !direct) {
        const uint32_t units = t0.units;
        auto per_wave = [&](uint32_t ks) { return (units + (1u << ks) - 1) >> ks; };
        p.ks_log2 = 0;
        while (p.ks_log2 < 4 && ((4 * groups) << (p.ks_log2 + 1)) <= 8192 && per_wave(p.ks_log2 + 1) >= 2)
            ++p.ks_log2;
        p.nb = per_wave(p.ks_log2);
        p.nbt = p.nb <= 2 ? 2 : p.nb <= 3 ? 3 : p.nb <= 5 ? 5 : 8;
        p.waves = 1u << p.ks_log2;
        p.stage_bytes = 16 * 16 * (units | 1u) + 16 * 4 * q4_meta_stride(units);
        p.lds_bytes = p.stage_bytes + (p.waves - 1) * kWaveSize * 16;
        if (p.lds_bytes > kMfmaLdsLimit) return hipErrorInvalidValue;
    }
    MfmaArgs a{};
    uint32_t grid = 0;
    for (uint32_t i = 0; i < static_cast<uint32_t>(kMaxGroup); ++i) {
        a.job_block[i] = grid;
        if (i < count) {
            const DeviceTensor &t = *tensors[i];
            a.payload[i] = direct ? t.mfma_payload : t.payload;
            a.meta[i] = direct ? t.mfma_meta : t.meta;
            a.output[i] = outputs[i];
            a.rows[i] = t.rows;
            a.tiles[i] = t.tiles;
            a.output_stride[i] = output_strides && output_strides[i] ? output_strides[i] : t.rows;
            a.bias[i] = biases ? biases[i] : nullptr;
            if (a.output_stride[i] % 4 == 0 && (reinterpret_cast<uintptr_t>(outputs[i]) & 15u) == 0 &&
                (reinterpret_cast<uintptr_t>(a.bias[i]) & 15u) == 0)
                a.vec_out |= 1u << i;
            if (!swiglu || i == 0)
                grid += split ? 4 * ((t.rows + 15) / 16) : direct ? (t.rows + 15) / 16 : (t.rows + 16 * p.rt - 1) / (16 * p.rt);
        }
    }
    a.job_block[kMaxGroup] = grid;
    a.tile_payload_bytes = t0.tile_payload_bytes;
    a.tile_meta_bytes = t0.tile_meta_bytes;
    a.units = t0.units;
    a.nblk = mfma_steps(t0);
    a.lanes_log2 = static_cast<uint32_t>(__builtin_ctz(t0.lanes));
    a.rows_per_wave_log2 = static_cast<uint32_t>(__builtin_ctz(t0.rows_per_wave));
    a.ks_log2 = p.ks_log2;
    a.nb = p.nb;
    a.stage_bytes = p.stage_bytes;
    a.image = image;
    a.group_image_bytes = mfma_image_bytes(t0);
    a.scales = scales;
    a.ntok = batch;
    a.accumulate = accumulate ? 1u : 0u;
    a.dump = dump;
    a.pad_p = t0.stage_pad_p;
    a.pad_m = t0.stage_pad_m;
    if (direct && t0.kind == kQ4_0) {
        // the fewest waves (up to 8) that keep a wave's units (of the row's,
        // or of a split's quarter) within one unrolled chunk of 5
        const uint32_t span = split ? (t0.units + 3) / 4 : t0.units;
        auto per_wave = [&](uint32_t ks) { return (span + (1u << ks) - 1) >> ks; };
        p.ks_log2 = 0;
        // a pair runs both jobs' waves: at most 4 per job
        const uint32_t ks_max = swiglu ? 2u : 3u;
        while (p.ks_log2 < ks_max && per_wave(p.ks_log2) > 5) ++p.ks_log2;
        p.nb = per_wave(p.ks_log2);
        p.nbt = p.nb <= 2 ? 2 : p.nb <= 3 ? 3 : 5;
        p.waves = 1u << p.ks_log2;
        a.ks_log2 = p.ks_log2;
        a.nb = p.nb;
        const uint32_t jobs = swiglu ? 2u : 1u;
        const uint32_t threads = jobs * p.waves * kWaveSize;
        const size_t lds = static_cast<size_t>(jobs * (p.waves - 1) + (swiglu ? 1 : 0)) * kWaveSize * 16;
        if (jobs * p.waves > static_cast<uint32_t>(kMfmaMaxWaves)) return hipErrorInvalidValue;
#define QWN_Q4D(NBV, SP, DU) hipLaunchKernelGGL((mfma_q4_direct_kernel<NBV, SP, DU>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream, a)
#define QWN_Q4P(NBV) hipLaunchKernelGGL((mfma_q4_direct_kernel<NBV, false, false, true>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream, a)
        if (swiglu) {
            switch (p.nbt) {
            case 2: QWN_Q4P(2); break;
            case 3: QWN_Q4P(3); break;
            default: QWN_Q4P(5); break;
            }
        } else if (split) {
            switch (p.nbt) {
            case 2: QWN_Q4D(2, true, false); break;
            case 3: QWN_Q4D(3, true, false); break;
            default: QWN_Q4D(5, true, false); break;
            }
        } else if (dump) {
            switch (p.nbt) {
            case 2: QWN_Q4D(2, false, true); break;
            case 3: QWN_Q4D(3, false, true); break;
            default: QWN_Q4D(5, false, true); break;
            }
        } else {
            switch (p.nbt) {
            case 2: QWN_Q4D(2, false, false); break;
            case 3: QWN_Q4D(3, false, false); break;
            default: QWN_Q4D(5, false, false); break;
            }
        }
#undef QWN_Q4P
#undef QWN_Q4D
        return hipGetLastError();
    }
    if (direct) {
        // the fewest waves that keep a wave's units (of the row's, or of a
        // split's quarter) within one unrolled chunk of 5 (a wave's loads all
        // in flight at once)
        const uint32_t span = split ? (t0.units + 3) / 4 : t0.units;
        auto per_wave = [&](uint32_t ks) { return (span + (1u << ks) - 1) >> ks; };
        p.ks_log2 = 0;
        // a pair runs both jobs' waves: at most 4 per job
        const uint32_t ks_max = swiglu ? 2u : 3u;
        while (p.ks_log2 < ks_max && per_wave(p.ks_log2) > 5) ++p.ks_log2;
        p.nb = per_wave(p.ks_log2);
        p.nbt = p.nb <= 2 ? 2 : p.nb <= 3 ? 3 : 5;
        p.waves = 1u << p.ks_log2;
        a.ks_log2 = p.ks_log2;
        a.nb = p.nb;
        const uint32_t jobs = swiglu ? 2u : 1u;
        const uint32_t threads = jobs * p.waves * kWaveSize;
        const size_t lds = static_cast<size_t>(jobs * (p.waves - 1) + (swiglu ? 1 : 0)) * kWaveSize * 16;
        if (jobs * p.waves > static_cast<uint32_t>(kMfmaMaxWaves)) return hipErrorInvalidValue;
#define QWN_HVD(NBV, SP, DU) hipLaunchKernelGGL((mfma_direct_kernel<NBV, SP, DU>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream, a)
#define QWN_HVP(NBV) hipLaunchKernelGGL((mfma_direct_kernel<NBV, false, false, true>), dim3(grid, mfma_groups(a)), dim3(threads), lds, stream, a)
        if (swiglu) {
            switch (p.nbt) {
            case 2: QWN_HVP(2); break;
            case 3: QWN_HVP(3); break;
            default: QWN_HVP(5); break;
            }
        } else if (split) {
            switch (p.nbt) {
            case 2: QWN_HVD(2, true, false); break;
            case 3: QWN_HVD(3, true, false); break;
            default: QWN_HVD(5, true, false); break;
            }
        } else if (dump) {
            switch (p.nbt) {
            case 2: QWN_HVD(2, false, true); break;
            case 3: QWN_HVD(3, false, true); break;
            default: QWN_HVD(5, false, true); break;
            }
        } else {
            switch (p.nbt) {
            case 2: QWN_HVD(2, false, false); break;
            case 3: QWN_HVD(3, false, false); break;
            default: QWN_HVD(5, false, false); break;
            }
        }
#undef QWN_HVP
#undef QWN_HVD
        return hipGetLastError();
    }
    if (split) {
        const uint32_t threads = p.waves * kWaveSize;
        switch (p.nbt) {
        case 2: hipLaunchKernelGGL(mfma_q4_split_kernel<2>, dim3(grid, mfma_groups(a)), dim3(threads), p.lds_bytes, stream, a); break;
        case 3: hipLaunchKernelGGL(mfma_q4_split_kernel<3>, dim3(grid, mfma_groups(a)), dim3(threads), p.lds_bytes, stream, a); break;
        case 5: hipLaunchKernelGGL(mfma_q4_split_kernel<5>, dim3(grid, mfma_groups(a)), dim3(threads), p.lds_bytes, stream, a); break;
        default: hipLaunchKernelGGL(mfma_q4_split_kernel<8>, dim3(grid, mfma_groups(a)), dim3(threads), p.lds_bytes, stream, a); break;
        }
        return hipGetLastError();
    }
    if (t0.kind == kQ4_0) {
        switch (p.nbt) {
        case 2: return launch_mfma_nb<kQ4_0, 2>(p, grid, a, stream);
        case 3: return launch_mfma_nb<kQ4_0, 3>(p, grid, a, stream);
        case 5: return launch_mfma_nb<kQ4_0, 5>(p, grid, a, stream);
        default: return launch_mfma_nb<kQ4_0, 8>(p, grid, a, stream);
        }
    }
    switch (p.nbt) {
    case 2: return launch_mfma_nb<kHvsq2, 2>(p, grid, a, stream);
    case 3: return launch_mfma_nb<kHvsq2, 3>(p, grid, a, stream);
    default: return launch_mfma_nb<kHvsq2, 5>(p, grid, a, stream);
    }
}

hipError_t launch_gemm_mfma(const DeviceTensor &t, const uint8_t *image, const float *scales, float *output,
                            uint32_t batch, uint32_t output_stride, hipStream_t stream) {
    const DeviceTensor *ts[1] = {&t};
    float *outs[1] = {output};
    const uint32_t strides[1] = {output_stride};
    return launch_gemm_mfma_group(ts, outs, 1, image, scales, batch, strides, stream);
}

hipError_t launch_norm_image(const DeviceTensor &t, const float *x, const float *norm, float eps, uint8_t *image,
                             hipStream_t stream, uint32_t count, uint32_t x_stride, uint32_t image_stride) {
    if (t.kind != kF16 || count == 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(norm_image_kernel, dim3(count), dim3(1024), 0, stream, x, norm, t.cols, t.units, eps, image,
                       x_stride, image_stride);
    return hipGetLastError();
}

// First index of the largest value of each row of [rows][cols] fp32
// (c/qwanto_decode.c:2048-2065; NaN never wins), in two launches: each row
// split over `parts` workgroups of 256 threads, each reducing its slice to
// one key (float4 loads, four in flight per thread where the row allows),
// then one workgroup per row reducing the parts' keys.  A row of the
// 151936-entry vocabulary was one workgroup's 37 dependent load rounds.
__device__ __forceinline__ uint64_t max_key(uint64_t a, uint64_t b) { return a > b ? a : b; }

__global__ __launch_bounds__(256) void rows_argmax_part_kernel(const float *__restrict__ v, uint32_t cols,
                                                               uint32_t stride, uint32_t parts,
                                                               uint64_t *__restrict__ keys) {
    __shared__ uint64_t red[256 / kWaveSize];
    const uint32_t row = blockIdx.y, part = blockIdx.x;
    const float *r = v + static_cast<size_t>(row) * stride;
    const uint32_t span = (cols + parts - 1) / parts;
    const uint32_t c0 = part * span, c1 = min(cols, c0 + span);
    uint64_t key = 0;
    // vector loads only where the whole float4 lies in [c0, c1) and the row
    // start keeps them 16-byte aligned; the rest element by element
    const bool vec = (reinterpret_cast<uintptr_t>(r) & 15u) == 0;
    const uint32_t a0 = vec ? min(c1, (c0 + 3u) & ~3u) : c1;
    const uint32_t a1 = vec ? max(a0, c1 & ~3u) : c1;
    for (uint32_t i = c0 + threadIdx.x; i < a0; i += blockDim.x) key = max_key(key, argmax_key(r[i], i));
    for (uint32_t i = a1 + threadIdx.x; i < c1; i += blockDim.x) key = max_key(key, argmax_key(r[i], i));
    const float4 *r4 = reinterpret_cast<const float4 *>(r);
    const uint32_t q0 = a0 / 4, q1 = a1 / 4;
    uint32_t q = q0 + threadIdx.x;
    for (; q + 3 * blockDim.x < q1; q += 4 * blockDim.x) {
        float4 f[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) f[k] = r4[q + k * blockDim.x];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t e = 4 * (q + k * blockDim.x);
            key = max_key(key, max_key(max_key(argmax_key(f[k].x, e), argmax_key(f[k].y, e + 1)),
                                       max_key(argmax_key(f[k].z, e + 2), argmax_key(f[k].w, e + 3))));
        }
    }
    for (; q < q1; q += blockDim.x) {
        const float4 f = r4[q];
        const uint32_t e = 4 * q;
        key = max_key(key, max_key(max_key(argmax_key(f.x, e), argmax_key(f.y, e + 1)),
                                   max_key(argmax_key(f.z, e + 2), argmax_key(f.w, e + 3))));
    }
    for (int off = kWaveSize / 2; off > 0; off >>= 1) key = max_key(key, shfl_xor_u64(key, off));
    if (threadIdx.x % kWaveSize == 0) red[threadIdx.x / kWaveSize] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t best = red[0];
        for (uint32_t w = 1; w < blockDim.x / kWaveSize; ++w) best = max_key(best, red[w]);
        keys[static_cast<size_t>(row) * parts + part] = best;
    }
}

__global__ __launch_bounds__(64) void rows_argmax_finish_kernel(const uint64_t *__restrict__ keys, uint32_t parts,
                                                                int32_t *__restrict__ ids, int32_t *last_out) {
    const uint32_t row = blockIdx.x;
    uint64_t key = 0;
    for (uint32_t i = threadIdx.x; i < parts; i += blockDim.x) key = max_key(key, keys[static_cast<size_t>(row) * parts + i]);
    for (int off = kWaveSize / 2; off > 0; off >>= 1) key = max_key(key, shfl_xor_u64(key, off));
    if (threadIdx.x == 0) {
        const int32_t id = key ? static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(key)) : 0;
        ids[row] = id;
        if (last_out && row == gridDim.x - 1) *last_out = id;
    }
}

uint32_t rows_argmax_parts(uint32_t cols) { return std::min<uint32_t>(kRowsArgmaxMaxParts, (cols + 4095) / 4096); }

hipError_t launch_rows_argmax(const float *v, uint32_t rows, uint32_t cols, uint32_t stride, int32_t *ids,
                              int32_t *last_out, uint64_t *keys, hipStream_t stream) {
    if (rows == 0 || cols == 0 || !keys) return hipErrorInvalidValue;
    const uint32_t parts = rows_argmax_parts(cols);
    hipLaunchKernelGGL(rows_argmax_part_kernel, dim3(parts, rows), dim3(256), 0, stream, v, cols, stride, parts,
                       keys);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(rows_argmax_finish_kernel, dim3(rows), dim3(64), 0, stream, keys, parts, ids, last_out);
    return hipGetLastError();
}

hipError_t launch_argmax_finish(const uint64_t *partials, uint32_t n, int32_t *index_out, hipStream_t stream) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(1024), 0, stream, partials, n, index_out);
    return hipGetLastError();
}

}  // namespace qwn
