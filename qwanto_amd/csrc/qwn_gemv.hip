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

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int sdot8(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot8(static_cast<int>(a), static_cast<int>(b), c, false);
}
__device__ __forceinline__ int udot8(uint32_t a, uint32_t b, int c) {
    return static_cast<int>(__builtin_amdgcn_udot8(a, b, static_cast<uint32_t>(c), false));
}

// Sum over aligned groups of `lanes` consecutive lanes (a power of two);
// the total lands in the last lane of each group.  row_shr steps add the
// lanes 1, 2, 4, 8 below within each 16-lane row; row_bcast:15/31 carry
// row totals into the next row for groups of 32 and 64.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, true);
    return v + __builtin_bit_cast(float, moved);
}
__device__ __forceinline__ float group_sum(float v, uint32_t lanes) {
    if (lanes >= 2) v = dpp_add<0x111, 0xf>(v);   // row_shr:1
    if (lanes >= 4) v = dpp_add<0x112, 0xf>(v);   // row_shr:2
    if (lanes >= 8) v = dpp_add<0x114, 0xf>(v);   // row_shr:4
    if (lanes >= 16) v = dpp_add<0x118, 0xf>(v);  // row_shr:8
    if (lanes >= 32) v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    if (lanes >= 64) v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return v;
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

// Per-token int8 quantization (c/qwanto_kernels.c:354-433) fused with the
// image: x fp32 [M][x_stride] -> scales [M], image [M][image_stride] and,
// when q8 is given, the int8 token [M][q8_stride] zero padded.  grid (M).
template <int KIND>
__global__ __launch_bounds__(256) void quantize_image_kernel(const float *__restrict__ x, uint32_t K,
                                                             uint32_t x_stride, uint32_t units, uint8_t *image,
                                                             uint32_t image_stride, float *scales, int8_t *q8,
                                                             uint32_t q8_stride) {
    __shared__ float wave_max[256 / kWaveSize];
    const uint32_t t = blockIdx.x;
    const float *row = x + static_cast<size_t>(t) * x_stride;
    float amax = 0.0f;
    for (uint32_t k = threadIdx.x; k < K; k += blockDim.x) amax = fmaxf(amax, fabsf(row[k]));
    for (int off = kWaveSize / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (threadIdx.x % kWaveSize == 0) wave_max[threadIdx.x / kWaveSize] = amax;
    __syncthreads();
    amax = wave_max[0];
    for (uint32_t w = 1; w < blockDim.x / kWaveSize; ++w) amax = fmaxf(amax, wave_max[w]);
    // IEEE division and reciprocal, as the CPU path (c/qwanto_kernels.c:385-386)
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) scales[t] = scale;
    const uint32_t nblk = units * unit_elems(KIND) / 32;
    uint8_t *img = image ? image + static_cast<size_t>(t) * image_stride : nullptr;
    for (uint32_t b = threadIdx.x; b < nblk; b += blockDim.x) {
        uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t i = 0; i < 32; ++i) {
            const uint32_t k = b * 32 + i;
            if (k >= K) break;
            const float v = fminf(127.0f, fmaxf(-127.0f, row[k] * inv));
            const uint32_t q = static_cast<uint8_t>(static_cast<int8_t>(__builtin_rintf(v)));
            w[i >> 2] |= q << (8 * (i & 3));
        }
        if (image) put_block32<KIND>(img, units, b, w);
        if (q8) {
            int8_t *dst = q8 + static_cast<size_t>(t) * q8_stride;
            for (uint32_t i = 0; i < 32 && b * 32 + i < q8_stride; ++i)
                dst[b * 32 + i] = static_cast<int8_t>((w[i >> 2] >> (8 * (i & 3))) & 0xffu);
        }
    }
    if (q8)
        for (uint32_t k = nblk * 32 + threadIdx.x; k < q8_stride; k += blockDim.x)
            q8[static_cast<size_t>(t) * q8_stride + k] = 0;
}

// Copy `ntok` token images (global stride `stride`, `bytes` each, a
// multiple of 16) into LDS back to back, one 16-byte direct load per lane;
// returns after issuing (the caller waits).
__device__ __forceinline__ void issue_image_copy(const uint8_t *__restrict__ image, uint32_t stride,
                                                 uint32_t bytes, uint32_t ntok, uint8_t *lds) {
    const uint32_t per_tok = bytes / 16;
    const uint32_t total = per_tok * ntok;
    const uint32_t lane = threadIdx.x % kWaveSize;
    for (uint32_t c0 = (threadIdx.x / kWaveSize) * kWaveSize; c0 < total; c0 += blockDim.x) {
        const uint32_t c = c0 + lane;
        if (c < total) {
            const uint32_t t = c / per_tok, r = c - t * per_tok;
            __builtin_amdgcn_global_load_lds(image + static_cast<size_t>(t) * stride + r * 16,
                                             (lds_void *)(lds + c0 * 16), 16, 0, 0);
        }
    }
}

// s_waitcnt vmcnt(n) (n <= 63), expcnt and lgkmcnt left alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    constexpr int n = N > 63 ? 63 : N;
    __builtin_amdgcn_s_waitcnt((n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8));
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
    const uint8_t *payload;
    const uint8_t *meta;
    size_t tile_payload_bytes;
    size_t tile_meta_bytes;
    const uint8_t *image;
    const float *scales;
    float scale;
    float *output;
    uint32_t rows;
    uint32_t units;
    uint32_t lanes;
    uint32_t rows_per_wave;
    uint32_t ntok;
    uint32_t image_stride;
    uint32_t image_bytes;
    uint32_t output_stride;
};

template <int KIND, int MT, int UPL>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int CH = 4;
    const uint32_t lane = threadIdx.x % kWaveSize;
    const uint32_t wave = threadIdx.x / kWaveSize;
    const uint32_t L = a.lanes;
    const uint32_t grp = lane / L;
    const uint32_t j = lane - grp * L;
    const uint32_t tile = blockIdx.x * kGemvWaves + wave;
    const uint32_t row = tile * a.rows_per_wave + grp;
    const bool active = grp < a.rows_per_wave && row < a.rows;

    // 0. Token scales (uniform loads, needed only at the very end but
    //    issued first so their latency hides under the weight stream), then
    //    the activation images -> LDS (direct loads).
    float tok_scale[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) tok_scale[t] = a.scales ? a.scales[t < static_cast<int>(a.ntok) ? t : 0] : a.scale;
    issue_image_copy(a.image, a.image_stride, a.image_bytes, a.ntok, smem);
    __builtin_amdgcn_sched_barrier(0);

    // 1. Every weight load of this lane, metadata before codes.  Lanes
    //    without a unit load from the tile start instead of branching, so
    //    the loads stay one unconditional burst.
    const uint8_t *tile_p = a.payload + tile * a.tile_payload_bytes;
    const uint8_t *tile_m = a.meta + tile * a.tile_meta_bytes;
    // Unit slot i holds units i*L + j, n = min(L, units - i*L) of them,
    // stored compactly (qwn_internal.h).
    const size_t R = a.rows_per_wave;
    uint2 met[UPL];
    uint4 pay[UPL][CH];
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
    __builtin_amdgcn_sched_barrier(0);

    // 2. Wait for this wave's image loads only (vector memory loads retire
    //    in issue order), then for every wave's share of the copy.  A bare
    //    s_barrier: __syncthreads() would also wait for the weight loads.
    wait_vmcnt<(KIND == kF16 ? 4 : 5) * UPL>();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // 3. Dot products.
    const uint32_t ib = a.image_bytes;
    const uint32_t act_bytes = a.units * unit_lds_bytes(KIND);
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
                for (int b = 0; b < 4; ++b) {
                    const float d = half_to_float(sc[b >> 1] >> (16 * (b & 1)));
                    const int raw = q4_block_dot(pay[i][b], at[2 * b], at[2 * b + 1]) - cb[b];
                    acc[t] = fmaf(static_cast<float>(raw), d, acc[t]);
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t h[4] = {pay[i][q].x, pay[i][q].y, pay[i][q].z, pay[i][q].w};
                float wf[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    wf[2 * k] = half_to_float(h[k] & 0xffffu);
                    wf[2 * k + 1] = half_to_float(h[k] >> 16);
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
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = group_sum(acc[t], L);
    if (active && j == L - 1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (static_cast<uint32_t>(t) >= a.ntok) break;
            float s = acc[t];
            if (KIND != kF16) s *= tok_scale[t];
            a.output[static_cast<size_t>(t) * a.output_stride + row] = s;
        }
    }
}

// Integer dump: one thread per (row, unit), token 0 only.  Same image and
// per-unit cores as gemv_kernel; used by the bit-exactness tests.
//   HyperVSQ-2: out[row][unit*8 + oct] = sum (code-1)*a
//   Q4_0:       out[row][block]       = sum (nibble-8)*a
template <int KIND>
__global__ __launch_bounds__(kGemvThreads) void dump_kernel(GemvArgs a, int32_t *out, uint32_t out_row) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.rows * a.units) return;
    const uint32_t row = idx / a.units, u = idx % a.units;
    uint4 pay[4];
    for (uint32_t q = 0; q < 4; ++q) {
        const UnitAddr ad = unit_addr(row, u, q, a.lanes, a.rows_per_wave, a.units, a.tile_payload_bytes,
                                      a.tile_meta_bytes);
        pay[q] = *reinterpret_cast<const uint4 *>(a.payload + ad.payload);
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
    const uint8_t *src;
    uint8_t *payload;
    uint8_t *meta;
    uint32_t rows, cols, units, lanes, rows_per_wave;
    size_t tile_payload, tile_meta;
};

__device__ inline uint32_t load_u32_unaligned(const uint8_t *p) {
    return p[0] | (p[1] << 8) | (p[2] << 16) | (static_cast<uint32_t>(p[3]) << 24);
}

template <int KIND>
__global__ void repack_kernel(RepackArgs r) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<size_t>(r.rows) * r.units) return;
    const uint32_t row = idx / r.units, u = idx % r.units;
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
            const uint8_t *blk = r.src + (static_cast<size_t>(row) * nb + b) * 18;
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
                const uint8_t *src = r.src + (static_cast<size_t>(row) * r.cols + k0) * 2;
                const uint32_t n = min(8u, r.cols - k0);
                for (uint32_t i = 0; i < n; ++i)
                    h[i >> 1] |= static_cast<uint32_t>(src[2 * i] | (src[2 * i + 1] << 8)) << (16 * (i & 1));
            }
            *reinterpret_cast<uint4 *>(r.payload + ad[q].payload) = make_uint4(h[0], h[1], h[2], h[3]);
        }
    }
}

template <int KIND, int MT, int UPL>
hipError_t launch_one(const GemvPlan &p, const GemvArgs &args, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_kernel<KIND, MT, UPL>), dim3(p.grid), dim3(kGemvThreads), p.lds_bytes,
                       stream, args);
    return hipGetLastError();
}

template <int KIND, int MT>
hipError_t dispatch_upl(const GemvPlan &p, const GemvArgs &args, int upl, hipStream_t stream) {
    switch (upl) {
    case 1: return launch_one<KIND, MT, 1>(p, args, stream);
    case 2: return launch_one<KIND, MT, 2>(p, args, stream);
    case 3: return launch_one<KIND, MT, 3>(p, args, stream);
    case 4: return launch_one<KIND, MT, 4>(p, args, stream);
    case 5: return launch_one<KIND, MT, 5>(p, args, stream);
    case 6: return launch_one<KIND, MT, 6>(p, args, stream);
    case 8: return launch_one<KIND, MT, 8>(p, args, stream);
    case 10: return launch_one<KIND, MT, 10>(p, args, stream);
    case 12: return launch_one<KIND, MT, 12>(p, args, stream);
    case 16: return launch_one<KIND, MT, 16>(p, args, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int KIND>
hipError_t dispatch_mt(const GemvPlan &p, const GemvArgs &args, int upl, hipStream_t stream) {
    switch (p.tokens) {
    case 1: return dispatch_upl<KIND, 1>(p, args, upl, stream);
    case 2: return dispatch_upl<KIND, 2>(p, args, upl, stream);
    case 4: return dispatch_upl<KIND, 4>(p, args, upl, stream);
    case 8: return dispatch_upl<KIND, 8>(p, args, upl, stream);
    case 16: return dispatch_upl<KIND, 16>(p, args, upl, stream);
    default: return hipErrorInvalidValue;
    }
}

GemvArgs args_of(const DeviceTensor &t) {
    GemvArgs a{};
    a.payload = t.payload;
    a.meta = t.meta;
    a.tile_payload_bytes = t.tile_payload_bytes;
    a.tile_meta_bytes = t.tile_meta_bytes;
    a.rows = t.rows;
    a.units = t.units;
    a.lanes = t.lanes;
    a.rows_per_wave = t.rows_per_wave;
    a.image_bytes = static_cast<uint32_t>(image_bytes(t.kind, t.units));
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

bool layout_tensor_with(DeviceTensor &t, uint32_t lanes, uint32_t upl) {
    if (!set_units(t)) return false;
    bool upl_ok = false;
    for (int w : kUplWidths) upl_ok |= static_cast<uint32_t>(w) == upl;
    if (!upl_ok || lanes == 0 || lanes > 64 || (lanes & (lanes - 1)) || lanes * upl < t.units) return false;
    t.lanes = lanes;
    t.upl = upl;
    t.rows_per_wave = kWaveSize / lanes;
    t.tiles = (t.rows + t.rows_per_wave - 1) / t.rows_per_wave;
    // whole workgroups of tiles, so a workgroup never reads past the end
    t.tiles = (t.tiles + kGemvWaves - 1) / kGemvWaves * kGemvWaves;
    // compact tiles: only real units are stored (idle lanes load nothing new)
    t.tile_payload_bytes = static_cast<size_t>(t.rows_per_wave) * t.units * t.chunks * 16;
    t.tile_meta_bytes = t.kind == kF16 ? 0 : static_cast<size_t>(t.rows_per_wave) * t.units * 8;
    const size_t payload = t.tile_payload_bytes * t.tiles;
    const size_t meta = t.tile_meta_bytes * t.tiles;
    t.device_bytes = ((payload + 255) & ~static_cast<size_t>(255)) + meta;
    return true;
}

// Lane plan: one unit per lane where the row allows it (L = the power of
// two covering the row, at most 64), so the post-load work per lane is
// short and the grid is large; longer rows take more units per lane.
// Idle lanes cost VALU slots but no memory traffic (compact tiles).
bool layout_tensor(DeviceTensor &t) {
    if (!set_units(t)) return false;
    uint32_t L = 1;
    while (L < t.units && L < static_cast<uint32_t>(kWaveSize)) L *= 2;
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

hipError_t repack_tensor(const DeviceTensor &t, const uint8_t *staging, hipStream_t stream) {
    hipError_t e = hipMemsetAsync(t.payload, 0, t.device_bytes, stream);
    if (e != hipSuccess) return e;
    RepackArgs r{};
    r.src = staging;
    r.payload = t.payload;
    r.meta = t.meta;
    r.rows = t.rows;
    r.cols = t.cols;
    r.units = t.units;
    r.lanes = t.lanes;
    r.rows_per_wave = t.rows_per_wave;
    r.tile_payload = t.tile_payload_bytes;
    r.tile_meta = t.tile_meta_bytes;
    const size_t n = static_cast<size_t>(t.rows) * t.units;
    const dim3 grid((n + 255) / 256);
    if (t.kind == kHvsq2) hipLaunchKernelGGL(repack_kernel<kHvsq2>, grid, dim3(256), 0, stream, r);
    else if (t.kind == kQ4_0) hipLaunchKernelGGL(repack_kernel<kQ4_0>, grid, dim3(256), 0, stream, r);
    else hipLaunchKernelGGL(repack_kernel<kF16>, grid, dim3(256), 0, stream, r);
    return hipGetLastError();
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
    if (t.kind == kHvsq2)
        hipLaunchKernelGGL(quantize_image_kernel<kHvsq2>, dim3(batch), dim3(256), 0, stream, x, t.cols, x_stride,
                           t.units, image, image_stride, scales, q8, q8_stride);
    else if (t.kind == kQ4_0)
        hipLaunchKernelGGL(quantize_image_kernel<kQ4_0>, dim3(batch), dim3(256), 0, stream, x, t.cols, x_stride,
                           t.units, image, image_stride, scales, q8, q8_stride);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvLaunch &g, hipStream_t stream) {
    const DeviceTensor &t = *g.tensor;
    GemvArgs args = args_of(t);
    args.output_stride = g.output_stride;
    args.image = static_cast<const uint8_t *>(g.image);
    args.image_stride = g.image_stride;

    if (g.debug_sums) {
        if (t.kind == kF16) return hipErrorInvalidValue;
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

    const GemvPlan p = plan_gemv(t, static_cast<int>(g.batch));
    if (p.tokens == 0 || p.lds_bytes > kGemvLdsLimit) return hipErrorInvalidValue;
    for (uint32_t t0 = 0; t0 < g.batch; t0 += p.tokens) {
        args.ntok = std::min<uint32_t>(p.tokens, g.batch - t0);
        args.image = static_cast<const uint8_t *>(g.image) + static_cast<size_t>(t0) * g.image_stride;
        args.scales = g.scales ? g.scales + t0 : nullptr;
        args.scale = g.scale;
        args.output = g.output + static_cast<size_t>(t0) * g.output_stride;
        hipError_t e;
        if (t.kind == kHvsq2) e = dispatch_mt<kHvsq2>(p, args, t.upl, stream);
        else if (t.kind == kQ4_0) e = dispatch_mt<kQ4_0>(p, args, t.upl, stream);
        else e = dispatch_mt<kF16>(p, args, t.upl, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace qwn
