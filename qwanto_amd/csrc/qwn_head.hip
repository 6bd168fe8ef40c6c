// qwn_head.hip -- the LM head over a block of up to 16 tokens (speculative
// verify: every drafted token's logits) on the matrix cores.
//
// The reference runs each token's head as an fp32 dot product of the F16 or
// BF16 rows with the fp32 normed activation (qwn_matmul_f32,
// c/qwanto_kernels.c:1531-1616, called per token from
// c/qwanto_decode.c:2007).  Here the activation of each token is written as
// an exact-sum of narrow pieces:
//   F16 rows:  x * 2^s = p0 + p1 (two f16, s a per-token power of two that
//              puts max|x| * 2^s just under 2^15), |x*2^s - p0 - p1| <=
//              2^-22 |x*2^s| (+ a subnormal step for tiny x)
//   BF16 rows: x = p0 + p1 + p2 (three bf16, 24 significant bits)
// so that W x = sum_p W p_p (* 2^-s) with every product exact in the
// v_mfma_f32_16x16x32_{f16,bf16} fp32 accumulation: the head is read once for
// 16 tokens instead of once per 8 on the fp32 GEMV.
//
// Pieces image [piece][unit (32 columns)][quarter q][token 0..15][8 x 16-bit]:
// lane l of an MFMA takes token l % 16, columns 8 (l / 16) .. +7 of a unit:
// one 16-byte LDS read.  The weight operand: lane l takes row l % 16 of the
// 16-row tile, the same 8 columns, one 16-byte chunk of the wave-tile
// layout.  Output C[row][token]: lane l holds rows 4 (l / 16) + i, token
// l % 16.
#include "qwn_device.h"
#include "qwn_internal.h"

#include <algorithm>
#include <type_traits>

namespace qwn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf168 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kHeadTokens = 16;
constexpr int kHeadWaves = 8;
constexpr int kHeadStage = 4;   // units whose weight chunks are loaded one stage ahead

__device__ __forceinline__ uint16_t bf16_rne(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __builtin_bit_cast(float, uint32_t{h} << 16); }

// grid (tokens), 1024 threads: RMSNorm of the token (the fp32 arithmetic of
// the head's norm image: x * (1 / sqrt(mean x^2 + eps)) * w, the sum in the
// same per-thread order), then its pieces; unscale[t] = 2^-s (1 for BF16).
template <bool BF16, int EPT, int TS>
__global__ __launch_bounds__(1024) void head_pieces_kernel(const float *__restrict__ x, uint32_t x_stride,
                                                           const float *__restrict__ norm, float eps, uint32_t K,
                                                           uint32_t units, uint16_t *__restrict__ pieces,
                                                           float *__restrict__ unscale) {
    constexpr int NP = BF16 ? 3 : 2;
    __shared__ float red[2][1024 / kWaveSize];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, W = blockDim.x / kWaveSize;
    const float *row = x + static_cast<size_t>(t) * x_stride;
    float xv[EPT], wv[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const uint32_t k = tid + 1024u * e, kk = k < K ? k : 0u;
        xv[e] = row[kk];
        wv[e] = norm[kk];
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
        if (tid + 1024u * e < K) ss = fmaf(xv[e], xv[e], ss);
    ss = wave_sum_all(ss);
    if (tid % kWaveSize == 0) red[0][tid / kWaveSize] = ss;
    lds_barrier();
    float tot = 0.0f;
    for (uint32_t i = 0; i < W; ++i) tot += red[0][i];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
    float v[EPT];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        v[e] = tid + 1024u * e < K ? (xv[e] * inv) * wv[e] : 0.0f;
        amax = fmaxf(amax, fabsf(v[e]));
    }
    float scale = 1.0f, back = 1.0f;
    if (!BF16) {
        amax = wave_max_all(amax);
        if (tid % kWaveSize == 0) red[1][tid / kWaveSize] = amax;
        lds_barrier();
        amax = red[1][0];
        for (uint32_t i = 1; i < W; ++i) amax = fmaxf(amax, red[1][i]);
        int e2 = 0;
        if (amax > 0.0f && amax < INFINITY) {
            (void)frexpf(amax, &e2);   // amax = m 2^e2, m in [0.5, 1)
            const int s = min(max(15 - e2, -100), 100);
            scale = ldexpf(1.0f, s);
            back = ldexpf(1.0f, -s);
        }
    }
    if (tid == 0) unscale[t] = back;
    const size_t plane = static_cast<size_t>(units) * 4 * TS * 8;   // elements per piece
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const uint32_t k = tid + 1024u * e;
        if (k < units * 32) {
            const uint32_t u = k / 32, q = (k % 32) / 8, j = k % 8;
            const size_t at = ((static_cast<size_t>(u) * 4 + q) * TS + t) * 8 + j;
            if (BF16) {
                const float x0 = v[e];
                const uint16_t h0 = bf16_rne(x0);
                const float r1 = x0 - bf16_to_f32(h0);
                const uint16_t h1 = bf16_rne(r1);
                const float r2 = r1 - bf16_to_f32(h1);
                pieces[at] = h0;
                pieces[plane + at] = h1;
                pieces[2 * plane + at] = bf16_rne(r2);
            } else {
                const float xs = v[e] * scale;
                const _Float16 h0 = static_cast<_Float16>(xs);
                const _Float16 h1 = static_cast<_Float16>(xs - static_cast<float>(h0));
                pieces[at] = __builtin_bit_cast(uint16_t, h0);
                pieces[plane + at] = __builtin_bit_cast(uint16_t, h1);
            }
        }
    }
    (void)NP;
}

struct HeadArgs {
    const uint8_t *payload;
    size_t tile_payload;
    uint32_t lanes, lanes_log2, rows_per_wave, rpw_log2, units, rows, padded_rows;
    const uint8_t *pieces;
    const float *unscale;
    uint32_t ntok;
    float *out;
    uint32_t out_stride;
};

// grid (workgroups), kHeadWaves waves: the pieces image is copied into LDS
// once, then each wave takes 16-row tiles rt = wave id, + total waves, ...
// and runs its K loop with the next stage's weight chunks in flight.  A
// weight load touches 64 lines (16 rows x 4 column groups of the wave-tile
// layout) and uses 16 bytes of each; the stage's next loads use the rest.
// Measured at 151936 x 1536 F16, 16 tokens: 133 us per launch (3.5 TB/s),
// against 450 us for two 8-token fp32 GEMV launches; 4 or 16 waves, and
// stages of 8 or 16 units, measured no faster.
template <bool BF16>
__global__ __launch_bounds__(64 * kHeadWaves) void mfma_head_kernel(HeadArgs a) {
    constexpr int NP = BF16 ? 3 : 2;
    extern __shared__ __align__(16) uint8_t smem[];   // pieces image: NP * units KB
    const uint32_t tid = threadIdx.x, lane = tid % kWaveSize;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWaveSize);
    const uint32_t units = a.units;
    {
        const uint32_t total = NP * units * 64;   // 16-byte pieces, a multiple of 64
        for (uint32_t c0 = wave * kWaveSize; c0 < total; c0 += blockDim.x)
            __builtin_amdgcn_global_load_lds(a.pieces + static_cast<size_t>(c0 + lane) * 16,
                                             (lds_void *)(smem + static_cast<size_t>(c0) * 16), 16, 0, 0);
        wait_vmcnt<0>();
        lds_barrier();
    }
    const uint32_t col = lane % 16, kq = lane / 16;
    const uint32_t L = a.lanes, R = a.rows_per_wave;
    const uint32_t ntiles = (a.rows + 15) / 16;
    const uint32_t nstage = (units + kHeadStage - 1) / kHeadStage;
    for (uint32_t rt = blockIdx.x * kHeadWaves + wave; rt < ntiles; rt += gridDim.x * kHeadWaves) {
        const uint32_t row = min(rt * 16 + col, a.padded_rows - 1);
        const uint32_t tile = row >> a.rpw_log2, grp = row & (R - 1);
        const uint8_t *tbase = a.payload + static_cast<size_t>(tile) * a.tile_payload;
        // byte offset of chunk kq of unit u of this lane's row (wave-tile layout)
        auto chunk_at = [&](uint32_t u) -> const uint4 * {
            const uint32_t i = u >> a.lanes_log2, jj = u & (L - 1);
            const uint32_t n = min(L, units - i * L);
            return reinterpret_cast<const uint4 *>(tbase + static_cast<size_t>(64) * R * L * i +
                                                   (static_cast<size_t>(kq) * R * n + grp * n + jj) * 16);
        };
        // two stage buffers used in turn (never copied: a copy of a register
        // a load is still writing would wait for that load)
        uint4 wa[kHeadStage], wb[kHeadStage];
        auto load_stage = [&](uint4 (&w)[kHeadStage], uint32_t st) {
#pragma unroll
            for (int i = 0; i < kHeadStage; ++i) w[i] = *chunk_at(min(st * kHeadStage + i, units - 1));
        };
        float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
        auto run_stage = [&](const uint4 (&w)[kHeadStage], uint32_t st) {
#pragma unroll
            for (int i = 0; i < kHeadStage; ++i) {
                const uint32_t u = st * kHeadStage + i;
                if (u < units) {
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        const uint4 bw = *reinterpret_cast<const uint4 *>(
                            smem + ((((static_cast<size_t>(p) * units + u) * 4 + kq) * kHeadTokens + col) * 16));
                        if constexpr (BF16)
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf168, w[i]),
                                                                          __builtin_bit_cast(bf168, bw), acc, 0, 0, 0);
                        else
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, w[i]),
                                                                         __builtin_bit_cast(half8, bw), acc, 0, 0, 0);
                    }
                }
            }
        };
        load_stage(wa, 0);
        for (uint32_t st = 0; st < nstage; st += 2) {
            if (st + 1 < nstage) load_stage(wb, st + 1);
            run_stage(wa, st);
            if (st + 1 < nstage) {
                if (st + 2 < nstage) load_stage(wa, st + 2);
                run_stage(wb, st + 1);
            }
        }
        // rows 4 kq + i of the tile, token col
        if (col < a.ntok) {
            const float back = a.unscale[col];
            const uint32_t r = rt * 16 + 4 * kq;
            float *dst = a.out + static_cast<size_t>(col) * a.out_stride + r;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (r + i < a.rows) dst[i] = acc[i] * back;
        }
    }
}

// 17 to 32 tokens (pieces written for 32: head_pieces_bytes_32): grid
// (workgroups, 2), blockIdx.y the half of the units
// this workgroup covers (its pieces of both 16-token groups, [piece][unit -
// u0][quarter][token 0..31][16 B], the LDS of one 16-token launch over all
// units), each weight chunk fed to both groups' products; the two halves'
// partial logits are added into the cleared output (two adds onto zero: the
// same sum in either order).  The head is read once per 32 tokens.
template <bool BF16>
__global__ __launch_bounds__(64 * kHeadWaves) void mfma_head2_kernel(HeadArgs a) {
    constexpr int NP = BF16 ? 3 : 2;
    constexpr int TS = 2 * kHeadTokens;
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, lane = tid % kWaveSize;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWaveSize);
    const uint32_t units = a.units, uh = (units + 1) / 2;
    const uint32_t u0 = blockIdx.y * uh, u1 = min(units, u0 + uh), nu = u1 - u0;
    {
        // each piece plane's units [u0, u1) are one contiguous run
        const uint32_t per_plane = nu * 4 * TS;   // 16-byte pieces (8 elements each), a multiple of 64
        const uint32_t total = NP * per_plane;
        for (uint32_t c0 = wave * kWaveSize; c0 < total; c0 += blockDim.x) {
            const uint32_t c = c0 + lane, p = c / per_plane, r = c - p * per_plane;
            const size_t src = (static_cast<size_t>(p) * units * 4 * TS + static_cast<size_t>(u0) * 4 * TS + r) * 16;
            __builtin_amdgcn_global_load_lds(a.pieces + src, (lds_void *)(smem + static_cast<size_t>(c0) * 16), 16,
                                             0, 0);
        }
        wait_vmcnt<0>();
        lds_barrier();
    }
    if (nu == 0) return;   // a one-unit row: the second half is empty
    const uint32_t col = lane % 16, kq = lane / 16;
    const uint32_t L = a.lanes, R = a.rows_per_wave;
    const uint32_t ntiles = (a.rows + 15) / 16;
    const uint32_t nstage = (nu + kHeadStage - 1) / kHeadStage;
    for (uint32_t rt = blockIdx.x * kHeadWaves + wave; rt < ntiles; rt += gridDim.x * kHeadWaves) {
        const uint32_t row = min(rt * 16 + col, a.padded_rows - 1);
        const uint32_t tile = row >> a.rpw_log2, grp = row & (R - 1);
        const uint8_t *tbase = a.payload + static_cast<size_t>(tile) * a.tile_payload;
        auto chunk_at = [&](uint32_t u) -> const uint4 * {
            const uint32_t i = u >> a.lanes_log2, jj = u & (L - 1);
            const uint32_t n = min(L, units - i * L);
            return reinterpret_cast<const uint4 *>(tbase + static_cast<size_t>(64) * R * L * i +
                                                   (static_cast<size_t>(kq) * R * n + grp * n + jj) * 16);
        };
        uint4 wa[kHeadStage], wb[kHeadStage];
        auto load_stage = [&](uint4 (&w)[kHeadStage], uint32_t st) {
#pragma unroll
            for (int i = 0; i < kHeadStage; ++i) w[i] = *chunk_at(u0 + min(st * kHeadStage + i, nu - 1));
        };
        float4v acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
        auto run_stage = [&](const uint4 (&w)[kHeadStage], uint32_t st) {
#pragma unroll
            for (int i = 0; i < kHeadStage; ++i) {
                const uint32_t ul = st * kHeadStage + i;
                if (ul < nu) {
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        const uint8_t *bp = smem + (((static_cast<size_t>(p) * nu + ul) * 4 + kq) * TS + col) * 16;
                        const uint4 b0 = *reinterpret_cast<const uint4 *>(bp);
                        const uint4 b1 = *reinterpret_cast<const uint4 *>(bp + kHeadTokens * 16);
                        if constexpr (BF16) {
                            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf168, w[i]),
                                                                           __builtin_bit_cast(bf168, b0), acc0, 0, 0, 0);
                            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf168, w[i]),
                                                                           __builtin_bit_cast(bf168, b1), acc1, 0, 0, 0);
                        } else {
                            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, w[i]),
                                                                          __builtin_bit_cast(half8, b0), acc0, 0, 0, 0);
                            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, w[i]),
                                                                          __builtin_bit_cast(half8, b1), acc1, 0, 0, 0);
                        }
                    }
                }
            }
        };
        load_stage(wa, 0);
        for (uint32_t st = 0; st < nstage; st += 2) {
            if (st + 1 < nstage) load_stage(wb, st + 1);
            run_stage(wa, st);
            if (st + 1 < nstage) {
                if (st + 2 < nstage) load_stage(wa, st + 2);
                run_stage(wb, st + 1);
            }
        }
        // rows 4 kq + i of the tile, tokens col and 16 + col
        const uint32_t r = rt * 16 + 4 * kq;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t tok = g * kHeadTokens + col;
            if (tok < a.ntok) {
                const float back = a.unscale[tok];
                float *dst = a.out + static_cast<size_t>(tok) * a.out_stride + r;
                const float4v &acc = g == 0 ? acc0 : acc1;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (r + i < a.rows) unsafeAtomicAdd(dst + i, acc[i] * back);
            }
        }
    }
}

// rows [0, n) x [0, cols) of a [n][stride] fp32 array set to zero
__global__ __launch_bounds__(256) void clear_rows_kernel(float *__restrict__ out, uint32_t cols, uint32_t stride) {
    float *row = out + static_cast<size_t>(blockIdx.y) * stride;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < cols; k += gridDim.x * blockDim.x) row[k] = 0.0f;
}

}  // namespace

size_t head_pieces_bytes(const DeviceTensor &t) {
    return static_cast<size_t>(t.bf16 ? 3 : 2) * t.units * 1024;
}

size_t head_pieces_bytes_32(const DeviceTensor &t) { return 2 * head_pieces_bytes(t); }

bool mfma_head_supported(const DeviceTensor &t) {
    return t.kind == kF16 && t.units > 0 && (t.lanes & (t.lanes - 1)) == 0 &&
           (t.rows_per_wave & (t.rows_per_wave - 1)) == 0 && t.cols <= 16384 &&
           head_pieces_bytes(t) <= kHeadLdsLimit;
}

hipError_t launch_head_pieces(const DeviceTensor &t, const float *x, uint32_t x_stride, const float *norm, float eps,
                              uint32_t ntok, uint8_t *pieces, float *unscale, hipStream_t stream) {
    if (!mfma_head_supported(t) || ntok == 0 || ntok > static_cast<uint32_t>(2 * kHeadTokens))
        return hipErrorInvalidValue;
    const uint32_t per = (t.units * 32 + 1023) / 1024;
    auto go = [&](auto bf_c, auto ept_c) {
        constexpr bool B = decltype(bf_c)::value;
        constexpr int E = decltype(ept_c)::value;
        if (ntok > static_cast<uint32_t>(kHeadTokens))
            hipLaunchKernelGGL((head_pieces_kernel<B, E, 2 * kHeadTokens>), dim3(ntok), dim3(1024), 0, stream, x,
                               x_stride, norm, eps, t.cols, t.units, reinterpret_cast<uint16_t *>(pieces), unscale);
        else
            hipLaunchKernelGGL((head_pieces_kernel<B, E, kHeadTokens>), dim3(ntok), dim3(1024), 0, stream, x,
                               x_stride, norm, eps, t.cols, t.units, reinterpret_cast<uint16_t *>(pieces), unscale);
    };
    auto by_ept = [&](auto bf_c) {
        if (per <= 1) go(bf_c, std::integral_constant<int, 1>{});
        else if (per <= 2) go(bf_c, std::integral_constant<int, 2>{});
        else if (per <= 4) go(bf_c, std::integral_constant<int, 4>{});
        else if (per <= 8) go(bf_c, std::integral_constant<int, 8>{});
        else go(bf_c, std::integral_constant<int, 16>{});
    };
    if (t.bf16) by_ept(std::true_type{});
    else by_ept(std::false_type{});
    return hipGetLastError();
}

hipError_t launch_mfma_head(const DeviceTensor &t, const uint8_t *pieces, const float *unscale, uint32_t ntok,
                            float *out, uint32_t out_stride, hipStream_t stream) {
    if (!mfma_head_supported(t) || ntok == 0 || ntok > static_cast<uint32_t>(2 * kHeadTokens) || out_stride < t.rows)
        return hipErrorInvalidValue;
    HeadArgs a{};
    a.payload = t.payload;
    a.tile_payload = t.tile_payload_bytes;
    a.lanes = t.lanes;
    a.lanes_log2 = static_cast<uint32_t>(__builtin_ctz(t.lanes));
    a.rows_per_wave = t.rows_per_wave;
    a.rpw_log2 = static_cast<uint32_t>(__builtin_ctz(t.rows_per_wave));
    a.units = t.units;
    a.rows = t.rows;
    a.padded_rows = t.tiles * t.rows_per_wave;
    a.pieces = pieces;
    a.unscale = unscale;
    a.ntok = ntok;
    a.out = out;
    a.out_stride = out_stride;
    const uint32_t ntiles = (t.rows + 15) / 16;
    const uint32_t grid = std::max(1u, std::min(256u, (ntiles + kHeadWaves - 1) / kHeadWaves));
    const size_t lds = head_pieces_bytes(t);
    if (ntok > static_cast<uint32_t>(kHeadTokens)) {
        // the two unit halves add into a cleared output; LDS: the pieces of
        // the larger half for 32 tokens; half the workgroups per half (one
        // round of the chip for both halves: 2.404 -> 2.385 ms per 64-node
        // tree against the full grid per half)
        const size_t lds2 = static_cast<size_t>(t.bf16 ? 3 : 2) * ((t.units + 1) / 2) * 2048;
        const uint32_t grid2 = std::max(1u, grid / 2);
        hipLaunchKernelGGL(clear_rows_kernel, dim3((t.rows + 1023) / 1024, ntok), dim3(256), 0, stream, out, t.rows,
                           out_stride);
        if (t.bf16) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&mfma_head2_kernel<true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds2));
            hipLaunchKernelGGL(mfma_head2_kernel<true>, dim3(grid2, 2), dim3(64 * kHeadWaves), lds2, stream, a);
        } else {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&mfma_head2_kernel<false>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds2));
            hipLaunchKernelGGL(mfma_head2_kernel<false>, dim3(grid2, 2), dim3(64 * kHeadWaves), lds2, stream, a);
        }
        return hipGetLastError();
    }
    if (t.bf16) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&mfma_head_kernel<true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        hipLaunchKernelGGL(mfma_head_kernel<true>, dim3(grid), dim3(64 * kHeadWaves), lds, stream, a);
    } else {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&mfma_head_kernel<false>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        hipLaunchKernelGGL(mfma_head_kernel<false>, dim3(grid), dim3(64 * kHeadWaves), lds, stream, a);
    }
    return hipGetLastError();
}

}  // namespace qwn
