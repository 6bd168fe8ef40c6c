// Device-side helpers shared by the qwn_hip kernels: fp16 decode, the
// activation-image packing of one 32-element block, and the address of a
// weight unit in the wave-tile layout (qwn_internal.h).
#pragma once

#include "qwn_internal.h"

namespace qwn {

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

__device__ __forceinline__ float half_to_float(uint32_t bits) {
    // v_cvt_f32_f16 keeps fp16 subnormals (the default f16 denormal mode),
    // matching the CPU's exact conversion (c/qwanto_kernels.c:264-285).
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}


// ---- cross-lane reductions (DPP) -----------------------------------------

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

// Max over each 16-lane row, in the row's last lane: lanes with no source
// lane keep their own value (bound_ctrl off, old = v).
template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float v) {
    const int moved = __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), CTRL,
                                                  0xf, 0xf, false);
    return fmaxf(v, __builtin_bit_cast(float, moved));
}

// LDS address space, for the direct global-to-LDS loads
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(n) (n <= 63), expcnt and lgkmcnt left alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    constexpr int n = N > 63 ? 63 : N;
    __builtin_amdgcn_s_waitcnt((n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Compiler-level fence plus the hardware barrier, without the vmcnt(0)
// that __syncthreads() implies: LDS writes before it are visible after it,
// global loads and stores in flight stay in flight.
// The int8 of c, |c| <= 127, rounded half to even, in the low byte of the
// result: c + 1.5 * 2^23 lies where the fp32 spacing is 1, so the add
// rounds c to the nearest even integer n and leaves 0x4b400000 + n as the
// bits (one add where rintf and a float-to-int conversion take two).
__device__ __forceinline__ uint32_t q8_low_byte(float c) { return __builtin_bit_cast(uint32_t, c + 12582912.0f); }

// The low bytes of a, b, c, d as bytes 0..3 of one word (three byte
// permutes: v_perm_b32 selects bytes 0-3 from its second operand and 4-7
// from its first, 0x0c gives zero).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Whole-wave sum / max, returned to every lane (row reductions by DPP, then
// the four row totals read as scalars and combined in row order).
__device__ __forceinline__ float wave_sum_all(float v) {
    v = group_sum(v, 16);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 47));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ float wave_max_all(float v) {
    v = dpp_max_step<0x111>(v);
    v = dpp_max_step<0x112>(v);
    v = dpp_max_step<0x114>(v);
    v = dpp_max_step<0x118>(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 47));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}


// ---- activation images --------------------------------------------------------

// The value of lane ^ 1 / lane ^ 2 within each quad, by DPP quad
// permutes (a VALU operand, where __shfl_xor goes through the LDS crossbar).
__device__ __forceinline__ int quad_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false); }
__device__ __forceinline__ int quad_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false); }

// Nibble-pack 8 int8 values (two dwords, element order) into the high
// (signed, a >> 4) and low (a & 15) nibble words, nibble k = element k.
// Per word the nibbles of bytes 0-1 and 2-3 fold into bytes 0 and 2 (x | x
// >> 4 on the masked nibbles), then one byte permute gathers them; the high
// nibble is bits 4-7 of the byte, the arithmetic >> 4 of the int8 as a
// nibble.
__device__ __forceinline__ void split8(uint32_t a, uint32_t b, uint32_t &hi, uint32_t &lo) {
    const uint32_t la = a & 0x0f0f0f0fu, lb = b & 0x0f0f0f0fu;
    const uint32_t ha = (a >> 4) & 0x0f0f0f0fu, hb = (b >> 4) & 0x0f0f0f0fu;
    lo = __builtin_amdgcn_perm(lb | (lb >> 4), la | (la >> 4), 0x06040200u);
    hi = __builtin_amdgcn_perm(hb | (hb >> 4), ha | (ha >> 4), 0x06040200u);
}

// Even/odd split of 16 int8 values for the HyperVSQ-2 masks: returns the
// high/low nibble words of elements {0,2,..,14} and {1,3,..,15}.
// Word q holds elements 4q .. 4q+3: m | (m >> 12) on its masked nibbles
// puts those of elements 4q, 4q+2 (even) in byte 0 and of 4q+1, 4q+3 (odd)
// in byte 1; byte permutes then gather bytes 0 and bytes 1 of the four
// words.
__device__ __forceinline__ uint4 split16_evenodd(const uint32_t w[4]) {
    uint32_t t[4], g[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t m = w[q] & 0x0f0f0f0fu, h = (w[q] >> 4) & 0x0f0f0f0fu;
        t[q] = m | (m >> 12);
        g[q] = h | (h >> 12);
    }
    // [x0.b0, x1.b0, x0.b1, x1.b1] of a pair of words
    const uint32_t t01 = __builtin_amdgcn_perm(t[1], t[0], 0x05010400u);
    const uint32_t t23 = __builtin_amdgcn_perm(t[3], t[2], 0x05010400u);
    const uint32_t g01 = __builtin_amdgcn_perm(g[1], g[0], 0x05010400u);
    const uint32_t g23 = __builtin_amdgcn_perm(g[3], g[2], 0x05010400u);
    return make_uint4(__builtin_amdgcn_perm(g23, g01, 0x05040100u), __builtin_amdgcn_perm(t23, t01, 0x05040100u),
                      __builtin_amdgcn_perm(g23, g01, 0x07060302u), __builtin_amdgcn_perm(t23, t01, 0x07060302u));
}

// Write one 32-activation block (8 dwords of int8, element order) into a
// token image: its nibble words and its correction term.
template <int KIND>
__device__ __forceinline__ void put_block32(uint8_t *img, uint32_t units, uint32_t b, const uint32_t w[8]) {
    const uint32_t e0 = b * 32;
    int32_t *sums = reinterpret_cast<int32_t *>(img + units * unit_lds_bytes(KIND));
    if (KIND == kHvsq2) {
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = sdot4(w[i], 0x01010101u, s);
        sums[b] = s;
        const uint32_t u = e0 / 256, off = e0 % 256;
#pragma unroll
        for (int g = 0; g < 2; ++g)
            *reinterpret_cast<uint4 *>(img + u * 272 + (off / 16 + g) * 16) = split16_evenodd(w + 4 * g);
    } else {
        const uint32_t u = e0 / 128, off = e0 % 128;
        int lsum = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t hi, lo;
            split8(w[2 * g], w[2 * g + 1], hi, lo);
            lsum = static_cast<int>(__builtin_amdgcn_udot8(lo, 0x11111111u, static_cast<uint32_t>(lsum), false));
            *reinterpret_cast<uint2 *>(img + u * 144 + (off / 8 + g) * 8) = make_uint2(hi, lo);
        }
        sums[b] = 8 * lsum;
    }
}


// Sub-block sb (E = 16 int8 for HyperVSQ-2, 8 for Q4_0, four per word) of
// the fused prologue's image: its nibble words, and the per-32 correction
// term summed over the 32/E adjacent lanes holding one 32-block (every lane
// takes part in the exchange; only sub-blocks below nsub are written).
template <int KIND>
__device__ __forceinline__ void put_sub_block(uint8_t *img, uint32_t units, uint32_t sb, uint32_t nsub,
                                              const uint32_t *w) {
    int32_t *sums = reinterpret_cast<int32_t *>(img + units * unit_lds_bytes(KIND));
    if (KIND == kHvsq2) {
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) s = sdot4(w[i], 0x01010101u, s);
        s += quad_xor1(s);
        if (sb < nsub) {
            const uint32_t e0 = sb * 16, u = e0 / 256, off = e0 % 256;
            *reinterpret_cast<uint4 *>(img + u * 272 + off) = split16_evenodd(w);
            if (sb % 2 == 0) sums[sb / 2] = s;
        }
    } else {
        uint32_t hi, lo;
        split8(w[0], w[1], hi, lo);
        int lsum = static_cast<int>(__builtin_amdgcn_udot8(lo, 0x11111111u, 0u, false));
        lsum += quad_xor1(lsum);
        lsum += quad_xor2(lsum);
        if (sb < nsub) {
            const uint32_t e0 = sb * 8, u = e0 / 128, off = e0 % 128;
            *reinterpret_cast<uint2 *>(img + u * 144 + off) = make_uint2(hi, lo);
            if (sb % 4 == 0) sums[sb / 4] = 8 * lsum;
        }
    }
}

// Byte address of chunk q of unit u of a row, and of its metadata.
struct UnitAddr {
    size_t payload, meta;
};
__host__ __device__ inline UnitAddr unit_addr(uint32_t row, uint32_t u, uint32_t q, uint32_t lanes,
                                              uint32_t rows_per_wave, uint32_t units, size_t tile_payload,
                                              size_t tile_meta) {
    const uint32_t tile = row / rows_per_wave, grp = row % rows_per_wave;
    const uint32_t i = u / lanes, jj = u % lanes;
    const uint32_t n = units - i * lanes < lanes ? units - i * lanes : lanes;  // units in plane i
    UnitAddr r;
    r.payload = tile * tile_payload + static_cast<size_t>(64) * rows_per_wave * lanes * i +
                (static_cast<size_t>(q) * rows_per_wave * n + grp * n + jj) * 16;
    r.meta = tile * tile_meta + static_cast<size_t>(8) * rows_per_wave * lanes * i +
             (static_cast<size_t>(grp) * n + jj) * 8;
    return r;
}


}  // namespace qwn
