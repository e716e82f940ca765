// Device-side building blocks for the gfx950 FlashAttention-3 backward:
// vector types, the two MFMA shapes used, LDS transposed reads and the
// bank-conflict-free LDS swizzles of the Q/dO tiles and the dS^T tile.
//
// Lane layouts (verified on MI355X by an in-bounds probe of the builtins):
//   v_mfma_f32_32x32x16_f16   lane l, h = l / 32:
//     A[m][k]: m = l % 32, k = 8h + t (t = 0..7, the 8 halves of the operand)
//     B[k][n]: n = l % 32, k = 8h + t
//     C[m][n]: n = l % 32, m = 8 * (i / 4) + 4h + (i % 4)  (i = 0..15)
//   ds_read_b64_tr_b16, per group of 16 lanes (r = lane % 16), with A_i the
//     element address supplied by lane i of the group:
//     result[r][j] = lds16[A_{4j + r/4} + (r % 4)]   (j = 0..3)
//     i.e. if lane i points at row (i >> 2), column c0 + 4 * (i & 3) of a
//     row-major 16-bit matrix, lane r receives column c0 + r of those 4 rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fa3 {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define FA3_LDS __attribute__((address_space(3)))

constexpr int kWave = 64;
constexpr float kLog2e = 1.44269504088896340736f;

// Partial dot product of 8 pairs of 16-bit values (fp16, or bf16 bits when
// kBf16), accumulated in fp32 in a fixed order.
template <bool kBf16>
__device__ __forceinline__ float dot8(f16x8 a, f16x8 b, float acc) {
    if constexpr (kBf16) {
        const bf16x8 x = __builtin_bit_cast(bf16x8, a), y = __builtin_bit_cast(bf16x8, b);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = __builtin_fmaf((float)x[i], (float)y[i], acc);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f16x2 x = {a[2 * i], a[2 * i + 1]}, y = {b[2 * i], b[2 * i + 1]};
            acc = __builtin_amdgcn_fdot2(x, y, acc, false);
        }
    }
    return acc;
}

// 16-byte chunk of D that lane group g4 (= lane / 16) reads in k-step s of
// a 16x16x32 MFMA operand taken from 16 consecutive rows of a [64][D] tile.
// ds_read_b128 serves a wave in four groups of 16 lanes, lane l belonging to
// group (l / 32, parity of bits 2..4 of l); with the tile swizzle of
// tile_off<D> these orders give every group 16 distinct bank quads (the
// order 4 s + g4 would put two lanes of a group on one quad).
template <int D>
__device__ __forceinline__ int p1_chunk(int s, int g4) {
    if constexpr (D == 128) return s + 4 * g4;
    else return s + 2 * (g4 >> 1) + 4 * (g4 & 1);
}

// x of the lane that DPP control kCtrl selects (all rows and banks enabled).
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}

// delta = sum_d fp32(dO[row, d]) * fp32(O[row, d]) of one query row whose
// elements start at `elem`: lane `sub` of the row's D / 8 consecutive lanes
// takes the 16-byte chunk sub (dot8), then a butterfly over those lanes.
template <int D, bool kBf16 = false>
__device__ __forceinline__ float row_delta(const _Float16* dout, const _Float16* out, size_t elem,
                                           int sub) {
    const size_t c = elem + (size_t)sub * 8;
    float acc = dot8<kBf16>(*(const f16x8*)(dout + c), *(const f16x8*)(out + c), 0.f);
    if constexpr (D == 128) {
        // The row's 16 lanes are one DPP row: the butterfly's partners at
        // distance 8, 4, 2, 1 through row_ror:8, row_ror:4 and two quad
        // permutations instead of four LDS-crossbar shuffles.  After the
        // first step a lane's value depends on lane % 8 only, so the lane 4
        // places round the row holds the same value as the lane at xor 4:
        // the same sums in the same order.
        acc += dpp_f32<0x128>(acc);  // row_ror:8
        acc += dpp_f32<0x124>(acc);  // row_ror:4
        acc += dpp_f32<0x4E>(acc);   // quad_perm [2, 3, 0, 1]
        acc += dpp_f32<0xB1>(acc);   // quad_perm [1, 0, 3, 2]
    } else {
#pragma unroll
        for (int off = D / 16; off > 0; off >>= 1) acc += __shfl_xor(acc, off, D / 8);
    }
    return acc;
}

__device__ __forceinline__ f32x16 mfma_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Transposed 4 x 16-bit read; `byte_off` is the LDS byte address this lane
// supplies (see the layout note at the top of the file).
__device__ __forceinline__ f16x4 lds_read_tr4(const FA3_LDS char* lds, uint32_t byte_off) {
    typedef __fp16 raw4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
    raw4 r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((FA3_LDS raw4*)(lds + byte_off));
    return __builtin_bit_cast(f16x4, r);
}

__device__ __forceinline__ f16x8 concat4(f16x4 lo, f16x4 hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ f16x8 lds_read_b128(const FA3_LDS char* lds, uint32_t byte_off) {
    return *(const FA3_LDS f16x8*)(lds + byte_off);
}

__device__ __forceinline__ void lds_write_b128(FA3_LDS char* lds, uint32_t byte_off, f16x8 v) {
    *(FA3_LDS f16x8*)(lds + byte_off) = v;
}

__device__ __forceinline__ void lds_write_b64(FA3_LDS char* lds, uint32_t byte_off, f16x4 v) {
    *(FA3_LDS f16x4*)(lds + byte_off) = v;
}

// Swizzle of a 128-byte row (8 chunks of 16 B, two rows per 64-bank line):
// rows of equal parity get distinct 3-bit masks over 8 consecutive rows, and
// rows r, r + 2 (r % 4 == 0) differ in bit 2, so 4 rows x 4 consecutive
// chunks of a transposed read land on 16 distinct 4-bank windows.
__device__ __forceinline__ int swz128(int row) {
    return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
}

// Row-major [rows][D] fp16 tile with 16-byte chunks XOR-swizzled per row.
// For D = 128 (16 chunks, one row per 64-bank line) the mask
// 4 * (r % 4) + (r / 4) % 4 makes both access patterns conflict free:
// 16 consecutive rows reading one logical chunk (ds_read_b128), and 4
// consecutive rows x 4 consecutive chunks (ds_read_b64_tr_b16, 32 lanes).
template <int D>
__device__ __forceinline__ uint32_t tile_off(int row, int chunk) {
    constexpr int kChunks = D / 8;
    static_assert(kChunks == 16 || kChunks == 8, "head dim 64 or 128");
    int sw;
    if constexpr (kChunks == 16) {
        sw = ((row & 3) << 2) | ((row >> 2) & 3);
    } else {
        sw = swz128(row);
    }
    return (uint32_t)(row * (D * 2) + ((chunk ^ sw) & (kChunks - 1)) * 16);
}

}  // namespace fa3
