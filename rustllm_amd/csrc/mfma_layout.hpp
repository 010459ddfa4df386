// mfma_layout.hpp -- operand layouts shared by the matrix-core kernels of
// attention.hip and gqa.hip (gfx950, wave64).
//
// v_mfma_f32_32x32x16_f16 and v_mfma_f32_32x32x2_f32 take A / B operands
// with lane l holding row (A) or column (B) l % 32 and the inner-dimension
// slice l / 32; the 32 x 32 result leaves lane l with column l % 32 and, in
// register r, row 8 (r / 4) + 4 (l / 32) + r % 4.  The key orders below
// choose which key each result row holds so that a lane's registers come
// out in the operand layout of the next product.
#ifndef RUSTLLM_MFMA_LAYOUT_HPP
#define RUSTLLM_MFMA_LAYOUT_HPP

#include "common.hpp"

namespace rl {
namespace {

typedef half_t h8 __attribute__((ext_vector_type(8)));
typedef half_t h4 __attribute__((ext_vector_type(4)));
typedef half_t h2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// f16: row i of a 32-key S^T tile holds key perm32(i), bits 2 and 3 of i
// swapped; register r of lane l then holds key 16 (r / 8) + 8 (l / 32) +
// r % 8 -- eight consecutive keys per lane half, the B operand layout of
// the P V product over 16 keys.
__device__ inline uint32_t perm32(uint32_t i) {
    return (i & ~12u) | ((i & 4u) << 1) | ((i & 8u) >> 1);
}

// f32: LDS row i = 8a + 4h + b of a 32-key tile holds key 8a + 2b + h (the
// low three bits rotated), so that register r of a lane in half h holds key
// 2r + h -- the B operand of the P V step over keys 2r and 2r + 1.
// key_row32 is the row of key j.
__device__ inline uint32_t key_row32(uint32_t j) {
    return (j & ~7u) | ((j & 1u) << 2) | ((j >> 1) & 3u);
}

// Row stride (halves) of V in LDS for the transpose reads: the 32 lanes one
// LDS cycle serves read 4 rows x 2 runs of 16 bytes; with 64 banks of 4
// bytes those land on distinct banks when the stride in dwords is 16 or 48
// modulo 64.  Smallest such stride >= D (in steps of 8 halves).
__host__ __device__ constexpr int v_stride_tr(int d) {
    int s = d;
    while ((s / 2) % 64 != 16 && (s / 2) % 64 != 48) s += 8;
    return s;
}

// Row strides (floats) of f32 tiles in LDS.  An operand read that takes one
// element of 32 rows (lanes 0-31) and the next element of the same rows
// (lanes 32-63) hits 64 banks at a stride of 2 mod 64; one that takes 32
// consecutive elements of two adjacent rows does at 32 mod 64.
__host__ __device__ constexpr int f32_stride(int d, int residue) {
    int s = d;
    while (s % 64 != residue) ++s;
    return s;
}

// ds_read_b64_tr_b16: in each group of 16 lanes, lanes 4j .. 4j + 3 read 8
// bytes each (row j of a 4 x 16 block of halves); lane i of the group
// receives column i of that block, one half from each row.
__device__ inline h4 lds_read_transposed(const half_t* p) {
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(p));
    return __builtin_bit_cast(h4, r);
}

}  // namespace
}  // namespace rl

#endif
