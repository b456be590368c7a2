// int2_decode.hpp -- in-register unpack of the packed 2-bit weight word.
//
// A B word holds the codes of 16 consecutive K rows of one column, row j at
// bits 2j..2j+1, codes {0, 1, 3} = {0, +1, -1} (int2_fp16_upcvt.cl:6-19).
//
// GEMV decode ("mantissa-field" decode, 1.1-1.4 VALU ops per weight).
// After t = w ^ 0xAAAAAAAA every 2-bit field holds x = v + 2 (v the signed
// weight value: code 0 -> 2, 1 -> 3, 3 -> 1).  One v_and_or_b32
//   d = (t & ((3 << p) | (3 << (p + 16)))) | BASE2
// then puts the field of row j (low half) and of row j + 8 (high half) into the
// low mantissa bits of two DT numbers equal to BASE + x * 2^p exactly
// (BASE = 1024 for fp16, whose mantissa LSB is 1 there; 128 for bf16).  A dot
// product with the activations pre-scaled by 2^-p gives
//   sum a'(BASE + 2^p x) = BASE * sum a' + sum a x,   sum a v = sum a x - 2 sum a,
// so one correction per 128-row group, beta = BASE * sum a' + 2 * sum a, which
// depends only on the activations, recovers sum a v.
//
// The 8 pairs of a word, pair j = (row j, row j + 8), field shift p_j:
//   fp16: t at p = 0,2,4,6,8 (j = 0..4), t >> 8 at p = 2,4,6 (j = 5..7)
//   bf16: t at p = 0,2,4 (j = 0..2), t >> 6 at p = 0,2,4 (j = 3..5),
//         t >> 12 at p = 0,2 (j = 6,7)
#pragma once
#include <stdint.h>

namespace tcl {

// field shift of pair j
__host__ __device__ constexpr int gemv_pair_shift(bool bf16, int j) {
    return bf16 ? (j < 3 ? 2 * j : (j < 6 ? 2 * (j - 3) : 2 * (j - 6)))
                : (j < 5 ? 2 * j : 2 * (j - 4));
}
__host__ __device__ constexpr float gemv_base(bool bf16) { return bf16 ? 128.0f : 1024.0f; }
__host__ __device__ constexpr uint32_t gemv_base2(bool bf16) { return bf16 ? 0x43004300u : 0x64006400u; }

// One v_and_or_b32.  gfx9 VOP3 encodings take no literal constant, so the
// mask goes in an SGPR and the base in a VGPR (one of each keeps the constant
// bus limit); written as inline asm because the compiler otherwise emits a
// v_and_b32 + v_or_b32 pair with literals.
__device__ __forceinline__ uint32_t and_or(uint32_t t, uint32_t mask, uint32_t base2) {
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(t), "s"(mask), "v"(base2));
    return d;
}
__device__ __forceinline__ uint32_t fld(uint32_t t, int p, uint32_t base2) {
    return and_or(t, (3u << p) | (3u << (p + 16)), base2);
}

// base2: a register holding 0x64006400 (fp16 1024, 1024) or 0x43004300 (bf16
// 128, 128), see gemv_base2().
template <bool BF16>
__device__ __forceinline__ void gemv_decode_word(uint32_t w, uint32_t d[8], uint32_t B2) {
    const uint32_t t = w ^ 0xAAAAAAAAu;
    if constexpr (!BF16) {
        d[0] = fld(t, 0, B2);
        d[1] = fld(t, 2, B2);
        d[2] = fld(t, 4, B2);
        d[3] = fld(t, 6, B2);
        d[4] = fld(t, 8, B2);
        const uint32_t t1 = t >> 8;
        d[5] = fld(t1, 2, B2);
        d[6] = fld(t1, 4, B2);
        d[7] = fld(t1, 6, B2);
    } else {
        d[0] = fld(t, 0, B2);
        d[1] = fld(t, 2, B2);
        d[2] = fld(t, 4, B2);
        const uint32_t t1 = t >> 6;
        d[3] = fld(t1, 0, B2);
        d[4] = fld(t1, 2, B2);
        d[5] = fld(t1, 4, B2);
        const uint32_t t2 = t >> 12;
        d[6] = fld(t2, 0, B2);
        d[7] = fld(t2, 2, B2);
    }
}

// Reference-semantics unpack (int2_fp16_upcvt.cl:95-116): the DT weight of
// row j of the word, +0 / +s / s ^ 0x8000.
__device__ __forceinline__ uint32_t dq_one(uint32_t w, int j, uint32_t s) {
    const uint32_t c = (w >> (2 * j)) & 3u;
    return (c & 1u) ? (s ^ ((c & 2u) << 14)) : 0u;
}

}  // namespace tcl
