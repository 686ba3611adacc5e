// sp_mfma_codes.h -- packed band codes -> fp16 A operands of v_mfma_f32_16x16x32_f16,
// shared by the fused attention kernels (ship records, hier skeleton bands).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Code pairs as fp16 2^BITS + u (exact): the code sits in the top BITS bits of
// the mantissa under the exponent of 2^BITS. The MFMA accumulator starts at
// -(2^BITS + m_b) * sum(B column over the band), which centres the codes. The
// offset 2^BITS is kept as small as the format allows: the fp32 accumulator
// holds (2^BITS + m_b) * sum|q~| before the centring cancels it, so each bit of
// offset costs a bit of score precision.
// Two adjacent BITS-bit codes y = c0 | c1 << BITS at bit `off` of x: y times
// 2^(10-BITS) + 2^(26-2*BITS) puts c0 at bits [10-BITS, 10) and c1 at
// [26-BITS, 26) (the other two copies land in disjoint fields, so nothing
// carries), and the mask keeps those two. The mask and the exponent bits
// arrive in registers (kmask, kbias) so one three-input bit operation,
// (a & b) | c, finishes the pair.
template <int BITS>
__device__ __forceinline__ constexpr uint32_t code_mask() {
    return (((1u << BITS) - 1u) << (10 - BITS)) * 0x10001u;
}
template <int BITS>
__device__ __forceinline__ constexpr uint32_t code_bias() {
    return ((uint32_t)(15 + BITS) << 10) * 0x10001u;  // fp16 2^BITS in both halves
}
template <int BITS>
__device__ __forceinline__ uint32_t code_pair(uint32_t x, uint32_t off, uint32_t kmask, uint32_t kbias) {
    const uint32_t y = __builtin_amdgcn_ubfe(x, off, 2 * BITS);
    return __builtin_amdgcn_bitop3_b32(y * ((1u << (10 - BITS)) + (1u << (26 - 2 * BITS))),
                                       kmask, kbias, 0xEA);
}

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(half8_t, v);
}

// Eight consecutive codes of one band (bits [sh, sh + 8*BITS) of d1:d0) -> the
// lane's 8-slot A operand of v_mfma_f32_16x16x32_f16. 5- and 3-bit bands: slot
// e holds code e. 4-bit band: codes i and i + 4 sit 16 bits apart already, so
// the slots hold codes (0,4,1,5,2,6,3,7).
template <int BITS>
__device__ __forceinline__ half8_t band_codes(uint32_t d0, uint32_t d1, uint32_t sh, uint32_t kmask, uint32_t kbias) {
    const uint32_t lo = __builtin_amdgcn_alignbit(d1, d0, sh);  // window bits 0..31
    if (BITS == 4)  // codes k and k + 4 (bits 4k, 4k + 16) move to bits 6..9 and 22..25
        return as_half8(__builtin_amdgcn_bitop3_b32(lo << 6, kmask, kbias, 0xEA),
                        __builtin_amdgcn_bitop3_b32(lo << 2, kmask, kbias, 0xEA),
                        __builtin_amdgcn_bitop3_b32(lo >> 2, kmask, kbias, 0xEA),
                        __builtin_amdgcn_bitop3_b32(lo >> 6, kmask, kbias, 0xEA));
    uint32_t p67;
    if (BITS == 5) p67 = code_pair<5>(__builtin_amdgcn_alignbit(d1 >> sh, lo, 30), 0, kmask, kbias);  // bits 30..39
    else p67 = code_pair<BITS>(lo, 6 * BITS, kmask, kbias);
    return as_half8(code_pair<BITS>(lo, 0, kmask, kbias), code_pair<BITS>(lo, 2 * BITS, kmask, kbias),
                    code_pair<BITS>(lo, 4 * BITS, kmask, kbias), p67);
}

// Slot (0..7) of a lane's band operand for code c (0..7) of its run of eight,
// for a band of `bits`-bit codes (see band_codes: 4-bit bands interleave).
__device__ __forceinline__ int code_slot_bits(int bits, int c) {
    return bits == 4 ? ((((c & 3) >> 1) << 2) | ((c & 1) << 1) | (c >> 2)) : c;
}

}  // namespace
