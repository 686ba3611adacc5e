// sp_device.h -- device helpers and launch plans shared by the gfx950 kernels.
//
// Floating-point contract: every file including this is compiled with
// -ffp-contract=off, so a*b+c is two rounded operations unless a kernel calls
// fmaf() explicitly (only the attention kernel does, where results are
// compared within a tolerance rather than bit-exactly).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SP_WAVE 64
#define SP_MAX_BANDS_DEV 16
#define SP_MAX_CHUNKS 128     // head_dim / 8 for head_dim <= 1024
#define SP_GEN_MAX_N 512      // generic (one vector per wave) kernels: padded dim <= 512
#define SP_GEN_MAX_REC 1024   // generic kernels: record bytes <= 1024

// Cas tables for the primes 2,3,5,7,11 packed back to back.
#define SP_CAS_OFF2 0
#define SP_CAS_OFF3 4
#define SP_CAS_OFF5 13
#define SP_CAS_OFF7 38
#define SP_CAS_OFF11 87
#define SP_CAS_TOTAL 208

// Launch plan of one band configuration (host-built, passed by value).
struct SpPlan {
    int hd;           // coefficients per vector (transform length for the ship path)
    int n_bands;
    int total_bytes;  // record bytes
    int norm;         // 0: final 1/sqrt(n) multiply, 1: per-stage 1/sqrt(2)
    float inv_sqrt_n; // 1.0f / sqrtf((float)hd)
    int max_bands;    // decode: bands >= max_bands reconstruct as 0.0f
    int n_factors;    // Vilenkin stage primes (non power-of-2 transforms)
    int chunk_ok;     // 1 when every band boundary is a multiple of 8 coefficients
    int skip_transform; // 1: identity transform (quantize/dequantize-only launchers)
    int order_default;  // 1: the Mobius table passed with this plan is the default squarefree-first order
    unsigned char factors[16];
    unsigned char band_bits[SP_MAX_BANDS_DEV];
    short band_off[SP_MAX_BANDS_DEV];
    short band_sz[SP_MAX_BANDS_DEV];
    short band_byte_off[SP_MAX_BANDS_DEV];
    unsigned char chunk_band[SP_MAX_CHUNKS];
    unsigned char chunk_first[SP_MAX_CHUNKS];
    unsigned char chunk_last[SP_MAX_CHUNKS];
    short chunk_byte_off[SP_MAX_CHUNKS];
    float cas[SP_CAS_TOTAL];
    float isp[5];     // 1.0f/sqrtf(p) for p = 2,3,5,7,11
};

__device__ __forceinline__ int sp_cas_off(int p) {
    return p == 2 ? SP_CAS_OFF2 : p == 3 ? SP_CAS_OFF3 : p == 5 ? SP_CAS_OFF5
         : p == 7 ? SP_CAS_OFF7 : SP_CAS_OFF11;
}
__device__ __forceinline__ int sp_prime_idx(int p) {
    return p == 2 ? 0 : p == 3 ? 1 : p == 5 ? 2 : p == 7 ? 3 : 4;
}

// IEEE round-to-nearest-even float -> binary16 bits, in integer arithmetic so
// the result is defined independent of the hardware converter's modes.
__device__ __forceinline__ uint32_t sp_f32_to_f16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    int e = (int)(ax >> 23) - 127;
    uint32_t m = ax & 0x7fffffu;
    if (e > 15) return sign | 0x7c00u;
    if (e >= -14) {
        uint32_t keep = m >> 13, rem = m & 0x1fffu;
        uint32_t r = ((uint32_t)(e + 15) << 10) | keep;
        if (rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) r += 1;
        return sign | r;
    }
    if (ax == 0) return sign;
    int shift = -e - 1;
    if (shift > 24) return sign;
    uint32_t mfull = m | 0x800000u;
    uint32_t keep = mfull >> shift;
    uint32_t rem = mfull & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (keep & 1u))) keep += 1;
    return sign | keep;
}

__device__ __forceinline__ float sp_f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (unsigned short)h);
    return (float)v;
}

// Stored scale -> multiplier used by dequantization: non-finite -> 0.
__device__ __forceinline__ float sp_scale_from_bits(uint32_t h) {
    if ((h & 0x7c00u) == 0x7c00u) return 0.0f;
    return sp_f16_bits_to_f32(h);
}

// rint (half-even), NaN -> 0, clamp to [-m, m].
__device__ __forceinline__ int sp_q_rint_clamp(float v, int m) {
    float r = __builtin_rintf(v);
    if (r != r) return 0;
    float fm = (float)m;
    r = r > fm ? fm : r;
    r = r < -fm ? -fm : r;
    return (int)r;
}

// Truncation toward zero with NaN -> 0 and saturation (C (int) cast semantics
// of the reference's residual quantizer).
__device__ __forceinline__ int sp_trunc_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483647.0f) return 2147483647;
    if (x <= -2147483648.0f) return (int)0x80000000u;
    return (int)x;
}

__device__ __forceinline__ int sp_rint_sat(float x) {
    float r = __builtin_rintf(x);
    if (r != r) return 0;
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return (int)0x80000000u;
    return (int)r;
}

// Correctly rounded fp32 division (IEEE), independent of fast-math flags.
__device__ __forceinline__ float sp_div(float a, float b) { return __fdiv_rn(a, b); }

// Wave-wide all-reduce on the VALU (no LDS round trips): DPP quad permutes and row
// mirrors inside each row of 16 lanes, then the gfx950 row swaps across rows.
// permlane16/32_swap(v, v) return this lane's value and its partner's (lane ^ 16,
// lane ^ 32) in an order that depends on the lane, so a commutative op of the two
// gives every lane the same result. Call with the whole wave active.
template <class Op>
__device__ __forceinline__ float sp_wave_allreduce(float v, Op op) {
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));   // quad [1,0,3,2]
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));   // quad [2,3,0,1]
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));  // row_half_mirror
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));  // row_mirror
    u32x2_t t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(t[0]), __uint_as_float(t[1]));
    t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
// sum and maximum (of non-NaN values) over the wave, every lane active
__device__ __forceinline__ float sp_wave_sum_dpp(float v) {
    return sp_wave_allreduce(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float sp_wave_max_dpp(float v) {
    return sp_wave_allreduce(v, [](float a, float b) { return fmaxf(a, b); });
}

// Wave-wide max of non-NaN values.
__device__ __forceinline__ float sp_wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, SP_WAVE));
    return v;
}

// Sum in the order of a 256-thread shared-memory tree reduction: slot t
// accumulates v[t], v[t+256], ... from 0.0f, then slot[t] += slot[t+s] for
// s = 128, 64, ..., 1. Lane l holds slots l, l+64, l+128, l+192. `vals` is LDS.
// Result valid in every lane.
__device__ __forceinline__ float sp_wave_tree256_sum(const float *vals, int n, int take_abs,
                                                     int lane) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    for (int i = lane; i < n; i += 256) { float a = vals[i]; s0 += take_abs ? fabsf(a) : a; }
    for (int i = lane + 64; i < n; i += 256) { float a = vals[i]; s1 += take_abs ? fabsf(a) : a; }
    for (int i = lane + 128; i < n; i += 256) { float a = vals[i]; s2 += take_abs ? fabsf(a) : a; }
    for (int i = lane + 192; i < n; i += 256) { float a = vals[i]; s3 += take_abs ? fabsf(a) : a; }
    s0 += s2;  // s = 128: slot l += slot l+128
    s1 += s3;  //          slot l+64 += slot l+192
    s0 += s1;  // s = 64
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) s0 += __shfl_down(s0, s, SP_WAVE);
    return __shfl(s0, 0, SP_WAVE);
}
