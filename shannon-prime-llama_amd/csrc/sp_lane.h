// sp_lane.h -- device building blocks of the one-vector-per-lane codec kernels:
// compile-time band layouts and the Mobius order, register transforms (p = 2
// VHT2 and the staged Vilenkin-Hartley transform), record bit fields, band
// quantize/dequantize, 64-row tiles moved through LDS with coalesced buffer
// loads and stores, and the host-side launch helpers they share.
#pragma once
#include <stdlib.h>

#include <algorithm>

#include "sp_internal.h"

namespace {


typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

typedef float float2v __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr uint32_t BUF_WORD3 = 0x00020000u;  // raw buffer resource, dword data (gfx9 family)
constexpr int BUF_NT = 2;                    // non-temporal cache policy (streamed rows and records)

// Raw buffer over [p, p + nbytes): loads past nbytes return 0 (the range check
// covers the vector, scalar and immediate offsets alike).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, int nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, nbytes, BUF_WORD3);
}

constexpr bool c_squarefree(int n) {
    for (int p = 2; p * p <= n; p++)
        if (n % (p * p) == 0) return false;
    return true;
}

// Squarefree-first order (i+1 squarefree ascending, then the rest ascending):
// the same table the host builds for d_mobius_order.
template <int N>
struct MobOrder {
    int v[N];
    constexpr MobOrder() : v() {
        int r = 0;
        for (int i = 0; i < N; i++)
            if (c_squarefree(i + 1)) v[r++] = i;
        for (int i = 0; i < N; i++)
            if (!c_squarefree(i + 1)) v[r++] = i;
    }
};
template <int N>
__device__ constexpr MobOrder<N> kMob{};

// coefficient feeding reordered position r (identity without Mobius)
template <int HD, bool MOB>
__device__ __forceinline__ constexpr int src_idx(int r) { return MOB ? kMob<HD>.v[r] : r; }

template <int HD, int... BITS>
struct Layout {
    static constexpr int hd = HD;
    static constexpr int nb = sizeof...(BITS);
    static constexpr int bits[nb] = {BITS...};
    static constexpr int bsz = HD / nb;
    static constexpr int off(int b) { return b * bsz; }
    static constexpr int sz(int b) { return b == nb - 1 ? HD - b * bsz : bsz; }
    static constexpr int byte_off(int b) {
        int o = 0;
        for (int i = 0; i < b; i++) o += 2 + (sz(i) * bits[i] + 7) / 8;
        return o;
    }
    static constexpr int total = byte_off(nb);
    static constexpr int dwords = (total + 3) / 4;
};

constexpr int c_log2(int n) { return n <= 1 ? 0 : 1 + c_log2(n / 2); }

// Insert / extract a field of width w at bit position pos of the record
// dwords. Called from fully unrolled loops, so pos and w fold to constants.
template <int DW>
__device__ __forceinline__ void rec_insert(uint32_t (&rec)[DW], int pos, int w, uint32_t val) {
    const int d = pos / 32, sh = pos % 32;
    rec[d] |= val << sh;
    if (sh + w > 32) rec[d + 1] |= val >> (32 - sh);
}

// Add val << pos into the record words (val < 2^w, the field's bits zero before):
// with disjoint fields, addition is insertion, and a chain of these folds into
// one shift-and-add per field.
template <int DW>
__device__ __forceinline__ void rec_add(uint32_t (&rec)[DW], int pos, int w, uint32_t val) {
    const int d = pos / 32, sh = pos % 32;
    rec[d] += val << sh;
    if (sh + w > 32) rec[d + 1] += val >> (32 - sh);
}

// The code field of one quantized coefficient, from tb = bits(fl(v + 1.5*2^23))
// with rint(v) = q in [-m, m]: tb = 0x4B400000 + q exactly, so the code q + m
// is tb + (m - 0x4B400000) in 32-bit arithmetic. A field inside one word adds
// (tb << sh) and the compile-time constant (m - 0x4B400000) << sh, which the
// compiler merges across the word's fields into one constant: one shift-and-add
// per code. A field that crosses into the next word forms the code first.
template <int DW>
__device__ __forceinline__ void rec_add_code(uint32_t (&rec)[DW], int pos, int w, uint32_t tb, int m) {
    const int d = pos / 32, sh = pos % 32;
    const uint32_t bias = (uint32_t)m - 0x4B400000u;
    if (sh + w <= 32) {
        rec[d] += (tb << sh) + (bias << sh);
    } else {
        const uint32_t code = tb + bias;
        rec[d] += code << sh;
        rec[d + 1] += code >> (32 - sh);
    }
}

// fp16 pair (lo, hi) of w -> (lo + hi, lo - hi) in fp32: v_fma_mix widens each
// half exactly and rounds once, the same result as convert-then-add.
__device__ __forceinline__ void bfly_f16_pair(uint32_t w, float &s, float &d) {
    __asm__("v_fma_mix_f32 %0, %2, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[1,0,1]\n\t"
            "v_fma_mix_f32 %1, %2, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[1,0,1]"
            : "=&v"(s), "=v"(d)
            : "v"(w));
}

template <int DW>
__device__ __forceinline__ uint32_t rec_extract(const uint32_t (&rec)[DW], int pos, int w) {
    const int d = pos / 32, sh = pos % 32;
    const uint32_t mask = (1u << w) - 1u;
    if (sh + w <= 32) return (rec[d] >> sh) & mask;
    return __builtin_amdgcn_alignbit(rec[d + 1], rec[d], sh) & mask;
}

// 32-bit field at a byte offset of the record dwords (the f32 magnitude).
template <int DW>
__device__ __forceinline__ void rec_put32(uint32_t (&rec)[DW], int byte, uint32_t v) {
    const int d = byte / 4, sh = 8 * (byte % 4);
    rec[d] |= v << sh;
    if (sh) rec[d + 1] |= v >> (32 - sh);
}

template <int DW>
__device__ __forceinline__ uint32_t rec_get32(const uint32_t (&rec)[DW], int byte) {
    const int d = byte / 4, sh = 8 * (byte % 4);
    return sh ? __builtin_amdgcn_alignbit(rec[d + 1], rec[d], sh) : rec[d];
}

// a + b with |.| applied to the operands flagged (source modifiers of one v_add_f32;
// the same rounding as the separate absolute values and add)
template <bool AA, bool AB>
__device__ __forceinline__ float add_abs_mod(float a, float b) {
    if constexpr (!AA && !AB) return a + b;
    float r;
    if constexpr (AA && AB) __asm__("v_add_f32_e64 %0, |%1|, |%2|" : "=v"(r) : "v"(a), "v"(b));
    else if constexpr (AA) __asm__("v_add_f32_e64 %0, |%1|, %2" : "=v"(r) : "v"(a), "v"(b));
    else __asm__("v_add_f32_e64 %0, %1, |%2|" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Whether slot t of tree256_sum<N> still holds a raw v[t] after stage s (s = 256: the
// v[t + 256] pass, then 128..1): every slot's first add applies the |.| it owes.
template <int N>
__device__ constexpr bool tree_slot_raw(int t, int s) {
    if (t + 256 < N) return false;  // paired with v[t + 256] first
    int n = N < 256 ? N : 256;
    for (int k = 128; k >= s && k > 0; k >>= 1) {
        if (t < k && t + k < n) return false;  // accumulated at stage k
        if (t >= k && t < n) return false;     // added into slot t - k at stage k
        n = n < k ? n : k;
    }
    return true;
}

// Sum in the order of the reference's 256-slot block reductions over n values
// (slot t accumulates v[t], v[t + 256] from 0.0f, then slot[t] += slot[t + s]
// for s = 128..1); slots at or past n hold +0.0f, so adding them is skipped.
// ABS: |v| terms (never -0, so the 0.0f start drops out). For signed terms the
// result is the plain tree sum plus 0.0f: every difference the 0.0f starts can
// make is the sign of a zero sum, which the final + 0.0f maps to the
// reference's +0.
template <int N, bool ABS>
__device__ __forceinline__ float tree256_sum(const float *v) {
    static_assert(N <= 512, "at most two values per slot");
    constexpr int NS = N < 256 ? N : 256;
    float sl[NS];
    if constexpr (ABS) {
        // the absolute values ride on the first add each term takes part in
#pragma unroll
        for (int t = 0; t < NS; t++) sl[t] = t + 256 < N ? add_abs_mod<true, true>(v[t], v[t + 256]) : v[t];
        int n = NS;
#pragma unroll
        for (int s = 128; s > 0; s >>= 1) {
#pragma unroll
            for (int t = 0; t < s; t++) {
                if (t + s < n) {
                    const bool ra = tree_slot_raw<N>(t, 2 * s), rb = tree_slot_raw<N>(t + s, 2 * s);
                    if (ra && rb) sl[t] = add_abs_mod<true, true>(sl[t], sl[t + s]);
                    else if (ra) sl[t] = add_abs_mod<true, false>(sl[t], sl[t + s]);
                    else if (rb) sl[t] = add_abs_mod<false, true>(sl[t], sl[t + s]);
                    else sl[t] = sl[t] + sl[t + s];
                }
            }
            n = n < s ? n : s;
        }
        return tree_slot_raw<N>(0, 1) ? fabsf(sl[0]) : sl[0];
    } else {
#pragma unroll
        for (int t = 0; t < NS; t++) sl[t] = v[t];
#pragma unroll
        for (int t = 0; t + 256 < N; t++) sl[t] = sl[t] + v[t + 256];
        int n = NS;
#pragma unroll
        for (int s = 128; s > 0; s >>= 1) {
#pragma unroll
            for (int t = 0; t < s; t++)
                if (t + s < n) sl[t] = sl[t] + sl[t + s];
            n = n < s ? n : s;
        }
        return sl[0] + 0.0f;
    }
}

// p=2 VHT2 over a register-resident vector: stages len = 1, 2, ..., HD/2 in
// order (the stage order fixes the fp32 rounding), then the final 1/sqrt(n)
// multiply (NORM 0) or per-stage 1/sqrt(2) (NORM 1).
template <int HD, int NORM>
__device__ __forceinline__ void vht2_reg(float (&x)[HD], float inv_sqrt_n, bool first_done) {
    const float s2 = 0.70710678118654752440f;
#pragma unroll
    for (int len = first_done ? 2 : 1; len < HD; len <<= 1) {
#pragma unroll
        for (int k = 0; k < HD / 2; k++) {
            const int i = (k / len) * 2 * len + (k % len);
            const float u = x[i], v = x[i + len];
            if (NORM == 1) {
                x[i] = (u + v) * s2;
                x[i + len] = (u - v) * s2;
            } else {
                x[i] = u + v;
                x[i + len] = u - v;
            }
        }
    }
    if (NORM == 0) {
#pragma unroll
        for (int i = 0; i < HD; i++) x[i] *= inv_sqrt_n;
    }
}

// ---- staged Vilenkin-Hartley transform for non-power-of-two lengths ----
// Constants of the transforms, passed by value (they land in scalar registers):
// cas[pi][m] = (float)(cos(2*pi*m/p) + sin(2*pi*m/p)) and isp[pi] = 1.0f/sqrtf(p)
// for p = 2, 3, 5, 7, 11 (pi = 0..4), exactly the values of the host plan.
struct XfConst {
    float inv_sqrt_n;
    float isp[5];
    float cas[5][11];
};

constexpr int c_prime(int i) { return i == 0 ? 2 : i == 1 ? 3 : i == 2 ? 5 : i == 3 ? 7 : 11; }
constexpr int c_prime_idx(int p) { return p == 2 ? 0 : p == 3 ? 1 : p == 5 ? 2 : p == 7 ? 3 : 4; }
constexpr bool c_pow2(int n) { return n > 0 && (n & (n - 1)) == 0; }

// prime factors of N among {2, 3, 5, 7, 11}, ascending with multiplicity
template <int N>
struct Factors {
    int p[16];
    int n;
    int rest;
    constexpr Factors() : p(), n(0), rest(N) {
        for (int i = 0; i < 5; i++)
            while (rest % c_prime(i) == 0 && n < 16) {
                p[n++] = c_prime(i);
                rest /= c_prime(i);
            }
    }
};

// One stage with prime P at stride S (kernel_vilenkin_inplace order,
// shannon_prime_sqfree.cu:66-106): each group {base + k*S} becomes
// r[k] = (sum_j C[k][j] * g[j]) * (1/sqrt(P)), the sum running from 0.0f over j
// ascending with separately rounded products and adds. C[k][0] = C[0][j] = 1
// exactly and C = -1 exactly for P = 2 (the host checks), so those products are
// the value itself; 0.0f + g[0] is kept (it maps -0 to +0 as the reference does).
template <int N, int P, int S>
__device__ __forceinline__ void vil_stage(float (&x)[N], const XfConst &K) {
    constexpr int PI = c_prime_idx(P), BLOCK = S * P;
    const float isp = K.isp[PI];
#pragma unroll
    for (int blk = 0; blk < N / BLOCK; blk++) {
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int base = blk * BLOCK + s;
            float g[P];
#pragma unroll
            for (int k = 0; k < P; k++) g[k] = x[base + k * S];
            const float z = 0.0f + g[0];
#pragma unroll
            for (int k = 0; k < P; k++) {
                float sum = z;
#pragma unroll
                for (int j = 1; j < P; j++) {
                    const int m = (k * j) % P;
                    if (m == 0) sum = sum + g[j];
                    else if (P == 2) sum = sum - g[j];
                    else sum = sum + K.cas[PI][m] * g[j];
                }
                x[base + k * S] = sum * isp;
            }
        }
    }
}

template <int N, int FI, int S>
__device__ __forceinline__ void vil_stages(float (&x)[N], const XfConst &K) {
    constexpr Factors<N> F{};
    if constexpr (FI < F.n) {
        constexpr int P = F.p[FI];
        vil_stage<N, P, S>(x, K);
        vil_stages<N, FI + 1, S * P>(x, K);
    }
}

// First stage (P = 2, stride 1) straight from fp16 pairs: v_fma_mix widens
// exactly and rounds once, so z = lo + 0.0f, r0 = z + hi, r1 = z - hi match
// the fp32 stage bit for bit.
__device__ __forceinline__ void vil_first_f16_pair(uint32_t w, float isp, float &r0, float &r1) {
    float z, a, b;
    __asm__("v_fma_mix_f32 %0, %1, 1.0, 0 op_sel_hi:[1,0,0]" : "=v"(z) : "v"(w));
    __asm__("v_fma_mix_f32 %0, %2, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %1, -%2, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "=&v"(a), "=v"(b)
            : "v"(w), "v"(z));
    r0 = a * isp;
    r1 = b * isp;
}

__device__ __forceinline__ uint32_t f16_normal(uint32_t h) {
    const uint32_t e = h & 0x7c00u;
    return e != 0u && e != 0x7c00u;
}

template <int DT>
constexpr int row_bytes(int hd) { return hd * (DT == SP_DT_F16 ? 2 : 4); }


// Chunk k of lane j of a 64-row tile moved with wave-wide 16-byte accesses:
// chunk 64k + j is row (64k + j) / CPR, column (64k + j) % CPR. When CPR
// divides 64 the row offset splits into a lane part (vector offset) and a
// uniform part k * (64 / CPR) rows (scalar offset); otherwise the whole
// offset is per lane.
template <int CPR>
struct TileChunk {
    int row, col, krow;
    __device__ __forceinline__ TileChunk(int k, int lane) {
        if (64 % CPR == 0) {
            row = lane / CPR, col = lane % CPR, krow = k * (64 / CPR);
        } else {
            const int c = 64 * k + lane;
            row = c / CPR, col = c % CPR, krow = 0;
        }
    }
    __device__ __forceinline__ int vofs(int rowb) const { return row * rowb + col * 16; }
    __device__ __forceinline__ int sofs(int rowb) const { return krow * rowb; }
    __device__ __forceinline__ int lds(int rp) const { return (row + krow) * rp + col * 16; }
};

struct TileMap {
    int tpo;      // tiles per outer row
    int n_inner;
    __device__ __forceinline__ void at(int t, int &o, int &i0, int &nvalid) const {
        o = t / tpo;
        i0 = (t - o * tpo) * 64;
        nvalid = min(64, n_inner - i0);
    }
};


// a / m for a finite a >= 0 and a band's largest level m = 2^(bits-1) - 1: with
// r = fl(1/m), q0 = fl(a*r), the remainder a - q0*m is exact in one fma and
// fl(q0 + rem*r) is the correctly rounded quotient. This was checked against
// IEEE division for every fp32 significand and every m in {1, 3, 7, ..., 127};
// the steps scale exactly with the exponent while the quotient is a normal
// number. (Smaller quotients only occur for amax < 2^-119, whose fp16 scale is
// 0 either way; a 1-bit band, m = 0, gets a non-finite scale and the exact path.)
__device__ __forceinline__ float div_by_level(float a, int m) {
    const float fm = (float)m, r = 1.0f / fm;  // compile-time constants
    const float q0 = a * r;
    const float rem = __builtin_fmaf(-q0, fm, a);
    return __builtin_fmaf(rem, r, q0);
}

// 1/s correctly rounded for s > 0 an fp16 value widened to fp32: one Newton
// step with fma from v_rcp_f32 (specified to 1 ulp). Checked for all 1024 fp16
// significands with the starting value anywhere within +-3 ulp of 1/s; s and
// 1/s stay normal fp32 numbers, so the exponent scales out exactly.
__device__ __forceinline__ float rcp_f16_scale(float s) {
    const float r0 = __builtin_amdgcn_rcpf(s);
    const float e = __builtin_fmaf(-s, r0, 1.0f);
    return __builtin_fmaf(e, r0, r0);
}

// Band-quantize coefficients x[src_idx(r)], r in [0, LY::hd), into the record
// bits [0, 8 * LY::total) of rec (which must start zeroed there):
// kernel_band_quantize_simple (shannon_prime_cuda.cu:131-204). fastv: every
// coefficient is finite.
//
// Fast path, for every lane: when the band's stored fp16 scale is a normal
// number, |x*inv| <= maxv*(1 + 2^-10) < maxv + 1/2, so rint never needs the
// clamp, and t = x*inv + 1.5*2^23 rounds x*inv to the nearest integer q with
// ties to even (the added constant is even): bits(t) = 0x4B400000 + q, and the
// codes are summed into the record words (rec_add_code). A band whose scale is
// 0 uses inv = 0, as the reference does, and gets q = 0 everywhere. When any
// band has a subnormal or non-finite scale, or an input is not finite, the lane
// clears the record and redoes every band with the exact clamped rounding (a
// rare, divergent branch that overwrites the whole result).
template <class LY, bool MOB, int N, int DWR>
__device__ __forceinline__ void quant_bands(const float (&x)[N], bool fastv, uint32_t (&rec)[DWR]) {
    constexpr int HD = LY::hd;
    static_assert(DWR >= LY::dwords && N >= HD, "record and vector must hold the layout");
    bool ok = fastv;
#pragma unroll
    for (int b = 0; b < LY::nb; b++) {
        const int off = LY::off(b), sz = LY::sz(b), bits = LY::bits[b];
        const int maxv = (1 << (bits - 1)) - 1, bo = LY::byte_off(b);
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < sz; e++) amax = fmaxf(amax, fabsf(x[src_idx<HD, MOB>(off + e)]));
        float sc = div_by_level(amax, maxv);
        __asm__ volatile("" : "+v"(sc));  // keep the division and the conversion apart
        const uint32_t hf = (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)sc);
        const bool zero = hf == 0u;
        ok = ok && (zero || f16_normal(hf));
        const float inv = zero ? 0.0f : rcp_f16_scale(sp_f16_bits_to_f32(hf));
        rec_add(rec, 8 * bo, 16, hf);
#pragma unroll
        for (int e = 0; e < sz; e++) {
            const float t = x[src_idx<HD, MOB>(off + e)] * inv + 12582912.0f;
            rec_add_code(rec, 8 * (bo + 2) + e * bits, bits, __float_as_uint(t), maxv);
        }
    }
    if (!ok) {
        constexpr int TW = LY::total / 4, TB = LY::total % 4;
#pragma unroll
        for (int d = 0; d < TW; d++) rec[d] = 0u;
        if (TB) rec[TW] &= ~((1u << (8 * TB)) - 1u);
#pragma unroll
        for (int b = 0; b < LY::nb; b++) {
            const int off = LY::off(b), sz = LY::sz(b), bits = LY::bits[b];
            const int maxv = (1 << (bits - 1)) - 1, bo = LY::byte_off(b);
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < sz; e++) amax = fmaxf(amax, fabsf(x[src_idx<HD, MOB>(off + e)]));
            const float scale = (amax > 0.0f) ? sp_div(amax, (float)maxv) : 0.0f;
            const uint32_t h = sp_f32_to_f16_bits(scale);
            const float ss = sp_f16_bits_to_f32(h);
            const float inv = (ss > 0.0f) ? sp_div(1.0f, ss) : 0.0f;
            rec_insert(rec, 8 * bo, 16, h);
#pragma unroll
            for (int e = 0; e < sz; e++) {
                const int q = sp_q_rint_clamp(x[src_idx<HD, MOB>(off + e)] * inv, maxv);
                rec_insert(rec, 8 * (bo + 2) + e * bits, bits, (uint32_t)(q + maxv));
            }
        }
    }
}

// Dequantize the record's bands into x[src_idx(r)] (bands >= max_bands read as
// 0 unless FULL): kernel_band_dequantize_simple (shannon_prime_cuda.cu:210-270)
// with the partial-read rule of shannon_prime_llama.h:240-255.
template <class LY, bool MOB, bool FULL, int N, int DWR>
__device__ __forceinline__ void dequant_bands(const uint32_t (&rec)[DWR], int max_bands, float (&x)[N]) {
    constexpr int HD = LY::hd;
    static_assert(DWR >= LY::dwords && N >= HD, "record and vector must hold the layout");
#pragma unroll
    for (int b = 0; b < LY::nb; b++) {
        const int off = LY::off(b), sz = LY::sz(b), bits = LY::bits[b];
        const int maxv = (1 << (bits - 1)) - 1, bo = LY::byte_off(b);
        const bool live = FULL || b < max_bands;  // FULL: every band is read
        const float scale = live ? sp_scale_from_bits(rec_extract(rec, 8 * bo, 16)) : 0.0f;
        const float bias = 12582912.0f + (float)maxv;
#pragma unroll
        for (int e = 0; e < sz; e++) {
            const uint32_t u = rec_extract(rec, 8 * (bo + 2) + e * bits, bits);
            const float d = __uint_as_float(u | 0x4B400000u) - bias;  // (float)(u - maxv), exact
            x[src_idx<HD, MOB>(off + e)] = live ? d * scale : 0.0f;
        }
    }
}

// A tile's records (64 contiguous records of B bytes) with coalesced 16-byte
// loads: load k of lane j reads bytes [16(64k+j), 16(64k+j)+16). The raw
// buffer covers the valid records only; a tile index past the last tile gives
// an empty range, so the prefetch is issued unconditionally and reads nothing.
// The range check drops every dword that does not end inside the range, so
// when the valid bytes end inside a dword (B not a multiple of 4) the last
// bytes come from exactly range-checked narrow loads, `tail` (one 2-byte load
// for even B, three 1-byte loads for odd B), which the caller writes into LDS
// after the chunks.
template <class LY>
struct RecTile {
    static constexpr int NCK = (64 * LY::total / 16 + 63) / 64;
    static constexpr int NT = LY::total % 4 == 0 ? 0 : (LY::total % 2 == 0 ? 1 : 3);
    u32x4 pre[NCK];
    uint32_t tail[NT > 0 ? NT : 1];
};

template <class LY>
__device__ __forceinline__ void rec_tile_load(RecTile<LY> &R, const unsigned char *src, long long so,
                                              const TileMap &M, int t, int n_tiles, int lane) {
    constexpr int B = LY::total, NT = RecTile<LY>::NT;
    int o, i0, nv;
    M.at(t, o, i0, nv);
    if (t >= n_tiles) o = 0, i0 = 0, nv = 0;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(src + (long long)o * so + (long long)i0 * B, nv * B);
#pragma unroll
    for (int k = 0; k < RecTile<LY>::NCK; k++)
        R.pre[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, k * 1024, 0);  // default policy: ~3% faster decodes
    if (NT == 1) R.tail[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, nv > 0 ? nv * B - 2 : 0, 0, BUF_NT);
    if (NT == 3) {
#pragma unroll
        for (int k = 0; k < 3; k++)
            R.tail[k] = __builtin_amdgcn_raw_buffer_load_b8(rs, nv > 0 ? nv * B - 3 + k : 0, 0, BUF_NT);
    }
}

// Stage tile t's records into LDS (chunks, then the tail bytes).
template <class LY>
__device__ __forceinline__ void rec_tile_stage(const RecTile<LY> &R, unsigned char *stage, const TileMap &M, int t,
                                               int lane) {
    constexpr int B = LY::total, NT = RecTile<LY>::NT;
#pragma unroll
    for (int k = 0; k < RecTile<LY>::NCK; k++) *reinterpret_cast<u32x4 *>(stage + k * 1024 + lane * 16) = R.pre[k];
    if (NT > 0) {
        int o, i0, nv;
        M.at(t, o, i0, nv);
        if (lane == 0) {
            if (NT == 1) *reinterpret_cast<unsigned short *>(stage + nv * B - 2) = (unsigned short)R.tail[0];
#pragma unroll
            for (int k = 0; k < (NT == 3 ? 3 : 0); k++) stage[nv * B - 3 + k] = (unsigned char)R.tail[k];
        }
    }
}

// The lane's own record out of the tile staged in LDS: dword reads at a stride
// of B bytes (B/4 odd for the 76-byte K records: no bank conflicts).
template <class LY>
__device__ __forceinline__ void rec_from_lds(uint32_t (&rec)[LY::dwords], const unsigned char *stage, int lane) {
    constexpr int B = LY::total, DW = LY::dwords;
    if (B % 4 == 0) {
        const uint32_t *p = reinterpret_cast<const uint32_t *>(stage + lane * B);
#pragma unroll
        for (int d = 0; d < DW; d++) rec[d] = p[d];
    } else {
        // unaligned records: read the covering dwords and funnel-shift by the byte offset
        const int a = lane * B;
        const uint32_t *p = reinterpret_cast<const uint32_t *>(stage + (a & ~3));
        const uint32_t sh = (a & 3) * 8;
        uint32_t w[DW + 1];
#pragma unroll
        for (int d = 0; d <= DW; d++) w[d] = p[d];
#pragma unroll
        for (int d = 0; d < DW; d++) rec[d] = __builtin_amdgcn_alignbit(w[d + 1], w[d], sh);
        if (B % 4 != 0) rec[DW - 1] &= (1u << (8 * (B % 4))) - 1u;
    }
}

// Tile t's input rows (64 rows of HD values, row i0 + j at (o*so + (i0+j)*si)
// elements from src) into LDS rows padded to RB + 16 bytes (tile_rows_stage),
// then lane j's row into in[] (tile_rows_in): wave-wide 16-byte buffer loads
// (rows past the tile's valid ones read as 0) and bank-conflict-free LDS row
// reads.
template <int DT, int HD>
__device__ __forceinline__ void tile_rows_stage(const void *src, long long so, long long si, const TileMap &M, int t,
                                                int lane, unsigned char *rows) {
    constexpr int RB = row_bytes<DT>(HD), RP = RB + 16, CPR = RB / 16, esz = DT == SP_DT_F16 ? 2 : 4;
    const int rowb = (int)(si * esz);  // launchers keep 64 rows of offsets in 32 bits
    int o, i0, nv;
    M.at(t, o, i0, nv);
    const unsigned char *g = reinterpret_cast<const unsigned char *>(src) + ((long long)o * so + (long long)i0 * si) * esz;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(g, (nv - 1) * rowb + RB);
    u32x4 v[CPR];
#pragma unroll
    for (int k = 0; k < CPR; k++) {
        const TileChunk<CPR> ch(k, lane);
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, ch.vofs(rowb), ch.sofs(rowb), BUF_NT);
    }
#pragma unroll
    for (int k = 0; k < CPR; k++) {
        const TileChunk<CPR> ch(k, lane);
        *reinterpret_cast<u32x4 *>(rows + ch.lds(RP)) = v[k];
    }
    __syncthreads();
}

// The same in two halves, so a tile's loads can be in flight while the previous
// tile computes: tile_rows_load issues the wave-wide loads into registers,
// tile_rows_put stores them to the LDS rows and hands lane j its row.
template <int DT, int HD>
__device__ __forceinline__ void tile_rows_load(const void *src, long long so, long long si, const TileMap &M, int t,
                                               int lane, u32x4 (&v)[row_bytes<DT>(HD) / 16]) {
    constexpr int RB = row_bytes<DT>(HD), CPR = RB / 16, esz = DT == SP_DT_F16 ? 2 : 4;
    const int rowb = (int)(si * esz);
    int o, i0, nv;
    M.at(t, o, i0, nv);
    const unsigned char *g = reinterpret_cast<const unsigned char *>(src) + ((long long)o * so + (long long)i0 * si) * esz;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(g, (nv - 1) * rowb + RB);
#pragma unroll
    for (int k = 0; k < CPR; k++) {
        const TileChunk<CPR> ch(k, lane);
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, ch.vofs(rowb), ch.sofs(rowb), BUF_NT);
    }
}
template <int DT, int HD>
__device__ __forceinline__ void tile_rows_put(const u32x4 (&v)[row_bytes<DT>(HD) / 16], int lane, unsigned char *rows,
                                              uint4 (&in)[row_bytes<DT>(HD) / 16]) {
    constexpr int RP = row_bytes<DT>(HD) + 16, CPR = row_bytes<DT>(HD) / 16;
    __syncthreads();  // the previous tile's reads of the rows are done
#pragma unroll
    for (int k = 0; k < CPR; k++) {
        const TileChunk<CPR> ch(k, lane);
        *reinterpret_cast<u32x4 *>(rows + ch.lds(RP)) = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CPR; c++) in[c] = *reinterpret_cast<const uint4 *>(rows + lane * RP + c * 16);
}

template <int DT, int HD>
__device__ __forceinline__ void tile_rows_in(const void *src, long long so, long long si, const TileMap &M, int t,
                                             int lane, unsigned char *rows, uint4 (&in)[row_bytes<DT>(HD) / 16]) {
    constexpr int RP = row_bytes<DT>(HD) + 16, CPR = row_bytes<DT>(HD) / 16;
    tile_rows_stage<DT, HD>(src, so, si, M, t, lane, rows);
#pragma unroll
    for (int c = 0; c < CPR; c++) in[c] = *reinterpret_cast<const uint4 *>(rows + lane * RP + c * 16);
}

// Tile t's records (lane j's record of B bytes in rec) out to dst: staged in
// LDS (stage holds LDSB bytes and may alias the input rows: the first barrier
// orders every lane's row reads before the stage writes), then wave-wide
// 16-byte stores over the whole 16-byte chunks and one 2-byte (odd B: 1-byte)
// store per lane over the rest. Each raw buffer's range drops the stores past
// its end, so the store count is the same for every tile.
template <int B, int LDSB, int DWR>
__device__ __forceinline__ void tile_records_out(const uint32_t (&rec)[DWR], unsigned char *stage, unsigned char *dst,
                                                 long long dout, const TileMap &M, int t, int lane) {
    constexpr int NCK = (64 * B / 16 + 63) / 64;
    static_assert(DWR * 4 >= B, "record registers must hold the record");
    static_assert(NCK * 1024 <= LDSB && 64 * B + 128 <= LDSB, "stage reads stay in the stage");
    int o, i0, nvalid;
    M.at(t, o, i0, nvalid);
    __syncthreads();
    if (lane < nvalid) {
        unsigned char *p = stage + lane * B;
        if (B % 4 == 0) {
#pragma unroll
            for (int d = 0; d < B / 4; d++) *reinterpret_cast<uint32_t *>(p + 4 * d) = rec[d];
        } else if (B % 2 == 0) {
#pragma unroll
            for (int hw = 0; hw < B / 2; hw++)
                *reinterpret_cast<unsigned short *>(p + 2 * hw) = (unsigned short)(rec[hw / 2] >> (16 * (hw % 2)));
        } else {
#pragma unroll
            for (int by = 0; by < B; by++) p[by] = (unsigned char)(rec[by / 4] >> (8 * (by % 4)));
        }
    }
    __syncthreads();
    unsigned char *gdst = dst + (long long)o * dout + (long long)i0 * B;
    const int nbytes = nvalid * B, nfull = nbytes & ~15;
    const __amdgpu_buffer_rsrc_t ws = buf_rsrc(gdst, nfull);
#pragma unroll
    for (int k = 0; k < NCK; k++) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + k * 1024 + lane * 16);
        __builtin_amdgcn_raw_buffer_store_b128(v, ws, lane * 16, k * 1024, BUF_NT);
    }
    const __amdgpu_buffer_rsrc_t wt = buf_rsrc(gdst + nfull, nbytes - nfull);
    if (B % 2 == 0) {
        const unsigned short h = *reinterpret_cast<const unsigned short *>(stage + nfull + 2 * lane);
        __builtin_amdgcn_raw_buffer_store_b16(h, wt, lane * 2, 0, BUF_NT);
    } else {
        __builtin_amdgcn_raw_buffer_store_b8(stage[nfull + lane], wt, lane, 0, BUF_NT);
    }
}

// Tile t's output rows (lane j's vector x[0, HD)) out to dst (row i0 + j at
// (o*dout + (i0+j)*din) elements): converted (fp16: one packed IEEE
// round-to-nearest-even conversion per pair) into LDS rows padded to RB + 16
// bytes, then wave-wide 16-byte buffer stores whose range check drops rows past
// the tile's valid ones. The first barrier orders the previous tile's stage
// reads before these writes.
template <int DT, int HD, int N>
__device__ __forceinline__ void rows_to_stage(const float (&x)[N], unsigned char *stage, int lane) {
    constexpr int RB = row_bytes<DT>(HD), RP = RB + 16;
    static_assert(N >= HD, "vector must hold the row");
    if (DT == SP_DT_F16) {
#pragma unroll
        for (int c = 0; c < HD / 8; c++) {
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float2v ab = {x[c * 8 + 2 * k], x[c * 8 + 2 * k + 1]};
                __asm__ volatile("" : "+v"(ab));  // no multiply-into-convert fusion
                w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(ab, half2v));
            }
            *reinterpret_cast<uint4 *>(stage + lane * RP + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else {
#pragma unroll
        for (int c = 0; c < HD / 4; c++)
            *reinterpret_cast<float4 *>(stage + lane * RP + c * 16) =
                make_float4(x[c * 4], x[c * 4 + 1], x[c * 4 + 2], x[c * 4 + 3]);
    }
}

// Listed positions: the lane's own record at byte address g, as the dwords that
// cover it, funnel-shifted to its byte offset (the cache must hold at least 4
// bytes past its last record).
template <class LY>
__device__ __forceinline__ void rec_load_direct(uint32_t (&rec)[LY::dwords], const unsigned char *g) {
    constexpr int B = LY::total, DW = LY::dwords;
    const uintptr_t a = (uintptr_t)g;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3) * 8;
    uint32_t w[DW + 1];
#pragma unroll
    for (int d = 0; d <= DW; d++) w[d] = p[d];
#pragma unroll
    for (int d = 0; d < DW; d++) rec[d] = __builtin_amdgcn_alignbit(w[d + 1], w[d], sh);
    if (B % 4 != 0) rec[DW - 1] &= (1u << (8 * (B % 4))) - 1u;
}

// Listed positions: lane j's row (x) to row `pos` of lane j (dst + (o*dout +
// pos*din) elements) for j < nvalid, through the padded LDS stage with RB/16
// lanes per row, so each row leaves as one contiguous run of 16-byte stores.
template <int DT, int HD, int N>
__device__ __forceinline__ void rows_out_listed(const float (&x)[N], unsigned char *stage, void *dst, long long dout,
                                                long long din, int o, int pos, int nvalid, int lane) {
    constexpr int RB = row_bytes<DT>(HD), RP = RB + 16, CPR = RB / 16;
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    __syncthreads();  // the previous tile's stage reads are done
    rows_to_stage<DT, HD>(x, stage, lane);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < CPR; q++) {
        const int idx = q * 64 + lane, r = idx / CPR, piece = idx - r * CPR;
        const int prow = __shfl(pos, r, 64);
        if (r < nvalid) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + r * RP + piece * 16);
            *reinterpret_cast<u32x4 *>(reinterpret_cast<unsigned char *>(dst) +
                                       ((long long)o * dout + (long long)prow * din) * esz + piece * 16) = v;
        }
    }
}

template <int DT, int HD, int N>
__device__ __forceinline__ void tile_rows_out(const float (&x)[N], unsigned char *stage, void *dst, long long dout,
                                              long long din, const TileMap &M, int t, int lane) {
    constexpr int RB = row_bytes<DT>(HD), RP = RB + 16, CPR = RB / 16, esz = DT == SP_DT_F16 ? 2 : 4;
    int o, i0, nvalid;
    M.at(t, o, i0, nvalid);
    __syncthreads();
    rows_to_stage<DT, HD>(x, stage, lane);
    __syncthreads();
    const int rowb = (int)(din * esz);  // launchers keep 64 rows of offsets in 32 bits
    unsigned char *gdst = reinterpret_cast<unsigned char *>(dst) + ((long long)o * dout + (long long)i0 * din) * esz;
    const __amdgpu_buffer_rsrc_t ws = buf_rsrc(gdst, (nvalid - 1) * rowb + RB);
#pragma unroll
    for (int k = 0; k < CPR; k++) {
        const TileChunk<CPR> ch(k, lane);
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + ch.lds(RP));
        __builtin_amdgcn_raw_buffer_store_b128(v, ws, ch.vofs(rowb), ch.sofs(rowb), BUF_NT);
    }
}

// Hier record [skeleton bands][mag f32 LE][NT residual levels, LSB-first]
// (shannon_prime_hier.cu:331-335), for skeleton band layout SL.
template <int NT, int RBITS, class SL>
struct HierRec {
    static constexpr int mag_byte = SL::total;
    static constexpr int res_bit = 8 * (SL::total + 4);
    static constexpr int total = SL::total + 4 + (NT * RBITS + 7) / 8;
    static constexpr int dwords = (total + 3) / 4;
};

// ---- host side ----
// Persistent grid size: enough single-wave blocks for several resident waves
// per SIMD on every CU (queried once per process).
int device_cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 256;
        if (hipGetDevice(&dev) == hipSuccess) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
                n = prop.multiProcessorCount;
        }
        cus = n;
    }
    return cus;
}
// SP_HIP_MAX_BLOCKS=n (read at each launch) caps the persistent and resident grids,
// so that tests reach the multi-tile loops (cross-tile prefetch, every block walking
// several tiles) with inputs small enough for the CPU oracle.
int grid_cap(int blocks) {
    if (const char *e = getenv("SP_HIP_MAX_BLOCKS")) {
        const int n = atoi(e);
        if (n > 0 && n < blocks) return n;
    }
    return blocks;
}
int persistent_blocks() { return grid_cap(device_cu_count() * 16); }
// Single-wave blocks that are resident at once for a kernel that fits `waves_per_simd`
// waves on a SIMD: a grid of that size keeps every block walking several tiles, so a
// tile's loads overlap the previous tile's compute.
int resident_blocks(int waves_per_simd) { return grid_cap(device_cu_count() * 4 * waves_per_simd); }

// Kernel constants from the host plan: cas[pi][m] is row 1 of the plan's p x p
// table (C[1][m] = cas(2*pi*m/p)), which holds every value C[k][j] takes.
XfConst xf_const(const SpPlan &P) {
    static const int primes[5] = {2, 3, 5, 7, 11};
    static const int offs[5] = {SP_CAS_OFF2, SP_CAS_OFF3, SP_CAS_OFF5, SP_CAS_OFF7, SP_CAS_OFF11};
    XfConst K{};
    K.inv_sqrt_n = P.inv_sqrt_n;
    for (int pi = 0; pi < 5; pi++) {
        K.isp[pi] = P.isp[pi];
        for (int m = 0; m < primes[pi]; m++) K.cas[pi][m] = P.cas[offs[pi] + primes[pi] + m];
    }
    return K;
}

// The register Vilenkin stages take C = 1 for k*j = 0 (mod p) and C = -1 for
// p = 2, k*j = 1 as exact; the host plan's values must be exactly those.
bool vil_consts_exact(const SpPlan &P) {
    static const int primes[5] = {2, 3, 5, 7, 11};
    static const int offs[5] = {SP_CAS_OFF2, SP_CAS_OFF3, SP_CAS_OFF5, SP_CAS_OFF7, SP_CAS_OFF11};
    for (int pi = 0; pi < 5; pi++) {
        const int p = primes[pi];
        for (int k = 0; k < p; k++)
            for (int j = 0; j < p; j++)
                if ((k * j) % p == 0 && P.cas[offs[pi] + k * p + j] != 1.0f) return false;
    }
    return P.cas[SP_CAS_OFF2 + 3] == -1.0f;
}

template <class LY>
bool layout_matches(const SpPlan &P) {
    if (P.hd != LY::hd || P.n_bands != LY::nb || P.total_bytes != LY::total) return false;
    if (P.skip_transform) return false;
    if (!c_pow2(LY::hd) && !vil_consts_exact(P)) return false;
    for (int b = 0; b < LY::nb; b++)
        if (P.band_bits[b] != LY::bits[b]) return false;
    return true;
}

}  // namespace
