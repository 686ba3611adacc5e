// sp_ship_lane.hip -- one-vector-per-lane ship codec kernels for the shipping
// band layouts (compile-time record geometry and Mobius order).
//
// Each lane owns a whole head_dim vector in registers, so all 7 butterfly
// stages are register adds (no lane exchanges), the Mobius permutation is a
// compile-time register renaming, and every code's bit position in the record
// is a constant. A 64-vector tile is staged through LDS in both directions so
// global loads and stores stay coalesced.
//
// Quantization fast path: for a band whose stored fp16 scale is a normal
// number and a vector whose inputs are finite, |x*inv| <= max_val*(1+2^-10)
// < max_val + 0.5 for max_val <= 127, so rint never needs the clamp, and
// rint(v) is exact in the low bits of fl(v + 1.5*2^23) (ties-to-even, since
// 1.5*2^23 is even and the ulp there is 1); adding max_val as an integer
// gives the code. Bands that fail the condition (subnormal/zero/inf scale,
// non-finite input) take the exact clamp path, so codes are bit-identical to
// kernel_band_quantize_simple (shannon_prime_cuda.cu:131-204) in every case.
#include <algorithm>
#include <type_traits>

#include "sp_internal.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

typedef float float2v __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr uint32_t BUF_WORD3 = 0x00020000u;  // raw buffer resource, dword data (gfx9 family)
constexpr int BUF_NT = 2;                    // non-temporal load policy

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

// Overwrite the w-bit field at bit position pos with val (val < 2^w).
template <int DW>
__device__ __forceinline__ void rec_replace(uint32_t (&rec)[DW], int pos, int w, uint32_t val) {
    const int d = pos / 32, sh = pos % 32;
    const uint32_t mask = (1u << w) - 1u;
    rec[d] = (rec[d] & ~(mask << sh)) | (val << sh);
    if (sh + w > 32) rec[d + 1] = (rec[d + 1] & ~(mask >> (32 - sh))) | (val >> (32 - sh));
}

// Insert the low w bits of v (higher bits are ignored) at bit position pos:
// one shift and one three-input bit operation (v << sh) & mask | rec.
template <int DW>
__device__ __forceinline__ void rec_insert_low(uint32_t (&rec)[DW], int pos, int w, uint32_t v) {
    const int d = pos / 32, sh = pos % 32;
    const uint32_t mask = (1u << w) - 1u;
    rec[d] = __builtin_amdgcn_bitop3_b32(v << sh, mask << sh, rec[d], 0xEA);
    if (sh + w > 32) rec[d + 1] = __builtin_amdgcn_bitop3_b32(v >> (32 - sh), mask >> (32 - sh), rec[d + 1], 0xEA);
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

}  // namespace

// ---------------------------------------------------------------------------
// Tiles of 64 vectors (one per lane) handled by single-wave blocks over a
// persistent grid. Each wave prefetches the next tile's inputs into registers
// before computing the current tile, so HBM latency overlaps with the
// arithmetic even at one wave per SIMD.
// ---------------------------------------------------------------------------
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

template <class LY, int DT, int NORM, bool MOB>
__device__ __forceinline__ void enc_tile(const uint4 (&in)[row_bytes<DT>(LY::hd) / 16], const XfConst &K,
                                         uint32_t (&rec)[LY::dwords]) {
    constexpr int HD = LY::hd, DW = LY::dwords;
    const float inv_sqrt_n = K.inv_sqrt_n;
    float x[HD];
    bool fastv;
    if constexpr (!c_pow2(HD)) {
        // Vilenkin lengths: the stage growth is at most sqrt(2p) per stage, so fp16
        // inputs stay finite and inf/NaN inputs reach the DC coefficient x[0]
        float mx = 0.0f;
        if (DT == SP_DT_F16) {
            static_assert(Factors<HD>{}.p[0] == 2, "the fused fp16 stage needs an even length");
#pragma unroll
            for (int c = 0; c < HD / 8; c++) {
                const uint32_t w[4] = {in[c].x, in[c].y, in[c].z, in[c].w};
#pragma unroll
                for (int k = 0; k < 4; k++) vil_first_f16_pair(w[k], K.isp[0], x[c * 8 + k * 2], x[c * 8 + k * 2 + 1]);
            }
            vil_stages<HD, 1, 2>(x, K);
        } else {
#pragma unroll
            for (int c = 0; c < HD / 4; c++) {
                x[c * 4 + 0] = __uint_as_float(in[c].x);
                x[c * 4 + 1] = __uint_as_float(in[c].y);
                x[c * 4 + 2] = __uint_as_float(in[c].z);
                x[c * 4 + 3] = __uint_as_float(in[c].w);
            }
#pragma unroll
            for (int i = 0; i < HD; i++) mx = fmaxf(mx, fabsf(x[i]));
            vil_stages<HD, 0, 1>(x, K);
        }
        fastv = (DT == SP_DT_F16 || mx < 1.2676506e30f) && __builtin_isfinite(x[0]);
    } else if (DT == SP_DT_F16) {
        // first butterfly stage fused with the exact f16 -> f32 widening
#pragma unroll
        for (int c = 0; c < HD / 8; c++) {
            const uint32_t w[4] = {in[c].x, in[c].y, in[c].z, in[c].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = c * 8 + k * 2;
                if (NORM == 1) {
                    const float a = sp_f16_bits_to_f32(w[k] & 0xffffu);
                    const float b = sp_f16_bits_to_f32(w[k] >> 16);
                    const float s2 = 0.70710678118654752440f;
                    x[i] = (a + b) * s2;
                    x[i + 1] = (a - b) * s2;
                } else {
                    bfly_f16_pair(w[k], x[i], x[i + 1]);
                }
            }
        }
        vht2_reg<HD, NORM>(x, inv_sqrt_n, true);
        // fp16 inputs cannot overflow the transform; an inf/NaN input makes
        // the DC coefficient non-finite
        fastv = __builtin_isfinite(x[0]);
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int c = 0; c < HD / 4; c++) {
            x[c * 4 + 0] = __uint_as_float(in[c].x);
            x[c * 4 + 1] = __uint_as_float(in[c].y);
            x[c * 4 + 2] = __uint_as_float(in[c].z);
            x[c * 4 + 3] = __uint_as_float(in[c].w);
        }
#pragma unroll
        for (int i = 0; i < HD; i++) mx = fmaxf(mx, fabsf(x[i]));
        vht2_reg<HD, NORM>(x, inv_sqrt_n, false);
        // |x| < 2^100 keeps every butterfly sum finite; NaN inputs reach x[0]
        fastv = (mx < 1.2676506e30f) && __builtin_isfinite(x[0]);
    }
#pragma unroll
    for (int d = 0; d < DW; d++) rec[d] = 0u;
#pragma unroll
    for (int b = 0; b < LY::nb; b++) {
        const int off = LY::off(b), sz = LY::sz(b), bits = LY::bits[b];
        const int maxv = (1 << (bits - 1)) - 1, bo = LY::byte_off(b);
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < sz; e++) amax = fmaxf(amax, fabsf(x[src_idx<HD, MOB>(off + e)]));
        const float scale = (amax > 0.0f) ? sp_div(amax, (float)maxv) : 0.0f;
        // Fast path for every lane: the hardware conversion is IEEE round-to-nearest-even
        // for finite scales, and for a normal fp16 scale |x*inv| < maxv + 1/2, so
        // t = x*inv + 1.5*2^23 rounds x*inv to the nearest integer q with ties to even (the
        // added constant is even) and bits(t) = 0x4B400000 + q: the low bits of
        // bits(t) + maxv are the code q + maxv. Lanes outside those conditions redo the
        // band below (a rare, divergent branch that only overwrites fields, so both
        // sides define every record word).
        float sc = scale;
        __asm__ volatile("" : "+v"(sc));  // keep the division and the conversion apart
        const uint32_t hf = (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)sc);
        {
            const float ss = sp_f16_bits_to_f32(hf);
            const float inv = (ss > 0.0f) ? sp_div(1.0f, ss) : 0.0f;
            rec_insert_low(rec, 8 * bo, 16, hf);
#pragma unroll
            for (int e = 0; e < sz; e++) {
                const float t = x[src_idx<HD, MOB>(off + e)] * inv + 12582912.0f;
                rec_insert_low(rec, 8 * (bo + 2) + e * bits, bits, __float_as_uint(t) + (uint32_t)maxv);
            }
        }
        if (!(fastv && f16_normal(hf))) {
            const uint32_t h = sp_f32_to_f16_bits(scale);
            const float ss = sp_f16_bits_to_f32(h);
            const float inv = (ss > 0.0f) ? sp_div(1.0f, ss) : 0.0f;
            rec_replace(rec, 8 * bo, 16, h);
#pragma unroll
            for (int e = 0; e < sz; e++) {
                const int q = sp_q_rint_clamp(x[src_idx<HD, MOB>(off + e)] * inv, maxv);
                rec_replace(rec, 8 * (bo + 2) + e * bits, bits, (uint32_t)(q + maxv));
            }
        }
    }
}

// Each single-wave block loads its tile with coalesced 16-byte loads and
// transposes it through LDS; with no prefetch registers held across the
// arithmetic, two waves fit per SIMD and one's loads overlap the other's work.
template <class LY, int DT, int NORM, bool MOB>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(DT == SP_DT_F16 ? 2 : 1)))
k_ship_encode_lane(const void *__restrict__ src, long long so, long long si,
                   unsigned char *__restrict__ dst, long long dout, int n_inner, int tiles_per_outer,
                   int n_tiles, const XfConst K) {
    constexpr int RB = row_bytes<DT>(LY::hd), RP = RB + 16, CPR = RB / 16, B = LY::total, DW = LY::dwords;
    // the record stage reuses the row buffer once the rows are in registers:
    // 17 KB per single-wave block lets two waves share each SIMD
    __shared__ __attribute__((aligned(16))) unsigned char rows[64 * RP];
    static_assert(64 * B + 16 <= 64 * RP, "record stage must fit in the row buffer");
    unsigned char *const stage = rows;
    const int lane = threadIdx.x;
    const TileMap M{tiles_per_outer, n_inner};
    constexpr int esz = DT == SP_DT_F16 ? 2 : 4;
    const int rowb = (int)(si * esz);  // the launcher keeps 64 rows of offsets in 32 bits
    for (int t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        {
            // load k of lane j reads chunk 64k+j of the tile: row (64k+j)/CPR, column
            // (64k+j)%CPR; rows past the tile's valid ones read as 0
            int o, i0, nv;
            M.at(t, o, i0, nv);
            const unsigned char *g =
                reinterpret_cast<const unsigned char *>(src) + ((long long)o * so + (long long)i0 * si) * esz;
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
        }
        __syncthreads();
        uint4 in[CPR];
#pragma unroll
        for (int c = 0; c < CPR; c++) in[c] = *reinterpret_cast<const uint4 *>(rows + lane * RP + c * 16);
        uint32_t rec[DW];
        enc_tile<LY, DT, NORM, MOB>(in, K, rec);
        int o, i0, nvalid;
        M.at(t, o, i0, nvalid);
        __syncthreads();  // every lane holds its row before the stage overwrites the buffer
        if (lane < nvalid) {
            unsigned char *p = stage + lane * B;
            if (B % 4 == 0) {
#pragma unroll
                for (int d = 0; d < B / 4; d++) *reinterpret_cast<uint32_t *>(p + 4 * d) = rec[d];
            } else {
                static_assert(B % 2 == 0, "record bytes must be even");
#pragma unroll
                for (int hw = 0; hw < B / 2; hw++)
                    *reinterpret_cast<unsigned short *>(p + 2 * hw) = (unsigned short)(rec[hw / 2] >> (16 * (hw % 2)));
            }
        }
        __syncthreads();
        // the tile's nvalid*B record bytes leave as wave-wide 16-byte stores over
        // the whole 16-byte chunks, then one 2-byte store per lane over the rest;
        // each raw buffer's range drops the stores past its end, so the store
        // count is the same for every tile
        unsigned char *gdst = dst + (long long)o * dout + (long long)i0 * B;
        const int nbytes = nvalid * B, nfull = nbytes & ~15;
        {
            constexpr int NCK = (64 * B / 16 + 63) / 64;
            static_assert(NCK * 1024 <= 64 * RP && 64 * B + 128 <= 64 * RP, "stage reads stay in the row buffer");
            const __amdgpu_buffer_rsrc_t ws = buf_rsrc(gdst, nfull);
#pragma unroll
            for (int k = 0; k < NCK; k++) {
                const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + k * 1024 + lane * 16);
                __builtin_amdgcn_raw_buffer_store_b128(v, ws, lane * 16, k * 1024, BUF_NT);
            }
            const __amdgpu_buffer_rsrc_t wt = buf_rsrc(gdst + nfull, nbytes - nfull);
            const unsigned short h = *reinterpret_cast<const unsigned short *>(stage + nfull + 2 * lane);
            __builtin_amdgcn_raw_buffer_store_b16(h, wt, lane * 2, 0, BUF_NT);
        }
    }
}

// ---------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------
// Decode one tile whose records are in registers and write its rows: through
// LDS, then as wave-wide 16-byte buffer stores whose range check drops rows
// past the tile's valid ones (no lane-dependent branch anywhere, so the
// compiler can count outstanding memory operations exactly).
template <class LY, int DT, int NORM, bool MOB, bool FULL>
__device__ __forceinline__ void dec_tile(const uint32_t (&rec)[LY::dwords], unsigned char *stage, void *dst,
                                         long long dout, long long din, const TileMap &M, int t, int lane,
                                         const XfConst &K, int max_bands) {
    constexpr int HD = LY::hd, RB = row_bytes<DT>(HD), RP = RB + 16, CPR = RB / 16;
    constexpr int esz = DT == SP_DT_F16 ? 2 : 4;
    float x[HD];
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
    if constexpr (c_pow2(HD)) vht2_reg<HD, NORM>(x, K.inv_sqrt_n, false);
    else vil_stages<HD, 0, 1>(x, K);
    int o, i0, nvalid;
    M.at(t, o, i0, nvalid);
    __syncthreads();  // previous tile's rows have been read out of LDS
    if (DT == SP_DT_F16) {
#pragma unroll
        for (int c = 0; c < HD / 8; c++) {
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float2v ab = {x[c * 8 + 2 * k], x[c * 8 + 2 * k + 1]};
                __asm__ volatile("" : "+v"(ab));  // no multiply-into-convert fusion
                // one packed IEEE round-to-nearest-even conversion per pair
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
    __syncthreads();
    // store k of lane j writes chunk 64k+j of the tile: row (64k+j)/CPR, column (64k+j)%CPR
    const int rowb = (int)(din * esz);  // the launcher keeps 64 rows of offsets in 32 bits
    unsigned char *gdst = reinterpret_cast<unsigned char *>(dst) + ((long long)o * dout + (long long)i0 * din) * esz;
    const __amdgpu_buffer_rsrc_t ws = buf_rsrc(gdst, (nvalid - 1) * rowb + RB);
#pragma unroll
    for (int k = 0; k < CPR; k++) {
        const TileChunk<CPR> ch(k, lane);
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + ch.lds(RP));
        __builtin_amdgcn_raw_buffer_store_b128(v, ws, ch.vofs(rowb), ch.sofs(rowb), BUF_NT);
    }
}

// A tile's records (64 contiguous records of B bytes) with coalesced 16-byte
// loads: load k of lane j reads bytes [16(64k+j), 16(64k+j)+16). The raw
// buffer covers the valid records only; a tile index past the last tile gives
// an empty range, so the prefetch is issued unconditionally and reads nothing.
// The range check drops every dword that does not end inside the range, so
// when the valid bytes end 2 bytes into a dword (B = 2 mod 4 and an odd count
// of records) those 2 bytes come from an exactly range-checked 2-byte load,
// `tail`, which the caller writes into LDS after the chunks.
template <class LY>
struct RecTile {
    static constexpr int NCK = (64 * LY::total / 16 + 63) / 64;
    u32x4 pre[NCK];
    uint32_t tail;
};

template <class LY>
__device__ __forceinline__ void rec_tile_load(RecTile<LY> &R, const unsigned char *src, long long so,
                                              const TileMap &M, int t, int n_tiles, int lane) {
    constexpr int B = LY::total;
    int o, i0, nv;
    M.at(t, o, i0, nv);
    if (t >= n_tiles) o = 0, i0 = 0, nv = 0;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(src + (long long)o * so + (long long)i0 * B, nv * B);
#pragma unroll
    for (int k = 0; k < RecTile<LY>::NCK; k++)
        R.pre[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, k * 1024, BUF_NT);
    if (B % 4 != 0) R.tail = __builtin_amdgcn_raw_buffer_load_b16(rs, nv > 0 ? nv * B - 2 : 0, 0, BUF_NT);
}

// Stage tile t's records into LDS (chunks, then the 2-byte tail).
template <class LY>
__device__ __forceinline__ void rec_tile_stage(const RecTile<LY> &R, unsigned char *stage, const TileMap &M, int t,
                                               int lane) {
    constexpr int B = LY::total;
#pragma unroll
    for (int k = 0; k < RecTile<LY>::NCK; k++) *reinterpret_cast<u32x4 *>(stage + k * 1024 + lane * 16) = R.pre[k];
    if (B % 4 != 0) {
        int o, i0, nv;
        M.at(t, o, i0, nv);
        if (lane == 0) *reinterpret_cast<unsigned short *>(stage + nv * B - 2) = (unsigned short)R.tail;
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
        // 2-byte aligned records: read the covering dwords and funnel-shift odd lanes by 16 bits
        const int a = lane * B;
        const uint32_t *p = reinterpret_cast<const uint32_t *>(stage + (a & ~3));
        const uint32_t sh = (a & 2) * 8;
        uint32_t w[DW + 1];
#pragma unroll
        for (int d = 0; d <= DW; d++) w[d] = p[d];
#pragma unroll
        for (int d = 0; d < DW; d++) rec[d] = __builtin_amdgcn_alignbit(w[d + 1], w[d], sh);
        if (B % 4 != 0) rec[DW - 1] &= 0xffffu;
    }
}

// Persistent single-wave blocks walk tiles t, t + G, t + 2G, ... (G = grid size).
// Each tile's records arrive as coalesced 16-byte loads, issued one tile ahead
// into registers, and are transposed through the LDS row stage (the records
// are in registers before the stage is overwritten with output rows).
template <class LY, int DT, int NORM, bool MOB, bool FULL>
__global__ void __launch_bounds__(64)
k_ship_decode_lane(const unsigned char *__restrict__ src, long long so, void *__restrict__ dst,
                   long long dout, long long din, int n_inner, int tiles_per_outer, int n_tiles,
                   const XfConst K, int max_bands) {
    constexpr int RP = row_bytes<DT>(LY::hd) + 16, DW = LY::dwords, B = LY::total;
    constexpr int NCK = (64 * B / 16 + 63) / 64;
    static_assert(NCK * 1024 + 16 <= 64 * RP, "record tile must fit in the row stage");
    __shared__ __attribute__((aligned(16))) unsigned char stage[64 * RP];
    const int lane = threadIdx.x, G = gridDim.x;
    const TileMap M{tiles_per_outer, n_inner};
    RecTile<LY> R;
    int t = blockIdx.x;
    if (t >= n_tiles) return;
    rec_tile_load<LY>(R, src, so, M, t, n_tiles, lane);
    for (; t < n_tiles; t += G) {
        rec_tile_stage<LY>(R, stage, M, t, lane);
        __syncthreads();
        rec_tile_load<LY>(R, src, so, M, t + G, n_tiles, lane);
        uint32_t rec[DW];
        rec_from_lds<LY>(rec, stage, lane);
        dec_tile<LY, DT, NORM, MOB, FULL>(rec, stage, dst, dout, din, M, t, lane, K, max_bands);
    }
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
namespace {

using K128 = Layout<128, 5, 5, 4, 3>;
using V128 = Layout<128, 3>;
using K64 = Layout<64, 5, 5, 4, 3>;
using V64 = Layout<64, 5>;
// Phi-3-mini-shaped hd 96 (Vilenkin 2^5 * 3) with the bridge's defaults, K 5/4/4 and V 5
// (shannon_prime_llama.c:240-248)
using K96 = Layout<96, 5, 4, 4>;
using V96 = Layout<96, 5>;

// Persistent grid size: enough single-wave blocks for several resident waves
// per SIMD on every CU (queried once per process).
int persistent_blocks() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, cus = 256;
        if (hipGetDevice(&dev) == hipSuccess) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
                cus = prop.multiProcessorCount;
        }
        n = cus * 16;
    }
    return n;
}

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

template <class LY, int DT, bool MOB>
hipError_t enc_launch(const SpPlan &P, bool mob, const void *src, long long so, long long si,
                      unsigned char *dst, long long dout, int n_outer, int n_inner, hipStream_t s) {
    if (mob != MOB || P.norm != 0) return hipErrorNotSupported;
    const int tpo = (n_inner + 63) / 64;
    const long long n_tiles = (long long)n_outer * tpo;
    if (n_tiles > 0x7fffffffLL) return hipErrorNotSupported;
    // a tile's 64 rows are addressed by 32-bit buffer offsets
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    if (si < 0 || 64 * si * esz + row_bytes<DT>(LY::hd) > 0x7fffffffLL) return hipErrorNotSupported;
    const dim3 grid((unsigned)std::min<long long>(n_tiles, persistent_blocks())), block(64);
    hipLaunchKernelGGL((k_ship_encode_lane<LY, DT, 0, MOB>), grid, block, 0, s, src, so, si, dst, dout, n_inner, tpo,
                       (int)n_tiles, xf_const(P));
    return hipGetLastError();
}

template <class LY, int DT, bool MOB>
hipError_t dec_launch(const SpPlan &P, bool mob, const unsigned char *src, long long so, void *dst,
                      long long dout, long long din, int n_outer, int n_inner, hipStream_t s) {
    if (mob != MOB || P.norm != 0) return hipErrorNotSupported;
    const int tpo = (n_inner + 63) / 64;
    const long long n_tiles = (long long)n_outer * tpo;
    if (n_tiles > 0x7fffffffLL) return hipErrorNotSupported;
    // a tile's 64 output rows are addressed by 32-bit buffer offsets, rows never overlap
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    if (din < LY::hd || 64 * din * esz + row_bytes<DT>(LY::hd) > 0x7fffffffLL) return hipErrorNotSupported;
    const dim3 grid((unsigned)std::min<long long>(n_tiles, persistent_blocks())), block(64);
    if (P.max_bands < 0 || P.max_bands >= LY::nb)
        hipLaunchKernelGGL((k_ship_decode_lane<LY, DT, 0, MOB, true>), grid, block, 0, s, src, so, dst, dout, din,
                           n_inner, tpo, (int)n_tiles, xf_const(P), P.max_bands);
    else
        hipLaunchKernelGGL((k_ship_decode_lane<LY, DT, 0, MOB, false>), grid, block, 0, s, src, so, dst, dout, din,
                           n_inner, tpo, (int)n_tiles, xf_const(P), P.max_bands);
    return hipGetLastError();
}

template <int DT>
hipError_t enc_dispatch(const SpPlan &P, bool mob, const void *src, long long so, long long si,
                        unsigned char *dst, long long dout, int n_outer, int n_inner, hipStream_t s) {
#define SP_TRY(LY, MOB) \
    if (layout_matches<LY>(P)) return enc_launch<LY, DT, MOB>(P, mob, src, so, si, dst, dout, n_outer, n_inner, s);
    SP_TRY(K128, true) SP_TRY(V128, false) SP_TRY(K64, true) SP_TRY(V64, false) SP_TRY(K96, true) SP_TRY(V96, false)
#undef SP_TRY
    return hipErrorNotSupported;
}

template <int DT>
hipError_t dec_dispatch(const SpPlan &P, bool mob, const unsigned char *src, long long so, void *dst,
                        long long dout, long long din, int n_outer, int n_inner, hipStream_t s) {
#define SP_TRY(LY, MOB) \
    if (layout_matches<LY>(P)) return dec_launch<LY, DT, MOB>(P, mob, src, so, dst, dout, din, n_outer, n_inner, s);
    SP_TRY(K128, true) SP_TRY(V128, false) SP_TRY(K64, true) SP_TRY(V64, false) SP_TRY(K96, true) SP_TRY(V96, false)
#undef SP_TRY
    return hipErrorNotSupported;
}

}  // namespace

// Returns hipErrorNotSupported (nothing launched) when no specialization fits:
// the caller then uses the general kernels.
hipError_t sp_launch_ship_encode_lane(const SpPlan &P, bool default_order, const void *src, int dtype,
                                      long long so, long long si, unsigned char *dst, long long dout,
                                      int n_outer, int n_inner, hipStream_t s) {
    const int esz = dtype == SP_DT_F16 ? 2 : 4;
    if (((uintptr_t)src % 16) || ((so * esz) % 16) || ((si * esz) % 16)) return hipErrorNotSupported;
    if (((uintptr_t)dst % 4) || (dout % 4)) return hipErrorNotSupported;
    if (dtype == SP_DT_F16) return enc_dispatch<SP_DT_F16>(P, default_order, src, so, si, dst, dout, n_outer, n_inner, s);
    return enc_dispatch<SP_DT_F32>(P, default_order, src, so, si, dst, dout, n_outer, n_inner, s);
}

hipError_t sp_launch_ship_decode_lane(const SpPlan &P, bool default_order, const unsigned char *src,
                                      long long so, void *dst, int dtype, long long dout, long long din,
                                      int n_outer, int n_inner, hipStream_t s) {
    const int esz = dtype == SP_DT_F16 ? 2 : 4;
    if (((uintptr_t)dst % 16) || ((dout * esz) % 16) || ((din * esz) % 16)) return hipErrorNotSupported;
    if (((uintptr_t)src % 4) || (so % 4)) return hipErrorNotSupported;
    if (dtype == SP_DT_F16) return dec_dispatch<SP_DT_F16>(P, default_order, src, so, dst, dout, din, n_outer, n_inner, s);
    return dec_dispatch<SP_DT_F32>(P, default_order, src, so, dst, dout, din, n_outer, n_inner, s);
}
