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
__device__ __forceinline__ void enc_tile(const uint4 (&in)[row_bytes<DT>(LY::hd) / 16], float inv_sqrt_n,
                                         uint32_t (&rec)[LY::dwords]) {
    constexpr int HD = LY::hd, DW = LY::dwords;
    float x[HD];
    bool fastv;
    if (DT == SP_DT_F16) {
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
                   int n_tiles, float inv_sqrt_n) {
    constexpr int RB = row_bytes<DT>(LY::hd), RP = RB + 16, CPR = RB / 16, B = LY::total, DW = LY::dwords;
    // the record stage reuses the row buffer once the rows are in registers:
    // 17 KB per single-wave block lets two waves share each SIMD
    __shared__ __attribute__((aligned(16))) unsigned char rows[64 * RP];
    static_assert(64 * B + 16 <= 64 * RP, "record stage must fit in the row buffer");
    unsigned char *const stage = rows;
    const int lane = threadIdx.x;
    const TileMap M{tiles_per_outer, n_inner};
    constexpr int esz = DT == SP_DT_F16 ? 2 : 4, RPL = 64 / CPR;  // rows per wave-wide load
    static_assert(64 % CPR == 0, "a wave-wide 16-byte load must cover whole rows");
    const int rowb = (int)(si * esz);  // the launcher keeps 64 rows of offsets in 32 bits
    const int voff = (lane / CPR) * rowb + (lane % CPR) * 16;
    unsigned char *lrow = rows + (lane / CPR) * RP + (lane % CPR) * 16;
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
            for (int k = 0; k < CPR; k++) v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, k * RPL * rowb, BUF_NT);
#pragma unroll
            for (int k = 0; k < CPR; k++) *reinterpret_cast<u32x4 *>(lrow + k * RPL * RP) = v[k];
        }
        __syncthreads();
        uint4 in[CPR];
#pragma unroll
        for (int c = 0; c < CPR; c++) in[c] = *reinterpret_cast<const uint4 *>(rows + lane * RP + c * 16);
        uint32_t rec[DW];
        enc_tile<LY, DT, NORM, MOB>(in, inv_sqrt_n, rec);
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
                                         float inv_sqrt_n, int max_bands) {
    constexpr int HD = LY::hd, RB = row_bytes<DT>(HD), RP = RB + 16, CPR = RB / 16;
    constexpr int esz = DT == SP_DT_F16 ? 2 : 4, RPL = 64 / CPR;  // rows per wave-wide store
    static_assert(64 % CPR == 0, "a wave-wide 16-byte store must cover whole rows");
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
    vht2_reg<HD, NORM>(x, inv_sqrt_n, false);
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
    const int voff = (lane / CPR) * rowb + (lane % CPR) * 16;
    const unsigned char *lrow = stage + (lane / CPR) * RP + (lane % CPR) * 16;
#pragma unroll
    for (int k = 0; k < CPR; k++) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(lrow + k * RPL * RP);
        __builtin_amdgcn_raw_buffer_store_b128(v, ws, voff, k * RPL * rowb, BUF_NT);
    }
}

// A tile's records (64 contiguous records of B bytes) with coalesced 16-byte
// loads: load k of lane j reads bytes [16(64k+j), 16(64k+j)+16). The raw
// buffer covers the valid records only; a tile index past the last tile gives
// an empty range, so the prefetch is issued unconditionally and reads nothing.
template <class LY>
__device__ __forceinline__ void rec_tile_load(u32x4 (&pre)[(64 * LY::total / 16 + 63) / 64], const unsigned char *src,
                                              long long so, const TileMap &M, int t, int n_tiles, int lane) {
    constexpr int B = LY::total, NCK = (64 * B / 16 + 63) / 64;
    int o, i0, nv;
    M.at(t, o, i0, nv);
    if (t >= n_tiles) o = 0, i0 = 0, nv = 0;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(src + (long long)o * so + (long long)i0 * B, nv * B);
#pragma unroll
    for (int k = 0; k < NCK; k++) pre[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, k * 1024, BUF_NT);
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
                   float inv_sqrt_n, int max_bands) {
    constexpr int RP = row_bytes<DT>(LY::hd) + 16, DW = LY::dwords, B = LY::total;
    constexpr int NCK = (64 * B / 16 + 63) / 64;
    static_assert(NCK * 1024 + 16 <= 64 * RP, "record tile must fit in the row stage");
    __shared__ __attribute__((aligned(16))) unsigned char stage[64 * RP];
    const int lane = threadIdx.x, G = gridDim.x;
    const TileMap M{tiles_per_outer, n_inner};
    u32x4 pre[NCK];
    int t = blockIdx.x;
    if (t >= n_tiles) return;
    rec_tile_load<LY>(pre, src, so, M, t, n_tiles, lane);
    for (; t < n_tiles; t += G) {
#pragma unroll
        for (int k = 0; k < NCK; k++) *reinterpret_cast<u32x4 *>(stage + k * 1024 + lane * 16) = pre[k];
        __syncthreads();
        rec_tile_load<LY>(pre, src, so, M, t + G, n_tiles, lane);
        uint32_t rec[DW];
        rec_from_lds<LY>(rec, stage, lane);
        dec_tile<LY, DT, NORM, MOB, FULL>(rec, stage, dst, dout, din, M, t, lane, inv_sqrt_n, max_bands);
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

template <class LY>
bool layout_matches(const SpPlan &P) {
    if (P.hd != LY::hd || P.n_bands != LY::nb || P.total_bytes != LY::total) return false;
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
                       (int)n_tiles, P.inv_sqrt_n);
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
                           n_inner, tpo, (int)n_tiles, P.inv_sqrt_n, P.max_bands);
    else
        hipLaunchKernelGGL((k_ship_decode_lane<LY, DT, 0, MOB, false>), grid, block, 0, s, src, so, dst, dout, din,
                           n_inner, tpo, (int)n_tiles, P.inv_sqrt_n, P.max_bands);
    return hipGetLastError();
}

template <int DT>
hipError_t enc_dispatch(const SpPlan &P, bool mob, const void *src, long long so, long long si,
                        unsigned char *dst, long long dout, int n_outer, int n_inner, hipStream_t s) {
#define SP_TRY(LY, MOB) \
    if (layout_matches<LY>(P)) return enc_launch<LY, DT, MOB>(P, mob, src, so, si, dst, dout, n_outer, n_inner, s);
    SP_TRY(K128, true) SP_TRY(V128, false) SP_TRY(K64, true) SP_TRY(V64, false)
#undef SP_TRY
    return hipErrorNotSupported;
}

template <int DT>
hipError_t dec_dispatch(const SpPlan &P, bool mob, const unsigned char *src, long long so, void *dst,
                        long long dout, long long din, int n_outer, int n_inner, hipStream_t s) {
#define SP_TRY(LY, MOB) \
    if (layout_matches<LY>(P)) return dec_launch<LY, DT, MOB>(P, mob, src, so, dst, dout, din, n_outer, n_inner, s);
    SP_TRY(K128, true) SP_TRY(V128, false) SP_TRY(K64, true) SP_TRY(V64, false)
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
