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

#include "sp_lane.h"


// ---------------------------------------------------------------------------
// Tiles of 64 vectors (one per lane) handled by single-wave blocks over a
// persistent grid. Each wave prefetches the next tile's inputs into registers
// before computing the current tile, so HBM latency overlaps with the
// arithmetic even at one wave per SIMD.
// ---------------------------------------------------------------------------
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
    quant_bands<LY, MOB>(x, fastv, rec);
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
    for (int t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        uint4 in[CPR];
        tile_rows_in<DT, LY::hd>(src, so, si, M, t, lane, rows, in);
        uint32_t rec[DW];
        enc_tile<LY, DT, NORM, MOB>(in, K, rec);
        tile_records_out<B, 64 * RP>(rec, stage, dst, dout, M, t, lane);
    }
}

// ---------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------
// Decode one tile whose records are in registers and write its rows: through
// LDS, then as wave-wide 16-byte buffer stores whose range check drops rows
// past the tile's valid ones (no lane-dependent branch anywhere, so the
// compiler can count outstanding memory operations exactly).
// A record in registers -> the lane's reconstructed vector (dequantize, then the
// inverse transform, which is the same orthonormal self-inverse transform).
template <class LY, int NORM, bool MOB, bool FULL>
__device__ __forceinline__ void dec_vec(const uint32_t (&rec)[LY::dwords], const XfConst &K, int max_bands,
                                        float (&x)[LY::hd]) {
    constexpr int HD = LY::hd;
    dequant_bands<LY, MOB, FULL>(rec, max_bands, x);
    if constexpr (c_pow2(HD)) vht2_reg<HD, NORM>(x, K.inv_sqrt_n, false);
    else vil_stages<HD, 0, 1>(x, K);
}

template <class LY, int DT, int NORM, bool MOB, bool FULL>
__device__ __forceinline__ void dec_tile(const uint32_t (&rec)[LY::dwords], unsigned char *stage, void *dst,
                                         long long dout, long long din, const TileMap &M, int t, int lane,
                                         const XfConst &K, int max_bands) {
    float x[LY::hd];
    dec_vec<LY, NORM, MOB, FULL>(rec, K, max_bands, x);
    tile_rows_out<DT, LY::hd>(x, stage, dst, dout, din, M, t, lane);
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
// in-place round trip over cache cells
// ---------------------------------------------------------------------------
// The device form of llama_sp_post_compute's per-layer loop
// (llama-cpp-b8861-full-engine.patch:997-1360): lane j of tile (h, g) takes cell
// c = cells[64g + j] of head h, whose element d sits at c*cs + (h*HD + d)*es in
// the llama.cpp cache tensor x (es = 1: rows; cs = 1, es = kv_size: the
// transposed V layout). It compresses the vector into the record at position c
// of head h, then decompresses that record (bands < max_bands unless FULL) and
// writes the reconstruction back over the vector. Cells outside [0, max_seq)
// and lanes past n_cells load cell cells[0]'s data and store nothing. CONTIG
// (es = 1 and 16-byte aligned rows) moves whole rows as 16-byte pieces;
// otherwise element by element (coalesced across lanes when the cells are
// consecutive and cs = 1).
template <class LY, int DT, bool MOB, bool FULL, bool CONTIG>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_ship_roundtrip_lane(void *__restrict__ x, long long cs, long long es, const int *__restrict__ cells, int n_cells,
                      int max_seq, unsigned char *__restrict__ rec_base, long long rec_head_stride, int n_tiles,
                      const XfConst K, int max_bands) {
    constexpr int HD = LY::hd, CPR = row_bytes<DT>(HD) / 16, B = LY::total, DW = LY::dwords;
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    const int lane = threadIdx.x, tpg = (n_cells + 63) / 64;
    for (int t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        const int h = t / tpg, i = (t - h * tpg) * 64 + lane;
        const int c0 = cells[i < n_cells ? i : 0];
        const bool live = i < n_cells && c0 >= 0 && c0 < max_seq;
        const long long c = live ? c0 : (long long)((cells[0] >= 0 && cells[0] < max_seq) ? cells[0] : 0);
        unsigned char *v = reinterpret_cast<unsigned char *>(x) + (c * cs + (long long)h * HD * es) * esz;
        uint4 in[CPR];
        if (CONTIG) {
#pragma unroll
            for (int q = 0; q < CPR; q++) in[q] = *reinterpret_cast<const uint4 *>(v + 16 * q);
        } else {
            uint32_t w[CPR * 4];
#pragma unroll
            for (int k = 0; k < CPR * 4; k++) {
                if (DT == SP_DT_F16)
                    w[k] = (uint32_t)*reinterpret_cast<const unsigned short *>(v + (2 * k) * es * 2) |
                           ((uint32_t)*reinterpret_cast<const unsigned short *>(v + (2 * k + 1) * es * 2) << 16);
                else
                    w[k] = *reinterpret_cast<const uint32_t *>(v + k * es * 4);
            }
#pragma unroll
            for (int q = 0; q < CPR; q++) in[q] = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
        }
        uint32_t rec[DW];
        enc_tile<LY, DT, 0, MOB>(in, K, rec);
        float y[HD];
        dec_vec<LY, 0, MOB, FULL>(rec, K, max_bands, y);
        if (live) {
            unsigned char *r = rec_base + (long long)h * rec_head_stride + c * B;
            if (B % 4 == 0) {
#pragma unroll
                for (int d = 0; d < B / 4; d++) reinterpret_cast<uint32_t *>(r)[d] = rec[d];
            } else {
#pragma unroll
                for (int hw = 0; hw < B / 2; hw++)
                    reinterpret_cast<unsigned short *>(r)[hw] = (unsigned short)(rec[hw / 2] >> (16 * (hw % 2)));
            }
            uint32_t o[CPR * 4];
#pragma unroll
            for (int k = 0; k < CPR * 4; k++) {
                if (DT == SP_DT_F16) {
                    float2v ab = {y[2 * k], y[2 * k + 1]};
                    __asm__ volatile("" : "+v"(ab));  // no multiply-into-convert fusion
                    o[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(ab, half2v));
                } else {
                    o[k] = __float_as_uint(y[k]);
                }
            }
            if (CONTIG) {
#pragma unroll
                for (int q = 0; q < CPR; q++)
                    *reinterpret_cast<uint4 *>(v + 16 * q) = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
            } else {
#pragma unroll
                for (int k = 0; k < CPR * 4; k++) {
                    if (DT == SP_DT_F16) {
                        *reinterpret_cast<unsigned short *>(v + (2 * k) * es * 2) = (unsigned short)o[k];
                        *reinterpret_cast<unsigned short *>(v + (2 * k + 1) * es * 2) = (unsigned short)(o[k] >> 16);
                    } else {
                        *reinterpret_cast<uint32_t *>(v + k * es * 4) = o[k];
                    }
                }
            }
        }
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
// Gemma-shaped hd 256, K 5/5/4/3 and V 3: decode both, encode V (K's encode with the
// Mobius gather needs more than the 512 registers of a lane and stays on the
// 8-coefficients-per-lane kernel)
using K256 = Layout<256, 5, 5, 4, 3>;
using V256 = Layout<256, 3>;


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

template <class LY, int DT, bool MOB>
hipError_t rt_launch(const SpPlan &P, bool mob, void *x, long long cs, long long es, const int *cells, int n_cells,
                     int max_seq, unsigned char *rec_base, long long rec_head_stride, int n_heads, int max_bands,
                     hipStream_t s) {
    if (mob != MOB || P.norm != 0) return hipErrorNotSupported;
    const long long n_tiles = (long long)n_heads * ((n_cells + 63) / 64);
    if (n_tiles > 0x7fffffffLL) return hipErrorNotSupported;
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    const bool contig = es == 1 && ((uintptr_t)x % 16) == 0 && (cs * esz) % 16 == 0 && (LY::hd * esz) % 16 == 0;
    const bool full = max_bands < 0 || max_bands >= LY::nb;
    const dim3 grid((unsigned)std::min<long long>(n_tiles, persistent_blocks())), block(64);
#define SP_RT(FULLV, CONTIGV)                                                                                      \
    hipLaunchKernelGGL((k_ship_roundtrip_lane<LY, DT, MOB, FULLV, CONTIGV>), grid, block, 0, s, x, cs, es, cells, \
                       n_cells, max_seq, rec_base, rec_head_stride, (int)n_tiles, xf_const(P), max_bands)
    if (full) {
        if (contig) SP_RT(true, true);
        else SP_RT(true, false);
    } else {
        if (contig) SP_RT(false, true);
        else SP_RT(false, false);
    }
#undef SP_RT
    return hipGetLastError();
}

template <int DT>
hipError_t rt_dispatch(const SpPlan &P, bool mob, void *x, long long cs, long long es, const int *cells, int n_cells,
                       int max_seq, unsigned char *rec_base, long long rec_head_stride, int n_heads, int max_bands,
                       hipStream_t s) {
#define SP_TRY(LY, MOB)                                                                                          \
    if (layout_matches<LY>(P))                                                                                   \
        return rt_launch<LY, DT, MOB>(P, mob, x, cs, es, cells, n_cells, max_seq, rec_base, rec_head_stride, n_heads, \
                                      max_bands, s);
    SP_TRY(K128, true) SP_TRY(V128, false) SP_TRY(K64, true) SP_TRY(V64, false) SP_TRY(K96, true) SP_TRY(V96, false)
#undef SP_TRY
    return hipErrorNotSupported;
}

template <int DT>
hipError_t enc_dispatch(const SpPlan &P, bool mob, const void *src, long long so, long long si,
                        unsigned char *dst, long long dout, int n_outer, int n_inner, hipStream_t s) {
#define SP_TRY(LY, MOB) \
    if (layout_matches<LY>(P)) return enc_launch<LY, DT, MOB>(P, mob, src, so, si, dst, dout, n_outer, n_inner, s);
    SP_TRY(K128, true) SP_TRY(V128, false) SP_TRY(K64, true) SP_TRY(V64, false) SP_TRY(K96, true) SP_TRY(V96, false) SP_TRY(V256, false)
#undef SP_TRY
    return hipErrorNotSupported;
}

template <int DT>
hipError_t dec_dispatch(const SpPlan &P, bool mob, const unsigned char *src, long long so, void *dst,
                        long long dout, long long din, int n_outer, int n_inner, hipStream_t s) {
#define SP_TRY(LY, MOB) \
    if (layout_matches<LY>(P)) return dec_launch<LY, DT, MOB>(P, mob, src, so, dst, dout, din, n_outer, n_inner, s);
    SP_TRY(K128, true) SP_TRY(V128, false) SP_TRY(K64, true) SP_TRY(V64, false) SP_TRY(K96, true) SP_TRY(V96, false) SP_TRY(K256, true) SP_TRY(V256, false)
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

// In-place round trip of every head's vectors at n_cells cache cells (see
// k_ship_roundtrip_lane). hipErrorNotSupported when the layout has no lane
// specialization.
hipError_t sp_launch_ship_roundtrip_lane(const SpPlan &P, bool default_order, void *x, int dtype, long long cs,
                                         long long es, const int *cells, int n_cells, int max_seq,
                                         unsigned char *rec_base, long long rec_head_stride, int n_heads,
                                         int max_bands, hipStream_t s) {
    if (n_cells <= 0 || n_heads <= 0) return hipSuccess;
    if (((uintptr_t)rec_base % 4) || (rec_head_stride % 4)) return hipErrorNotSupported;
    if (dtype == SP_DT_F16)
        return rt_dispatch<SP_DT_F16>(P, default_order, x, cs, es, cells, n_cells, max_seq, rec_base, rec_head_stride,
                                      n_heads, max_bands, s);
    return rt_dispatch<SP_DT_F32>(P, default_order, x, cs, es, cells, n_cells, max_seq, rec_base, rec_head_stride,
                                  n_heads, max_bands, s);
}
