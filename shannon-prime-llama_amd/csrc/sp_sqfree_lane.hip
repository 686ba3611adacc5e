// sp_sqfree_lane.hip -- one-vector-per-lane sqfree+spinor codec kernels for the
// shipping geometry: head_dim 128 padded to 154 = 2*7*11, skeleton bands
// 5/4/4/4/5 over the first SK squarefree-first coefficients (SK = 77, the
// reference CUDA default, or 115 = 0.75 of the pad), 3-bit residuals, spinor
// sheet on; at SK = 115 also one 3-bit skeleton band (configs[3]'s V).
//
// Each lane owns one vector: the pad, the staged Vilenkin transform, the
// skeleton gather, the CSR Mobius prediction, the spinor choice and every
// record field are register operations with compile-time positions (the Knight
// mask is a compile-time table here). 64-vector tiles move through LDS with
// coalesced loads and stores, as in the ship lane kernels. The arithmetic and
// its order are those of k_sqfree_encode / k_sqfree_decode (and of
// sp_cuda_sqfree_write_one / read_one, shannon_prime_sqfree.cu:750-950), so
// records and reconstructions are bit-identical to them.
#include "sp_sqfree_lane.h"

namespace {

template <int DT, int HD, int PAD, int SK, int RBITS, bool SPIN, class SL>
__global__ void __launch_bounds__(64)
k_sqfree_encode_lane(const void *__restrict__ src, long long so, long long si, unsigned char *__restrict__ dst,
                     long long dout, int n_inner, int tiles_per_outer, int n_tiles, const XfConst K) {
    using G = SqRec<PAD, SK, RBITS, SPIN, SL>;
    constexpr int RB = row_bytes<DT>(HD), RP = RB + 16, CPR = RB / 16, NR = PAD - SK, DWR = G::dwords;
    constexpr auto &KN = kKnight<PAD, SK>;
    static_assert(SL::hd == SK, "skeleton layout must cover the skeleton");
    __shared__ __attribute__((aligned(16))) unsigned char rows[64 * RP];  // input rows, then the record stage
    const int lane = threadIdx.x;
    const TileMap M{tiles_per_outer, n_inner};
    // the next tile's rows are in flight while this one computes
    u32x4 pre[CPR];
    if (blockIdx.x < n_tiles) tile_rows_load<DT, HD>(src, so, si, M, blockIdx.x, lane, pre);
    for (int t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        uint4 in[CPR];
        tile_rows_put<DT, HD>(pre, lane, rows, in);
        if (t + (int)gridDim.x < n_tiles) tile_rows_load<DT, HD>(src, so, si, M, t + gridDim.x, lane, pre);
        float c[PAD];
        float mx = 0.0f;
#pragma unroll
        for (int q = 0; q < CPR; q++) {
            const uint32_t w[4] = {in[q].x, in[q].y, in[q].z, in[q].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (DT == SP_DT_F16) {
                    c[q * 8 + 2 * k] = sp_f16_bits_to_f32(w[k] & 0xffffu);
                    c[q * 8 + 2 * k + 1] = sp_f16_bits_to_f32(w[k] >> 16);
                } else {
                    c[q * 4 + k] = __uint_as_float(w[k]);
                }
            }
        }
        if (DT != SP_DT_F16) {
#pragma unroll
            for (int i = 0; i < HD; i++) mx = fmaxf(mx, fabsf(c[i]));
        }
        // pad with the true mean (kernel_sqfree_pad, summed in the reference's
        // block-reduction order, divided by (float)hd)
        const float mean = sp_div(tree256_sum<HD, false>(c), (float)HD);
#pragma unroll
        for (int i = HD; i < PAD; i++) c[i] = mean;
        vil_stages<PAD, 0, 1>(c, K);
        // growth is at most sqrt(2p) per stage: fp16 inputs stay finite, fp32
        // inputs below 2^100 too; inf/NaN inputs reach the DC coefficient
        const bool fastv = (DT == SP_DT_F16 || mx < 1.2676506e30f) && __builtin_isfinite(c[0]);
        float sk[SK];
#pragma unroll
        for (int s = 0; s < SK; s++) sk[s] = c[KN.skel[s]];
        uint32_t rec[DWR];
#pragma unroll
        for (int d = 0; d < DWR; d++) rec[d] = 0u;
        quant_bands<SL, false>(sk, fastv, rec);
        if constexpr (NR > 0) {
            // deviation from the prediction of the unquantized skeleton; spinor
            // takes the sign with the smaller |deviation| (strict <, :231)
            float dv[NR];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const float p = csr_predict<PAD, SK>(sk, r), a = c[KN.res[r]];
                if (SPIN) {
                    const float vp = a - p, vm = a + p;
                    const bool um = fabsf(vm) < fabsf(vp);
                    dv[r] = um ? vm : vp;
                    rec_insert(rec, G::sheet_bit + r, 1, um ? 1u : 0u);
                } else {
                    dv[r] = a - p;
                }
            }
            float mag = sp_div(tree256_sum<NR, true>(dv), (float)NR);
            mag = mag < 1e-12f ? 1e-12f : mag;
            rec_put32(rec, G::mag_byte, __float_as_uint(mag));
            // residual levels (kernel_quantize_residual, shannon_prime_sqfree.cu:514-532)
            constexpr int L = 1 << RBITS;
            const float center = 0.5f * (float)(L - 1);
            const float sat = (mag > 1e-12f) ? (mag * (float)RBITS) : 1e-12f;
            const float step = sp_div(2.0f * sat, (float)(L - 1));
            const float inv_step = sp_div(1.0f, step);
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const float qf = dv[r] * inv_step + center;
                int level = sp_trunc_sat(qf + 0.5f);
                level = level < 0 ? 0 : (level >= L ? L - 1 : level);
                rec_insert(rec, G::res_bit + r * RBITS, RBITS, (uint32_t)level);
            }
        }
        tile_records_out<G::total, 64 * RP>(rec, rows, dst, dout, M, t, lane);
    }
}

template <int DT, int HD, int PAD, int SK, int RBITS, bool SPIN, class SL>
__global__ void __launch_bounds__(64)
k_sqfree_decode_lane(const unsigned char *__restrict__ src, long long so, void *__restrict__ dst, long long dout,
                     long long din, int n_inner, int tiles_per_outer, int n_tiles, const XfConst K) {
    using G = SqRec<PAD, SK, RBITS, SPIN, SL>;
    constexpr int RP = row_bytes<DT>(HD) + 16, NR = PAD - SK, DWR = G::dwords;
    constexpr auto &KN = kKnight<PAD, SK>;
    static_assert(RecTile<G>::NCK * 1024 + 16 <= 64 * RP, "record tile must fit in the row stage");
    __shared__ __attribute__((aligned(16))) unsigned char stage[64 * RP];
    const int lane = threadIdx.x, Gs = gridDim.x;
    const TileMap M{tiles_per_outer, n_inner};
    RecTile<G> R;
    int t = blockIdx.x;
    if (t >= n_tiles) return;
    rec_tile_load<G>(R, src, so, M, t, n_tiles, lane);
    for (; t < n_tiles; t += Gs) {
        rec_tile_stage<G>(R, stage, M, t, lane);
        __syncthreads();
        rec_tile_load<G>(R, src, so, M, t + Gs, n_tiles, lane);
        uint32_t rec[DWR];
        rec_from_lds<G>(rec, stage, lane);
        float sk[SK];
        dequant_bands<SL, false, true>(rec, SL::nb, sk);
        float c[PAD];
#pragma unroll
        for (int s = 0; s < SK; s++) c[KN.skel[s]] = sk[s];
        if constexpr (NR > 0) {
            // prediction from the dequantized skeleton, spinor sign, residual
            // (lvl - center) * step with step = 2*mag*bits/(L-1) (:535-548, :249-283)
            const float mag = __uint_as_float(rec_get32(rec, G::mag_byte));
            constexpr int L = 1 << RBITS;
            const float center = 0.5f * (float)(L - 1);
            const float sat = mag * (float)RBITS;
            const float step = (L > 1) ? sp_div(2.0f * sat, (float)(L - 1)) : 0.0f;
#pragma unroll
            for (int r = 0; r < NR; r++) {
                float p = csr_predict<PAD, SK>(sk, r);
                if (SPIN && rec_extract(rec, G::sheet_bit + r, 1)) p = -p;
                const float d = ((float)rec_extract(rec, G::res_bit + r * RBITS, RBITS) - center) * step;
                c[KN.res[r]] = p + d;
            }
        }
        vil_stages<PAD, 0, 1>(c, K);
        tile_rows_out<DT, HD>(c, stage, dst, dout, din, M, t, lane);
    }
}

// Listed positions (the dual cache's System 2 rows): lane j of tile t decodes the
// record at position cells[i0 + j] of outer row o into row cells[i0 + j] of dst.
// Each lane reads its own record as the covering dwords, funnel-shifted to the
// record's byte offset (the cache keeps slack bytes past its last record); the
// rows leave through the padded LDS stage, CPR lanes per row, so every row is
// written as whole 16-byte pieces in one contiguous run.
template <int DT, int HD, int PAD, int SK, int RBITS, bool SPIN, class SL>
__global__ void __launch_bounds__(64)
k_sqfree_decode_lane_cells(const unsigned char *__restrict__ src, long long so, void *__restrict__ dst,
                           long long dout, long long din, const int *__restrict__ cells, int n_inner,
                           int tiles_per_outer, int n_tiles, const XfConst K) {
    using G = SqRec<PAD, SK, RBITS, SPIN, SL>;
    constexpr int RP = row_bytes<DT>(HD) + 16, NR = PAD - SK, DWR = G::dwords, B = G::total;
    constexpr auto &KN = kKnight<PAD, SK>;
    __shared__ __attribute__((aligned(16))) unsigned char stage[64 * RP];
    const int lane = threadIdx.x;
    const TileMap M{tiles_per_outer, n_inner};
    for (int t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        int o, i0, nvalid;
        M.at(t, o, i0, nvalid);
        const int pos = cells[lane < nvalid ? i0 + lane : i0];
        uint32_t rec[DWR];
        rec_load_direct<G>(rec, src + (long long)o * so + (long long)pos * B);
        float sk[SK];
        dequant_bands<SL, false, true>(rec, SL::nb, sk);
        float c[PAD];
#pragma unroll
        for (int s = 0; s < SK; s++) c[KN.skel[s]] = sk[s];
        if constexpr (NR > 0) {
            const float mag = __uint_as_float(rec_get32(rec, G::mag_byte));
            constexpr int L = 1 << RBITS;
            const float center = 0.5f * (float)(L - 1);
            const float sat = mag * (float)RBITS;
            const float step = (L > 1) ? sp_div(2.0f * sat, (float)(L - 1)) : 0.0f;
#pragma unroll
            for (int r = 0; r < NR; r++) {
                float pr = csr_predict<PAD, SK>(sk, r);
                if (SPIN && rec_extract(rec, G::sheet_bit + r, 1)) pr = -pr;
                const float d = ((float)rec_extract(rec, G::res_bit + r * RBITS, RBITS) - center) * step;
                c[KN.res[r]] = pr + d;
            }
        }
        vil_stages<PAD, 0, 1>(c, K);
        rows_out_listed<DT, HD>(c, stage, dst, dout, din, o, pos, nvalid, lane);
    }
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
using SkelL77 = Layout<77, 5, 4, 4, 4, 5>;
using SkelL115 = Layout<115, 5, 4, 4, 4, 5>;
using SkelL115V3 = Layout<115, 3>;  // configs[3]'s V: one 3-bit band over the 115-coefficient skeleton

template <int SK, class SL>
bool sq_geometry_matches(const SpPlan &P, const SpSqGeo &G) {
    using R = SqRec<154, SK, 3, true, SL>;
    return G.default_tables && G.hd == 128 && G.pad == 154 && G.sk_k == SK && G.n_res == 154 - SK && G.rbits == 3 &&
           G.spinor &&
           G.bytes == R::total && layout_matches<SL>(P) && vil_consts_exact(P);
}

template <int DT, int SK, class SL>
hipError_t sq_enc_launch(const SpPlan &P, const void *src, long long so, long long si, unsigned char *dst,
                         long long dout, int n_outer, int n_inner, hipStream_t s) {
    const int tpo = (n_inner + 63) / 64;
    const long long n_tiles = (long long)n_outer * tpo;
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    if (n_tiles > 0x7fffffffLL || si < 128 || 64 * si * esz + 128 * esz > 0x7fffffffLL) return hipErrorNotSupported;
    // one wave per SIMD fits (~330-460 registers): a resident grid, each block prefetching
    const dim3 grid((unsigned)std::min<long long>(n_tiles, resident_blocks(1))), block(64);
    hipLaunchKernelGGL((k_sqfree_encode_lane<DT, 128, 154, SK, 3, true, SL>), grid, block, 0, s, src, so, si, dst,
                       dout, n_inner, tpo, (int)n_tiles, xf_const(P));
    return hipGetLastError();
}

template <int DT, int SK, class SL>
hipError_t sq_dec_launch(const SpPlan &P, const unsigned char *src, long long so, void *dst, long long dout,
                         long long din, int n_outer, int n_inner, hipStream_t s) {
    const int tpo = (n_inner + 63) / 64;
    const long long n_tiles = (long long)n_outer * tpo;
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    if (n_tiles > 0x7fffffffLL || din < 128 || 64 * din * esz + 128 * esz > 0x7fffffffLL) return hipErrorNotSupported;
    // several skeleton bands (a longer tile): a resident grid at two waves per SIMD, each
    // block prefetching its next tile's records (one layer at sk 115: 46.8 -> 43.5 us); one
    // band (a shorter tile): the persistent grid, whose second round of blocks was faster
    // there (39.6 vs 43.6 us)
    const int nb_max = SL::nb > 1 ? resident_blocks(2) : persistent_blocks();
    const dim3 grid((unsigned)std::min<long long>(n_tiles, nb_max)), block(64);
    hipLaunchKernelGGL((k_sqfree_decode_lane<DT, 128, 154, SK, 3, true, SL>), grid, block, 0, s, src, so, dst, dout,
                       din, n_inner, tpo, (int)n_tiles, xf_const(P));
    return hipGetLastError();
}

template <int DT, int SK, class SL>
hipError_t sq_dec_cells_launch(const SpPlan &P, const unsigned char *src, long long so, void *dst, long long dout,
                               long long din, const int *cells, int n_outer, int n_inner, hipStream_t s) {
    const int tpo = (n_inner + 63) / 64;
    const long long n_tiles = (long long)n_outer * tpo;
    if (n_tiles > 0x7fffffffLL || din < 128) return hipErrorNotSupported;
    const dim3 grid((unsigned)std::min<long long>(n_tiles, persistent_blocks())), block(64);
    hipLaunchKernelGGL((k_sqfree_decode_lane_cells<DT, 128, 154, SK, 3, true, SL>), grid, block, 0, s, src, so, dst,
                       dout, din, cells, n_inner, tpo, (int)n_tiles, xf_const(P));
    return hipGetLastError();
}

}  // namespace

// Listed positions (see k_sqfree_decode_lane_cells); hipErrorNotSupported
// (nothing launched) when the geometry or the row alignment has no lane
// specialization. The cache must carry slack bytes past its last record.
hipError_t sp_launch_sqfree_decode_lane_cells(const SpPlan &P, const SpSqGeo &G, const unsigned char *src,
                                              long long so, void *dst, int dtype, long long dout, long long din,
                                              int n_outer, int n_inner, const int *cells, hipStream_t s) {
    const int esz = dtype == SP_DT_F16 ? 2 : 4;
    if (((uintptr_t)dst % 16) || ((dout * esz) % 16) || ((din * esz) % 16)) return hipErrorNotSupported;
    if (sq_geometry_matches<77, SkelL77>(P, G))
        return dtype == SP_DT_F16
                   ? sq_dec_cells_launch<SP_DT_F16, 77, SkelL77>(P, src, so, dst, dout, din, cells, n_outer, n_inner, s)
                   : sq_dec_cells_launch<SP_DT_F32, 77, SkelL77>(P, src, so, dst, dout, din, cells, n_outer, n_inner, s);
    if (sq_geometry_matches<115, SkelL115>(P, G))
        return dtype == SP_DT_F16
                   ? sq_dec_cells_launch<SP_DT_F16, 115, SkelL115>(P, src, so, dst, dout, din, cells, n_outer, n_inner, s)
                   : sq_dec_cells_launch<SP_DT_F32, 115, SkelL115>(P, src, so, dst, dout, din, cells, n_outer, n_inner, s);
    if (sq_geometry_matches<115, SkelL115V3>(P, G))
        return dtype == SP_DT_F16
                   ? sq_dec_cells_launch<SP_DT_F16, 115, SkelL115V3>(P, src, so, dst, dout, din, cells, n_outer, n_inner, s)
                   : sq_dec_cells_launch<SP_DT_F32, 115, SkelL115V3>(P, src, so, dst, dout, din, cells, n_outer, n_inner, s);
    return hipErrorNotSupported;
}

// Returns hipErrorNotSupported (nothing launched) when the geometry or the
// operand alignment has no lane specialization: the caller then uses the
// one-vector-per-wave kernels.
hipError_t sp_launch_sqfree_encode_lane(const SpPlan &P, const SpSqGeo &G, const void *src, int dtype, long long so,
                                        long long si, unsigned char *dst, long long dout, int n_outer, int n_inner,
                                        hipStream_t s) {
    const int esz = dtype == SP_DT_F16 ? 2 : 4;
    if (((uintptr_t)src % 16) || ((so * esz) % 16) || ((si * esz) % 16)) return hipErrorNotSupported;
    if (((uintptr_t)dst % 4) || (dout % 4)) return hipErrorNotSupported;
    if (sq_geometry_matches<77, SkelL77>(P, G))
        return dtype == SP_DT_F16 ? sq_enc_launch<SP_DT_F16, 77, SkelL77>(P, src, so, si, dst, dout, n_outer, n_inner, s)
                                  : sq_enc_launch<SP_DT_F32, 77, SkelL77>(P, src, so, si, dst, dout, n_outer, n_inner, s);
    if (sq_geometry_matches<115, SkelL115>(P, G))
        return dtype == SP_DT_F16 ? sq_enc_launch<SP_DT_F16, 115, SkelL115>(P, src, so, si, dst, dout, n_outer, n_inner, s)
                                  : sq_enc_launch<SP_DT_F32, 115, SkelL115>(P, src, so, si, dst, dout, n_outer, n_inner, s);
    if (sq_geometry_matches<115, SkelL115V3>(P, G))
        return dtype == SP_DT_F16 ? sq_enc_launch<SP_DT_F16, 115, SkelL115V3>(P, src, so, si, dst, dout, n_outer, n_inner, s)
                                  : sq_enc_launch<SP_DT_F32, 115, SkelL115V3>(P, src, so, si, dst, dout, n_outer, n_inner, s);
    return hipErrorNotSupported;
}

hipError_t sp_launch_sqfree_decode_lane(const SpPlan &P, const SpSqGeo &G, const unsigned char *src, long long so,
                                        void *dst, int dtype, long long dout, long long din, int n_outer,
                                        int n_inner, hipStream_t s) {
    const int esz = dtype == SP_DT_F16 ? 2 : 4;
    if (((uintptr_t)dst % 16) || ((dout * esz) % 16) || ((din * esz) % 16)) return hipErrorNotSupported;
    if (((uintptr_t)src % 4) || (so % 4)) return hipErrorNotSupported;
    if (sq_geometry_matches<77, SkelL77>(P, G))
        return dtype == SP_DT_F16 ? sq_dec_launch<SP_DT_F16, 77, SkelL77>(P, src, so, dst, dout, din, n_outer, n_inner, s)
                                  : sq_dec_launch<SP_DT_F32, 77, SkelL77>(P, src, so, dst, dout, din, n_outer, n_inner, s);
    if (sq_geometry_matches<115, SkelL115>(P, G))
        return dtype == SP_DT_F16 ? sq_dec_launch<SP_DT_F16, 115, SkelL115>(P, src, so, dst, dout, din, n_outer, n_inner, s)
                                  : sq_dec_launch<SP_DT_F32, 115, SkelL115>(P, src, so, dst, dout, din, n_outer, n_inner, s);
    if (sq_geometry_matches<115, SkelL115V3>(P, G))
        return dtype == SP_DT_F16 ? sq_dec_launch<SP_DT_F16, 115, SkelL115V3>(P, src, so, dst, dout, din, n_outer, n_inner, s)
                                  : sq_dec_launch<SP_DT_F32, 115, SkelL115V3>(P, src, so, dst, dout, din, n_outer, n_inner, s);
    return hipErrorNotSupported;
}
