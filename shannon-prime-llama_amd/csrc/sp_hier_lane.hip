// sp_hier_lane.hip -- one-vector-per-lane hierarchical Vilenkin codec kernels
// for the default geometry at head_dim 256: pad 330 = 2*3*5*11 (true-mean
// fill), skeleton = the first 30 squarefree-first coefficients in two 5-bit
// bands, targets = the other 300 with 2-bit residuals about the slot's fp16
// predictor W[300][30]. Record [skeleton bands 24 B][mag f32 LE][75 B residual
// codes] = 103 B (shannon_prime_hier.cu:331-335).
//
// The arithmetic and its order are those of k_hier_encode / k_hier_decode
// (sp_cuda_hier_write_one / read_one, shannon_prime_hier.cu:399-571), so records
// and reconstructions are bit-identical to them. Each lane owns one vector: the
// pad, the staged Vilenkin transform, the skeleton quantizer, the prediction,
// the residual quantizer and every record field are register operations at
// compile-time positions. A 64-vector tile never spans two slots, so a target's
// predictor row is the same for every lane: W streams through scalar loads and
// each product is one v_fma_mix taking the fp16 weight from a scalar register.
#include "sp_lane.h"

namespace {

// Default geometry (sp_hier_default_geometry): skeleton = the first NS entries
// of the squarefree-first order over [0, PAD), targets = the rest in order.
template <int PAD, int NS>
struct HierGeoC {
    static constexpr int NT = PAD - NS;
    int skel[NS];
    int tgt[NT];
    constexpr HierGeoC() : skel(), tgt() {
        const MobOrder<PAD> mo{};
        for (int s = 0; s < NS; s++) skel[s] = mo.v[s];
        for (int t = 0; t < NT; t++) tgt[t] = mo.v[NS + t];
    }
};
template <int PAD, int NS>
__device__ constexpr HierGeoC<PAD, NS> kHier{};

// Three predictions at once: ak += wk.lo*x0, then ak += wk.hi*x1 for k = 0..2, each
// step rounded once. v_fma_mix widens the fp16 weight (from a scalar register)
// exactly and rounds w*x + 0 (the + 0 turns a -0 product into +0, which a running
// sum started at +0.0f cannot tell apart: such a sum is never -0), then v_add_f32.
// The three independent chains give each add two free slots after its product; one
// asm block keeps products next to their adds, so the predictions stay serial chains
// in registers.
__device__ __forceinline__ void wmac3x2(float &a0, float &a1, float &a2, uint32_t w0, uint32_t w1, uint32_t w2,
                                        float x0, float x1) {
    float p0, p1, p2;
    __asm__("v_fma_mix_f32 %3, %6, %9, 0 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %4, %7, %9, 0 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %5, %8, %9, 0 op_sel_hi:[1,0,0]\n\t"
            "v_add_f32 %0, %0, %3\n\t"
            "v_add_f32 %1, %1, %4\n\t"
            "v_add_f32 %2, %2, %5\n\t"
            "v_fma_mix_f32 %3, %6, %10, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %4, %7, %10, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %5, %8, %10, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "v_add_f32 %0, %0, %3\n\t"
            "v_add_f32 %1, %1, %4\n\t"
            "v_add_f32 %2, %2, %5"
            : "+v"(a0), "+v"(a1), "+v"(a2), "=&v"(p0), "=&v"(p1), "=&v"(p2)
            : "s"(w0), "s"(w1), "s"(w2), "v"(x0), "v"(x1));
}

// The first step of wmac3x2 for sums started at +0.0f: 0 + w*x rounds to w*x + 0,
// which is what v_fma_mix gives (never -0), so the sums start at the first products
// (no zero moves, no first adds). after: a value the triple is ordered behind (an
// operand the block does not read).
__device__ __forceinline__ void wmac3x2_first(float &a0, float &a1, float &a2, uint32_t w0, uint32_t w1,
                                              uint32_t w2, float x0, float x1, float after) {
    float p0, p1, p2;
    __asm__("v_fma_mix_f32 %0, %6, %9, 0 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %1, %7, %9, 0 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %2, %8, %9, 0 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %3, %6, %10, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %4, %7, %10, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %5, %8, %10, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "v_add_f32 %0, %0, %3\n\t"
            "v_add_f32 %1, %1, %4\n\t"
            "v_add_f32 %2, %2, %5"
            : "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(p0), "=&v"(p1), "=&v"(p2)
            : "s"(w0), "s"(w1), "s"(w2), "v"(x0), "v"(x1), "v"(after));
}

// W is read through the constant address space: the tile-uniform row address
// then always becomes scalar loads (the scalar cache), whatever the compiler
// can prove about the kernel's other stores.
typedef const __attribute__((address_space(4))) uint32_t *wptr_t;

// pred = sum_s (float)W[t][s] * sk[s] from 0.0f, s ascending, separately rounded
// products and adds (kernel_hier_predict, shannon_prime_hier.cu:74-92), for targets
// t, t+1, t+2: w holds their three rows, NS/2 fp16 pairs each, in scalar registers.
// after: a value the triple is ordered behind.
//
// With MORE, the rows of the next triple are loaded into wn after the first
// products: the wait for w (loaded one triple earlier) comes before those products,
// and a scalar-load wait covers every scalar load in flight, so rows loaded before it
// would be waited for there too. The scheduling barriers keep the loads in that
// place, with three targets' products (~180 VALU instructions) in front of the next
// wait. Loaded where their own target pair started, the rows left the wave (one per
// SIMD) waiting ~600 times per tile; one pair ahead, two targets' products covered
// each wait.
template <int NS, bool MORE>
__device__ __forceinline__ void hier_predict3(const uint32_t (&w)[3 * NS / 2], uint32_t (&wn)[3 * NS / 2],
                                              wptr_t next, const float (&sk)[NS], float after, float &r0,
                                              float &r1, float &r2) {
    static_assert(NS % 2 == 0, "rows of fp16 pairs");
    constexpr int RW = NS / 2;
    float a0, a1, a2;
    wmac3x2_first(a0, a1, a2, w[0], w[RW], w[2 * RW], sk[0], sk[1], after);
    if constexpr (MORE) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 3 * RW; i++) wn[i] = next[i];
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int s = 2; s < NS; s += 2) wmac3x2(a0, a1, a2, w[s / 2], w[RW + s / 2], w[2 * RW + s / 2], sk[s], sk[s + 1]);
    r0 = a0, r1 = a1, r2 = a2;
}

// fp16 halves H of a and b: a + b rounded once (exact widening).
template <int H>
__device__ __forceinline__ float add_f16_halves(uint32_t a, uint32_t b) {
    float r;
    if (H)
        __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
    else
        __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

constexpr int HIER_HD = 256;

template <int DT, int PAD, int NS, int RBITS, class SL>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_hier_encode_lane(const void *__restrict__ src, long long so, long long si, unsigned char *__restrict__ dst,
                   long long dout, int n_inner, int tiles_per_outer, int n_tiles, const XfConst K,
                   const uint16_t *__restrict__ W, long long w_outer, const void *__restrict__ src2,
                   unsigned char *__restrict__ dst2, int n_sides) {
    constexpr int HD = HIER_HD, NT = PAD - NS;
    using G = HierRec<NT, RBITS, SL>;
    constexpr int RP = row_bytes<DT>(HD) + 16, DWR = G::dwords;
    constexpr auto &HG = kHier<PAD, NS>;
    static_assert(SL::hd == NS && (PAD - HD) % 2 == 0 && NT % 2 == 0, "geometry");
    __shared__ __attribute__((aligned(16))) unsigned char rows[64 * RP];  // input rows, then the record stage
    const int lane = threadIdx.x;
    const TileMap M{tiles_per_outer, n_inner};
    // n_sides == 2: tiles [n_tiles, 2 n_tiles) encode the second side (src2 -> dst2, the
    // same slots and W), so a layer's K and V share one launch
    for (int tt = blockIdx.x; tt < n_sides * n_tiles; tt += gridDim.x) {
        const bool second = tt >= n_tiles;
        const int t = second ? tt - n_tiles : tt;
        const void *const sp = second ? src2 : src;
        unsigned char *const dp = second ? dst2 : dst;
        tile_rows_stage<DT, HD>(sp, so, si, M, t, lane, rows);
        const unsigned char *row = rows + lane * RP;
        // pad mean: the first level of the 256-slot tree, x[i] + x[i + 128],
        // straight from the staged row, then the rest of the tree
        float l1[HD / 2];
        float mx = 0.0f;
        if (DT == SP_DT_F16) {
#pragma unroll
            for (int q = 0; q < HD / 16; q++) {
                const uint4 a = *reinterpret_cast<const uint4 *>(row + q * 16);
                const uint4 b = *reinterpret_cast<const uint4 *>(row + HD + q * 16);
                const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    l1[q * 8 + 2 * k] = add_f16_halves<0>(wa[k], wb[k]);
                    l1[q * 8 + 2 * k + 1] = add_f16_halves<1>(wa[k], wb[k]);
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < HD / 8; q++) {
                const float4 a = *reinterpret_cast<const float4 *>(row + q * 16);
                const float4 b = *reinterpret_cast<const float4 *>(row + 2 * HD + q * 16);
                const float fa[4] = {a.x, a.y, a.z, a.w}, fb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    l1[q * 4 + k] = fa[k] + fb[k];
                    mx = fmaxf(mx, fmaxf(fabsf(fa[k]), fabsf(fb[k])));
                }
            }
        }
#pragma unroll
        for (int s = HD / 4; s > 0; s >>= 1) {
#pragma unroll
            for (int i = 0; i < s; i++) l1[i] = l1[i] + l1[i + s];
        }
        const float mean = sp_div(l1[0] + 0.0f, (float)HD);
        float c[PAD];
        if (DT == SP_DT_F16) {
            // first stage (p = 2, stride 1) straight from the fp16 pairs; the pad
            // pairs are (mean, mean)
            const float isp2 = K.isp[0];
#pragma unroll
            for (int q = 0; q < HD / 8; q++) {
                const uint4 a = *reinterpret_cast<const uint4 *>(row + q * 16);
                const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int k = 0; k < 4; k++) vil_first_f16_pair(w[k], isp2, c[q * 8 + 2 * k], c[q * 8 + 2 * k + 1]);
            }
            const float z = 0.0f + mean, p0 = (z + mean) * isp2, p1 = (z - mean) * isp2;
#pragma unroll
            for (int i = HD; i < PAD; i += 2) {
                c[i] = p0;
                c[i + 1] = p1;
            }
            vil_stages<PAD, 1, 2>(c, K);
        } else {
#pragma unroll
            for (int q = 0; q < HD / 4; q++) {
                const float4 a = *reinterpret_cast<const float4 *>(row + q * 16);
                c[4 * q] = a.x, c[4 * q + 1] = a.y, c[4 * q + 2] = a.z, c[4 * q + 3] = a.w;
            }
#pragma unroll
            for (int i = HD; i < PAD; i++) c[i] = mean;
            vil_stages<PAD, 0, 1>(c, K);
        }
        // the transform completes here: without this the compiler sinks the last
        // stage's target outputs below the prediction loop, where the stage
        // inputs and the deviations are live at once and spill
#pragma unroll
        for (int i = 0; i < PAD; i++) __asm__ volatile("" : "+v"(c[i]));
        // growth is at most sqrt(2p) per stage: fp16 inputs stay finite, fp32
        // inputs below 2^100 too; inf/NaN inputs reach the DC coefficient
        const bool fastv = (DT == SP_DT_F16 || mx < 1.2676506e30f) && __builtin_isfinite(c[0]);
        float sk[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) sk[s] = c[HG.skel[s]];
        uint32_t rec[DWR];
#pragma unroll
        for (int d = 0; d < DWR; d++) rec[d] = 0u;
        quant_bands<SL, false>(sk, fastv, rec);
        // deviation of each target from the prediction of the unquantized skeleton
        int o, i0, nv;
        M.at(t, o, i0, nv);
        const wptr_t w32 = (wptr_t)(W + (long long)__builtin_amdgcn_readfirstlane(o) * w_outer);
        // the predictions of targets r, r+1 start after deviation r-1 exists, so
        // the target coefficients are consumed pair by pair: without the ordering
        // the subtractions sink to the tree sum and everything spills
        // W rows of target triples r and r + 3 alternate between wa and wb
        static_assert(NT % 6 == 0, "two target triples per step");
        constexpr int RW = NS / 2;
        uint32_t wa[3 * RW], wb[3 * RW];
#pragma unroll
        for (int i = 0; i < 3 * RW; i++) wa[i] = w32[i];
        float dv[NT];
#pragma unroll
        for (int r = 0; r < NT; r += 6) {
            float p0, p1, p2;
            hier_predict3<NS, true>(wa, wb, w32 + (r + 3) * RW, sk, r > 0 ? dv[r - 1] : sk[0], p0, p1, p2);
            dv[r] = c[HG.tgt[r]] - p0;
            dv[r + 1] = c[HG.tgt[r + 1]] - p1;
            dv[r + 2] = c[HG.tgt[r + 2]] - p2;
            if (r + 6 < NT)
                hier_predict3<NS, true>(wb, wa, w32 + (r + 6) * RW, sk, dv[r + 2], p0, p1, p2);
            else
                hier_predict3<NS, false>(wb, wa, w32, sk, dv[r + 2], p0, p1, p2);
            dv[r + 3] = c[HG.tgt[r + 3]] - p0;
            dv[r + 4] = c[HG.tgt[r + 4]] - p1;
            dv[r + 5] = c[HG.tgt[r + 5]] - p2;
        }
        float mag = sp_div(tree256_sum<NT, true>(dv), (float)NT);
        mag = mag < 1e-12f ? 1e-12f : mag;
        rec_put32(rec, G::mag_byte, __float_as_uint(mag));
        // levels rint(dev * inv_step + center) clamped to [0, L-1] with
        // step = 2*mag/(L-1) (shannon_prime_hier.cu:151-171); clamping before
        // the rounding gives the same level for every value, NaN (-> 0) included
        constexpr int L = 1 << RBITS;
        const float step = sp_div(2.0f * mag, (float)(L - 1));
        const float center = sp_div((float)(L - 1), 2.0f);
        const float inv_step = (step > 0.0f) ? sp_div(1.0f, step) : 0.0f;
        // cl + 1.5 * 2^23 rounds cl (in [0, L-1]) to the nearest integer, ties to even,
        // as rint does, into the low mantissa bits; rec_add_code sums it into the
        // (still zero) residual field with the exponent bits cancelled
#pragma unroll
        for (int r = 0; r < NT; r++) {
            const float v = dv[r] * inv_step + center;
            const float cl = fminf(fmaxf(v, 0.0f), (float)(L - 1));
            rec_add_code(rec, G::res_bit + r * RBITS, RBITS, __float_as_uint(cl + 12582912.0f), 0);
        }
        tile_records_out<G::total, 64 * RP>(rec, rows, dp, dout, M, t, lane);
    }
}

// LISTED: lane j of tile t decodes the record at position cells[i0 + j] into row
// cells[i0 + j] (the dual cache's System 2 rows): its own record read directly,
// rows out through rows_out_listed.
template <int DT, int PAD, int NS, int RBITS, class SL, bool LISTED>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_hier_decode_lane(const unsigned char *__restrict__ src, long long so, void *__restrict__ dst, long long dout,
                   long long din, int n_inner, int tiles_per_outer, int n_tiles, const XfConst K,
                   const uint16_t *__restrict__ W, long long w_outer, const int *__restrict__ cells) {
    constexpr int HD = HIER_HD, NT = PAD - NS;
    using G = HierRec<NT, RBITS, SL>;
    constexpr int RP = row_bytes<DT>(HD) + 16, DWR = G::dwords;
    constexpr auto &HG = kHier<PAD, NS>;
    static_assert(RecTile<G>::NCK * 1024 + 16 <= 64 * RP && 64 * G::total + 4 * DWR + 8 <= 64 * RP && NT % 2 == 0,
                  "record tile must fit in the row stage");
    __shared__ __attribute__((aligned(16))) unsigned char stage[64 * RP];
    const int lane = threadIdx.x, Gs = gridDim.x;
    const TileMap M{tiles_per_outer, n_inner};
    RecTile<G> R;
    int t = blockIdx.x;
    if (t >= n_tiles) return;
    if constexpr (!LISTED) rec_tile_load<G>(R, src, so, M, t, n_tiles, lane);
    for (; t < n_tiles; t += Gs) {
        uint32_t rec[DWR];
        int pos = 0;
        if constexpr (LISTED) {
            int o_, i0_, nv_;
            M.at(t, o_, i0_, nv_);
            pos = cells[lane < nv_ ? i0_ + lane : i0_];
            rec_load_direct<G>(rec, src + (long long)o_ * so + (long long)pos * G::total);
        } else {
            rec_tile_stage<G>(R, stage, M, t, lane);
            __syncthreads();
            rec_tile_load<G>(R, src, so, M, t + Gs, n_tiles, lane);
            rec_from_lds<G>(rec, stage, lane);
        }
        float sk[NS];
        dequant_bands<SL, false, true>(rec, SL::nb, sk);
        float c[PAD];
#pragma unroll
        for (int s = 0; s < NS; s++) c[HG.skel[s]] = sk[s];
        // targets: prediction from the dequantized skeleton plus (lvl - center) * step
        const float mag = __uint_as_float(rec_get32(rec, G::mag_byte));
        constexpr int L = 1 << RBITS;
        const float step = sp_div(2.0f * mag, (float)(L - 1));
        const float center = sp_div((float)(L - 1), 2.0f);
        int o, i0, nv;
        M.at(t, o, i0, nv);
        const wptr_t w32 = (wptr_t)(W + (long long)__builtin_amdgcn_readfirstlane(o) * w_outer);
        // W rows of target triples r and r + 3 alternate between wa and wb
        static_assert(NT % 6 == 0, "two target triples per step");
        constexpr int RW = NS / 2;
        uint32_t wa[3 * RW], wb[3 * RW];
#pragma unroll
        for (int i = 0; i < 3 * RW; i++) wa[i] = w32[i];
#pragma unroll
        for (int r = 0; r < NT; r += 3) {
            float p[3];
            uint32_t(&w)[3 * RW] = ((r / 3) & 1) ? wb : wa;
            uint32_t(&wn)[3 * RW] = ((r / 3) & 1) ? wa : wb;
            if (r + 3 < NT)
                hier_predict3<NS, true>(w, wn, w32 + (r + 3) * RW, sk, sk[0], p[0], p[1], p[2]);
            else
                hier_predict3<NS, false>(w, wn, w32, sk, sk[0], p[0], p[1], p[2]);
#pragma unroll
            for (int k = 0; k < 3; k++)
                c[HG.tgt[r + k]] = p[k] + ((float)rec_extract(rec, G::res_bit + (r + k) * RBITS, RBITS) - center) * step;
        }
        vil_stages<PAD, 0, 1>(c, K);
        if constexpr (LISTED)
            rows_out_listed<DT, HD>(c, stage, dst, dout, din, o, pos, nv, lane);
        else
            tile_rows_out<DT, HD>(c, stage, dst, dout, din, M, t, lane);
    }
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
using HierSkL = Layout<30, 5, 5>;
using HierR = HierRec<300, 2, HierSkL>;

bool hier_geometry_matches(const SpPlan &P, const SpHierGeo &G) {
    return G.default_geo && G.hd == HIER_HD && G.pad == 330 && G.n_skel == 30 && G.n_target == 300 && G.rbits == 2 &&
           G.bytes == HierR::total && layout_matches<HierSkL>(P) && vil_consts_exact(P) &&
           ((uintptr_t)G.W % 4) == 0 && (G.w_outer % 2) == 0;
}

template <int DT>
hipError_t hier_enc_launch(const SpPlan &P, const SpHierGeo &G, const void *src, long long so, long long si,
                           unsigned char *dst, long long dout, int n_outer, int n_inner, hipStream_t s,
                           const void *src2, unsigned char *dst2) {
    const int tpo = (n_inner + 63) / 64;
    const long long n_tiles = (long long)n_outer * tpo;
    const int sides = src2 ? 2 : 1;
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    if (sides * n_tiles > 0x7fffffffLL || si < HIER_HD || 64 * si * esz + HIER_HD * esz > 0x7fffffffLL)
        return hipErrorNotSupported;
    const dim3 grid((unsigned)std::min<long long>(sides * n_tiles, persistent_blocks())), block(64);
    hipLaunchKernelGGL((k_hier_encode_lane<DT, 330, 30, 2, HierSkL>), grid, block, 0, s, src, so, si, dst, dout,
                       n_inner, tpo, (int)n_tiles, xf_const(P), G.W, G.w_outer, src2, dst2, sides);
    return hipGetLastError();
}

template <int DT>
hipError_t hier_dec_launch(const SpPlan &P, const SpHierGeo &G, const unsigned char *src, long long so, void *dst,
                           long long dout, long long din, int n_outer, int n_inner, hipStream_t s, const int *cells) {
    const int tpo = (n_inner + 63) / 64;
    const long long n_tiles = (long long)n_outer * tpo;
    constexpr long long esz = DT == SP_DT_F16 ? 2 : 4;
    if (n_tiles > 0x7fffffffLL || din < HIER_HD || 64 * din * esz + HIER_HD * esz > 0x7fffffffLL)
        return hipErrorNotSupported;
    const dim3 grid((unsigned)std::min<long long>(n_tiles, persistent_blocks())), block(64);
    if (cells)
        hipLaunchKernelGGL((k_hier_decode_lane<DT, 330, 30, 2, HierSkL, true>), grid, block, 0, s, src, so, dst, dout,
                           din, n_inner, tpo, (int)n_tiles, xf_const(P), G.W, G.w_outer, cells);
    else
        hipLaunchKernelGGL((k_hier_decode_lane<DT, 330, 30, 2, HierSkL, false>), grid, block, 0, s, src, so, dst, dout,
                           din, n_inner, tpo, (int)n_tiles, xf_const(P), G.W, G.w_outer, nullptr);
    return hipGetLastError();
}

}  // namespace

// Returns hipErrorNotSupported (nothing launched) when the geometry or the
// operand alignment has no lane specialization: the caller then uses the
// one-vector-per-wave kernels.
// src2/dst2 (optional): a second side (V after K) with the same strides and slots,
// encoded by the same launch.
hipError_t sp_launch_hier_encode_lane(const SpPlan &P, const SpHierGeo &G, const void *src, int dtype, long long so,
                                      long long si, unsigned char *dst, long long dout, int n_outer, int n_inner,
                                      hipStream_t s, const void *src2, unsigned char *dst2) {
    const int esz = dtype == SP_DT_F16 ? 2 : 4;
    if (((uintptr_t)src % 16) || ((so * esz) % 16) || ((si * esz) % 16)) return hipErrorNotSupported;
    if (((uintptr_t)dst % 4) || (dout % 4)) return hipErrorNotSupported;
    if (src2 && (((uintptr_t)src2 % 16) || ((uintptr_t)dst2 % 4) || !dst2)) return hipErrorNotSupported;
    if (!hier_geometry_matches(P, G)) return hipErrorNotSupported;
    return dtype == SP_DT_F16 ? hier_enc_launch<SP_DT_F16>(P, G, src, so, si, dst, dout, n_outer, n_inner, s, src2, dst2)
                              : hier_enc_launch<SP_DT_F32>(P, G, src, so, si, dst, dout, n_outer, n_inner, s, src2, dst2);
}

hipError_t sp_launch_hier_decode_lane(const SpPlan &P, const SpHierGeo &G, const unsigned char *src, long long so,
                                      void *dst, int dtype, long long dout, long long din, int n_outer, int n_inner,
                                      hipStream_t s, const int *cells) {
    const int esz = dtype == SP_DT_F16 ? 2 : 4;
    if (((uintptr_t)dst % 16) || ((dout * esz) % 16) || ((din * esz) % 16)) return hipErrorNotSupported;
    if (((uintptr_t)src % 4) || (so % 4)) return hipErrorNotSupported;
    if (!hier_geometry_matches(P, G)) return hipErrorNotSupported;
    return dtype == SP_DT_F16 ? hier_dec_launch<SP_DT_F16>(P, G, src, so, dst, dout, din, n_outer, n_inner, s, cells)
                              : hier_dec_launch<SP_DT_F32>(P, G, src, so, dst, dout, din, n_outer, n_inner, s, cells);
}
