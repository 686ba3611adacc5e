// sp_attn_lane.hip -- fused decompress-attention decode over ship records for the
// layouts the matrix-core kernel does not take, one position per lane: head_dim 96
// (the bridge's default bands K 5/4/4 + V 5, Vilenkin 2^5 * 3; configs[2]) and
// head_dim 64 (K 5/5/4/3 + V 3).
//
// The algebra is that of the general kernel (sp_attn.hip): with q~ = kq_scale *
// reorder(transform(q)) prepared once per query head (k_attn_prep), q . K~_t is the
// dot product of q~ with K's dequantized record in record order, and
// sum_t p_t V~_t = transform(sum_t p_t dq(V_t)), finished per query head by
// k_attn_combine. Here the split kernel is one wave per block walking a run of
// 64-position tiles: lane = position, the record dequantized into the lane's
// registers (compile-time band layout), the scores as dot products with the prepared
// queries (scalar loads), an online softmax across the run's tiles, and the V
// coefficient sums through an LDS transpose in chunks of 32 coefficients (lanes c and
// c + 32 sum coefficient c over the tile's two halves of 32 positions, added at the end
// of the run). Partials [m, l, o~[hd]] per (query head, run), the layout
// k_attn_combine merges.
#include "sp_lane.h"

namespace {

constexpr int EP = 65;  // LDS row pitch (floats) of the transposed coefficient chunk

// wave reductions on DPP and the row swaps (every lane active at each call)
__device__ __forceinline__ float wmax(float v) { return sp_wave_max_dpp(v); }
__device__ __forceinline__ float wadd(float v) { return sp_wave_sum_dpp(v); }

// A record's codes centred, in record order, without their band scales: x = code -
// (2^(bits-1) - 1), exact (the magic-number conversion of dequant_bands), and each
// band's scale, 0 for bands >= max_bands (the read-as-0 rule; a finite sum times 0
// adds nothing). Attention applies a K band's scale once to the band's dot product
// and folds the V scale into the softmax weight, so no coefficient pays a multiply
// or a band-limit select.
template <class LY, int DWR>
__device__ __forceinline__ void codes_centred(const uint32_t (&rec)[DWR], int max_bands, float (&x)[LY::hd],
                                              float (&sc)[LY::nb]) {
#pragma unroll
    for (int b = 0; b < LY::nb; b++) {
        const int off = LY::off(b), sz = LY::sz(b), bits = LY::bits[b];
        const int bo = LY::byte_off(b);
        sc[b] = b < max_bands ? sp_scale_from_bits(rec_extract(rec, 8 * bo, 16)) : 0.0f;
        const float bias = 12582912.0f + (float)((1 << (bits - 1)) - 1);
#pragma unroll
        for (int e = 0; e < sz; e++)
            x[off + e] = __uint_as_float(rec_extract(rec, 8 * (bo + 2) + e * bits, bits) | 0x4B400000u) - bias;
    }
}

// Block (kvh, run) takes tiles run, run + n_runs, ... of KV head kvh. qt: prepared
// queries [n_q][hd] (record order). K bands >= kmb and V bands >= vmb read as 0.
template <class LK, class LV, int GM, bool OUT>
__global__ void __launch_bounds__(64)
k_attn_lane_split(const unsigned char *__restrict__ kc0, const unsigned char *__restrict__ vc0, long long k_slot,
                  long long v_slot, const SpSeqTab T, int G, const float *__restrict__ qt0, float *__restrict__ scores0,
                  float *__restrict__ part0, int n_runs, int kmb, int vmb) {
    constexpr int HD = LK::hd;
    static_assert(LV::hd == HD, "K and V layouts share head_dim");
    static_assert(LV::nb == 1, "V's scale rides on the softmax weight: one band");
    constexpr int NCK = RecTile<LK>::NCK > RecTile<LV>::NCK ? RecTile<LK>::NCK : RecTile<LV>::NCK;
    // V sums in chunks of 32 coefficients: lane (c, half) = (lane & 31, lane >> 5) sums
    // coefficient 32 ch + c over the tile's positions 32 half .. 32 half + 31
    constexpr int NCH = HD / 32;
    static_assert(HD % 32 == 0, "whole 32-coefficient chunks");
    __shared__ __attribute__((aligned(16))) unsigned char stage[NCK * 1024 + 16];
    __shared__ float E[32 * EP];
    __shared__ __attribute__((aligned(16))) float Pw[64 * GM];
    const int kvh = blockIdx.x, run = blockIdx.y, lane = threadIdx.x;
    // sequence blockIdx.z: its positions, prepared queries, score rows and partials
    const int seq = blockIdx.z, n_q = (int)gridDim.x * G, n_kv = T.len[seq];
    const unsigned char *__restrict__ kc = kc0 + (long long)T.start[seq] * LK::total;
    const unsigned char *__restrict__ vc = vc0 + (long long)T.start[seq] * LV::total;
    const long long s_stride = T.len[seq];
    float *__restrict__ scores = scores0 ? scores0 + T.soff[seq] : nullptr;
    const float *__restrict__ qt = qt0 + (long long)seq * n_q * HD;
    float *__restrict__ part = part0 + (long long)seq * n_q * n_runs * (HD + 2);
    const int h0 = kvh * G;
    const int tpo = (n_kv + 63) / 64;
    const int n_tiles = (int)gridDim.x * tpo;
    const TileMap M{tpo, n_kv};
    const float *__restrict__ pq = qt + (long long)h0 * HD;

    float m_run[GM], l_run[GM];
    float acc[NCH][GM];
#pragma unroll
    for (int h = 0; h < GM; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) acc[ch][h] = 0.0f;
    }
    const int vc_i = lane & 31, vp0 = 32 * (lane >> 5);

    // both record streams run one tile ahead: the next tile's K loads once this tile's
    // K records are out of the stage, its V once this tile's V records are
    RecTile<LK> Rk;
    RecTile<LV> Rv;
    int c = run;
    if (c < tpo) {
        rec_tile_load<LK>(Rk, kc, k_slot, M, kvh * tpo + c, n_tiles, lane);
        if (OUT) rec_tile_load<LV>(Rv, vc, v_slot, M, kvh * tpo + c, n_tiles, lane);
    }
    for (; c < tpo; c += n_runs) {
        const int t = kvh * tpo + c;
        __syncthreads();  // the previous tile is done with the stage
        rec_tile_stage<LK>(Rk, stage, M, t, lane);
        __syncthreads();
        uint32_t rk[LK::dwords];
        rec_from_lds<LK>(rk, stage, lane);
        if (c + n_runs < tpo) rec_tile_load<LK>(Rk, kc, k_slot, M, t + n_runs, n_tiles, lane);
        float e[HD], ks[LK::nb];
        codes_centred<LK>(rk, kmb, e, ks);  // record order; bands past kmb scale 0
        const int pos = c * 64 + lane;
        const bool live = pos < n_kv;
        float s[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            s[h] = -INFINITY;
            if (h < G) {
                const float *__restrict__ qh = pq + h * HD;
                float v = 0.0f;
#pragma unroll
                for (int b = 0; b < LK::nb; b++) {
                    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                    for (int j = LK::off(b); j < LK::off(b) + LK::sz(b); j += 2) {
                        a0 = fmaf(qh[j], e[j], a0);
                        if (j + 1 < LK::off(b) + LK::sz(b)) a1 = fmaf(qh[j + 1], e[j + 1], a1);
                    }
                    v = fmaf(ks[b], a0 + a1, v);
                }
                if (live) {
                    s[h] = v;
                    if (scores) scores[(long long)(h0 + h) * s_stride + pos] = v;
                }
            }
        }
        if (!OUT) continue;
        float alpha[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            alpha[h] = 1.0f;
            float pr = 0.0f;
            if (h < G) {
                const float mn = fmaxf(m_run[h], wmax(s[h]));
                alpha[h] = __expf(m_run[h] - mn);
                pr = live ? __expf(s[h] - mn) : 0.0f;
                l_run[h] = fmaf(l_run[h], alpha[h], wadd(pr));
                m_run[h] = mn;
            }
            Pw[lane * GM + h] = pr;
        }
        __syncthreads();  // every lane has read its K record from the stage
        rec_tile_stage<LV>(Rv, stage, M, t, lane);
        __syncthreads();
        uint32_t rv[LV::dwords];
        rec_from_lds<LV>(rv, stage, lane);
        if (c + n_runs < tpo) rec_tile_load<LV>(Rv, vc, v_slot, M, t + n_runs, n_tiles, lane);
        // V's one band: centred codes here, its scale in this position's weights
        float ev[HD], vs[1];
        codes_centred<LV>(rv, vmb, ev, vs);
#pragma unroll
        for (int h = 0; h < GM; h++) Pw[lane * GM + h] *= vs[0];
#pragma unroll
        for (int h = 0; h < GM; h++)
#pragma unroll
            for (int ch = 0; ch < NCH; ch++) acc[ch][h] *= alpha[h];
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
#pragma unroll
            for (int i = 0; i < 32; i++) E[i * EP + lane] = ev[32 * ch + i];
            __syncthreads();
#pragma unroll 4
            for (int p = 0; p < 32; p++) {
                const float ei = E[vc_i * EP + vp0 + p];
#pragma unroll
                for (int h = 0; h < GM; h++) acc[ch][h] = fmaf(Pw[(vp0 + p) * GM + h], ei, acc[ch][h]);
            }
            __syncthreads();
        }
    }
    if (!OUT) return;
    // ---- the run's partial per query head: [m, l, o~[hd]], the two position halves
    // of each coefficient added across lanes c and c + 32 ----
#pragma unroll
    for (int h = 0; h < GM; h++) {
        if (h >= G) continue;
        float *dst = part + ((long long)(h0 + h) * n_runs + run) * (HD + 2);
        if (lane == 0) {
            dst[0] = m_run[h];
            dst[1] = l_run[h];
        }
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            const float v = acc[ch][h] + __shfl_xor(acc[ch][h], 32, 64);
            if (lane < 32) dst[2 + 32 * ch + lane] = v;
        }
    }
}

template <class LK, class LV, int GM>
void launch_lane(const SpAttnArgs &A, const SpSeqTab &T, const float *qt, float *part, int n_runs, int kmb, int vmb,
                 hipStream_t s) {
    const dim3 grid(A.n_kvh, n_runs, T.n_seq), block(64);
    const int G = A.n_q / A.n_kvh;
    if (A.out)
        hipLaunchKernelGGL((k_attn_lane_split<LK, LV, GM, true>), grid, block, 0, s, A.kpack, A.vpack,
                           A.k_head_stride, A.v_head_stride, T, G, qt, A.scores, part, n_runs, kmb, vmb);
    else
        hipLaunchKernelGGL((k_attn_lane_split<LK, LV, GM, false>), grid, block, 0, s, A.kpack, A.vpack,
                           A.k_head_stride, A.v_head_stride, T, G, qt, A.scores, part, n_runs, kmb, vmb);
}

template <class LK, class LV>
void launch_lane_g(const SpAttnArgs &A, const SpSeqTab &T, const float *qt, float *part, int n_runs, int kmb, int vmb,
                   hipStream_t s) {
    const int G = A.n_q / A.n_kvh;
    if (G <= 1) launch_lane<LK, LV, 1>(A, T, qt, part, n_runs, kmb, vmb, s);
    else if (G <= 2) launch_lane<LK, LV, 2>(A, T, qt, part, n_runs, kmb, vmb, s);
    else if (G <= 4) launch_lane<LK, LV, 4>(A, T, qt, part, n_runs, kmb, vmb, s);
    else launch_lane<LK, LV, 8>(A, T, qt, part, n_runs, kmb, vmb, s);
}

template <class LY>
bool plan_is(const SpPlan &P) {
    if (P.hd != LY::hd || P.n_bands != LY::nb || P.total_bytes != LY::total || P.skip_transform) return false;
    for (int b = 0; b < LY::nb; b++)
        if (P.band_bits[b] != LY::bits[b] || P.band_off[b] != LY::off(b) || P.band_sz[b] != LY::sz(b)) return false;
    return true;
}

using K96 = Layout<96, 5, 4, 4>;
using V96 = Layout<96, 5>;
using K64 = Layout<64, 5, 5, 4, 3>;
using V64 = Layout<64, 3>;

// One-wave blocks of the instance for this call resident on a CU at once (registers
// and LDS decide; 4 when the runtime cannot say).
template <class LK, class LV, int GM>
int resident_per_cu(bool out) {
    int nb = 0;
    const hipError_t e = out ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_attn_lane_split<LK, LV, GM, true>,
                                                                           64, 0)
                             : hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_attn_lane_split<LK, LV, GM, false>,
                                                                           64, 0);
    return e == hipSuccess && nb > 0 ? nb : 4;
}
template <class LK, class LV>
int resident_per_cu_g(int G, bool out) {
    if (G <= 1) return resident_per_cu<LK, LV, 1>(out);
    if (G <= 2) return resident_per_cu<LK, LV, 2>(out);
    if (G <= 4) return resident_per_cu<LK, LV, 4>(out);
    return resident_per_cu<LK, LV, 8>(out);
}

}  // namespace

// Runs per KV head and sequence for the lane split kernel: at most the workspace's
// partial rows, at least one tile per run, and the instance's resident one-wave blocks
// spread over the sequences' KV heads (one round). 0 when no lane kernel serves the
// call's layouts.
int sp_attn_lane_runs(const SpPlan &KP, const SpPlan &VP, const SpAttnArgs &A, size_t part_floats, int n_seq) {
    const bool ok = (plan_is<K96>(KP) && plan_is<V96>(VP)) || (plan_is<K64>(KP) && plan_is<V64>(VP));
    if (!ok || A.n_q % A.n_kvh || A.n_q / A.n_kvh > 8) return 0;
    if (((uintptr_t)A.kpack % 4) || ((uintptr_t)A.vpack % 4) || (A.k_head_stride % 4) || (A.v_head_stride % 4))
        return 0;
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 256;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus = n;
    }
    const int tpo = (A.n_kv + 63) / 64;
    const long long cap = (long long)(part_floats / ((size_t)n_seq * A.n_q * (A.hd + 2)));
    const int G = A.n_q / A.n_kvh;
    const int per_cu = plan_is<K96>(KP) ? resident_per_cu_g<K96, V96>(G, A.out != nullptr)
                                        : resident_per_cu_g<K64, V64>(G, A.out != nullptr);
    long long r = std::min<long long>(tpo, std::max(1, (per_cu * cus) / (A.n_kvh * n_seq)));
    r = std::min<long long>(r, std::min<long long>(cap, 4096));
    // SP_HIP_ATTN_LANE_RUNS=n caps the runs per KV head (read at each call; tests use it
    // to give every run several tiles at small context lengths)
    if (const char *e = getenv("SP_HIP_ATTN_LANE_RUNS")) {
        const int n = atoi(e);
        if (n > 0) r = std::min<long long>(r, n);
    }
    return r > 0 ? (int)r : 0;
}

hipError_t sp_launch_attn_lane_split(const SpPlan &KP, const SpPlan &VP, const SpAttnArgs &A, const SpSeqTab &T,
                                     const float *qt, float *part, int n_runs, hipStream_t s) {
    if (n_runs <= 0 || T.n_seq < 1 || T.n_seq > SP_ATTN_MAX_SEQ) return hipErrorInvalidValue;
    if (plan_is<K96>(KP) && plan_is<V96>(VP))
        launch_lane_g<K96, V96>(A, T, qt, part, n_runs, KP.max_bands, VP.max_bands, s);
    else if (plan_is<K64>(KP) && plan_is<V64>(VP))
        launch_lane_g<K64, V64>(A, T, qt, part, n_runs, KP.max_bands, VP.max_bands, s);
    else return hipErrorNotSupported;
    return hipGetLastError();
}
