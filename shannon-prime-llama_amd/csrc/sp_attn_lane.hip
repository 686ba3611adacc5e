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
// coefficient sums through an LDS transpose (each lane sums one coefficient over the
// tile's 64 positions). Partials [m, l, o~[hd]] per (query head, run), the layout
// k_attn_combine merges.
#include "sp_lane.h"

namespace {

constexpr int EP = 65;  // LDS row pitch (floats) of the transposed coefficient chunk

__device__ __forceinline__ float wmax(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ __forceinline__ float wadd(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
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
    constexpr int NCK = RecTile<LK>::NCK > RecTile<LV>::NCK ? RecTile<LK>::NCK : RecTile<LV>::NCK;
    constexpr int NFULL = HD / 64;            // full 64-coefficient chunks
    constexpr int C2 = HD - 64 * NFULL;       // coefficients of the last, partial chunk
    constexpr bool HALVES = C2 > 0 && 2 * C2 <= 64 && GM > 1;  // two lanes per coefficient there
    constexpr int HG = HALVES ? (GM + 1) / 2 : GM;
    __shared__ __attribute__((aligned(16))) unsigned char stage[NCK * 1024 + 16];
    __shared__ float E[64 * EP];
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
    float acc[NFULL > 0 ? NFULL : 1][GM], acc2[HG];
#pragma unroll
    for (int h = 0; h < GM; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
#pragma unroll
        for (int c = 0; c < (NFULL > 0 ? NFULL : 1); c++) acc[c][h] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < HG; k++) acc2[k] = 0.0f;
    const int c2i = C2 > 0 ? lane % C2 : 0, hh = C2 > 0 ? lane / C2 : 0;
    const bool c2_on = C2 > 0 && hh < (HALVES ? 2 : 1);

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
        float e[HD];
        dequant_bands<LK, false, false>(rk, kmb, e);  // record order, bands past kmb read as 0
        const int pos = c * 64 + lane;
        const bool live = pos < n_kv;
        float s[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            s[h] = -INFINITY;
            if (h < G) {
                const float *__restrict__ qh = pq + h * HD;
                float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                for (int j = 0; j < HD; j += 2) {
                    a0 = fmaf(qh[j], e[j], a0);
                    a1 = fmaf(qh[j + 1], e[j + 1], a1);
                }
                const float v = a0 + a1;
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
        float ev[HD];
        dequant_bands<LV, false, false>(rv, vmb, ev);
#pragma unroll
        for (int h = 0; h < GM; h++)
#pragma unroll
            for (int cc = 0; cc < (NFULL > 0 ? NFULL : 1); cc++) acc[cc][h] *= alpha[h];
#pragma unroll
        for (int k = 0; k < HG; k++) {
            float a = 1.0f;
#pragma unroll
            for (int h = 0; h < GM; h++)
                if (h == hh * HG + k) a = alpha[h];
            acc2[k] *= a;
        }
#pragma unroll
        for (int ch = 0; ch < NFULL + (C2 > 0 ? 1 : 0); ch++) {
            const int i0 = 64 * ch, n_i = ch < NFULL ? 64 : C2;
#pragma unroll
            for (int i = 0; i < 64; i++)
                if (i < n_i) E[i * EP + lane] = ev[i0 + i];
            __syncthreads();
            if (ch < NFULL) {
#pragma unroll 4
                for (int p = 0; p < 64; p++) {
                    const float ei = E[lane * EP + p];
#pragma unroll
                    for (int h = 0; h < GM; h++) acc[ch][h] = fmaf(Pw[p * GM + h], ei, acc[ch][h]);
                }
            } else if (c2_on) {
#pragma unroll 4
                for (int p = 0; p < 64; p++) {
                    const float ei = E[c2i * EP + p];
#pragma unroll
                    for (int k = 0; k < HG; k++) acc2[k] = fmaf(Pw[p * GM + hh * HG + k], ei, acc2[k]);
                }
            }
            __syncthreads();
        }
    }
    if (!OUT) return;
    // ---- the run's partial per query head: [m, l, o~[hd]] ----
#pragma unroll
    for (int h = 0; h < GM; h++) {
        if (h >= G) continue;
        float *dst = part + ((long long)(h0 + h) * n_runs + run) * (HD + 2);
        if (lane == 0) {
            dst[0] = m_run[h];
            dst[1] = l_run[h];
        }
#pragma unroll
        for (int cc = 0; cc < NFULL; cc++) dst[2 + 64 * cc + lane] = acc[cc][h];
    }
    if (c2_on) {
#pragma unroll
        for (int k = 0; k < HG; k++) {
            const int h = hh * HG + k;
            if (h < G) part[((long long)(h0 + h) * n_runs + run) * (HD + 2) + 2 + 64 * NFULL + c2i] = acc2[k];
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

}  // namespace

// Runs per KV head for the lane split kernel: at most the workspace's partial rows,
// at least one tile per run, and about six resident one-wave blocks per CU spread
// over the KV heads. 0 when no lane kernel serves the call's layouts.
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
    long long r = std::min<long long>(tpo, std::max(1, (6 * cus) / (A.n_kvh * n_seq)));
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
