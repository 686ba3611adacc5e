// sp_hier_attn_lane.hip -- the split kernel of the fused decode attention over hier
// records, one position per lane, for the default geometry at head_dim 256 (pad
// 330, skeleton = 30 coefficients in two 5-bit bands, 300 targets at 2 bits;
// configs[4]).
//
// Same algebra and partial layout as k_hier_attn_split (sp_hier_attn.hip), between
// the same query preparation and merge kernels: with u = q~_skel + W^T q~_tgt and
// dev_t = (level_t - centre) * step_t,
//     q . K~_t = u . skel_t + step_t * (q~_tgt . level_t - centre * sum q~_tgt),
// and a run's partial per query head is [m, l, 0, 0, sum p skel (30), sum p dev (300)].
// Here a block is one wave walking its run of 64-position tiles: the K records of
// the next tile are in flight in registers while the current one computes (no
// block-wide chunk copies or barriers), lane = position for the scores (its record
// decoded at compile-time bit positions, the prepared queries through scalar
// loads) and an online softmax across the run's tiles; the V sums read the tile's
// records staged in LDS, each lane owning 32-bit windows of 16 target levels (or a
// skeleton coefficient) for a pair of query heads over a group of positions.
#include "sp_lane.h"

namespace {

constexpr int NS = 30, NT = 300, RB = 2, PADH = 330;
using SkelL = Layout<30, 5, 5>;
using HR = HierRec<NT, RB, SkelL>;  // 103 bytes
constexpr int NWIN = (NT * RB + 31) / 32;  // 19 windows of 16 levels (the last one 12)
constexpr int LPW = 32 / RB;
static_assert(HR::total == 103, "configs[4] hier record");

constexpr int PQ = 32 + 320 + 4;  // floats per prepared query

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

// 4 little-endian bytes at LDS byte offset o (any alignment) of a dword-aligned array.
__device__ __forceinline__ uint32_t lds_word(const unsigned char *base, int o) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(base + (o & ~3));
    return __builtin_amdgcn_alignbit(w[1], w[0], 8u * (uint32_t)(o & 3));
}

// prep: per query head [u (32) | q~_tgt (r32(300) = 320) | sum q~_tgt, 0, 0, 0] (ps floats);
// part: per (query head, run) [m, l, 0, 0, c_skel (30), dev (300)] (pp floats).
template <int GM, bool OUT>
__global__ void __launch_bounds__(64)
k_hier_attn_lane(const unsigned char *__restrict__ kc0, const unsigned char *__restrict__ vc0, long long slot_bytes,
                 const SpSeqTab T, int G, const float *__restrict__ prep0, int ps, float *__restrict__ scores0,
                 float *__restrict__ part0, int pp, int n_runs) {
    constexpr int NCK = RecTile<HR>::NCK;
    constexpr int NHP = (GM + 1) / 2;                         // head pairs
    constexpr int IT = NWIN * NHP, IS = NS * NHP;             // target-window and skeleton items
    constexpr int NGT = IT < 64 ? 64 / IT : 1, NGS = IS < 64 ? 64 / IS : 1;  // position groups
    constexpr int RT = (IT + 63) / 64, RS = (IS + 63) / 64;   // item rounds per lane
    constexpr int QO = 32, SO = 32 + 320;                     // prepared-query offsets
    constexpr int SB = NCK * 1024 + 16;                       // stage bytes (K, then V records)
    constexpr int RED = 4 * (NGT * GM * NWIN * LPW + NGS * GM * NS);
    __shared__ __attribute__((aligned(16))) unsigned char stage[SB > RED ? SB : RED];
    __shared__ __attribute__((aligned(16))) float pw[64 * GM];       // p * step (V targets)
    __shared__ __attribute__((aligned(16))) float psb[2 * 64 * GM];  // p * scale_b (V skeleton bands)
    __shared__ __attribute__((aligned(16))) float qs[GM * PQ];        // the G prepared queries
    const int kvh = blockIdx.x, run = blockIdx.y, lane = threadIdx.x;
    // sequence blockIdx.z: its positions, prepared queries, score rows and partials
    const int seq = blockIdx.z, n_q = (int)gridDim.x * G, n_kv = T.len[seq];
    const unsigned char *__restrict__ kc = kc0 + (long long)T.start[seq] * HR::total;
    const unsigned char *__restrict__ vc = vc0 + (long long)T.start[seq] * HR::total;
    const long long s_stride = T.len[seq];
    float *__restrict__ scores = scores0 ? scores0 + T.soff[seq] : nullptr;
    const float *__restrict__ prep = prep0 + (long long)seq * n_q * ps;
    float *__restrict__ part = part0 + (long long)seq * n_q * n_runs * pp;
    const int h0 = kvh * G;
    const int tpo = (n_kv + 63) / 64;
    const int n_tiles = (int)gridDim.x * tpo;
    const TileMap M{tpo, n_kv};
    constexpr float centre = 1.5f;  // (L - 1) / 2 at 2 bits
    // the G prepared queries into LDS (heads past G repeat head G - 1: their results
    // are discarded); the score loops read them as broadcast 16-byte loads
    for (int i = lane; i < GM * PQ; i += 64) {
        const int h = i / PQ;
        qs[i] = prep[(long long)(h0 + (h < G ? h : G - 1)) * ps + (i - h * PQ)];
    }
    __syncthreads();
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 *qs4 = reinterpret_cast<const f4 *>(qs);

    float m_run[GM], l_run[GM];
#pragma unroll
    for (int h = 0; h < GM; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
    }
    // V sums: target window items (window, head pair) and skeleton items (coefficient, head pair)
    float tacc[RT][LPW][2], tws[RT][2], sacc[RS][2];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        tws[r][0] = tws[r][1] = 0.0f;
#pragma unroll
        for (int k = 0; k < LPW; k++) tacc[r][k][0] = tacc[r][k][1] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < RS; r++) sacc[r][0] = sacc[r][1] = 0.0f;
    const int tg = NGT > 1 ? lane / IT : 0, sg = NGS > 1 ? lane / IS : 0;  // position groups

    RecTile<HR> Rk;
    int c = run;
    if (c < tpo) rec_tile_load<HR>(Rk, kc, slot_bytes, M, kvh * tpo + c, n_tiles, lane);
    for (; c < tpo; c += n_runs) {
        const int t = kvh * tpo + c;
        RecTile<HR> Rv;
        if (OUT) rec_tile_load<HR>(Rv, vc, slot_bytes, M, t, n_tiles, lane);
        __syncthreads();  // the previous tile is done with the stage
        rec_tile_stage<HR>(Rk, stage, M, t, lane);
        __syncthreads();
        uint32_t rk[HR::dwords];
        rec_from_lds<HR>(rk, stage, lane);
        if (c + n_runs < tpo) rec_tile_load<HR>(Rk, kc, slot_bytes, M, t + n_runs, n_tiles, lane);
        // ---- scores: lane = position ----
        float sk[NS];
        dequant_bands<SkelL, false, true>(rk, SkelL::nb, sk);
        const float step = sp_div(2.0f * __uint_as_float(rec_get32(rk, HR::mag_byte)), 3.0f);
        float a[GM], d[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) a[h] = d[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < NS; j += 4) {
#pragma unroll
            for (int h = 0; h < GM; h++) {
                const f4 u = qs4[(h * PQ + j) / 4];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (j + e < NS) a[h] = fmaf(u[e], sk[j + e], a[h]);
            }
        }
        // target levels: the K record staged in LDS, 32-bit windows of 16 levels (the
        // last window's 4 levels past the 300th meet zero-padded queries)
        const int lbase = lane * HR::total + HR::res_bit / 8;
#pragma unroll 1
        for (int w = 0; w < NWIN; w++) {
            const uint32_t win = lds_word(stage, lbase + 4 * w);
#pragma unroll
            for (int q = 0; q < LPW / 4; q++) {
                float lv[4];
#pragma unroll
                for (int e = 0; e < 4; e++) lv[e] = (float)((win >> (RB * (4 * q + e))) & 3u);
#pragma unroll
                for (int h = 0; h < GM; h++) {
                    const f4 qv = qs4[(h * PQ + QO) / 4 + 4 * w + q];
#pragma unroll
                    for (int e = 0; e < 4; e++) d[h] = fmaf(qv[e], lv[e], d[h]);
                }
            }
        }
        const int pos = c * 64 + lane;
        const bool live = pos < n_kv;
        float s[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            s[h] = -INFINITY;
            if (h < G) {
                const float v = fmaf(step, d[h] - centre * qs[h * PQ + SO], a[h]);
                if (live) {
                    s[h] = v;
                    if (scores) scores[(long long)(h0 + h) * s_stride + pos] = v;
                }
            }
        }
        if (!OUT) continue;
        // ---- online softmax over the tile ----
        float alpha[GM], pr[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            alpha[h] = 1.0f;
            pr[h] = 0.0f;
            if (h < G) {
                const float mn = fmaxf(m_run[h], wmax(s[h]));
                alpha[h] = __expf(m_run[h] - mn);
                pr[h] = live ? __expf(s[h] - mn) : 0.0f;
                l_run[h] = fmaf(l_run[h], alpha[h], wadd(pr[h]));
                m_run[h] = mn;
            }
        }
        // ---- V records of the tile; per position p * step and p * scale_b ----
        __syncthreads();  // every lane has read its K record from the stage
        rec_tile_stage<HR>(Rv, stage, M, t, lane);
        __syncthreads();
        {
            const int rb = lane * HR::total;
            const float vstep = sp_div(2.0f * __uint_as_float(lds_word(stage, rb + HR::mag_byte)), 3.0f);
            const float sc0 = sp_scale_from_bits(lds_word(stage, rb + SkelL::byte_off(0)) & 0xffffu);
            const float sc1 = sp_scale_from_bits(lds_word(stage, rb + SkelL::byte_off(1)) & 0xffffu);
#pragma unroll
            for (int h = 0; h < GM; h++) {
                pw[lane * GM + h] = pr[h] * vstep;
                psb[lane * GM + h] = pr[h] * sc0;
                psb[(64 + lane) * GM + h] = pr[h] * sc1;
            }
        }
        __syncthreads();
        // rescale the running sums of each item's two heads
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const int it = NGT > 1 ? lane % IT : lane + 64 * r;
            const int hp = it / NWIN;
            float fa = 1.0f, fb = 1.0f;
#pragma unroll
            for (int h = 0; h < GM; h++) {
                if (h == 2 * hp) fa = alpha[h];
                if (h == 2 * hp + 1) fb = alpha[h];
            }
            tws[r][0] *= fa;
            tws[r][1] *= fb;
#pragma unroll
            for (int k = 0; k < LPW; k++) {
                tacc[r][k][0] *= fa;
                tacc[r][k][1] *= fb;
            }
        }
#pragma unroll
        for (int r = 0; r < RS; r++) {
            const int it = NGS > 1 ? lane % IS : lane + 64 * r;
            const int hp = it / NS;
            float fa = 1.0f, fb = 1.0f;
#pragma unroll
            for (int h = 0; h < GM; h++) {
                if (h == 2 * hp) fa = alpha[h];
                if (h == 2 * hp + 1) fb = alpha[h];
            }
            sacc[r][0] *= fa;
            sacc[r][1] *= fb;
        }
        // ---- target windows: 16 levels of one 32-bit window for a head pair ----
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const int it = NGT > 1 ? lane % IT : lane + 64 * r;
            const bool on = NGT > 1 ? tg < NGT : it < IT;
            if (!on) continue;
            const int w = it % NWIN, hp = it / NWIN;
            const int ha = 2 * hp, hb = 2 * hp + 1 < GM ? 2 * hp + 1 : 2 * hp;
            const int wo = HR::res_bit / 8 + 4 * w;
#pragma unroll 2
            for (int p = tg; p < 64; p += NGT) {
                const uint32_t win = lds_word(stage, p * HR::total + wo);
                const float wa = pw[p * GM + ha], wb = pw[p * GM + hb];
                tws[r][0] += wa;
                tws[r][1] += wb;
#pragma unroll
                for (int k = 0; k < LPW; k++) {
                    const float lv = (float)((win >> (RB * k)) & 3u);
                    tacc[r][k][0] = fmaf(wa, lv, tacc[r][k][0]);
                    tacc[r][k][1] = fmaf(wb, lv, tacc[r][k][1]);
                }
            }
        }
        // ---- skeleton coefficients ----
#pragma unroll
        for (int r = 0; r < RS; r++) {
            const int it = NGS > 1 ? lane % IS : lane + 64 * r;
            const bool on = NGS > 1 ? sg < NGS : it < IS;
            if (!on) continue;
            const int j = it % NS, hp = it / NS;
            const int ha = 2 * hp, hb = 2 * hp + 1 < GM ? 2 * hp + 1 : 2 * hp;
            const int b = j < SkelL::sz(0) ? 0 : 1;
            const int bo = 8 * (SkelL::byte_off(b) + 2) + 5 * (j - SkelL::off(b));
            const float* wrow = psb + b * 64 * GM;
#pragma unroll 4
            for (int p = sg; p < 64; p += NGS) {
                const uint32_t wd = lds_word(stage, p * HR::total + (bo >> 3));
                const float cv = (float)((wd >> (bo & 7)) & 31u) - 15.0f;
                sacc[r][0] = fmaf(wrow[p * GM + ha], cv, sacc[r][0]);
                sacc[r][1] = fmaf(wrow[p * GM + hb], cv, sacc[r][1]);
            }
        }
    }
    if (!OUT) return;
    // ---- the run's partial per query head: groups summed through LDS ----
    float *Tr = reinterpret_cast<float *>(stage);  // [NGT][GM][NWIN * LPW]
    float *Sr = Tr + NGT * GM * NWIN * LPW;        // [NGS][GM][NS]
    __syncthreads();  // the last tile is done with the stage
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const int it = NGT > 1 ? lane % IT : lane + 64 * r;
        const bool on = NGT > 1 ? tg < NGT : it < IT;
        if (!on) continue;
        const int w = it % NWIN, hp = it / NWIN;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int h = 2 * hp + q;
            if (h >= GM) continue;
#pragma unroll
            for (int k = 0; k < LPW; k++)
                Tr[(tg * GM + h) * (NWIN * LPW) + w * LPW + k] = fmaf(-centre, tws[r][q], tacc[r][k][q]);
        }
    }
#pragma unroll
    for (int r = 0; r < RS; r++) {
        const int it = NGS > 1 ? lane % IS : lane + 64 * r;
        const bool on = NGS > 1 ? sg < NGS : it < IS;
        if (!on) continue;
        const int j = it % NS, hp = it / NS;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int h = 2 * hp + q;
            if (h < GM) Sr[(sg * GM + h) * NS + j] = sacc[r][q];
        }
    }
    __syncthreads();
    for (int h = 0; h < G; h++) {
        float *dst = part + ((long long)(h0 + h) * n_runs + run) * pp;
        if (lane == 0) {
            dst[0] = m_run[h];
            dst[1] = l_run[h];
            dst[2] = 0.0f;
            dst[3] = 0.0f;
        }
        for (int j = lane; j < NS + NT; j += 64) {
            float v = 0.0f;
            if (j < NS) {
#pragma unroll
                for (int g = 0; g < NGS; g++) v += Sr[(g * GM + h) * NS + j];
            } else {
#pragma unroll
                for (int g = 0; g < NGT; g++) v += Tr[(g * GM + h) * (NWIN * LPW) + (j - NS)];
            }
            dst[4 + j] = v;
        }
    }
}

template <int GM>
void launch_g(const SpHierAttnArgs &A, const SpSeqTab &T, const float *prep, float *part, int n_runs, hipStream_t s) {
    const dim3 grid(A.n_kvh, n_runs, T.n_seq), block(64);
    const int G = A.n_q / A.n_kvh;
    if (A.out)
        hipLaunchKernelGGL((k_hier_attn_lane<GM, true>), grid, block, 0, s, A.kcache, A.vcache, A.slot_bytes, T, G,
                           prep, A.ps, A.scores, part, A.pp, n_runs);
    else
        hipLaunchKernelGGL((k_hier_attn_lane<GM, false>), grid, block, 0, s, A.kcache, A.vcache, A.slot_bytes, T, G,
                           prep, A.ps, A.scores, part, A.pp, n_runs);
}

}  // namespace

// The lane split serves head_dim 256 at pad 330 with 30 skeleton coefficients in two
// 5-bit bands and 300 targets at 2 bits (any skeleton/target index tables: only the
// prep and merge read them), at most 8 query heads per KV head.
bool sp_hier_attn_lane_ok(const SpPlan &P, const SpHierAttnArgs &A) {
    if (A.hd != 256 || A.pad != PADH || A.n_skel != NS || A.n_target != NT || A.rbits != RB ||
        A.B != HR::total || A.n_q % A.n_kvh || A.n_q / A.n_kvh > 8)
        return false;
    if (P.n_bands != SkelL::nb || P.total_bytes != SkelL::total) return false;
    for (int b = 0; b < SkelL::nb; b++)
        if (P.band_bits[b] != SkelL::bits[b] || P.band_off[b] != SkelL::off(b) || P.band_sz[b] != SkelL::sz(b))
            return false;
    return A.ps == 32 + 320 + 4 && A.pp >= 4 + NS + NT;
}

// Runs per KV head: at least one tile per run, about six resident one-wave blocks
// per CU spread over the KV heads, at most the merge's limit.
int sp_hier_attn_lane_runs(const SpHierAttnArgs &A, int cus, int n_seq) {
    const int tpo = (A.n_kv + 63) / 64;
    const int per_head = std::max(1, (6 * cus) / std::max(1, A.n_kvh * n_seq));
    return std::max(1, std::min(std::min(tpo, per_head), 1024));
}

hipError_t sp_launch_hier_attn_lane(const SpPlan &P, const SpHierAttnArgs &A, const SpSeqTab &T, float *ws,
                                    size_t ws_floats, int n_runs, hipStream_t s) {
    if (n_runs <= 0 || n_runs > 1024 || T.n_seq < 1 || T.n_seq > SP_ATTN_MAX_SEQ ||
        sp_hier_attn_workspace_floats(A, n_runs, T.n_seq) > ws_floats)
        return hipErrorInvalidValue;
    float *prep = ws;
    float *part = ws + (size_t)T.n_seq * A.n_q * A.ps;
    hipError_t e = sp_launch_hier_attn_prep(P, A, T.n_seq, prep, s);
    if (e != hipSuccess) return e;
    const int G = A.n_q / A.n_kvh;
    if (G <= 2) launch_g<2>(A, T, prep, part, n_runs, s);
    else if (G <= 4) launch_g<4>(A, T, prep, part, n_runs, s);
    else launch_g<8>(A, T, prep, part, n_runs, s);
    e = hipGetLastError();
    if (e != hipSuccess || !A.out) return e;
    return sp_launch_hier_attn_merge(P, A, T.n_seq, part, n_runs, s);
}
