// sp_sqfree_attn.hip -- fused decode attention over sqfree+spinor records (the
// sqfree cache's K and V arrays) for the shipping geometry: head_dim 128 padded to
// 154, skeleton 77 or 115 (K bands 5/4/4/4/5; V 5/4/4/4/5, or one 3-bit band at
// skeleton 115), 3-bit residuals, spinor sheet on.
//
// The read path (sp_cuda_sqfree_read_one, shannon_prime_sqfree.cu:857-950) rebuilds
// the pad coefficients c~ (skeleton values from the bands; residual coefficient r as
// (sheet_r ? -pred_r : pred_r) + (level_r - centre) * step, pred = the Knight CSR over
// the dequantized skeleton) and returns V(c~)[0, hd), V the length-154 Vilenkin
// transform, which is symmetric and its own inverse. So nothing is reconstructed:
//   * with q~ = kq_scale * V(q zero-padded to 154) (once per query head),
//     q . K~_t = q~ . c~_t, a dot product in the coefficient domain;
//   * sum_t p_t V~_t = V(sum_t p_t c~_t)[0, hd): the weighted coefficient sums are
//     finished by one transform per query head.
//
// Three launches per layer: the hier attention's query preparation and merge
// kernels (sp_hier_attn.hip) with no predictor (W = 0: skeleton slots = the Knight
// skeleton, target slots = the residual coefficients), and the split kernel below:
// block (KV head, run) is one wave walking the run's 64-position tiles, lane =
// position, the record decoded into the lane's registers exactly as the read path
// decodes it (compile-time Knight CSR and record fields), the scores as dot products
// with the prepared queries, an online softmax across the run's tiles, and the
// weighted coefficient sums through LDS (the wave's coefficients transposed so that
// each lane sums one coefficient over the tile's 64 positions).
#include <cstdlib>

#include "sp_sqfree_lane.h"

namespace {

constexpr int PAD = 154;
constexpr int RBITS = 3;

// The record's pad coefficients in [skeleton slot s | residual r] order: the same
// arithmetic, in the same order, as k_sqfree_decode_lane before its transform.
template <int SK, class SL, int DW>
__device__ __forceinline__ void sq_coefficients(const uint32_t (&rec)[DW], float (&e)[PAD]) {
    using G = SqRec<PAD, SK, RBITS, true, SL>;
    constexpr int NR = PAD - SK;
    float sk[SK];
    dequant_bands<SL, false, true>(rec, SL::nb, sk);
#pragma unroll
    for (int s = 0; s < SK; s++) e[s] = sk[s];
    const float mag = __uint_as_float(rec_get32(rec, G::mag_byte));
    constexpr int L = 1 << RBITS;
    const float center = 0.5f * (float)(L - 1);
    const float sat = mag * (float)RBITS;
    const float step = sp_div(2.0f * sat, (float)(L - 1));
#pragma unroll
    for (int r = 0; r < NR; r++) {
        float p = csr_predict<PAD, SK>(sk, r);
        if (rec_extract(rec, G::sheet_bit + r, 1)) p = -p;
        const float d = ((float)rec_extract(rec, G::res_bit + r * RBITS, RBITS) - center) * step;
        e[SK + r] = p + d;
    }
}

// wave reductions on DPP and the row swaps (every lane active at each call)
__device__ __forceinline__ float wave_max(float v) { return sp_wave_max_dpp(v); }
__device__ __forceinline__ float wave_add(float v) { return sp_wave_sum_dpp(v); }

// The score factors of one query head in chunks of at most 16: the skeleton part
// (SK factors) then the residual part (PAD - SK), a chunk never spanning both.
template <int SK, int PAD>
struct QChunks {
    static constexpr int NS = (SK + 15) / 16, NR = (PAD - SK + 15) / 16, N = NS + NR;
    // coefficient index of chunk k's first factor, and the chunk's factor count
    static constexpr int first(int k) { return k < NS ? 16 * k : SK + 16 * (k - NS); }
    static constexpr int size(int k) {
        return k < NS ? (SK - 16 * k < 16 ? SK - 16 * k : 16) : (PAD - SK - 16 * (k - NS) < 16 ? PAD - SK - 16 * (k - NS) : 16);
    }
};

constexpr int EP = 65;  // LDS row pitch (floats) of the transposed coefficient chunk

// Scores, online softmax and the V records' weighted coefficient sums. Block
// (kvh, run) takes tiles run, run + n_runs, ... of KV head kvh (64 positions each).
// prep: the G query heads of KV head kvh at prep + (kvh * G + h) * ps:
// [q~ at the skeleton slots (r4(SK)) | q~ at the residual coefficients | ...], qo the
// residual part's offset. Partial per (query head, run) at part + ((h0 + h) * n_runs
// + run) * pp: [m, l, 0, 0, sum p c~ (PAD coefficients, skeleton then residuals)].
// OUT = false: scores only.
template <int SK, class SLK, class SLV, int GM, bool OUT>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))
k_sqfree_attn_split(const unsigned char *__restrict__ kc0, const unsigned char *__restrict__ vc0, long long k_slot,
                    long long v_slot, const SpSeqTab T, int G, int hs, const float *__restrict__ prep0, int ps, int qo,
                    float *__restrict__ scores0, float *__restrict__ part0, int pp, int n_runs) {
    using GK = SqRec<PAD, SK, RBITS, true, SLK>;
    using GV = SqRec<PAD, SK, RBITS, true, SLV>;
    constexpr int NCK = RecTile<GK>::NCK > RecTile<GV>::NCK ? RecTile<GK>::NCK : RecTile<GV>::NCK;
    constexpr int C2 = PAD - 128;  // coefficients of the third 64-coefficient chunk
    constexpr int HG = (GM + 1) / 2;  // heads per lane in the third chunk (two lanes per coefficient)
    static_assert(C2 > 0 && 2 * C2 <= 64, "three chunks of at most 64 coefficients");
    // the record stage and the transposed coefficient chunks share their memory: in
    // this one-wave block the stage's last reads (the V records) come before the first
    // chunk's writes, and the next tile's K records are staged after the last chunk's
    // barrier; the smaller block fits 8 per CU (two waves per SIMD) instead of 6
    __shared__ __attribute__((aligned(16))) float E[OUT ? 64 * EP : (NCK * 1024 + 16 + 3) / 4];
    static_assert(NCK * 1024 + 16 <= 64 * EP * 4, "the record stage fits the chunk memory");
    unsigned char *const stage = reinterpret_cast<unsigned char *>(E);
    __shared__ __attribute__((aligned(16))) float Pw[64 * GM];
    // block x: head group x (query heads x G .. x G + G - 1) of KV head x / hs
    const int hb = blockIdx.x, kvh = hb / hs, run = blockIdx.y, lane = threadIdx.x;
    // sequence blockIdx.z: its positions, prepared queries, score rows and partials
    const int seq = blockIdx.z, n_q = (int)gridDim.x * G, n_kv = T.len[seq];
    const unsigned char *__restrict__ kc = kc0 + (long long)T.start[seq] * GK::total;
    const unsigned char *__restrict__ vc = vc0 + (long long)T.start[seq] * GV::total;
    const long long s_stride = T.len[seq];
    float *__restrict__ scores = scores0 ? scores0 + T.soff[seq] : nullptr;
    const float *__restrict__ prep = prep0 + (long long)seq * n_q * ps;
    float *__restrict__ part = part0 + (long long)seq * n_q * n_runs * pp;
    const int h0 = hb * G;
    const int tpo = (n_kv + 63) / 64;
    const int n_tiles = ((int)gridDim.x / hs) * tpo;
    const TileMap M{tpo, n_kv};
    const float *__restrict__ pq = prep + (long long)h0 * ps;

    float m_run[GM], l_run[GM];
    float acc0[GM], acc1[GM], acc2[HG];
#pragma unroll
    for (int h = 0; h < GM; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
        acc0[h] = acc1[h] = 0.0f;
    }
#pragma unroll
    for (int h = 0; h < HG; h++) acc2[h] = 0.0f;
    // third chunk: coefficient 128 + c2i for heads hh * HG .. hh * HG + HG - 1
    const int c2i = lane % C2, hh = lane / C2;
    const bool c2_on = hh < (GM > 1 ? 2 : 1);

    // a tile's K and V records load at the tile's start (holding the next tile's K records
    // through a tile took the registers that keep the full instances from spilling at two
    // waves per SIMD; the other wave hides the load)
    for (int c = run; c < tpo; c += n_runs) {
        const int t = kvh * tpo + c;
        RecTile<GK> Rk;
        rec_tile_load<GK>(Rk, kc, k_slot, M, t, n_tiles, lane);
        RecTile<GV> Rv;
        if (OUT) rec_tile_load<GV>(Rv, vc, v_slot, M, t, n_tiles, lane);
        __syncthreads();  // the previous tile is done with the stage
        rec_tile_stage<GK>(Rk, stage, M, t, lane);
        __syncthreads();
        uint32_t rk[GK::dwords];
        rec_from_lds<GK>(rk, stage, lane);
        float e[PAD];
        sq_coefficients<SK, SLK>(rk, e);
        const int pos = c * 64 + lane;
        const bool live = pos < n_kv;
        float s[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            s[h] = -INFINITY;
            if (h < G) {
                // q~ . e: the head's factors are wave-uniform and arrive by scalar loads,
                // 16 at a time. In the full instances chunk k + 1 is loaded after the first
                // product of chunk k (a scalar-load wait covers every scalar load in flight,
                // so the next chunk cannot go out before the wait for the current one):
                // 2% faster there; the scores-only instances measured 4% slower with it and
                // keep the compiler's placement.
                const float *__restrict__ qh = pq + h * ps;
                using QC = QChunks<SK, PAD>;
                float qa[16], qb[16];
#pragma unroll
                for (int i = 0; i < QC::size(0); i++) qa[i] = qh[i];
                float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                for (int k = 0; k < QC::N; k++) {
                    float(&q)[16] = (k & 1) ? qb : qa;
                    float(&qn)[16] = (k & 1) ? qa : qb;
                    const int e0 = QC::first(k);
                    a0 = fmaf(q[0], e[e0], a0);
                    if (k + 1 < QC::N) {
                        const float *__restrict__ qs = qh + (k + 1 < QC::NS ? 16 * (k + 1) : qo + 16 * (k + 1 - QC::NS));
                        if constexpr (OUT) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int i = 0; i < QC::size(k + 1); i++) qn[i] = qs[i];
                        if constexpr (OUT) __builtin_amdgcn_sched_barrier(0);
                    }
#pragma unroll
                    for (int i = 1; i < QC::size(k); i++) {
                        if (i & 1) a1 = fmaf(q[i], e[e0 + i], a1);
                        else a0 = fmaf(q[i], e[e0 + i], a0);
                    }
                }
                const float v = a0 + a1;
                if (live) {
                    s[h] = v;
                    if (scores) scores[(long long)(h0 + h) * s_stride + pos] = v;
                }
            }
        }
        if (!OUT) continue;
        // ---- online softmax over the tile (wave-wide per head) ----
        float alpha[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            alpha[h] = 1.0f;
            if (h < G) {
                const float mn = fmaxf(m_run[h], wave_max(s[h]));
                alpha[h] = __expf(m_run[h] - mn);
                const float pr = live ? __expf(s[h] - mn) : 0.0f;
                l_run[h] = fmaf(l_run[h], alpha[h], wave_add(pr));
                m_run[h] = mn;
                Pw[lane * GM + h] = pr;
            } else {
                Pw[lane * GM + h] = 0.0f;
            }
        }
        // ---- V records of the tile, then their coefficients ----
        __syncthreads();  // every lane has read its K record from the stage
        rec_tile_stage<GV>(Rv, stage, M, t, lane);
        __syncthreads();
        uint32_t rv[GV::dwords];
        rec_from_lds<GV>(rv, stage, lane);
        float ev[PAD];
        sq_coefficients<SK, SLV>(rv, ev);
#pragma unroll
        for (int h = 0; h < GM; h++) {
            acc0[h] *= alpha[h];
            acc1[h] *= alpha[h];
        }
#pragma unroll
        for (int k = 0; k < HG; k++) {
            float a = 1.0f;
#pragma unroll
            for (int h = 0; h < GM; h++)
                if (h == hh * HG + k) a = alpha[h];
            acc2[k] *= a;
        }
        // ---- weighted coefficient sums: chunk of 64 coefficients transposed through
        // LDS (row = coefficient, column = position), lane = coefficient ----
#pragma unroll
        for (int ch = 0; ch < 3; ch++) {
            const int i0 = 64 * ch, n_i = ch < 2 ? 64 : C2;
#pragma unroll
            for (int i = 0; i < 64; i++)
                if (i < n_i) E[i * EP + lane] = ev[i0 + i];
            __syncthreads();
            if (ch == 0) {
#pragma unroll 4
                for (int p = 0; p < 64; p++) {
                    const float ei = E[lane * EP + p];
#pragma unroll
                    for (int h = 0; h < GM; h++) acc0[h] = fmaf(Pw[p * GM + h], ei, acc0[h]);
                }
            } else if (ch == 1) {
#pragma unroll 4
                for (int p = 0; p < 64; p++) {
                    const float ei = E[lane * EP + p];
#pragma unroll
                    for (int h = 0; h < GM; h++) acc1[h] = fmaf(Pw[p * GM + h], ei, acc1[h]);
                }
            } else if (c2_on) {
                // hh * HG + k < GM for every lane with c2_on (two halves of HG heads)
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
    // ---- the run's partial per query head ----
#pragma unroll
    for (int h = 0; h < GM; h++) {
        if (h >= G) continue;
        float *dst = part + ((long long)(h0 + h) * n_runs + run) * pp;
        if (lane == 0) {
            dst[0] = m_run[h];
            dst[1] = l_run[h];
            dst[2] = 0.0f;
            dst[3] = 0.0f;
        }
        dst[4 + lane] = acc0[h];
        dst[4 + 64 + lane] = acc1[h];
    }
    if (c2_on) {
#pragma unroll
        for (int k = 0; k < HG; k++) {
            const int h = hh * HG + k;
            if (h < G) part[((long long)(h0 + h) * n_runs + run) * pp + 4 + 128 + c2i] = acc2[k];
        }
    }
}

using SkelL77 = Layout<77, 5, 4, 4, 4, 5>;
using SkelL115 = Layout<115, 5, 4, 4, 4, 5>;
using SkelL115V3 = Layout<115, 3>;

// hs head groups per KV head (1 or 2): block x takes the query heads of group x.
template <int SK, class SLK, class SLV, int GM>
void launch_split(const SpSqAttnArgs &A, const SpSeqTab &T, const float *prep, float *part, int n_runs, int hs,
                  hipStream_t s) {
    const dim3 grid(A.n_kvh * hs, n_runs, T.n_seq), block(64);
    const int G = A.n_q / A.n_kvh / hs;
    if (A.out)
        hipLaunchKernelGGL((k_sqfree_attn_split<SK, SLK, SLV, GM, true>), grid, block, 0, s, A.kcache, A.vcache,
                           A.k_slot_bytes, A.v_slot_bytes, T, G, hs, prep, A.ps, A.qo, A.scores, part, A.pp, n_runs);
    else
        hipLaunchKernelGGL((k_sqfree_attn_split<SK, SLK, SLV, GM, false>), grid, block, 0, s, A.kcache, A.vcache,
                           A.k_slot_bytes, A.v_slot_bytes, T, G, hs, prep, A.ps, A.qo, A.scores, part, A.pp, n_runs);
}

template <int SK, class SLK, class SLV>
void launch_split_g(const SpSqAttnArgs &A, const SpSeqTab &T, const float *prep, float *part, int n_runs, int hs,
                    hipStream_t s) {
    const int G = A.n_q / A.n_kvh / hs;
    if (G <= 1) launch_split<SK, SLK, SLV, 1>(A, T, prep, part, n_runs, hs, s);
    else if (G <= 2) launch_split<SK, SLK, SLV, 2>(A, T, prep, part, n_runs, hs, s);
    else if (G <= 4) launch_split<SK, SLK, SLV, 4>(A, T, prep, part, n_runs, hs, s);
    else launch_split<SK, SLK, SLV, 8>(A, T, prep, part, n_runs, hs, s);
}

template <class SL>
bool bands_are(const SpPlan &P) {
    if (P.n_bands != SL::nb || P.total_bytes != SL::total) return false;
    for (int b = 0; b < SL::nb; b++)
        if (P.band_bits[b] != SL::bits[b] || P.band_off[b] != SL::off(b) || P.band_sz[b] != SL::sz(b)) return false;
    return true;
}

}  // namespace

// Which split kernel serves this cache geometry (0: none).
int sp_sqfree_attn_kind(const SpPlan &KP, const SpPlan &VP, const SpSqGeo &G) {
    if (!G.default_tables || G.hd != 128 || G.pad != PAD || G.rbits != RBITS || !G.spinor) return 0;
    if (G.sk_k == 77 && bands_are<SkelL77>(KP) && bands_are<SkelL77>(VP)) return 1;
    if (G.sk_k == 115 && bands_are<SkelL115>(KP) && bands_are<SkelL115>(VP)) return 2;
    if (G.sk_k == 115 && bands_are<SkelL115>(KP) && bands_are<SkelL115V3>(VP)) return 3;
    return 0;
}

namespace {
// One-wave blocks of the split kernel instance for this call that are resident on a CU
// at once (its registers and LDS decide; 4 when the runtime cannot say).
template <int SK, class SLK, class SLV, int GM>
int resident_per_cu(bool out) {
    int nb = 0;
    const hipError_t e =
        out ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_sqfree_attn_split<SK, SLK, SLV, GM, true>, 64, 0)
            : hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_sqfree_attn_split<SK, SLK, SLV, GM, false>, 64, 0);
    return e == hipSuccess && nb > 0 ? nb : 4;
}
// compute units of the current device (256 when the runtime cannot say)
int device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
        n = 256;
    return n;
}

template <int SK, class SLK, class SLV>
int resident_per_cu_g(int G, bool out) {
    if (G <= 1) return resident_per_cu<SK, SLK, SLV, 1>(out);
    if (G <= 2) return resident_per_cu<SK, SLK, SLV, 2>(out);
    if (G <= 4) return resident_per_cu<SK, SLK, SLV, 4>(out);
    return resident_per_cu<SK, SLK, SLV, 8>(out);
}
}  // namespace

// Runs per KV head and sequence: the blocks that are resident at once (the split
// kernel instance's occupancy) spread over the sequences' KV heads, so the launch runs
// in one round, every run getting at least one tile.
int sp_sqfree_attn_runs(const SpPlan &KP, const SpPlan &VP, const SpSqGeo &G, int n_q, int n_kvh, int n_kv, int cus,
                        int n_seq, bool out) {
    const int kind = sp_sqfree_attn_kind(KP, VP, G);
    if (!kind || n_kvh <= 0 || n_q % n_kvh) return 1;
    const int g = n_q / n_kvh;
    const int per_cu = kind == 1   ? resident_per_cu_g<77, SkelL77, SkelL77>(g, out)
                       : kind == 2 ? resident_per_cu_g<115, SkelL115, SkelL115>(g, out)
                                   : resident_per_cu_g<115, SkelL115, SkelL115V3>(g, out);
    const int tpo = (n_kv + 63) / 64;
    const int per_head = std::max(1, (per_cu * cus) / std::max(1, n_kvh * n_seq));
    return std::max(1, std::min(std::min(tpo, per_head), 1024));
}

hipError_t sp_launch_sqfree_attn(const SpPlan &KP, const SpPlan &VP, const SpSqGeo &G, const SpHierAttnArgs &HA,
                                 const SpSqAttnArgs &A, const SpSeqTab &T, float *ws, size_t ws_floats, int n_runs,
                                 hipStream_t s) {
    const int kind = sp_sqfree_attn_kind(KP, VP, G);
    if (!kind || A.n_kv <= 0 || A.n_q <= 0 || A.n_kvh <= 0 || A.n_q % A.n_kvh || A.n_q / A.n_kvh > 8 ||
        n_runs <= 0 || n_runs > 1024 || A.pp < 4 + PAD || A.ps != HA.ps || A.pp != HA.pp || T.n_seq < 1 ||
        T.n_seq > SP_ATTN_MAX_SEQ)
        return hipErrorInvalidValue;
    if (sp_hier_attn_workspace_floats(HA, n_runs, T.n_seq) > ws_floats) return hipErrorInvalidValue;
    float *prep = ws;
    float *part = ws + (size_t)T.n_seq * A.n_q * A.ps;
    hipError_t e = sp_launch_hier_attn_prep(KP, HA, T.n_seq, prep, s);
    if (e != hipSuccess) return e;
    // Two head groups per KV head when twice the blocks still run in one resident round
    // (a single sequence leaves half the wave slots empty otherwise): each tile's records
    // are then decoded twice, for half the heads each.
    int hs = 1;
    const int gq = A.n_q / A.n_kvh;
    if (gq % 2 == 0) {
        const bool out = A.out != nullptr;
        const int per_cu = kind == 1   ? resident_per_cu_g<77, SkelL77, SkelL77>(gq / 2, out)
                           : kind == 2 ? resident_per_cu_g<115, SkelL115, SkelL115>(gq / 2, out)
                                       : resident_per_cu_g<115, SkelL115, SkelL115V3>(gq / 2, out);
        if (2LL * A.n_kvh * n_runs * T.n_seq <= (long long)per_cu * device_cus()) hs = 2;
        // SP_HIP_SQFREE_ATTN_GROUPS=1 (read at each call) keeps one group (tests cover both)
        const char *eg = getenv("SP_HIP_SQFREE_ATTN_GROUPS");
        if (eg && eg[0] == '1') hs = 1;
    }
    if (kind == 1) launch_split_g<77, SkelL77, SkelL77>(A, T, prep, part, n_runs, hs, s);
    else if (kind == 2) launch_split_g<115, SkelL115, SkelL115>(A, T, prep, part, n_runs, hs, s);
    else launch_split_g<115, SkelL115, SkelL115V3>(A, T, prep, part, n_runs, hs, s);
    e = hipGetLastError();
    if (e != hipSuccess || !A.out) return e;
    return sp_launch_hier_attn_merge(KP, HA, T.n_seq, part, n_runs, s);
}
