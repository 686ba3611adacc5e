// sp_internal.h -- declarations shared by the kernel files and the host runtime.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sp_device.h"
#include "../../include/shannon_prime.h"
#include "../../include/sp_hip.h"

#define SP_DT_F32 0
#define SP_DT_F16 1

template <int DT>
__device__ __forceinline__ float sp_load1(const void *src, long long off) {
    if (DT == SP_DT_F16)
        return sp_f16_bits_to_f32(reinterpret_cast<const unsigned short *>(src)[off]);
    return reinterpret_cast<const float *>(src)[off];
}

template <int DT>
__device__ __forceinline__ void sp_store1(void *dst, long long off, float v) {
    if (DT == SP_DT_F16) {
        __asm__ volatile("" : "+v"(v));  // keep the fp32 rounding before the f16 one
        _Float16 h = (_Float16)v;
        reinterpret_cast<unsigned short *>(dst)[off] = __builtin_bit_cast(unsigned short, h);
    } else {
        reinterpret_cast<float *>(dst)[off] = v;
    }
}

// Pack n codes (< 2^bits each, bits <= 8) as one LSB-first bit stream into
// out[0, ceil(n*bits/8)). Each lane assembles whole output bytes.
__device__ __forceinline__ void sp_pack_bits_lds(const unsigned char *codes, int n, int bits,
                                                 unsigned char *out, int lane) {
    const int nb = (n * bits + 7) / 8;
    for (int kk = lane; kk < nb; kk += SP_WAVE) {
        const int bit0 = kk * 8;
        uint32_t acc = 0;
        for (int e = bit0 / bits; e < n && e * bits < bit0 + 8; e++) {
            const int sh = e * bits - bit0;
            const uint32_t u = codes[e];
            acc |= sh >= 0 ? (u << sh) : (u >> (-sh));
        }
        out[kk] = (unsigned char)(acc & 0xffu);
    }
}

// Code k of an LSB-first stream (reads one byte past the code; callers pad).
__device__ __forceinline__ uint32_t sp_unpack_bits_lds(const unsigned char *in, int k, int bits) {
    const int bit = k * bits;
    const uint32_t v = (uint32_t)in[bit >> 3] | ((uint32_t)in[(bit >> 3) + 1] << 8);
    return (v >> (bit & 7)) & ((1u << bits) - 1u);
}

// ---- LDS-staged stages used by the one-vector-per-wave kernels ----
// In-place transform of c[0, n) in LDS by the 64 lanes of one wave. Every wave
// of the block calls it with the same n, so the block barriers are uniform.
__device__ inline void sp_transform_lds(float *c, int n, const SpPlan &P, int lane) {
    if (P.skip_transform) return;
    if ((n & (n - 1)) == 0) {
        const float s2 = 0.70710678118654752440f;
        for (int len = 1; len < n; len <<= 1) {
            for (int k = lane; k < n / 2; k += SP_WAVE) {
                const int base = (k / len) * 2 * len + (k % len);
                const float u = c[base], v = c[base + len];
                if (P.norm == 1) {
                    c[base] = (u + v) * s2;
                    c[base + len] = (u - v) * s2;
                } else {
                    c[base] = u + v;
                    c[base + len] = u - v;
                }
            }
            __syncthreads();
        }
        if (P.norm != 1) {
            for (int k = lane; k < n; k += SP_WAVE) c[k] *= P.inv_sqrt_n;
            __syncthreads();
        }
        return;
    }
    int stride = 1;
    for (int f = 0; f < P.n_factors; f++) {
        const int p = P.factors[f];
        const float *C = P.cas + sp_cas_off(p);
        const float isp = P.isp[sp_prime_idx(p)];
        const int block = stride * p;
        for (int wi = lane; wi < n / p; wi += SP_WAVE) {
            const int base = (wi / stride) * block + (wi % stride);
            float gv[11], rv[11];
            for (int k = 0; k < p; k++) gv[k] = c[base + k * stride];
            for (int k = 0; k < p; k++) {
                float sum = 0.0f;
                for (int jj = 0; jj < p; jj++) sum += C[k * p + jj] * gv[jj];
                rv[k] = sum * isp;
            }
            for (int k = 0; k < p; k++) c[base + k * stride] = rv[k];
        }
        stride *= p;
        __syncthreads();
    }
}

// Quantize coefficients r[0, P.hd) (LDS) into record bytes rec (LDS);
// codes (LDS, >= P.hd bytes) is scratch. Ends with a block barrier.
__device__ inline void sp_band_quantize_lds(const float *r, unsigned char *rec, unsigned char *codes,
                                     const SpPlan &P, int lane) {
    for (int b = 0; b < P.n_bands; b++) {
        const int off = P.band_off[b], sz = P.band_sz[b], bits = P.band_bits[b];
        const int maxv = (1 << (bits - 1)) - 1;
        float m = 0.0f;
        for (int k = lane; k < sz; k += SP_WAVE) {
            float a = fabsf(r[off + k]);
            m = a > m ? a : m;
        }
        const float amax = sp_wave_max(m);
        const float scale = (amax > 0.0f) ? sp_div(amax, (float)maxv) : 0.0f;
        const uint32_t h = sp_f32_to_f16_bits(scale);
        const float ss = sp_f16_bits_to_f32(h);
        const float inv = (ss > 0.0f) ? sp_div(1.0f, ss) : 0.0f;
        for (int k = lane; k < sz; k += SP_WAVE)
            codes[off + k] = (unsigned char)(sp_q_rint_clamp(r[off + k] * inv, maxv) + maxv);
        if (lane == 0) {
            rec[P.band_byte_off[b]] = (unsigned char)(h & 0xffu);
            rec[P.band_byte_off[b] + 1] = (unsigned char)(h >> 8);
        }
    }
    __syncthreads();
    for (int b = 0; b < P.n_bands; b++)
        sp_pack_bits_lds(codes + P.band_off[b], P.band_sz[b], P.band_bits[b],
                         rec + P.band_byte_off[b] + 2, lane);
    __syncthreads();
}

// Dequantize record rec (LDS) into out[0, P.hd) (LDS). Ends with a barrier.
__device__ inline void sp_band_dequantize_lds(const unsigned char *rec, float *out, const SpPlan &P,
                                       int lane) {
    for (int b = 0; b < P.n_bands; b++) {
        const int off = P.band_off[b], sz = P.band_sz[b], bits = P.band_bits[b];
        const int maxv = (1 << (bits - 1)) - 1;
        const int bo = P.band_byte_off[b];
        const float scale = sp_scale_from_bits((uint32_t)rec[bo] | ((uint32_t)rec[bo + 1] << 8));
        const bool live = b < P.max_bands;
        for (int k = lane; k < sz; k += SP_WAVE) {
            const int u = (int)sp_unpack_bits_lds(rec + bo + 2, k, bits);
            out[off + k] = live ? (float)(u - maxv) * scale : 0.0f;
        }
    }
    __syncthreads();
}

// ---- host side ----
// Build the launch plan for band config bc with transform length n_transform.
int sp_build_plan(const sp_band_config_t *bc, int n_transform, int norm, int max_bands, SpPlan *P);

hipError_t sp_launch_ship_encode(const SpPlan &P, const int *order, const void *src, int dtype,
                                 long long so, long long si, unsigned char *dst, long long dout,
                                 int n_outer, int n_inner, hipStream_t s);
hipError_t sp_launch_ship_decode(const SpPlan &P, const int *order, const unsigned char *src,
                                 long long so, void *dst, int dtype, long long dout, long long din,
                                 int n_outer, int n_inner, hipStream_t s);
hipError_t sp_launch_ship_encode_generic(const SpPlan &P, const int *order, const void *src,
                                         int dtype, long long so, long long si, unsigned char *dst,
                                         long long dout, int n_outer, int n_inner, hipStream_t s);
hipError_t sp_launch_ship_decode_generic(const SpPlan &P, const int *order,
                                         const unsigned char *src, long long so, void *dst,
                                         int dtype, long long dout, long long din, int n_outer,
                                         int n_inner, hipStream_t s);
hipError_t sp_launch_transform(const SpPlan &P, float *data, int n_vecs, hipStream_t s);
// one-vector-per-lane kernels for the shipping layouts; hipErrorNotSupported when
// no specialization fits (nothing launched)
hipError_t sp_launch_ship_encode_lane(const SpPlan &P, bool default_order, const void *src, int dtype,
                                      long long so, long long si, unsigned char *dst, long long dout,
                                      int n_outer, int n_inner, hipStream_t s);
hipError_t sp_launch_ship_decode_lane(const SpPlan &P, bool default_order, const unsigned char *src,
                                      long long so, void *dst, int dtype, long long dout, long long din,
                                      int n_outer, int n_inner, hipStream_t s);
// in-place compress + decompress of every head's vectors at n_cells cache cells
// (element (c, h, d) at c*cs + (h*hd + d)*es of x; records at rec_base +
// h*rec_head_stride + c*B); hipErrorNotSupported when no specialization fits
hipError_t sp_launch_ship_roundtrip_lane(const SpPlan &P, bool default_order, void *x, int dtype, long long cs,
                                         long long es, const int *cells, int n_cells, int max_seq,
                                         unsigned char *rec_base, long long rec_head_stride, int n_heads,
                                         int max_bands, hipStream_t s);
// the same round trip with head_dim/8 lanes per vector and K and V in one launch
// (a null k or v skips that side; V element (c, h, d) at c*vcs + (h*hd + d)*ves, K
// at c*kcs + h*hd + d); any coefficient order; head_dim 64, 128 or 256 with band
// boundaries on multiples of 8, else hipErrorNotSupported
hipError_t sp_launch_ship_roundtrip_narrow(const SpPlan &KP, const int *korder, void *k, long long kcs,
                                           unsigned char *krec, long long krhs, const SpPlan &VP, void *v,
                                           long long vcs, long long ves, unsigned char *vrec, long long vrhs,
                                           int dtype, const int *cells, int n_cells, int max_seq, int n_heads,
                                           int max_bands, hipStream_t s);
hipError_t sp_launch_permute(float *data, const int *order, int n, int n_vecs, int inverse,
                             hipStream_t s);

// Sqfree / hier geometry handed to their kernels.
struct SpSqGeo {
    int hd, pad, sk_k, n_res, rbits, spinor, bytes;
    const int *skel_idx, *res_idx, *csr_off, *csr_slot, *csr_mu;
    int default_tables;  // the Knight tables are the squarefree-first ones (not recalibrated)
};
struct SpHierGeo {
    int hd, pad, n_skel, n_target, rbits, bytes;
    const int *skel_idx, *target_idx;
    const uint16_t *W;       // slot 0 predictor
    long long w_outer;       // elements between consecutive outer slots' W
    int default_geo;         // skeleton/targets are sp_hier_default_geometry's
};

// Sequences of one batched decode-attention call: sequence s attends positions
// [start[s], start[s] + len[s]) of the layer with its own n_q query rows (llama.cpp's
// unified cache, each sequence a range of cells); its scores are [n_q][len[s]] at
// element soff[s] = n_q * (len[0] + ... + len[s-1]). Passed by value to the split
// kernels (blockIdx.z = sequence); a single-sequence call is {1, n_kv, {0}, {n_kv}, {0}}.
#define SP_ATTN_MAX_SEQ 64
struct SpSeqTab {
    int n_seq;
    int max_len;  // the longest sequence
    int start[SP_ATTN_MAX_SEQ];
    int len[SP_ATTN_MAX_SEQ];
    long long soff[SP_ATTN_MAX_SEQ];
};

// Fused decode attention over hier records (sp_hier_attn.hip).
struct SpHierAttnArgs {
    const unsigned char *kcache, *vcache;  // records of slot (layer, KV head 0); KV head h at + h * slot_bytes
    long long slot_bytes;
    const uint16_t *W;                     // predictor of slot (layer, KV head 0); KV head h at + h * w_outer
    long long w_outer;
    const int *skel_idx, *tgt_idx;
    const float *q;                        // [n_q][hd]
    float kq_scale;
    float *scores;                         // [n_q][n_kv] or null
    float *out;                            // [n_q][hd] or null
    int n_q, n_kvh, n_kv, hd, pad, n_skel, n_target, rbits, B;
    int ps;                                // floats per query head of the prepared query
    int pp;                                // floats per (query head, run) partial
};
// Batched calls: A describes one sequence's shape (n_q query rows per sequence, n_kv the
// longest sequence); q and out hold n_seq blocks of n_q rows, scores the sequences'
// [n_q][len] blocks at T.soff, the workspace n_seq blocks of prepared queries and partials.
int sp_hier_attn_prep_floats(int n_skel, int n_target);  // the value SpHierAttnArgs::ps must hold
size_t sp_hier_attn_workspace_floats(const SpHierAttnArgs &A, int n_runs, int n_seq = 1);
int sp_hier_attn_runs(const SpHierAttnArgs &A, int cus, int n_seq = 1);
hipError_t sp_launch_hier_attn(const SpPlan &P, const SpHierAttnArgs &A, const SpSeqTab &T, float *ws,
                               size_t ws_floats, int n_runs, hipStream_t s);
// The hier attention's query preparation and merge alone (one block per query head of
// every sequence), for attention kernels whose records live in the same coefficient
// domain. A.W may be null: no predictor (u = q~_skel; merged target coefficients = the
// weighted sums).
hipError_t sp_launch_hier_attn_prep(const SpPlan &P, const SpHierAttnArgs &A, int n_seq, float *prep, hipStream_t s);
hipError_t sp_launch_hier_attn_merge(const SpPlan &P, const SpHierAttnArgs &A, int n_seq, const float *part,
                                     int n_runs, hipStream_t s);

// One-position-per-lane split kernel of the hier attention (sp_hier_attn_lane.hip) for
// hd 256 / pad 330 / skeleton 30 at 5/5 bits / 300 targets at 2 bits: whether it serves
// the call, its runs per KV head, and prep + split + merge.
bool sp_hier_attn_lane_ok(const SpPlan &P, const SpHierAttnArgs &A);
int sp_hier_attn_lane_runs(const SpHierAttnArgs &A, int cus, int n_seq = 1);
hipError_t sp_launch_hier_attn_lane(const SpPlan &P, const SpHierAttnArgs &A, const SpSeqTab &T, float *ws,
                                    size_t ws_floats, int n_runs, hipStream_t s);

// Fused decode attention over sqfree+spinor records (sp_sqfree_attn.hip): the split
// kernel's arguments (records of slot (layer, KV head 0), KV head h at + h * slot bytes).
struct SpSqAttnArgs {
    const unsigned char *kcache, *vcache;
    long long k_slot_bytes, v_slot_bytes;
    float *scores;  // [n_q][n_kv] or null
    float *out;     // [n_q][hd] or null
    int n_q, n_kvh, n_kv;
    int ps, qo, pp;  // prepared-query floats per head, its residual part's offset; partial floats
};
// 1..3: the lane specialization serving this geometry (skeleton 77 with 5/4/4/4/5 K and
// V; 115 with 5/4/4/4/5 K and V; 115 with V one 3-bit band), 0: none
int sp_sqfree_attn_kind(const SpPlan &KP, const SpPlan &VP, const SpSqGeo &G);
int sp_sqfree_attn_runs(const SpPlan &KP, const SpPlan &VP, const SpSqGeo &G, int n_q, int n_kvh, int n_kv, int cus,
                        int n_seq, bool out);
// HA: the prep/merge arguments (pad, skeleton/residual index tables as skel_idx /
// tgt_idx, W null, q, kq_scale, out); ws: prep [n_seq * n_q * ps] then partials.
hipError_t sp_launch_sqfree_attn(const SpPlan &KP, const SpPlan &VP, const SpSqGeo &G, const SpHierAttnArgs &HA,
                                 const SpSqAttnArgs &A, const SpSeqTab &T, float *ws, size_t ws_floats, int n_runs,
                                 hipStream_t s);

// one-vector-per-lane hier kernels for the default geometry at head_dim 256;
// hipErrorNotSupported (nothing launched) when no specialization fits. src2/dst2:
// an optional second side (V with K) encoded by the same launch.
hipError_t sp_launch_hier_encode_lane(const SpPlan &P, const SpHierGeo &G, const void *src, int dtype, long long so,
                                      long long si, unsigned char *dst, long long dout, int n_outer, int n_inner,
                                      hipStream_t s, const void *src2 = nullptr, unsigned char *dst2 = nullptr);
// cells (optional): listed positions, record and row at cells[i] (slack after the cache)
hipError_t sp_launch_hier_decode_lane(const SpPlan &P, const SpHierGeo &G, const unsigned char *src, long long so,
                                      void *dst, int dtype, long long dout, long long din, int n_outer, int n_inner,
                                      hipStream_t s, const int *cells = nullptr);

// one-vector-per-lane sqfree kernels for the shipping geometry; hipErrorNotSupported
// (nothing launched) when no specialization fits
hipError_t sp_launch_sqfree_encode_lane(const SpPlan &P, const SpSqGeo &G, const void *src, int dtype, long long so,
                                        long long si, unsigned char *dst, long long dout, int n_outer, int n_inner,
                                        hipStream_t s);
hipError_t sp_launch_sqfree_decode_lane(const SpPlan &P, const SpSqGeo &G, const unsigned char *src, long long so,
                                        void *dst, int dtype, long long dout, long long din, int n_outer,
                                        int n_inner, hipStream_t s);
// listed positions: record and row at cells[i] for i < n_inner (slack after the cache)
hipError_t sp_launch_sqfree_decode_lane_cells(const SpPlan &P, const SpSqGeo &G, const unsigned char *src,
                                              long long so, void *dst, int dtype, long long dout, long long din,
                                              int n_outer, int n_inner, const int *cells, hipStream_t s);
hipError_t sp_launch_sqfree_encode(const SpPlan &P, const SpSqGeo &G, const void *src, int dtype,
                                   long long so, long long si, unsigned char *dst, long long dout,
                                   int n_outer, int n_inner, hipStream_t s);
// cells (optional, device int32 [n_inner]): decode the records at positions
// cells[i] into rows cells[i] instead of positions 0..n_inner-1
hipError_t sp_launch_sqfree_decode(const SpPlan &P, const SpSqGeo &G, const unsigned char *src,
                                   long long so, void *dst, int dtype, long long dout,
                                   long long din, int n_outer, int n_inner, hipStream_t s,
                                   const int *cells = nullptr);
hipError_t sp_launch_hier_encode(const SpPlan &P, const SpHierGeo &G, const void *src, int dtype,
                                 long long so, long long si, unsigned char *dst, long long dout,
                                 int n_outer, int n_inner, hipStream_t s);
// K and V of the same slots in one lane launch when it applies; else two launches
hipError_t sp_launch_hier_encode_kv(const SpPlan &P, const SpHierGeo &G, const void *src_k, const void *src_v,
                                    int dtype, long long so, long long si, unsigned char *dst_k,
                                    unsigned char *dst_v, long long dout, int n_outer, int n_inner, hipStream_t s);
hipError_t sp_launch_hier_decode(const SpPlan &P, const SpHierGeo &G, const unsigned char *src,
                                 long long so, void *dst, int dtype, long long dout, long long din,
                                 int n_outer, int n_inner, hipStream_t s, const int *cells = nullptr);

// Disk layout v3 (sp_disk.hip): a record's segments (bands, then any residual
// tail); segment s of record (slot, pos) lives at base[s] + (slot*n_pos + pos)*len[s]
struct SpDiskSegs {
    int n;
    short off[SP_MAX_BANDS_DEV + 1];
    short len[SP_MAX_BANDS_DEV + 1];
    long long base[SP_MAX_BANDS_DEV + 1];
};
hipError_t sp_launch_disk_pack(const unsigned char *rec, long long slot_stride, int B, int n_slots, int n_pos,
                               const SpDiskSegs &S, unsigned char *out, hipStream_t s);
hipError_t sp_launch_disk_unpack(const unsigned char *in, long long slot_stride, int B, int n_slots, int n_pos,
                                 const SpDiskSegs &S, int n_load, unsigned char *rec, hipStream_t s);

// Fused decode attention (sp_attn.hip).
#define SP_CACHE_SLACK 256  // bytes allocated past the last record of a packed ship cache

struct SpAttnArgs {
    const unsigned char *kpack;  // layer base: [n_kvh][max_seq][kB]
    const unsigned char *vpack;
    long long k_head_stride, v_head_stride;  // bytes between KV heads
    int kB, vB;
    int n_kv, n_q, n_kvh, hd;
    float kq_scale;
    const float *q;     // [n_q][hd]
    float *scores;      // [n_q][n_kv] or null
    float *out;         // [n_q][hd] or null
};
hipError_t sp_launch_attn_decode(const SpPlan &KP, const SpPlan &VP, const int *order,
                                 const SpAttnArgs &A, float *workspace, size_t ws_floats,
                                 hipStream_t s);
size_t sp_attn_workspace_floats(int n_q, int hd, int max_kv);
// One-position-per-lane split kernel for the hd 96 (K 5/4/4, V 5) and hd 64 (K 5/5/4/3,
// V 3) layouts (sp_attn_lane.hip): runs per KV head that fit part_floats (0: no lane
// kernel for these layouts), and the launch writing [m, l, o~[hd]] per (query head, run).
int sp_attn_lane_runs(const SpPlan &KP, const SpPlan &VP, const SpAttnArgs &A, size_t part_floats, int n_seq = 1);
hipError_t sp_launch_attn_lane_split(const SpPlan &KP, const SpPlan &VP, const SpAttnArgs &A, const SpSeqTab &T,
                                     const float *qt, float *part, int n_runs, hipStream_t s);
// Batched decode attention through the query preparation, the lane split kernel and the
// combine (hd 96 / hd 64 layouts): q, out [n_seq][n_q][hd], scores at T.soff;
// ws holds n_seq * n_q * hd prepared-query floats, then the partials.
hipError_t sp_launch_attn_lane_seqs(const SpPlan &KP, const SpPlan &VP, const int *order, const SpAttnArgs &A,
                                    const SpSeqTab &T, float *ws, size_t ws_floats, int n_runs, hipStream_t s);
// Checks the arguments of a decode-attention call on one layer of a ship cache
// and fills its launch arguments and K/V plans (band limit applied); -1 with the
// error message set for bad arguments (sp_runtime.cpp).
int sp_attn_prepare(const sp_hip_cache_t *cc, int layer, int n_kv, const float *d_q, int n_q, float kq_scale,
                    float *d_scores, float *d_out, int max_bands, SpAttnArgs *out_args, SpPlan *out_kp,
                    SpPlan *out_vp);
// Sets the message sp_hip_last_error() returns (sp_runtime.cpp).
void sp_set_error(const char *fmt, ...);
// Words at the end of every attention workspace (sp_attn_workspace_floats) that
// hold the wave kernel's per-KV-head arrival counters, one per 256-byte line
// (SP_ATTN_COUNTER_STRIDE words) so the KV heads' atomics do not queue on one
// line: zero when the workspace is created, and back at zero after each call.
#define SP_ATTN_COUNTER_STRIDE 64
#define SP_ATTN_MAX_KVH 256
#define SP_ATTN_COUNTERS (SP_ATTN_MAX_KVH * SP_ATTN_COUNTER_STRIDE)
// Wave-tiled matrix-core kernel for the same layout (sp_attn_wave.hip): scores
// and/or the attention output in one launch (each block writes a spectral-domain
// partial [m, l, o~[hd]] per query head, at most part_floats floats, and the last
// block of each KV head merges them); hipErrorNotSupported for other layouts.
hipError_t sp_launch_attn_wave(const SpPlan &KP, const SpPlan &VP, const int *order, const SpAttnArgs &A, float *part,
                               size_t part_floats, int *counters, hipStream_t s);
hipError_t sp_launch_attn_f16(const unsigned short *k, const unsigned short *v,
                              long long head_stride, int n_kv, int n_q, int n_kvh, int hd,
                              float kq_scale, const float *q, float *scores, float *out,
                              float *workspace, size_t ws_floats, hipStream_t s);

// calibration passes (sp_calib.hip)
int sp_calib_moment_blocks(int n);
// moments of the transform over tlen coefficients of hd-element inputs (tlen > hd: mean padded)
hipError_t sp_launch_calib_moments(const SpPlan &P, int hd, int tlen, const void *src, int dtype, long long si, int n,
                                   double *partials, int n_blocks, hipStream_t s);
int sp_calib_gram_entries(int n_skel, int n_target);
hipError_t sp_launch_calib_hier_gram(const SpPlan &P, const SpHierGeo &G, const void *src, int dtype, long long si,
                                     int n, double *partials, int n_blocks, double *acc, hipStream_t s);
