// sp_attn.hip -- fused decompress-attention decode on gfx950.
//
// Replaces the CPU ggml custom op llama_sp_kq_compute
// (src/engine/llama_sp_fused_kq.cpp:83-165), which decompresses each packed K
// row (dequantize + inverse VHT2) and dots it with every query head, and the
// ggml softmax . V that follows it.
//
// Because the VHT2 is symmetric and orthonormal and the Mobius reorder is a
// permutation, q . K~_t = q~ . dq_t with q~ = reorder(VHT2(q)) and dq_t the
// dequantized spectral record. Likewise sum_t p_t V~_t = VHT2(sum_t p_t dq_t).
// So:
//   1. k_attn_prep:   q~ = kq_scale * reorder(VHT2(q))        (one wave / head)
//   2. k_attn_split:  per (kv head, 256-position split): scores straight from
//                     the packed K codes, partial softmax (m, l), and the
//                     spectral accumulation o~ = sum_t p_t dq(V_t); each packed
//                     K and V record is read once for all query heads of its
//                     GQA group.
//   3. k_attn_combine: merge splits (log-sum-exp), one inverse VHT2 per head.
// No full-precision K or V is materialized anywhere.
#include <stdlib.h>

#include "sp_internal.h"


#define ATT_CHUNK 256
#define ATT_MAX_G 8
#define ATT_MAX_HD 256
#define ATT_MAX_SPLITS 4096  // combine weights in LDS: n_kv <= 1M positions

__global__ void __launch_bounds__(64)
k_attn_prep(const SpPlan KP, const int *__restrict__ order, const float *__restrict__ q, int hd,
            float kq_scale, float *__restrict__ qt) {
    __shared__ float c[ATT_MAX_HD];
    const int h = blockIdx.x, lane = threadIdx.x;
    // the order entries load with the query row, not after the transform
    constexpr int EPL = ATT_MAX_HD / SP_WAVE;
    int src[EPL];
#pragma unroll
    for (int u = 0; u < EPL; u++) {
        const int k = lane + u * SP_WAVE;
        src[u] = (order && k < hd) ? order[k] : k;
    }
    for (int k = lane; k < hd; k += SP_WAVE) c[k] = q[(long long)h * hd + k];
    __syncthreads();
    sp_transform_lds(c, hd, KP, lane);
#pragma unroll
    for (int u = 0; u < EPL; u++) {
        const int k = lane + u * SP_WAVE;
        if (k < hd) qt[(long long)h * hd + k] = kq_scale * c[src[u]];
    }
}

__device__ __forceinline__ void att_tile_load(unsigned char *lds, const unsigned char *g, int nbytes,
                                              int tid, int nthr) {
    const int shift = (int)((uintptr_t)g & 3);
    int head = (4 - shift) & 3;
    if (head > nbytes) head = nbytes;
    if (tid < head) lds[tid] = g[tid];
    const int nw = (nbytes - head) >> 2;
    const uint32_t *gw = reinterpret_cast<const uint32_t *>(g + head);
    uint32_t *lw = reinterpret_cast<uint32_t *>(lds + head);
    for (int k = tid; k < nw; k += nthr) lw[k] = gw[k];
    for (int k = head + 4 * nw + tid; k < nbytes; k += nthr) lds[k] = g[k];
}

// ws layout per (q head, split): [m, l, o~[hd]]
__global__ void __launch_bounds__(256)
k_attn_split(const SpPlan KP, const SpPlan VP, const SpAttnArgs A, const float *__restrict__ qt,
             float *__restrict__ ws, int n_splits, int want_out) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    __shared__ float q_s[ATT_MAX_G][ATT_MAX_HD];
    __shared__ float s_s[ATT_MAX_G][ATT_CHUNK];
    __shared__ float ml_s[ATT_MAX_G][2];

    const int kvh = blockIdx.x, split = blockIdx.y, tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63;
    const int G = A.n_q / A.n_kvh, h0 = kvh * G, hd = A.hd;
    const int t0 = split * ATT_CHUNK;
    const int nt = min(ATT_CHUNK, A.n_kv - t0);

    const unsigned char *kg = A.kpack + (long long)kvh * A.k_head_stride + (long long)t0 * A.kB;
    unsigned char *krec = smem + ((uintptr_t)kg & 3);
    att_tile_load(krec, kg, nt * A.kB, tid, 256);
    unsigned char *vbase = smem + ((ATT_CHUNK * A.kB + 8 + 15) & ~15);
    const unsigned char *vg = A.vpack + (long long)kvh * A.v_head_stride + (long long)t0 * A.vB;
    unsigned char *vrec = vbase + ((uintptr_t)vg & 3);
    if (want_out) att_tile_load(vrec, vg, nt * A.vB, tid, 256);
    for (int k = tid; k < G * hd; k += 256) q_s[k / hd][k % hd] = qt[(long long)(h0 + k / hd) * hd + (k % hd)];
    __syncthreads();

    // ---- scores: one position per thread, straight from the packed codes ----
    if (tid < nt) {
        const unsigned char *rec = krec + tid * A.kB;
        float acc[ATT_MAX_G];
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) acc[h] = 0.0f;
        for (int b = 0; b < KP.max_bands; b++) {  // bands past the limit read as 0
            const int off = KP.band_off[b], sz = KP.band_sz[b], bits = KP.band_bits[b];
            const int maxv = (1 << (bits - 1)) - 1;
            const int bo = KP.band_byte_off[b];
            const float scale = sp_scale_from_bits((uint32_t)rec[bo] | ((uint32_t)rec[bo + 1] << 8));
            float part[ATT_MAX_G];
#pragma unroll
            for (int h = 0; h < ATT_MAX_G; h++) part[h] = 0.0f;
            const unsigned char *data = rec + bo + 2;
            for (int k = 0; k < sz; k++) {
                const float d = (float)((int)sp_unpack_bits_lds(data, k, bits) - maxv);
#pragma unroll
                for (int h = 0; h < ATT_MAX_G; h++)
                    if (h < G) part[h] = fmaf(q_s[h][off + k], d, part[h]);
            }
#pragma unroll
            for (int h = 0; h < ATT_MAX_G; h++) acc[h] = fmaf(scale, part[h], acc[h]);
        }
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++)
            if (h < G) {
                s_s[h][tid] = acc[h];
                if (A.scores) A.scores[(long long)(h0 + h) * A.n_kv + t0 + tid] = acc[h];
            }
    }
    __syncthreads();
    if (!want_out) return;

    // ---- partial softmax per head (wave w handles heads w, w+4) ----
    for (int h = w; h < G; h += 4) {
        float m = -INFINITY;
        for (int t = lane; t < nt; t += SP_WAVE) m = fmaxf(m, s_s[h][t]);
        m = sp_wave_max(m);
        float l = 0.0f;
        for (int t = lane; t < nt; t += SP_WAVE) {
            const float p = __expf(s_s[h][t] - m);
            s_s[h][t] = p;
            l += p;
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) l += __shfl_xor(l, s, SP_WAVE);
        if (lane == 0) { ml_s[h][0] = m; ml_s[h][1] = l; }
    }
    __syncthreads();

    // ---- spectral accumulation of V: thread owns element i ----
    for (int i = tid; i < hd; i += 256) {
        int b = 0;
        while (b + 1 < VP.n_bands && i >= VP.band_off[b + 1]) b++;
        const int bits = VP.band_bits[b], maxv = (1 << (bits - 1)) - 1;
        const int bo = VP.band_byte_off[b], k = i - VP.band_off[b];
        float o[ATT_MAX_G];
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) o[h] = 0.0f;
        const int nt_v = b < VP.max_bands ? nt : 0;  // a band past the limit reads as 0
        for (int t = 0; t < nt_v; t++) {
            const unsigned char *rec = vrec + t * A.vB;
            const float scale = sp_scale_from_bits((uint32_t)rec[bo] | ((uint32_t)rec[bo + 1] << 8));
            const float d = (float)((int)sp_unpack_bits_lds(rec + bo + 2, k, bits) - maxv) * scale;
#pragma unroll
            for (int h = 0; h < ATT_MAX_G; h++)
                if (h < G) o[h] = fmaf(s_s[h][t], d, o[h]);
        }
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++)
            if (h < G) ws[((long long)(h0 + h) * n_splits + split) * (hd + 2) + 2 + i] = o[h];
    }
    if (tid < G) {
        ws[((long long)(h0 + tid) * n_splits + split) * (hd + 2) + 0] = ml_s[tid][0];
        ws[((long long)(h0 + tid) * n_splits + split) * (hd + 2) + 1] = ml_s[tid][1];
    }
}

// Merge the split partials of one query head: M = max_s m_s, e_s = exp(m_s - M),
// L = sum_s l_s e_s, o~ = sum_s e_s o~_s / L, then one inverse VHT2.
// 1024 threads: thread (i, g) sums element i over splits g, g + ng, ...; its
// first 16 partial values are loaded before the weights are formed, so a
// typical combine costs one round trip to memory. n_splits <= ATT_MAX_SPLITS.
#define COMB_THREADS 1024
#define COMB_PRE 16
__device__ __forceinline__ float comb_block_reduce(float v, float *red, bool is_max) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float o = __shfl_xor(v, m, 64);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    __syncthreads();  // red may still be read by a previous reduction
    if (lane == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (int k = 1; k < COMB_THREADS / 64; k++) r = is_max ? fmaxf(r, red[k]) : r + red[k];
    return r;
}

__global__ void __launch_bounds__(COMB_THREADS)
k_attn_combine(const SpPlan VP, const float *__restrict__ ws, int n_splits, int hd,
               float *__restrict__ out) {
    __shared__ float e_s[ATT_MAX_SPLITS];
    __shared__ float red[COMB_THREADS];
    __shared__ float c[ATT_MAX_HD];
    const int h = blockIdx.x, tid = threadIdx.x;
    const long long row = hd + 2;
    const float *base = ws + (long long)h * n_splits * row;
    const int ng = COMB_THREADS / hd;  // element groups (>= 4 for hd <= 256)
    const int i = tid % hd, g = tid / hd;
    const bool active = g < ng;
    float pre[COMB_PRE];
#pragma unroll
    for (int r = 0; r < COMB_PRE; r++) {
        const int sp = g + ng * r;
        pre[r] = (active && sp < n_splits) ? base[sp * row + 2 + i] : 0.0f;
    }
    float M = -INFINITY;
    for (int sp = tid; sp < n_splits; sp += COMB_THREADS) M = fmaxf(M, base[sp * row]);
    M = comb_block_reduce(M, red, true);
    float L = 0.0f;
    for (int sp = tid; sp < n_splits; sp += COMB_THREADS) {
        const float e = __expf(base[sp * row] - M);
        e_s[sp] = e;
        L += base[sp * row + 1] * e;
    }
    L = comb_block_reduce(L, red, false);  // its barriers also publish e_s
    const float invL = 1.0f / L;
    float acc = 0.0f;
    if (active) {
#pragma unroll
        for (int r = 0; r < COMB_PRE; r++) {
            const int sp = g + ng * r;
            if (sp < n_splits) acc = fmaf(pre[r], e_s[sp], acc);
        }
#pragma unroll 8
        for (int sp = g + ng * COMB_PRE; sp < n_splits; sp += ng) acc = fmaf(base[sp * row + 2 + i], e_s[sp], acc);
    }
    __syncthreads();
    red[tid] = acc;
    __syncthreads();
    if (tid < hd) {
        float t = 0.0f;
        for (int k = 0; k < ng; k++) t += red[k * hd + tid];
        c[tid] = t * invL;
    }
    __syncthreads();
    // every thread reaches the transform's barriers; only wave 0 does its work
    sp_transform_lds(c, hd, VP, tid < SP_WAVE ? tid : hd);
    if (tid < SP_WAVE)
        for (int k = tid; k < hd; k += SP_WAVE) out[(long long)h * hd + k] = c[k];
}

// The same merge for rows of at most 64 splits by one wave per row: split `lane`'s m and
// l, a wave-wide max and sum (lane shuffles), the row's elements by lane (i = lane,
// lane + 64, ...), each summed over the splits in order, then the inverse transform.
// A batch of short sequences has a few splits per row, so the 1024-thread block of
// k_attn_combine would be mostly idle and its block reductions the cost.
__global__ void __launch_bounds__(64)
k_attn_combine_wave(const SpPlan VP, const float *__restrict__ ws, int n_splits, int hd, float *__restrict__ out) {
    __shared__ float e_s[SP_WAVE];
    __shared__ float c[ATT_MAX_HD];
    const int h = blockIdx.x, lane = threadIdx.x;
    const long long row = hd + 2;
    const float *base = ws + (long long)h * n_splits * row;
    const bool live = lane < n_splits;
    const float m = live ? base[lane * row] : -INFINITY;
    const float lv = live ? base[lane * row + 1] : 0.0f;
    // rows of at most CW splits (a batch of short sequences) load their elements at
    // entry with m and l, so the row waits on memory once; longer rows load them in the
    // sum below (their loads at entry measured slower)
    constexpr int CW = 8, EPL = ATT_MAX_HD / SP_WAVE;
    const bool pre = n_splits <= CW;
    float pv[CW][EPL];
    if (pre) {
#pragma unroll
        for (int sp = 0; sp < CW; sp++) {
#pragma unroll
            for (int u = 0; u < EPL; u++) {
                const int i = lane + u * SP_WAVE;
                pv[sp][u] = sp < n_splits && i < hd ? base[sp * row + 2 + i] : 0.0f;
            }
        }
    }
    float M = m;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, SP_WAVE));
    const float e = live ? __expf(m - M) : 0.0f;
    float L = lv * e;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += __shfl_xor(L, o, SP_WAVE);
    e_s[lane] = e;
    __syncthreads();
    const float invL = 1.0f / L;
    if (pre) {
#pragma unroll
        for (int u = 0; u < EPL; u++) {
            const int i = lane + u * SP_WAVE;
            if (i >= hd) continue;
            float acc = 0.0f;
#pragma unroll
            for (int sp = 0; sp < CW; sp++)
                if (sp < n_splits) acc = fmaf(pv[sp][u], e_s[sp], acc);
            c[i] = acc * invL;
        }
    } else {
        for (int i = lane; i < hd; i += SP_WAVE) {
            float acc = 0.0f;
#pragma unroll 8
            for (int sp = 0; sp < n_splits; sp++) acc = fmaf(base[sp * row + 2 + i], e_s[sp], acc);
            c[i] = acc * invL;
        }
    }
    __syncthreads();
    sp_transform_lds(c, hd, VP, lane);
    for (int k = lane; k < hd; k += SP_WAVE) out[(long long)h * hd + k] = c[k];
}

hipError_t sp_launch_attn_lane_seqs(const SpPlan &KP, const SpPlan &VP, const int *order, const SpAttnArgs &A,
                                    const SpSeqTab &T, float *ws, size_t ws_floats, int n_runs, hipStream_t s) {
    const size_t n_rows = (size_t)T.n_seq * A.n_q;
    if (T.n_seq < 1 || T.n_seq > SP_ATTN_MAX_SEQ || n_runs <= 0 || n_runs > ATT_MAX_SPLITS ||
        n_rows * A.hd + n_rows * n_runs * (A.hd + 2) > ws_floats)
        return hipErrorInvalidValue;
    float *qt = ws;
    float *part = ws + n_rows * A.hd;
    hipLaunchKernelGGL(k_attn_prep, dim3((unsigned)n_rows), dim3(64), 0, s, KP, order, A.q, A.hd, A.kq_scale, qt);
    const hipError_t le = sp_launch_attn_lane_split(KP, VP, A, T, qt, part, n_runs, s);
    if (le != hipSuccess) return le;
    if (A.out && n_runs <= SP_WAVE)
        hipLaunchKernelGGL(k_attn_combine_wave, dim3((unsigned)n_rows), dim3(SP_WAVE), 0, s, VP, part, n_runs, A.hd,
                           A.out);
    else if (A.out)
        hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)n_rows), dim3(COMB_THREADS), 0, s, VP, part, n_runs, A.hd,
                           A.out);
    return hipGetLastError();
}

size_t sp_attn_workspace_floats(int n_q, int hd, int max_kv) {
    const int n_splits = (max_kv + ATT_CHUNK - 1) / ATT_CHUNK;
    return (size_t)n_q * hd + (size_t)n_q * n_splits * (hd + 2) + SP_ATTN_COUNTERS + SP_ATTN_COUNTER_STRIDE;
}

hipError_t sp_launch_attn_decode(const SpPlan &KP, const SpPlan &VP, const int *order,
                                 const SpAttnArgs &A, float *workspace, size_t ws_floats,
                                 hipStream_t s) {
    if (A.n_kv <= 0 || A.n_q <= 0 || A.n_kvh <= 0 || A.n_q % A.n_kvh) return hipErrorInvalidValue;
    if (A.n_q / A.n_kvh > ATT_MAX_G || A.hd > ATT_MAX_HD) return hipErrorInvalidValue;
    if (sp_attn_workspace_floats(A.n_q, A.hd, A.n_kv) > ws_floats) return hipErrorInvalidValue;
    const int n_splits = (A.n_kv + ATT_CHUNK - 1) / ATT_CHUNK;
    if (n_splits > ATT_MAX_SPLITS) return hipErrorInvalidValue;
    float *qt = workspace;
    float *part = workspace + (size_t)A.n_q * A.hd;
    const int want_out = A.out != nullptr;
    {
        // the per-KV-head arrival counters: the workspace's last SP_ATTN_COUNTERS words
        // (plus up to one line of slack), starting on a 256-byte boundary
        const uintptr_t ctail = (uintptr_t)(workspace + ws_floats - SP_ATTN_COUNTERS - SP_ATTN_COUNTER_STRIDE);
        int *cnt = reinterpret_cast<int *>((ctail + 255) & ~(uintptr_t)255);
        const hipError_t we = sp_launch_attn_wave(
            KP, VP, order, A, part, ws_floats - (size_t)A.n_q * A.hd - SP_ATTN_COUNTERS - SP_ATTN_COUNTER_STRIDE, cnt, s);
        if (we != hipErrorNotSupported) return we;
    }
    {
        // hd 96 / hd 64 shipping layouts: the one-position-per-lane split kernel
        // (sp_attn_lane.hip) between the same query preparation and combine
        // (SP_HIP_NO_LANE_ATTN=1, read at each call, keeps them on the kernel below)
        const char *off = getenv("SP_HIP_NO_LANE_ATTN");
        const size_t part_floats = ws_floats - (size_t)A.n_q * A.hd - SP_ATTN_COUNTERS - SP_ATTN_COUNTER_STRIDE;
        const int n_runs = (off && off[0] == '1') ? 0 : sp_attn_lane_runs(KP, VP, A, part_floats);
        if (n_runs > 0) {
            SpSeqTab T;
            T.n_seq = 1;
            T.max_len = A.n_kv;
            T.start[0] = 0;
            T.len[0] = A.n_kv;
            T.soff[0] = 0;
            return sp_launch_attn_lane_seqs(KP, VP, order, A, T, workspace, ws_floats, n_runs, s);
        }
    }
    hipLaunchKernelGGL(k_attn_prep, dim3(A.n_q), dim3(64), 0, s, KP, order, A.q, A.hd, A.kq_scale, qt);
    const size_t lds = (size_t)((ATT_CHUNK * A.kB + 8 + 15) & ~15) + (size_t)ATT_CHUNK * A.vB + 8;
    hipLaunchKernelGGL(k_attn_split, dim3(A.n_kvh, n_splits), dim3(256), lds, s, KP, VP, A, qt, part,
                       n_splits, want_out);
    if (want_out)
        hipLaunchKernelGGL(k_attn_combine, dim3(A.n_q), dim3(COMB_THREADS), 0, s, VP, part, n_splits, A.hd, A.out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fp16 uncompressed baseline with the same split structure
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_attn_f16_split(const unsigned short *__restrict__ K, const unsigned short *__restrict__ V,
                 long long head_stride, int n_kv, int n_q, int n_kvh, int hd, float kq_scale,
                 const float *__restrict__ q, float *__restrict__ scores, float *__restrict__ ws,
                 int n_splits, int want_out) {
    __shared__ float q_s[ATT_MAX_G][ATT_MAX_HD];
    __shared__ float s_s[ATT_MAX_G][ATT_CHUNK];
    __shared__ float ml_s[ATT_MAX_G][2];
    const int kvh = blockIdx.x, split = blockIdx.y, tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63;
    const int G = n_q / n_kvh, h0 = kvh * G;
    const int t0 = split * ATT_CHUNK, nt = min(ATT_CHUNK, n_kv - t0);
    for (int k = tid; k < G * hd; k += 256) q_s[k / hd][k % hd] = q[(long long)(h0 + k / hd) * hd + (k % hd)] * kq_scale;
    __syncthreads();
    const unsigned short *Kh = K + (long long)kvh * head_stride;
    const unsigned short *Vh = V + (long long)kvh * head_stride;
    if (tid < nt) {
        const unsigned short *row = Kh + (long long)(t0 + tid) * hd;
        float acc[ATT_MAX_G];
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) acc[h] = 0.0f;
        for (int d0 = 0; d0 < hd; d0 += 8) {
            const uint4 wv = *reinterpret_cast<const uint4 *>(row + d0);
            const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float kv = sp_f16_bits_to_f32((ww[e >> 1] >> (16 * (e & 1))) & 0xffffu);
#pragma unroll
                for (int h = 0; h < ATT_MAX_G; h++)
                    if (h < G) acc[h] = fmaf(q_s[h][d0 + e], kv, acc[h]);
            }
        }
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++)
            if (h < G) {
                s_s[h][tid] = acc[h];
                if (scores) scores[(long long)(h0 + h) * n_kv + t0 + tid] = acc[h];
            }
    }
    __syncthreads();
    if (!want_out) return;
    for (int h = w; h < G; h += 4) {
        float m = -INFINITY;
        for (int t = lane; t < nt; t += SP_WAVE) m = fmaxf(m, s_s[h][t]);
        m = sp_wave_max(m);
        float l = 0.0f;
        for (int t = lane; t < nt; t += SP_WAVE) {
            const float p = __expf(s_s[h][t] - m);
            s_s[h][t] = p;
            l += p;
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) l += __shfl_xor(l, s, SP_WAVE);
        if (lane == 0) { ml_s[h][0] = m; ml_s[h][1] = l; }
    }
    __syncthreads();
    for (int i = tid; i < hd; i += 256) {
        float o[ATT_MAX_G];
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++) o[h] = 0.0f;
        for (int t = 0; t < nt; t++) {
            const float vv = sp_f16_bits_to_f32(Vh[(long long)(t0 + t) * hd + i]);
#pragma unroll
            for (int h = 0; h < ATT_MAX_G; h++)
                if (h < G) o[h] = fmaf(s_s[h][t], vv, o[h]);
        }
#pragma unroll
        for (int h = 0; h < ATT_MAX_G; h++)
            if (h < G) ws[((long long)(h0 + h) * n_splits + split) * (hd + 2) + 2 + i] = o[h];
    }
    if (tid < G) {
        ws[((long long)(h0 + tid) * n_splits + split) * (hd + 2) + 0] = ml_s[tid][0];
        ws[((long long)(h0 + tid) * n_splits + split) * (hd + 2) + 1] = ml_s[tid][1];
    }
}

__global__ void __launch_bounds__(64)
k_attn_f16_combine(const float *__restrict__ ws, int n_splits, int hd, float *__restrict__ out) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const float *base = ws + (long long)h * n_splits * (hd + 2);
    float M = -INFINITY;
    for (int s = 0; s < n_splits; s++) M = fmaxf(M, base[(long long)s * (hd + 2)]);
    float L = 0.0f;
    for (int s = 0; s < n_splits; s++) L += base[(long long)s * (hd + 2) + 1] * __expf(base[(long long)s * (hd + 2)] - M);
    const float invL = 1.0f / L;
    for (int i = lane; i < hd; i += SP_WAVE) {
        float acc = 0.0f;
        for (int s = 0; s < n_splits; s++) {
            const float *p = base + (long long)s * (hd + 2);
            acc = fmaf(p[2 + i], __expf(p[0] - M), acc);
        }
        out[(long long)h * hd + i] = acc * invL;
    }
}

hipError_t sp_launch_attn_f16(const unsigned short *k, const unsigned short *v,
                              long long head_stride, int n_kv, int n_q, int n_kvh, int hd,
                              float kq_scale, const float *q, float *scores, float *out,
                              float *workspace, size_t ws_floats, hipStream_t s) {
    if (n_kv <= 0 || n_q <= 0 || n_kvh <= 0 || n_q % n_kvh) return hipErrorInvalidValue;
    if (n_q / n_kvh > ATT_MAX_G || hd > ATT_MAX_HD || hd % 8) return hipErrorInvalidValue;
    if (sp_attn_workspace_floats(n_q, hd, n_kv) > ws_floats) return hipErrorInvalidValue;
    const int n_splits = (n_kv + ATT_CHUNK - 1) / ATT_CHUNK;
    float *part = workspace + (size_t)n_q * hd;
    const int want_out = out != nullptr;
    hipLaunchKernelGGL(k_attn_f16_split, dim3(n_kvh, n_splits), dim3(256), 0, s, k, v, head_stride,
                       n_kv, n_q, n_kvh, hd, kq_scale, q, scores, part, n_splits, want_out);
    if (want_out)
        hipLaunchKernelGGL(k_attn_f16_combine, dim3(n_q), dim3(64), 0, s, part, n_splits, hd, out);
    return hipGetLastError();
}
