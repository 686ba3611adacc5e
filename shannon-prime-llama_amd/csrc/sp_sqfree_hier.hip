// sp_sqfree_hier.hip -- gfx950 kernels of the sqfree+spinor and hierarchical
// Vilenkin codecs. One vector per wave, stages staged through LDS, one launch
// per batch (the reference issues ~10 launches and several device copies per
// vector: shannon_prime_sqfree.cu:750-853, shannon_prime_hier.cu:399-486).
//
// Sqfree write: pad (true mean fill) -> Vilenkin -> skeleton gather -> band
// quantize skeleton -> Mobius CSR predict -> spinor / plain deviation ->
// mag = max(mean|dev|, 1e-12) -> residual levels -> LSB-first pack -> sheet.
// Record: [skeleton bands][mag f32 LE][residual bits][sheet bits]
// (shannon_prime_sqfree.cu:683-686).
// Hier write: pad -> Vilenkin -> skeleton gather -> band quantize -> fp16 W
// GEMV prediction -> deviation -> mag -> rint levels -> pack. Record:
// [skeleton bands][mag f32 LE][residual bits] (shannon_prime_hier.cu:331-335).
#include <stdlib.h>

#include "sp_internal.h"

__device__ __forceinline__ void sp_pad_mean(float *c, int hd, int pad, int lane) {
    const float sum = sp_wave_tree256_sum(c, hd, 0, lane);
    const float mean = sp_div(sum, (float)hd);
    for (int k = hd + lane; k < pad; k += SP_WAVE) c[k] = mean;
    __syncthreads();
}

__device__ __forceinline__ float sp_mag_floor(const float *dv, int n, int lane) {
    float mag = sp_div(sp_wave_tree256_sum(dv, n, 1, lane), (float)n);
    return mag < 1e-12f ? 1e-12f : mag;
}

__device__ __forceinline__ void sp_put_f32(unsigned char *p, float v) {
    const uint32_t u = __float_as_uint(v);
    p[0] = (unsigned char)u;
    p[1] = (unsigned char)(u >> 8);
    p[2] = (unsigned char)(u >> 16);
    p[3] = (unsigned char)(u >> 24);
}

__device__ __forceinline__ float sp_get_f32(const unsigned char *p) {
    return __uint_as_float((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                           ((uint32_t)p[3] << 24));
}

// CSR Mobius prediction of residual r from skeleton values sk (LDS).
__device__ __forceinline__ float sp_csr_predict(const SpSqGeo &G, const float *sk, int r) {
    float p = 0.0f;
    for (int jj = G.csr_off[r]; jj < G.csr_off[r + 1]; jj++) p += (float)G.csr_mu[jj] * sk[G.csr_slot[jj]];
    return p;
}

template <int DT>
__global__ void __launch_bounds__(256)
k_sqfree_encode(const SpPlan P, const SpSqGeo G, const void *__restrict__ src, long long so,
                long long si, unsigned char *__restrict__ dst, long long dout, int n_outer,
                int n_inner) {
    __shared__ float c_s[4][SP_GEN_MAX_N];
    __shared__ float sk_s[4][SP_GEN_MAX_N];
    __shared__ float dv_s[4][SP_GEN_MAX_N];
    __shared__ unsigned char codes_s[4][SP_GEN_MAX_N];
    __shared__ unsigned char flag_s[4][SP_GEN_MAX_N];
    __shared__ __attribute__((aligned(16))) unsigned char rec_s[4][SP_GEN_MAX_REC];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long v = (long long)blockIdx.x * 4 + w;
    const bool valid = v < (long long)n_outer * n_inner;
    const int o = valid ? (int)(v / n_inner) : 0, i = valid ? (int)(v % n_inner) : 0;
    float *c = c_s[w], *sk = sk_s[w], *dv = dv_s[w];
    unsigned char *codes = codes_s[w], *flag = flag_s[w], *rec = rec_s[w];

    for (int k = lane; k < G.hd; k += SP_WAVE)
        c[k] = valid ? sp_load1<DT>(src, (long long)o * so + (long long)i * si + k) : 0.0f;
    for (int k = lane; k < SP_GEN_MAX_REC; k += SP_WAVE) rec[k] = 0;
    __syncthreads();
    sp_pad_mean(c, G.hd, G.pad, lane);
    sp_transform_lds(c, G.pad, P, lane);
    for (int s = lane; s < G.sk_k; s += SP_WAVE) sk[s] = c[G.skel_idx[s]];
    __syncthreads();
    sp_band_quantize_lds(sk, rec, codes, P, lane);
    const int skB = P.total_bytes;
    if (G.n_res > 0) {
        for (int r = lane; r < G.n_res; r += SP_WAVE) {
            const float p = sp_csr_predict(G, sk, r);
            const float a = c[G.res_idx[r]];
            float d;
            if (G.spinor) {
                const float vp = a - p, vm = a + p;
                const bool um = fabsf(vm) < fabsf(vp);
                d = um ? vm : vp;
                flag[r] = um ? 1 : 0;
            } else {
                d = a - p;
            }
            dv[r] = d;
        }
        __syncthreads();
        const float mag = sp_mag_floor(dv, G.n_res, lane);
        if (lane == 0) sp_put_f32(rec + skB, mag);
        const int L = 1 << G.rbits;
        const float center = 0.5f * (float)(L - 1);
        const float sat = (mag > 1e-12f) ? (mag * (float)G.rbits) : 1e-12f;
        const float step = sp_div(2.0f * sat, (float)(L - 1));
        const float inv_step = sp_div(1.0f, step);
        for (int r = lane; r < G.n_res; r += SP_WAVE) {
            const float qf = dv[r] * inv_step + center;
            int level = sp_trunc_sat(qf + 0.5f);
            level = level < 0 ? 0 : (level >= L ? L - 1 : level);
            codes[r] = (unsigned char)level;
        }
        const int res_bytes = (G.n_res * G.rbits + 7) / 8;
        if (G.spinor)
            for (int kk = lane; kk < (G.n_res + 7) / 8; kk += SP_WAVE) {
                uint32_t byte = 0;
                for (int t = 0; t < 8 && 8 * kk + t < G.n_res; t++) byte |= (uint32_t)flag[8 * kk + t] << t;
                rec[skB + 4 + res_bytes + kk] = (unsigned char)byte;
            }
        __syncthreads();
        sp_pack_bits_lds(codes, G.n_res, G.rbits, rec + skB + 4, lane);
        __syncthreads();
    }
    if (valid) {
        unsigned char *g = dst + (long long)o * dout + (long long)i * G.bytes;
        for (int k = lane; k < G.bytes; k += SP_WAVE) g[k] = rec[k];
    }
}

template <int DT>
__global__ void __launch_bounds__(256)
k_sqfree_decode(const SpPlan P, const SpSqGeo G, const unsigned char *__restrict__ src,
                long long so, void *__restrict__ dst, long long dout, long long din, int n_outer,
                int n_inner, const int *__restrict__ cells) {
    __shared__ float c_s[4][SP_GEN_MAX_N];
    __shared__ float sk_s[4][SP_GEN_MAX_N];
    __shared__ __attribute__((aligned(16))) unsigned char rec_s[4][SP_GEN_MAX_REC];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long v = (long long)blockIdx.x * 4 + w;
    const bool valid = v < (long long)n_outer * n_inner;
    const int o = valid ? (int)(v / n_inner) : 0, i0 = valid ? (int)(v % n_inner) : 0;
    const int i = cells ? (valid ? cells[i0] : 0) : i0;  // listed positions: record and row at cells[i0]
    float *c = c_s[w], *sk = sk_s[w];
    unsigned char *rec = rec_s[w];
    const unsigned char *g = src + (long long)o * so + (long long)i * G.bytes;
    for (int k = lane; k < SP_GEN_MAX_REC; k += SP_WAVE) rec[k] = (valid && k < G.bytes) ? g[k] : 0;
    for (int k = lane; k < G.pad; k += SP_WAVE) c[k] = 0.0f;
    __syncthreads();
    sp_band_dequantize_lds(rec, sk, P, lane);
    for (int s = lane; s < G.sk_k; s += SP_WAVE) c[G.skel_idx[s]] = sk[s];
    const int skB = P.total_bytes;
    if (G.n_res > 0) {
        const float mag = sp_get_f32(rec + skB);
        const int L = 1 << G.rbits;
        const float center = 0.5f * (float)(L - 1);
        const float sat = mag * (float)G.rbits;
        const float step = (L > 1) ? sp_div(2.0f * sat, (float)(L - 1)) : 0.0f;
        const int res_bytes = (G.n_res * G.rbits + 7) / 8;
        const unsigned char *sheet = rec + skB + 4 + res_bytes;
        for (int r = lane; r < G.n_res; r += SP_WAVE) {
            float p = sp_csr_predict(G, sk, r);
            if (G.spinor && (sheet[r >> 3] & (1u << (r & 7)))) p = -p;
            const uint32_t lv = sp_unpack_bits_lds(rec + skB + 4, r, G.rbits);
            const float d = ((float)lv - center) * step;
            c[G.res_idx[r]] = p + d;
        }
    }
    __syncthreads();
    sp_transform_lds(c, G.pad, P, lane);
    if (valid)
        for (int k = lane; k < G.hd; k += SP_WAVE)
            sp_store1<DT>(dst, (long long)o * dout + (long long)i * din + k, c[k]);
}

template <int DT>
__global__ void __launch_bounds__(256)
k_hier_encode(const SpPlan P, const SpHierGeo G, const void *__restrict__ src, long long so,
              long long si, unsigned char *__restrict__ dst, long long dout, int n_outer,
              int n_inner) {
    __shared__ float c_s[4][SP_GEN_MAX_N];
    __shared__ float sk_s[4][SP_GEN_MAX_N];
    __shared__ float dv_s[4][SP_GEN_MAX_N];
    __shared__ unsigned char codes_s[4][SP_GEN_MAX_N];
    __shared__ __attribute__((aligned(16))) unsigned char rec_s[4][SP_GEN_MAX_REC];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long v = (long long)blockIdx.x * 4 + w;
    const bool valid = v < (long long)n_outer * n_inner;
    const int o = valid ? (int)(v / n_inner) : 0, i = valid ? (int)(v % n_inner) : 0;
    float *c = c_s[w], *sk = sk_s[w], *dv = dv_s[w];
    unsigned char *codes = codes_s[w], *rec = rec_s[w];
    const uint16_t *Wslot = G.W + (long long)o * G.w_outer;

    for (int k = lane; k < G.hd; k += SP_WAVE)
        c[k] = valid ? sp_load1<DT>(src, (long long)o * so + (long long)i * si + k) : 0.0f;
    for (int k = lane; k < SP_GEN_MAX_REC; k += SP_WAVE) rec[k] = 0;
    __syncthreads();
    sp_pad_mean(c, G.hd, G.pad, lane);
    sp_transform_lds(c, G.pad, P, lane);
    for (int s = lane; s < G.n_skel; s += SP_WAVE) sk[s] = c[G.skel_idx[s]];
    __syncthreads();
    sp_band_quantize_lds(sk, rec, codes, P, lane);
    for (int t = lane; t < G.n_target; t += SP_WAVE) {
        const uint16_t *row = Wslot + (long long)t * G.n_skel;
        float acc = 0.0f;
        for (int s = 0; s < G.n_skel; s++) acc += sp_f16_bits_to_f32(row[s]) * sk[s];
        dv[t] = c[G.target_idx[t]] - acc;
    }
    __syncthreads();
    const float mag = sp_mag_floor(dv, G.n_target, lane);
    const int skB = P.total_bytes;
    if (lane == 0) sp_put_f32(rec + skB, mag);
    const int L = 1 << G.rbits;
    const float step = sp_div(2.0f * mag, (float)(L - 1));
    const float center = sp_div((float)(L - 1), 2.0f);
    const float inv_step = (step > 0.0f) ? sp_div(1.0f, step) : 0.0f;
    for (int t = lane; t < G.n_target; t += SP_WAVE) {
        int q = sp_rint_sat(dv[t] * inv_step + center);
        q = q < 0 ? 0 : (q >= L ? L - 1 : q);
        codes[t] = (unsigned char)q;
    }
    __syncthreads();
    sp_pack_bits_lds(codes, G.n_target, G.rbits, rec + skB + 4, lane);
    __syncthreads();
    if (valid) {
        unsigned char *g = dst + (long long)o * dout + (long long)i * G.bytes;
        for (int k = lane; k < G.bytes; k += SP_WAVE) g[k] = rec[k];
    }
}

template <int DT>
__global__ void __launch_bounds__(256)
k_hier_decode(const SpPlan P, const SpHierGeo G, const unsigned char *__restrict__ src,
              long long so, void *__restrict__ dst, long long dout, long long din, int n_outer,
              int n_inner, const int *__restrict__ cells) {
    __shared__ float c_s[4][SP_GEN_MAX_N];
    __shared__ float sk_s[4][SP_GEN_MAX_N];
    __shared__ __attribute__((aligned(16))) unsigned char rec_s[4][SP_GEN_MAX_REC];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long v = (long long)blockIdx.x * 4 + w;
    const bool valid = v < (long long)n_outer * n_inner;
    const int o = valid ? (int)(v / n_inner) : 0, i0 = valid ? (int)(v % n_inner) : 0;
    const int i = cells ? (valid ? cells[i0] : 0) : i0;  // listed positions: record and row at cells[i0]
    float *c = c_s[w], *sk = sk_s[w];
    unsigned char *rec = rec_s[w];
    const uint16_t *Wslot = G.W + (long long)o * G.w_outer;
    const unsigned char *g = src + (long long)o * so + (long long)i * G.bytes;
    for (int k = lane; k < SP_GEN_MAX_REC; k += SP_WAVE) rec[k] = (valid && k < G.bytes) ? g[k] : 0;
    for (int k = lane; k < G.pad; k += SP_WAVE) c[k] = 0.0f;
    __syncthreads();
    sp_band_dequantize_lds(rec, sk, P, lane);
    for (int s = lane; s < G.n_skel; s += SP_WAVE) c[G.skel_idx[s]] = sk[s];
    const int skB = P.total_bytes;
    const float mag = sp_get_f32(rec + skB);
    const int L = 1 << G.rbits;
    const float step = sp_div(2.0f * mag, (float)(L - 1));
    const float center = sp_div((float)(L - 1), 2.0f);
    for (int t = lane; t < G.n_target; t += SP_WAVE) {
        const uint16_t *row = Wslot + (long long)t * G.n_skel;
        float acc = 0.0f;
        for (int s = 0; s < G.n_skel; s++) acc += sp_f16_bits_to_f32(row[s]) * sk[s];
        const uint32_t lv = sp_unpack_bits_lds(rec + skB + 4, t, G.rbits);
        c[G.target_idx[t]] = acc + ((float)lv - center) * step;
    }
    __syncthreads();
    sp_transform_lds(c, G.pad, P, lane);
    if (valid)
        for (int k = lane; k < G.hd; k += SP_WAVE)
            sp_store1<DT>(dst, (long long)o * dout + (long long)i * din + k, c[k]);
}

// ---------------------------------------------------------------------------
static bool sq_fits(const SpPlan &P, int pad, int bytes) {
    return pad <= SP_GEN_MAX_N && P.hd <= SP_GEN_MAX_N && bytes + 8 <= SP_GEN_MAX_REC;
}

// SP_HIP_NO_LANE_KERNELS=1 routes the sqfree and hier geometries with a lane
// specialization through the one-vector-per-wave kernels (used by tests to
// cross-check them).
static bool getenv_lane_off_sq() {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("SP_HIP_NO_LANE_KERNELS");
        v = (e && e[0] == '1') ? 1 : 0;
    }
    return v == 1;
}

hipError_t sp_launch_sqfree_encode(const SpPlan &P, const SpSqGeo &G, const void *src, int dtype,
                                   long long so, long long si, unsigned char *dst, long long dout,
                                   int n_outer, int n_inner, hipStream_t s) {
    if (n_outer <= 0 || n_inner <= 0) return hipSuccess;
    if (!sq_fits(P, G.pad, G.bytes)) return hipErrorInvalidValue;
    if (!getenv_lane_off_sq()) {
        const hipError_t e = sp_launch_sqfree_encode_lane(P, G, src, dtype, so, si, dst, dout, n_outer, n_inner, s);
        if (e != hipErrorNotSupported) return e;
    }
    const long long nv = (long long)n_outer * n_inner;
    const dim3 grid((unsigned)((nv + 3) / 4)), block(256);
    if (dtype == SP_DT_F16)
        hipLaunchKernelGGL((k_sqfree_encode<SP_DT_F16>), grid, block, 0, s, P, G, src, so, si, dst, dout, n_outer, n_inner);
    else
        hipLaunchKernelGGL((k_sqfree_encode<SP_DT_F32>), grid, block, 0, s, P, G, src, so, si, dst, dout, n_outer, n_inner);
    return hipGetLastError();
}

hipError_t sp_launch_sqfree_decode(const SpPlan &P, const SpSqGeo &G, const unsigned char *src,
                                   long long so, void *dst, int dtype, long long dout,
                                   long long din, int n_outer, int n_inner, hipStream_t s, const int *cells) {
    if (n_outer <= 0 || n_inner <= 0) return hipSuccess;
    if (!sq_fits(P, G.pad, G.bytes)) return hipErrorInvalidValue;
    if (!getenv_lane_off_sq()) {
        const hipError_t e =
            cells ? sp_launch_sqfree_decode_lane_cells(P, G, src, so, dst, dtype, dout, din, n_outer, n_inner, cells, s)
                  : sp_launch_sqfree_decode_lane(P, G, src, so, dst, dtype, dout, din, n_outer, n_inner, s);
        if (e != hipErrorNotSupported) return e;
    }
    const long long nv = (long long)n_outer * n_inner;
    const dim3 grid((unsigned)((nv + 3) / 4)), block(256);
    if (dtype == SP_DT_F16)
        hipLaunchKernelGGL((k_sqfree_decode<SP_DT_F16>), grid, block, 0, s, P, G, src, so, dst, dout, din, n_outer, n_inner, cells);
    else
        hipLaunchKernelGGL((k_sqfree_decode<SP_DT_F32>), grid, block, 0, s, P, G, src, so, dst, dout, din, n_outer, n_inner, cells);
    return hipGetLastError();
}

hipError_t sp_launch_hier_encode(const SpPlan &P, const SpHierGeo &G, const void *src, int dtype,
                                 long long so, long long si, unsigned char *dst, long long dout,
                                 int n_outer, int n_inner, hipStream_t s) {
    if (n_outer <= 0 || n_inner <= 0) return hipSuccess;
    if (!sq_fits(P, G.pad, G.bytes)) return hipErrorInvalidValue;
    if (!getenv_lane_off_sq()) {
        const hipError_t e = sp_launch_hier_encode_lane(P, G, src, dtype, so, si, dst, dout, n_outer, n_inner, s);
        if (e != hipErrorNotSupported) return e;
    }
    const long long nv = (long long)n_outer * n_inner;
    const dim3 grid((unsigned)((nv + 3) / 4)), block(256);
    if (dtype == SP_DT_F16)
        hipLaunchKernelGGL((k_hier_encode<SP_DT_F16>), grid, block, 0, s, P, G, src, so, si, dst, dout, n_outer, n_inner);
    else
        hipLaunchKernelGGL((k_hier_encode<SP_DT_F32>), grid, block, 0, s, P, G, src, so, si, dst, dout, n_outer, n_inner);
    return hipGetLastError();
}

hipError_t sp_launch_hier_encode_kv(const SpPlan &P, const SpHierGeo &G, const void *src_k, const void *src_v,
                                    int dtype, long long so, long long si, unsigned char *dst_k,
                                    unsigned char *dst_v, long long dout, int n_outer, int n_inner, hipStream_t s) {
    if (n_outer <= 0 || n_inner <= 0) return hipSuccess;
    if (!sq_fits(P, G.pad, G.bytes)) return hipErrorInvalidValue;
    if (!getenv_lane_off_sq()) {
        const hipError_t e = sp_launch_hier_encode_lane(P, G, src_k, dtype, so, si, dst_k, dout, n_outer, n_inner, s,
                                                        src_v, dst_v);
        if (e != hipErrorNotSupported) return e;
    }
    const hipError_t e = sp_launch_hier_encode(P, G, src_k, dtype, so, si, dst_k, dout, n_outer, n_inner, s);
    if (e != hipSuccess) return e;
    return sp_launch_hier_encode(P, G, src_v, dtype, so, si, dst_v, dout, n_outer, n_inner, s);
}

hipError_t sp_launch_hier_decode(const SpPlan &P, const SpHierGeo &G, const unsigned char *src,
                                 long long so, void *dst, int dtype, long long dout, long long din,
                                 int n_outer, int n_inner, hipStream_t s, const int *cells) {
    if (n_outer <= 0 || n_inner <= 0) return hipSuccess;
    if (!sq_fits(P, G.pad, G.bytes)) return hipErrorInvalidValue;
    if (!getenv_lane_off_sq()) {
        const hipError_t e = sp_launch_hier_decode_lane(P, G, src, so, dst, dtype, dout, din, n_outer, n_inner, s, cells);
        if (e != hipErrorNotSupported) return e;
    }
    const long long nv = (long long)n_outer * n_inner;
    const dim3 grid((unsigned)((nv + 3) / 4)), block(256);
    if (dtype == SP_DT_F16)
        hipLaunchKernelGGL((k_hier_decode<SP_DT_F16>), grid, block, 0, s, P, G, src, so, dst, dout, din, n_outer, n_inner, cells);
    else
        hipLaunchKernelGGL((k_hier_decode<SP_DT_F32>), grid, block, 0, s, P, G, src, so, dst, dout, din, n_outer, n_inner, cells);
    return hipGetLastError();
}
