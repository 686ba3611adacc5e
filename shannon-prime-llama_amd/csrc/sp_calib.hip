// sp_calib.hip -- calibration passes that feed the codec's tables (the
// reference's calibrate_begin / feed / end, kv_cache.cpp:515-751):
//   * per-coefficient first and second moments of the forward transform of a
//     batch of vectors (sqfree: of the padded vector), for the variance-ranked
//     coefficient order and Knight skeleton (the CUDA branch of
//     KvCache::calibrate_feed transforms on the device and accumulates sum and
//     sum of squares per coefficient, :553-585);
//   * per-slot Gram matrices of the hierarchical skeleton and targets, for the
//     least-squares predictor W (sp_hier_cache_calibrate_feed / _end, :590-607,
//     uploaded at :724-751).
// The transforms are the codec's own (sp_transform_lds with the cache's plan),
// so the statistics describe exactly the coefficients the encoder quantizes.
// Sums are fp64 in a fixed order (per wave, then partials in block order), so
// repeated runs give identical results.
#include "sp_internal.h"

namespace {

constexpr int CAL_WAVES = 4;  // one vector per wave, four per block

// Wave w of block b takes vectors (r * grid + b) * 4 + w for rounds r; every wave
// runs every round (the transform has block barriers), idle ones on zeros.
template <int DT>
__global__ void __launch_bounds__(256)
k_calib_moments(const SpPlan P, int hd, int tlen, const void *__restrict__ src, long long si, int n,
                double *__restrict__ partials) {
    __shared__ float c_s[CAL_WAVES][SP_GEN_MAX_N];
    constexpr int MAXK = SP_GEN_MAX_N / SP_WAVE;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *c = c_s[w];
    double s1[MAXK], s2[MAXK];
#pragma unroll
    for (int m = 0; m < MAXK; m++) s1[m] = s2[m] = 0.0;
    const long long per_round = (long long)gridDim.x * CAL_WAVES;
    const int rounds = (int)((n + per_round - 1) / per_round);
    for (int r = 0; r < rounds; r++) {
        const long long v = ((long long)r * gridDim.x + blockIdx.x) * CAL_WAVES + w;
        const bool valid = v < n;
        for (int k = lane; k < hd; k += SP_WAVE) c[k] = valid ? sp_load1<DT>(src, v * si + k) : 0.0f;
        __syncthreads();
        if (tlen > hd) {  // sqfree pad: the true mean, summed in the tree-256 order
            const float mean = sp_div(sp_wave_tree256_sum(c, hd, 0, lane), (float)hd);
            for (int k = hd + lane; k < tlen; k += SP_WAVE) c[k] = mean;
            __syncthreads();
        }
        sp_transform_lds(c, tlen, P, lane);
        if (valid) {
#pragma unroll
            for (int m = 0; m < MAXK; m++) {
                const int k = lane + SP_WAVE * m;
                if (k < tlen) {
                    const double x = (double)c[k];
                    s1[m] += x;
                    s2[m] += x * x;
                }
            }
        }
        __syncthreads();
    }
    double *out = partials + ((long long)blockIdx.x * CAL_WAVES + w) * 2 * tlen;
#pragma unroll
    for (int m = 0; m < MAXK; m++) {
        const int k = lane + SP_WAVE * m;
        if (k < tlen) {
            out[k] = s1[m];
            out[tlen + k] = s2[m];
        }
    }
}

// Hierarchical Gram matrices of one slot: entry e < nt*ns is G_ts[e / ns][e % ns]
// = sum t_i s_j, entry nt*ns + (i*ns + j) is G_ss[i][j] = sum s_i s_j, over the
// padded (true-mean fill, tree-256 order) and transformed vectors. Each thread
// keeps its entries e = tid + 256*m in registers; per round the four waves
// transform four vectors and every thread adds their products. Block partials
// go to partials[block][entries].
constexpr int GRAM_MAXM = 40;  // entries per thread: (300*30 + 30*30) / 256 < 40

template <int DT>
__global__ void __launch_bounds__(256)
k_calib_hier_gram(const SpPlan P, const SpHierGeo G, const void *__restrict__ src, long long si, int n,
                  double *__restrict__ partials) {
    __shared__ float c_s[CAL_WAVES][SP_GEN_MAX_N];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
    const int ns = G.n_skel, nt = G.n_target, n_ent = nt * ns + ns * ns;
    // this thread's entries as LDS coefficient index pairs
    int ia[GRAM_MAXM], ib[GRAM_MAXM];
    double acc[GRAM_MAXM];
#pragma unroll
    for (int m = 0; m < GRAM_MAXM; m++) {
        const int e = tid + 256 * m;
        int a = 0, b = 0;
        if (e < nt * ns) {
            a = G.target_idx[e / ns];
            b = G.skel_idx[e % ns];
        } else if (e < n_ent) {
            const int f = e - nt * ns;
            a = G.skel_idx[f / ns];
            b = G.skel_idx[f % ns];
        }
        ia[m] = a, ib[m] = b, acc[m] = 0.0;
    }
    const long long per_round = (long long)gridDim.x * CAL_WAVES;
    const int rounds = (int)((n + per_round - 1) / per_round);
    for (int r = 0; r < rounds; r++) {
        const long long v = ((long long)r * gridDim.x + blockIdx.x) * CAL_WAVES + w;
        const bool valid = v < n;
        float *c = c_s[w];
        for (int k = lane; k < G.hd; k += SP_WAVE) c[k] = valid ? sp_load1<DT>(src, v * si + k) : 0.0f;
        __syncthreads();
        const float mean = sp_div(sp_wave_tree256_sum(c, G.hd, 0, lane), (float)G.hd);
        for (int k = G.hd + lane; k < G.pad; k += SP_WAVE) c[k] = mean;
        __syncthreads();
        sp_transform_lds(c, G.pad, P, lane);
        const int nv = (int)min((long long)CAL_WAVES, (long long)n - ((long long)r * gridDim.x + blockIdx.x) * CAL_WAVES);
        for (int u = 0; u < nv; u++) {
            const float *cu = c_s[u];
#pragma unroll
            for (int m = 0; m < GRAM_MAXM; m++)
                if (tid + 256 * m < n_ent) acc[m] = fma((double)cu[ia[m]], (double)cu[ib[m]], acc[m]);
        }
        __syncthreads();
    }
    double *out = partials + (long long)blockIdx.x * n_ent;
#pragma unroll
    for (int m = 0; m < GRAM_MAXM; m++)
        if (tid + 256 * m < n_ent) out[tid + 256 * m] = acc[m];
}

// acc[e] += sum over blocks b (in order) of partials[b][e].
__global__ void __launch_bounds__(256)
k_calib_reduce(const double *__restrict__ partials, int n_blocks, int n_ent, double *__restrict__ acc) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= n_ent) return;
    double s = acc[e];
    for (int b = 0; b < n_blocks; b++) s += partials[(long long)b * n_ent + e];
    acc[e] = s;
}

}  // namespace

int sp_calib_moment_blocks(int n) {
    const int b = (n + CAL_WAVES - 1) / CAL_WAVES;
    return b < 1 ? 1 : (b > 256 ? 256 : b);
}

hipError_t sp_launch_calib_moments(const SpPlan &P, int hd, int tlen, const void *src, int dtype, long long si, int n,
                                   double *partials, int n_blocks, hipStream_t s) {
    if (tlen > SP_GEN_MAX_N || hd > tlen || n <= 0) return hipErrorInvalidValue;
    if (dtype == SP_DT_F16)
        hipLaunchKernelGGL(k_calib_moments<SP_DT_F16>, dim3(n_blocks), dim3(256), 0, s, P, hd, tlen, src, si, n, partials);
    else
        hipLaunchKernelGGL(k_calib_moments<SP_DT_F32>, dim3(n_blocks), dim3(256), 0, s, P, hd, tlen, src, si, n, partials);
    return hipGetLastError();
}

int sp_calib_gram_entries(int n_skel, int n_target) { return n_target * n_skel + n_skel * n_skel; }

hipError_t sp_launch_calib_hier_gram(const SpPlan &P, const SpHierGeo &G, const void *src, int dtype, long long si,
                                     int n, double *partials, int n_blocks, double *acc, hipStream_t s) {
    const int n_ent = sp_calib_gram_entries(G.n_skel, G.n_target);
    if (G.pad > SP_GEN_MAX_N || n <= 0 || n_ent > 256 * GRAM_MAXM) return hipErrorInvalidValue;
    if (dtype == SP_DT_F16)
        hipLaunchKernelGGL(k_calib_hier_gram<SP_DT_F16>, dim3(n_blocks), dim3(256), 0, s, P, G, src, si, n, partials);
    else
        hipLaunchKernelGGL(k_calib_hier_gram<SP_DT_F32>, dim3(n_blocks), dim3(256), 0, s, P, G, src, si, n, partials);
    hipLaunchKernelGGL(k_calib_reduce, dim3((n_ent + 255) / 256), dim3(256), 0, s, partials, n_blocks, n_ent, acc);
    return hipGetLastError();
}
