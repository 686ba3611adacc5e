// sp_hier_attn.hip -- fused decode attention over hierarchical-Vilenkin records
// (the hier cache's K and V arrays), any hier geometry.
//
// A hier record holds the skeleton coefficients (band-quantized) and the target
// coefficients as residual levels about the slot's linear prediction W * skel;
// the read path rebuilds c (pad coefficients) and returns V(c)[0, hd), V the
// length-pad Vilenkin transform (shannon_prime_hier.cu:490-571). V is symmetric
// and its own inverse, so nothing is ever reconstructed:
//   * with q~ = kq_scale * V(q zero-padded to pad) (once per query head),
//     q . K~_t = u . skel_t + q~_tgt . dev_t,   u = q~_skel + W^T q~_tgt,
//     and dev_t = (level_t - centre) * step_t, so a score is one dot product
//     with the skeleton values plus step_t * (q~_tgt . level_t - centre * sum q~_tgt);
//   * sum_t p_t V~_t = V(c)[0, hd) with c_skel = sum_t p_t skel_t and
//     c_tgt = W c_skel + sum_t p_t dev_t: the weighted sums stay in the record's
//     coefficient domain and one transform per query head finishes them.
// The 9000-term prediction W * skel is paid once per query head instead of once
// per position.
//
// Three launches per layer:
//   k_hier_attn_prep   one block per query head: q~ (LDS transform), u, q~_tgt, sum q~_tgt;
//   k_hier_attn_split  block (KV head, run): 256-position chunks of the run, one
//                      position per thread for the scores, an online softmax
//                      across the run's chunks, and the weighted coefficient sums
//                      of the V records;
//   k_hier_attn_merge  one block per query head: the runs' partials merged,
//                      c rebuilt and transformed.
// Residual levels of 2, 4 or 8 bits (RB) are read as 32-bit windows of the level
// stream (32 / RB levels per window, compile-time shifts): for the scores a
// thread walks its record's windows against q~_tgt (zero-padded to whole
// windows), and for V a thread owns one window of target coefficients for two
// query heads over a group of positions (the sums of the position groups meet
// in LDS at the end of the run). Other level widths take a bit-serial path.
#include "sp_internal.h"

#include <algorithm>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int NT = 256;      // threads per block
constexpr int CH = 256;      // positions per chunk
constexpr int MAX_G = 8;     // query heads per KV head
constexpr int MAX_COEF_PER_THREAD = (SP_GEN_MAX_N + NT - 1) / NT;

__host__ __device__ constexpr int r4(int x) { return (x + 3) & ~3; }
__host__ __device__ constexpr int r32(int x) { return (x + 31) & ~31; }

// Prepared query per head: [u (r4(ns)) | q~_tgt zero-padded to r32(nt) | sum q~_tgt, 0, 0, 0].
__host__ __device__ constexpr int prep_qt_off(int ns) { return r4(ns); }
__host__ __device__ constexpr int prep_sum_off(int ns, int nt) { return r4(ns) + r32(nt); }

// dst[i] = src[i] (i < n), 0 (n <= i < total): U loads per thread in flight at once.
template <typename T, int U>
__device__ __forceinline__ void copy_to_lds(T *dst, const T *__restrict__ src, int n, int total, int tid) {
    for (int i0 = tid; i0 < total; i0 += NT * U) {
        T v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * NT;
            v[u] = i < n ? src[i] : T(0);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * NT;
            if (i < total) dst[i] = v[u];
        }
    }
}

// REC_U * NT record dwords staged through registers by range-checked buffer loads
// (dwords past n read as 0), so neither the loads nor the LDS stores need a per-element
// test: the destination holds REC_U * NT dwords and takes them all, zeros included.
constexpr int REC_U = 26;  // covers a chunk of 256 records of up to 103 B, plus the readers' look-ahead
struct RecStage {
    uint32_t v[REC_U];
    __device__ void load(const uint32_t *__restrict__ src, int n, int tid) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, 4 * n, 0x00020000);
#pragma unroll
        for (int u = 0; u < REC_U; u++) v[u] = __builtin_amdgcn_raw_buffer_load_b32(r, 4 * (tid + u * NT), 0, 0);
    }
    __device__ void store(uint32_t *dst, int tid) const {
#pragma unroll
        for (int u = 0; u < REC_U; u++) dst[tid + u * NT] = v[u];
    }
};
// LDS bytes of the record staging for record length B: the chunk with its 32-byte
// slack, and at least the whole RecStage area.
__host__ __device__ constexpr int rec_stage_bytes(int B) {
    return (((CH * B + 32) + 15) & ~15) > 4 * REC_U * NT ? (((CH * B + 32) + 15) & ~15) : 4 * REC_U * NT;
}
constexpr int K_STAGE = REC_U;  // K record dwords per thread staged through registers (256 x 103 B chunks)
constexpr int W_Q = 5;       // 16-byte W loads (8 fp16 each) per merge thread: n_target * n_skel <= 10240
constexpr int W_DW = 20;     // W dwords (fp16 pairs) per prep thread staged through registers
constexpr int MERGE_RUNS_PER_THREAD = 4;  // runs per merge thread (n_runs <= 4 * NT)

// Record geometry of the split kernel: read from the call (GeoRt), or fixed at compile
// time (GeoCt: NB skeleton bands of SZ codes of BITS bits, band b's bytes at b *
// band_bytes, then the fp32 magnitude, then NTG 2-bit target levels), which turns the
// skeleton bit positions and the LDS offsets of the level windows into constants.
struct GeoRt {
    static constexpr bool ct = false;
    static constexpr int nb = 0, sz = 0, bits = 0, band_bytes = 0, skB = 0, ns = 0, nt = 0, B = 0;
};
template <int NB, int SZ, int BITS, int NTG>
struct GeoCt {
    static constexpr bool ct = true;
    static constexpr int nb = NB, sz = SZ, bits = BITS, band_bytes = 2 + (SZ * BITS + 7) / 8;
    static constexpr int skB = NB * band_bytes, ns = NB * SZ, nt = NTG, B = skB + 4 + (2 * NTG + 7) / 8;
};
using Geo330 = GeoCt<2, 15, 5, 300>;  // the default hier geometry at pad 330 (hd 256): 103-byte records

// 4 little-endian bytes at LDS byte offset o (any alignment) of a dword-aligned array.
__device__ __forceinline__ uint32_t lds_u32_at(const unsigned char *base, int o) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(base + (o & ~3));
    return __builtin_amdgcn_alignbit(w[1], w[0], 8u * (uint32_t)(o & 3));
}

// nbits (<= 8) bits at bit `bit` (0..7) of byte offset o.
__device__ __forceinline__ uint32_t lds_bits_at(const unsigned char *base, int o, int bit, int nbits) {
    return __builtin_amdgcn_ubfe(lds_u32_at(base, o), (uint32_t)bit, (uint32_t)nbits);
}

// N bits at bit `pos` (a constant after unrolling) of the dword array r.
template <int N, int W>
__device__ __forceinline__ uint32_t ct_field(const uint32_t (&r)[W], int pos) {
    const int w = pos >> 5, sh = pos & 31;
    if (sh + N <= 32) return __builtin_amdgcn_ubfe(r[w], (uint32_t)sh, (uint32_t)N);
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(r[w + 1], r[w], (uint32_t)sh), 0u, (uint32_t)N);
}

// LSB-first bit stream starting at byte offset o of a dword-aligned LDS array.
// The stream is read in 32-bit windows [32j, 32j + 32) through funnel shifts of
// aligned dwords, so every lane refills at the same code index whatever its start
// byte (the refill branch stays uniform). Reads up to 12 bytes past the stream.
struct LdsBits {
    const uint32_t *dw;
    uint32_t fs, prev;
    uint64_t buf;
    int nbits;
    __device__ LdsBits(const unsigned char *base, int o) {
        dw = reinterpret_cast<const uint32_t *>(base + (o & ~3));
        fs = 8u * (uint32_t)(o & 3);
        prev = dw[0];
        buf = win();
        buf |= (uint64_t)win() << 32;
        nbits = 64;
    }
    __device__ uint32_t win() {
        const uint32_t cur = dw[1];
        const uint32_t w = __builtin_amdgcn_alignbit(cur, prev, fs);
        prev = cur;
        dw++;
        return w;
    }
    __device__ uint32_t get(int bits) {
        if (nbits < bits) {
            buf |= (uint64_t)win() << nbits;
            nbits += 32;
        }
        const uint32_t v = (uint32_t)buf & ((1u << bits) - 1u);
        buf >>= bits;
        nbits -= bits;
        return v;
    }
};

// floor(a / d) for 0 <= a < 2^20 and 1 <= d < 2^10 from the float reciprocal of d:
// (a + 0.5) / d lies at least 1/(2d) from an integer, far beyond the rounding of the
// reciprocal and the product, so the truncation is exact (an integer division by a
// runtime divisor costs ~30 VALU instructions).
__device__ __forceinline__ int div_small(int a, float inv_d) { return (int)(((float)a + 0.5f) * inv_d); }

// One Vilenkin stage of radix p from src to dst (stride `stride`), one output
// element per thread: dst[e] = isp * sum_jj C[k][jj] src[base + jj*stride] for
// e = base + k*stride (the same sums, in the same order, as a whole group per
// thread, with p times the parallelism), the p x p cas matrix C read from LDS.
template <int p>
__device__ __forceinline__ void vil_stage(const float *src, float *dst, int n, int stride, const float *C, float isp,
                                          int tid) {
    const int block = stride * p;
    const float inv_block = 1.0f / (float)block, inv_stride = 1.0f / (float)stride;
    for (int e = tid; e < n; e += NT) {
        const int b0 = div_small(e, inv_block) * block, r = e - b0, k = div_small(r, inv_stride);
        const int base = b0 + (r - k * stride);
        float sum = 0.0f;
#pragma unroll
        for (int jj = 0; jj < p; jj++) sum += C[k * p + jj] * src[base + jj * stride];
        dst[e] = sum * isp;
    }
}

// The plan's cas tables, one entry per thread, loaded at kernel entry (so the load
// overlaps the kernel's other first loads) and stored to LDS before the transform.
static_assert(SP_CAS_TOTAL <= NT, "one cas entry per thread");
__device__ __forceinline__ float cas_entry(const SpPlan &P, int tid) { return tid < SP_CAS_TOTAL ? P.cas[tid] : 0.0f; }

// Transform of c[0, n) in LDS by the whole block (tmp: n more floats of LDS): the
// stages of sp_transform_lds (same arithmetic), ping-ponging between c and tmp, with
// this thread's cas entry (cas_entry) stored to LDS (cas_s, SP_CAS_TOTAL floats)
// first. The result ends in c. Ends with a barrier.
__device__ __forceinline__ void transform_block(float *c, float *tmp, int n, const SpPlan &P, float *cas_s, float cas_v,
                                                int tid) {
    if ((n & (n - 1)) == 0 || P.skip_transform) {
        sp_transform_lds(c, n, P, tid < SP_WAVE ? tid : n);
        __syncthreads();
        return;
    }
    if (tid < SP_CAS_TOTAL) cas_s[tid] = cas_v;
    __syncthreads();
    float *src = c, *dst = tmp;
    int stride = 1;
    for (int f = 0; f < P.n_factors; f++) {
        const int p = P.factors[f];
        const float *C = cas_s + sp_cas_off(p);
        const float isp = P.isp[sp_prime_idx(p)];
        switch (p) {
            case 2: vil_stage<2>(src, dst, n, stride, C, isp, tid); break;
            case 3: vil_stage<3>(src, dst, n, stride, C, isp, tid); break;
            case 5: vil_stage<5>(src, dst, n, stride, C, isp, tid); break;
            case 7: vil_stage<7>(src, dst, n, stride, C, isp, tid); break;
            default: vil_stage<11>(src, dst, n, stride, C, isp, tid); break;
        }
        stride *= p;
        __syncthreads();
        float *t = src;
        src = dst;
        dst = t;
    }
    if (src != c) {  // an odd number of stages
        for (int i = tid; i < n; i += NT) c[i] = src[i];
        __syncthreads();
    }
}

// Power of two p with amax * p in [2^11, 2^12) (1 when amax is 0 or not finite).
__device__ __forceinline__ float pow2_norm(float amax) {
    if (!(amax > 0.0f) || !(amax < INFINITY)) return 1.0f;
    int e;
    (void)frexpf(amax, &e);
    return ldexpf(1.0f, 12 - e);
}

// v + the value of lane ^ 1 (DPP quad permute [1,0,3,2]).
__device__ __forceinline__ float add_xor1(float v) {
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}

// v_perm_b32 selector taking bytes b and b + 1 (b < 4) of the dword pair (hi:lo) into
// bytes 1 and 3, zeros elsewhere (selector bytes 0-3 pick lo's bytes, 4-7 hi's, 0x0C
// gives zero).
__device__ __forceinline__ uint32_t level_bytes_sel(uint32_t b) { return 0x000C000Cu | (b << 8) | ((b + 1u) << 24); }

// Eight 2-bit levels held as byte 1 (levels 0-3 at bits 8 + 2e) and byte 3 (levels
// 4-7 at bits 24 + 2e) of x -> the A operand slots of v_mfma_f32_16x16x32_f16 as fp16
// 4 + level (exact): dword m takes levels m and m + 4 (slots 2m and 2m + 1), shifted
// to bits 8-9 and 24-25, with the exponent bits of 4.0 in both halves.
__device__ __forceinline__ half8_t level_quads2(uint32_t x) {
    u32x4 v;
#pragma unroll
    for (int m = 0; m < 4; m++) v[m] = __builtin_amdgcn_bitop3_b32(x >> (2 * m), 0x03000300u, 0x44004400u, 0xEA);
    return __builtin_bit_cast(half8_t, v);
}

typedef __attribute__((address_space(3))) const uint32_t lds_cu32;

// LDS byte address of p (a pointer into the kernel's shared memory) as a plain value:
// the compiler then folds constant offsets into the LDS reads instead of re-adding
// the shared array's address at every use.
__device__ __forceinline__ uint32_t lds_addr(const unsigned char *p) {
    uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)p;
    __asm__ volatile("" : "+v"(a));
    return a;
}

// The eight positions' fields of one V row-block operand: position e's field starts
// at bit sh[e] of the dword pair at LDS byte address ad[e] + off; all sixteen dwords
// are read before the funnel shifts, so the reads overlap.
__device__ __forceinline__ void vm_fields(const uint32_t (&ad)[8], const uint32_t (&sh)[8], uint32_t off,
                                          uint32_t (&x)[8]) {
    uint32_t d[8][2];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        lds_cu32 *w = (lds_cu32 *)(uintptr_t)(ad[e] + off);
        d[e][0] = w[0];
        d[e][1] = w[1];
    }
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = __builtin_amdgcn_alignbit(d[e][1], d[e][0], sh[e]);
}

// The dwords holding eight positions' 2-bit levels (a level's bit offset 8 * byte +
// 2 * coefficient is even, so it never crosses a dword).
__device__ __forceinline__ void vm_level_dwords(const uint32_t (&ad)[8], uint32_t off, uint32_t (&d)[8]) {
#pragma unroll
    for (int e = 0; e < 8; e++) d[e] = *(lds_cu32 *)(uintptr_t)(ad[e] + off);
}

// A operand of the V level sums (v_mfma_f32_16x16x32_f16, rows = coefficients, K =
// positions): the lane's 2-bit level at eight positions as fp16 level - 1.5 (exact).
// Positions m and m + 4 (slots 2m and 2m + 1) have their level at the same bit of their
// dwords d[m], d[m + 4] (their records are 4 record lengths apart, a whole number of
// dwords): a byte permute (selector sel[m]) takes the level's byte of each into bytes 1
// and 3, one shift by k[m] = bit % 8 puts the levels at bits 8-9 and 24-25, the and-or
// makes fp16 4 + level in both halves, and a packed subtract of 5.5 centres it (centring
// at the end of a run instead, from a weight sum, lost too much precision over long
// runs of positions).
__device__ __forceinline__ half8_t vm_levels(const uint32_t (&d)[8], const uint32_t (&sel)[4],
                                             const uint32_t (&k)[4]) {
    u32x4 v;
#pragma unroll
    for (int m = 0; m < 4; m++)
        v[m] = __builtin_amdgcn_bitop3_b32(__builtin_amdgcn_perm(d[m + 4], d[m], sel[m]) >> k[m], 0x03000300u,
                                           0x44004400u, 0xEA);
    return __builtin_bit_cast(half8_t, v) - (_Float16)5.5f;
}

// The same for a skeleton band's `bits`-bit codes (bits <= 8): fp16 2^bits + code from the
// code's byte (exponent bits `base`, the code shifted by 10 - bits under `mask`), minus
// `sub` = 2^bits + the band's offset (exact).
__device__ __forceinline__ half8_t vm_codes(const uint32_t (&ad)[8], const uint32_t (&sh)[8], uint32_t off,
                                            uint32_t sh10, uint32_t mask, uint32_t base, _Float16 sub) {
    uint32_t x[8];
    vm_fields(ad, sh, off, x);
    u32x4 v;
#pragma unroll
    for (int m = 0; m < 4; m++)
        v[m] = __builtin_amdgcn_bitop3_b32(__builtin_amdgcn_perm(x[2 * m + 1], x[2 * m], 0x0C040C00u) << sh10, mask,
                                           base, 0xEA);
    return __builtin_bit_cast(half8_t, v) - sub;
}

// wave reductions on DPP and the row swaps (every lane active at each call)
__device__ __forceinline__ float wave_sum(float v) { return sp_wave_sum_dpp(v); }
__device__ __forceinline__ float wave_max(float v) { return sp_wave_max_dpp(v); }

// ---------------------------------------------------------------------------
// Query preparation. Dynamic LDS: c[pad], qt[r32(n_target)], part[8][r4(n_skel)]
// floats, then the KV head's W [n_target][n_skel] fp16.
__global__ void __launch_bounds__(NT)
k_hier_attn_prep(const SpPlan P, const SpHierAttnArgs A, float *__restrict__ prep) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
    __shared__ float wsum[NT / SP_WAVE];
    __shared__ float cas_s[SP_CAS_TOTAL];
    __shared__ float tsm[SP_GEN_MAX_N];
    const int h = blockIdx.x, tid = threadIdx.x;  // query row h of n_seq * n_q
    const int G = A.n_q / A.n_kvh, kvh = (h % A.n_q) / G;
    const int ns = A.n_skel, nt = A.n_target, ns4 = r4(ns), nt32 = r32(nt);
    float *c = reinterpret_cast<float *>(dsm);
    float *qt = c + r4(A.pad);
    float *part = qt + nt32;
    unsigned short *Ws = reinterpret_cast<unsigned short *>(part + 8 * ns4);
    const unsigned short *Wk = reinterpret_cast<const unsigned short *>(A.W) + (long long)kvh * A.w_outer;
    // the query row, the target indices and W (as dwords of two fp16) all load at once
    // through range-checked buffer loads (unconditional: reads past a range return 0),
    // W reaching LDS while the query is transformed
    constexpr int PU = (SP_GEN_MAX_N + NT - 1) / NT;
    const bool has_w = A.W != nullptr;  // no predictor: u = q~_skel
    const int nw = has_w ? nt * ns : 0, nwd = nw >> 1;  // W dwords (an odd count's last half loads alone)
    const bool w_reg = nwd <= W_DW * NT && ((uintptr_t)Wk & 3) == 0;
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc((void *)(A.q + (long long)h * A.hd), (short)0, A.hd * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc((void *)A.tgt_idx, (short)0, nt * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)Wk, (short)0, nwd * 4, 0x00020000);
    float qv[PU];
    int ti[PU];
    const float cas_v = cas_entry(P, tid);
#pragma unroll
    for (int u = 0; u < PU; u++) {
        qv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, 4 * (tid + u * NT), 0, 0));
        ti[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(rt, 4 * (tid + u * NT), 0, 0);
    }
    uint32_t wd[W_DW];
    if (w_reg) {
#pragma unroll
        for (int u = 0; u < W_DW; u++) wd[u] = __builtin_amdgcn_raw_buffer_load_b32(rw, 4 * (tid + u * NT), 0, 0);
    } else if (has_w) {
        copy_to_lds<unsigned short, 16>(Ws, Wk, nw, nw, tid);
    }
#pragma unroll
    for (int u = 0; u < PU; u++)
        if (tid + u * NT < A.pad) c[tid + u * NT] = qv[u];  // zero past hd (out of range)
    __syncthreads();
    transform_block(c, tsm, A.pad, P, cas_s, cas_v, tid);
    if (w_reg) {
        uint32_t *Ws32 = reinterpret_cast<uint32_t *>(Ws);
#pragma unroll
        for (int u = 0; u < W_DW; u++)
            if (tid + u * NT < nwd) Ws32[tid + u * NT] = wd[u];
        if ((nw & 1) && tid == 0) Ws[nw - 1] = Wk[nw - 1];
    }
#pragma unroll
    for (int u = 0; u < (SP_GEN_MAX_N + NT - 1) / NT; u++) {
        const int t = tid + u * NT;
        if (t < nt32) qt[t] = t < nt ? A.kq_scale * c[ti[u]] : 0.0f;
    }
    __syncthreads();
    // W^T q~_tgt in 8 interleaved partial sums per skeleton coefficient (0 without W)
    for (int i = tid; i < 8 * ns; i += NT) {
        const int s = i % ns, g = i / ns;
        float acc = 0.0f;
        if (has_w) {
#pragma unroll 4
            for (int t = g; t < nt; t += 8) acc = fmaf(sp_f16_bits_to_f32(Ws[t * ns + s]), qt[t], acc);
        }
        part[g * ns4 + s] = acc;
    }
    __syncthreads();
    float *pr = prep + (long long)h * A.ps;
    for (int s = tid; s < ns4; s += NT) {
        float u = 0.0f;
        if (s < ns) {
            u = A.kq_scale * c[A.skel_idx[s]];
            for (int g = 0; g < 8; g++) u += part[g * ns4 + s];
        }
        pr[s] = u;
    }
    float qs = 0.0f;
    for (int t = tid; t < nt32; t += NT) {
        pr[ns4 + t] = qt[t];
        qs += qt[t];
    }
    qs = wave_sum(qs);
    if ((tid & 63) == 0) wsum[tid >> 6] = qs;
    __syncthreads();
    if (tid < 4) pr[prep_sum_off(ns, nt) + tid] = tid == 0 ? (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]) : 0.0f;
}

// ---------------------------------------------------------------------------
// Scores, softmax and the V records' weighted coefficient sums. Block
// (kvh, run) takes chunks run, run + n_runs, ... of KV head kvh. RB: residual
// level bits read as 32-bit windows (2, 4, 8), or 0 for the bit-serial path.
// Dynamic LDS (bytes, 16-aligned pieces):
//   rec   r16(CH * B + 32)  K, then V records of the chunk (dword-staged from a shift of
//                           0..3 bytes, then 12 zero bytes for the bit readers' look-ahead)
//   prep  G * ps floats     the G query heads' prepared queries
//   sc    G * CH floats     scores, then the softmax weights p
//   pw    G * CH floats     p * step (V targets)
//   psb   n_bands * G * CH  p * scale_b (V skeleton bands)
//   red   8 * MAX_G floats  block reductions
// (RB > 0: at the end of the run the same memory holds the position groups' sums.)
// Partial per (query head, run): [m, l, -, -, c_skel sum (n_skel), dev sum (n_target)].
// OUT = false: scores only (no V half), with the next chunk's K records prefetched
// into registers while the current chunk's scores run.
// VM (RB == 2, OUT): the V coefficient sums on the matrix cores instead of the window
// items. pw and psb then hold the weights as fp16 hi and lo rows ([h][hi, lo][CH] and
// [b][h][hi, lo][CH], the same bytes), scaled by a power of two per chunk; the sums
// need no position-group reduction at the end of the run.
template <int RB, int GM, bool OUT, bool VM, class GEO>
__global__ void __launch_bounds__(NT, 3)
k_hier_attn_split(const SpPlan P, const SpHierAttnArgs A0, const SpSeqTab T, const float *__restrict__ prep0,
                  float *__restrict__ part0, int n_runs) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
    const int kvh = blockIdx.x, run = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // sequence blockIdx.z: its positions, prepared queries, partials and score rows
    const int seq = blockIdx.z;
    SpHierAttnArgs A = A0;
    A.kcache += (long long)T.start[seq] * A0.B;
    A.vcache += (long long)T.start[seq] * A0.B;
    A.n_kv = T.len[seq];
    const long long s_stride = T.len[seq];
    if (A0.scores) A.scores += T.soff[seq];
    const float *__restrict__ prep = prep0 + (long long)seq * A0.n_q * A0.ps;
    float *__restrict__ part = part0 + (long long)seq * A0.n_q * n_runs * A0.pp;
    const int G = A.n_q / A.n_kvh, h0 = kvh * G;
    const int ns = GEO::ct ? GEO::ns : A.n_skel, nt = GEO::ct ? GEO::nt : A.n_target;
    const int B = GEO::ct ? GEO::B : A.B, nb = GEO::ct ? GEO::nb : P.n_bands;
    // band b's layout (constants for a compile-time geometry)
    auto band_bits = [&](int b) { return GEO::ct ? GEO::bits : (int)P.band_bits[b]; };
    auto band_off = [&](int b) { return GEO::ct ? b * GEO::sz : (int)P.band_off[b]; };
    auto band_sz = [&](int b) { return GEO::ct ? GEO::sz : (int)P.band_sz[b]; };
    auto band_byte_off = [&](int b) { return GEO::ct ? b * GEO::band_bytes : (int)P.band_byte_off[b]; };
    const int qo = prep_qt_off(ns), so = prep_sum_off(ns, nt);
    constexpr bool want_out = OUT;
    const int rec_bytes = rec_stage_bytes(B);
    unsigned char *rec = dsm;
    uint32_t *rec32 = reinterpret_cast<uint32_t *>(dsm);
    float *prep_s = reinterpret_cast<float *>(dsm + rec_bytes);
    float *sc = prep_s + G * A.ps;
    float *pw = sc + G * CH;
    float *psb = pw + G * CH;
    float *red = psb + nb * G * CH;
    const int skB = GEO::ct ? GEO::skB : P.total_bytes;
    const int Lv = 1 << A.rbits;
    const float step_div = (float)(Lv - 1);
    const float centre = sp_div((float)(Lv - 1), 2.0f);

    copy_to_lds<float, 4>(prep_s, prep + (long long)h0 * A.ps, G * A.ps, G * A.ps, tid);

    // RB == 2: the target dots run on v_mfma_f32_16x16x32_f16 with the levels as the A
    // operand (rows = positions, fp16 4 + level) and q~_tgt as B: column c16 = (head
    // c16 >> 1, hi / lo fp16 part c16 & 1) of q~_tgt scaled by a power of two per head.
    // bq[j][q4][c16]: the 8 B-operand halves of levels 32 j + 8 q4 + e, e < 8, in the
    // A operand's order (slot 2 (e & 3) + (e >> 2): levels e and e + 4 share a dword);
    // cin[c16]: the accumulator start -(4 + centre) * (column sum), which centres the
    // levels; unh: the inverse scale. The skeleton bands stay on the position threads.
    constexpr bool KM = RB == 2;
    const int n_kb = r32(nt) / 32;
    u32x4 *bq = reinterpret_cast<u32x4 *>(red + 8 * MAX_G);
    float *cin = reinterpret_cast<float *>(bq + n_kb * 64);
    float *unh = cin + 16;
    float *fh = unh + 16;
    float *psum = fh + 8;
    if (KM) {
        __syncthreads();
        for (int h = wv; h < G; h += NT / SP_WAVE) {
            float am = 0.0f;
            for (int kk = lane; kk < nt; kk += SP_WAVE) am = fmaxf(am, fabsf(prep_s[h * A.ps + qo + kk]));
            am = wave_max(am);
            if (lane == 0) fh[h] = pow2_norm(am);
        }
        __syncthreads();
        unsigned short *bqh = reinterpret_cast<unsigned short *>(bq);
        const int c16 = tid & 15, hq = c16 >> 1;
        float colsum = 0.0f;
        for (int kk = tid >> 4; kk < n_kb * 32; kk += NT / 16) {
            const float v = hq < G ? prep_s[hq * A.ps + qo + kk] * fh[hq] : 0.0f;
            const _Float16 hi = (_Float16)v;
            const _Float16 lo = (_Float16)(v - (float)hi);
            const _Float16 x = (c16 & 1) ? lo : hi;
            colsum += (float)x;
            bqh[(((kk >> 5) * 4 + ((kk >> 3) & 3)) * 16 + c16) * 8 + 2 * (kk & 3) + ((kk >> 2) & 1)] =
                __builtin_bit_cast(unsigned short, x);
        }
        psum[(tid >> 4) * 16 + c16] = colsum;
        __syncthreads();
        if (tid < 16) {
            float sum = 0.0f;
            for (int g = 0; g < 16; g++) sum += psum[g * 16 + tid];
            cin[tid] = -(4.0f + centre) * sum;
            unh[tid] = (tid >> 1) < G ? 1.0f / fh[tid >> 1] : 0.0f;
        }
        // the chunk loop's first barrier orders these before their use
    }

    // compile-time geometry: each skeleton band's query sum per head (identical in every
    // thread; prep_s is visible after the matrix-core setup's barriers)
    static_assert(!GEO::ct || KM, "the compile-time geometry has 2-bit levels");
    float qsk[GM][GEO::ct ? GEO::nb : 1];
    if constexpr (GEO::ct) {
#pragma unroll
        for (int h = 0; h < GM; h++)
#pragma unroll
            for (int b = 0; b < GEO::nb; b++) {
                float t = 0.0f;
                if (h < G)
                    for (int i = 0; i < GEO::sz; i++) t += prep_s[h * A.ps + b * GEO::sz + i];
                qsk[h][b] = t;
            }
    }

    // running softmax state per head (identical in every thread)
    float m_run[GM], l_run[GM];
#pragma unroll
    for (int h = 0; h < GM; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
    }
    // V sums. Bit-serial path: coefficient j = tid + NT * r (skeleton first, then targets)
    // for every head. Window path: one target window (32 / RB coefficients) and one
    // skeleton coefficient, each for head pair (2 hp, 2 hp + 1), over a group of positions.
    constexpr int LPW = RB > 0 ? 32 / RB : 1;
    constexpr uint32_t LMASK = RB > 0 ? (1u << RB) - 1u : 1u;
    constexpr int NCOEF = RB > 0 ? 1 : MAX_COEF_PER_THREAD;
    float acc[NCOEF][GM];
    float tacc[LPW][2], twsum[2], sacc[2];
#pragma unroll
    for (int r = 0; r < NCOEF; r++)
#pragma unroll
        for (int h = 0; h < GM; h++) acc[r][h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        twsum[j] = sacc[j] = 0.0f;
#pragma unroll
        for (int k = 0; k < LPW; k++) tacc[k][j] = 0.0f;
    }
    const int n_win = RB > 0 ? (nt * RB + 31) / 32 : 1;
    const int n_hp = (G + 1) / 2;
    const int t_items = n_win * n_hp, s_items = ns * n_hp;
    const int npg_t = max(1, NT / t_items), npg_s = max(1, NT / s_items);
    const bool t_on = tid < t_items * npg_t, s_on = tid < s_items * npg_s;
    const int t_item = tid % t_items, t_pg = tid / t_items, t_w = t_item % n_win, t_hp = t_item / n_win;
    const int s_item = tid % s_items, s_pg = tid / s_items, s_s = s_item % ns, s_hp = s_item / ns;
    const int t_ha = 2 * t_hp, t_hb = min(2 * t_hp + 1, G - 1);
    const int s_ha = 2 * s_hp, s_hb = min(2 * s_hp + 1, G - 1);
    int s_b = 0;
    while (s_b + 1 < nb && s_s >= band_off(s_b + 1)) s_b++;
    const int s_bits = band_bits(s_b), s_bo = (s_s - band_off(s_b)) * s_bits;
    const int s_byte = band_byte_off(s_b) + 2 + (s_bo >> 3), s_bit = s_bo & 7;
    const float s_off = (float)((1 << (s_bits - 1)) - 1);

    // VM: row blocks of 16 coefficients. Target window wv + 4 i (i < VM_TB) belongs to
    // wave wv: every wave runs VM_TB of them (the launcher takes 4 VM_TB - 3 .. 4 VM_TB
    // windows; a window past the last reads the record tail and is never written out).
    // The skeleton bands in blocks of 16 follow: block k to wave (n_win + k) % 4, at most
    // one per wave (the launcher checks). Sums per (coefficient, column) in the
    // v_mfma_f32_16x16x32_f16 accumulator layout, kept across the chunks: lane = column
    // (head jc >> 1, hi / lo part jc & 1) of rows 4 kq .. 4 kq + 3.
    constexpr int VM_TB = 5;
    int vm_nsb = 0;
    if (VM)
        for (int b = 0; b < nb; b++) vm_nsb += (band_sz(b) + 15) >> 4;
    // this wave's skeleton block (vm_s), band vm_b, coefficients 16 vm_k ..
    bool vm_s = false;
    int vm_b = 0, vm_k = 0;
    if (VM) {
        int sb = ((wv - n_win) % 4 + 4) % 4;
        if (sb < vm_nsb) {
            vm_s = true;
            while (vm_b + 1 < nb && sb >= ((band_sz(vm_b) + 15) >> 4)) sb -= (band_sz(vm_b++) + 15) >> 4;
            vm_k = sb;
        }
    }
    float4_t vacc[VM ? VM_TB : 1], vsk = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < (VM ? VM_TB : 1); i++) vacc[i] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int n_chunks = (A.n_kv + CH - 1) / CH;
    // scores only: chunk ch's K records wait in registers (kst) from the previous chunk on
    // (the staging's reads cover ndw + 3 dwords: the records and the readers' look-ahead)
    const bool k_pre = !OUT && (CH * B + 6) / 4 + 3 <= REC_U * NT;
    const bool rec_fast = (CH * B + 6) / 4 + 3 <= REC_U * NT;  // one RecStage covers a chunk
    RecStage kst;
    auto k_src = [&](int chn, int &shift_, int &ndw_) {
        const int c0_ = chn * CH, n_t_ = min(CH, A.n_kv - c0_);
        const unsigned char *kg_ = A.kcache + (long long)kvh * A.slot_bytes + (long long)c0_ * B;
        shift_ = (int)((uintptr_t)kg_ & 3);
        ndw_ = (n_t_ * B + shift_ + 3) >> 2;
        return reinterpret_cast<const uint32_t *>(kg_ - shift_);
    };
    if (k_pre && run < n_chunks) {
        int sh_, nd_;
        const uint32_t *src_ = k_src(run, sh_, nd_);
        kst.load(src_, nd_, tid);
    }
    for (int ch = run; ch < n_chunks; ch += n_runs) {
        const int c0 = ch * CH;
        const int n_t = min(CH, A.n_kv - c0);
        // ---- K records of the chunk into LDS (aligned dwords; records from byte `shift`) ----
        int shift, ndw;
        const uint32_t *ksrc = k_src(ch, shift, ndw);
        __syncthreads();  // the previous chunk is done with rec / sc
        if (k_pre) {
            kst.store(rec32, tid);  // zeros past the records: the bit readers' look-ahead
            if (ch + n_runs < n_chunks) {
                int sh_, nd_;
                const uint32_t *src_ = k_src(ch + n_runs, sh_, nd_);
                kst.load(src_, nd_, tid);
            }
        } else if (rec_fast) {
            RecStage st;
            st.load(ksrc, ndw, tid);
            st.store(rec32, tid);
        } else {
            copy_to_lds<uint32_t, 32>(rec32, ksrc, ndw, ndw + 3, tid);
        }
        __syncthreads();
        if (KM) {
            // ---- target dots of this wave's 64 positions on the matrix cores -> sc ----
            const int r = lane & 15, q4 = lane >> 4;
            const float ci = cin[r], un = unh[r];
            const bool wr = !(r & 1) && (r >> 1) < G;
            const uint32_t rec_k = lds_addr(rec);
#pragma unroll
            for (int sub = 0; sub < 4; sub++) {
                const int pos0 = 64 * wv + 16 * sub;
                float4_t acc = {ci, ci, ci, ci};
                // the lane's 16 level bits of window j start at byte ob + 8 j: a byte permute
                // with a per-lane selector takes those two bytes of the aligned dword pair
                const int ob = shift + (pos0 + r) * B + skB + 4 + 2 * q4;
                const uint32_t ka = rec_k + (uint32_t)(ob & ~3);
                const uint32_t ksel = level_bytes_sel((uint32_t)ob & 3u);
                constexpr int KJ_UNROLL = GEO::ct ? 32 : 1;  // constant window offsets when unrolled
#pragma unroll KJ_UNROLL
                for (int j = 0; j < n_kb; j++) {
                    lds_cu32 *w = (lds_cu32 *)(uintptr_t)(ka + 8u * (uint32_t)j);
                    const half8_t code = level_quads2(__builtin_amdgcn_perm(w[1], w[0], ksel));
                    const half8_t bv = __builtin_bit_cast(half8_t, bq[(j * 4 + q4) * 16 + r]);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(code, bv, acc, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float v = add_xor1(acc[i]) * un;  // hi + lo columns
                    if (wr) sc[(r >> 1) * CH + pos0 + 4 * q4 + i] = v;
                }
            }
            __asm__ volatile("" ::: "memory");  // the wave's position threads read sc next
        }
        // ---- scores: thread = position ----
        if (tid < n_t) {
            const int rb = shift + tid * B;
            // compile-time geometry: the record's skeleton bytes and magnitude as dwords
            // aligned to the record's start (rsk[k] = record bytes 4k .. 4k + 3)
            constexpr int SKW = GEO::ct ? (GEO::skB + 4 + 3) / 4 : 1;
            uint32_t rsk[SKW];
            if constexpr (GEO::ct) {
                lds_cu32 *w = (lds_cu32 *)(uintptr_t)(lds_addr(rec) + (uint32_t)(rb & ~3));
                uint32_t d[SKW + 1];
#pragma unroll
                for (int k = 0; k <= SKW; k++) d[k] = w[k];
                const uint32_t fs = 8u * (uint32_t)(rb & 3);
#pragma unroll
                for (int k = 0; k < SKW; k++) rsk[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], fs);
            }
            const float mag = __uint_as_float(GEO::ct ? rsk[SKW - 1] : lds_u32_at(rec, rb + skB));
            const float step = sp_div(2.0f * mag, step_div);
            for (int hp = 0; hp < G; hp += 2) {
                const int ha = hp, hb = hp + 1 < G ? hp + 1 : hp;
                const float *ua = prep_s + ha * A.ps, *ub = prep_s + hb * A.ps;
                float s0 = 0.0f, s1 = 0.0f;
                if constexpr (GEO::ct) {
                    // codes at constant bits; the offset 2^(bits-1) - 1 comes off as that
                    // times the band's query sum (qsk)
                    constexpr int maxv = (1 << (GEO::bits - 1)) - 1;
#pragma unroll
                    for (int b = 0; b < GEO::nb; b++) {
                        const float scale = sp_scale_from_bits(ct_field<16>(rsk, 8 * b * GEO::band_bytes));
                        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                        for (int i = 0; i < GEO::sz; i++) {
                            const float cv = (float)ct_field<GEO::bits>(rsk, 8 * (b * GEO::band_bytes + 2) + GEO::bits * i);
                            a0 = fmaf(ua[b * GEO::sz + i], cv, a0);
                            a1 = fmaf(ub[b * GEO::sz + i], cv, a1);
                        }
                        a0 = fmaf(-(float)maxv, qsk[ha][b], a0);
                        a1 = fmaf(-(float)maxv, qsk[hb][b], a1);
                        s0 = fmaf(scale, a0, s0);
                        s1 = fmaf(scale, a1, s1);
                    }
                } else
                for (int b = 0; b < nb; b++) {
                    const int bits = band_bits(b), off = band_off(b), sz = band_sz(b);
                    const int maxv = (1 << (bits - 1)) - 1;
                    const float scale = sp_scale_from_bits(lds_u32_at(rec, rb + band_byte_off(b)) & 0xffffu);
                    LdsBits br(rec, rb + band_byte_off(b) + 2);
                    float a0 = 0.0f, a1 = 0.0f;
                    for (int i = 0; i < sz; i++) {
                        const float cv = (float)((int)br.get(bits) - maxv);
                        a0 = fmaf(ua[off + i], cv, a0);
                        a1 = fmaf(ub[off + i], cv, a1);
                    }
                    s0 = fmaf(scale, a0, s0);
                    s1 = fmaf(scale, a1, s1);
                }
                float d0 = 0.0f, d1 = 0.0f;
                if (KM) {
                    d0 = sc[ha * CH + tid] + centre * ua[so];  // centred on the matrix cores
                    d1 = sc[hb * CH + tid] + centre * ub[so];
                } else if (RB > 0) {
                    // window w of the level stream against q~_tgt[w * LPW ..] (zero past n_target)
                    const int o = rb + skB + 4;
                    const uint32_t *dw = reinterpret_cast<const uint32_t *>(rec + (o & ~3));
                    const uint32_t fs = 8u * (uint32_t)(o & 3);
                    uint32_t prev = dw[0];
                    for (int w = 0; w < n_win; w++) {
                        const uint32_t cur = dw[w + 1];
                        const uint32_t win = __builtin_amdgcn_alignbit(cur, prev, fs);
                        prev = cur;
                        const float *qa = ua + qo + w * LPW, *qb = ub + qo + w * LPW;
#pragma unroll
                        for (int k = 0; k < LPW; k++) {
                            const float lv = (float)((win >> (k * RB)) & LMASK);
                            d0 = fmaf(qa[k], lv, d0);
                            d1 = fmaf(qb[k], lv, d1);
                        }
                    }
                } else {
                    LdsBits br(rec, rb + skB + 4);
                    for (int t = 0; t < nt; t++) {
                        const float lv = (float)br.get(A.rbits);
                        d0 = fmaf(ua[qo + t], lv, d0);
                        d1 = fmaf(ub[qo + t], lv, d1);
                    }
                }
                s0 = fmaf(step, d0 - centre * ua[so], s0);
                s1 = fmaf(step, d1 - centre * ub[so], s1);
                sc[ha * CH + tid] = s0;
                if (hb != ha) sc[hb * CH + tid] = s1;
                if (A.scores) {
                    A.scores[(long long)(h0 + ha) * s_stride + c0 + tid] = s0;
                    if (hb != ha) A.scores[(long long)(h0 + hb) * s_stride + c0 + tid] = s1;
                }
            }
        }
        if (!want_out) continue;
        __syncthreads();
        // ---- online softmax over the chunk (per head: block max, then block sum) ----
        float alpha[GM];
        {
            float mx[GM];
#pragma unroll
            for (int h = 0; h < GM; h++) mx[h] = (h < G && tid < n_t) ? sc[h * CH + tid] : -INFINITY;
#pragma unroll
            for (int h = 0; h < GM; h++) {
                if (h < G) {
                    const float v = wave_max(mx[h]);
                    if (lane == 0) red[wv * MAX_G + h] = v;
                }
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < GM; h++) {
                if (h < G) {
                    const float cm = fmaxf(fmaxf(red[h], red[MAX_G + h]), fmaxf(red[2 * MAX_G + h], red[3 * MAX_G + h]));
                    const float mn = fmaxf(m_run[h], cm);
                    alpha[h] = __expf(m_run[h] - mn);
                    m_run[h] = mn;
                } else {
                    alpha[h] = 1.0f;
                }
            }
            float pl[GM];
#pragma unroll
            for (int h = 0; h < GM; h++) {
                const float p = (h < G && tid < n_t) ? __expf(sc[h * CH + tid] - m_run[h]) : 0.0f;
                if (h < G) sc[h * CH + tid] = p;
                pl[h] = p;
            }
#pragma unroll
            for (int h = 0; h < GM; h++) {
                if (h < G) {
                    const float v = wave_sum(pl[h]);
                    if (lane == 0) red[4 * MAX_G + wv * MAX_G + h] = v;
                }
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < GM; h++) {
                if (h < G) {
                    const float *rs = red + 4 * MAX_G;
                    l_run[h] = fmaf(l_run[h], alpha[h], (rs[h] + rs[MAX_G + h]) + (rs[2 * MAX_G + h] + rs[3 * MAX_G + h]));
                }
            }
        }
        // ---- V records of the chunk; per position: p * step and p * scale_b ----
        const unsigned char *vg = A.vcache + (long long)kvh * A.slot_bytes + (long long)c0 * B;
        const int vshift = (int)((uintptr_t)vg & 3);
        const int vdw = (n_t * B + vshift + 3) >> 2;
        if (rec_fast) {
            RecStage st;
            st.load(reinterpret_cast<const uint32_t *>(vg - vshift), vdw, tid);
            st.store(rec32, tid);
        } else {
            copy_to_lds<uint32_t, 32>(rec32, reinterpret_cast<const uint32_t *>(vg - vshift), vdw, vdw + 3, tid);
        }
        __syncthreads();
        if constexpr (VM) {
            // ---- weights as fp16 hi + lo rows, scaled by f (a power of two putting the
            // chunk's largest step or band scale in [2^11, 2^12); every p <= 1) ----
            const int rb = vshift + tid * B;
            const bool live = tid < n_t;
            const float vstep = live ? sp_div(2.0f * __uint_as_float(lds_u32_at(rec, rb + skB)), step_div) : 0.0f;
            float wmax = vstep;
            for (int b = 0; b < nb; b++)
                if (live) wmax = fmaxf(wmax, sp_scale_from_bits(lds_u32_at(rec, rb + band_byte_off(b)) & 0xffffu));
            wmax = wave_max(wmax);
            if (lane == 0) red[wv] = wmax;
            __syncthreads();
            const float f = pow2_norm(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
            _Float16 *pwq = reinterpret_cast<_Float16 *>(pw);
            _Float16 *psq = reinterpret_cast<_Float16 *>(psb);
            // target weights in the level operand's position order: within each group of
            // eight, position e at slot 2 (e & 3) + (e >> 2)
            const int wslot = (tid & ~7) | (2 * (tid & 3)) | ((tid >> 2) & 1);
            for (int h = 0; h < G; h++) {
                const float v = sc[h * CH + tid] * vstep * f;
                const _Float16 hi = (_Float16)v;
                pwq[(2 * h) * CH + wslot] = hi;
                pwq[(2 * h + 1) * CH + wslot] = (_Float16)(v - (float)hi);
            }
            for (int b = 0; b < nb; b++) {
                const float scale =
                    live ? sp_scale_from_bits(lds_u32_at(rec, rb + band_byte_off(b)) & 0xffffu) : 0.0f;
                for (int h = 0; h < G; h++) {
                    const float v = sc[h * CH + tid] * scale * f;
                    const _Float16 hi = (_Float16)v;
                    psq[((b * G + h) * 2) * CH + tid] = hi;
                    psq[((b * G + h) * 2 + 1) * CH + tid] = (_Float16)(v - (float)hi);
                }
            }
            __syncthreads();
            // ---- the wave's row blocks over the chunk's 32-position groups: rows =
            // coefficients (lane jc of the block), K = positions 8 kq .. 8 kq + 7 of the
            // group, columns = (head, hi / lo) ----
            const int jc = lane & 15, kq = lane >> 4;
            float ac = 1.0f;  // the column's alpha, times f: the run's sums rescaled to this chunk
#pragma unroll
            for (int h = 0; h < GM; h++)
                if (h == (jc >> 1)) ac = alpha[h];
            ac *= f;
#pragma unroll
            for (int i = 0; i < VM_TB; i++) vacc[i] *= ac;
            vsk *= ac;
            // dword address of each K position's first row-block field at group 0 (the
            // groups step by 32 B bytes, a whole number of dwords), and for the level
            // windows the byte permute and shift of the position pairs (m, m + 4)
            uint32_t ta[8], tsel[4], tk[4], sa[8], ssh[8];
            const uint32_t rec_lds = lds_addr(rec);
            const int vbits = band_bits(vm_b);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int p0 = vshift + (8 * kq + e) * B;
                const int tb = 8 * (p0 + skB + 4 + 4 * wv) + 2 * jc;
                ta[e] = rec_lds + ((uint32_t)(tb >> 5) << 2);
                if (e < 4) {
                    const uint32_t bsel = ((uint32_t)tb & 31u) >> 3;
                    tsel[e] = 0x000C000Cu | (bsel << 8) | ((4u + bsel) << 24);
                    tk[e] = (uint32_t)tb & 7u;
                }
                const int sbp = 8 * (p0 + band_byte_off(vm_b) + 2) + vbits * (16 * vm_k + jc);
                sa[e] = rec_lds + ((uint32_t)(sbp >> 5) << 2);
                ssh[e] = (uint32_t)sbp & 31u;
                if (GEO::ct) {
                    if (e < 4) {
                        // one register per address pair: the unrolled groups' reads add constants
                        __asm__ volatile("" : "+v"(ta[e]), "+v"(sa[e]));
                    } else {
                        // position e - 4's fields lie 4 records (B dwords) earlier at the same bits
                        ta[e] = ta[e - 4] + 4u * GEO::B;
                        sa[e] = sa[e - 4] + 4u * GEO::B;
                    }
                }
            }
            const uint32_t sh10 = 10u - (uint32_t)vbits;
            const uint32_t smask = (((1u << vbits) - 1u) << sh10) * 0x00010001u;
            const uint32_t sbase = ((15u + (uint32_t)vbits) << 10) * 0x00010001u;
            const _Float16 ssub = (_Float16)(float)((1 << vbits) + (1 << (vbits - 1)) - 1);
            const bool col_on = jc < 2 * G;
            // columns past the heads read a live column's weights (finite values whose sums
            // are never written out), so every lane loads without a branch
            const int jr = col_on ? jc : jc & 1;
            const _Float16 *btrow = pwq + jr * CH;
            const _Float16 *bsrow = psq + ((vm_b * G + (jr >> 1)) * 2 + (jr & 1)) * CH;
            const int ng = (n_t + 31) >> 5;
            const uint32_t gstep = 32u * (uint32_t)B;  // bytes per group: the addresses advance in place
            // group g's fields sit goff bytes past group 0's
            auto group = [&](int g, uint32_t goff) {
                const int pq = 32 * g + 8 * kq;
                const half8_t bt = *reinterpret_cast<const half8_t *>(btrow + pq);
                if (vm_s) {
                    const half8_t bsk = *reinterpret_cast<const half8_t *>(bsrow + pq);
                    const half8_t a = vm_codes(sa, ssh, goff, sh10, smask, sbase, ssub);
                    vsk = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bsk, vsk, 0, 0, 0);
                }
                // window i + 1's dwords are read while window i converts
                uint32_t dw[2][8];
                vm_level_dwords(ta, goff, dw[0]);
#pragma unroll
                for (int i = 0; i < VM_TB; i++) {
                    if (i + 1 < VM_TB) vm_level_dwords(ta, goff + 16u * (i + 1), dw[(i + 1) & 1]);
                    const half8_t a = vm_levels(dw[i & 1], tsel, tk);
                    vacc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bt, vacc[i], 0, 0, 0);
                }
            };
            if constexpr (GEO::ct) {
                // every group's offsets are constants: the LDS reads carry them
#pragma unroll
                for (int g = 0; g < CH / 32; g++)
                    if (g < ng) group(g, (uint32_t)(g * 32 * GEO::B));
            } else {
                for (int g = 0; g < ng; g++) {
                    group(g, 0u);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        ta[e] += gstep;
                        sa[e] += gstep;
                    }
                }
            }
            const float inv_f = 1.0f / f;  // exact: f is a power of two
#pragma unroll
            for (int i = 0; i < VM_TB; i++) vacc[i] *= inv_f;
            vsk *= inv_f;
            continue;
        }
        {
            const int rb = vshift + tid * B;
            const bool live = tid < n_t;
            const float vstep = live ? sp_div(2.0f * __uint_as_float(lds_u32_at(rec, rb + skB)), step_div) : 0.0f;
            for (int h = 0; h < G; h++) pw[h * CH + tid] = sc[h * CH + tid] * vstep;
            for (int b = 0; b < nb; b++) {
                const float scale =
                    live ? sp_scale_from_bits(lds_u32_at(rec, rb + band_byte_off(b)) & 0xffffu) : 0.0f;
                for (int h = 0; h < G; h++) psb[(b * G + h) * CH + tid] = sc[h * CH + tid] * scale;
            }
        }
        __syncthreads();
        if (RB > 0) {
            // ---- window sums: target window t_w and skeleton coefficient s_s for a head pair ----
            float fa = 1.0f, fb = 1.0f, ga = 1.0f, gb = 1.0f;
#pragma unroll
            for (int h = 0; h < GM; h++) {
                if (h == t_ha) fa = alpha[h];
                if (h == t_hb) fb = alpha[h];
                if (h == s_ha) ga = alpha[h];
                if (h == s_hb) gb = alpha[h];
            }
            twsum[0] *= fa;
            twsum[1] *= fb;
#pragma unroll
            for (int k = 0; k < LPW; k++) {
                tacc[k][0] *= fa;
                tacc[k][1] *= fb;
            }
            sacc[0] *= ga;
            sacc[1] *= gb;
            if (t_on) {
                const int wo = skB + 4 + 4 * t_w;
#pragma unroll 2
                for (int t = t_pg; t < n_t; t += npg_t) {
                    const uint32_t win = lds_u32_at(rec, vshift + t * B + wo);
                    const float wa = pw[t_ha * CH + t], wb = pw[t_hb * CH + t];
                    twsum[0] += wa;
                    twsum[1] += wb;
#pragma unroll
                    for (int k = 0; k < LPW; k++) {
                        const float lv = (float)((win >> (k * RB)) & LMASK);
                        tacc[k][0] = fmaf(wa, lv, tacc[k][0]);
                        tacc[k][1] = fmaf(wb, lv, tacc[k][1]);
                    }
                }
            }
            if (s_on) {
                const float *wa_row = psb + (s_b * G + s_ha) * CH, *wb_row = psb + (s_b * G + s_hb) * CH;
#pragma unroll 4
                for (int t = s_pg; t < n_t; t += npg_s) {
                    const float cv = (float)lds_bits_at(rec, vshift + t * B + s_byte, s_bit, s_bits) - s_off;
                    sacc[0] = fmaf(wa_row[t], cv, sacc[0]);
                    sacc[1] = fmaf(wb_row[t], cv, sacc[1]);
                }
            }
        } else {
            // ---- bit-serial path: coefficient j = tid + NT*r, positions of the chunk in order ----
#pragma unroll
            for (int r = 0; r < NCOEF; r++) {
#pragma unroll
                for (int h = 0; h < GM; h++) acc[r][h] *= alpha[h];
                const int j = tid + NT * r;
                if (j >= ns + nt) continue;
                int byte0, bit0, bits;
                float offv;
                const float *wrow;
                if (j < ns) {
                    int b = 0;
                    while (b + 1 < nb && j >= band_off(b + 1)) b++;
                    bits = band_bits(b);
                    const int bo = (j - band_off(b)) * bits;
                    byte0 = band_byte_off(b) + 2 + (bo >> 3);
                    bit0 = bo & 7;
                    offv = (float)((1 << (bits - 1)) - 1);
                    wrow = psb + b * G * CH;
                } else {
                    bits = A.rbits;
                    const int bo = (j - ns) * bits;
                    byte0 = skB + 4 + (bo >> 3);
                    bit0 = bo & 7;
                    offv = centre;
                    wrow = pw;
                }
#pragma unroll 4
                for (int t = 0; t < n_t; t++) {
                    const float cv = (float)lds_bits_at(rec, vshift + t * B + byte0, bit0, bits) - offv;
#pragma unroll
                    for (int h = 0; h < GM; h++)
                        if (h < G) acc[r][h] = fmaf(wrow[h * CH + t], cv, acc[r][h]);
                }
            }
        }
    }
    if (!want_out) return;
    // ---- the run's partial per query head ----
    const int pp = A.pp;
    if (tid == 0) {
        for (int h = 0; h < G; h++) {
            float *dst = part + ((long long)(h0 + h) * n_runs + run) * pp;
            dst[0] = m_run[h];
            dst[1] = l_run[h];
        }
    }
    if constexpr (VM) {
        // hi + lo columns (lane jc and jc + 1), one coefficient per accumulator row
        const int jc = lane & 15, kq = lane >> 4;
        const int h = jc >> 1;
        float *dst = part + ((long long)(h0 + h) * n_runs + run) * pp + 4;
        const bool col = !(jc & 1) && h < G;
#pragma unroll
        for (int i = 0; i < VM_TB; i++) {
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                const float v = add_xor1(vacc[i][ii]);
                const int c = 16 * (wv + 4 * i) + 4 * kq + ii;
                if (col && c < nt) dst[ns + c] = v;
            }
        }
#pragma unroll
        for (int ii = 0; ii < 4; ii++) {
            const float v = add_xor1(vsk[ii]);
            const int c = 16 * vm_k + 4 * kq + ii;
            if (vm_s && col && c < band_sz(vm_b)) dst[band_off(vm_b) + c] = v;
        }
        return;
    }
    if (RB > 0) {
        // position groups' sums through LDS: Tr [npg_t][G][n_win * LPW], Sr [npg_s][G][ns]
        const int tw = n_win * LPW;
        float *Tr = reinterpret_cast<float *>(dsm);
        float *Sr = Tr + npg_t * G * tw;
        __syncthreads();  // the last chunk is done with the staging memory
        if (t_on) {
#pragma unroll
            for (int k = 0; k < LPW; k++) Tr[(t_pg * G + t_ha) * tw + t_w * LPW + k] = fmaf(-centre, twsum[0], tacc[k][0]);
            if (t_hb != t_ha) {
#pragma unroll
                for (int k = 0; k < LPW; k++)
                    Tr[(t_pg * G + t_hb) * tw + t_w * LPW + k] = fmaf(-centre, twsum[1], tacc[k][1]);
            }
        }
        if (s_on) {
            Sr[(s_pg * G + s_ha) * ns + s_s] = sacc[0];
            if (s_hb != s_ha) Sr[(s_pg * G + s_hb) * ns + s_s] = sacc[1];
        }
        __syncthreads();
        for (int i = tid; i < G * (ns + nt); i += NT) {
            const int h = i / (ns + nt), j = i - h * (ns + nt);
            float v = 0.0f;
            if (j < ns)
                for (int g = 0; g < npg_s; g++) v += Sr[(g * G + h) * ns + j];
            else
                for (int g = 0; g < npg_t; g++) v += Tr[(g * G + h) * tw + (j - ns)];
            part[((long long)(h0 + h) * n_runs + run) * pp + 4 + j] = v;
        }
    } else {
        for (int h = 0; h < G; h++) {
            float *dst = part + ((long long)(h0 + h) * n_runs + run) * pp;
#pragma unroll
            for (int r = 0; r < NCOEF; r++) {
                const int j = tid + NT * r;
                if (j < ns + nt) dst[4 + j] = acc[r][h];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Merge of the runs' partials for query head blockIdx.x, then c and its transform.
// Dynamic LDS: c[pad], cs[n_skel], e[n_runs] floats, then the KV head's W fp16 (rounded up
// to whole 16-byte chunks). The partial rows' pitch pp is a multiple of 4 floats.
__global__ void __launch_bounds__(NT)
k_hier_attn_merge(const SpPlan P, const SpHierAttnArgs A, const float *__restrict__ part, int n_runs) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
    __shared__ float red[2 * (NT / SP_WAVE)];
    __shared__ float cas_s[SP_CAS_TOTAL];
    __shared__ float tsm[SP_GEN_MAX_N];
    __shared__ float red4[4 * NT];  // the run groups' coefficient sums
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;  // row h of n_seq * n_q
    const int G = A.n_q / A.n_kvh, kvh = (h % A.n_q) / G;
    const int ns = A.n_skel, nt = A.n_target, pp = A.pp;
    float *c = reinterpret_cast<float *>(dsm);
    float *cs = c + r4(A.pad);
    float *e = cs + r4(ns);
    unsigned short *Ws = reinterpret_cast<unsigned short *>(e + r4(n_runs));
    const unsigned short *Wk = reinterpret_cast<const unsigned short *>(A.W) + (long long)kvh * A.w_outer;
    const float *ph = part + (long long)h * n_runs * pp;
    // range-checked buffer loads: rows past the last run and offsets past the buffer read
    // as 0 with no traffic, so every load of a pass is unconditional and in flight
    // before the first wait
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc((void *)ph, (short)0, n_runs * pp * 4, 0x00020000);
    // the runs' m and l first: their round trip gates the first barrier, and loads
    // complete in issue order
    float mr[MERGE_RUNS_PER_THREAD], lr[MERGE_RUNS_PER_THREAD];
#pragma unroll
    for (int u = 0; u < MERGE_RUNS_PER_THREAD; u++) {
        const int r = tid + u * NT;
        mr[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, r * pp * 4, 0, 0));
        lr[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, r * pp * 4 + 4, 0, 0));
        if (r >= n_runs) mr[u] = -INFINITY;
    }
    // W (no predictor: c_tgt is the weighted sum alone) in 16-byte loads while the
    // partials are merged, stored to LDS after the sums
    const bool has_w = A.W != nullptr;
    const bool w_reg = has_w && nt * ns <= W_Q * 8 * NT;
    u32x4 wq[W_Q];
    if (w_reg) {
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)Wk, (short)0, 2 * nt * ns, 0x00020000);
#pragma unroll
        for (int u = 0; u < W_Q; u++)
            wq[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (tid + u * NT) * 16, 0, 0));
    } else if (has_w) {
        copy_to_lds<unsigned short, 16>(Ws, Wk, nt * ns, nt * ns, tid);
    }
    // coefficient sums: thread tid takes the quad q = tid % NQ (coefficients 4q..4q+3,
    // one 16-byte load per run; the row pitch is a multiple of 4 floats) over the runs
    // g, g + RG, ... of run group g = tid / NQ; the RG groups' sums meet in LDS
    const int ncoef = ns + nt, NQ = (ncoef + 3) >> 2, RG = min(NT / NQ, 8);
    const int q = tid % NQ, g = tid / NQ;
    const int qo = g < RG ? (4 + 4 * q) * 4 : 0x40000000;
    const int KR = g < RG ? (n_runs - g + RG - 1) / RG : 0;  // this thread's runs
    constexpr int MP4 = 48;
    u32x4 v[MP4];
    // (the run differs between the lanes of a wave, so its row offset goes in the
    // per-lane offset, not the wave-uniform one)
    auto load_pass = [&](int k0) {
#pragma unroll
        for (int k = 0; k < MP4; k++) {
            const int r = g + RG * (k0 + k);
            v[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rp, k0 + k < KR ? qo + r * pp * 4 : 0x40000000, 0, 0));
        }
    };
    load_pass(0);
    auto coef_idx = [&](int j) { return j < ns ? A.skel_idx[j] : A.tgt_idx[j - ns]; };
    const int ci0 = tid < ncoef ? coef_idx(tid) : 0, ci1 = tid + NT < ncoef ? coef_idx(tid + NT) : 0;
    const int ti0 = tid < nt ? A.tgt_idx[tid] : 0, ti1 = tid + NT < nt ? A.tgt_idx[tid + NT] : 0;
    const float cas_v = cas_entry(P, tid);
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < MERGE_RUNS_PER_THREAD; u++) mx = fmaxf(mx, mr[u]);
    mx = wave_max(mx);
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.0f;
#pragma unroll
    for (int u = 0; u < MERGE_RUNS_PER_THREAD; u++) {
        const int r = tid + u * NT;
        const float w = __expf(mr[u] - M);  // 0 for a run without positions (m = -inf)
        if (r < n_runs) e[r] = w;
        l = fmaf(lr[u], w, l);
    }
    l = wave_sum(l);
    if (lane == 0) red[NT / SP_WAVE + wv] = l;
    for (int k = tid; k < A.pad; k += NT) c[k] = 0.0f;
    __syncthreads();
    const float inv_l = sp_div(1.0f, (red[4] + red[5]) + (red[6] + red[7]));
    float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < KR; k0 += MP4) {
        if (k0 > 0) load_pass(k0);
#pragma unroll
        for (int k = 0; k < MP4; k++) {
            const float w = k0 + k < KR ? e[g + RG * (k0 + k)] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) s4[i] = fmaf(__uint_as_float(v[k][i]), w, s4[i]);
        }
    }
    if (g < RG) {
#pragma unroll
        for (int i = 0; i < 4; i++) red4[g * 4 * NQ + 4 * q + i] = s4[i];
    }
    __syncthreads();
    for (int j = tid; j < ncoef; j += NT) {
        float sj = 0.0f;
        for (int gg = 0; gg < RG; gg++) sj += red4[gg * 4 * NQ + j];
        sj *= inv_l;
        const int ci = j == tid ? ci0 : j == tid + NT ? ci1 : coef_idx(j);
        if (j < ns) cs[j] = sj;
        c[ci] = sj;  // targets: the dev part; W c_skel is added below
    }
    if (w_reg) {
        u32x4 *Wq = reinterpret_cast<u32x4 *>(Ws);
#pragma unroll
        for (int u = 0; u < W_Q; u++) {
            const int i = tid + u * NT;
            if (i * 8 < nt * ns) Wq[i] = wq[u];
        }
    }
    __syncthreads();
    for (int t = tid; has_w && t < nt; t += NT) {
        float pred = 0.0f;
#pragma unroll 4
        for (int s = 0; s < ns; s++) pred = fmaf(sp_f16_bits_to_f32(Ws[t * ns + s]), cs[s], pred);
        c[t == tid ? ti0 : t == tid + NT ? ti1 : A.tgt_idx[t]] += pred;
    }
    __syncthreads();
    transform_block(c, tsm, A.pad, P, cas_s, cas_v, tid);
    for (int k = tid; k < A.hd; k += NT) A.out[(long long)h * A.hd + k] = c[k];
}

// Level width of the window path for this call (0: bit-serial): the windows and
// skeleton coefficients of a head pair must each fit the block once.
int window_bits(const SpHierAttnArgs &A) {
    const int rb = A.rbits;
    if (rb != 2 && rb != 4 && rb != 8) return 0;
    const int n_hp = (A.n_q / A.n_kvh + 1) / 2;
    if ((A.n_target * rb + 31) / 32 * n_hp > NT || A.n_skel * n_hp > NT) return 0;
    return rb;
}

// Whether the V sums of a full (2-bit level) call run on the matrix cores: skeleton
// bands of at most 8 bits, at most 4 skeleton row blocks (one per wave), and 17-20
// target windows (257-320 target coefficients, five windows per wave: a window past the
// last reads at most 19 bytes past its record, inside the staging memory's 32-byte slack); the launcher
// takes it up to 4 query heads per KV head (more keep the window items).
// SP_HIP_HIER_ATTN_VM=0 (read at each call) keeps the window items.
bool vm_ok(const SpPlan &P, const SpHierAttnArgs &A) {
    if (A.rbits != 2) return false;
    int nsb = 0;
    for (int b = 0; b < P.n_bands; b++) {
        if (P.band_bits[b] < 1 || P.band_bits[b] > 8) return false;
        nsb += (P.band_sz[b] + 15) / 16;
    }
    const int n_win = (A.n_target * 2 + 31) / 32;  // five per wave, the last wave's fifth maybe past the end
    if (nsb > 4 || n_win < 17 || n_win > 20) return false;
    const char *e = getenv("SP_HIP_HIER_ATTN_VM");
    return !(e && e[0] == '0');
}

// Whether the call's record geometry is Geo330's (the compile-time instances then run).
// SP_HIP_HIER_ATTN_CT=0 (read at each call) keeps the runtime-geometry instances.
bool geo330(const SpPlan &P, const SpHierAttnArgs &A) {
    using Gc = Geo330;
    if (A.rbits != 2 || A.n_skel != Gc::ns || A.n_target != Gc::nt || A.B != Gc::B || P.n_bands != Gc::nb ||
        P.total_bytes != Gc::skB)
        return false;
    for (int b = 0; b < Gc::nb; b++)
        if (P.band_bits[b] != Gc::bits || P.band_sz[b] != Gc::sz || P.band_off[b] != b * Gc::sz ||
            P.band_byte_off[b] != b * Gc::band_bytes)
            return false;
    const char *e = getenv("SP_HIP_HIER_ATTN_CT");
    return !(e && e[0] == '0');
}

// The split kernel's instance for this call's level width, output mode and geometry.
template <bool OUT>
void launch_split(const SpPlan &P, const SpHierAttnArgs &A, const SpSeqTab &T, const float *prep, float *part,
                  int n_runs, int rb, int G, bool vm, bool ct, size_t lds_split, hipStream_t s) {
    const dim3 grid(A.n_kvh, n_runs, T.n_seq);
#define SP_SPLIT(RB_, GM_, VM_, GEO_)                                                                              \
    hipLaunchKernelGGL((k_hier_attn_split<RB_, GM_, OUT, VM_, GEO_>), grid, dim3(NT), lds_split, s, P, A, T, prep, \
                       part, n_runs)
    // ct (the compile-time geometry) comes with the matrix-core V sums at up to 4 query
    // heads per KV head, so a call's scores-only and full instances share their score code
    if (ct && G <= 2) {
        SP_SPLIT(2, 2, OUT, Geo330);
    } else if (ct && G <= 4) {
        SP_SPLIT(2, 4, OUT, Geo330);
    } else if (rb == 2 && G <= 2) {
        if (OUT && vm) SP_SPLIT(2, 2, OUT, GeoRt);
        else SP_SPLIT(2, 2, false, GeoRt);
    } else if (OUT && rb == 2 && G <= 4 && vm) {
        if constexpr (OUT) SP_SPLIT(2, 4, true, GeoRt);
    } else if (rb == 2) {
        SP_SPLIT(2, MAX_G, false, GeoRt);
    } else if (rb == 4) {
        SP_SPLIT(4, MAX_G, false, GeoRt);
    } else if (rb == 8) {
        SP_SPLIT(8, MAX_G, false, GeoRt);
    } else {
        SP_SPLIT(0, MAX_G, false, GeoRt);
    }
#undef SP_SPLIT
}

}  // namespace

int sp_hier_attn_prep_floats(int n_skel, int n_target) { return prep_sum_off(n_skel, n_target) + 4; }

size_t sp_hier_attn_workspace_floats(const SpHierAttnArgs &A, int n_runs, int n_seq) {
    return (size_t)n_seq * ((size_t)A.n_q * A.ps + (size_t)A.n_q * n_runs * A.pp);
}

// Runs per KV head and sequence: the blocks that are resident at once (three per CU)
// spread over the sequences' KV heads, so the split kernel runs in one round.
int sp_hier_attn_runs(const SpHierAttnArgs &A, int cus, int n_seq) {
    const int n_chunks = (A.n_kv + CH - 1) / CH;
    const int per_head = std::max(1, (3 * cus) / std::max(1, A.n_kvh * n_seq));
    return std::max(1, std::min(std::min(n_chunks, per_head), MERGE_RUNS_PER_THREAD * NT));
}

// LDS bytes of the merge's W copy: whole 16-byte chunks (the register path stores them so).
static size_t w_lds_bytes(const SpHierAttnArgs &A) { return (2 * (size_t)A.n_target * A.n_skel + 15) & ~(size_t)15; }

hipError_t sp_launch_hier_attn(const SpPlan &P, const SpHierAttnArgs &A, const SpSeqTab &T, float *ws,
                               size_t ws_floats, int n_runs, hipStream_t s) {
    if (A.n_kv <= 0 || A.n_q <= 0 || A.n_kvh <= 0 || A.n_q % A.n_kvh || A.n_q / A.n_kvh > MAX_G ||
        A.pad > SP_GEN_MAX_N || A.n_skel + A.n_target > SP_GEN_MAX_N || A.hd > A.pad || n_runs <= 0 ||
        A.ps != sp_hier_attn_prep_floats(A.n_skel, A.n_target) || A.pp < 4 + A.n_skel + A.n_target || A.pp % 4)
        return hipErrorInvalidValue;
    if (T.n_seq < 1 || T.n_seq > SP_ATTN_MAX_SEQ || sp_hier_attn_workspace_floats(A, n_runs, T.n_seq) > ws_floats ||
        n_runs > MERGE_RUNS_PER_THREAD * NT)
        return hipErrorInvalidValue;
    const int G = A.n_q / A.n_kvh;
    const int rb = window_bits(A);
    const size_t lds_prep = 4 * (size_t)(r4(A.pad) + r32(A.n_target) + 8 * r4(A.n_skel)) +
                            2 * (size_t)A.n_target * A.n_skel;
    const size_t rec_bytes = (size_t)rec_stage_bytes(A.B);
    size_t lds_split = rec_bytes + 4 * ((size_t)G * A.ps + (size_t)(2 + P.n_bands) * G * CH + 8 * MAX_G);
    if (rb == 2) lds_split += (size_t)r32(A.n_target) / 32 * 1024 + 4 * (16 + 16 + 8 + 256);
    if (rb > 0) {
        const int n_win = (A.n_target * rb + 31) / 32, n_hp = (G + 1) / 2;
        const int npg_t = std::max(1, NT / (n_win * n_hp)), npg_s = std::max(1, NT / (A.n_skel * n_hp));
        const size_t red_b = 4 * ((size_t)npg_t * G * n_win * (32 / rb) + (size_t)npg_s * G * A.n_skel);
        lds_split = std::max(lds_split, red_b);
    }
    const size_t lds_merge = 4 * (size_t)(r4(A.pad) + r4(A.n_skel) + r4(n_runs)) + w_lds_bytes(A);
    if (lds_prep > 65536 || lds_split > 65536 || lds_merge > 65536) return hipErrorInvalidValue;
    float *prep = ws;
    float *part = ws + (size_t)T.n_seq * A.n_q * A.ps;
    hipLaunchKernelGGL(k_hier_attn_prep, dim3(T.n_seq * A.n_q), dim3(NT), lds_prep, s, P, A, prep);
    const bool vm = rb == 2 && vm_ok(P, A);
    const bool ct = vm && G <= 4 && geo330(P, A);
    if (A.out) launch_split<true>(P, A, T, prep, part, n_runs, rb, G, vm, ct, lds_split, s);
    else launch_split<false>(P, A, T, prep, part, n_runs, rb, G, vm, ct, lds_split, s);
    if (A.out)
        hipLaunchKernelGGL(k_hier_attn_merge, dim3(T.n_seq * A.n_q), dim3(NT), lds_merge, s, P, A, part, n_runs);
    return hipGetLastError();
}

// The two launches that do not touch records, for the sqfree attention (A.W may be null).
static bool prep_merge_args_ok(const SpHierAttnArgs &A) {
    return A.n_q > 0 && A.n_kvh > 0 && A.n_q % A.n_kvh == 0 && A.n_q / A.n_kvh <= MAX_G && A.pad <= SP_GEN_MAX_N &&
           A.n_skel + A.n_target <= SP_GEN_MAX_N && A.hd <= A.pad && A.ps == sp_hier_attn_prep_floats(A.n_skel, A.n_target) &&
           A.pp >= 4 + A.n_skel + A.n_target && A.pp % 4 == 0;
}

hipError_t sp_launch_hier_attn_prep(const SpPlan &P, const SpHierAttnArgs &A, int n_seq, float *prep, hipStream_t s) {
    if (!prep_merge_args_ok(A) || n_seq < 1) return hipErrorInvalidValue;
    const size_t lds_prep = 4 * (size_t)(r4(A.pad) + r32(A.n_target) + 8 * r4(A.n_skel)) +
                            (A.W ? 2 * (size_t)A.n_target * A.n_skel : 0);
    if (lds_prep > 65536) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hier_attn_prep, dim3(n_seq * A.n_q), dim3(NT), lds_prep, s, P, A, prep);
    return hipGetLastError();
}

hipError_t sp_launch_hier_attn_merge(const SpPlan &P, const SpHierAttnArgs &A, int n_seq, const float *part,
                                     int n_runs, hipStream_t s) {
    if (!prep_merge_args_ok(A) || !A.out || n_seq < 1 || n_runs <= 0 || n_runs > MERGE_RUNS_PER_THREAD * NT)
        return hipErrorInvalidValue;
    const size_t lds_merge = 4 * (size_t)(r4(A.pad) + r4(A.n_skel) + r4(n_runs)) + (A.W ? w_lds_bytes(A) : 0);
    if (lds_merge > 65536) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hier_attn_merge, dim3(n_seq * A.n_q), dim3(NT), lds_merge, s, P, A, part, n_runs);
    return hipGetLastError();
}
