/*
 * sp_oracle.c -- CPU restatement of the Shannon-Prime codec (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: see sp_oracle.h. Built with
 * -O2 -ffp-contract=off -fno-fast-math so the fp32 expression trees below are
 * evaluated exactly as written (no FMA contraction).
 */
#include "sp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* band geometry                                                            */
/* ------------------------------------------------------------------------ */

/* Band layout: band_size = hd / n_bands, the last band absorbs the remainder
 * (shannon_prime_cuda.cu:149-151); record = per band [fp16 scale LE][packed
 * ceil(sz*bits/8) bytes] (shannon_prime_cuda.cu:171-202). Ternary bands are
 * stored at 2 bits (max_val 1, codes {0,1,2}) regardless of band_bits[b]
 * (CHANGELOG.md:109-116 "quantised to {-1,0,+1} at 2 bpp"). */
void spo_band_config_init_ext(spo_band_config_t *bc, int head_dim, int n_bands,
                              const int *bits, uint32_t ternary_mask) {
    memset(bc, 0, sizeof(*bc));
    if (n_bands < 1) n_bands = 1;
    if (n_bands > SPO_MAX_BANDS) n_bands = SPO_MAX_BANDS;
    bc->head_dim = head_dim;
    bc->n_bands = n_bands;
    bc->band_size = head_dim / n_bands;
    bc->ternary_mask = ternary_mask;
    int byte_off = 0;
    for (int b = 0; b < n_bands; b++) {
        int bb = bits[b];
        if (ternary_mask & (1u << b)) bb = 2;
        bc->band_bits[b] = bb;
        int off = b * bc->band_size;
        int sz = (b == n_bands - 1) ? (head_dim - off) : bc->band_size;
        bc->band_off[b] = off;
        bc->band_sz[b] = sz;
        bc->band_byte_off[b] = byte_off;
        byte_off += 2 + (sz * bb + 7) / 8;
    }
    bc->total_bytes = byte_off;
}

void spo_band_config_init(spo_band_config_t *bc, int head_dim, int n_bands, const int *bits) {
    spo_band_config_init_ext(bc, head_dim, n_bands, bits, 0u);
}

void spo_band_span(const spo_band_config_t *bc, int b, int *off, int *sz) {
    *off = bc->band_off[b];
    *sz = bc->band_sz[b];
}

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32                                               */
/* ------------------------------------------------------------------------ */

/* Round-to-nearest-even float -> half, written from the IEEE 754 encoding
 * (the CUDA path stores __float2half(scale), an RNE conversion,
 * shannon_prime_cuda.cu:171). Overflow -> +-inf, subnormals kept. */
uint16_t spo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    int e = (int)(ax >> 23) - 127;
    uint32_t m = ax & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        uint32_t keep = m >> 13, rem = m & 0x1fffu;
        uint32_t r = ((uint32_t)(e + 15) << 10) | keep;
        if (rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) r += 1; /* carry may reach inf */
        return (uint16_t)(sign | r);
    }
    /* subnormal half: value = mfull * 2^(e-23), unit 2^-24 */
    uint32_t mfull = m | 0x800000u;
    int shift = -e - 1; /* mfull >> shift gives units of 2^-24 */
    if (ax == 0) return (uint16_t)sign;
    if (shift > 24) return (uint16_t)sign;
    uint32_t keep = mfull >> shift;
    uint32_t rem = mfull & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (keep & 1u))) keep += 1;
    return (uint16_t)(sign | keep);
}

/* Exact half -> float (subnormals included), as __half2float
 * (shannon_prime_cuda.cu:244). */
float spo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, f;
    if (e == 0) {
        if (m == 0) {
            f = sign;
        } else {
            int ee = -14;
            while (!(m & 0x400u)) { m <<= 1; ee--; }
            m &= 0x3ffu;
            f = sign | ((uint32_t)(ee + 127) << 23) | (m << 13);
        }
    } else if (e == 31) {
        f = sign | 0x7f800000u | (m << 13);
    } else {
        f = sign | ((e + 112u) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &f, 4);
    return r;
}

/* ------------------------------------------------------------------------ */
/* transforms                                                               */
/* ------------------------------------------------------------------------ */

/* Factor n over {2,3,5,7,11}, ascending (shannon_prime_cuda.cu:288-299). */
int spo_factor_small(int n, int *factors, int max_factors) {
    static const int primes[5] = {2, 3, 5, 7, 11};
    int nf = 0, d = n;
    if (n < 1) return -1;
    for (int i = 0; i < 5; i++)
        while (d % primes[i] == 0 && nf < max_factors) { factors[nf++] = primes[i]; d /= primes[i]; }
    return d == 1 ? nf : -1;
}

/* p x p Hartley kernel C[k][j] = cas(2*pi*k*j/p) = cos + sin, evaluated in
 * double and rounded once to float (kernel_vilenkin_inplace computes the same
 * entries per element with __cosf/__sinf, shannon_prime_sqfree.cu:41-43,89-95). */
void spo_cas_table(int p, float *C) {
    for (int k = 0; k < p; k++)
        for (int j = 0; j < p; j++) {
            double a = 2.0 * M_PI * (double)((k * j) % p) / (double)p;
            C[k * p + j] = (float)(cos(a) + sin(a));
        }
}

float spo_inv_sqrt_n(int n) { return 1.0f / sqrtf((float)n); }

/* p=2 VHT2: stages len = 1,2,4,...,n/2, butterfly (u+v, u-v) in natural order.
 * NORM_FINAL: unnormalised butterflies then x *= 1.0f/sqrtf(n)
 *   (shannon_prime_adreno.c:276-309, logged bit-equal to the CPU core,
 *    android_build/test_adreno_phone.log "NEON WHT vs Core max_err=0").
 * NORM_STAGE: (u+v)*0.70710678f, (u-v)*0.70710678f per stage
 *   (shannon_prime_cuda.cu:54-69). */
void spo_vht2_p2(float *x, int n, int norm_mode) {
    const float s2 = 0.70710678118654752440f;
    for (int len = 1; len < n; len <<= 1)
        for (int i = 0; i < n; i += len << 1)
            for (int j = 0; j < len; j++) {
                float u = x[i + j], v = x[i + j + len];
                if (norm_mode == SPO_NORM_STAGE) {
                    x[i + j] = (u + v) * s2;
                    x[i + j + len] = (u - v) * s2;
                } else {
                    x[i + j] = u + v;
                    x[i + j + len] = u - v;
                }
            }
    if (norm_mode != SPO_NORM_STAGE) {
        const float inv = spo_inv_sqrt_n(n);
        for (int i = 0; i < n; i++) x[i] *= inv;
    }
}

/* Staged Vilenkin-Hartley transform: for each prime factor p (ascending),
 * stride *= p; groups {base + k*stride}; result[k] = (sum_j C[k][j]*g[j]) *
 * (1/sqrt(p)), sum from 0.0f over j ascending (shannon_prime_sqfree.cu:66-106).
 * 1/sqrt(p) is 1.0f/sqrtf((float)p). */
void spo_vilenkin(float *x, int n, const int *factors, int n_factors) {
    int stride = 1;
    float C[11 * 11], g[11], r[11];
    for (int f = 0; f < n_factors; f++) {
        int p = factors[f];
        spo_cas_table(p, C);
        float isp = spo_inv_sqrt_n(p);
        int block = stride * p;
        for (int blk = 0; blk < n / block; blk++)
            for (int s = 0; s < stride; s++) {
                int base = blk * block + s;
                for (int k = 0; k < p; k++) g[k] = x[base + k * stride];
                for (int k = 0; k < p; k++) {
                    float sum = 0.0f;
                    for (int j = 0; j < p; j++) sum += C[k * p + j] * g[j];
                    r[k] = sum * isp;
                }
                for (int k = 0; k < p; k++) x[base + k * stride] = r[k];
            }
        stride *= p;
    }
}

/* Power-of-2 n -> p=2 butterfly; otherwise the staged Vilenkin kernel
 * (dispatch rule of sp_cuda_vht2_forward, shannon_prime_cuda.cu:303-327). */
void spo_vht2_forward(float *x, int n, int norm_mode) {
    if (n > 0 && (n & (n - 1)) == 0) {
        spo_vht2_p2(x, n, norm_mode);
        return;
    }
    int f[16];
    int nf = spo_factor_small(n, f, 16);
    if (nf <= 0) return; /* reference leaves the data unchanged (:314-318) */
    spo_vilenkin(x, n, f, nf);
}

/* ------------------------------------------------------------------------ */
/* Mobius squarefree-first order                                            */
/* ------------------------------------------------------------------------ */

int spo_is_squarefree(int n) {
    if (n < 1) return 0;
    for (int p = 2; p * p <= n; p++)
        if (n % (p * p) == 0) return 0;
    return 1;
}

int spo_mobius_mu(int n) {
    if (n < 1) return 0;
    int mu = 1;
    for (int p = 2; p * p <= n; p++)
        if (n % p == 0) {
            n /= p;
            if (n % p == 0) return 0;
            mu = -mu;
        }
    if (n > 1) mu = -mu;
    return mu;
}

/* order[r] = coefficient index placed at reordered position r: indices i with
 * i+1 squarefree, ascending, then the remaining indices ascending. The
 * reference builds this table in the absent core (sp_mobius_mask_init, used
 * shannon_prime_cuda.cu:428-445); the rule here is this build's documented
 * choice. Kernels consume it as data. */
void spo_mobius_order(int n, int *order) {
    int r = 0;
    for (int i = 0; i < n; i++) if (spo_is_squarefree(i + 1)) order[r++] = i;
    for (int i = 0; i < n; i++) if (!spo_is_squarefree(i + 1)) order[r++] = i;
}

/* ------------------------------------------------------------------------ */
/* band quantizer                                                           */
/* ------------------------------------------------------------------------ */

/* rint (half-even) then saturating int conversion with NaN -> 0, clamped to
 * [-m, m] (__float2int_rn + clamp, shannon_prime_cuda.cu:186-188). */
static int q_rint_clamp(float v, int m) {
    float r = rintf(v);
    if (r != r) return 0;
    if (r > (float)m) return m;
    if (r < (float)-m) return -m;
    return (int)r;
}

/* kernel_band_quantize_simple (shannon_prime_cuda.cu:131-204):
 * amax (strict >), scale = amax/max_val, stored fp16 (RNE); inv from the
 * stored half; q = rint(x*inv) clamped; u = q+max_val packed LSB-first. */
void spo_band_quantize(const float *in, uint8_t *out, const spo_band_config_t *bc) {
    int offset = 0;
    for (int b = 0; b < bc->n_bands; b++) {
        int off = bc->band_off[b], sz = bc->band_sz[b], bits = bc->band_bits[b];
        int max_val = (1 << (bits - 1)) - 1;
        const float *band = in + off;
        float amax = 0.0f;
        for (int i = 0; i < sz; i++) {
            float a = fabsf(band[i]);
            if (a > amax) amax = a;
        }
        float scale = (amax > 0.0f) ? amax / (float)max_val : 0.0f;
        uint16_t h = spo_f32_to_f16(scale);
        out[offset] = (uint8_t)(h & 0xff);
        out[offset + 1] = (uint8_t)(h >> 8);
        offset += 2;
        float ss = spo_f16_to_f32(h);
        float inv = (ss > 0.0f) ? 1.0f / ss : 0.0f;
        uint64_t buf = 0;
        int bp = 0;
        for (int i = 0; i < sz; i++) {
            int q = q_rint_clamp(band[i] * inv, max_val);
            uint32_t u = (uint32_t)(q + max_val);
            buf |= (uint64_t)u << bp;
            bp += bits;
            while (bp >= 8) { out[offset++] = (uint8_t)(buf & 0xff); buf >>= 8; bp -= 8; }
        }
        if (bp > 0) out[offset++] = (uint8_t)(buf & 0xff);
    }
}

/* kernel_band_dequantize_simple (shannon_prime_cuda.cu:210-270): non-finite
 * scale -> 0, x = (float)(u - max_val) * scale. Partial (shannon_prime_llama.h
 * :240-255): max_bands < 0 or >= n_bands -> full; bands >= max_bands -> 0.0f. */
void spo_band_dequantize_partial(const uint8_t *in, float *out,
                                 const spo_band_config_t *bc, int max_bands) {
    if (max_bands < 0 || max_bands > bc->n_bands) max_bands = bc->n_bands;
    for (int b = 0; b < bc->n_bands; b++) {
        int off = bc->band_off[b], sz = bc->band_sz[b], bits = bc->band_bits[b];
        int offset = bc->band_byte_off[b];
        float *band = out + off;
        if (b >= max_bands) {
            for (int i = 0; i < sz; i++) band[i] = 0.0f;
            continue;
        }
        int max_val = (1 << (bits - 1)) - 1;
        uint32_t mask = (1u << bits) - 1u;
        uint16_t h = (uint16_t)(in[offset] | ((uint16_t)in[offset + 1] << 8));
        float scale = spo_f16_to_f32(h);
        if (!isfinite(scale)) scale = 0.0f;
        offset += 2;
        uint64_t buf = 0;
        int bp = 0;
        for (int i = 0; i < sz; i++) {
            while (bp < bits) { buf |= (uint64_t)in[offset++] << bp; bp += 8; }
            uint32_t u = (uint32_t)(buf & mask);
            buf >>= bits;
            bp -= bits;
            band[i] = (float)((int)u - max_val) * scale;
        }
    }
}

void spo_band_dequantize(const uint8_t *in, float *out, const spo_band_config_t *bc) {
    spo_band_dequantize_partial(in, out, bc, -1);
}

/* ------------------------------------------------------------------------ */
/* ship codec                                                               */
/* ------------------------------------------------------------------------ */

/* Write path: VHT2 -> (K) Mobius reorder r[i] = c[order[i]] -> band quantize
 * (sp_cuda_write_k, shannon_prime_cuda.cu:474-500; V without reorder :502-521;
 * gather kernel :85-95). */
void spo_ship_compress(const float *vec, uint8_t *out, const spo_band_config_t *bc,
                       const int *order, int norm_mode) {
    int n = bc->head_dim;
    float c[1024], r[1024];
    memcpy(c, vec, (size_t)n * sizeof(float));
    spo_vht2_forward(c, n, norm_mode);
    if (order) {
        for (int i = 0; i < n; i++) r[i] = c[order[i]];
        spo_band_quantize(r, out, bc);
    } else {
        spo_band_quantize(c, out, bc);
    }
}

/* Read path: dequantize(partial) -> (K) unreorder c[order[i]] = r[i] -> VHT2
 * (self-inverse) (sp_cuda_read_k, shannon_prime_cuda.cu:524-542; scatter
 * kernel :99-111). */
void spo_ship_decompress(const uint8_t *in, float *out, const spo_band_config_t *bc,
                         const int *order, int norm_mode, int max_bands) {
    int n = bc->head_dim;
    float r[1024];
    if (order) {
        spo_band_dequantize_partial(in, r, bc, max_bands);
        for (int i = 0; i < n; i++) out[order[i]] = r[i];
    } else {
        spo_band_dequantize_partial(in, out, bc, max_bands);
    }
    spo_vht2_forward(out, n, norm_mode);
}

void spo_ship_compress_batch_f16(const uint16_t *in, uint8_t *out, int n, int hd,
                                 const spo_band_config_t *bc, const int *order, int norm_mode) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++) {
        float v[1024];
        for (int i = 0; i < hd; i++) v[i] = spo_f16_to_f32(in[(size_t)t * hd + i]);
        spo_ship_compress(v, out + (size_t)t * bc->total_bytes, bc, order, norm_mode);
    }
}

void spo_ship_compress_batch_f32(const float *in, uint8_t *out, int n, int hd,
                                 const spo_band_config_t *bc, const int *order, int norm_mode) {
    for (int t = 0; t < n; t++)
        spo_ship_compress(in + (size_t)t * hd, out + (size_t)t * bc->total_bytes, bc, order,
                          norm_mode);
}

void spo_ship_decompress_batch_f32(const uint8_t *in, float *out, int n, int hd,
                                   const spo_band_config_t *bc, const int *order,
                                   int norm_mode, int max_bands) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++)
        spo_ship_decompress(in + (size_t)t * bc->total_bytes, out + (size_t)t * hd, bc, order,
                            norm_mode, max_bands);
}

void spo_ship_decompress_batch_f16(const uint8_t *in, uint16_t *out, int n, int hd,
                                   const spo_band_config_t *bc, const int *order,
                                   int norm_mode, int max_bands) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++) {
        float v[1024];
        spo_ship_decompress(in + (size_t)t * bc->total_bytes, v, bc, order, norm_mode, max_bands);
        for (int i = 0; i < hd; i++) out[(size_t)t * hd + i] = spo_f32_to_f16(v[i]);
    }
}

void spo_ship_roundtrip_batch_f16_omp(const uint16_t *in, uint8_t *packed, uint16_t *out,
                                      int n, int hd, const spo_band_config_t *bc,
                                      const int *order, int norm_mode, int n_threads) {
#ifdef _OPENMP
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel for num_threads(n_threads) schedule(static)
#endif
    for (int t = 0; t < n; t++) {
        float v[1024];
        for (int i = 0; i < hd; i++) v[i] = spo_f16_to_f32(in[(size_t)t * hd + i]);
        spo_ship_compress(v, packed + (size_t)t * bc->total_bytes, bc, order, norm_mode);
        spo_ship_decompress(packed + (size_t)t * bc->total_bytes, v, bc, order, norm_mode, -1);
        for (int i = 0; i < hd; i++) out[(size_t)t * hd + i] = spo_f32_to_f16(v[i]);
    }
    (void)n_threads;
}

/* ------------------------------------------------------------------------ */
/* reductions                                                               */
/* ------------------------------------------------------------------------ */

/* The summation order of the reference's 256-thread block reductions
 * (kernel_mean_abs, shannon_prime_sqfree.cu:493-509; kernel_residual_magnitude,
 * shannon_prime_hier.cu:115-144): slot t accumulates v[t], v[t+256], ... from
 * 0.0f, then slot[t] += slot[t+s] for s = 128, 64, ..., 1. */
float spo_tree256_sum(const float *v, int n, int take_abs) {
    float slot[256];
    for (int t = 0; t < 256; t++) {
        float acc = 0.0f;
        for (int i = t; i < n; i += 256) acc += take_abs ? fabsf(v[i]) : v[i];
        slot[t] = acc;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int t = 0; t < s; t++) slot[t] += slot[t + s];
    return slot[0];
}

/* ------------------------------------------------------------------------ */
/* sqfree + spinor                                                          */
/* ------------------------------------------------------------------------ */

static int is_11_smooth(int n) {
    static const int primes[5] = {2, 3, 5, 7, 11};
    for (int i = 0; i < 5; i++) while (n % primes[i] == 0) n /= primes[i];
    return n == 1;
}

/* Smallest squarefree 11-smooth integer >= hd (reproduces the three pads the
 * reference documents: 64->66, 128->154, 256->330; patches/README.md,
 * shannon_prime_sqfree.cu:39). */
int spo_sqfree_pad_dim(int hd) {
    for (int n = hd; n < 16 * hd + 64; n++)
        if (spo_is_squarefree(n) && is_11_smooth(n)) return n;
    return -1;
}

/* Knight mask: skeleton = first sk_k entries of the squarefree-first order over
 * [0, pad); residual = the rest (in that order). CSR for residual coefficient
 * c (n = c+1): one term per proper divisor d of n (ascending) whose coefficient
 * d-1 is in the skeleton and mu(n/d) != 0, with sign mu(n/d). The reference's
 * builder (sp_knight_mask_init, called shannon_prime_sqfree.cu:606) is absent;
 * this is the build's documented rule, consumed by the kernels as data. */
int spo_knight_mask_init(spo_knight_mask_t *m, int pad_dim, int sk_k) {
    memset(m, 0, sizeof(*m));
    if (pad_dim <= 0 || sk_k <= 0 || sk_k > pad_dim) return -1;
    int *order = (int *)malloc(sizeof(int) * (size_t)pad_dim);
    int *slot_of = (int *)malloc(sizeof(int) * (size_t)pad_dim);
    spo_mobius_order(pad_dim, order);
    m->pad_dim = pad_dim;
    m->sk_k = sk_k;
    m->n_res = pad_dim - sk_k;
    m->skeleton_idx = (int *)malloc(sizeof(int) * (size_t)sk_k);
    m->residual_idx = (int *)malloc(sizeof(int) * (size_t)(m->n_res > 0 ? m->n_res : 1));
    m->csr_offsets = (int *)malloc(sizeof(int) * (size_t)(m->n_res + 1));
    for (int i = 0; i < pad_dim; i++) slot_of[i] = -1;
    for (int s = 0; s < sk_k; s++) { m->skeleton_idx[s] = order[s]; slot_of[order[s]] = s; }
    for (int r = 0; r < m->n_res; r++) m->residual_idx[r] = order[sk_k + r];
    int cap = 16 * (m->n_res + 1), nt = 0;
    m->csr_skel_slot = (int *)malloc(sizeof(int) * (size_t)cap);
    m->csr_mu_sign = (int8_t *)malloc((size_t)cap);
    for (int r = 0; r < m->n_res; r++) {
        m->csr_offsets[r] = nt;
        int n = m->residual_idx[r] + 1;
        for (int d = 1; d < n; d++) {
            if (n % d) continue;
            int c = d - 1, mu = spo_mobius_mu(n / d);
            if (mu == 0 || slot_of[c] < 0) continue;
            if (nt >= cap) {
                cap *= 2;
                m->csr_skel_slot = (int *)realloc(m->csr_skel_slot, sizeof(int) * (size_t)cap);
                m->csr_mu_sign = (int8_t *)realloc(m->csr_mu_sign, (size_t)cap);
            }
            m->csr_skel_slot[nt] = slot_of[c];
            m->csr_mu_sign[nt] = (int8_t)mu;
            nt++;
        }
    }
    m->csr_offsets[m->n_res] = nt;
    m->n_terms = nt;
    free(order);
    free(slot_of);
    return 0;
}

void spo_knight_mask_free(spo_knight_mask_t *m) {
    free(m->skeleton_idx);
    free(m->residual_idx);
    free(m->csr_offsets);
    free(m->csr_skel_slot);
    free(m->csr_mu_sign);
    memset(m, 0, sizeof(*m));
}

/* Pad: copy hd values, fill [hd, pad) with their mean (kernel_sqfree_pad,
 * shannon_prime_sqfree.cu:118-151). The reference kernel's mean sums only the
 * first warp's partials (:133-144); this build uses the true mean, summed in
 * the tree256 order, divided by (float)hd. */
void spo_sqfree_pad(const float *in, float *out, int hd, int pad) {
    float mean = spo_tree256_sum(in, hd, 0) / (float)hd;
    for (int i = 0; i < pad; i++) out[i] = (i < hd) ? in[i] : mean;
}

int spo_sqfree_bytes(const spo_band_config_t *skel_bc, int n_res, int rbits, int spinor) {
    return skel_bc->total_bytes + 4 + (n_res * rbits + 7) / 8 + (spinor ? (n_res + 7) / 8 : 0);
}

/* LSB-first bit packing of small levels (kernel_pack_levels,
 * shannon_prime_sqfree.cu:552-564). */
void spo_pack_levels(const uint8_t *lv, int n, int bits, uint8_t *out) {
    int nb = (n * bits + 7) / 8;
    memset(out, 0, (size_t)nb);
    for (int i = 0; i < n; i++) {
        int bo = i * bits;
        out[bo / 8] |= (uint8_t)(lv[i] << (bo % 8));
        if ((bo % 8) + bits > 8 && (bo / 8 + 1) < nb) out[bo / 8 + 1] |= (uint8_t)(lv[i] >> (8 - bo % 8));
    }
}

/* kernel_unpack_levels, shannon_prime_sqfree.cu:567-579. */
void spo_unpack_levels(const uint8_t *in, int n, int bits, uint8_t *lv) {
    int nb = (n * bits + 7) / 8;
    uint32_t mask = (1u << bits) - 1u;
    for (int i = 0; i < n; i++) {
        int bo = i * bits;
        uint32_t w = (uint32_t)in[bo / 8] >> (bo % 8);
        if ((bo % 8) + bits > 8 && (bo / 8 + 1) < nb) w |= (uint32_t)in[bo / 8 + 1] << (8 - bo % 8);
        lv[i] = (uint8_t)(w & mask);
    }
}

/* (int)(x) truncation with NaN -> 0 and saturation (cvt.rzi semantics). */
static int trunc_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483647.0f) return 2147483647;
    if (x <= -2147483648.0f) return (-2147483647 - 1);
    return (int)x;
}

static float mean_abs_floor(const float *dev, int n) {
    float mag = spo_tree256_sum(dev, n, 1) / (float)n;
    if (mag < 1e-12f) mag = 1e-12f;
    return mag;
}

/* CSR Mobius prediction: pred[r] = sum_j (float)mu[j] * skel[slot[j]], from
 * 0.0f in CSR order (kernel_mobius_predict, shannon_prime_sqfree.cu:179-203). */
void spo_mobius_predict(const float *skel, const spo_knight_mask_t *m, float *pred) {
    for (int r = 0; r < m->n_res; r++) {
        float p = 0.0f;
        for (int j = m->csr_offsets[r]; j < m->csr_offsets[r + 1]; j++)
            p += (float)m->csr_mu_sign[j] * skel[m->csr_skel_slot[j]];
        pred[r] = p;
    }
}

/* Spinor sheet choice (kernel_spinor_extract, shannon_prime_sqfree.cu:212-240):
 * v+ = a - p, v- = a + p; the sheet bit is 1 iff |v-| < |v+| (strict, so a tie
 * keeps v+ and bit 0); dev = the winner; bits LSB-first, sheet zeroed first. */
void spo_spinor_extract(const float *a, const float *p, int n, float *dev, uint8_t *sheet) {
    memset(sheet, 0, (size_t)((n + 7) / 8));
    for (int r = 0; r < n; r++) {
        float vp = a[r] - p[r], vm = a[r] + p[r];
        int use_minus = fabsf(vm) < fabsf(vp);
        dev[r] = use_minus ? vm : vp;
        if (use_minus) sheet[r / 8] |= (uint8_t)(1u << (r % 8));
    }
}

/* Sqfree residual quantizer (kernel_mean_abs + kernel_quantize_residual,
 * shannon_prime_sqfree.cu:493-532): mag = max(tree-256 sum of |dev| / n, 1e-12);
 * L = 2^bits, center = (L-1)/2, sat = mag*bits (1e-12 when mag is at the floor),
 * step = 2*sat/(L-1), level = (int)(dev*(1/step) + center + 0.5) (truncation),
 * clamped to [0, L-1]. Returns the mag the record stores. */
float spo_sqfree_residual_quantize(const float *dev, int n, int bits, uint8_t *lv) {
    float mag = mean_abs_floor(dev, n);
    int L = 1 << bits;
    float center = 0.5f * (float)(L - 1);
    float sat = (mag > 1e-12f) ? (mag * (float)bits) : 1e-12f;
    float step = (2.0f * sat) / (float)(L - 1);
    float inv_step = 1.0f / step;
    for (int r = 0; r < n; r++) {
        float qf = dev[r] * inv_step + center;
        int level = trunc_sat(qf + 0.5f);
        if (level < 0) level = 0;
        if (level >= L) level = L - 1;
        lv[r] = (uint8_t)level;
    }
    return mag;
}

/* Sqfree residual dequantizer (kernel_dequantize_residual,
 * shannon_prime_sqfree.cu:535-548): step = 2*mag*bits/(L-1) (no floor test),
 * dev = (level - center) * step. */
void spo_sqfree_residual_dequantize(const uint8_t *lv, int n, int bits, float mag, float *dev) {
    int L = 1 << bits;
    float center = 0.5f * (float)(L - 1);
    float sat = mag * (float)bits;
    float step = (L > 1) ? (2.0f * sat / (float)(L - 1)) : 0.0f;
    for (int r = 0; r < n; r++) dev[r] = ((float)lv[r] - center) * step;
}

/* Sqfree write (sp_cuda_sqfree_write_one, shannon_prime_sqfree.cu:750-853):
 * pad -> Vilenkin -> skeleton gather -> band quantize skeleton -> CSR predict
 * from the (unquantized) skeleton -> spinor or plain deviation -> mag =
 * max(mean|dev|, 1e-12) stored f32 LE -> residual levels (kernel_quantize_residual
 * :514-532) -> LSB-first pack -> sheet bits. Record [skel][mag][res][sheet]
 * (:683-686). */
void spo_sqfree_compress(const float *vec, uint8_t *out, int hd, const spo_knight_mask_t *m,
                         const spo_band_config_t *skel_bc, int rbits, int spinor) {
    int pd = m->pad_dim, sk = m->sk_k, nr = m->n_res;
    float c[1024], skel[1024], pred[1024], dev[1024];
    uint8_t lv[1024];
    int f[16];
    int nf = spo_factor_small(pd, f, 16);
    spo_sqfree_pad(vec, c, hd, pd);
    spo_vilenkin(c, pd, f, nf);
    for (int s = 0; s < sk; s++) skel[s] = c[m->skeleton_idx[s]];
    spo_band_quantize(skel, out, skel_bc);
    if (nr == 0) return;
    spo_mobius_predict(skel, m, pred);
    int res_bytes = (nr * rbits + 7) / 8;
    uint8_t *sheet = out + skel_bc->total_bytes + 4 + res_bytes;
    float act[1024];
    for (int r = 0; r < nr; r++) act[r] = c[m->residual_idx[r]];
    if (spinor) {
        spo_spinor_extract(act, pred, nr, dev, sheet);
    } else {
        for (int r = 0; r < nr; r++) dev[r] = act[r] - pred[r];
    }
    float mag = spo_sqfree_residual_quantize(dev, nr, rbits, lv);
    memcpy(out + skel_bc->total_bytes, &mag, 4);
    spo_pack_levels(lv, nr, rbits, out + skel_bc->total_bytes + 4);
}

/* Sqfree read (sp_cuda_sqfree_read_one, shannon_prime_sqfree.cu:857-950):
 * dequantize skeleton, scatter, predict from the dequantized skeleton, residual
 * (lvl - center) * step with step = 2*mag*bits/(L-1) (:535-548), spinor sign
 * flip (:249-283), inverse Vilenkin, unpad. */
void spo_sqfree_decompress(const uint8_t *in, float *out, int hd, const spo_knight_mask_t *m,
                           const spo_band_config_t *skel_bc, int rbits, int spinor) {
    int pd = m->pad_dim, sk = m->sk_k, nr = m->n_res;
    float c[1024], skel[1024], pred[1024];
    uint8_t lv[1024];
    int f[16];
    int nf = spo_factor_small(pd, f, 16);
    spo_band_dequantize(in, skel, skel_bc);
    for (int i = 0; i < pd; i++) c[i] = 0.0f;
    for (int s = 0; s < sk; s++) c[m->skeleton_idx[s]] = skel[s];
    if (nr > 0) {
        spo_mobius_predict(skel, m, pred);
        float mag;
        memcpy(&mag, in + skel_bc->total_bytes, 4);
        int res_bytes = (nr * rbits + 7) / 8;
        spo_unpack_levels(in + skel_bc->total_bytes + 4, nr, rbits, lv);
        float dv[1024];
        spo_sqfree_residual_dequantize(lv, nr, rbits, mag, dv);
        const uint8_t *sheet = in + skel_bc->total_bytes + 4 + res_bytes;
        for (int r = 0; r < nr; r++) {
            float p = pred[r];
            if (spinor && (sheet[r / 8] & (1u << (r % 8)))) p = -p;  /* kernel_spinor_reconstruct :249-283 */
            c[m->residual_idx[r]] = p + dv[r];
        }
    }
    spo_vilenkin(c, pd, f, nf);
    for (int i = 0; i < hd; i++) out[i] = c[i];
}

void spo_sqfree_compress_batch_f16(const uint16_t *in, uint8_t *out, int n, int hd,
                                   const spo_knight_mask_t *m, const spo_band_config_t *skel_bc,
                                   int rbits, int spinor) {
    int B = spo_sqfree_bytes(skel_bc, m->n_res, rbits, spinor);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++) {
        float v[1024];
        for (int i = 0; i < hd; i++) v[i] = spo_f16_to_f32(in[(size_t)t * hd + i]);
        spo_sqfree_compress(v, out + (size_t)t * B, hd, m, skel_bc, rbits, spinor);
    }
}

void spo_sqfree_decompress_batch_f32(const uint8_t *in, float *out, int n, int hd,
                                     const spo_knight_mask_t *m, const spo_band_config_t *skel_bc,
                                     int rbits, int spinor) {
    int B = spo_sqfree_bytes(skel_bc, m->n_res, rbits, spinor);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++)
        spo_sqfree_decompress(in + (size_t)t * B, out + (size_t)t * hd, hd, m, skel_bc, rbits,
                              spinor);
}

/* ------------------------------------------------------------------------ */
/* hierarchical                                                             */
/* ------------------------------------------------------------------------ */

/* Skeleton size ~9% of pad (shannon_prime_hier.cu describes the skeleton as a
 * small "Kronecker sub-projection"; the geometry builder is absent): n_skel =
 * ceil(0.09*pad), so pad 330 -> 30 skeleton / 300 targets. */
void spo_hier_default_geometry(int pad, int *n_skel) {
    int s = (pad * 9 + 99) / 100;
    if (s < 1) s = 1;
    *n_skel = s;
}

/* skeleton = first n_skel entries of the squarefree-first order over [0,pad);
 * targets = the remaining entries in that order. */
void spo_hier_indices(int pad, int n_skel, int *skel_idx, int *target_idx) {
    int *order = (int *)malloc(sizeof(int) * (size_t)pad);
    spo_mobius_order(pad, order);
    for (int s = 0; s < n_skel; s++) skel_idx[s] = order[s];
    for (int t = 0; t < pad - n_skel; t++) target_idx[t] = order[n_skel + t];
    free(order);
}

int spo_hier_bytes(const spo_band_config_t *skel_bc, int n_target, int rbits) {
    return skel_bc->total_bytes + 4 + (n_target * rbits + 7) / 8;
}

/* pred[t] = sum_s (float)W[t][s] * skel[s] from 0.0f (kernel_hier_predict,
 * shannon_prime_hier.cu:74-92). */
void spo_hier_predict(const uint16_t *W, const float *skel, float *pred, int nt, int ns) {
    for (int t = 0; t < nt; t++) {
        float acc = 0.0f;
        for (int s = 0; s < ns; s++) acc += spo_f16_to_f32(W[(size_t)t * ns + s]) * skel[s];
        pred[t] = acc;
    }
}

/* Hier residual quantizer (kernel_residual_magnitude + kernel_quantize_residual,
 * shannon_prime_hier.cu:115-171): m = max(tree-256 sum of |dev| / n, 1e-12);
 * L = 2^bits, step = 2*m/(L-1), center = (L-1)/2, inv_step = 1/step (0 if step
 * is 0), level = rint(dev*inv_step + center) (__float2int_rn: half to even),
 * clamped to [0, L-1]. Returns the stored m. */
float spo_hier_residual_quantize(const float *dev, int n, int bits, uint8_t *lv) {
    float mag = mean_abs_floor(dev, n);
    int L = 1 << bits;
    float step = 2.0f * mag / (float)(L - 1);
    float center = (float)(L - 1) / 2.0f;
    float inv_step = (step > 0.0f) ? 1.0f / step : 0.0f;
    for (int t = 0; t < n; t++) {
        float v = rintf(dev[t] * inv_step + center);
        int q = (v != v) ? 0 : (v >= 2147483647.0f ? 2147483647 : (v <= -2147483648.0f ? (-2147483647 - 1) : (int)v));
        if (q < 0) q = 0;
        if (q >= L) q = L - 1;
        lv[t] = (uint8_t)q;
    }
    return mag;
}

/* Hier residual dequantizer (kernel_dequantize_residual, shannon_prime_hier.cu:177-193):
 * dev = (level - center) * (2*m/(L-1)). */
void spo_hier_residual_dequantize(const uint8_t *lv, int n, int bits, float mag, float *dev) {
    int L = 1 << bits;
    float step = 2.0f * mag / (float)(L - 1);
    float center = (float)(L - 1) / 2.0f;
    for (int t = 0; t < n; t++) dev[t] = ((float)lv[t] - center) * step;
}

/* Hier write (sp_cuda_hier_write_one, shannon_prime_hier.cu:399-486):
 * pad -> Vilenkin -> skeleton gather -> band quantize -> pred = W*skel ->
 * dev = c[target] - pred -> mag = max(mean|dev|,1e-12) -> levels
 * rint(dev*inv_step + center) with step = 2m/(L-1) (:151-171) -> pack. */
void spo_hier_compress(const float *vec, uint8_t *out, int hd, int pad,
                       int n_skel, const int *skel_idx, int n_target, const int *target_idx,
                       const spo_band_config_t *skel_bc, const uint16_t *W, int rbits) {
    float c[1024], skel[1024], pred[1024], dev[1024];
    uint8_t lv[1024];
    int f[16];
    int nf = spo_factor_small(pad, f, 16);
    spo_sqfree_pad(vec, c, hd, pad);
    spo_vilenkin(c, pad, f, nf);
    for (int s = 0; s < n_skel; s++) skel[s] = c[skel_idx[s]];
    spo_band_quantize(skel, out, skel_bc);
    spo_hier_predict(W, skel, pred, n_target, n_skel);
    for (int t = 0; t < n_target; t++) dev[t] = c[target_idx[t]] - pred[t];
    float mag = spo_hier_residual_quantize(dev, n_target, rbits, lv);
    memcpy(out + skel_bc->total_bytes, &mag, 4);
    spo_pack_levels(lv, n_target, rbits, out + skel_bc->total_bytes + 4);
}

/* Hier read (sp_cuda_hier_read_one, shannon_prime_hier.cu:490-571). */
void spo_hier_decompress(const uint8_t *in, float *out, int hd, int pad,
                         int n_skel, const int *skel_idx, int n_target, const int *target_idx,
                         const spo_band_config_t *skel_bc, const uint16_t *W, int rbits) {
    float c[1024], skel[1024], pred[1024];
    uint8_t lv[1024];
    int f[16];
    int nf = spo_factor_small(pad, f, 16);
    spo_band_dequantize(in, skel, skel_bc);
    spo_hier_predict(W, skel, pred, n_target, n_skel);
    float mag;
    memcpy(&mag, in + skel_bc->total_bytes, 4);
    spo_unpack_levels(in + skel_bc->total_bytes + 4, n_target, rbits, lv);
    float dv[1024];
    spo_hier_residual_dequantize(lv, n_target, rbits, mag, dv);
    for (int i = 0; i < pad; i++) c[i] = 0.0f;
    for (int s = 0; s < n_skel; s++) c[skel_idx[s]] = skel[s];
    for (int t = 0; t < n_target; t++) c[target_idx[t]] = pred[t] + dv[t];
    spo_vilenkin(c, pad, f, nf);
    for (int i = 0; i < hd; i++) out[i] = c[i];
}

void spo_hier_compress_batch_f16(const uint16_t *in, uint8_t *out, int n, int hd, int pad,
                                 int n_skel, const int *skel_idx, int n_target,
                                 const int *target_idx, const spo_band_config_t *skel_bc,
                                 const uint16_t *W, int rbits) {
    int B = spo_hier_bytes(skel_bc, n_target, rbits);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++) {
        float v[1024];
        for (int i = 0; i < hd; i++) v[i] = spo_f16_to_f32(in[(size_t)t * hd + i]);
        spo_hier_compress(v, out + (size_t)t * B, hd, pad, n_skel, skel_idx, n_target,
                          target_idx, skel_bc, W, rbits);
    }
}

void spo_hier_decompress_batch_f32(const uint8_t *in, float *out, int n, int hd, int pad,
                                   int n_skel, const int *skel_idx, int n_target,
                                   const int *target_idx, const spo_band_config_t *skel_bc,
                                   const uint16_t *W, int rbits) {
    int B = spo_hier_bytes(skel_bc, n_target, rbits);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; t++)
        spo_hier_decompress(in + (size_t)t * B, out + (size_t)t * hd, hd, pad, n_skel, skel_idx,
                            n_target, target_idx, skel_bc, W, rbits);
}

/* ------------------------------------------------------------------------ */
/* decode attention                                                         */
/* ------------------------------------------------------------------------ */

/* Decode attention over records, in double: every K~ / V~ row of a KV head is
 * reconstructed by the codec's own read path (row(), the records' decompress),
 * then, per query head h of the head's group (llama.cpp's GQA grouping
 * h -> h / (n_q / n_kvh)), s_t = kq_scale * sum_d q[h][d] K~_t[d] accumulated
 * over d in order, softmax with the maximum subtracted, and
 * out[h] = sum_t p_t V~_t / sum_t p_t accumulated over t in order. The rows of
 * a head are reconstructed in parallel (each row independently, so the result
 * does not depend on the thread count); the sums are serial. */
typedef void (*spo_row_fn)(const void *ctx, int is_v, int kvh, int t, float *row);

static void attn_core(const float *q, int n_q, int n_kvh, int n_ctx, int hd, float kq_scale,
                      spo_row_fn row, const void *ctx, float *scores, float *out) {
    int grp = n_q / n_kvh;
    size_t nr = (size_t)(n_ctx > 0 ? n_ctx : 1);
    float *rows = (float *)malloc(sizeof(float) * nr * (size_t)hd);
    double *s = (double *)malloc(sizeof(double) * nr * (size_t)grp);
    double *o = (double *)malloc(sizeof(double) * (size_t)hd);
    for (int kh = 0; kh < n_kvh; kh++) {
#pragma omp parallel for schedule(static)
        for (int t = 0; t < n_ctx; t++) row(ctx, 0, kh, t, rows + (size_t)t * hd);
        for (int g = 0; g < grp; g++) {
            int h = kh * grp + g;
            double *sh = s + (size_t)g * nr;
            for (int t = 0; t < n_ctx; t++) {
                const float *kt = rows + (size_t)t * hd;
                double acc = 0.0;
                for (int d = 0; d < hd; d++) acc += (double)q[(size_t)h * hd + d] * (double)kt[d];
                sh[t] = acc * (double)kq_scale;
                if (scores) scores[(size_t)h * n_ctx + t] = (float)sh[t];
            }
        }
        if (!out) continue;
#pragma omp parallel for schedule(static)
        for (int t = 0; t < n_ctx; t++) row(ctx, 1, kh, t, rows + (size_t)t * hd);
        for (int g = 0; g < grp; g++) {
            int h = kh * grp + g;
            const double *sh = s + (size_t)g * nr;
            double mx = -INFINITY;
            for (int t = 0; t < n_ctx; t++)
                if (sh[t] > mx) mx = sh[t];
            double l = 0.0;
            for (int d = 0; d < hd; d++) o[d] = 0.0;
            for (int t = 0; t < n_ctx; t++) {
                double p = exp(sh[t] - mx);
                l += p;
                const float *vt = rows + (size_t)t * hd;
                for (int d = 0; d < hd; d++) o[d] += p * (double)vt[d];
            }
            for (int d = 0; d < hd; d++) out[(size_t)h * hd + d] = (float)(o[d] / l);
        }
    }
    free(rows);
    free(s);
    free(o);
}

/* ship records: the read path with bands >= max_bands read as 0 */
typedef struct {
    const uint8_t *kpack, *vpack;
    int n_ctx;
    const spo_band_config_t *kbc, *vbc;
    const int *order;
    int norm_mode, max_bands;
} ship_rows_t;

static void ship_row(const void *ctx, int is_v, int kvh, int t, float *row) {
    const ship_rows_t *c = (const ship_rows_t *)ctx;
    const spo_band_config_t *bc = is_v ? c->vbc : c->kbc;
    const uint8_t *pk = is_v ? c->vpack : c->kpack;
    spo_ship_decompress(pk + ((size_t)kvh * c->n_ctx + t) * bc->total_bytes, row, bc, is_v ? NULL : c->order,
                        c->norm_mode, c->max_bands);
}

/* hier records: spo_hier_decompress with the KV head's predictor W[kvh] */
typedef struct {
    const uint8_t *kpack, *vpack;
    int n_ctx, hd, pad, n_skel, n_target, rbits, B;
    const int *skel_idx, *target_idx;
    const spo_band_config_t *skel_bc;
    const uint16_t *W;
} hier_rows_t;

static void hier_row(const void *ctx, int is_v, int kvh, int t, float *row) {
    const hier_rows_t *c = (const hier_rows_t *)ctx;
    const uint8_t *pk = is_v ? c->vpack : c->kpack;
    spo_hier_decompress(pk + ((size_t)kvh * c->n_ctx + t) * c->B, row, c->hd, c->pad, c->n_skel, c->skel_idx,
                        c->n_target, c->target_idx, c->skel_bc, c->W + (size_t)kvh * c->n_target * c->n_skel,
                        c->rbits);
}

/* sqfree records: spo_sqfree_decompress, K and V each with their skeleton bands */
typedef struct {
    const uint8_t *kpack, *vpack;
    int n_ctx, hd, rbits, spinor;
    const spo_knight_mask_t *m;
    const spo_band_config_t *kbc, *vbc;
} sqfree_rows_t;

static void sqfree_row(const void *ctx, int is_v, int kvh, int t, float *row) {
    const sqfree_rows_t *c = (const sqfree_rows_t *)ctx;
    const spo_band_config_t *bc = is_v ? c->vbc : c->kbc;
    const uint8_t *pk = is_v ? c->vpack : c->kpack;
    int B = spo_sqfree_bytes(bc, c->m->n_res, c->rbits, c->spinor);
    spo_sqfree_decompress(pk + ((size_t)kvh * c->n_ctx + t) * B, row, c->hd, c->m, bc, c->rbits, c->spinor);
}

/* Score semantics of llama_sp_kq_compute (src/engine/llama_sp_fused_kq.cpp:
 * 83-165): dst[qh][kv] = sum_d q[qh][d] * K~[kv][d], K~ decompressed from the
 * packed archive. This oracle decompresses with the full read path (including
 * the Mobius unreorder the reference op omits, :131-139), applies llama.cpp's
 * GQA grouping qh -> qh / (n_q / n_kvh) and kq_scale, then softmax and . V~. */
void spo_attn_decode(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                     int n_q, int n_kvh, int n_ctx, int hd,
                     const spo_band_config_t *kbc, const spo_band_config_t *vbc,
                     const int *order, int norm_mode, float kq_scale,
                     float *scores, float *out) {
    spo_attn_decode_bands(q, kpack, vpack, n_q, n_kvh, n_ctx, hd, kbc, vbc, order, norm_mode, kq_scale,
                          scores, out, -1);
}

/* Attention over the partial reconstructions (bands >= max_bands read as 0, the
 * read_k/v_partial semantics of shannon_prime_llama.h:240-255, applied to K and V
 * as the post-decode hook does, llama-cpp-b8861-full-engine.patch:1336-1337). */
void spo_attn_decode_bands(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                           int n_q, int n_kvh, int n_ctx, int hd,
                           const spo_band_config_t *kbc, const spo_band_config_t *vbc,
                           const int *order, int norm_mode, float kq_scale,
                           float *scores, float *out, int max_bands) {
    ship_rows_t c = {kpack, vpack, n_ctx, kbc, vbc, order, norm_mode, max_bands};
    attn_core(q, n_q, n_kvh, n_ctx, hd, kq_scale, ship_row, &c, scores, out);
}

/* The same scores / softmax / . V in double over hier records: a position's K~
 * and V~ are spo_hier_decompress of its records with its KV head's predictor
 * W[kh]. Not a reference op (the reference's fused op is ship-only,
 * llama_sp_fused_kq.cpp:14-34); it is the attention a caller gets by reading the
 * hier cache back and attending over it. */
void spo_hier_attn_decode(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                          int n_q, int n_kvh, int n_ctx, int hd, int pad,
                          int n_skel, const int *skel_idx, int n_target, const int *target_idx,
                          const spo_band_config_t *skel_bc, const uint16_t *W, int rbits,
                          float kq_scale, float *scores, float *out) {
    hier_rows_t c = {kpack, vpack, n_ctx, hd, pad, n_skel, n_target, rbits,
                     spo_hier_bytes(skel_bc, n_target, rbits), skel_idx, target_idx, skel_bc, W};
    attn_core(q, n_q, n_kvh, n_ctx, hd, kq_scale, hier_row, &c, scores, out);
}

/* The same attention over sqfree(+spinor) records: K~ and V~ are
 * spo_sqfree_decompress of the records (the read path of sp_cuda_sqfree_read_one,
 * shannon_prime_sqfree.cu:857-950, which the reference's hook calls per vector
 * before its attention, llama-cpp-b8861-full-engine.patch:1205-1207), K with the
 * K skeleton bands and V with the V bands, one Knight mask for both. Not a
 * reference op (the reference's fused op is ship-only, llama_sp_fused_kq.cpp:
 * 14-34). */
void spo_sqfree_attn_decode(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                            int n_q, int n_kvh, int n_ctx, int hd, const spo_knight_mask_t *m,
                            const spo_band_config_t *kbc, const spo_band_config_t *vbc, int rbits, int spinor,
                            float kq_scale, float *scores, float *out) {
    sqfree_rows_t c = {kpack, vpack, n_ctx, hd, rbits, spinor, m, kbc, vbc};
    attn_core(q, n_q, n_kvh, n_ctx, hd, kq_scale, sqfree_row, &c, scores, out);
}

/* Pearson correlation, accumulated in double (the fidelity metric of the
 * reference's validate_k, shannon_prime_llama.c:914-922). */
float spo_correlation_f32(const float *a, const float *b, int n) {
    double ma = 0, mb = 0;
    for (int i = 0; i < n; i++) { ma += a[i]; mb += b[i]; }
    ma /= n;
    mb /= n;
    double sab = 0, saa = 0, sbb = 0;
    for (int i = 0; i < n; i++) {
        double x = a[i] - ma, y = b[i] - mb;
        sab += x * y;
        saa += x * x;
        sbb += y * y;
    }
    if (saa <= 0 || sbb <= 0) return 0.0f;
    return (float)(sab / sqrt(saa * sbb));
}
