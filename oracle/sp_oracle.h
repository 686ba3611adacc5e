/*
 * sp_oracle.h -- CPU restatement of the Shannon-Prime KV-cache codec.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * product library (libshannon_prime_hip.so). Only tests/, the smoke() entry
 * and bench.py's cpu_baseline leg load it; no product code links or calls it.
 *
 * The reference's core math library (lib/shannon-prime, a git submodule) is
 * absent from the reference checkout, so every function below restates the
 * algorithm from the in-tree restatements that survive:
 *   - src/backends/cuda/shannon_prime_cuda.cu     (ship codec kernels)
 *   - src/backends/cuda/shannon_prime_sqfree.cu   (Vilenkin, sqfree, spinor)
 *   - src/backends/cuda/shannon_prime_hier.cu     (hierarchical predictor)
 *   - src/backends/adreno/shannon_prime_adreno.c  (CPU VHT2 operation order)
 *   - src/engine/llama_sp_fused_kq.cpp            (fused decompress-KQ)
 * Each function's comment names the file:line it follows.
 *
 * Floating-point contract: built with -O2 -ffp-contract=off -fno-fast-math,
 * so every a*b+c below is a multiply followed by a separately rounded add.
 *
 * Parity pinning (what checks each function; see tests/test_oracle_*.py):
 *   - VHT2 p=2: closed form H_n/sqrt(n) (Sylvester, natural order) in double,
 *     self-inverse, symmetric, Parseval.
 *   - Vilenkin: Kronecker product of cas blocks in double, self-inverse.
 *   - band geometry / record sizes: the reference's logged compression
 *     ratios and the "42 B at hd=64 5/5/4/3" figure.
 *   - quantizer: amax element maps to +-max_val, scale-overflow zeroes the
 *     band, amax=0, LSB-first packing known answers, brute-force minimality
 *     of the code (rint of x/scale).
 *   - fidelity: K corr > 0.985, V corr > 0.95 at hd=128 (test_adreno log).
 *   - sqfree / spinor / hier: every stage (pad mean, residual quantizers and
 *     dequantizers, spinor choice, level packing, CSR and W.skel predictions)
 *     and every whole record are compared with an independent numpy
 *     restatement of the reference's CUDA text (tests/np_restate.py,
 *     tests/test_oracle_variants.py) on inputs where the plausible misreadings
 *     differ: round-half-up vs rint, sat = mag*bits vs mag, the 1e-12 floor,
 *     the strict spinor comparison, the serial predictor order, the 256-slot
 *     reduction order; mu(n) against known values and the Mertens function;
 *     the Knight CSR against a brute-force divisor enumeration.
 *   - attention (spo_attn_decode_bands): a dense float64 softmax over the
 *     separately pinned decompressions, band-limited calls included.
 *   - hier and sqfree attention (spo_hier_attn_decode, spo_sqfree_attn_decode):
 *     against their definitions (the pinned decompressions, then a float64
 *     softmax with the GQA grouping) and against a float64 numpy restatement of
 *     the coefficient-domain algebra from the record layout alone (zero-padded
 *     query transform; hier: u = q~_skel + W^T q~_tgt; sqfree: the sheet sign on
 *     the prediction, step = 2 mag rbits / (L - 1)), tests/test_oracle_hier_attn.py
 *     and tests/test_oracle_sqfree_attn.py.
 *   - Mobius order, Knight skeleton/CSR construction rule, hier geometry: the
 *     construction rules are NOT fixed by the reference (the builder lives in
 *     the absent core); they are host-side index tables, the tests pin this
 *     build's stated rule, and the kernels' parity does not depend on how the
 *     tables are built ("parity unpinned" for the choice of rule only).
 */
#ifndef SP_ORACLE_H
#define SP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPO_MAX_BANDS 16

typedef struct {
    int head_dim;                 /* number of coefficients quantized */
    int n_bands;
    int band_bits[SPO_MAX_BANDS]; /* effective bits (ternary bands -> 2) */
    int band_size;                /* head_dim / n_bands (last band absorbs remainder) */
    int total_bytes;              /* sum_b 2 + ceil(size_b*bits_b/8) */
    uint32_t ternary_mask;
    int band_off[SPO_MAX_BANDS];       /* first coefficient of band b */
    int band_sz[SPO_MAX_BANDS];        /* coefficients in band b */
    int band_byte_off[SPO_MAX_BANDS];  /* byte offset of band b's fp16 scale */
} spo_band_config_t;

/* Normalisation convention of the p=2 VHT2 butterfly. */
enum {
    SPO_NORM_FINAL = 0, /* unnormalised butterflies, then x*(1/sqrtf(n)) (CPU core / NEON) */
    SPO_NORM_STAGE = 1  /* (u+-v)*0.70710678f per stage (CUDA kernel_vht2_p2) */
};

/* ---- config ---- */
void spo_band_config_init(spo_band_config_t *bc, int head_dim, int n_bands, const int *bits);
void spo_band_config_init_ext(spo_band_config_t *bc, int head_dim, int n_bands,
                              const int *bits, uint32_t ternary_mask);
void spo_band_span(const spo_band_config_t *bc, int b, int *off, int *sz);

/* ---- fp16 ---- */
uint16_t spo_f32_to_f16(float f);
float    spo_f16_to_f32(uint16_t h);

/* ---- transforms ---- */
int   spo_factor_small(int n, int *factors, int max_factors);
void  spo_cas_table(int p, float *C);                 /* p*p, row k col j */
float spo_inv_sqrt_n(int n);                          /* 1.0f / sqrtf((float)n) */
void  spo_vht2_p2(float *x, int n, int norm_mode);
void  spo_vilenkin(float *x, int n, const int *factors, int n_factors);
void  spo_vht2_forward(float *x, int n, int norm_mode); /* dispatch pow2 / Vilenkin */

/* ---- Mobius squarefree-first order ---- */
int  spo_is_squarefree(int n);
void spo_mobius_order(int n, int *order);             /* r -> source coefficient */
int  spo_mobius_mu(int n);

/* ---- band quantizer ---- */
void spo_band_quantize(const float *in, uint8_t *out, const spo_band_config_t *bc);
void spo_band_dequantize(const uint8_t *in, float *out, const spo_band_config_t *bc);
void spo_band_dequantize_partial(const uint8_t *in, float *out,
                                 const spo_band_config_t *bc, int max_bands);

/* ---- ship codec, one vector ---- */
void spo_ship_compress(const float *vec, uint8_t *out, const spo_band_config_t *bc,
                       const int *order, int norm_mode);
void spo_ship_decompress(const uint8_t *in, float *out, const spo_band_config_t *bc,
                         const int *order, int norm_mode, int max_bands);

/* batches: n vectors, contiguous */
void spo_ship_compress_batch_f16(const uint16_t *in, uint8_t *out, int n, int hd,
                                 const spo_band_config_t *bc, const int *order, int norm_mode);
void spo_ship_compress_batch_f32(const float *in, uint8_t *out, int n, int hd,
                                 const spo_band_config_t *bc, const int *order, int norm_mode);
void spo_ship_decompress_batch_f32(const uint8_t *in, float *out, int n, int hd,
                                   const spo_band_config_t *bc, const int *order,
                                   int norm_mode, int max_bands);
void spo_ship_decompress_batch_f16(const uint8_t *in, uint16_t *out, int n, int hd,
                                   const spo_band_config_t *bc, const int *order,
                                   int norm_mode, int max_bands);
/* same, split over n_threads OpenMP threads (CPU baseline, all-core variant) */
void spo_ship_roundtrip_batch_f16_omp(const uint16_t *in, uint8_t *packed, uint16_t *out,
                                      int n, int hd, const spo_band_config_t *bc,
                                      const int *order, int norm_mode, int n_threads);

/* ---- reductions ---- */
float spo_tree256_sum(const float *v, int n, int take_abs);

/* ---- sqfree + spinor ---- */
int  spo_sqfree_pad_dim(int hd);
typedef struct {
    int pad_dim, sk_k, n_res, n_terms;
    int *skeleton_idx;   /* [sk_k]   coefficient index of skeleton slot   */
    int *residual_idx;   /* [n_res]  coefficient index of residual r      */
    int *csr_offsets;    /* [n_res+1]                                     */
    int *csr_skel_slot;  /* [n_terms] skeleton slot feeding the term      */
    int8_t *csr_mu_sign; /* [n_terms] +-1                                 */
} spo_knight_mask_t;
int  spo_knight_mask_init(spo_knight_mask_t *m, int pad_dim, int sk_k);
void spo_knight_mask_free(spo_knight_mask_t *m);
void spo_sqfree_pad(const float *in, float *out, int hd, int pad);
/* stages of the sqfree write/read, each pinned on its own */
void  spo_pack_levels(const uint8_t *lv, int n, int bits, uint8_t *out);
void  spo_unpack_levels(const uint8_t *in, int n, int bits, uint8_t *lv);
void  spo_mobius_predict(const float *skel, const spo_knight_mask_t *m, float *pred);
void  spo_spinor_extract(const float *a, const float *p, int n, float *dev, uint8_t *sheet);
float spo_sqfree_residual_quantize(const float *dev, int n, int bits, uint8_t *lv);
void  spo_sqfree_residual_dequantize(const uint8_t *lv, int n, int bits, float mag, float *dev);
int  spo_sqfree_bytes(const spo_band_config_t *skel_bc, int n_res, int rbits, int spinor);
void spo_sqfree_compress(const float *vec, uint8_t *out, int hd, const spo_knight_mask_t *m,
                         const spo_band_config_t *skel_bc, int rbits, int spinor);
void spo_sqfree_decompress(const uint8_t *in, float *out, int hd, const spo_knight_mask_t *m,
                           const spo_band_config_t *skel_bc, int rbits, int spinor);
void spo_sqfree_compress_batch_f16(const uint16_t *in, uint8_t *out, int n, int hd,
                                   const spo_knight_mask_t *m, const spo_band_config_t *skel_bc,
                                   int rbits, int spinor);
void spo_sqfree_decompress_batch_f32(const uint8_t *in, float *out, int n, int hd,
                                     const spo_knight_mask_t *m, const spo_band_config_t *skel_bc,
                                     int rbits, int spinor);

/* ---- hierarchical ---- */
void spo_hier_default_geometry(int pad, int *n_skel);
void spo_hier_indices(int pad, int n_skel, int *skel_idx, int *target_idx);
int  spo_hier_bytes(const spo_band_config_t *skel_bc, int n_target, int rbits);
/* stages of the hier write/read, each pinned on its own */
void  spo_hier_predict(const uint16_t *W, const float *skel, float *pred, int nt, int ns);
float spo_hier_residual_quantize(const float *dev, int n, int bits, uint8_t *lv);
void  spo_hier_residual_dequantize(const uint8_t *lv, int n, int bits, float mag, float *dev);
void spo_hier_compress(const float *vec, uint8_t *out, int hd, int pad,
                       int n_skel, const int *skel_idx, int n_target, const int *target_idx,
                       const spo_band_config_t *skel_bc, const uint16_t *W, int rbits);
void spo_hier_decompress(const uint8_t *in, float *out, int hd, int pad,
                         int n_skel, const int *skel_idx, int n_target, const int *target_idx,
                         const spo_band_config_t *skel_bc, const uint16_t *W, int rbits);
void spo_hier_compress_batch_f16(const uint16_t *in, uint8_t *out, int n, int hd, int pad,
                                 int n_skel, const int *skel_idx, int n_target,
                                 const int *target_idx, const spo_band_config_t *skel_bc,
                                 const uint16_t *W, int rbits);
void spo_hier_decompress_batch_f32(const uint8_t *in, float *out, int n, int hd, int pad,
                                   int n_skel, const int *skel_idx, int n_target,
                                   const int *target_idx, const spo_band_config_t *skel_bc,
                                   const uint16_t *W, int rbits);

/* ---- decode attention over compressed K/V ---- */
/* q: [n_q][hd] fp32; kpack/vpack: [n_kvh][n_ctx][B]; grouping qh -> qh / (n_q/n_kvh).
 * scores (optional): [n_q][n_ctx] = kq_scale * q . K~ ; out (optional): [n_q][hd]
 * softmax(scores) . V~ . Computed in double from the oracle's fp32 reconstructions. */
void spo_attn_decode(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                     int n_q, int n_kvh, int n_ctx, int hd,
                     const spo_band_config_t *kbc, const spo_band_config_t *vbc,
                     const int *order, int norm_mode, float kq_scale,
                     float *scores, float *out);
/* The same over the partial reconstructions: K and V bands >= max_bands read as 0
 * (max_bands < 0: every band). */
void spo_attn_decode_bands(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                           int n_q, int n_kvh, int n_ctx, int hd,
                           const spo_band_config_t *kbc, const spo_band_config_t *vbc,
                           const int *order, int norm_mode, float kq_scale,
                           float *scores, float *out, int max_bands);

/* Decode attention over hier records (the hier cache's K and V arrays,
 * [n_kvh][n_ctx][bytes] each, W [n_kvh][n_target][n_skel] fp16 per KV head):
 * spo_attn_decode's arithmetic with K~ and V~ from spo_hier_decompress. */
void spo_hier_attn_decode(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                          int n_q, int n_kvh, int n_ctx, int hd, int pad,
                          int n_skel, const int *skel_idx, int n_target, const int *target_idx,
                          const spo_band_config_t *skel_bc, const uint16_t *W, int rbits,
                          float kq_scale, float *scores, float *out);
/* spo_attn_decode's arithmetic with K~ and V~ from spo_sqfree_decompress (K with
 * the K skeleton bands kbc, V with vbc; one Knight mask). */
void spo_sqfree_attn_decode(const float *q, const uint8_t *kpack, const uint8_t *vpack,
                            int n_q, int n_kvh, int n_ctx, int hd, const spo_knight_mask_t *m,
                            const spo_band_config_t *kbc, const spo_band_config_t *vbc, int rbits, int spinor,
                            float kq_scale, float *scores, float *out);

/* ---- metrics ---- */
float spo_correlation_f32(const float *a, const float *b, int n);

#ifdef __cplusplus
}
#endif
#endif
