/*
 * shannon_prime.h -- core types and the sp_shadow_cache_t write/read API,
 * implemented on MI355X (gfx950) by libshannon_prime_hip.so.
 *
 * This re-declares the core C API that the reference bridge and engine call.
 * The reference header (lib/shannon-prime/core/shannon_prime.h, included at
 * src/tools/shannon_prime_llama.h:87) is absent from the reference checkout;
 * the signatures below are inferred from its call sites, cited per entry.
 *
 * Every codec call below runs on the GPU: host vectors are staged to device
 * memory, the HIP kernels compress or reconstruct them, and results come back
 * to the caller's host buffers. There is no CPU codec path in this library;
 * when no gfx950 device is present the init calls fail (return -1 / NULL).
 */
#ifndef SHANNON_PRIME_H
#define SHANNON_PRIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SP_MAX_BANDS    16
#define SP_MAX_HEAD_DIM 1024

/* VHT2 p=2 normalisation convention (extension; the reference's CPU core and
 * its CUDA kernel disagree, see shannon_prime_adreno.c:276-309 vs
 * shannon_prime_cuda.cu:54-69). FINAL is the default. */
#define SP_VHT2_NORM_FINAL 0
#define SP_VHT2_NORM_STAGE 1

/* Codec configuration. Fields used by the reference bridge:
 * shannon_prime_llama.c:219-294 (head_dim, n_layers, n_heads_kv, k/v_n_bands,
 * k/v_band_bits, use_mobius_mask, k/v_ternary_mask, use_fp8). */
typedef struct {
    int      head_dim;
    int      n_layers;
    int      n_heads_kv;
    int      k_n_bands;
    int      k_band_bits[SP_MAX_BANDS];
    int      v_n_bands;
    int      v_band_bits[SP_MAX_BANDS];
    int      use_mobius_mask;
    uint32_t k_ternary_mask;
    uint32_t v_ternary_mask;
    int      use_fp8;    /* advisory; this library has no fp8 path (int codes) */
    int      vht2_norm;  /* SP_VHT2_NORM_FINAL (default) or SP_VHT2_NORM_STAGE */
} sp_config_t;

/* Banded quantizer geometry (sp_band_config_t; fields used at
 * shannon_prime_cuda.cu:360-375, shannon_prime_vulkan.c:559-578). */
typedef struct {
    int      head_dim;
    int      n_bands;
    int      band_bits[SP_MAX_BANDS];
    int      band_size;     /* head_dim / n_bands; last band absorbs remainder */
    int      total_bytes;   /* sum_b 2 + ceil(size_b * bits_b / 8) */
    uint32_t ternary_mask;  /* bit b: band b stored as {-1,0,+1} at 2 bits */
} sp_band_config_t;

/* Mobius squarefree-first permutation (sp_mobius_mask_t; .order used at
 * shannon_prime_cuda.cu:428-445). order[r] = coefficient at position r. */
typedef struct {
    int  n;
    int *order;
} sp_mobius_mask_t;

/* Ship shadow cache (sp_shadow_cache_t; fields used at
 * shannon_prime_llama.c:413-428 and kv_cache.cpp:361-376). k_cache/v_cache are
 * allocated by the CALLER: n_slots pointers, each max_seq * total_bytes bytes,
 * slot = layer * n_heads_kv + head, record at pos * total_bytes. */
typedef struct {
    sp_config_t      config;
    sp_band_config_t k_bands;
    sp_band_config_t v_bands;
    sp_mobius_mask_t mobius_mask;
    uint8_t        **k_cache;
    uint8_t        **v_cache;
    /* calibration (fields the engine reads and writes, kv_cache.cpp:553-585, 633-641):
     * per-coefficient sums of the forward transform of the fed K vectors, the count,
     * and after sp_shadow_calibrate_end the coefficients ranked by descending variance */
    int              calibrating;
    double          *calib_sum;    /* [head_dim] */
    double          *calib_sum2;   /* [head_dim] */
    long long        calib_n;
    int             *var_order;    /* [head_dim] */
    int              use_var_reorder;
    void            *dev;   /* device-side state owned by the library */
} sp_shadow_cache_t;

/* ---- config (sp_config_init: shannon_prime_llama.c:220; kv_cache.cpp:298) ---- */
void sp_config_init(sp_config_t *cfg, int head_dim, int n_layers, int n_heads_kv);
void sp_config_print(const sp_config_t *cfg);

/* ---- band geometry (sp_band_config_init: shannon_prime_cuda.cu:413-416;
 *      _ext: CHANGELOG.md:109-116; sp_band_span: shannon_prime_vulkan.c:559) ---- */
void sp_band_config_init(sp_band_config_t *bc, int head_dim, int n_bands, const int *band_bits);
void sp_band_config_init_ext(sp_band_config_t *bc, int head_dim, int n_bands,
                             const int *band_bits, uint32_t ternary_mask);
void sp_band_span(const sp_band_config_t *bc, int band, int *offset, int *size);

/* ---- Mobius mask (shannon_prime_cuda.cu:428-445) ---- */
int  sp_mobius_mask_init(sp_mobius_mask_t *mask, int n);
void sp_mobius_mask_free(sp_mobius_mask_t *mask);

/* ---- shadow cache (shannon_prime_llama.c:413, 596-825) ----
 * init returns 0 on success, -1 on bad config or when no GPU is usable. */
int  sp_shadow_cache_init(sp_shadow_cache_t *sc, const sp_config_t *cfg);
void sp_shadow_cache_free(sp_shadow_cache_t *sc);

void sp_shadow_write_k(sp_shadow_cache_t *sc, int layer, int head, int pos, const float *k_vec);
void sp_shadow_write_v(sp_shadow_cache_t *sc, int layer, int head, int pos, const float *v_vec);
void sp_shadow_write_k_batch(sp_shadow_cache_t *sc, int layer, int head,
                             int start_pos, int n_pos, const float *k_vecs);
void sp_shadow_write_v_batch(sp_shadow_cache_t *sc, int layer, int head,
                             int start_pos, int n_pos, const float *v_vecs);

void sp_shadow_read_k(const sp_shadow_cache_t *sc, int layer, int head, int pos, float *k_out);
void sp_shadow_read_v(const sp_shadow_cache_t *sc, int layer, int head, int pos, float *v_out);
void sp_shadow_read_k_partial(const sp_shadow_cache_t *sc, int layer, int head, int pos,
                              float *k_out, int max_bands);
void sp_shadow_read_v_partial(const sp_shadow_cache_t *sc, int layer, int head, int pos,
                              float *v_out, int max_bands);
void sp_shadow_read_k_batch(const sp_shadow_cache_t *sc, int layer, int head,
                            int start_pos, int n_pos, float *k_out);
void sp_shadow_read_v_batch(const sp_shadow_cache_t *sc, int layer, int head,
                            int start_pos, int n_pos, float *v_out);

/* ---- Knight mask (sp_knight_mask_init / _free, shannon_prime_sqfree.cu:606-657):
 *      skeleton = the first sk_k coefficients of `ranking` (NULL: the squarefree-first
 *      order), residuals = the rest; CSR row r lists the skeleton slots of the proper
 *      divisors d of n = residual_idx[r] + 1 with coefficient d - 1 in the skeleton
 *      and mu(n/d) != 0, with sign mu(n/d). Host memory; _free releases it. ---- */
typedef struct {
    int     pad_dim;
    int     sk_k;
    int     n_res;
    int     n_terms;
    int    *skeleton_idx;   /* [sk_k] */
    int    *residual_idx;   /* [n_res] */
    int    *csr_offsets;    /* [n_res + 1] */
    int    *csr_skel_slot;  /* [n_terms] */
    int8_t *csr_mu_sign;    /* [n_terms] */
} sp_knight_mask_t;
int  sp_knight_mask_init(sp_knight_mask_t *m, int pad_dim, int sk_k, const int *ranking);
void sp_knight_mask_free(sp_knight_mask_t *m);

/* ---- per-vector core calls on host pointers (the absent core's sp_vht2_forward_f32,
 *      used at llama_sp_fused_kq.cpp:33 and kv_cache.cpp:399, and its band codec
 *      sp_band_quantize / sp_band_dequantize / _partial, semantics at
 *      shannon_prime_llama.h:240-255): computed on the device by the caches' kernels
 *      through a staging round trip; VHT2 with the final 1/sqrt(n) normalisation. ---- */
void sp_vht2_forward_f32(float *data, int n);
void sp_band_quantize(const float *in, uint8_t *out, const sp_band_config_t *bc);
void sp_band_dequantize(const uint8_t *in, float *out, const sp_band_config_t *bc);
void sp_band_dequantize_partial(const uint8_t *in, float *out, const sp_band_config_t *bc, int max_bands);

/* ---- disk (sp_shadow_cache_save / _load, kv_cache.cpp:1549, 1572; the partial load
 *      of the disk tier, CHANGELOG.md): the v3 files of sp_hip_cache_save (one per
 *      layer, {prefix}.L{layer}.bin), read and written from the host record buffers;
 *      the header carries the model hash (strict unless SP_DISK_HASH_STRICT=0).
 *      save returns 0, the loads the n_pos stored; -1 on any error. ---- */
int  sp_shadow_cache_save(const sp_shadow_cache_t *sc, const char *prefix, int n_pos, uint64_t model_hash);
int  sp_shadow_cache_load(sp_shadow_cache_t *sc, const char *prefix, uint64_t expected_hash);
int  sp_shadow_cache_load_partial(sp_shadow_cache_t *sc, const char *prefix, uint64_t expected_hash, int max_bands);
/* Positions each caller-owned slot buffer (k_cache[s], v_cache[s]) holds. Extension: the
 * reference's API never tells the core, but save and load need it to stay inside the
 * buffers: they refuse files (or n_pos) beyond it, and fail until it is set. The loads
 * check every layer's file before changing any record. 0, or -1 for bad arguments. */
int  sp_shadow_cache_set_slot_capacity(sp_shadow_cache_t *sc, int n_positions);

/* ---- calibration (sp_shadow_calibrate_begin/feed/end, called at kv_cache.cpp:525,
 * 587, 610). begin clears the sums; feed adds one host fp32 K vector's transform
 * (computed on the device by the cache's own transform); end ranks the coefficients
 * by descending variance sum2/n - (sum/n)^2 (ties: lower index first) into var_order,
 * sets use_var_reorder and makes var_order the K coefficient order of every later
 * write and read. 0 on success, -1 without data. ---- */
int  sp_shadow_calibrate_begin(sp_shadow_cache_t *sc);
void sp_shadow_calibrate_feed(sp_shadow_cache_t *sc, const float *vec);
int  sp_shadow_calibrate_end(sp_shadow_cache_t *sc);

/* ---- utilities (shannon_prime_llama.c:919, 932; shannon_prime_hexagon.c:234-242) ---- */
float    sp_correlation_f32(const float *a, const float *b, int n);
float    sp_compression_ratio(const sp_config_t *cfg);
float    sp_f16_to_f32(uint16_t h);
uint16_t sp_f32_to_f16(float f);

/* ---- sqfree geometry (sp_sqfree_pad_dim: shannon_prime_sqfree.cu:600) ---- */
int sp_sqfree_pad_dim(int head_dim);

/* ---- sqfree + spinor cache on host vectors: the absent core's sp_sqfree_cache_t,
 * as the b8861 hook calls it (llama-cpp-b8861-full-engine.patch:790-791 init,
 * :851/:866 free, :1206-1207 K and :1274-1275, :1333-1334 V write/read round
 * trips), the sqfree bridge (shannon_prime_llama_sqfree.c:145-240) and the
 * engine (kv_cache.cpp:337-346, 523, 549, 608, 1547, 1570). The records live in
 * HBM in a device cache the library owns (sp_hip_sqfree_cache_t); each call
 * stages its vector through pinned host memory and runs the device kernels, so
 * records and reconstructions equal the device cache's bit for bit. A GPU is
 * required: init returns -1 without one. Skeleton = pad_dim / 2 as in the
 * reference's sqfree cache (shannon_prime_sqfree.cu:606); K bands over the
 * skeleton from cfg->k_band_bits (default 5,4,4,4,5), V from cfg->v_band_bits.
 * Record [skeleton bands][f32 mag][residual][sheet] (shannon_prime_sqfree.cu:683-686). */
typedef struct {
    sp_config_t      config;
    int              pad_dim;
    sp_knight_mask_t mask;          /* host copy of the tables the device uses */
    sp_band_config_t k_bands;       /* over mask.sk_k skeleton coefficients */
    sp_band_config_t v_bands;
    int              residual_bits;
    int              use_spinor;
    int              max_seq_len;
    int              bytes_per_pos_k;
    int              bytes_per_pos_v;
    void            *dev;           /* device cache and staging owned by the library */
} sp_sqfree_cache_t;

int  sp_sqfree_cache_init(sp_sqfree_cache_t *c, const sp_config_t *cfg, int max_seq_len,
                          int residual_bits, int use_spinor);
void sp_sqfree_cache_free(sp_sqfree_cache_t *c);
/* void calls ignore bad arguments, as the reference's writers and readers do */
void sp_sqfree_write_k(sp_sqfree_cache_t *c, int layer, int head, int pos, const float *k_vec);
void sp_sqfree_write_v(sp_sqfree_cache_t *c, int layer, int head, int pos, const float *v_vec);
void sp_sqfree_read_k(const sp_sqfree_cache_t *c, int layer, int head, int pos, float *k_out);
void sp_sqfree_read_v(const sp_sqfree_cache_t *c, int layer, int head, int pos, float *v_out);
/* Knight-mask recalibration (kv_cache.cpp:523, 549, 608): begin clears, feed adds
 * one host K vector's padded transform, end ranks the coefficients by variance and
 * rebuilds the Knight tables (device and c->mask) for later writes and reads.
 * 0 on success, -1 without data. */
int  sp_sqfree_calibrate_begin(sp_sqfree_cache_t *c);
void sp_sqfree_calibrate_feed(sp_sqfree_cache_t *c, const float *vec);
int  sp_sqfree_calibrate_end(sp_sqfree_cache_t *c);
/* v3 files as sp_hip_sqfree_cache_save/load (kv_cache.cpp:1547, 1570). */
int  sp_sqfree_cache_save(const sp_sqfree_cache_t *c, const char *prefix, int n_pos, uint64_t model_hash);
int  sp_sqfree_cache_load(sp_sqfree_cache_t *c, const char *prefix, uint64_t expected_hash);

/* ---- hierarchical cache on host vectors: the absent core's sp_hier_cache_t as the
 * engine calls it (kv_cache.cpp:326-336 init, 211-212 free, 444-446 / 502-504
 * write and read, 521, 594, 606, 765 calibration, 1545 / 1568 disk) and reads its
 * predictors (:270-277, 724-751, 870-876). Records live in HBM in a device cache
 * the library owns (sp_hip_hier_cache_t), as for the sqfree cache above. Every
 * slot shares the geometry (sp_hier_default_geometry); predictors[s].W is a host
 * copy of slot s's fp16 predictor [n_target][n_skeleton], zero until calibrated,
 * refreshed by calibrate_end(_ema) and load (changes made to it are not used by
 * the device). */
typedef struct {
    int              pad_dim;
    int              n_skeleton;
    int              n_target;
    int             *skeleton_idx;    /* [n_skeleton] */
    int             *target_idx;      /* [n_target] */
    sp_band_config_t skel_bands;
    int              target_res_bits;
    uint16_t        *W;               /* [n_target][n_skeleton] fp16 */
} sp_hier_predictor_t;

typedef struct {
    sp_config_t          config;
    int                  pad_dim;
    int                  n_slots;      /* n_layers * n_heads_kv */
    int                  max_seq_len;
    int                  level;
    sp_hier_predictor_t *predictors;   /* [n_slots] */
    int                  bytes_per_pos;
    void                *dev;          /* device cache and staging owned by the library */
} sp_hier_cache_t;

/* level 0 (the engine's default, "auto") selects sp_hier_default_geometry; other
 * levels are refused (-1): their grouping rule lives in the absent core.
 * n_skel_bands / skel_bits: skeleton band bits (default 5,5); res_bits 1..4
 * (default 2). 0 on success, -1 on bad arguments or without a GPU. */
int  sp_hier_cache_init(sp_hier_cache_t *hc, const sp_config_t *cfg, int max_seq_len, int level,
                        int n_skel_bands, const int *skel_bits, int res_bits);
void sp_hier_cache_free(sp_hier_cache_t *hc);
void sp_hier_cache_write_k(sp_hier_cache_t *hc, int layer, int head, int pos, const float *k_vec);
void sp_hier_cache_write_v(sp_hier_cache_t *hc, int layer, int head, int pos, const float *v_vec);
void sp_hier_cache_read_k(const sp_hier_cache_t *hc, int layer, int head, int pos, float *k_out);
void sp_hier_cache_read_v(const sp_hier_cache_t *hc, int layer, int head, int pos, float *v_out);
/* Predictor fit per slot (ridge 1e-6 of trace/n_skeleton, as sp_hip_hier_calibrate_end). */
int  sp_hier_cache_calibrate_begin(sp_hier_cache_t *hc);
void sp_hier_cache_calibrate_feed(sp_hier_cache_t *hc, int slot, const float *vec);
int  sp_hier_cache_calibrate_end(sp_hier_cache_t *hc);
int  sp_hier_cache_calibrate_end_ema(sp_hier_cache_t *hc, float keep_frac);
int  sp_hier_cache_save(const sp_hier_cache_t *hc, const char *prefix, int n_pos, uint64_t model_hash);
int  sp_hier_cache_load(sp_hier_cache_t *hc, const char *prefix, uint64_t expected_hash);

/* ---- hier geometry. The reference's core chooses it inside sp_hier_cache_init
 * (called at kv_cache.cpp:326-329; "n_target typically ~130" at
 * shannon_prime_hier.cu:114); its rule is not recoverable. This build's default:
 * skeleton = the first ceil(0.09 * pad_dim) entries of the squarefree-first order
 * over [0, pad_dim), targets = the rest in that order. Returns n_skeleton (or -1);
 * skeleton_idx [n_skeleton] and target_idx [pad_dim - n_skeleton] may be NULL. */
int sp_hier_default_geometry(int pad_dim, int *skeleton_idx, int *target_idx);

#ifdef __cplusplus
}
#endif
#endif /* SHANNON_PRIME_H */
