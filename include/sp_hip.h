/*
 * sp_hip.h -- MI355X (gfx950) device API of the Shannon-Prime KV codec.
 *
 * Replaces the reference's CUDA backend boundary (src/backends/cuda/
 * shannon_prime_cuda.h:29-378): the same cache objects (ship, sqfree, hier)
 * with device pointers and a stream (void* = hipStream_t, NULL = default
 * stream), plus fp16 entry points, layer-wide device-resident writes/reads
 * and the fused decompress-attention launcher (replacing the CPU ggml custom
 * op llama_sp_kq_compute, src/engine/llama_sp_fused_kq.h:95-99).
 *
 * Conventions: functions returning int give 0 on success and -1 on a bad
 * argument (nothing is launched); void functions ignore bad arguments like the
 * reference's. All launches are asynchronous on the cache's stream.
 */
#ifndef SP_HIP_H
#define SP_HIP_H

#include "shannon_prime.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SP_DTYPE_F32 0
#define SP_DTYPE_F16 1

/* ======================================================================== */
/* Ship cache  (sp_cuda_cache_t, shannon_prime_cuda.h:29-46)                */
/* ======================================================================== */

typedef struct {
    sp_config_t      config;
    sp_band_config_t k_bands;
    sp_band_config_t v_bands;
    void            *d_k_cache;       /* [n_layers*n_heads_kv][max_seq][k_bytes] */
    void            *d_v_cache;       /* [n_layers*n_heads_kv][max_seq][v_bytes] */
    int              max_seq_len;
    int             *d_mobius_order;  /* [head_dim] r -> coefficient (NULL: no Mobius) */
    int             *d_mobius_inv;    /* [head_dim] coefficient -> r */
    void            *stream;
    void            *priv;            /* library-owned launch plans and workspace */
} sp_hip_cache_t;

/* shannon_prime_cuda.h:50-52 */
int  sp_hip_cache_init(sp_hip_cache_t *cc, const sp_config_t *cfg, int max_seq_len, void *stream);
void sp_hip_cache_free(sp_hip_cache_t *cc);

/* single vector, device fp32 (shannon_prime_cuda.h:61-81) */
void sp_hip_write_k(sp_hip_cache_t *cc, int layer, int head, int pos, const float *d_k_vec);
void sp_hip_write_v(sp_hip_cache_t *cc, int layer, int head, int pos, const float *d_v_vec);
void sp_hip_read_k(const sp_hip_cache_t *cc, int layer, int head, int pos, float *d_k_out);
void sp_hip_read_v(const sp_hip_cache_t *cc, int layer, int head, int pos, float *d_v_out);

/* batches of one slot, [n_pos][head_dim] contiguous (shannon_prime_cuda.h:91-110) */
void sp_hip_write_k_batch(sp_hip_cache_t *cc, int layer, int head, int start_pos, int n_pos,
                          const float *d_k_vecs);
void sp_hip_write_v_batch(sp_hip_cache_t *cc, int layer, int head, int start_pos, int n_pos,
                          const float *d_v_vecs);
void sp_hip_read_k_batch(const sp_hip_cache_t *cc, int layer, int head, int start_pos, int n_pos,
                         float *d_k_out);
void sp_hip_read_v_batch(const sp_hip_cache_t *cc, int layer, int head, int start_pos, int n_pos,
                         float *d_v_out);

/* Partial-band batch reads (semantics of shannon_prime_llama.h:240-255). */
void sp_hip_read_k_batch_partial(const sp_hip_cache_t *cc, int layer, int head, int start_pos,
                                 int n_pos, float *d_k_out, int max_bands);
void sp_hip_read_v_batch_partial(const sp_hip_cache_t *cc, int layer, int head, int start_pos,
                                 int n_pos, float *d_v_out, int max_bands);

/* fp16 batches (precedent: sp_adreno_write_k_f16, shannon_prime_adreno.h). */
void sp_hip_write_k_batch_f16(sp_hip_cache_t *cc, int layer, int head, int start_pos, int n_pos,
                              const void *d_k_f16);
void sp_hip_write_v_batch_f16(sp_hip_cache_t *cc, int layer, int head, int start_pos, int n_pos,
                              const void *d_v_f16);
void sp_hip_read_k_batch_f16(const sp_hip_cache_t *cc, int layer, int head, int start_pos,
                             int n_pos, void *d_k_f16);
void sp_hip_read_v_batch_f16(const sp_hip_cache_t *cc, int layer, int head, int start_pos,
                             int n_pos, void *d_v_f16);

/* Layer-wide, device-resident (replaces the per-token x per-head loops of
 * KvCache::write_gpu/read_gpu, kv_cache.cpp:1045-1228, and the gather/scatter
 * of llama_sp_post_compute, llama-cpp-b8861-full-engine.patch:997-1360).
 * K/V rows use llama.cpp's cache layout: element (t, h, d) at
 * t*row_stride + h*head_dim + d, row_stride >= n_heads_kv*head_dim elements.
 * One launch covers every head and token of the layer for K and one for V. */
int sp_hip_write_layer(sp_hip_cache_t *cc, int layer, int start_pos, int n_tok,
                       const void *d_k, const void *d_v, long long row_stride, int dtype);
int sp_hip_read_layer(const sp_hip_cache_t *cc, int layer, int start_pos, int n_tok,
                      void *d_k, void *d_v, long long row_stride, int dtype, int max_bands);

/* Device form of the patch's post-decode hook (llama_sp_post_compute,
 * llama-cpp-b8861-full-engine.patch:997-1360, which gathers each new cell's
 * vector to the host, calls sp_llama_write_k/v and sp_llama_read_k/v_partial per
 * vector and scatters the reconstruction back): for every head and each of the
 * n_cells cache cells listed in d_cells (device int32, any order), compress the
 * vector held in the llama.cpp cache tensor into the records at that cell and
 * overwrite the vector with its reconstruction (bands >= max_bands read as 0;
 * max_bands < 0 reads every band). One launch for the whole layer.
 * K: element (cell, h, d) at cell*k_cell_stride + h*head_dim + d.
 * V: element (cell, h, d) at cell*v_cell_stride + (h*head_dim + d)*v_elem_stride:
 *    rows (v_elem_stride 1, v_cell_stride >= n_heads_kv*head_dim) or llama.cpp's
 *    transposed V (v_trans: v_cell_stride 1, v_elem_stride = kv_size >= max_seq).
 * NULL d_k or d_v skips that side; cells outside [0, max_seq) are skipped.
 * Head_dim 64, 128 or 256 with band boundaries on multiples of 8 coefficients
 * takes any coefficient order (default Mobius or calibrated); hd 96 needs K 5/4/4 +
 * V 5 and the default order. Returns -1 for any other layout. The power-of-two
 * widths run head_dim/8 lanes per vector with K and V in one launch; hd 96 runs one
 * vector per lane, one launch per side (SP_HIP_RT_KERNEL=narrow|lane forces either
 * kernel where its layout allows). */
int sp_hip_roundtrip_cells(sp_hip_cache_t *cc, int layer, const int *d_cells, int n_cells,
                           void *d_k, long long k_cell_stride, void *d_v, long long v_cell_stride,
                           long long v_elem_stride, int dtype, int max_bands, void *stream);

/* Calibration of the K coefficient order (the CUDA branch of KvCache::calibrate_feed,
 * kv_cache.cpp:553-585, and the order sync of calibrate_end, :626-652), for device
 * vectors: feed accumulates per-coefficient sums and sums of squares of the cache's
 * forward transform of n_vecs K vectors (row i at d_vecs + i*row_stride elements)
 * in fp64; end ranks the coefficients by descending variance (ties: lower index
 * first) into var_order_out [head_dim] (may be NULL) and, with apply != 0, makes that
 * ranking the K coefficient order of later writes, reads and attention. */
int sp_hip_calibrate_begin(sp_hip_cache_t *cc);
int sp_hip_calibrate_feed(sp_hip_cache_t *cc, const void *d_vecs, long long row_stride, int n_vecs, int dtype);
int sp_hip_calibrate_end(sp_hip_cache_t *cc, int *var_order_out, int apply);

/* Every slot at once: src/dst [n_layers*n_heads_kv][n_pos][head_dim] for positions
 * [start_pos, start_pos+n_pos) of each slot (bulk prefill / bulk reconstruct). */
int sp_hip_write_all(sp_hip_cache_t *cc, int start_pos, int n_pos,
                     const void *d_k, const void *d_v, int dtype);
int sp_hip_read_all(const sp_hip_cache_t *cc, int start_pos, int n_pos,
                    void *d_k, void *d_v, int dtype, int max_bands);

/* Host-buffer I/O on the device cache (stages through device memory and
 * returns after the copy back): used by the bridge's HIP backend for the
 * host-pointer sp_llama_write_* / sp_llama_read_* calls. */
int sp_hip_write_host(sp_hip_cache_t *cc, int is_v, int layer, int head, int start_pos, int n_pos,
                      const float *h_vecs);
int sp_hip_read_host(const sp_hip_cache_t *cc, int is_v, int layer, int head, int start_pos,
                     int n_pos, float *h_out, int max_bands);

/* ---- stage launchers exposed for testing (shannon_prime_cuda.h:116-134) ---- */
void sp_hip_vht2_forward(float *d_data, int n, int n_vecs, int vht2_norm, void *stream);
void sp_hip_mobius_reorder(float *d_data, const int *d_order, int n, int n_vecs, void *stream);
void sp_hip_mobius_unreorder(float *d_data, const int *d_order, int n, int n_vecs, void *stream);
void sp_hip_band_quantize(const float *d_input, void *d_output, const sp_band_config_t *bc,
                          int n_vecs, void *stream);
void sp_hip_band_dequantize(const void *d_input, float *d_output, const sp_band_config_t *bc,
                            int n_vecs, void *stream);

/* ---- generic strided codec (what every ship entry point above launches) ----
 * encode: vector (o, i) for o < n_outer, i < n_inner is read at element offset
 *   o*src_outer + i*src_inner of d_src (dtype) and written as a record at byte
 *   offset o*dst_outer + i*bc->total_bytes of d_dst.
 * decode: the reverse; max_bands < 0 reconstructs every band.
 * d_order: device [head_dim] Mobius order or NULL. */
int sp_hip_ship_encode(const sp_band_config_t *bc, const int *d_order, int vht2_norm,
                       const void *d_src, int src_dtype, long long src_outer, long long src_inner,
                       void *d_dst, long long dst_outer, int n_outer, int n_inner, void *stream);
int sp_hip_ship_decode(const sp_band_config_t *bc, const int *d_order, int vht2_norm,
                       int max_bands, const void *d_src, long long src_outer,
                       void *d_dst, int dst_dtype, long long dst_outer, long long dst_inner,
                       int n_outer, int n_inner, void *stream);

/* ======================================================================== */
/* Fused decompress-attention decode (replaces llama_sp_kq_compute,        */
/* src/engine/llama_sp_fused_kq.cpp:83-165, and the ggml softmax . V after  */
/* it). Scores are taken against the spectral-domain keys: the query is     */
/* transformed and Mobius-reordered once, packed K codes are dotted in      */
/* place, and sum_t p_t * dequant(V_t) is accumulated in the spectral       */
/* domain with one inverse transform per head, so no full-precision K or V  */
/* is materialized.                                                         */
/* ======================================================================== */

/* q: [n_q][head_dim] fp32 for one decode token. Query head h reads KV head
 * h / (n_q / n_heads_kv) (llama.cpp GQA grouping). Positions [0, n_kv) of
 * `layer` are attended. scores (optional): [n_q][n_kv] fp32 = kq_scale*q.K~.
 * out (optional): [n_q][head_dim] fp32 = softmax(scores) . V~.
 * Returns -1 for bad arguments or n_kv beyond the workspace sized at init. */
int sp_hip_attn_decode(const sp_hip_cache_t *cc, int layer, int n_kv,
                       const float *d_q, int n_q, float kq_scale,
                       float *d_scores, float *d_out, void *stream);

/* Band-limited attention, the phase-3 attention short-circuit
 * (llama-cpp-b8861-full-engine.patch:1442-1452 and :347-359, SHANNON_PRIME_DEFAULT_BANDS):
 * K and V bands >= max_bands read as 0, as in sp_llama_read_k/v_partial
 * (shannon_prime_llama.h:240-255), so the result equals attention over the
 * partial reconstructions; the skipped bands cost no matrix-core work.
 * max_bands < 0 (or >= n_bands) is sp_hip_attn_decode. */
int sp_hip_attn_decode_bands(const sp_hip_cache_t *cc, int layer, int n_kv,
                             const float *d_q, int n_q, float kq_scale,
                             float *d_scores, float *d_out, int max_bands, void *stream);

/* sp_hip_attn_decode_bands with no allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, allocation-free serving loops, harnesses that forbid hipMalloc).
 * Same arguments, checks and results as sp_hip_attn_decode_bands; the
 * attention workspace comes from a fixed per-GPU device array of
 * sp_hip_attn_noalloc_max_floats() floats (16 MiB, held until the process
 * ends) instead of the cache's workspace, and the call makes no hipMalloc /
 * hipFree. Returns -1 when the call needs more than that
 * (n_q*head_dim + n_q*ceil(n_kv/256)*(head_dim + 2) floats plus 16448 floats of
 * arrival counters: at head_dim 128 up to 256768 positions with 32 query heads and
 * 128256 with 64) or when `stream` is not on the current device. The counters
 * must start at zero: the array starts zeroed and every completed call leaves
 * them at zero. Calls that overlap on one GPU share the array and race. */
int sp_hip_attn_decode_bands_noalloc(const sp_hip_cache_t *cc, int layer, int n_kv,
                                     const float *d_q, int n_q, float kq_scale,
                                     float *d_scores, float *d_out, int max_bands, void *stream);
size_t sp_hip_attn_noalloc_max_floats(void);

/* Batched decode attention: n_seq sequences (1..64) of one layer in one launch sequence.
 * No counterpart in the reference, whose fused op (llama_sp_kq_compute,
 * llama_sp_fused_kq.cpp:83-165) runs one sequence per graph node; this is the same
 * contract for llama.cpp's unified cache holding several sequences, each a range of
 * cells. Sequence s attends positions [seq_start[s], seq_start[s] + seq_len[s]) of every
 * KV head (host arrays; ranges inside [0, max_seq_len), non-empty, may overlap) with its
 * own queries d_q[s] ([n_seq][n_q][head_dim] fp32): d_out [n_seq][n_q][head_dim] and
 * d_scores, sequence s's [n_q][seq_len[s]] block starting at element
 * n_q * (seq_len[0] + ... + seq_len[s-1]). Results equal n_seq separate calls over those
 * ranges. The hd 96 (K 5/4/4, V 5) and hd 64 (K 5/5/4/3, V 3) layouts run every sequence
 * in one launch each of the query preparation, the split kernel and the combine (workspace
 * grown on demand); other layouts run the single-sequence kernels once per sequence. */
int sp_hip_attn_decode_seqs(const sp_hip_cache_t *cc, int layer, int n_seq, const int *seq_start,
                            const int *seq_len, const float *d_q, int n_q, float kq_scale, float *d_scores,
                            float *d_out, void *stream);

/* Memory report to stderr (sp_cuda_print_memory, shannon_prime_cuda.h:140-141): the
 * records' MiB against an fp16 K+V cache of the same shape. */
void sp_hip_print_memory(const sp_hip_cache_t *cc);

/* Every layer of one decode step in one launch sequence: q [n_layers][n_q][hd],
 * out [n_layers][n_q][hd] (benchmark helper; per-layer semantics above). */
int sp_hip_attn_decode_all_layers(const sp_hip_cache_t *cc, int n_kv, const float *d_q,
                                  int n_q, float kq_scale, float *d_out, void *stream);

/* The scores-only form of the same loop, band-limited as sp_hip_attn_decode_bands
 * (max_bands -1: every band): q [n_layers][n_q][hd], scores [n_layers][n_q][n_kv]
 * (benchmark helper; per-layer semantics above). */
int sp_hip_attn_scores_all_layers(const sp_hip_cache_t *cc, int n_kv, const float *d_q,
                                  int n_q, float kq_scale, float *d_scores, int max_bands,
                                  void *stream);

/* fp16 reference attention over an uncompressed cache, same layout contract
 * as the compressed one ([slot][pos][head_dim] fp16): the baseline the fused
 * kernel is compared against. */
int sp_hip_attn_decode_f16(const void *d_k, const void *d_v, int n_heads_kv, int max_seq,
                           int head_dim, int layer, int n_kv, const float *d_q, int n_q,
                           float kq_scale, float *d_scores, float *d_out, void *stream);

/* ======================================================================== */
/* Sqfree + spinor cache (sp_cuda_sqfree_cache_t, shannon_prime_cuda.h:153-230) */
/* ======================================================================== */

typedef struct {
    sp_config_t      config;
    int              pad_dim;
    int              sk_k;
    int              n_res;
    int              n_terms;
    int              residual_bits;
    int              use_spinor;
    sp_band_config_t k_bands;   /* over the sk_k skeleton coefficients */
    sp_band_config_t v_bands;
    int             *d_skeleton_idx;
    int             *d_residual_idx;
    int             *d_csr_offsets;
    int             *d_csr_skel_slot;
    int             *d_csr_mu_sign;
    unsigned char   *d_k_cache;
    unsigned char   *d_v_cache;
    int              bytes_per_pos_k;
    int              bytes_per_pos_v;
    int              max_seq_len;
    int              n_slots;
    void            *stream;
    void            *priv;
} sp_hip_sqfree_cache_t;

/* shannon_prime_cuda.h:197-203. Skeleton = pad_dim/2 as the reference CUDA
 * path (shannon_prime_sqfree.cu:606). */
int  sp_hip_sqfree_cache_init(sp_hip_sqfree_cache_t *cc, const sp_config_t *cfg, int max_seq_len,
                              int residual_bits, int use_spinor, void *stream);
/* Extension: explicit skeleton size (SHANNON_PRIME_SK_FRAC * pad_dim, parsed by
 * shannon_prime_llama_sqfree.c:68-71); sk_k <= 0 selects pad_dim/2. */
int  sp_hip_sqfree_cache_init_ex(sp_hip_sqfree_cache_t *cc, const sp_config_t *cfg,
                                 int max_seq_len, int residual_bits, int use_spinor, int sk_k,
                                 void *stream);
void sp_hip_sqfree_cache_free(sp_hip_sqfree_cache_t *cc);

void sp_hip_sqfree_write_k(sp_hip_sqfree_cache_t *cc, int layer, int head, int pos, const float *d_k_vec);
void sp_hip_sqfree_write_v(sp_hip_sqfree_cache_t *cc, int layer, int head, int pos, const float *d_v_vec);
void sp_hip_sqfree_read_k(const sp_hip_sqfree_cache_t *cc, int layer, int head, int pos, float *d_k_out);
void sp_hip_sqfree_read_v(const sp_hip_sqfree_cache_t *cc, int layer, int head, int pos, float *d_v_out);
void sp_hip_sqfree_read_k_batch(const sp_hip_sqfree_cache_t *cc, int layer, int head,
                                int start_pos, int n_pos, float *d_k_out);
void sp_hip_sqfree_read_v_batch(const sp_hip_sqfree_cache_t *cc, int layer, int head,
                                int start_pos, int n_pos, float *d_v_out);
/* Extension: batched writes, fp32 or fp16 source [n_pos][head_dim]. */
int  sp_hip_sqfree_write_batch(sp_hip_sqfree_cache_t *cc, int is_v, int layer, int head,
                               int start_pos, int n_pos, const void *d_src, int dtype);
int  sp_hip_sqfree_read_batch(const sp_hip_sqfree_cache_t *cc, int is_v, int layer, int head,
                              int start_pos, int n_pos, void *d_dst, int dtype);
/* Extension: every head of one layer in one launch per K/V (the sqfree branch of
 * KvCache::write_gpu/read_gpu, kv_cache.cpp:1069-1080 and :1139-1197), rows in
 * llama.cpp's cache layout as for sp_hip_write_layer: element (t, h, d) at
 * t*row_stride + h*head_dim + d. NULL d_k or d_v skips that side. */
int  sp_hip_sqfree_write_layer(sp_hip_sqfree_cache_t *cc, int layer, int start_pos, int n_tok,
                               const void *d_k, const void *d_v, long long row_stride, int dtype);
int  sp_hip_sqfree_read_layer(const sp_hip_sqfree_cache_t *cc, int layer, int start_pos, int n_tok,
                              void *d_k, void *d_v, long long row_stride, int dtype);
/* Knight-mask recalibration (sp_sqfree_calibrate_begin/feed/end, kv_cache.cpp:523,
 * 546-548, 608, and the mask sync of :654-722): feed accumulates per-coefficient fp64
 * sums and sums of squares of the padded transforms of n_vecs device vectors; end
 * ranks the pad_dim coefficients by descending variance (ties: lower index first)
 * into ranking_out [pad_dim] (may be NULL) and, with apply != 0, rebuilds the Knight
 * tables with that ranking in place of the squarefree-first order (skeleton = its
 * first sk_k entries; the CSR rule is unchanged) for later writes and reads. */
int sp_hip_sqfree_calibrate_begin(sp_hip_sqfree_cache_t *cc);
int sp_hip_sqfree_calibrate_feed(sp_hip_sqfree_cache_t *cc, const void *d_vecs, long long row_stride, int n_vecs,
                                 int dtype);
int sp_hip_sqfree_calibrate_end(sp_hip_sqfree_cache_t *cc, int *ranking_out, int apply);
/* Extension: fused decode attention over the sqfree cache's records of one layer
 * (positions [0, n_kv) of every KV head), the contract of sp_hip_attn_decode:
 * d_q [n_q][head_dim] fp32 (GQA: query head h reads KV head h / (n_q / n_heads_kv),
 * at most 8 per KV head), d_scores [n_q][n_kv] = kq_scale * q . K~ and d_out
 * [n_q][head_dim] = softmax(scores) . V~, with K~ and V~ what sp_hip_sqfree_read_*
 * returns (the read path of sp_cuda_sqfree_read_one, shannon_prime_sqfree.cu:857-950,
 * which the reference's hook runs per vector before its attention,
 * llama-cpp-b8861-full-engine.patch:1205-1207); either output may be NULL (not both).
 * Nothing is reconstructed: the query moves into the records' coefficient domain
 * (q~ = V(q zero-padded to pad_dim)) once per query head and each record's skeleton
 * and residual coefficients (+-prediction + deviation, the spinor sheet's sign) are
 * dotted in place; sum p V~ is finished by one transform per query head. The
 * reference's fused op is ship-only (llama_sp_fused_kq.cpp:14-34). Geometry: head_dim
 * 128 (pad 154), skeleton 77 or 115 with K bands 5/4/4/4/5, V bands 5/4/4/4/5 (the
 * hook's mirror of K) or, at 115, one 3-bit band; 3-bit residuals; spinor; default
 * Knight tables. Other geometries return -1. The workspace is allocated on the first
 * call and grown when a call needs more. 0 or -1. */
int  sp_hip_sqfree_attn_decode(const sp_hip_sqfree_cache_t *cc, int layer, int n_kv, const float *d_q, int n_q,
                               float kq_scale, float *d_scores, float *d_out, void *stream);
/* Batched form (the sequence, query, score and output layout of sp_hip_attn_decode_seqs):
 * every sequence in one launch each of the query preparation, the split kernel and the
 * merge. No counterpart in the reference. */
int  sp_hip_sqfree_attn_decode_seqs(const sp_hip_sqfree_cache_t *cc, int layer, int n_seq, const int *seq_start,
                                    const int *seq_len, const float *d_q, int n_q, float kq_scale,
                                    float *d_scores, float *d_out, void *stream);
/* Host copies of the Knight tables (for tests and calibration tools). */
int  sp_hip_sqfree_get_tables(const sp_hip_sqfree_cache_t *cc, int *skeleton_idx,
                              int *residual_idx, int *csr_offsets, int *csr_skel_slot,
                              int *csr_mu_sign);

/* ======================================================================== */
/* Hierarchical cache (sp_cuda_hier_cache_t, shannon_prime_cuda.h:300-377)   */
/* ======================================================================== */

typedef struct {
    sp_config_t      config;
    int              pad_dim;
    int              n_skeleton;
    int              n_target;
    int              target_res_bits;
    int              n_slots;
    int              max_seq_len;
    uint16_t        *d_W;             /* [n_slots][n_target][n_skeleton] fp16 */
    int             *d_skeleton_idx;
    int             *d_target_idx;
    sp_band_config_t skel_bands;
    unsigned char   *d_k_cache;
    unsigned char   *d_v_cache;
    int              bytes_per_pos_k;
    int              bytes_per_pos_v;
    void            *stream;
    void            *priv;
} sp_hip_hier_cache_t;

int  sp_hip_hier_cache_init(sp_hip_hier_cache_t *hc, const sp_config_t *cfg,
                            int pad_dim, int n_skeleton, int n_target, int target_res_bits,
                            const int *skeleton_idx, const int *target_idx,
                            const sp_band_config_t *skel_bands, int max_seq_len, int n_slots,
                            void *stream);
void sp_hip_hier_cache_free(sp_hip_hier_cache_t *hc);
int  sp_hip_hier_cache_upload_W(sp_hip_hier_cache_t *hc, const uint16_t *W_all);
/* Predictor fit (sp_hier_cache_calibrate_begin/feed/end, kv_cache.cpp:519-521,
 * 590-597, 606-607, with the W upload of :724-751): feed accumulates, on the device
 * in fp64, the Gram matrices G_ss = sum s s^T and G_ts = sum t s^T of the slot's
 * padded, transformed vectors (s = skeleton, t = target coefficients, unquantized);
 * end solves W = G_ts (G_ss + lambda I)^-1 per fed slot (Cholesky in double,
 * lambda = ridge * trace(G_ss) / n_skeleton), rounds it to fp16 (via fp32) and
 * uploads it; slots without data keep their W. */
int  sp_hip_hier_calibrate_begin(sp_hip_hier_cache_t *hc);
int  sp_hip_hier_calibrate_feed(sp_hip_hier_cache_t *hc, int slot, const void *d_vecs, long long row_stride,
                                int n_vecs, int dtype);
int  sp_hip_hier_calibrate_end(sp_hip_hier_cache_t *hc, double ridge);
/* Sticky-EMA end (KvCache::calibrate_end_ema, kv_cache.h:103-107, kv_cache.cpp:758-797):
 * each fed slot gets W = keep_frac * W_old + (1 - keep_frac) * W_fit (in double, then
 * fp16 via fp32); keep_frac in [0, 1], 0 is calibrate_end. */
int  sp_hip_hier_calibrate_end_ema(sp_hip_hier_cache_t *hc, double ridge, float keep_frac);

void sp_hip_hier_write_k(sp_hip_hier_cache_t *hc, int layer, int head, int pos, const float *d_k_vec);
void sp_hip_hier_write_v(sp_hip_hier_cache_t *hc, int layer, int head, int pos, const float *d_v_vec);
void sp_hip_hier_read_k(const sp_hip_hier_cache_t *hc, int layer, int head, int pos, float *d_k_out);
void sp_hip_hier_read_v(const sp_hip_hier_cache_t *hc, int layer, int head, int pos, float *d_v_out);
/* Extension: batched writes/reads of one slot, fp32 or fp16 [n_pos][head_dim]. */
int  sp_hip_hier_write_batch(sp_hip_hier_cache_t *hc, int is_v, int layer, int head,
                             int start_pos, int n_pos, const void *d_src, int dtype);
int  sp_hip_hier_read_batch(const sp_hip_hier_cache_t *hc, int is_v, int layer, int head,
                            int start_pos, int n_pos, void *d_dst, int dtype);
/* Extension: every head of one layer in one launch per K/V (the hier branch of
 * KvCache::write_gpu/read_gpu, kv_cache.cpp:1056-1068 and :1114-1128), rows as for
 * sp_hip_write_layer. NULL d_k or d_v skips that side. */
int  sp_hip_hier_write_layer(sp_hip_hier_cache_t *hc, int layer, int start_pos, int n_tok,
                             const void *d_k, const void *d_v, long long row_stride, int dtype);
int  sp_hip_hier_read_layer(const sp_hip_hier_cache_t *hc, int layer, int start_pos, int n_tok,
                            void *d_k, void *d_v, long long row_stride, int dtype);
/* Extension: fused decode attention over the hier cache's records of one layer
 * (positions [0, n_kv) of every KV head), the contract of sp_hip_attn_decode:
 * d_q [n_q][head_dim] fp32 (GQA: query head h reads KV head h / (n_q / n_heads_kv),
 * at most 8 per KV head), d_scores [n_q][n_kv] = kq_scale * q . K~ and d_out
 * [n_q][head_dim] = softmax(scores) . V~, with K~ and V~ what sp_hip_hier_read_*
 * returns; either output may be NULL (not both). Neither is reconstructed: the
 * query is moved into the records' coefficient domain (q~ = V(q zero-padded),
 * u = q~_skel + W^T q~_tgt) once per query head, so a score costs one pass over
 * the record. The reference's fused op is ship-only (llama_sp_fused_kq.cpp:14-34);
 * this serves the hier cache the same way. The workspace is allocated on the
 * first call and grown when a call needs more. 0 or -1. */
int  sp_hip_hier_attn_decode(const sp_hip_hier_cache_t *hc, int layer, int n_kv, const float *d_q, int n_q,
                             float kq_scale, float *d_scores, float *d_out, void *stream);
/* Batched form (the sequence, query, score and output layout of sp_hip_attn_decode_seqs):
 * the batch of a decode step in one launch each of the query preparation (n_seq * n_q
 * blocks), the split kernel (grid: KV head x run x sequence) and the merge. No counterpart
 * in the reference. */
int  sp_hip_hier_attn_decode_seqs(const sp_hip_hier_cache_t *hc, int layer, int n_seq, const int *seq_start,
                                  const int *seq_len, const float *d_q, int n_q, float kq_scale, float *d_scores,
                                  float *d_out, void *stream);

/* ======================================================================== */
/* System 1/2 dual cache (DualKvCache, kv_cache.h:238-310,                  */
/* kv_cache.cpp:1641-1877)                                                  */
/* ======================================================================== */
/* System 1 is a ship cache; System 2 a sqfree or hier cache of the same
 * n_layers, n_heads_kv, head_dim and max_seq_len on the same stream. Both are
 * initialised and freed by the caller; the dual cache holds the per-position
 * route table (all positions start in System 1). */
#define SP_DUAL_SQFREE 1
#define SP_DUAL_HIER   2
typedef struct {
    sp_hip_cache_t  *sys1;
    void            *sys2;            /* sp_hip_sqfree_cache_t* or sp_hip_hier_cache_t* */
    int              sys2_kind;       /* SP_DUAL_SQFREE or SP_DUAL_HIER */
    float            entropy_threshold;
    int              max_seq_len;
    void            *priv;            /* route table, device list of System 2 positions */
} sp_hip_dual_cache_t;

/* DualKvCache::create_gpu (:1641-1690) over caches the caller built; -1 when the
 * shapes or streams differ. */
int  sp_hip_dual_init(sp_hip_dual_cache_t *dc, sp_hip_cache_t *sys1, int sys2_kind, void *sys2,
                      float entropy_threshold);
void sp_hip_dual_free(sp_hip_dual_cache_t *dc);
/* DualKvCache::route_position (:1692-1697): System 2 when entropy >= the threshold;
 * returns 1 for System 2, 0 for System 1 (and for pos outside [0, max_seq)). */
int  sp_hip_dual_route_position(sp_hip_dual_cache_t *dc, int pos, float entropy);
/* DualKvCache::owner_of (:1699-1702): 1 or 2; 1 outside [0, max_seq). */
int  sp_hip_dual_owner_of(const sp_hip_dual_cache_t *dc, int pos);
/* DualKvCache::sys1_count / sys2_count (:1862-1876): over all max_seq positions. */
int  sp_hip_dual_sys1_count(const sp_hip_dual_cache_t *dc);
int  sp_hip_dual_sys2_count(const sp_hip_dual_cache_t *dc);
/* DualKvCache::write_gpu (:1733-1751): each of positions [start_pos, start_pos +
 * n_tok) goes to its owner only, one layer-wide write per run of positions with
 * the same owner; rows as for sp_hip_write_layer. */
int  sp_hip_dual_write_layer(sp_hip_dual_cache_t *dc, int layer, int start_pos, int n_tok,
                             const void *d_k, const void *d_v, long long row_stride, int dtype);
/* DualKvCache::read_merged_gpu (:1832-1860), with the per-position merge its
 * comment leaves for later: positions [0, kv_len) of `layer`, each from its owner,
 * into rows (t, h, d) at t*row_stride + h*head_dim + d. System 1 is decoded over
 * the whole range, then System 2 over its own positions only, overwriting those
 * rows on the shared stream. NULL d_k or d_v skips that side. */
int  sp_hip_dual_read_merged(sp_hip_dual_cache_t *dc, int layer, int kv_len, void *d_k, void *d_v,
                             long long row_stride, int dtype);

/* ======================================================================== */
/* Disk serialisation, format v3 (KvCache::save_to_disk / load_from_disk,   */
/* kv_cache.h:132-146, kv_cache.cpp:1533-1585; band-major partial load of   */
/* the disk-tier notes, CHANGELOG.md)                                       */
/* ======================================================================== */
/* One file per layer, {prefix}.L{layer}.bin: a 64-byte header ("VHT2", version 3,
 * model hash, n_pos, layer, n_heads, head_dim, cache kind, record bytes and
 * segment counts of K and V, a check of the K coefficient order, FNV-1a of the
 * first 56 bytes), then K and V band-major: for each band (sqfree/hier: each
 * skeleton band, then the residual tail) the bytes of every head's positions
 * [0, n_pos). Saves return 0, loads the n_pos stored (-1 on any error). A model
 * hash mismatch fails the load unless SP_DISK_HASH_STRICT=0, which only warns
 * (the reference's strict hash guard and its opt-out). */
uint64_t sp_fnv1a64(const void *data, size_t n);   /* the model_hash of a path string */
int sp_hip_cache_save(const sp_hip_cache_t *cc, const char *prefix, int n_pos, uint64_t model_hash);
int sp_hip_cache_load(sp_hip_cache_t *cc, const char *prefix, uint64_t expected_hash);
/* sp_shadow_cache_load_partial / KvCache::load_from_disk_partial: reads only the
 * first max_bands bands of K and of V from each file and clears the others'
 * bytes, so they decode as 0 (max_bands >= 0). */
int sp_hip_cache_load_partial(sp_hip_cache_t *cc, const char *prefix, uint64_t expected_hash, int max_bands);
int sp_hip_sqfree_cache_save(const sp_hip_sqfree_cache_t *cc, const char *prefix, int n_pos, uint64_t model_hash);
int sp_hip_sqfree_cache_load(sp_hip_sqfree_cache_t *cc, const char *prefix, uint64_t expected_hash);
/* The hier cache also writes and reads {prefix}.hier_w.bin (every slot's fp16 W). */
int sp_hip_hier_cache_save(const sp_hip_hier_cache_t *hc, const char *prefix, int n_pos, uint64_t model_hash);
int sp_hip_hier_cache_load(sp_hip_hier_cache_t *hc, const char *prefix, uint64_t expected_hash);

/* ======================================================================== */
/* Runtime                                                                  */
/* ======================================================================== */

/* 1 when a gfx950 device is visible and usable, else 0. */
int         sp_hip_available(void);
/* Last error text of the calling thread ("" when none). */
const char *sp_hip_last_error(void);
/* Stream-ordered event timing helpers (milliseconds between two records). */
void       *sp_hip_event_create(void);
void        sp_hip_event_destroy(void *ev);
int         sp_hip_event_record(void *ev, void *stream);
float       sp_hip_event_elapsed_ms(void *ev_start, void *ev_end);
int         sp_hip_stream_sync(void *stream);
/* Stream-ordered byte fill of device memory (used by sp_llama_clear_range). */
int         sp_hip_memset(void *d_ptr, int value, size_t bytes, void *stream);
/* Test hooks: the same codec through the generic (one vector per wave)
 * kernels only, to cross-check the two kernel families. */
int sp_hip_ship_encode_generic(const sp_band_config_t *bc, const int *d_order, int vht2_norm,
                               const void *d_src, int src_dtype, long long src_outer,
                               long long src_inner, void *d_dst, long long dst_outer, int n_outer,
                               int n_inner, void *stream);
int sp_hip_ship_decode_generic(const sp_band_config_t *bc, const int *d_order, int vht2_norm,
                               int max_bands, const void *d_src, long long src_outer, void *d_dst,
                               int dst_dtype, long long dst_outer, long long dst_inner, int n_outer,
                               int n_inner, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* SP_HIP_H */
