/*
 * shannon_prime_llama.h -- llama.cpp bridge of the Shannon-Prime KV codec,
 * backed by libshannon_prime_hip.so on MI355X.
 *
 * Same C ABI as the reference bridge (src/tools/shannon_prime_llama.h:97-341):
 * the params struct, opaque context, role-aware init, void writers/readers,
 * partial and batch reads, memory stats, diagnostics and the archive getters.
 * Differences:
 *   - SP_BACKEND_HIP (= 5) selects the device-resident cache (compressed K/V
 *     live in HBM). The reference's commented-out CUDA slot
 *     (shannon_prime_llama.c:58, 502) maps to it as well.
 *   - SP_BACKEND_CPU keeps the reference's host-resident storage layout
 *     (caller-visible k_cache/v_cache slots) but its codec runs on the GPU.
 *   - ADRENO / HEXAGON / VULKAN are not built; selecting them falls back to
 *     SP_BACKEND_CPU with a one-line warning, as the reference does when its
 *     DSP is unreachable (shannon_prime_llama.c:449-468).
 *   - PrimePE (SHANNON_PRIME_PE) changes the model's RoPE, not the codec, and
 *     is not implemented: the freq-factor getters return NULL / 0, which the
 *     reference documents as "PrimePE disabled".
 *
 * Environment variables read by sp_llama_init_with_role (same names and
 * precedence as the reference, shannon_prime_llama.c:209-397):
 *   SHANNON_PRIME_ENABLED, _K_BITS, _V_BITS, _MOBIUS, _K_TERNARY_BANDS,
 *   _V_TERNARY_BANDS, _FP8 (advisory), _BACKEND (cpu|hip|gpu|cuda|rocm),
 *   _VERBOSE, and the role-aware SHANNON_PRIME_DRAFT_* variants plus
 *   SHANNON_PRIME_DRAFT_PRESET (aggressive|ternary|ship).
 *   SHANNON_PRIME_VHT2_NORM=stage selects the per-stage 1/sqrt(2) convention.
 */
#ifndef SHANNON_PRIME_LLAMA_H
#define SHANNON_PRIME_LLAMA_H

#include "shannon_prime.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int head_dim;
    int n_layers;
    int n_heads_kv;
    int max_seq_len;
    enum {
        SP_BACKEND_CPU     = 0,
        SP_BACKEND_CUDA    = 1,
        SP_BACKEND_VULKAN  = 2,
        SP_BACKEND_ADRENO  = 3,
        SP_BACKEND_HEXAGON = 4,
        SP_BACKEND_HIP     = 5
    } backend;
    void       *gpu_context;   /* hipStream_t for SP_BACKEND_HIP (NULL: default stream) */
    const char *arch_name;
} sp_llama_params_t;

typedef struct sp_llama_ctx_s sp_llama_ctx_t;

typedef enum {
    SP_LLAMA_ROLE_DEFAULT = 0,
    SP_LLAMA_ROLE_TARGET  = 1,
    SP_LLAMA_ROLE_DRAFT   = 2
} sp_llama_role_t;

/* The configuration and backend sp_llama_init_with_role would use, from the
 * environment alone (no caches are created): 1 with *cfg and *backend filled,
 * 0 when SHANNON_PRIME_ENABLED (or the draft's) is off, -1 for NULL arguments.
 * Extension: the reference resolves these inline in sp_llama_init_with_role
 * (shannon_prime_llama.c:209-307); exported so hosts and tests can see the
 * configuration without a GPU. */
int sp_llama_resolve_env(const sp_llama_params_t *params, sp_llama_role_t role, sp_config_t *cfg,
                         int *backend);

/* ---- lifecycle (shannon_prime_llama.h:163-185) ---- */
sp_llama_ctx_t *sp_llama_init(const sp_llama_params_t *params);
sp_llama_ctx_t *sp_llama_init_with_role(const sp_llama_params_t *params, sp_llama_role_t role);
sp_llama_ctx_t *sp_llama_init_config(const sp_llama_params_t *params, const sp_config_t *cfg);
void            sp_llama_free(sp_llama_ctx_t *ctx);

/* ---- write path (shannon_prime_llama.h:199-221) ---- */
void sp_llama_write_kv(sp_llama_ctx_t *ctx, int layer, int head, int pos,
                       const float *k_vec, const float *v_vec);
void sp_llama_write_k(sp_llama_ctx_t *ctx, int layer, int head, int pos, const float *k_vec);
void sp_llama_write_v(sp_llama_ctx_t *ctx, int layer, int head, int pos, const float *v_vec);
void sp_llama_write_k_batch(sp_llama_ctx_t *ctx, int layer, int head, int start_pos, int n_pos,
                            const float *k_vecs);
void sp_llama_write_v_batch(sp_llama_ctx_t *ctx, int layer, int head, int start_pos, int n_pos,
                            const float *v_vecs);

/* ---- read path (shannon_prime_llama.h:232-266) ---- */
void sp_llama_read_k(const sp_llama_ctx_t *ctx, int layer, int head, int pos, float *k_out);
void sp_llama_read_v(const sp_llama_ctx_t *ctx, int layer, int head, int pos, float *v_out);
void sp_llama_read_k_partial(const sp_llama_ctx_t *ctx, int layer, int head, int pos,
                             float *k_out, int max_bands);
void sp_llama_read_v_partial(const sp_llama_ctx_t *ctx, int layer, int head, int pos,
                             float *v_out, int max_bands);
void sp_llama_read_k_batch(const sp_llama_ctx_t *ctx, int layer, int head, int start_pos,
                           int n_pos, float *k_out);
void sp_llama_read_v_batch(const sp_llama_ctx_t *ctx, int layer, int head, int start_pos,
                           int n_pos, float *v_out);

/* ---- cache management (shannon_prime_llama.h:273-284) ---- */
void sp_llama_clear_range(sp_llama_ctx_t *ctx, int start_pos, int end_pos);

typedef struct {
    size_t compressed_bytes;
    size_t baseline_bytes;
    float  compression_ratio;
    int    n_positions;
} sp_llama_memory_t;

sp_llama_memory_t sp_llama_memory(const sp_llama_ctx_t *ctx);

/* ---- diagnostics (shannon_prime_llama.h:291-295) ---- */
float sp_llama_validate_k(sp_llama_ctx_t *ctx, const float *k_vec, int head_dim);
void  sp_llama_print_config(const sp_llama_ctx_t *ctx);

/* ---- PrimePE getters (shannon_prime_llama.h:317-320): NULL / 0 here ---- */
const float *sp_llama_get_freq_factors(const sp_llama_ctx_t *ctx);
int          sp_llama_get_n_freqs(const sp_llama_ctx_t *ctx);

/* ---- packed-K archive getters (shannon_prime_llama.h:339-341) ----
 * The Hexagon-specific getters are kept for ABI compatibility and return
 * NULL / 0. The generalised getters return the packed archive of the active
 * backend, layout [position][total_bytes] per (layer, head): a host pointer for
 * SP_BACKEND_CPU, a device pointer for SP_BACKEND_HIP. Owned by the context. */
const void *sp_llama_get_hexagon_k_buf(const sp_llama_ctx_t *ctx, int layer, int head);
int         sp_llama_get_hexagon_k_total_bytes(const sp_llama_ctx_t *ctx);
const void *sp_llama_get_k_buf(const sp_llama_ctx_t *ctx, int layer, int head);
const void *sp_llama_get_v_buf(const sp_llama_ctx_t *ctx, int layer, int head);
int         sp_llama_get_k_total_bytes(const sp_llama_ctx_t *ctx);
int         sp_llama_get_v_total_bytes(const sp_llama_ctx_t *ctx);
/* Active backend after fallbacks (an SP_BACKEND_* value); -1 for NULL. */
int         sp_llama_get_backend(const sp_llama_ctx_t *ctx);
/* Device cache of SP_BACKEND_HIP (for device-resident callers and the fused
 * attention launcher in sp_hip.h), else NULL. Returned as void* to keep this
 * header free of the device API. */
void       *sp_llama_get_hip_cache(const sp_llama_ctx_t *ctx);

/* ======================================================================== */
/* Sqfree + spinor bridge (src/tools/shannon_prime_llama_sqfree.c:48-240)   */
/* ======================================================================== */
/* Environment (shannon_prime_llama_sqfree.c:48-101): SHANNON_PRIME_SQFREE=1
 * enables the path; SHANNON_PRIME_SPINOR=1 adds the sheet bit and turns SQFREE
 * on with a message; _RESIDUAL_BITS (1..4, default 3); _SK_FRAC (0.1..1.0,
 * default 0.75; parsed and kept but, as in the reference, not passed to the
 * cache: the skeleton is pad_dim / 2); _K_BITS (default 5,4,4,4,5; V mirrors
 * K); _DUMP_K=<path> with _DUMP_K_LIMIT (default 8192, 0 = no limit) appends
 * each written K vector as raw fp32. The variables are exactly "1" to enable. */
typedef struct {
    int   sqfree_enabled;
    int   spinor_enabled;
    int   residual_bits;
    float sk_frac;
    int   k_band_bits[SP_MAX_BANDS];
    int   n_k_bands;
} sp_llama_sqfree_config_t;

/* Extension: the environment as sp_llama_sqfree_init reads it. */
void sp_llama_sqfree_config_from_env(sp_llama_sqfree_config_t *out);

typedef struct sp_llama_sqfree_ctx_s sp_llama_sqfree_ctx_t;

/* NULL when SHANNON_PRIME_SQFREE is off or the cache cannot be created
 * (shannon_prime_llama_sqfree.c:123-190). */
sp_llama_sqfree_ctx_t *sp_llama_sqfree_init(int head_dim, int n_layers, int n_heads_kv, int max_seq_len);
void  sp_llama_sqfree_free(sp_llama_sqfree_ctx_t *ctx);
void  sp_llama_sqfree_write_kv(sp_llama_sqfree_ctx_t *ctx, int layer, int head, int pos,
                               const float *k_vec, const float *v_vec);
void  sp_llama_sqfree_read_k(const sp_llama_sqfree_ctx_t *ctx, int layer, int head, int pos, float *k_out);
void  sp_llama_sqfree_read_v(const sp_llama_sqfree_ctx_t *ctx, int layer, int head, int pos, float *v_out);
/* Round trip through slot (0, 0, 0) and the correlation with the input (:229-239). */
float sp_llama_sqfree_validate_k(sp_llama_sqfree_ctx_t *ctx, const float *k_vec, int head_dim);
/* The context's core cache (for its pad_dim and Knight tables). */
const sp_sqfree_cache_t *sp_llama_sqfree_get_cache(const sp_llama_sqfree_ctx_t *ctx);

#ifdef __cplusplus
}
#endif
#endif /* SHANNON_PRIME_LLAMA_H */
