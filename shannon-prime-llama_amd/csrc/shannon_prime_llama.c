/*
 * shannon_prime_llama.c -- llama.cpp bridge over the MI355X codec library.
 *
 * Env-driven configuration with the reference's names, defaults and role
 * precedence (src/tools/shannon_prime_llama.c:73-397); backend dispatch to
 * the GPU-backed shadow cache (host storage, SP_BACKEND_CPU) or the
 * device-resident cache (SP_BACKEND_HIP).
 */
#include "../../include/shannon_prime_llama.h"
#include "../../include/sp_hip.h"
#include "sp_env.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct sp_llama_ctx_s {
    sp_llama_params_t params;
    sp_config_t       config;
    int               active_backend;
    int               n_positions;
    sp_shadow_cache_t cpu_cache;   /* SP_BACKEND_CPU: host storage, GPU codec */
    sp_hip_cache_t    hip_cache;   /* SP_BACKEND_HIP: device storage */
};

/* ---- configuration from the environment ----
 * Names, defaults and precedence are the reference bridge's
 * (shannon_prime_llama.c:73-307); the decoders live in sp_env.c. */

/* Draft presets: band tables a draft context starts from before its explicit
 * K_BITS / V_BITS (shannon_prime_llama.c:177-199). k_n == 0 keeps the
 * head-dim defaults. */
static const struct draft_preset {
    const char *name;
    int k_n, k_bits[2];
    int v_n, v_bits[1];
} k_presets[] = {
    {"aggressive", 2, {2, 1}, 1, {1}},
    {"ternary", 2, {2, 2}, 1, {2}},
    {"ship", 0, {0, 0}, 0, {0}},
};

static void apply_preset(const char *name, sp_config_t *cfg) {
    if (!name || !name[0]) return;
    for (size_t i = 0; i < sizeof(k_presets) / sizeof(k_presets[0]); i++) {
        const struct draft_preset *pr = &k_presets[i];
        if (strcmp(name, pr->name) != 0) continue;
        if (pr->k_n) {
            cfg->k_n_bands = pr->k_n;
            memcpy(cfg->k_band_bits, pr->k_bits, sizeof(pr->k_bits));
            cfg->v_n_bands = pr->v_n;
            memcpy(cfg->v_band_bits, pr->v_bits, sizeof(pr->v_bits));
        }
        return;
    }
    fprintf(stderr, "[Shannon-Prime] unknown SHANNON_PRIME_DRAFT_PRESET '%s' "
                    "(known: aggressive, ternary, ship); ignoring\n", name);
}

/* Backend names: the reference's (cpu, hexagon, adreno) plus this build's. */
static const struct backend_name {
    const char *name;
    int backend;
} k_backends[] = {
    {"cpu", SP_BACKEND_CPU},   {"hip", SP_BACKEND_HIP},       {"gpu", SP_BACKEND_HIP},
    {"rocm", SP_BACKEND_HIP},  {"cuda", SP_BACKEND_HIP},      {"hexagon", SP_BACKEND_HEXAGON},
    {"adreno", SP_BACKEND_ADRENO}, {"vulkan", SP_BACKEND_VULKAN},
};

int sp_llama_resolve_env(const sp_llama_params_t *params, sp_llama_role_t role, sp_config_t *cfg,
                         int *backend) {
    if (!params || !cfg) return -1;
    const int draft = role == SP_LLAMA_ROLE_DRAFT;
    if (!sp_env_flag(sp_env_text("ENABLED", draft), 0)) return 0;

    sp_config_init(cfg, params->head_dim, params->n_layers, params->n_heads_kv);
    /* head-dim adaptive defaults (shannon_prime_llama.c:235-252): K 5/5/4/3 and
     * V 3 from head_dim 128 on, K 5/4/4 and V 5 below */
    const int wide = params->head_dim >= 128;
    const int kdef[4] = {5, wide ? 5 : 4, 4, wide ? 3 : 4};
    cfg->k_n_bands = wide ? 4 : 3;
    memcpy(cfg->k_band_bits, kdef, sizeof(int) * (size_t)cfg->k_n_bands);
    cfg->v_n_bands = 1;
    cfg->v_band_bits[0] = wide ? 3 : 5;
    if (draft) apply_preset(getenv("SHANNON_PRIME_DRAFT_PRESET"), cfg);

    int n = sp_env_int_list(sp_env_text("K_BITS", draft), cfg->k_band_bits, SP_MAX_BANDS);
    if (n > 0) cfg->k_n_bands = n;
    n = sp_env_int_list(sp_env_text("V_BITS", draft), cfg->v_band_bits, SP_MAX_BANDS);
    if (n > 0) cfg->v_n_bands = n;
    cfg->use_mobius_mask = sp_env_flag(sp_env_text("MOBIUS", draft), 1);
    cfg->k_ternary_mask = sp_env_index_mask(sp_env_text("K_TERNARY_BANDS", draft));
    cfg->v_ternary_mask = sp_env_index_mask(sp_env_text("V_TERNARY_BANDS", draft));
    cfg->use_fp8 = sp_env_flag(sp_env_text("FP8", draft), 0);
    const char *norm = sp_env_text("VHT2_NORM", draft);
    if (norm && strcmp(norm, "stage") == 0) cfg->vht2_norm = SP_VHT2_NORM_STAGE;

    int be = params->backend;
    const char *bname = sp_env_text("BACKEND", draft);
    if (bname)
        for (size_t i = 0; i < sizeof(k_backends) / sizeof(k_backends[0]); i++)
            if (strcmp(bname, k_backends[i].name) == 0) be = k_backends[i].backend;
    if (backend) *backend = be;
    return 1;
}

/* ---- lifecycle ---- */

sp_llama_ctx_t *sp_llama_init(const sp_llama_params_t *params) {
    return sp_llama_init_with_role(params, SP_LLAMA_ROLE_DEFAULT);
}

sp_llama_ctx_t *sp_llama_init_with_role(const sp_llama_params_t *params, sp_llama_role_t role) {
    sp_config_t cfg;
    int backend = 0;
    if (sp_llama_resolve_env(params, role, &cfg, &backend) != 1) return NULL;
    sp_llama_params_t p = *params;
    p.backend = backend;
    if (cfg.use_fp8)
        fprintf(stderr, "[Shannon-Prime]%s SHANNON_PRIME_FP8=1 requested but this library has "
                        "no fp8 path; using integer band codes.\n",
                role == SP_LLAMA_ROLE_DRAFT ? " [draft]" : role == SP_LLAMA_ROLE_TARGET ? " [target]" : "");
    return sp_llama_init_config(&p, &cfg);
}

static int alloc_host_slots(sp_llama_ctx_t *ctx) {
    const int n_slots = ctx->config.n_layers * ctx->config.n_heads_kv;
    if (sp_shadow_cache_set_slot_capacity(&ctx->cpu_cache, ctx->params.max_seq_len) != 0) return -1;
    ctx->cpu_cache.k_cache = (uint8_t **)calloc((size_t)n_slots, sizeof(uint8_t *));
    ctx->cpu_cache.v_cache = (uint8_t **)calloc((size_t)n_slots, sizeof(uint8_t *));
    if (!ctx->cpu_cache.k_cache || !ctx->cpu_cache.v_cache) return -1;
    for (int i = 0; i < n_slots; i++) {
        ctx->cpu_cache.k_cache[i] = (uint8_t *)calloc((size_t)ctx->params.max_seq_len,
                                                      (size_t)ctx->cpu_cache.k_bands.total_bytes);
        ctx->cpu_cache.v_cache[i] = (uint8_t *)calloc((size_t)ctx->params.max_seq_len,
                                                      (size_t)ctx->cpu_cache.v_bands.total_bytes);
        if (!ctx->cpu_cache.k_cache[i] || !ctx->cpu_cache.v_cache[i]) return -1;
    }
    return 0;
}

static void free_host_slots(sp_llama_ctx_t *ctx) {
    const int n_slots = ctx->config.n_layers * ctx->config.n_heads_kv;
    if (ctx->cpu_cache.k_cache)
        for (int i = 0; i < n_slots; i++) free(ctx->cpu_cache.k_cache[i]);
    if (ctx->cpu_cache.v_cache)
        for (int i = 0; i < n_slots; i++) free(ctx->cpu_cache.v_cache[i]);
    free(ctx->cpu_cache.k_cache);
    free(ctx->cpu_cache.v_cache);
    ctx->cpu_cache.k_cache = ctx->cpu_cache.v_cache = NULL;
}

sp_llama_ctx_t *sp_llama_init_config(const sp_llama_params_t *params, const sp_config_t *cfg) {
    if (!params || !cfg || params->max_seq_len <= 0) return NULL;
    sp_llama_ctx_t *ctx = (sp_llama_ctx_t *)calloc(1, sizeof(*ctx));
    if (!ctx) return NULL;
    ctx->params = *params;
    ctx->config = *cfg;
    int backend = params->backend;
    if (backend == SP_BACKEND_CUDA) backend = SP_BACKEND_HIP;
    if (backend == SP_BACKEND_ADRENO || backend == SP_BACKEND_HEXAGON || backend == SP_BACKEND_VULKAN) {
        fprintf(stderr, "[Shannon-Prime] backend %d is not built in this library; "
                        "falling back to CPU storage\n", backend);
        backend = SP_BACKEND_CPU;
    }
    if (backend == SP_BACKEND_HIP) {
        if (sp_hip_cache_init(&ctx->hip_cache, cfg, params->max_seq_len, params->gpu_context) != 0) {
            fprintf(stderr, "[Shannon-Prime] cache init failed: %s; compression stays off\n", sp_hip_last_error());
            free(ctx);
            return NULL;
        }
    } else {
        backend = SP_BACKEND_CPU;
        if (sp_shadow_cache_init(&ctx->cpu_cache, cfg) != 0) {
            fprintf(stderr, "[Shannon-Prime] cache init failed: %s; compression stays off "
                            "(the CPU-storage backend runs its codec on the GPU)\n", sp_hip_last_error());
            free(ctx);
            return NULL;
        }
        if (alloc_host_slots(ctx) != 0) {
            free_host_slots(ctx);
            sp_shadow_cache_free(&ctx->cpu_cache);
            free(ctx);
            return NULL;
        }
    }
    ctx->active_backend = backend;
    if (sp_env_flag(getenv("SHANNON_PRIME_VERBOSE"), 0)) sp_llama_print_config(ctx);
    return ctx;
}

void sp_llama_free(sp_llama_ctx_t *ctx) {
    if (!ctx) return;
    if (ctx->active_backend == SP_BACKEND_HIP) {
        sp_hip_cache_free(&ctx->hip_cache);
    } else {
        free_host_slots(ctx);
        sp_shadow_cache_free(&ctx->cpu_cache);
    }
    free(ctx);
}

/* ---- write / read ---- */

static void note_pos(sp_llama_ctx_t *ctx, int last) {
    if (last + 1 > ctx->n_positions) ctx->n_positions = last + 1;
}

static int pos_ok(const sp_llama_ctx_t *ctx, int layer, int head, int pos, int n) {
    return ctx && layer >= 0 && layer < ctx->config.n_layers && head >= 0 &&
           head < ctx->config.n_heads_kv && pos >= 0 && n > 0 &&
           (long long)pos + n <= ctx->params.max_seq_len;
}

void sp_llama_write_kv(sp_llama_ctx_t *ctx, int layer, int head, int pos, const float *k_vec,
                       const float *v_vec) {
    sp_llama_write_k(ctx, layer, head, pos, k_vec);
    sp_llama_write_v(ctx, layer, head, pos, v_vec);
}

static void write_any(sp_llama_ctx_t *ctx, int is_v, int layer, int head, int start, int n,
                      const float *vecs) {
    if (!pos_ok(ctx, layer, head, start, n) || !vecs) return;
    if (ctx->active_backend == SP_BACKEND_HIP) {
        sp_hip_write_host(&ctx->hip_cache, is_v, layer, head, start, n, vecs);
    } else if (is_v) {
        sp_shadow_write_v_batch(&ctx->cpu_cache, layer, head, start, n, vecs);
    } else {
        sp_shadow_write_k_batch(&ctx->cpu_cache, layer, head, start, n, vecs);
    }
    if (!is_v) note_pos(ctx, start + n - 1);
}

static void read_any(const sp_llama_ctx_t *ctx, int is_v, int layer, int head, int start, int n,
                     float *out, int max_bands) {
    if (!pos_ok(ctx, layer, head, start, n) || !out) return;
    if (ctx->active_backend == SP_BACKEND_HIP) {
        sp_hip_read_host(&ctx->hip_cache, is_v, layer, head, start, n, out, max_bands);
        return;
    }
    if (n == 1) {
        if (is_v) sp_shadow_read_v_partial(&ctx->cpu_cache, layer, head, start, out, max_bands);
        else sp_shadow_read_k_partial(&ctx->cpu_cache, layer, head, start, out, max_bands);
    } else {
        if (is_v) sp_shadow_read_v_batch(&ctx->cpu_cache, layer, head, start, n, out);
        else sp_shadow_read_k_batch(&ctx->cpu_cache, layer, head, start, n, out);
    }
}

void sp_llama_write_k(sp_llama_ctx_t *c, int l, int h, int p, const float *v) { write_any(c, 0, l, h, p, 1, v); }
void sp_llama_write_v(sp_llama_ctx_t *c, int l, int h, int p, const float *v) { write_any(c, 1, l, h, p, 1, v); }
void sp_llama_write_k_batch(sp_llama_ctx_t *c, int l, int h, int s, int n, const float *v) { write_any(c, 0, l, h, s, n, v); }
void sp_llama_write_v_batch(sp_llama_ctx_t *c, int l, int h, int s, int n, const float *v) {
    write_any(c, 1, l, h, s, n, v);
}
void sp_llama_read_k(const sp_llama_ctx_t *c, int l, int h, int p, float *o) { read_any(c, 0, l, h, p, 1, o, -1); }
void sp_llama_read_v(const sp_llama_ctx_t *c, int l, int h, int p, float *o) { read_any(c, 1, l, h, p, 1, o, -1); }
void sp_llama_read_k_partial(const sp_llama_ctx_t *c, int l, int h, int p, float *o, int mb) { read_any(c, 0, l, h, p, 1, o, mb); }
void sp_llama_read_v_partial(const sp_llama_ctx_t *c, int l, int h, int p, float *o, int mb) { read_any(c, 1, l, h, p, 1, o, mb); }
void sp_llama_read_k_batch(const sp_llama_ctx_t *c, int l, int h, int s, int n, float *o) { read_any(c, 0, l, h, s, n, o, -1); }
void sp_llama_read_v_batch(const sp_llama_ctx_t *c, int l, int h, int s, int n, float *o) { read_any(c, 1, l, h, s, n, o, -1); }

/* ---- management (shannon_prime_llama.c:845-908) ---- */

void sp_llama_clear_range(sp_llama_ctx_t *ctx, int start_pos, int end_pos) {
    if (!ctx || start_pos < 0 || end_pos <= start_pos) return;
    if (end_pos > ctx->params.max_seq_len) end_pos = ctx->params.max_seq_len;
    const int n_slots = ctx->config.n_layers * ctx->config.n_heads_kv;
    if (ctx->active_backend == SP_BACKEND_HIP) {
        /* zero the records of every slot in [start_pos, end_pos) */
        for (int is_v = 0; is_v < 2; is_v++) {
            const int B = is_v ? ctx->hip_cache.v_bands.total_bytes : ctx->hip_cache.k_bands.total_bytes;
            unsigned char *base = (unsigned char *)(is_v ? ctx->hip_cache.d_v_cache : ctx->hip_cache.d_k_cache);
            for (int s = 0; s < n_slots; s++) {
                unsigned char *p = base + ((size_t)s * ctx->params.max_seq_len + start_pos) * B;
                sp_hip_memset(p, 0, (size_t)(end_pos - start_pos) * B, ctx->hip_cache.stream);
            }
        }
        sp_hip_stream_sync(ctx->hip_cache.stream);
        return;
    }
    for (int s = 0; s < n_slots; s++) {
        memset(ctx->cpu_cache.k_cache[s] + (size_t)start_pos * ctx->cpu_cache.k_bands.total_bytes, 0,
               (size_t)(end_pos - start_pos) * ctx->cpu_cache.k_bands.total_bytes);
        memset(ctx->cpu_cache.v_cache[s] + (size_t)start_pos * ctx->cpu_cache.v_bands.total_bytes, 0,
               (size_t)(end_pos - start_pos) * ctx->cpu_cache.v_bands.total_bytes);
    }
}

static int k_bytes(const sp_llama_ctx_t *ctx) {
    return ctx->active_backend == SP_BACKEND_HIP ? ctx->hip_cache.k_bands.total_bytes
                                                 : ctx->cpu_cache.k_bands.total_bytes;
}
static int v_bytes(const sp_llama_ctx_t *ctx) {
    return ctx->active_backend == SP_BACKEND_HIP ? ctx->hip_cache.v_bands.total_bytes
                                                 : ctx->cpu_cache.v_bands.total_bytes;
}

sp_llama_memory_t sp_llama_memory(const sp_llama_ctx_t *ctx) {
    sp_llama_memory_t mem;
    memset(&mem, 0, sizeof(mem));
    if (!ctx) return mem;
    const size_t n_slots = (size_t)ctx->config.n_layers * ctx->config.n_heads_kv;
    const int n = ctx->n_positions, hd = ctx->config.head_dim;
    mem.compressed_bytes = n_slots * (size_t)n * (size_t)(k_bytes(ctx) + v_bytes(ctx));
    mem.baseline_bytes = n_slots * (size_t)n * (size_t)hd * 2 * 2;
    mem.compression_ratio = mem.compressed_bytes > 0
        ? (float)mem.baseline_bytes / (float)mem.compressed_bytes : 0.0f;
    mem.n_positions = n;
    return mem;
}

/* validate_k round-trips slot (0, 0, pos 0) like the reference (:914-922). */
float sp_llama_validate_k(sp_llama_ctx_t *ctx, const float *k_vec, int head_dim) {
    if (!ctx || !k_vec || head_dim != ctx->config.head_dim) return 0.0f;
    float *recon = (float *)malloc(sizeof(float) * (size_t)head_dim);
    if (!recon) return 0.0f;
    sp_llama_write_k(ctx, 0, 0, 0, k_vec);
    sp_llama_read_k(ctx, 0, 0, 0, recon);
    float corr = sp_correlation_f32(k_vec, recon, head_dim);
    free(recon);
    return corr;
}

void sp_llama_print_config(const sp_llama_ctx_t *ctx) {
    if (!ctx) return;
    fprintf(stderr, "[Shannon-Prime] llama.cpp integration\n  Backend:  %s\n",
            ctx->active_backend == SP_BACKEND_HIP ? "HIP (MI355X, device-resident)"
                                                  : "CPU storage, HIP codec");
    sp_config_print(&ctx->config);
}

const float *sp_llama_get_freq_factors(const sp_llama_ctx_t *ctx) { (void)ctx; return NULL; }
int sp_llama_get_n_freqs(const sp_llama_ctx_t *ctx) { (void)ctx; return 0; }
const void *sp_llama_get_hexagon_k_buf(const sp_llama_ctx_t *ctx, int layer, int head) {
    (void)ctx; (void)layer; (void)head;
    return NULL;
}
int sp_llama_get_hexagon_k_total_bytes(const sp_llama_ctx_t *ctx) { (void)ctx; return 0; }

static const void *slot_buf(const sp_llama_ctx_t *ctx, int is_v, int layer, int head) {
    if (!ctx || layer < 0 || layer >= ctx->config.n_layers || head < 0 || head >= ctx->config.n_heads_kv)
        return NULL;
    const size_t slot = (size_t)layer * ctx->config.n_heads_kv + head;
    if (ctx->active_backend == SP_BACKEND_HIP) {
        const unsigned char *base = (const unsigned char *)(is_v ? ctx->hip_cache.d_v_cache : ctx->hip_cache.d_k_cache);
        return base + slot * (size_t)ctx->params.max_seq_len * (size_t)(is_v ? v_bytes(ctx) : k_bytes(ctx));
    }
    return is_v ? ctx->cpu_cache.v_cache[slot] : ctx->cpu_cache.k_cache[slot];
}

const void *sp_llama_get_k_buf(const sp_llama_ctx_t *ctx, int layer, int head) { return slot_buf(ctx, 0, layer, head); }
const void *sp_llama_get_v_buf(const sp_llama_ctx_t *ctx, int layer, int head) { return slot_buf(ctx, 1, layer, head); }
int sp_llama_get_k_total_bytes(const sp_llama_ctx_t *ctx) { return ctx ? k_bytes(ctx) : 0; }
int sp_llama_get_v_total_bytes(const sp_llama_ctx_t *ctx) { return ctx ? v_bytes(ctx) : 0; }
int sp_llama_get_backend(const sp_llama_ctx_t *ctx) { return ctx ? ctx->active_backend : -1; }
void *sp_llama_get_hip_cache(const sp_llama_ctx_t *ctx) {
    return (ctx && ctx->active_backend == SP_BACKEND_HIP) ? (void *)&ctx->hip_cache : NULL;
}
