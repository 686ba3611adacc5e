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

/* ---- env parsing (shannon_prime_llama.c:73-165) ---- */

static int parse_env_bool(const char *name, int default_val) {
    const char *v = getenv(name);
    if (!v) return default_val;
    return (v[0] == '1' || v[0] == 'y' || v[0] == 'Y');
}

static int parse_env_bits_autocount(const char *name, int *bits, int max_n) {
    const char *v = getenv(name);
    if (!v || !*v) return 0;
    int i = 0;
    const char *p = v;
    while (i < max_n && *p) {
        bits[i++] = atoi(p);
        while (*p && *p != ',') p++;
        if (*p == ',') p++;
    }
    return i;
}

static const char *resolve_role_name(const char *base, sp_llama_role_t role, char *out, size_t n) {
    if (role == SP_LLAMA_ROLE_DRAFT) {
        snprintf(out, n, "SHANNON_PRIME_DRAFT_%s", base);
        const char *v = getenv(out);
        if (v && *v) return out;
    }
    snprintf(out, n, "SHANNON_PRIME_%s", base);
    return out;
}

static const char *role_getenv(const char *base, sp_llama_role_t role) {
    char name[160];
    return getenv(resolve_role_name(base, role, name, sizeof(name)));
}

static int parse_role_bool(const char *base, sp_llama_role_t role, int def) {
    char name[160];
    return parse_env_bool(resolve_role_name(base, role, name, sizeof(name)), def);
}

static int parse_role_bits(const char *base, sp_llama_role_t role, int *bits, int max_n) {
    char name[160];
    return parse_env_bits_autocount(resolve_role_name(base, role, name, sizeof(name)), bits, max_n);
}

static uint32_t parse_role_ternary_mask(const char *base, sp_llama_role_t role) {
    const char *v = role_getenv(base, role);
    if (!v || !*v) return 0u;
    uint32_t mask = 0u;
    const char *p = v;
    while (*p) {
        while (*p == ',' || *p == ' ' || *p == '\t') p++;
        if (!*p) break;
        if (*p < '0' || *p > '9') {
            while (*p && *p != ',') p++;
            continue;
        }
        int idx = atoi(p);
        if (idx >= 0 && idx < 32) mask |= (1u << idx);
        while (*p && *p != ',') p++;
    }
    return mask;
}

/* Draft presets (shannon_prime_llama.c:177-199). */
static int apply_draft_preset(int *k_bits, int *k_n, int *v_bits, int *v_n) {
    const char *preset = getenv("SHANNON_PRIME_DRAFT_PRESET");
    if (!preset || !*preset) return 0;
    if (strcmp(preset, "aggressive") == 0) {
        k_bits[0] = 2; k_bits[1] = 1; *k_n = 2;
        v_bits[0] = 1; *v_n = 1;
        return 1;
    }
    if (strcmp(preset, "ternary") == 0) {
        k_bits[0] = 2; k_bits[1] = 2; *k_n = 2;
        v_bits[0] = 2; *v_n = 1;
        return 1;
    }
    if (strcmp(preset, "ship") == 0) return 1;
    fprintf(stderr, "[Shannon-Prime] unknown SHANNON_PRIME_DRAFT_PRESET '%s' "
                    "(known: aggressive, ternary, ship); ignoring\n", preset);
    return 0;
}

/* ---- lifecycle ---- */

sp_llama_ctx_t *sp_llama_init(const sp_llama_params_t *params) {
    return sp_llama_init_with_role(params, SP_LLAMA_ROLE_DEFAULT);
}

sp_llama_ctx_t *sp_llama_init_with_role(const sp_llama_params_t *params, sp_llama_role_t role) {
    if (!params) return NULL;
    if (!parse_role_bool("ENABLED", role, 0)) return NULL;

    sp_config_t cfg;
    sp_config_init(&cfg, params->head_dim, params->n_layers, params->n_heads_kv);
    /* head-dim adaptive defaults (shannon_prime_llama.c:235-252) */
    static const int k128[4] = {5, 5, 4, 3}, k64[4] = {5, 4, 4, 4};
    if (params->head_dim >= 128) {
        cfg.k_n_bands = 4;
        memcpy(cfg.k_band_bits, k128, sizeof(k128));
        cfg.v_band_bits[0] = 3;
    } else {
        cfg.k_n_bands = 3;
        memcpy(cfg.k_band_bits, k64, sizeof(k64));
        cfg.v_band_bits[0] = 5;
    }
    cfg.v_n_bands = 1;
    if (role == SP_LLAMA_ROLE_DRAFT)
        apply_draft_preset(cfg.k_band_bits, &cfg.k_n_bands, cfg.v_band_bits, &cfg.v_n_bands);
    int kn = parse_role_bits("K_BITS", role, cfg.k_band_bits, SP_MAX_BANDS);
    if (kn > 0) cfg.k_n_bands = kn;
    int vn = parse_role_bits("V_BITS", role, cfg.v_band_bits, SP_MAX_BANDS);
    if (vn > 0) cfg.v_n_bands = vn;
    cfg.use_mobius_mask = parse_role_bool("MOBIUS", role, 1);
    cfg.k_ternary_mask = parse_role_ternary_mask("K_TERNARY_BANDS", role);
    cfg.v_ternary_mask = parse_role_ternary_mask("V_TERNARY_BANDS", role);
    cfg.use_fp8 = parse_role_bool("FP8", role, 0);
    const char *norm = role_getenv("VHT2_NORM", role);
    if (norm && strcmp(norm, "stage") == 0) cfg.vht2_norm = SP_VHT2_NORM_STAGE;

    sp_llama_params_t p = *params;
    const char *b = role_getenv("BACKEND", role);
    if (b) {
        if (strcmp(b, "cpu") == 0) p.backend = SP_BACKEND_CPU;
        else if (!strcmp(b, "hip") || !strcmp(b, "gpu") || !strcmp(b, "rocm") || !strcmp(b, "cuda"))
            p.backend = SP_BACKEND_HIP;
        else if (!strcmp(b, "hexagon")) p.backend = SP_BACKEND_HEXAGON;
        else if (!strcmp(b, "adreno")) p.backend = SP_BACKEND_ADRENO;
        else if (!strcmp(b, "vulkan")) p.backend = SP_BACKEND_VULKAN;
    }
    if (cfg.use_fp8)
        fprintf(stderr, "[Shannon-Prime]%s SHANNON_PRIME_FP8=1 requested but this library has "
                        "no fp8 path; using integer band codes.\n",
                role == SP_LLAMA_ROLE_DRAFT ? " [draft]" : role == SP_LLAMA_ROLE_TARGET ? " [target]" : "");
    return sp_llama_init_config(&p, &cfg);
}

static int alloc_host_slots(sp_llama_ctx_t *ctx) {
    const int n_slots = ctx->config.n_layers * ctx->config.n_heads_kv;
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
            free(ctx);
            return NULL;
        }
    } else {
        backend = SP_BACKEND_CPU;
        if (sp_shadow_cache_init(&ctx->cpu_cache, cfg) != 0) {
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
    if (parse_env_bool("SHANNON_PRIME_VERBOSE", 0)) sp_llama_print_config(ctx);
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
