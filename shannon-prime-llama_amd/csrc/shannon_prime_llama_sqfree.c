/*
 * shannon_prime_llama_sqfree.c -- the sqfree + spinor bridge
 * (src/tools/shannon_prime_llama_sqfree.c:48-240) over the core sqfree cache
 * of this library (sp_sqfree_cache_t, records in HBM, codec on the GPU).
 */
#include "../../include/shannon_prime_llama.h"
#include "../../include/sp_hip.h"
#include "sp_env.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct sp_llama_sqfree_ctx_s {
    sp_sqfree_cache_t        cache;
    sp_llama_sqfree_config_t env;
    FILE                    *dump;        /* SHANNON_PRIME_DUMP_K target, or NULL */
    long long                dump_count;
    long long                dump_limit;  /* 0: no limit */
};

/* An opt-in switch of this bridge: on only for the exact text "1". */
static int switched_on(const char *name) {
    const char *t = getenv(name);
    return t && strcmp(t, "1") == 0;
}

void sp_llama_sqfree_config_from_env(sp_llama_sqfree_config_t *out) {
    static const int k_sqfree_bits[5] = {5, 4, 4, 4, 5};  /* five skeleton bands */
    static const int k_ship_bits[4] = {5, 5, 4, 3};
    if (!out) return;
    memset(out, 0, sizeof(*out));
    out->sqfree_enabled = switched_on("SHANNON_PRIME_SQFREE");
    out->spinor_enabled = switched_on("SHANNON_PRIME_SPINOR");
    if (out->spinor_enabled && !out->sqfree_enabled) {
        fprintf(stderr, "[Shannon-Prime] SPINOR=1 requires SQFREE=1. Enabling SQFREE.\n");
        out->sqfree_enabled = 1;
    }
    const char *rb = getenv("SHANNON_PRIME_RESIDUAL_BITS");
    int bits = rb ? atoi(rb) : 3;
    out->residual_bits = bits < 1 ? 1 : bits > 4 ? 4 : bits;
    const char *sf = getenv("SHANNON_PRIME_SK_FRAC");
    float frac = sf ? (float)atof(sf) : 0.75f;
    out->sk_frac = frac < 0.1f ? 0.1f : frac > 1.0f ? 1.0f : frac;
    const char *kb = getenv("SHANNON_PRIME_K_BITS");
    if (kb) {
        out->n_k_bands = sp_env_int_list(kb, out->k_band_bits, SP_MAX_BANDS);
    } else if (out->sqfree_enabled) {
        out->n_k_bands = 5;
        memcpy(out->k_band_bits, k_sqfree_bits, sizeof(k_sqfree_bits));
    } else {
        out->n_k_bands = 4;
        memcpy(out->k_band_bits, k_ship_bits, sizeof(k_ship_bits));
    }
}

sp_llama_sqfree_ctx_t *sp_llama_sqfree_init(int head_dim, int n_layers, int n_heads_kv, int max_seq_len) {
    sp_llama_sqfree_config_t env;
    sp_llama_sqfree_config_from_env(&env);
    if (!env.sqfree_enabled) return NULL;
    sp_llama_sqfree_ctx_t *ctx = (sp_llama_sqfree_ctx_t *)calloc(1, sizeof(*ctx));
    if (!ctx) return NULL;
    ctx->env = env;
    sp_config_t cfg;
    sp_config_init(&cfg, head_dim, n_layers, n_heads_kv);
    cfg.k_n_bands = env.n_k_bands;
    cfg.v_n_bands = env.n_k_bands;  /* V takes K's allocation on this path */
    for (int b = 0; b < env.n_k_bands; b++) cfg.k_band_bits[b] = cfg.v_band_bits[b] = env.k_band_bits[b];
    if (sp_sqfree_cache_init(&ctx->cache, &cfg, max_seq_len, env.residual_bits, env.spinor_enabled) != 0) {
        fprintf(stderr, "[Shannon-Prime SQFREE] cache init failed: %s\n", sp_hip_last_error());
        free(ctx);
        return NULL;
    }
    const char *dump_path = getenv("SHANNON_PRIME_DUMP_K");
    if (dump_path && dump_path[0]) {
        ctx->dump = fopen(dump_path, "wb");
        if (ctx->dump) {
            const char *lim = getenv("SHANNON_PRIME_DUMP_K_LIMIT");
            ctx->dump_limit = lim ? atoll(lim) : 8192;
            fprintf(stderr, "[Shannon-Prime] K dump -> %s (limit=%lld vectors)\n", dump_path, ctx->dump_limit);
        } else {
            fprintf(stderr, "[Shannon-Prime] warning: failed to open K dump '%s'\n", dump_path);
        }
    }
    if (getenv("SHANNON_PRIME_VERBOSE")) {
        fprintf(stderr, "[Shannon-Prime SQFREE] head_dim=%d pad_dim=%d skeleton=%d residual=%d "
                        "residual_bits=%d spinor=%s K bits=",
                head_dim, ctx->cache.pad_dim, ctx->cache.mask.sk_k, ctx->cache.mask.n_res, env.residual_bits,
                env.spinor_enabled ? "on" : "off");
        for (int b = 0; b < env.n_k_bands; b++)
            fprintf(stderr, "%d%s", env.k_band_bits[b], b + 1 < env.n_k_bands ? "," : "\n");
    }
    return ctx;
}

void sp_llama_sqfree_free(sp_llama_sqfree_ctx_t *ctx) {
    if (!ctx) return;
    if (ctx->dump) {
        fprintf(stderr, "[Shannon-Prime] K dump closed (%lld vectors written)\n", ctx->dump_count);
        fclose(ctx->dump);
    }
    sp_sqfree_cache_free(&ctx->cache);
    free(ctx);
}

void sp_llama_sqfree_write_kv(sp_llama_sqfree_ctx_t *ctx, int layer, int head, int pos, const float *k_vec,
                              const float *v_vec) {
    if (!ctx) return;
    if (ctx->dump && k_vec && (ctx->dump_limit == 0 || ctx->dump_count < ctx->dump_limit)) {
        fwrite(k_vec, sizeof(float), (size_t)ctx->cache.config.head_dim, ctx->dump);
        ctx->dump_count++;
    }
    sp_sqfree_write_k(&ctx->cache, layer, head, pos, k_vec);
    sp_sqfree_write_v(&ctx->cache, layer, head, pos, v_vec);
}

void sp_llama_sqfree_read_k(const sp_llama_sqfree_ctx_t *ctx, int layer, int head, int pos, float *k_out) {
    if (ctx) sp_sqfree_read_k(&ctx->cache, layer, head, pos, k_out);
}

void sp_llama_sqfree_read_v(const sp_llama_sqfree_ctx_t *ctx, int layer, int head, int pos, float *v_out) {
    if (ctx) sp_sqfree_read_v(&ctx->cache, layer, head, pos, v_out);
}

float sp_llama_sqfree_validate_k(sp_llama_sqfree_ctx_t *ctx, const float *k_vec, int head_dim) {
    if (!ctx || !k_vec || head_dim != ctx->cache.config.head_dim) return 0.0f;
    float *back = (float *)malloc(sizeof(float) * (size_t)head_dim);
    if (!back) return 0.0f;
    sp_sqfree_write_k(&ctx->cache, 0, 0, 0, k_vec);
    sp_sqfree_read_k(&ctx->cache, 0, 0, 0, back);
    const float corr = sp_correlation_f32(k_vec, back, head_dim);
    free(back);
    return corr;
}

const sp_sqfree_cache_t *sp_llama_sqfree_get_cache(const sp_llama_sqfree_ctx_t *ctx) {
    return ctx ? &ctx->cache : NULL;
}
