/*
 * sqfree_patch_replay.c -- replays the sqfree call sequence of the reference's
 * llama.cpp hook (patches/llama-cpp-b8861-full-engine.patch) and of its sqfree
 * bridge (src/tools/shannon_prime_llama_sqfree.c) against this library's
 * headers, linking libshannon_prime_hip.so alone.
 *
 *   init  (patch :752-806): sp_config_init, K bits 5,4,4,4,5 (or
 *         SHANNON_PRIME_K_BITS), V mirrors K, residual bits and spinor from the
 *         environment, sp_sqfree_cache_init(&c, &cfg, max_seq, rb, spinor),
 *         the pad_dim it reports;
 *   hook  (patch :1205-1207, :1273-1275): per token, layer and KV head,
 *         sp_sqfree_write_k(c, il, h, 0, gather) then sp_sqfree_read_k(c, il,
 *         h, 0, recon), and the same for V;
 *   free  (patch :866): sp_sqfree_cache_free;
 *   bridge: sp_llama_sqfree_init / write_kv at the token's position / read_k /
 *         read_v / validate_k / free.
 *
 * Input <dir>/x.bin: [2][n_layers][n_tok][n_heads][head_dim] fp32 (K then V).
 * Output <dir>/hook.bin and <dir>/bridge.bin in the same layout, and one line
 * "pad_dim sk_k n_res bytes_k corr" on stdout.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "shannon_prime.h"
#include "shannon_prime_llama.h"

static int env_int(const char *name, int def) {
    const char *t = getenv(name);
    return t ? atoi(t) : def;
}

int main(int argc, char **argv) {
    if (argc != 6) {
        fprintf(stderr, "usage: sqfree_patch_replay <dir> <head_dim> <n_layers> <n_heads_kv> <n_tok>\n");
        return 2;
    }
    const char *dir = argv[1];
    const int hd = atoi(argv[2]), L = atoi(argv[3]), H = atoi(argv[4]), T = atoi(argv[5]);
    const size_t n = (size_t)2 * L * T * H * hd;
    float *x = (float *)malloc(n * sizeof(float)), *y = (float *)calloc(n, sizeof(float));
    float *z = (float *)calloc(n, sizeof(float));
    char path[4096];
    snprintf(path, sizeof(path), "%s/x.bin", dir);
    FILE *f = fopen(path, "rb");
    if (!x || !y || !z || !f || fread(x, sizeof(float), n, f) != n) { fprintf(stderr, "read %s\n", path); return 3; }
    fclose(f);

    /* ---- the hook's sqfree path ---- */
    sp_config_t cfg;
    sp_config_init(&cfg, hd, L, H);
    cfg.k_n_bands = 5;
    const int bits[5] = {5, 4, 4, 4, 5};
    memcpy(cfg.k_band_bits, bits, sizeof(bits));
    cfg.v_n_bands = cfg.k_n_bands;
    memcpy(cfg.v_band_bits, cfg.k_band_bits, sizeof(int) * (size_t)cfg.k_n_bands);
    int rb = env_int("SHANNON_PRIME_RESIDUAL_BITS", 3);
    if (rb < 1) rb = 1;
    if (rb > 4) rb = 4;
    const char *sp = getenv("SHANNON_PRIME_SPINOR");
    const int spinor = sp && sp[0] == '1';
    sp_sqfree_cache_t c;
    if (sp_sqfree_cache_init(&c, &cfg, T, rb, spinor) != 0) { fprintf(stderr, "sqfree init failed\n"); return 4; }
    for (int t = 0; t < T; t++)
        for (int il = 0; il < L; il++)
            for (int h = 0; h < H; h++)
                for (int side = 0; side < 2; side++) {
                    const size_t off = ((((size_t)side * L + il) * T + t) * H + h) * hd;
                    if (side == 0) {
                        sp_sqfree_write_k(&c, il, h, 0, x + off);
                        sp_sqfree_read_k(&c, il, h, 0, y + off);
                    } else {
                        sp_sqfree_write_v(&c, il, h, 0, x + off);
                        sp_sqfree_read_v(&c, il, h, 0, y + off);
                    }
                }
    const int pad = c.pad_dim, sk = c.mask.sk_k, nres = c.mask.n_res, bk = c.bytes_per_pos_k;
    sp_sqfree_cache_free(&c);

    /* ---- the sqfree bridge ---- */
    sp_llama_sqfree_ctx_t *ctx = sp_llama_sqfree_init(hd, L, H, T);
    if (!ctx) { fprintf(stderr, "bridge init failed\n"); return 5; }
    for (int t = 0; t < T; t++)
        for (int il = 0; il < L; il++)
            for (int h = 0; h < H; h++) {
                const size_t k = ((((size_t)0 * L + il) * T + t) * H + h) * hd;
                const size_t v = ((((size_t)1 * L + il) * T + t) * H + h) * hd;
                sp_llama_sqfree_write_kv(ctx, il, h, t, x + k, x + v);
            }
    for (int t = 0; t < T; t++)
        for (int il = 0; il < L; il++)
            for (int h = 0; h < H; h++) {
                const size_t k = ((((size_t)0 * L + il) * T + t) * H + h) * hd;
                const size_t v = ((((size_t)1 * L + il) * T + t) * H + h) * hd;
                sp_llama_sqfree_read_k(ctx, il, h, t, z + k);
                sp_llama_sqfree_read_v(ctx, il, h, t, z + v);
            }
    const float corr = sp_llama_sqfree_validate_k(ctx, x, hd);
    sp_llama_sqfree_free(ctx);

    snprintf(path, sizeof(path), "%s/hook.bin", dir);
    f = fopen(path, "wb");
    if (!f || fwrite(y, sizeof(float), n, f) != n || fclose(f)) return 6;
    snprintf(path, sizeof(path), "%s/bridge.bin", dir);
    f = fopen(path, "wb");
    if (!f || fwrite(z, sizeof(float), n, f) != n || fclose(f)) return 6;
    printf("%d %d %d %d %.6f\n", pad, sk, nres, bk, corr);
    free(x);
    free(y);
    free(z);
    return 0;
}
