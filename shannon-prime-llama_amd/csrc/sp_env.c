/*
 * sp_env.c -- text decoders for the SHANNON_PRIME_* environment (see sp_env.h).
 */
#include "sp_env.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

const char *sp_env_text(const char *key, int draft) {
    char name[192];
    if (draft) {
        snprintf(name, sizeof(name), "SHANNON_PRIME_DRAFT_%s", key);
        const char *t = getenv(name);
        if (t && t[0]) return t;
    }
    snprintf(name, sizeof(name), "SHANNON_PRIME_%s", key);
    return getenv(name);
}

int sp_env_flag(const char *text, int fallback) {
    if (!text) return fallback;
    return text[0] == '1' || text[0] == 'y' || text[0] == 'Y';
}

int sp_env_int_list(const char *text, int *out, int cap) {
    int n = 0;
    if (!text) return 0;
    const char *tok = text;
    while (*tok && n < cap) {
        out[n++] = (int)strtol(tok, NULL, 10);
        const char *comma = strchr(tok, ',');
        if (!comma) break;
        tok = comma + 1;
    }
    return n;
}

uint32_t sp_env_index_mask(const char *text) {
    uint32_t mask = 0u;
    if (!text) return 0u;
    const char *tok = text;
    for (;;) {
        const char *c = tok;
        while (*c == ' ' || *c == '\t') c++;
        if (*c >= '0' && *c <= '9') {
            const long idx = strtol(c, NULL, 10);
            if (idx < 32) mask |= 1u << idx;
        }
        const char *comma = strchr(tok, ',');
        if (!comma) break;
        tok = comma + 1;
    }
    return mask;
}
