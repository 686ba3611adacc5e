/*
 * sp_env.h -- reading the SHANNON_PRIME_* environment for the bridges.
 *
 * The variable names, their defaults and the draft-role precedence are the
 * reference bridges' interface (src/tools/shannon_prime_llama.c:73-199,
 * src/tools/shannon_prime_llama_sqfree.c:48-101); the code here is a small
 * table of keys over three text decoders.
 */
#ifndef SP_ENV_H
#define SP_ENV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Text of SHANNON_PRIME_<key>. For a draft context (draft != 0) a non-empty
 * SHANNON_PRIME_DRAFT_<key> takes precedence. NULL when the variable is unset. */
const char *sp_env_text(const char *key, int draft);

/* Flag: NULL -> fallback; otherwise 1 exactly when the text starts with '1',
 * 'y' or 'Y' (an empty text is 0). */
int sp_env_flag(const char *text, int fallback);

/* Comma-separated integers, each read like atoi from the start of its token
 * (an empty token reads 0). Fills at most cap values and returns how many;
 * 0 for NULL or empty text. */
int sp_env_int_list(const char *text, int *out, int cap);

/* Comma-separated band indices -> bit mask. Each token may start with spaces
 * or tabs; a token whose first other character is not a digit is skipped;
 * indices of 32 and above are dropped. 0 for NULL or empty text. */
uint32_t sp_env_index_mask(const char *text);

#ifdef __cplusplus
}
#endif
#endif
