/*
 * locus_host.h - C ABI of the host-side helpers of the sampling path, for
 * FFI callers (the reference exposes these as C++ only):
 *   JSON grammar      JsonGrammar::feed/complete (src/locus/model/grammar.hpp:24-57)
 *   JSON allow mask   the per-token allows() of JsonTokenConstraint
 *                     (src/locus/server/server.cpp:154-185), as V/32 words
 *   n-gram draft      ngram_draft (src/locus/model/speculative.hpp:9-19)
 *   backend choice    resolve_backend's rules (src/locus/backend/registry.hpp:124-131)
 * Functions return 0 on success, a negative code on error (lch_last_error()).
 */
#ifndef LOCUS_HOST_H
#define LOCUS_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lch_json lch_json;
typedef struct lch_mask_builder lch_mask_builder;

/* Message of the calling thread's last error. */
const char* lch_last_error(void);

lch_json* lch_json_new(void);
lch_json* lch_json_clone(const lch_json* g);
void lch_json_free(lch_json* g);
/* 1 if byte b continues a valid JSON value (the state advances), else 0. */
int lch_json_feed(lch_json* g, uint8_t b);
int lch_json_complete(const lch_json* g);

/* Token pieces: piece t is blob[offsets[t], offsets[t+1]). */
lch_mask_builder* lch_mask_builder_new(const uint8_t* blob, const uint64_t* offsets, uint32_t n_pieces,
                                       uint32_t cache_entries);
void lch_mask_builder_free(lch_mask_builder* b);
/* words[ceil(vocab/32)]: bit t&31 of word t>>5 set iff token t is allowed
 * after the bytes fed to g (tokens >= n_pieces are always allowed). */
int lch_mask_build(const lch_mask_builder* b, const lch_json* g, uint32_t vocab, uint32_t* words);
void lch_mask_cache_stats(const lch_mask_builder* b, uint64_t* hits, uint64_t* misses);

/* Writes up to min(max_draft, cap) draft ids to out; returns the count. */
uint32_t lch_ngram_draft(const int32_t* ctx, uint32_t n, uint32_t ngram, uint32_t max_draft,
                         int32_t* out, uint32_t cap);

/* Resolves a sampler backend name (explicit, else LOCUS_SAMPLER_BACKEND,
 * else the best available): 0 and the name in name_out; -1 for an unknown
 * or unusable name (std::invalid_argument); -2 when none is usable. */
int lch_resolve_sampler_backend(const char* choice, char* name_out, uint32_t cap);

#ifdef __cplusplus
}
#endif

#endif
