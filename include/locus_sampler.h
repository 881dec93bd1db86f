/*
 * locus_sampler.h - C ABI of the MI355X (gfx950) token sampler.
 *
 * The drop-in boundary for the reference's per-step sampling path. The
 * reference has no C ABI for it: its callers use free C++ functions
 * (src/locus/model/sampling.hpp:70-89, llama.hpp:352) on host spans, one
 * row at a time (engine.cpp:423-450, engine.cpp:357-396). This ABI is what a
 * backend-registry entry (registry.hpp:107-131) or any FFI binds: plain
 * pointers and sizes, no exceptions, stream-ordered and asynchronous.
 *
 * All buffer pointers in lcs_batch / lcs_out / lcs_verify_* are DEVICE
 * pointers unless the field says "host". Every call is asynchronous on the
 * given HIP stream (a hipStream_t passed as void*, NULL = default stream);
 * outputs are valid once the stream has been synchronised. One context must
 * not be used by two threads at once; separate contexts are independent.
 */
#ifndef LOCUS_SAMPLER_H
#define LOCUS_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lcs_ctx lcs_ctx;

/* A row's raw statistics, as the fused lm-head's epilogue leaves them
 * (lcs_lmhead_out.stats): the log-normaliser of logprobs_from
 * (sampling.cpp:155-163) and the first index of the max (llama.cpp:1237-1245)
 * over the row's raw logits. 16 bytes. */
typedef struct lcs_row_stats {
    double log_z;              /* log sum_i exp(logit_i) */
    float max;                 /* largest raw logit */
    int32_t argmax;            /* its first index */
} lcs_row_stats;

enum lcs_status {
    LCS_OK = 0,
    LCS_ERR_INVALID_ARG = -1, /* bad pointer, size, alignment or dtype */
    LCS_ERR_NO_DEVICE = -2,   /* no usable gfx950 device */
    LCS_ERR_HIP = -3,         /* a HIP runtime call failed (see lcs_last_error) */
    LCS_ERR_CAPACITY = -4     /* request exceeds the context's create-time limits */
};

enum lcs_dtype { LCS_F32 = 0, LCS_BF16 = 1 };

enum lcs_flags {
    LCS_WANT_LOGPROBS = 1u,   /* write chosen_lp and the n_top alternatives */
    LCS_WRITE_PENALIZED = 2u  /* write penalised logits back in place (f32 only) */
};

/* Per-row sampling parameters: field-for-field the reference's
 * SamplingParams (src/locus/model/sampling.hpp:23-40), 32 bytes. */
typedef struct lcs_params {
    float temperature;        /* <= 0: greedy (argmax) */
    uint32_t top_k;           /* 0: disabled */
    float top_p;              /* 1: disabled */
    float min_p;              /* 0: disabled */
    float repeat_penalty;     /* 1: disabled */
    float frequency_penalty;  /* 0: disabled */
    float presence_penalty;   /* 0: disabled */
    uint32_t repeat_last_n;   /* trailing history entries the penalties see */
} lcs_params;

/* One batch of rows to sample: the batched form of
 * sample(logits, params, history, rng, constraint) (sampling.hpp:70-73)
 * followed, when LCS_WANT_LOGPROBS is set, by
 * logprobs_from(raw logits, chosen, n_top, ...) (sampling.hpp:86-89),
 * per row exactly as Engine::sample_from does (engine.cpp:423-450). */
typedef struct lcs_batch {
    uint32_t rows;
    uint32_t vocab;            /* V, 1 <= V <= 262144 */
    uint32_t dtype;            /* lcs_dtype */
    uint32_t flags;            /* lcs_flags */
    uint64_t row_stride;       /* elements between rows; multiple of 4 (f32) / 8 (bf16) */
    const void* logits;        /* rows x row_stride, 16-byte aligned, raw logits */
    const lcs_params* params;  /* rows */
    const lcs_params* params_host; /* optional HOST copy of params (dispatch hint) or NULL */
    const uint32_t* hist_off;  /* rows + 1 CSR offsets into hist_ids, or NULL */
    const int32_t* hist_ids;   /* token history (the request's generated ids) */
    const double* u;           /* rows: uniform in [0,1) per stochastic row, the
                                  generate_canonical<double,53> draw of the row's
                                  mt19937_64 (libstdc++ random.tcc:3348-3380).
                                  May be NULL only when params_host is given and
                                  no row has temperature > 0; otherwise a NULL u
                                  returns LCS_ERR_INVALID_ARG before any launch */
    const uint32_t* mask;      /* rows x mask_words allow-bits (bit t&31 of word
                                  t>>5, LSB first), or NULL for no constraint */
    const uint8_t* has_mask;   /* rows, nonzero = row constrained; NULL = all rows
                                  constrained when mask != NULL */
    uint32_t mask_words;       /* >= ceil(V/32) when mask != NULL */
    uint32_t n_top;            /* alternatives per row (<= the context's max_top) */
    const int32_t* lp_ids;     /* rows, or NULL: with LCS_WANT_LOGPROBS, chosen_lp
                                  reports the logprob of lp_ids[row] instead of the
                                  sampled id (logprobs_from's `chosen` argument,
                                  sampling.hpp:86-89); ids outside [0, V) give 0 */
    /* Device-resident penalty windows (lcs_windows_reserve). NULL: every row's
     * window comes from hist_off / hist_ids. Otherwise every row must be a
     * min-p window row (temperature > 0, min_p > 0, top_k 0, no mask; checked
     * against params_host, which is then required): */
    const int32_t* win_slot;   /* rows: the row's window slot, or -1 (hist_off / hist_ids) */
    const int32_t* win_push;   /* rows: the id the sequence appended since the slot's last
                                  call (its previous sample, engine.cpp:436), read when
                                  win_len grows by one */
    const uint32_t* win_len;   /* rows: the history length after that append: the slot's
                                  stored length (nothing appended) or one more; the slot's
                                  window, vocabulary and repeat_last_n must match the row,
                                  else the row gets id -1 and LCS_STATUS_WINDOW */
    /* Optional (NULL: computed here): each row's raw statistics over the same
     * logits, from the lcs_lmhead call that wrote them (lcs_lmhead_out.stats).
     * With LCS_WANT_LOGPROBS, greedy, min-p window and sliced top-k rows then
     * take their log-normaliser from it instead of summing the row's
     * exponentials again; the other paths compute their own. */
    const lcs_row_stats* raw_stats;
} lcs_batch;

/* Per-row diagnostics (optional output): the survivor set of the reference's
 * candidate walk (sampling.cpp:70-147). */
typedef struct lcs_row_diag {
    uint32_t n_cand;    /* candidates after the constraint */
    uint32_t keep;      /* survivors after top-k, top-p, min-p (0 for greedy) */
    float maxl;         /* max penalised candidate logit */
    float boundary;     /* logit of the last survivor */
    uint32_t path;      /* implementation path taken (LCS_PATH_*) */
    uint32_t reserved;
    double sum;         /* softmax normaliser over the candidate list */
    double kept_sum;    /* mass of the survivors */
} lcs_row_diag;

enum lcs_path {
    LCS_PATH_GREEDY = 1u,     /* sliced argmax */
    LCS_PATH_WINDOW = 2u,     /* sliced min-p window, certified normaliser */
    LCS_PATH_WINDOW_EXACT = 3u, /* window with an exactly recomputed normaliser */
    LCS_PATH_GENERAL = 4u,    /* single-workgroup exact selection */
    LCS_PATH_TOPK = 5u,       /* sliced exact top-k (k <= 64) */
    LCS_PATH_NUCLEUS = 6u     /* sliced histogram passes, exact decisions (no top-k) */
};

typedef struct lcs_out {
    int32_t* ids;              /* rows: sampled token id */
    float* chosen_lp;          /* rows (LCS_WANT_LOGPROBS) */
    int32_t* top_ids;          /* rows x n_top (LCS_WANT_LOGPROBS) */
    float* top_lp;             /* rows x n_top (LCS_WANT_LOGPROBS) */
    lcs_row_diag* diag;        /* rows, or NULL */
} lcs_out;

/* Speculative-decoding verify (engine.cpp:357-396): row j of sequence s holds
 * the logits that predict draft[s*rows_per_seq + j]. */
typedef struct lcs_verify_batch {
    uint32_t n_seq;
    uint32_t rows_per_seq;     /* 1..64 */
    uint32_t vocab;
    uint32_t dtype;            /* lcs_dtype */
    uint64_t row_stride;       /* elements; multiple of 4 (f32) / 8 (bf16) */
    const void* logits;        /* (n_seq * rows_per_seq) x row_stride */
    const int32_t* draft;      /* n_seq * rows_per_seq draft ids */
} lcs_verify_batch;

typedef struct lcs_verify_out {
    int32_t* argmax_ids;       /* per row: argmax (llama.cpp:1237-1245) */
    float* draft_lp;           /* per row: logprobs_from(row, draft, 0).chosen_lp */
    uint32_t* accept_len;      /* per sequence: leading rows whose argmax == draft */
} lcs_verify_out;

/* Prompt-lookup drafts for a batch of device-resident contexts: per
 * sequence, the reference's ngram_draft (src/locus/model/speculative.cpp:7-28,
 * declared at speculative.hpp:9-19). */
typedef struct lcs_draft_batch {
    uint32_t n_seq;
    uint32_t ngram;            /* 0..64 (0: every draft empty) */
    uint32_t max_draft;        /* 0..256 */
    const uint32_t* ctx_off;   /* n_seq + 1 CSR offsets into ctx_ids */
    const int32_t* ctx_ids;    /* each sequence's context (prompt + generated) */
} lcs_draft_batch;

typedef struct lcs_draft_out {
    int32_t* draft;            /* n_seq x max_draft; entries past the draft are -1 */
    uint32_t* draft_len;       /* n_seq: the draft's length (0..max_draft) */
} lcs_draft_out;

/* The lm-head product with the sampler's first statistics in its epilogue:
 * logits = x w^T for bf16 x (rows x hidden, the normed hidden states) and w
 * (vocab x hidden, the output weight), accumulated in f32 - the reference's
 * matvec(out_w, norm(x)) per token (src/locus/model/llama.cpp:512-513,
 * 754-761). From the epilogue, without re-reading the logits: each row's
 * argmax (llama.cpp:1237-1245) and log-normaliser, the log-probability of a
 * draft token (logprobs_from with chosen = draft, sampling.cpp:150-170) and
 * each sequence's acceptance length (engine.cpp:357-383). */
typedef struct lcs_lmhead_batch {
    uint32_t rows;             /* hidden vectors, <= the context's max_rows */
    uint32_t vocab;            /* <= the context's max_vocab */
    uint32_t hidden;           /* multiple of 64 */
    uint32_t rows_per_seq;     /* 1..64 rows per sequence (accept_len), or 0 */
    const void* x;             /* rows x hidden bf16, 16-byte aligned */
    const void* w;             /* vocab x hidden bf16, 16-byte aligned */
    const int32_t* draft;      /* rows, or NULL: the token whose logprob each row reports */
} lcs_lmhead_batch;

typedef struct lcs_lmhead_out {
    float* logits;             /* rows x ld_logits f32, or NULL: not written */
    uint64_t ld_logits;        /* elements between rows of logits (>= vocab) */
    int32_t* argmax_ids;       /* rows */
    float* log_z;              /* rows: log sum exp of the row, or NULL */
    float* draft_lp;           /* rows (when draft != NULL), 0 for ids outside [0, vocab) */
    uint32_t* accept_len;      /* rows / rows_per_seq, or NULL */
    lcs_row_stats* stats;      /* rows, or NULL: each row's log_z, max and argmax, for
                                  lcs_batch.raw_stats of the lcs_sample call that samples
                                  these logits */
} lcs_lmhead_out;

/* Number of usable gfx950 devices (0 when none). Replaces the runtime probe
 * that sets Backend::available (registry.cpp:148-223, cuda_stub.cpp:29). */
int lcs_probe(int* n_devices);

/* Allocates the per-context workspace on `device` once; no call below
 * allocates device memory. Returns NULL on failure (lcs_last_error(NULL)). */
lcs_ctx* lcs_create(int device, uint32_t max_rows, uint32_t max_vocab,
                    uint32_t max_hist, uint32_t max_top);
void lcs_destroy(lcs_ctx* ctx);

/* Device-resident penalty windows: the counts apply_penalties builds from
 * the history's last repeat_last_n ids (sampling.cpp:22-28) kept per
 * sequence slot on the device and updated in place by each lcs_sample call
 * that names the slot (one id enters the window, at most one leaves), so a
 * serving loop uploads no history. Allocates room for `slots` slots of
 * windows up to `max_window` ids (<= 4096), once (call it before the hot
 * loop; calling again with larger limits reallocates and clears every slot).
 * No counterpart in the reference, which rescans the history per call. */
int lcs_windows_reserve(lcs_ctx* ctx, uint32_t slots, uint32_t max_window);

/* (Re)starts slot `slot` for a sequence whose generated history so far is
 * ids[0..n) (device memory; n may be 0, ids may then be NULL), penalised
 * over its last `window` ids (1..max_window: the rows' repeat_last_n) for
 * a vocabulary of `vocab` ids. Asynchronous on `stream`. */
int lcs_windows_load(lcs_ctx* ctx, uint32_t slot, const int32_t* ids, uint32_t n, uint32_t window,
                     uint32_t vocab, void* stream);

/* Batched sample (+ logprobs): replaces per-row sample()/logprobs_from()
 * (sampling.hpp:70-89) as called from engine.cpp:430-442. */
int lcs_sample(lcs_ctx* ctx, const lcs_batch* batch, const lcs_out* out, void* stream);

/* Batched logprobs_from (sampling.hpp:86-89, sampling.cpp:150-190) with no
 * draw: per row, into out->chosen_lp, the log-probability of chosen[row]
 * under the row's raw logits (0 for an id outside [0, V); chosen NULL: of the
 * row's argmax), and into out->top_ids / top_lp the batch's n_top most likely
 * ids with theirs; out->ids, when given, receives each row's argmax. Reads
 * rows, vocab, dtype, row_stride, logits, n_top and raw_stats of batch and
 * ignores the rest (params, history, u, mask, flags, windows). The backend
 * registry's logprobs_batch op. */
int lcs_logprobs(lcs_ctx* ctx, const lcs_batch* batch, const int32_t* chosen, const lcs_out* out, void* stream);

/* lcs_sample without a context, allocating nothing: for callers that cannot
 * call hipMalloc (code under HIP graph capture, tight serving loops, harnesses
 * that forbid it). No counterpart in the reference. Runs on the current
 * device with the same batch, outputs and results as lcs_sample; its
 * workspace is one static device array per GPU (about 38 MiB, held until the
 * process ends), sized for rows <= 64, any vocabulary up to 262144, n_top <=
 * 20 and penalty windows up to 8192. More rows return LCS_ERR_CAPACITY with
 * nothing launched. Calls share that array: calls that overlap on one GPU
 * (two streams, or two threads) race and must be serialised by the caller.
 * Its status bits are not readable (lcs_get_status needs a context); failures
 * are reported by lcs_last_error(NULL). */
int lcs_sample_noalloc(const lcs_batch* batch, const lcs_out* out, void* stream);

/* Batched greedy verify: replaces the argmax loop of engine.cpp:357-396 and
 * adds the draft logprob (sampling.cpp:150-170 with chosen = draft). */
int lcs_verify(lcs_ctx* ctx, const lcs_verify_batch* batch, const lcs_verify_out* out,
               void* stream);

/* Batched n-gram drafts: replaces the per-sequence host call of
 * engine.cpp:328-329 (speculative.cpp:7-28) when contexts live on the device.
 * Drafts feed lcs_verify. Allocates nothing and uses no context workspace, so
 * n_seq is not bounded by the context's max_rows. */
int lcs_ngram_draft(lcs_ctx* ctx, const lcs_draft_batch* batch, const lcs_draft_out* out, void* stream);

/* The fused lm-head product (see lcs_lmhead_batch); no counterpart call in
 * the reference, which computes the logits with matvec and reads them again
 * in argmax / logprobs_from. Allocates nothing. */
int lcs_lmhead(lcs_ctx* ctx, const lcs_lmhead_batch* batch, const lcs_lmhead_out* out, void* stream);

/* Sticky device-side status bits of ctx (LCS_STATUS_*), set by kernels that
 * met an input they could not serve. Every bit comes with id -1 on each
 * affected row (also from lcs_sample_noalloc, whose status is not readable),
 * so a caller that sees no -1 id needs no status read. Blocking:
 * reads device memory; call after the work's stream has been synchronised.
 * No counterpart in the reference (its sampler cannot fail). */
int lcs_get_status(lcs_ctx* ctx, uint32_t* status_out, int reset);

enum lcs_status_bits {
    LCS_STATUS_HIST_CAPACITY = 1u,  /* a penalty window exceeded max_hist */
    LCS_STATUS_SELECT = 2u,         /* a selection bin exceeded its capacity */
    LCS_STATUS_WINDOW = 4u          /* a row's window slot did not match it (win_len, window,
                                       vocabulary) */
};

/* Message of the last failure on ctx (or, when NULL, of the last lcs_create
 * or lcs_sample_noalloc on this thread). */
const char* lcs_last_error(const lcs_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif /* LOCUS_SAMPLER_H */
