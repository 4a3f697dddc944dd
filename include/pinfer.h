/* pinfer — public C API of nibblemac_amd's MI355X engine (libpinfer.so).
 *
 * Drop-in for the reference engine's API (engine/include/pinfer.h:1-197): the same function
 * names, struct layouts (field order and types), error codes and version. The engine runs
 * Qwen3.5 hybrid models stored in .pq files whose matrices are Q4K_G32; the forward pass, the
 * Gated DeltaNet state and the KV cache live in HBM of one MI355X and every weight product,
 * recurrence and attention runs as a gfx950 HIP kernel (include/nmx.h). Speculative greedy
 * decoding with the MTP head verifies k drafts per pass and returns exactly the tokens of plain
 * greedy decoding.
 *
 * Every function returns 0 on success or a negative PINFER_E* code unless noted. One call at a
 * time per context.
 */
#ifndef PINFER_H
#define PINFER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PINFER_VERSION_MAJOR 0
#define PINFER_VERSION_MINOR 3
#define PINFER_VERSION_PATCH 0

enum {
    PINFER_OK = 0,
    PINFER_E_IO = -1,       /* the model file cannot be opened or mapped */
    PINFER_E_FORMAT = -2,   /* not a valid .pq file, or a dtype / shape this engine lacks */
    PINFER_E_NOMEM = -3,    /* host or device memory */
    PINFER_E_ARG = -4,      /* invalid argument */
    PINFER_E_CTX_FULL = -5, /* more tokens than max_ctx */
};

typedef struct pinfer_ctx pinfer_ctx;

/* KV-cache storage formats (engine/include/pinfer.h:29-38): fp32 rows, binary16 rows (round
 * to nearest even), or int8 rows with one fp32 scale per row. All three are supported; state
 * blobs record the format and load only into a context of the same format. */
enum {
    PINFER_KV_F32 = 0,
    PINFER_KV_F16 = 1,
    PINFER_KV_I8 = 2,
};

typedef struct {
    int n_threads;   /* host threads (unused by the device path; kept for the ABI) */
    int max_ctx;     /* tokens kept in the KV cache; <= 0 means 4096 */
    int kv_dtype;    /* PINFER_KV_F32, PINFER_KV_F16 or PINFER_KV_I8 */
    float gpu_split; /* kept for the ABI; the whole model runs on the device */
} pinfer_params;

pinfer_params pinfer_default_params(void);

/* Load a .pq model onto device 0 (PINFER_DEVICE selects another). NULL on failure; *err (if
 * not NULL) receives the error code. */
pinfer_ctx *pinfer_load(const char *path, const pinfer_params *params, int *err);
void pinfer_free(pinfer_ctx *ctx);

/* Forget all tokens (KV cache position, recurrent and conv states). */
void pinfer_reset(pinfer_ctx *ctx);

/* Feed n tokens in order; logits (if not NULL) receives n_vocab floats for the LAST token. */
int pinfer_eval(pinfer_ctx *ctx, const int32_t *tokens, int n, float *logits);

/* pinfer_eval, then the last token's logits of ids[0..n_ids) only (equal bit for bit to the
 * full logits at those ids). */
int pinfer_eval_select(pinfer_ctx *ctx, const int32_t *tokens, int n, const int32_t *ids,
                       int n_ids, float *out);

/* ---- speculative greedy decoding with the MTP head ------------------------------------- */
#define PINFER_SPEC_MAX_K 8

typedef struct {
    int k;           /* drafts per verification pass, 0..PINFER_SPEC_MAX_K; 0 = plain */
    int draft_vocab; /* drafts are the argmax over ids [0, draft_vocab); <= 0: full vocabulary */
    int adaptive;    /* 1: each MTP round's width is chosen on the host (the role of
                      * engine/src/spec_adapt.c, by a policy of this engine's own): the width w
                      * (1 = a plain step, else 1 + drafts, at most k + 1) that maximises the
                      * expected tokens per second, from decayed per-draft-position acceptance
                      * counts and the measured seconds of each width's rounds, the stalest
                      * width re-measured every 32 rounds; prompt-lookup rounds are not part
                      * of that model. Speed only: the tokens equal the fixed-k and the plain
                      * greedy output */
    int ngram;       /* prompt-lookup drafts of up to ngram tokens (0..PINFER_SPEC_MAX_K), tried
                      * before the MTP drafts each round (engine/src/spec.c:133-151) */
} pinfer_spec_params;

typedef struct {
    int64_t rounds;
    int64_t drafted;
    int64_t accepted;
    int64_t ngram_rounds;
    int64_t ngram_drafted;
    int64_t ngram_accepted;
} pinfer_spec_stats;

pinfer_spec_params pinfer_default_spec_params(void);
int pinfer_has_mtp(const pinfer_ctx *ctx);

/* Reset, feed the prompt, then greedily generate up to n_max tokens into out (stopping after
 * EOS, included). Returns the count or a negative PINFER_E* code. */
int pinfer_generate_greedy(pinfer_ctx *ctx, const int32_t *prompt, int n_prompt,
                           int32_t *out, int n_max, const pinfer_spec_params *sp,
                           pinfer_spec_stats *stats);

typedef struct {
    const int32_t *stop_ids;
    int n_stop;
    int (*on_token)(int32_t tok, void *user);
    void *user;
} pinfer_gen_opts;

int pinfer_generate_greedy_ex(pinfer_ctx *ctx, const int32_t *prompt, int n_prompt,
                              int32_t *out, int n_max, const pinfer_spec_params *sp,
                              const pinfer_gen_opts *opts, pinfer_spec_stats *stats,
                              int *status);

/* Like _ex without the reset: the prompt is appended to the tokens already in context. */
int pinfer_generate_greedy_cont(pinfer_ctx *ctx, const int32_t *prompt, int n_prompt,
                                int32_t *out, int n_max, const pinfer_spec_params *sp,
                                const pinfer_gen_opts *opts, pinfer_spec_stats *stats,
                                int *status);

/* ---- conversation state (engine/include/pinfer.h:139-175) -------------------------------
 * A snapshot of everything the context keeps for the tokens consumed so far (conv and
 * recurrent states, KV rows, the MTP head's rows), in the reference's blob format (header
 * with the model fingerprint; state format version 2), so blobs move between engines.
 * Restoring it and feeding more tokens gives bit-identical results. */
size_t pinfer_state_size(const pinfer_ctx *ctx);   /* bytes a save needs right now */
/* PINFER_OK, or PINFER_E_ARG when cap < pinfer_state_size(ctx). */
int pinfer_state_save(const pinfer_ctx *ctx, void *buf, size_t cap);
/* Replaces the context's state. PINFER_E_FORMAT: not a state blob of this model file / KV
 * format; PINFER_E_CTX_FULL: more tokens than max_ctx. Drops the checkpoint. */
int pinfer_state_load(pinfer_ctx *ctx, const void *buf, size_t len);

/* In-context checkpoint: one rewind point (a device copy of the conv and recurrent states and
 * the position). pinfer_reset, pinfer_state_load and pinfer_generate_greedy / _ex drop it;
 * pinfer_eval, pinfer_eval_select and pinfer_generate_greedy_cont keep it; its memory stays
 * until pinfer_checkpoint_clear or pinfer_free. */
int pinfer_checkpoint(pinfer_ctx *ctx);   /* PINFER_OK, PINFER_E_ARG (NULL), PINFER_E_NOMEM */
int pinfer_rewind(pinfer_ctx *ctx);       /* PINFER_E_ARG if there is no checkpoint */
void pinfer_checkpoint_clear(pinfer_ctx *ctx);
int pinfer_checkpoint_n_past(const pinfer_ctx *ctx); /* its position, or -1 if none */

/* Benchmark helper (the reference CLI's timing, engine/tools/pinfer_run.c:384-430): reset,
 * prefill (timed), then exactly n_gen tokens with EOS ignored (timed). */
int pinfer_bench_generate(pinfer_ctx *ctx, const int32_t *prompt, int n_prompt, int32_t *out,
                          int n_gen, const pinfer_spec_params *sp, pinfer_spec_stats *stats,
                          double *prefill_s, double *decode_s);

int pinfer_n_vocab(const pinfer_ctx *ctx);
int pinfer_n_past(const pinfer_ctx *ctx);
int pinfer_eos_id(const pinfer_ctx *ctx);
int pinfer_argmax(const float *logits, int n);
const char *pinfer_version(void);

#ifdef __cplusplus
}
#endif
#endif
