/* Prompt-lookup drafts: an index of the token history that proposes, as the next round's
 * draft, the tokens that followed the most recent earlier occurrence of the history's newest
 * n-gram (n = E_NG_MIN..E_NG_MAX, the longest match wins). Restates the algorithm of
 * engine/src/ngram.c:1-87 (ngram.h:1-47): one direct-mapped table per n maps a hash of an
 * n-gram to the end position + 1 of its most recent occurrence (0 = empty), newer occurrences
 * overwrite older ones, and every hit is checked against the history, so a collision can only
 * lose a match. Positions are indexed lazily by the next lookup. The hash and the table size
 * are the reference's, so the same history gives the same drafts (the speculative statistics
 * then match; the emitted tokens never depend on the drafts). Host code, no device work. */
#include <stdlib.h>
#include <string.h>

#include "engine.h"

#define NG_TABLES (E_NG_MAX - E_NG_MIN + 1)

/* engine/src/ngram.c:8-12: FNV-1a offset basis seeded with n, a multiplicative mix per token,
 * the top `bits` bits as the bucket */
static uint32_t ng_hash(const int32_t *t, int n, int bits) {
    uint32_t h = 0x811C9DC5u ^ (uint32_t)n;
    for (int i = 0; i < n; i++) h = (h ^ (uint32_t)t[i]) * 0x9E3779B1u;
    return h >> (32 - bits);
}

static int32_t *ng_slot(e_ngram *g, int n, const int32_t *t) {
    return g->tab + ((size_t)(n - E_NG_MIN) << g->bits) + ng_hash(t, n, g->bits);
}

void e_ngram_free(e_ngram *g) {
    free(g->tok);
    free(g->tab);
    memset(g, 0, sizeof *g);
}

int e_ngram_init(e_ngram *g, int cap) {
    if (g->tok && g->cap >= cap) return 0;
    e_ngram_free(g);
    int bits = 10; /* buckets: the first power of two >= 2 cap, in 2^10 .. 2^24 */
    while (bits < 24 && (1 << bits) < 2 * cap) bits++;
    g->tok = malloc((size_t)cap * sizeof(int32_t));
    g->tab = calloc((size_t)NG_TABLES << bits, sizeof(int32_t));
    if (!g->tok || !g->tab) {
        e_ngram_free(g);
        return -1;
    }
    g->cap = cap;
    g->bits = bits;
    return 0;
}

void e_ngram_reset(e_ngram *g) {
    if (!g->tab) return;
    memset(g->tab, 0, ((size_t)NG_TABLES << g->bits) * sizeof(int32_t));
    g->n = g->indexed = 0;
}

void e_ngram_push(e_ngram *g, const int32_t *t, int m) {
    if (!g->tok) return;
    if (m > g->cap - g->n) m = g->cap - g->n; /* past the capacity: drafts only get weaker */
    if (m <= 0) return;
    memcpy(g->tok + g->n, t, (size_t)m * sizeof(int32_t));
    g->n += m;
}

void e_ngram_pop(e_ngram *g) {
    if (g->n > 0) g->n--;
    if (g->indexed > g->n) g->indexed = g->n; /* entries past the end fail the checks */
}

/* every n-gram that ends at a position in [indexed, upto) enters its table */
static void ng_index(e_ngram *g, int upto) {
    for (int q = g->indexed; q < upto; q++)
        for (int n = E_NG_MIN; n <= E_NG_MAX && n <= q + 1; n++)
            *ng_slot(g, n, g->tok + q - n + 1) = q + 1;
    if (upto > g->indexed) g->indexed = upto;
}

int e_ngram_draft(e_ngram *g, int32_t *out, int max, int *match) {
    const int n = g->n;
    if (match) *match = 0;
    if (!g->tok || max <= 0 || n < E_NG_MIN + 1) return 0;
    ng_index(g, n - 1); /* an earlier occurrence ends before the newest token */
    for (int k = E_NG_MAX; k >= E_NG_MIN; k--) {
        if (k > n - 1) continue;
        const int32_t *tail = g->tok + n - k;
        const int q = *ng_slot(g, k, tail) - 1; /* end of the candidate occurrence */
        if (q < k - 1 || q >= n - 1 ||
            memcmp(g->tok + q - k + 1, tail, (size_t)k * sizeof(int32_t)))
            continue;
        const int m = n - 1 - q < max ? n - 1 - q : max;
        memcpy(out, g->tok + q + 1, (size_t)m * sizeof(int32_t));
        if (match) { /* how far back the two occurrences agree (up to E_NG_EXT tokens) */
            int e = k;
            while (e < E_NG_EXT && q - e >= 0 && g->tok[q - e] == g->tok[n - 1 - e]) e++;
            *match = e;
        }
        return m;
    }
    return 0;
}
