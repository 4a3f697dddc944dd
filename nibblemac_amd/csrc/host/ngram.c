/* Prompt-lookup drafts (the role of engine/src/ngram.h:1-47 in the reference's speculative
 * loop, engine/src/spec.c:133-151): when the newest tokens of the history occurred before, the
 * tokens that followed that earlier occurrence are proposed as the next round's draft. The
 * emitted tokens never depend on the drafts, only the round count does.
 *
 * Design: a hash-chain match finder, as in LZ77 compressors. Every history position q >= 1 is
 * the end of the 2-gram (tok[q-1], tok[q]); head[] maps a 2-gram's bucket to the newest indexed
 * position in it and link[q] to the next older position of the same bucket, so one chain walk
 * visits the earlier occurrences of the history's last 2-gram newest first. Each candidate is
 * scored by how far back it agrees with the history's tail (up to E_NG_EXT tokens); the
 * longest agreement wins, the newest among equals. A bucket collision costs a wasted candidate,
 * never a wrong draft, because agreement is counted on the tokens themselves. Positions are
 * indexed lazily at the next lookup, and removing the newest token unlinks the positions that
 * no longer have a successor, so the index always equals the one of a fresh build. Host code. */
#include <stdlib.h>
#include <string.h>

#include "engine.h"

#define NG_CHAIN 64 /* candidates examined per lookup */

static uint32_t bucket_of(const e_ngram *g, int q) {
    const uint64_t key = ((uint64_t)(uint32_t)g->tok[q - 1] << 32) | (uint32_t)g->tok[q];
    return (uint32_t)((key * 0x9E3779B97F4A7C15ull) >> (64 - g->bits));
}

void e_ngram_free(e_ngram *g) {
    free(g->tok);
    free(g->link);
    free(g->head);
    memset(g, 0, sizeof *g);
}

int e_ngram_init(e_ngram *g, int cap) {
    if (g->tok && g->cap >= cap) return 0;
    e_ngram_free(g);
    int bits = 10; /* at least one bucket per position, 2^10 .. 2^22 buckets */
    while (bits < 22 && (1 << bits) < cap) bits++;
    g->tok = malloc((size_t)cap * sizeof(int32_t));
    g->link = malloc((size_t)cap * sizeof(int32_t));
    g->head = malloc(((size_t)1 << bits) * sizeof(int32_t));
    if (!g->tok || !g->link || !g->head) {
        e_ngram_free(g);
        return -1;
    }
    g->cap = cap;
    g->bits = bits;
    e_ngram_reset(g);
    return 0;
}

void e_ngram_reset(e_ngram *g) {
    if (!g->head) return;
    memset(g->head, 0xff, ((size_t)1 << g->bits) * sizeof(int32_t)); /* -1: empty */
    g->n = 0;
    g->indexed = 1; /* position 0 ends no 2-gram */
}

void e_ngram_push(e_ngram *g, const int32_t *t, int m) {
    if (!g->tok) return;
    if (m > g->cap - g->n) m = g->cap - g->n; /* a full history stops growing: drafts get stale */
    if (m <= 0) return;
    memcpy(g->tok + g->n, t, (size_t)m * sizeof(int32_t));
    g->n += m;
}

/* Unlink the newest indexed positions down to `upto` (each is its chain's head). */
static void unindex(e_ngram *g, int upto) {
    if (upto < 1) upto = 1;
    while (g->indexed > upto) {
        const int q = --g->indexed;
        g->head[bucket_of(g, q)] = g->link[q];
    }
}

void e_ngram_pop(e_ngram *g) {
    if (!g->tok || g->n == 0) return;
    g->n--;
    unindex(g, g->n - 1); /* an occurrence must be followed by a token of the history */
}

int e_ngram_draft(e_ngram *g, int32_t *out, int max, int *match) {
    if (match) *match = 0;
    const int n = g->n;
    if (!g->tok || max <= 0 || n < 3) return 0;
    /* index every position that has a successor, except the tail's own end n - 1 */
    for (; g->indexed < n - 1; g->indexed++) {
        const int q = g->indexed;
        const uint32_t b = bucket_of(g, q);
        g->link[q] = g->head[b];
        g->head[b] = q;
    }
    const int32_t *tail = g->tok + n - 1; /* tail[-j] = the history's j-th newest token */
    int best_q = -1, best_len = 0;
    int q = g->head[bucket_of(g, n - 1)];
    for (int step = 0; q >= 1 && step < NG_CHAIN; step++, q = g->link[q]) {
        int len = 0;
        while (len < E_NG_EXT && q - len >= 0 && g->tok[q - len] == tail[-len]) len++;
        if (len > best_len) {
            best_len = len;
            best_q = q;
            if (len == E_NG_EXT) break;
        }
    }
    if (best_len < E_NG_MIN) return 0; /* not even the 2-gram agrees (collisions only) */
    const int avail = n - 1 - best_q, m = avail < max ? avail : max;
    memcpy(out, g->tok + best_q + 1, (size_t)m * sizeof(int32_t));
    if (match) *match = best_len;
    return m;
}
