/* The adaptive speculation policy (pinfer_spec_params.adaptive; the role of
 * engine/src/spec_adapt.c in the reference's loop, engine/src/spec.c:300-312): before each
 * round it picks the verify width w (1 = a plain step, w = ke + 1 for ke drafts) that
 * maximises the expected tokens per second. It changes which rounds are speculative and how
 * many drafts they verify, never a token.
 *
 * Model. Draft j of a round is reached when drafts 1..j-1 were accepted; p_j estimates the
 * probability that it is then accepted (decayed hit / try counts with a uniform prior, so an
 * unseen position counts as 1/2). A round of width w emits E(w) = 1 + sum_{s<w} prod_{j<=s} p_j
 * tokens on average and takes T(w) seconds, the running average of that width's measured
 * rounds (the whole round: MTP drafts, verify pass, commit). The policy plays argmax E(w)/T(w).
 *
 * Exploration. A width never measured is costed as the cheapest measured one (so a wider
 * round is tried whenever its expected tokens could pay, and a plain step is tried early,
 * since it is costed below everything until measured); every E_AD_PROBE rounds the width with
 * the oldest measurement is played once, so the costs follow the context as it grows. Host
 * code. */
#include <string.h>

#include "engine.h"

#define E_AD_ALPHA 0.25   /* weight of a new round time in its running average */
#define E_AD_FORGET 0.97  /* decay of the acceptance counts per observed draft */
#define E_AD_PROBE 32     /* rounds between re-measurements of the stalest width */

void e_adapt_init(e_adapt *a, int k) {
    memset(a, 0, sizeof *a);
    a->k = k < 0 ? 0 : k > PINFER_SPEC_MAX_K ? PINFER_SPEC_MAX_K : k;
}

static double p_accept(const e_adapt *a, int j) {
    return (a->hits[j] + 1.0) / (a->tries[j] + 2.0);
}

/* expected tokens of a round of width w */
static double expected_tokens(const e_adapt *a, int w) {
    double e = 1.0, reach = 1.0;
    for (int j = 1; j < w; j++) {
        reach *= p_accept(a, j);
        e += reach;
    }
    return e;
}

int e_adapt_width(e_adapt *a) {
    const int wmax = a->k + 1;
    a->rounds++;
    double cheapest = 0.0;
    for (int w = 1; w <= wmax; w++)
        if (a->t[w] > 0 && (cheapest <= 0 || a->t[w] < cheapest)) cheapest = a->t[w];
    if (cheapest <= 0) return wmax; /* nothing measured: the full width first */
    if (a->rounds % E_AD_PROBE == 0) { /* re-measure the stalest width */
        int w_old = 1;
        for (int w = 2; w <= wmax; w++)
            if (a->seen[w] < a->seen[w_old]) w_old = w;
        return w_old;
    }
    int best = wmax;
    double best_rate = -1.0;
    for (int w = 1; w <= wmax; w++) {
        /* an unmeasured plain step is costed below the cheapest round, so it is tried once */
        const double t = a->t[w] > 0 ? a->t[w] : w == 1 ? 0.5 * cheapest : cheapest;
        const double rate = expected_tokens(a, w) / t;
        if (rate > best_rate) {
            best_rate = rate;
            best = w;
        }
    }
    return best;
}

void e_adapt_observe(e_adapt *a, int w, int accepted, double sec) {
    if (w < 1 || w > a->k + 1) return;
    a->t[w] = a->t[w] > 0 ? a->t[w] + E_AD_ALPHA * (sec - a->t[w]) : sec;
    a->seen[w] = a->rounds;
    /* drafts 1..accepted were accepted; draft accepted + 1 (if verified) was rejected */
    for (int j = 1; j < w && j <= accepted + 1; j++) {
        a->hits[j] = E_AD_FORGET * a->hits[j] + (j <= accepted ? 1.0 : 0.0);
        a->tries[j] = E_AD_FORGET * a->tries[j] + 1.0;
    }
}
