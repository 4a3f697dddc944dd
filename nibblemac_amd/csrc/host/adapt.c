/* The adaptive speculation policy (pinfer_spec_params.adaptive), restating
 * engine/src/spec_adapt.c:1-102 (state in spec.h:49-57). It changes only which rounds are
 * speculative and how long the MTP chains are, never a token.
 *
 *  - chain length: draft s + 1 is chained only while the newest draft's top-1 probability is
 *    at least E_AD_TAU (the device computes that comparison, nmx_top1_gate);
 *  - plain mode: after E_AD_MIN_ROUNDS speculative rounds (2 when a 2-token verify costs at
 *    least 1.5 plain steps), a speculative rate (decayed tokens / seconds) below E_AD_MARGIN of
 *    the plain-step rate switches to plain steps; after E_AD_PROBE0, 2x, .. E_AD_PROBE_MAX plain
 *    steps, E_AD_PROBE_ROUNDS speculative rounds are judged on their own. The plain step's time
 *    is measured when plain steps were taken, else estimated from the verify passes of widths 2
 *    and 3 as 2 tv(2) - tv(3) (at least tv(2) / 2); without either, only a rate below
 *    1 / (cheapest verify pass) counts as slow, since any pass of n >= 2 tokens costs at least
 *    one plain step.
 * Host code; the constants are the reference's, so the same timings give the same decisions. */
#include <string.h>

#include "engine.h"

#define E_AD_ALPHA 0.25      /* weight of a new pass time in its running average */
#define E_AD_DECAY 0.95      /* memory of the speculative rate per round */
#define E_AD_MARGIN 0.95
#define E_AD_MIN_ROUNDS 8
#define E_AD_PROBE_ROUNDS 2
#define E_AD_PROBE0 8
#define E_AD_PROBE_MAX 64

static double running(double old, double x) { return old <= 0 ? x : old + E_AD_ALPHA * (x - old); }

void e_adapt_init(e_adapt *a) {
    memset(a, 0, sizeof *a);
    a->probe_after = E_AD_PROBE0;
}

int e_adapt_plain_now(e_adapt *a) {
    if (!a->plain_mode) return 0;
    if (a->plain_run < a->probe_after) return 1;
    if (!a->probing) { /* a probe begins, judged on its own rounds */
        a->probing = 1;
        a->n_spec = 0;
        a->r_tok = a->r_sec = 0.0;
    }
    return 0;
}

void e_adapt_plain(e_adapt *a, double sec) {
    a->t_plain = running(a->t_plain, sec);
    if (a->plain_mode) a->plain_run++;
}

/* seconds of a plain step: measured, else estimated from verify widths 2 and 3, else 0 */
static double plain_seconds(const e_adapt *a) {
    if (a->t_plain > 0) return a->t_plain;
    if (a->tv[2] > 0 && a->tv[3] > 0) {
        const double t = 2.0 * a->tv[2] - a->tv[3];
        return t > 0.5 * a->tv[2] ? t : 0.5 * a->tv[2];
    }
    return 0.0;
}

void e_adapt_round(e_adapt *a, int n, int emitted, double sec, double t_verify) {
    if (n < 2 || n >= E_AD_W) return;
    a->tv[n] = running(a->tv[n], t_verify);
    a->r_tok = E_AD_DECAY * a->r_tok + emitted;
    a->r_sec = E_AD_DECAY * a->r_sec + sec;
    a->n_spec++;
    double tv_min = 0.0;
    for (int i = 2; i < E_AD_W; i++)
        if (a->tv[i] > 0 && (tv_min <= 0 || a->tv[i] < tv_min)) tv_min = a->tv[i];
    const double ts = plain_seconds(a);
    const int slow = a->r_tok * tv_min < E_AD_MARGIN * a->r_sec ||
                     (ts > 0 && a->r_tok * ts < E_AD_MARGIN * a->r_sec);
    if (a->plain_mode) { /* a probe round */
        if (a->n_spec < E_AD_PROBE_ROUNDS) return;
        a->probing = 0;
        a->plain_mode = slow;
        if (!slow) a->probe_after = E_AD_PROBE0;
        else a->probe_after = 2 * a->probe_after < E_AD_PROBE_MAX ? 2 * a->probe_after : E_AD_PROBE_MAX;
        a->plain_run = 0;
        a->n_spec = 0;
        if (slow) a->r_tok = a->r_sec = 0.0;
    } else if (slow && (a->n_spec >= E_AD_MIN_ROUNDS ||
                        (ts > 0 && a->tv[2] >= 1.5 * ts && a->n_spec >= 2))) {
        a->plain_mode = 1;
        a->plain_run = 0;
        a->probe_after = E_AD_PROBE0;
    }
}
