/* Seeded synthetic weights and the Q4K_G32 packer (include/pqtool.h). */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "pqtool.h"

static uint64_t mix64(uint64_t z) { /* splitmix64 finaliser */
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* Box-Muller on two 53-bit uniforms drawn from the counter (seed, stream, pair index). */
void pqt_gauss(uint64_t seed, uint64_t stream, uint64_t first, float std, float *out, size_t n) {
    const uint64_t key = mix64(seed * 0x9e3779b97f4a7c15ull + mix64(stream + 0x632be59bd9b4e019ull));
    for (size_t k = 0; k < n; k++) {
        const uint64_t idx = first + k, pair = idx >> 1;
        const uint64_t a = mix64(key ^ (2 * pair)), b = mix64(key ^ (2 * pair + 1));
        const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0, 1] */
        const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
        const double z = (idx & 1) ? r * sin(th) : r * cos(th);
        out[k] = (float)(z * (double)std);
    }
}

/* binary32 -> binary16 bits, round to nearest even (what the reference's __fp16 casts do). */
static uint16_t to_half(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, e = (u >> 23) & 0xffu;
    uint32_t m = u & 0x7fffffu;
    const int ex = (int)e - 112;
    if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u | (m >> 13) : 0));
    if (ex >= 31) return (uint16_t)(sign | 0x7c00u);
    if (ex <= 0) {
        if (ex < -10) return (uint16_t)sign;
        m |= 0x800000u;
        const uint32_t sh = (uint32_t)(14 - ex), rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        uint32_t h = m >> sh;
        if (rem > half || (rem == half && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)ex << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)h;
}

static float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu, u;
    if (e == 0) {
        if (!m) u = sign;
        else {
            int s = 0;
            while (!(m & 0x400u)) { m <<= 1; s++; }
            u = sign | ((uint32_t)(113 - s) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) u = sign | 0x7f800000u | (m << 13);
    else u = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float clamp15(float x) { return x < 0.0f ? 0.0f : x > 15.0f ? 15.0f : x; }

/* 32 six-bit values (index 4k + i) -> 24 bytes: 16 bytes of low nibbles (byte j: values j and
 * j + 16), 8 bytes of high bit pairs (byte j: values j, j + 8, j + 16, j + 24). */
static void pack6(uint8_t *p, const int *v) {
    for (int j = 0; j < 16; j++) p[j] = (uint8_t)((v[j] & 15) | (v[j + 16] & 15) << 4);
    for (int j = 0; j < 8; j++)
        p[16 + j] = (uint8_t)((v[j] >> 4) | (v[j + 8] >> 4) << 2 | (v[j + 16] >> 4) << 4 |
                              (v[j + 24] >> 4) << 6);
}

/* One superblock: the 4 rows x 256 columns at w (row stride cols). Per 32-column group the
 * range [min(lo, 0), hi]; per row D = max group scale / 63 and M = max group offset / 63 in
 * fp16; 6-bit sub-scale ceil(scale / D) (16 levels still cover the group), sub-offset
 * rint(offset / M); codes rint((x + m) / d) in [0, 15]. */
static void pack_superblock(const float *w, int cols, uint8_t *p) {
    int sv[32], mv[32];
    for (int i = 0; i < 4; i++) {
        const float *x0 = w + (size_t)i * cols;
        float gs[8], go[8], smax = 0.0f, omax = 0.0f;
        for (int g = 0; g < 8; g++) {
            const float *x = x0 + 32 * g;
            float lo = x[0], hi = x[0];
            for (int j = 1; j < 32; j++) {
                lo = fminf(lo, x[j]);
                hi = fmaxf(hi, x[j]);
            }
            lo = fminf(lo, 0.0f);
            gs[g] = (hi - lo) / 15.0f;
            go[g] = -lo;
            smax = fmaxf(smax, gs[g]);
            omax = fmaxf(omax, go[g]);
        }
        const uint16_t hd = to_half(smax / 63.0f), hm = to_half(omax / 63.0f);
        memcpy(p + 2 * i, &hd, 2);
        memcpy(p + 8 + 2 * i, &hm, 2);
        const float D = from_half(hd), M = from_half(hm);
        for (int g = 0; g < 8; g++) {
            const int s = D > 0.0f ? (int)fminf(ceilf(gs[g] / D), 63.0f) : 0;
            const int m = M > 0.0f ? (int)lrintf(fminf(go[g] / M, 63.0f)) : 0;
            sv[4 * g + i] = s;
            mv[4 * g + i] = m;
            const float dd = D * (float)s, mm = M * (float)m, inv = dd > 0.0f ? 1.0f / dd : 0.0f;
            const float *x = x0 + 32 * g;
            uint8_t *c = p + 64 + 64 * g + 16 * i;
            for (int j = 0; j < 16; j++) {
                const int lo = (int)lrintf(clamp15((x[j] + mm) * inv));
                const int hi = (int)lrintf(clamp15((x[j + 16] + mm) * inv));
                c[j] = (uint8_t)(lo | hi << 4);
            }
        }
    }
    pack6(p + 16, sv);
    pack6(p + 40, mv);
}

int pqt_quantize_q4k(const float *w, int rows, int cols, uint8_t *out) {
    if (!w || !out || rows <= 0 || cols <= 0 || rows % 4 || cols % 256) return -1;
    const int nsb = cols / 256;
    for (int t = 0; t < rows / 4; t++)
        for (int sb = 0; sb < nsb; sb++)
            pack_superblock(w + (size_t)4 * t * cols + (size_t)256 * sb, cols,
                            out + ((size_t)t * nsb + sb) * 576);
    return 0;
}

typedef struct {
    uint64_t seed, stream;
    int rows, cols, t0, t1;
    float std;
    uint8_t *out;
    int rc;
} gq_job;

static void *gq_run(void *arg) {
    gq_job *j = arg;
    float *w = malloc((size_t)4 * j->cols * sizeof(float));
    if (!w) { j->rc = -1; return NULL; }
    const size_t tile_bytes = (size_t)(j->cols / 256) * 576;
    for (int t = j->t0; t < j->t1; t++) {
        pqt_gauss(j->seed, j->stream, (uint64_t)t * 4 * j->cols, j->std, w, (size_t)4 * j->cols);
        pqt_quantize_q4k(w, 4, j->cols, j->out + (size_t)t * tile_bytes);
    }
    free(w);
    return NULL;
}

int pqt_gauss_q4k(uint64_t seed, uint64_t stream, int rows, int cols, float std, uint8_t *out,
                  int threads) {
    if (!out || rows <= 0 || cols <= 0 || rows % 4 || cols % 256) return -1;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    const int tiles = rows / 4;
    if (threads > tiles) threads = tiles;
    pthread_t th[64];
    gq_job jobs[64];
    for (int k = 0; k < threads; k++) {
        jobs[k] = (gq_job){seed, stream, rows, cols, tiles * k / threads, tiles * (k + 1) / threads,
                           std, out, 0};
        if (k > 0 && pthread_create(&th[k], NULL, gq_run, &jobs[k]) != 0) return -1;
    }
    gq_run(&jobs[0]);
    int rc = jobs[0].rc;
    for (int k = 1; k < threads; k++) {
        pthread_join(th[k], NULL);
        rc |= jobs[k].rc;
    }
    return rc ? -1 : 0;
}
