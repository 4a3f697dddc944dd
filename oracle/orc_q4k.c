/* ORACLE — test infrastructure only (see oracle.h). Q4K_G32 format, A8 activations and the
 * exact Q4K x A8 matmul of the reference engine. */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define SB_BYTES 576 /* engine/src/pq_quant.h:34: 64 B scale line + 4 rows x 128 B codes */

size_t orc_q4k_nbytes(int rows, int cols) { /* pq_quant.h:40-43 */
    if (rows <= 0 || cols <= 0 || rows % 4 || cols % 256) return 0;
    return (size_t)(rows / 4) * (size_t)(cols / 256) * SB_BYTES;
}

static float f16_at(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return orc_f16_to_f32(h);
}

/* Value j of a packed 6-bit array (engine/src/kern_act.c:47-50): 16 bytes of low nibbles
 * (byte i: values i and i + 16), then 8 bytes of high bit pairs (byte i: bits 4..5 of values
 * i, i + 8, i + 16, i + 24 at bits 0, 2, 4, 6). */
int orc_get6(const uint8_t *p, int j) {
    const int lo = j < 16 ? p[j] & 15 : p[j - 16] >> 4;
    return lo | ((p[16 + j % 8] >> (2 * (j / 8))) & 3) << 4;
}

/* Dequantized row (engine/src/kern_act.c:53-88, Q4K branch): w = (D * s) * u - (M * m),
 * with the product and the difference rounded separately. */
void orc_q4k_get_row(const uint8_t *W, int rows, int cols, int row, float *dst) {
    (void)rows;
    const int nsb = cols / 256, i = row % 4;
    const uint8_t *p = W + (size_t)(row / 4) * nsb * SB_BYTES;
    for (int sb = 0; sb < nsb; sb++, p += SB_BYTES, dst += 256) {
        const float D = f16_at(p + 2 * i), M = f16_at(p + 8 + 2 * i);
        for (int k = 0; k < 8; k++) {
            const float dd = D * (float)orc_get6(p + 16, k * 4 + i);
            const float mm = M * (float)orc_get6(p + 40, k * 4 + i);
            const uint8_t *q = p + 64 + k * 64 + i * 16;
            for (int j = 0; j < 16; j++) {
                const float a = dd * (float)(q[j] & 15), b = dd * (float)(q[j] >> 4);
                dst[k * 32 + j] = a - mm;
                dst[k * 32 + 16 + j] = b - mm;
            }
        }
    }
}

/* 6-bit packing of 32 values, the inverse of orc_get6 (engine/bench/kbench_util.c:89-96). */
static void put6(uint8_t *p, const int *v) {
    memset(p, 0, 24);
    for (int j = 0; j < 32; j++) {
        p[j % 16] |= (uint8_t)((v[j] & 15) << (j < 16 ? 0 : 4));
        p[16 + j % 8] |= (uint8_t)((v[j] >> 4) << (2 * (j / 8)));
    }
}

static float clampf(float x, float lo, float hi) { return x < lo ? lo : x > hi ? hi : x; }

/* One superblock (4 rows x 256 cols at w, row stride cols) as engine/bench/kbench_util.c:
 * 100-132 packs it: per 32-col group the range [min(mn, 0), mx]; D = max group scale / 63,
 * M = max group offset / 63 (fp16); sub-scale = ceil(dg / D) (so 16 levels still span the
 * group), sub-min = rint(mg / M); codes = rint((x + m) / d) clamped to [0, 15]. */
static void pack_q4k_sb(const float *w, int cols, uint8_t *p) {
    int s6[32], m6[32];
    for (int i = 0; i < 4; i++) {
        float dg[8], mg[8], dmax = 0, mmax = 0;
        for (int g = 0; g < 8; g++) {
            const float *x = w + (size_t)i * cols + g * 32;
            float mn = x[0], mx = x[0];
            for (int j = 1; j < 32; j++) mn = fminf(mn, x[j]), mx = fmaxf(mx, x[j]);
            mn = fminf(mn, 0.0f);
            dg[g] = (mx - mn) / 15.0f, mg[g] = -mn;
            dmax = fmaxf(dmax, dg[g]), mmax = fmaxf(mmax, mg[g]);
        }
        const uint16_t hD = orc_f32_to_f16(dmax / 63.0f), hM = orc_f32_to_f16(mmax / 63.0f);
        memcpy(p + 2 * i, &hD, 2);
        memcpy(p + 8 + 2 * i, &hM, 2);
        const float D = orc_f16_to_f32(hD), M = orc_f16_to_f32(hM);
        for (int g = 0; g < 8; g++) {
            s6[g * 4 + i] = D > 0 ? (int)fminf(ceilf(dg[g] / D), 63) : 0;
            m6[g * 4 + i] = M > 0 ? (int)lrintf(fminf(mg[g] / M, 63)) : 0;
            const float d = D * (float)s6[g * 4 + i], m = M * (float)m6[g * 4 + i];
            const float id = d > 0 ? 1.0f / d : 0.0f;
            const float *x = w + (size_t)i * cols + g * 32;
            uint8_t *q = p + 64 + g * 64 + i * 16;
            for (int j = 0; j < 16; j++) {
                const int a = (int)lrintf(clampf((x[j] + m) * id, 0, 15));
                const int b = (int)lrintf(clampf((x[j + 16] + m) * id, 0, 15));
                q[j] = (uint8_t)(a | b << 4);
            }
        }
    }
    put6(p + 16, s6);
    put6(p + 40, m6);
}

void orc_q4k_quantize(const float *w, int rows, int cols, uint8_t *out) {
    const int nsb = cols / 256;
    for (int t = 0; t < rows / 4; t++)
        for (int sb = 0; sb < nsb; sb++)
            pack_q4k_sb(w + (size_t)4 * t * cols + sb * 256, cols,
                        out + ((size_t)t * nsb + sb) * SB_BYTES);
}

/* Activation quantization per 32-column block (engine/src/kern_act.c:14-42, GPU restatement
 * engine/metal/kernels.metal:9-27): amax = max |x|; id = amax > 0 ? 127 / amax : 0; code =
 * round-half-even(x * id) saturated to int8 (the sum uses the unsaturated value, as the
 * NEON int32 lanes do); d = amax / 127; fsum = d * (float)sum. Layout block-major: element
 * (b, v) at b * n + v, codes [cols/32][n][32]. */
void orc_quant_a8(const float *X, int n, int cols, int8_t *q, float *d, float *fsum) {
    const int nb = cols / 32;
    for (int v = 0; v < n; v++)
        for (int b = 0; b < nb; b++) {
            const float *x = X + (size_t)v * cols + b * 32;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) {
                const float a = fabsf(x[j]);
                if (a > amax) amax = a;
            }
            const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
            const size_t k = (size_t)b * n + v;
            int32_t sum = 0;
            for (int j = 0; j < 32; j++) {
                const int32_t c = (int32_t)rintf(x[j] * id);
                sum += c;
                q[k * 32 + j] = (int8_t)(c > 127 ? 127 : c < -128 ? -128 : c);
            }
            d[k] = amax / 127.0f;
            fsum[k] = d[k] * (float)sum;
        }
}

/* Exact Q4K x A8 product for rows [r0, r1) (engine/src/kern_quant.c:148-245 per vector;
 * the clearest statement is engine/metal/kernels.metal:223-259). Per (row r, vector v):
 * acc = +0; for every block (32 columns) in column order:
 *   dot = sum_j lo_j * x_j + hi_j * x_{j+16}          (int32, exact)
 *   acc = fmaf((float)dot, (D_i * s) * d_v, acc)       (D_i * s exact; * d_v rounds)
 *   acc = fmaf(-(M_i * m), fsum_v, acc)                (M_i * m exact)
 * The result of a vector does not depend on the others (batch == single). */
static void matmul_rows(const uint8_t *W, int rows, int cols, const int8_t *q, const float *d,
                        const float *fs, int n, float *Y, int32_t *dots, int r0, int r1) {
    const int nsb = cols / 256, nb = cols / 32;
    for (int r = r0; r < r1; r++) {
        const int i = r % 4;
        const uint8_t *tile = W + (size_t)(r / 4) * nsb * SB_BYTES;
        for (int v = 0; v < n; v++) {
            float acc = 0.0f;
            for (int sb = 0; sb < nsb; sb++) {
                const uint8_t *p = tile + (size_t)sb * SB_BYTES;
                const float D = f16_at(p + 2 * i), M = f16_at(p + 8 + 2 * i);
                for (int k = 0; k < 8; k++) {
                    const float sc = D * (float)orc_get6(p + 16, 4 * k + i);
                    const float of = M * (float)orc_get6(p + 40, 4 * k + i);
                    const uint8_t *c = p + 64 + 64 * k + 16 * i;
                    const int blk = sb * 8 + k;
                    const int8_t *x = q + ((size_t)blk * n + v) * 32;
                    int32_t dot = 0;
                    for (int j = 0; j < 16; j++)
                        dot += (int32_t)(c[j] & 15) * x[j] + (int32_t)(c[j] >> 4) * x[j + 16];
                    if (dots) dots[((size_t)v * rows + r) * nb + blk] = dot;
                    const size_t a = (size_t)blk * n + v;
                    acc = fmaf((float)dot, sc * d[a], acc);
                    acc = fmaf(-of, fs[a], acc);
                }
            }
            Y[(size_t)v * rows + r] = acc;
        }
    }
}

void orc_q4k_matmul(const uint8_t *W, int rows, int cols, const int8_t *q, const float *d,
                    const float *fsum, int n, float *Y, int32_t *dots) {
    matmul_rows(W, rows, cols, q, d, fsum, n, Y, dots, 0, rows);
}

void orc_q4k_matmul_rows(const uint8_t *W, int rows, int cols, const int8_t *q, const float *d,
                         const float *fsum, int n, float *Y, int r0, int r1) {
    matmul_rows(W, rows, cols, q, d, fsum, n, Y, NULL, r0, r1);
}

typedef struct {
    const uint8_t *W;
    int rows, cols, n, r0, r1;
    const int8_t *q;
    const float *d, *fs;
    float *Y;
} mt_job;

static void *mt_run(void *arg) {
    const mt_job *j = arg;
    matmul_rows(j->W, j->rows, j->cols, j->q, j->d, j->fs, j->n, j->Y, NULL, j->r0, j->r1);
    return NULL;
}

void orc_q4k_matmul_mt(const uint8_t *W, int rows, int cols, const int8_t *q, const float *d,
                       const float *fsum, int n, float *Y, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    const int tiles = rows / 4;
    pthread_t th[256];
    mt_job jobs[256];
    for (int t = 0; t < threads; t++) {
        jobs[t] = (mt_job){W, rows, cols, n, tiles * t / threads * 4, tiles * (t + 1) / threads * 4,
                           q, d, fsum, Y};
        if (t > 0) pthread_create(&th[t], NULL, mt_run, &jobs[t]);
    }
    mt_run(&jobs[0]);
    for (int t = 1; t < threads; t++) pthread_join(th[t], NULL);
}
