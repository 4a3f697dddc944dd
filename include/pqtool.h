/* pqtool — .pq format tools in their own library, libpqtool.so (libpinfer.so exports the
 * pinfer_* API only, like engine/pkg/pinfer.map:3-8): a seeded Gaussian weight generator and the Q4K_G32 packer, used to build synthetic random-init models
 * of the Qwen3.5 shapes (the role of the reference's tools/quant.py + tools/convert.py for a
 * checkpoint, and of engine/bench/kbench_util.c's kb_fill_matrix for benchmarks). */
#ifndef PQTOOL_H
#define PQTOOL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* n values ~ N(0, std^2) for (seed, stream): counter-based, so any chunking / thread split
 * of a stream gives the same values (out[i] depends only on seed, stream and first + i). */
void pqt_gauss(uint64_t seed, uint64_t stream, uint64_t first, float std, float *out, size_t n);

/* Pack w [rows][cols] (rows % 4 == 0, cols % 256 == 0) as Q4K_G32 (engine/FORMAT.md:107-136)
 * with the benchmark quantizer of engine/bench/kbench_util.c:100-132. Returns 0 or -1. */
int pqt_quantize_q4k(const float *w, int rows, int cols, uint8_t *out);

/* rows x cols weights ~ N(0, std^2) (stream = `stream`, row-major element order) packed as
 * Q4K_G32 into out (rows/4 * cols/256 * 576 bytes), on `threads` threads. Returns 0 or -1. */
int pqt_gauss_q4k(uint64_t seed, uint64_t stream, int rows, int cols, float std, uint8_t *out,
                  int threads);

#ifdef __cplusplus
}
#endif
#endif
