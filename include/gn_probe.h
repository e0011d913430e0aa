/* gn_probe.h — measurement helpers exported by libgn_probe.so, a library of its own built next
 * to libgn_bwd.so (they are not part of the backward ABI).  They have no counterpart in the
 * reference: bench.py --ceilings uses them to re-measure the MFMA and HBM ceilings on the box it
 * runs on.  All launches go on `stream`; no allocation. */
#ifndef GN_PROBE_H
#define GN_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* `blocks` x 256 threads; every wave issues iters x 8 v_mfma_f32_32x32x16_bf16 on independent
 * accumulators (32768 FLOP each) and writes one float per thread to out[blocks * 256]. */
int gn_probe_mfma(float* out, int blocks, int iters, void* stream);

/* dst[0 .. bytes) = src[0 .. bytes) with 16-byte loads and stores (bytes read + bytes written),
 * grid-stride: mode 0 four vectors in flight per thread, non-temporal; 1 four, plain; 2 eight,
 * plain.  Mode 3 only reads src (eight vectors in flight, non-temporal) and writes one word
 * per thread to dst (bytes read + 4 per thread written). */
int gn_probe_copy(void* dst, const void* src, size_t bytes, int mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif
