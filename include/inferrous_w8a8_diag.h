/* inferrous_w8a8_diag.h -- diagnostics of libinferrous_w8a8.so (gfx950).
 *
 * Nothing here has a counterpart in the reference, and nothing on the
 * inference path calls it.  It exists for measurement: `bench.py --timeline`
 * uses it to show where a decode GEMV launch spends its time.  Status codes
 * are those of inferrous_w8a8.h.
 */
#ifndef INFERROUS_W8A8_DIAG_H
#define INFERROUS_W8A8_DIAG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Number of uint64 stamps w8a8_diag_linear_timeline writes for an M = 1
 * projection of n rows and width k: 3 per wave of its launch; 0 when k is
 * neither 4096 nor 12288 (the widths the timed kernel is built for). */
size_t w8a8_diag_linear_timeline_stamps(size_t n, uint32_t k);

/* w8a8_linear at M = 1 on one matrix, run by the same kernel body with the
 * same launch shape, timed: out gets the same values as w8a8_linear, and
 * wave g of the grid writes the device's 100 MHz clock (s_memrealtime) into
 * stamps[3g] at its start, stamps[3g + 1] once all its activation, scale and
 * weight loads have landed, and stamps[3g + 2] once its output store is
 * acknowledged.  The two extra waits make the launch slightly slower than
 * w8a8_linear's.  stamps_len must be at least
 * w8a8_diag_linear_timeline_stamps(n, k) (W8A8_EWORKSPACE otherwise); other
 * checks as w8a8_linear's. */
int w8a8_diag_linear_timeline(void *stream, const int8_t *q, const float *asc,
                              const int8_t *w, const float *ws, size_t n,
                              uint32_t k, void *out, int out_dtype,
                              uint64_t *stamps, size_t stamps_len);

#ifdef __cplusplus
}
#endif

#endif /* INFERROUS_W8A8_DIAG_H */
