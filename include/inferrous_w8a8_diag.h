/* inferrous_w8a8_diag.h -- diagnostics of libinferrous_w8a8.so (gfx950).
 *
 * Nothing here has a counterpart in the reference, and nothing on the
 * inference path calls it.  It exists for measurement and checking:
 * `bench.py --timeline` uses the timed GEMV to show where a decode GEMV
 * launch spends its time, and the CPU tests replay every kernel route's
 * index arithmetic from the launch routes below.  Status codes are those of
 * inferrous_w8a8.h.
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

/* Number of uint64 stamps w8a8_diag_gemm_timeline writes for an (m, n, k)
 * projection given workspace_bytes of split-K workspace: 4 per wave of the
 * gemm_tall launch; 0 when the route is not gemm_tall (M > 256, K % 128 != 0,
 * or a small-M shape the narrow or skinny kernel takes). */
size_t w8a8_diag_gemm_timeline_stamps(size_t m, size_t n, uint32_t k,
                                      size_t workspace_bytes);

/* w8a8_linear_ex with BF16 outputs (out: m x n) on its gemm_tall route, run
 * by the same kernel with the same launch (and, for a split-K route, the same
 * slab epilogue launch after it), timed: out gets the same values as
 * w8a8_linear_ex, and wave w of workgroup b writes the device's 100 MHz clock
 * (s_memrealtime) into stamps[4 (8 b + w) .. + 3]: at its start, once stage
 * 0 of both rings has landed, after its last MFMA (or, for a wave that holds
 * no rows, its last DMA) issue, and once its stores are acknowledged.
 * W8A8_ESHAPE when the route is not gemm_tall; stamps_len at least
 * w8a8_diag_gemm_timeline_stamps(m, n, k, workspace_bytes). */
int w8a8_diag_gemm_timeline(void *stream, const int8_t *q, const float *asc,
                            size_t m, const int8_t *w, const float *ws,
                            size_t n, uint32_t k, void *out, void *workspace,
                            size_t workspace_bytes, uint64_t *stamps,
                            size_t stamps_len);

/* ------------------------------------------------------------ launch routes
 * The kernel launch a call makes, decided on the host and returned as
 * W8A8_DIAG_ROUTE_LEN int32 values, so that host-side checks (the indexing
 * replay in tests/test_indexing.py) can replay each kernel's address
 * arithmetic over exactly the grid the library launches.  Nothing runs on a
 * device; no device is needed.
 *   [0] family: 0 none (m or n is 0), 1 gemv_m1_one, 2 gemv_m1, 3 gemv_mt,
 *       11 gemm_skinny, 12 gemm_tall, 13 gemm_dma, 14 gemm_tiled, 15 gemm_narrow
 *   [1] grid x  [2] grid y  [3] threads per workgroup
 *   [4] BM  [5] BN  [6] WM  [7] WN  [8] SA (gemm_narrow: ring stages)  [9] SB
 *   [10] MA (gemm_tall's M tile)
 *   [11] MT (skinny, narrow: 16-row tiles; gemv_mt: activation rows per pass)
 *   [12] S (skinny, narrow: waves)  [13] U (skinny: unroll; narrow: live
 *        activation DMA loads per stage)  [14] split-K slabs (1: none)
 *   [15] slabs streamed  [16] split-K epilogue columns per thread (4 or 8)
 *   [17] GEMV rows per wave  [18] GEMV K / 1024  [19] GEMV waves per workgroup
 * Unused fields are 0. */
#define W8A8_DIAG_ROUTE_LEN 20

/* The route of w8a8_linear_path (W8A8_PATH_AUTO, _DOT4 or _MFMA) for an
 * (m, n, k) projection with out_dtype, with (residual != 0) or without a
 * residual, and workspace_bytes of split-K workspace (0: none), operands
 * taken as 16-byte aligned.  W8A8_ESHAPE for k not a positive multiple of
 * 16 or m, n above 2^32 - 1; W8A8_EARG for an unknown dtype or path, or a
 * residual with i32 outputs; W8A8_EWORKSPACE when route_len is short. */
int w8a8_diag_linear_route(size_t m, size_t n, uint32_t k, int out_dtype,
                           int residual, int path, size_t workspace_bytes,
                           int32_t *route, size_t route_len);

/* The route of w8a8_linear_argmax's GEMV for an n x k head (the fused
 * selection's finalize launch follows it). */
int w8a8_diag_argmax_route(size_t n, uint32_t k, int32_t *route,
                           size_t route_len);

#ifdef __cplusplus
}
#endif

#endif /* INFERROUS_W8A8_DIAG_H */
