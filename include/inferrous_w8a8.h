/*
 * inferrous_w8a8.h -- C ABI of the MI355X (gfx950) W8A8 linear-layer path.
 *
 * This is the drop-in boundary for the operator API that the reference's
 * Qwen3 forward pass calls (bitemyapp/inferrous, crates/inferrous-qwen3/).
 * There, ops are methods of the `LoadedModule` produced by
 * `#[cuda_module] pub mod device` (src/kernels.rs:322-323) and created by
 * `device::load(&ctx)` (src/gpu.rs:250).  Each entry point below names the
 * reference kernel or runtime primitive it replaces (file:line relative to
 * crates/inferrous-qwen3/).
 *
 * Conventions (mirroring src/gpu.rs and eng safety contract):
 *  - All pointers are device pointers unless the name says host.  The caller
 *    owns every buffer; ops allocate nothing, never synchronise, and run in
 *    stream order on `stream` (a hipStream_t; NULL = the default stream), so
 *    they are capturable into hip graphs.
 *  - Shapes are explicit element counts: m activation rows (tokens), n output
 *    channels, k = width (reduction length).  Weights are [n, k] int8 with k
 *    contiguous (src/model.rs:23-28), activations [m, k], outputs [m, n].
 *  - Every function returns an int status: 0 = ok, negative = invalid
 *    argument detected on the host before any launch (see W8A8_E*), positive
 *    = the hipError_t of a failed HIP call.  Nothing throws across the ABI.
 *  - Launch geometry is chosen by the library; the reference's
 *    LaunchConfig and L2-prefetch hint arguments have no counterpart.
 */
#ifndef INFERROUS_W8A8_H
#define INFERROUS_W8A8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W8A8_ABI_VERSION 1

/* status codes (negative: host-side validation) */
#define W8A8_OK 0
#define W8A8_ENULL (-1)      /* required pointer is NULL                 */
#define W8A8_ESHAPE (-2)     /* inconsistent or unsupported dimensions   */
#define W8A8_EALIGN (-3)     /* pointer alignment below the requirement  */
#define W8A8_EINIT (-4)      /* w8a8_init not called / failed            */
#define W8A8_EWORKSPACE (-5) /* workspace missing or too small           */
#define W8A8_EARG (-6)       /* invalid enum or flag value               */
#define W8A8_ENODEV (-7)     /* no usable gfx950 device                  */

/* output element types for the dequant epilogue */
#define W8A8_OUT_F32 0  /* f32 holding a BF16 value: the reference's buffers
                           (src/kernels.rs:11-15 `bf` returns f32)           */
#define W8A8_OUT_BF16 1 /* BF16 bits (uint16)                                 */
#define W8A8_OUT_I32 2  /* raw exact INT32 accumulators, no epilogue          */

/* kernel family selection for w8a8_linear_path (tests/bench); AUTO is what
 * w8a8_linear uses: the dot4 GEMV at M = 1; at M = 2 the MFMA family where
 * its route is the narrow kernel or the unsplit one-M-tile kernel, the dot4
 * GEMV otherwise; the MFMA family from M = 3 (at M = 3 and 4 the dot4 GEMV
 * when the shape's split-K plan needs a workspace the call did not give) */
#define W8A8_PATH_AUTO 0
#define W8A8_PATH_DOT4 1 /* v_dot4 GEMV, wave per row group           */
#define W8A8_PATH_MFMA 2 /* MFMA GEMM: LDS-staged v_mfma_i32_32x32x32_i8,
                            or 16x16x64_i8 streaming for small M on
                            narrow N                                  */

/* ------------------------------------------------------------------ runtime
 * Replaces cuda_core's CudaContext::new / new_stream / DeviceBuffer /
 * PinnedHostBuffer / synchronize as used at src/gpu.rs:248-250,
 * src/gpu.rs:59-61, src/gpu.rs:101, src/gpu.rs:147-181, src/gpu.rs:876,
 * src/gpu.rs:910. */
int w8a8_abi_version(void);
const char *w8a8_status_string(int status);
/* CudaContext::new(device) + device::load(&ctx) (src/gpu.rs:248-250):
 * selects the device, checks it is gfx950, loads the kernels.  Idempotent. */
int w8a8_init(int device);
int w8a8_device_count(int *count);
/* number of compute units and arch name of the current device */
int w8a8_device_info(int *cu_count, char *arch_name, size_t arch_len);
/* peak engine clock of the current device in kHz, as the driver reports it
 * (for deriving the matrix-core peak: CUs x 4 SIMDs x ops/clk x clock) */
int w8a8_device_clock_khz(int *khz);
/* ctx.new_stream() (src/gpu.rs:249); *stream receives a hipStream_t */
int w8a8_stream_create(void **stream);
int w8a8_stream_destroy(void *stream);
/* stream.synchronize() (src/gpu.rs:910) */
int w8a8_stream_synchronize(void *stream);
/* DeviceBuffer::zeroed (src/gpu.rs:101): zero-filled, 256-byte aligned */
int w8a8_malloc(void **ptr, size_t bytes);
int w8a8_free(void *ptr);
/* PinnedHostBuffer (src/gpu.rs:147-181): page-locked host memory */
int w8a8_host_malloc(void **ptr, size_t bytes);
int w8a8_host_free(void *ptr);
/* DeviceBuffer::from_host / copy_from_host / to_host_vec
 * (src/gpu.rs:59-61, src/gpu.rs:876): stream-ordered copies */
int w8a8_memcpy_htod(void *dst, const void *host_src, size_t bytes, void *stream);
int w8a8_memcpy_dtoh(void *host_dst, const void *src, size_t bytes, void *stream);
int w8a8_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream);
/* zero a device range with a fill kernel (no hipMemsetAsync, graph-safe) */
int w8a8_fill_zero(void *dst, size_t bytes, void *stream);
/* events (timing); replaces the CUPTI/event timing of the reference tools */
int w8a8_event_create(void **event);
int w8a8_event_destroy(void *event);
int w8a8_event_record(void *event, void *stream);
int w8a8_event_synchronize(void *event);
int w8a8_event_elapsed_ms(float *ms, void *start, void *stop);
/* hip graph capture of a stream (src/graph.rs:330-458 equivalent, minimal) */
int w8a8_graph_capture_begin(void *stream);
int w8a8_graph_capture_end(void *stream, void **graph_exec);
int w8a8_graph_launch(void *graph_exec, void *stream);
int w8a8_graph_destroy(void *graph_exec);

/* ------------------------------------------------------------------ ops */

/* `rounding_probe` (src/kernels.rs:325-333): out[i] = round(input[i]) with
 * clamp to [-127,127], round-half-even, NaN -> 0 (src/kernels.rs:24-34). */
int w8a8_rounding_probe(void *stream, const float *input, size_t n, int8_t *out);

/* `quantize` (src/kernels.rs:414-452): per row r of x[rows, width]:
 *   m = max(1e-8, max_j |x_j|) ignoring NaN;  s = RN(m / 127);
 *   q_j = round(RN(x_j / s));  scales[r] = s.
 * If maxima_reset != NULL, also writes bits(1e-8f) to maxima_reset[r], the
 * reset done by the quantize tail of `norm_quantize` (src/kernels.rs:566).
 * x_bf16 variant: BF16 input bits, widened exactly (src/kernels.rs:16-19). */
int w8a8_quantize(void *stream, const float *x, uint32_t width, size_t rows,
                  int8_t *q, float *scales, uint32_t *maxima_reset);
int w8a8_quantize_bf16(void *stream, const uint16_t *x, uint32_t width,
                       size_t rows, int8_t *q, float *scales,
                       uint32_t *maxima_reset);

/* `quantize_with_max` (src/kernels.rs:453-475): as w8a8_quantize with
 * m = from_bits(maxima[r]) published by the producer (src/kernels.rs:133-147). */
int w8a8_quantize_with_max(void *stream, const float *x, uint32_t width,
                           size_t rows, const uint32_t *maxima, int8_t *q,
                           float *scales);

/* `norm_quantize` (src/kernels.rs:476-575; host wrapper src/gpu.rs:340-363,
 * decode call sites src/gpu.rs:552, :713): RMSNorm of each 4096-wide row of
 * x[rows, 4096] with gain[4096], then the row's quantization:
 *   sum = the reference's sum tree of RN(x^2) (src/kernels.rs:354-392);
 *   inv = 1 / sqrt(RN(RN(sum / 4096) + 1e-6));
 *   out_j = bf(RN(RN(x_j * inv) * gain_j))        (f32 holding BF16 values)
 *   (q, scales) = quantize(out);  maxima[r] = bits(1e-8f).
 * inv is 1/sqrt in binary64 rounded to binary32; the reference's approximate
 * rsqrt is not reproduced, so `out` agrees with it within the reference's
 * tolerance, and q / scales equal w8a8_quantize(out) exactly.  width must be
 * 4096 (the reference's fixed hidden width). */
int w8a8_norm_quantize(void *stream, const float *x, const float *gain,
                       size_t rows, uint32_t width, float *out, int8_t *q,
                       float *scales, uint32_t *maxima);

/* The reference's BF16 lm_head, stored losslessly packed.
 *
 * w8a8_bf16_pack (host only; `PackedBf16::new`, src/packing.rs:8-46): codes n
 * BF16 values (n % 256 == 0) into words[n / 8 * 3], offsets[n / 256] and
 * exceptions[*exceptions_len] (at most n, at least 1 entry; capacity
 * exceptions_cap).  A value whose exponent is in [109, 124) takes 12 bits;
 * others escape to the chunk's exception list.  Lossless for every BF16
 * pattern.
 *
 * w8a8_head_packed (`head_packed`, src/kernels.rs:2258-2373; host call site
 * src/gpu.rs:800-810): exceptions_len is the packer's *exceptions_len (it
 * bounds the last chunk's list).  Logits out[r] for rows of 4096 packed values against
 * the last 4096 values of x (x_len >= 4096; that row 16-byte aligned), with
 * the reference's FP32 order:
 * 32 lane sums over j = l, l + 32, ... then the halving tree; out = bf(sum).
 * Bit-identical to the unpacked `head` (src/kernels.rs:2233-2257).
 *
 * w8a8_unpack_bf16 (`unpack_head`, src/kernels.rs:2376-2388): the n values
 * back as BF16 bits. */
int w8a8_bf16_pack(const uint16_t *in, size_t n, uint32_t *words,
                   uint32_t *offsets, uint16_t *exceptions,
                   size_t exceptions_cap, size_t *exceptions_len);
int w8a8_head_packed(void *stream, const float *x, size_t x_len,
                     const uint32_t *words, const uint32_t *offsets,
                     const uint16_t *exceptions, size_t exceptions_len,
                     size_t rows, float *out);
int w8a8_unpack_bf16(void *stream, const uint32_t *words,
                     const uint32_t *offsets, const uint16_t *exceptions,
                     size_t n, uint16_t *out);

/* `linear` (src/kernels.rs:807-845) for any m, and the M>1 GEMMs
 * `linear_prefill` / `linear_splitk` / `linear_tiled` / `linear_large`
 * (src/kernels.rs:846-1289) behind one entry, dispatched as
 * `GpuModel::linear_quantized` does (src/gpu.rs:450-509):
 *   acc[r][c] = sum_k q[r][k] * w[c][k]  (exact INT32)
 *   out[r][c] = bf16(RN(RN(f32(acc) * asc[r]) * ws[c]))
 * out_dtype: W8A8_OUT_F32 / _BF16 / _I32.  Requires k % 16 == 0 and
 * 16-byte aligned q and w. */
int w8a8_linear(void *stream, const int8_t *q, const float *asc, size_t m,
                const int8_t *w, const float *ws, size_t n, uint32_t k,
                void *out, int out_dtype);
/* same with an explicit kernel family (W8A8_PATH_*) */
int w8a8_linear_path(void *stream, const int8_t *q, const float *asc, size_t m,
                     const int8_t *w, const float *ws, size_t n, uint32_t k,
                     void *out, int out_dtype, int path);

/* w8a8_linear / w8a8_linear_path / w8a8_linear_residual in one entry point
 * with an optional caller-owned workspace (no counterpart in the reference,
 * whose M > 1 kernels take precomputed tensor maps instead, src/gpu.rs:465-475).
 * residual == NULL selects plain linear (combined must then be NULL too).
 * With a workspace of at least w8a8_linear_workspace_bytes(m, n, k) bytes
 * (16-byte aligned), shapes that gain from it are computed split-K: i32
 * partial sums in the workspace, added exactly by an epilogue kernel.
 * Results are identical with or without the workspace; a smaller or NULL
 * workspace selects the unsplit kernels.  Calls sharing one workspace must
 * not overlap. */
size_t w8a8_linear_workspace_bytes(size_t m, size_t n, uint32_t k);
/* The same for one route: 0 for W8A8_PATH_DOT4, and for W8A8_PATH_AUTO
 * where AUTO runs the dot4 GEMV whatever the workspace (m = 1, and m = 2
 * unless the MFMA route there is the narrow kernel or the unsplit one-M-tile
 * kernel, which need none); the MFMA family's need otherwise.  Size a per-call workspace with this. */
size_t w8a8_linear_workspace_bytes_path(size_t m, size_t n, uint32_t k, int path);
/* The largest w8a8_linear_workspace_bytes(m, n, k) over m = 1 .. max_m.
 * The need is not monotone in m: 6144 x 4096 needs 25.2 MB at m = 256 and
 * none at m = 512, and 4096 x 12288 needs 16.8 MB at m = 256, 8.4 MB at
 * m = 257 and 16.8 MB at m = 512.  A buffer shared by every batch size up
 * to max_m is sized with this, taken over every projection shape the
 * caller runs. */
size_t w8a8_linear_workspace_bytes_upto(size_t max_m, size_t n, uint32_t k);
int w8a8_linear_ex(void *stream, const int8_t *q, const float *asc, size_t m,
                   const int8_t *w, const float *ws, size_t n, uint32_t k,
                   const float *residual, void *out, void *combined,
                   int out_dtype, int path, void *workspace,
                   size_t workspace_bytes);

/* `linear_residual` (src/kernels.rs:577-618): the linear output plus
 * combined = bf16(RN(residual + out)) (src/kernels.rs:615).  out and
 * combined share out_dtype (F32 or BF16); residual is f32 [m, n]. */
int w8a8_linear_residual(void *stream, const int8_t *q, const float *asc,
                         size_t m, const int8_t *w, const float *ws, size_t n,
                         uint32_t k, const float *residual, void *out,
                         void *combined, int out_dtype);

/* `quantize_with_max` (src/kernels.rs:453-475) feeding `linear_residual`
 * (src/kernels.rs:577-618) or `linear`, the decode chain of
 * GpuModel::linear_residual at K = 12288 (src/gpu.rs:371-406): q / scales
 * receive the quantized activations exactly as w8a8_quantize_with_max
 * writes them, and out / combined exactly as w8a8_linear_residual (or
 * w8a8_linear when residual is NULL) computes them from q / scales.  The two
 * steps run back to back on the stream. */
int w8a8_linear_quantize_with_max(void *stream, const float *x,
                                  const uint32_t *maxima, size_t m, uint32_t k,
                                  int8_t *q, float *scales, const int8_t *w,
                                  const float *ws, size_t n,
                                  const float *residual, void *out,
                                  void *combined, int out_dtype);

/* `linear_pair` (src/kernels.rs:696-735), `linear_triple`
 * (src/kernels.rs:736-806) and the gate/up projections of `linear_swiglu`
 * (src/kernels.rs:619-695): `count` (1..4) sibling projections that share
 * the activations q/asc, in one launch.  w, ws, n, out are host arrays of
 * length count; each projection writes its own out[i] [m, n[i]]. */
int w8a8_linear_grouped(void *stream, const int8_t *q, const float *asc,
                        size_t m, uint32_t k, int count,
                        const int8_t *const *w, const float *const *ws,
                        const size_t *n, void *const *out, int out_dtype);

/* `linear_swiglu` (src/kernels.rs:619-695): gate and up projections of the
 * same activations (each exactly as w8a8_linear) and
 *   act = bf16(RN(RN(gate / RN(1 + exp(-gate))) * up))      (src/kernels.rs:681)
 * gate, up, act are [m, n] in out_dtype (F32 or BF16).  If maxima != NULL,
 * each row r's largest bits(|act|) (NaN -> 0) is folded into maxima[r] with
 * atomicMax (the producer half of the `quantize_with_max` protocol,
 * src/kernels.rs:133-147, :684-694); the caller resets maxima beforehand
 * (w8a8_quantize's maxima_reset writes the 1e-8 floor).  The reference
 * kernel is M = 1 only; larger m runs the two projections and w8a8_swiglu.
 * exp is the device library's expf: act is tolerance-checked against the
 * reference (its exp is an approximate exp2); gate, up and maxima-of-act are
 * exact functions of their inputs. */
int w8a8_linear_swiglu(void *stream, const int8_t *q, const float *asc,
                       size_t m, uint32_t k, const int8_t *w_gate,
                       const float *ws_gate, const int8_t *w_up,
                       const float *ws_up, size_t n, void *gate, void *up,
                       void *act, uint32_t *maxima, int out_dtype);

/* The decode MLP's linear_swiglu (src/gpu.rs:730) followed by the
 * quantize_with_max of its act (src/gpu.rs:381, src/kernels.rs:453-475) in
 * one call: gate, up, act and maxima exactly as w8a8_linear_swiglu, then
 * q_out [m, n] int8 and scales_out [m] exactly as w8a8_quantize_with_max
 * writes them from act and the folded maxima.  maxima is required (the
 * caller resets it beforehand, as for w8a8_linear_swiglu).  At m = 1 it is
 * two launches (the GEMV, then one workgroup that folds the maximum and
 * quantizes the row); the separate calls take three. */
int w8a8_linear_swiglu_quantize(void *stream, const int8_t *q, const float *asc,
                                size_t m, uint32_t k, const int8_t *w_gate,
                                const float *ws_gate, const int8_t *w_up,
                                const float *ws_up, size_t n, void *gate,
                                void *up, void *act, uint32_t *maxima,
                                int8_t *q_out, float *scales_out,
                                int out_dtype);

/* norm_quantize of one 4096-wide f32 row (as w8a8_norm_quantize with
 * rows = 1) followed by linear (residual == NULL) or linear_residual of its
 * codes at M = 1, in one launch.  No counterpart in the reference, which
 * runs the two kernels (src/gpu.rs:552 then the projection at :565-590).
 * Every workgroup of the GEMV recomputes the row's codes and scale with the
 * producer's arithmetic and order; workgroup 0 also writes them.  Results
 * are bit-identical to the two calls:
 *   q[4096] (16-byte aligned), scale[1];
 *   maxima[0] reset to bits(1e-8f) when maxima is not NULL;
 *   out_norm[4096], the normalised row, when out_norm is not NULL;
 *   out[n], and combined[n] with residual[n], as w8a8_linear /
 *   w8a8_linear_residual write them for w[n, 4096], ws[n].
 * n >= 1.  out_dtype is F32 or BF16, or I32 without a residual.  x and gain
 * must not overlap any output. */
int w8a8_norm_quantize_linear(void *stream, const float *x,
                              const float *gain, float *out_norm, int8_t *q,
                              float *scale, uint32_t *maxima,
                              const int8_t *w, const float *ws, size_t n,
                              const float *residual, void *out,
                              void *combined, int out_dtype);

/* norm_quantize of one 4096-wide f32 row followed by the decode SwiGLU
 * projection of its codes (K = 4096), the reference's src/gpu.rs:713 then
 * :730 with w8a8_linear_swiglu_quantize's outputs, in two launches (the
 * GEMV with the norm folded in, then the row tail that folds the act
 * maximum).  No counterpart in the reference.  Bit-identical to
 * w8a8_norm_quantize then w8a8_linear_swiglu (q_out == NULL) or
 * w8a8_linear_swiglu_quantize:
 *   q[4096] (16-byte aligned) and scale[1] of the normalised row, which is
 *   written to out_norm[4096] when it is not NULL;
 *   gate[n], up[n], act[n] (F32 or BF16) for w_gate / w_up [n, 4096];
 *   maxima[0] (required): reset by the norm, then the act maximum folded in;
 *   q_out[n] and scales_out[1] (both or neither): act quantized with it.
 * n >= 1.  x and gain must not overlap any output. */
int w8a8_norm_quantize_linear_swiglu(void *stream, const float *x,
                                     const float *gain, float *out_norm,
                                     int8_t *q, float *scale,
                                     const int8_t *w_gate,
                                     const float *ws_gate,
                                     const int8_t *w_up, const float *ws_up,
                                     size_t n, void *gate, void *up,
                                     void *act, uint32_t *maxima,
                                     int8_t *q_out, float *scales_out,
                                     int out_dtype);

/* The decode MLP block at M = 1 in two launches: norm_quantize of one
 * 4096-wide f32 row, the SwiGLU projection of its codes (K = 4096), then
 * quantize_with_max of act and the down projection (K = 12288) with an
 * optional residual -- the reference's src/gpu.rs:713 (norm_quantize),
 * :724-745 (linear_swiglu) and :775-786 (linear_residual, which runs
 * quantize_with_max at :377-389 before its kernel).  No counterpart in the
 * reference as one call.  The first launch is w8a8_norm_quantize_linear_swiglu's
 * GEMV; the act row tail (maximum fold, quantize_with_max) runs inside the
 * down GEMV, every workgroup recomputing the row's codes.  Bit-identical to
 * w8a8_norm_quantize_linear_swiglu (with q_out / scales_out) followed by
 * w8a8_linear_residual, or w8a8_linear without a residual, on those codes:
 *   q[4096], scale[1], out_norm[4096] (optional), gate / up / act[n_ff] in
 *   act_dtype (F32 or BF16) as w8a8_norm_quantize_linear_swiglu writes them;
 *   maxima[0] (required): reset by the norm, then act's maximum folded in;
 *   q_act[n_ff] (16-byte aligned) and scale_act[1] (both or neither): act's
 *   codes and scale;
 *   out[n] (required) and, with residual[n] (f32), combined[n] =
 *   bf16(RN(residual + out)), in out_dtype (F32 or BF16), for
 *   w_down / ws_down [n, n_ff].
 * n_ff must be 12288; n >= 1.  x and gain must not overlap any output, and
 * act must not overlap maxima, q_act, scale_act, out or combined. */
int w8a8_norm_quantize_mlp(void *stream, const float *x, const float *gain,
                           float *out_norm, int8_t *q, float *scale,
                           const int8_t *w_gate, const float *ws_gate,
                           const int8_t *w_up, const float *ws_up,
                           size_t n_ff, void *gate, void *up, void *act,
                           int act_dtype, uint32_t *maxima, int8_t *q_act,
                           float *scale_act, const int8_t *w_down,
                           const float *ws_down, size_t n,
                           const float *residual, void *out, void *combined,
                           int out_dtype);

/* quantize of one f32 row of width 4096 (as w8a8_quantize with rows = 1)
 * followed by linear or linear_residual of its codes at M = 1, in one
 * launch: the reference's host linear_residual at decode (src/gpu.rs:364-415:
 * quantize at :397, then the kernel at :402-415) as one kernel.  Outputs
 * and rules as for w8a8_norm_quantize_linear (maxima_reset as w8a8_quantize's
 * maxima_reset); width must be 4096. */
int w8a8_quantize_linear(void *stream, const float *x, uint32_t width,
                         int8_t *q, float *scale, uint32_t *maxima_reset,
                         const int8_t *w, const float *ws, size_t n,
                         const float *residual, void *out, void *combined,
                         int out_dtype);

/* `swiglu` (src/kernels.rs:2172-2190): act = as above, elementwise over
 * gate/up [rows, width] in dtype (F32 or BF16); maxima as above, per row
 * (the reference publishes only for its single 12288-wide decode row). */
int w8a8_swiglu(void *stream, const void *gate, const void *up, size_t rows,
                uint32_t width, void *act, uint32_t *maxima, int dtype);

/* Greedy selection (`select_token`, src/kernels.rs:2191-2231): the largest
 * value, lowest index on ties (-0 == +0); empty input or any non-finite
 * value gives 0xFFFFFFFF.  Multi-workgroup: needs a device workspace of at
 * least w8a8_select_workspace_bytes(n) bytes (one 8-byte key per
 * workgroup).  It needs no initialisation: each call writes every key it
 * reads.  Calls that share one workspace must not overlap. */
size_t w8a8_select_workspace_bytes(size_t n);
int w8a8_select_token(void *stream, const float *x, size_t n, uint32_t *token,
                      void *workspace, size_t workspace_bytes);

/* W8A8 lm_head with fused greedy selection: `linear` at m = 1 over n vocab
 * rows followed by `select_token` over the BF16-rounded logits
 * (src/gpu.rs:801-812 composition).  logits may be NULL; otherwise it
 * receives the logits in logits_dtype (F32 or BF16).  Workspace as for
 * w8a8_select_token, sized by w8a8_linear_argmax_workspace_bytes(n). */
size_t w8a8_linear_argmax_workspace_bytes(size_t n);
int w8a8_linear_argmax(void *stream, const int8_t *q, const float *asc,
                       const int8_t *w, const float *ws, size_t n, uint32_t k,
                       uint32_t *token, void *logits, int logits_dtype,
                       void *workspace, size_t workspace_bytes);

/* ------------------------------------------------------------ decode sequence
 * A dependent sequence of M = 1 projections in one launch: the decode
 * step's linear / linear_residual calls (src/kernels.rs:577-618, :807-845,
 * call sites src/gpu.rs:571-790) and, as the last entry, the lm_head GEMV
 * with select_token (src/kernels.rs:2191-2231, src/gpu.rs:800-812).  It
 * replaces the reference's captured decode graph with programmatic edges
 * (src/graph.rs:56-110; griddepcontrol.wait, src/kernels.rs:173-184): entry
 * i + 1 reads its activation row only after every workgroup has finished
 * entry i, while the weights of the entries ahead, which no entry writes,
 * are requested before that barrier.  Outputs equal w8a8_linear /
 * w8a8_linear_residual / w8a8_linear_argmax of each entry bit for bit.
 *
 * Contract: the activation rows (q, asc), weights, scales and residuals are
 * inputs of the call -- nothing in the call writes them -- and the outputs
 * are visible when the call completes (stream order).  The launch holds one
 * workgroup on every CU until it ends, so sequence calls on one GPU must be
 * stream-ordered with each other and with other work that needs CUs
 * meanwhile; the call is not graph-capturable (W8A8_EARG under capture).
 * Every wait inside the launch is bounded by wait_us (0: 100 ms): a wait
 * that runs out marks the device's sequence state aborted, the launch ends,
 * and later sequence launches return at once until
 * w8a8_linear_sequence_reset.  w8a8_linear_sequence_status reads that
 * state (0 = ok, 1 = a wait ran out). */
typedef struct w8a8_seq_entry {
  const int8_t *w;        /* [n, k], 16-byte aligned */
  const float *ws;        /* [n] */
  const int8_t *q;        /* [k] activation codes, 16-byte aligned */
  const float *asc;       /* [1] activation scale */
  void *out;              /* [n] in out_dtype; NULL only for a selecting entry */
  const float *residual;  /* [n] f32, or NULL (then combined is NULL) */
  void *combined;         /* [n] bf16(residual + out) in out_dtype */
  size_t n;               /* 1 .. 64 * 15 * CUs */
  uint32_t k;             /* 4096, 8192 or 12288 */
  int out_dtype;          /* W8A8_OUT_F32 or W8A8_OUT_BF16 */
  int flags;              /* W8A8_SEQ_SELECT on the last entry: greedy token */
} w8a8_seq_entry;
#define W8A8_SEQ_SELECT 1
/* Bytes of the device table for count entries (64 per entry). */
size_t w8a8_linear_sequence_table_bytes(size_t count);
/* Validate entries[0 .. count) on the host and write their device table
 * (16-byte aligned device memory of table_bytes) with a synchronous copy.
 * The first call on a device also allocates its 4 KiB sequence control
 * block (uncached device memory, held until the process ends). */
int w8a8_linear_sequence_prepare(const w8a8_seq_entry *entries, size_t count,
                                 void *table, size_t table_bytes);
/* Selection keys a selecting sequence needs: 8 bytes per CU. */
size_t w8a8_linear_sequence_workspace_bytes(void);
/* Run a prepared table (same count).  token and workspace (8-byte aligned,
 * w8a8_linear_sequence_workspace_bytes) are used when the last entry
 * selects; pass NULL otherwise. */
int w8a8_linear_sequence(void *stream, const void *table, size_t count,
                         uint32_t *token, void *workspace,
                         size_t workspace_bytes, uint32_t wait_us);
/* The current device's sequence state; synchronises the device first. */
int w8a8_linear_sequence_status(uint32_t *status);
/* Clear an aborted state; synchronises the device first. */
int w8a8_linear_sequence_reset(void);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): w8a8_linear_argmax with its selection keys in a fixed device
 * array inside the library instead of a caller workspace.  Same results as
 * w8a8_linear_argmax.  The array holds the keys of at most
 * W8A8_NOALLOC_MAX_ROWS vocabulary rows (512 KiB on each GPU the library
 * runs on, kept until the process ends); larger n returns W8A8_ESHAPE.
 * Nothing is allocated and no state carries between calls (each call writes
 * every key it reads), but every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, or two threads) race and may
 * return a wrong token. */
#define W8A8_NOALLOC_MAX_ROWS 262144
int w8a8_linear_argmax_noalloc(void *stream, const int8_t *q, const float *asc,
                               const int8_t *w, const float *ws, size_t n,
                               uint32_t k, uint32_t *token, void *logits,
                               int logits_dtype);

/* ------------------------------------------------------------------ synthetic
 * Seeded generators for benches and tests (no reference counterpart; the
 * reference loads exported bundles, src/model.rs:46-165).  Pure functions of
 * (seed, stream, index), identical to the host definition used by the
 * checker: element i of an int8 tensor takes 16 bits (i % 4) of
 * hash(seed, stream, i / 4) mapped to [-127, 127]; an f32 tensor element is
 * lo + RN(u * RN(hi - lo)) with u = (hash(seed, stream, i) >> 40) * 2^-24. */
int w8a8_synth_i8(void *stream, int8_t *out, size_t n, uint64_t seed,
                  uint64_t stream_id);
int w8a8_synth_f32(void *stream, float *out, size_t n, uint64_t seed,
                   uint64_t stream_id, float lo, float hi);

#ifdef __cplusplus
}
#endif
#endif /* INFERROUS_W8A8_H */
