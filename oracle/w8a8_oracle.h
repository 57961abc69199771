/*
 * w8a8_oracle.h -- CPU restatement of the reference's W8A8 linear-layer
 * arithmetic.  TEST INFRASTRUCTURE ONLY: this library is the checker used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The
 * product path (inferrous_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line whose semantics it restates.
 * Paths are relative to crates/inferrous-qwen3/ in bitemyapp/inferrous.
 */
#ifndef W8A8_ORACLE_H
#define W8A8_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/kernels.rs:11-15 `bf`: f32 -> BF16 round-to-nearest-even kept in f32,
 * computed on the bit pattern exactly as the reference does (including its
 * behaviour on NaN/overflow encodings). */
float orc_bf16_rne(float x);
/* Same value as BF16 bits (high half of orc_bf16_rne). */
uint16_t orc_bf16_bits(float x);

/* src/kernels.rs:24-34 `round`: clamp(x,-127,127), round half to even,
 * NaN -> 0, low byte as i8. */
int8_t orc_round_i8(float x);
void orc_round_many(const float *x, size_t n, int8_t *out);

/* Row absmax as the reference's quantizers see it (src/kernels.rs:433-438,
 * f32::max ignores NaN, floor 1e-8), returned as f32 bits.  Equals the
 * producer-published maximum of src/kernels.rs:133-147 seeded with
 * bits(1e-8) (src/kernels.rs:566). */
uint32_t orc_absmax_bits(const float *x, size_t n);

/* src/kernels.rs:414-452 `quantize` per row: s = RN(m/127),
 * q_j = round(RN(x_j/s)).  rows x width, row-major. */
void orc_quantize_rows(const float *x, size_t rows, size_t width, int8_t *q,
                       float *scales);
/* Same with BF16 input bits (values widened exactly to f32 first,
 * src/kernels.rs:16-19 `widen`). */
void orc_quantize_rows_bf16(const uint16_t *x, size_t rows, size_t width,
                            int8_t *q, float *scales);
/* src/kernels.rs:453-475 `quantize_with_max`: m = from_bits(maxima[r]). */
void orc_quantize_rows_with_max(const float *x, size_t rows, size_t width,
                                const uint32_t *maxima, int8_t *q,
                                float *scales);

/* Exact INT32 accumulators acc[r][c] = sum_k q[r][k] * w[c][k]
 * (src/kernels.rs:268-291, src/kernels.rs:807-845; weights [N,K] with K
 * contiguous per src/model.rs:23-28).  nthreads<=0 -> single thread. */
void orc_linear_i32(const int8_t *q, size_t m, const int8_t *w, size_t n,
                    size_t k, int32_t *acc, int nthreads);

/* Epilogue of src/kernels.rs:289-290 / :839-843 / :918-930:
 * out = bf(RN(RN(f32(acc) * asc[r]) * ws[c])).  out_f32 and/or out_bf16
 * may be NULL. */
void orc_epilogue(const int32_t *acc, const float *asc, size_t m,
                  const float *ws, size_t n, float *out_f32,
                  uint16_t *out_bf16);

/* Full linear (i32 GEMM + epilogue). Any output pointer may be NULL. */
void orc_linear(const int8_t *q, const float *asc, size_t m, const int8_t *w,
                const float *ws, size_t n, size_t k, int32_t *acc_out,
                float *out_f32, uint16_t *out_bf16, int nthreads);

/* src/kernels.rs:615 / :2163-2170: combined = bf(RN(residual + out)). */
void orc_residual(const float *residual, const float *out, size_t n,
                  float *combined);

/* SiLU product of src/kernels.rs:681 / :2181:
 * bf(RN(RN(g / RN(1 + exp(-g))) * u)), with exp = C99 expf.  The
 * reference's exp is an approximate exp2 (src/kernels.rs:21-23) that is
 * not reproduced, so results are compared within the reference's own
 * tolerance (src/conformance.rs:663: |a-b| <= 2e-4 + 0.01|b|). */
float orc_silu_mul(float g, float u);
/* src/kernels.rs:2172-2190 `swiglu` over n elements; returns the
 * published maximum fold(1e-8, max |act|) as f32 bits
 * (src/conformance.rs:596-603). */
uint32_t orc_swiglu(const float *gate, const float *up, size_t n, float *act);

/* src/kernels.rs:347-393 `norm` (hidden width 4096) and src/kernels.rs:476-575
 * `norm_quantize`, which keeps norm's BF16 boundary and sum tree:
 *   p[t] = sequential RN sum of RN(x[t + 256 i]^2), i = 0..15, t = 0..255;
 *   halving tree p[t] = RN(p[t] + p[t + d]), d = 128, 64, ..., 1;
 *   inv = rsqrt(RN(RN(p[0] / 4096) + 1e-6));
 *   out_j = bf(RN(RN(x_j * inv) * gain_j));
 *   (q, scale) = quantize(out) (src/kernels.rs:414-452); maxima = bits(1e-8).
 * The reference's rsqrt is NVIDIA's approximate rsqrt (src/kernels.rs:5-6),
 * which is not reproduced: here inv is 1/sqrt evaluated in IEEE binary64 and
 * rounded to binary32, so `out` is compared with the reference within its
 * tolerance, and (q, scale) equal quantize(out) exactly. */
float orc_norm_sum_sq(const float *x); /* the tree sum p[0] of one row */
void orc_norm_rows(const float *x, const float *gain, size_t rows, float *out);
void orc_norm_quantize(const float *x, const float *gain, size_t rows,
                       float *out, int8_t *q, float *scales, uint32_t *maxima);

/* src/packing.rs:8-46 `PackedBf16::new`: lossless 12-bit coding of BF16 values
 * in 256-value chunks.  Exponents 109..123 code as ((e - 109) << 8) | sign << 7
 * | mantissa; anything else escapes to 0xF00 | index into the chunk's
 * exception list.  32 lane streams of eight codes, interleaved in 96 words
 * per chunk.  n % 256 == 0; words[n/8*3], offsets[n/256], exceptions[<= n]
 * (at least one entry).  Returns the number of exceptions written. */
size_t orc_bf16_pack(const uint16_t *in, size_t n, uint32_t *words,
                     uint32_t *offsets, uint16_t *exceptions);
/* src/kernels.rs:295-314 `unpack_code` / `unpack_bf16`: value i. */
uint16_t orc_bf16_unpack_at(const uint32_t *words, const uint32_t *offsets,
                            const uint16_t *exceptions, size_t i);
/* src/kernels.rs:2233-2257 `head` (= `head_packed` :2258-2373 bit for bit):
 * for each row, 32 lane sums, lane l the sequential RN sum of
 * RN(x[j] * w[row][j]) over j = l, l + 32, ..., then the halving tree over the
 * 32 lanes (d = 16 .. 1); out = bf(sum).  x is the last 4096 values of the
 * activation; w is BF16 bits [rows, 4096]. */
void orc_head_bf16(const float *x4096, const uint16_t *w, size_t rows, float *out);

/* src/kernels.rs:2191-2231 `select_token` (equal to src/model.rs:206-218
 * `argmax` when that returns Ok): largest value, lowest index on ties,
 * -0 == +0; empty input or any non-finite value -> 0xFFFFFFFF. */
uint32_t orc_argmax(const float *x, size_t n);

/* lm_head composition (linear at N=vocab, then select_token over the BF16
 * logits). logits_f32 may be NULL. */
uint32_t orc_linear_argmax(const int8_t *q, const float *asc, const int8_t *w,
                           const float *ws, size_t n, size_t k,
                           float *logits_f32, int nthreads);

/* ---- Seeded synthetic generators (shared definition with the device
 * generator in inferrous_amd/csrc/synth.hip).  Pure functions of
 * (seed, stream, index); used to regenerate spot rows on the host. ---- */
uint64_t orc_mix64(uint64_t x);
uint64_t orc_synth_hash(uint64_t seed, uint64_t stream, uint64_t index);
/* int8 uniform over the 255 values [-127,127]. */
void orc_synth_i8(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                  int8_t *out);
/* f32 uniform in [lo, hi): lo + u*(hi-lo), u = (h>>40)*2^-24, two RN ops. */
void orc_synth_f32(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                   float lo, float hi, float *out);

#ifdef __cplusplus
}
#endif
#endif
