/*
 * w8a8_oracle.c -- CPU restatement of the reference's W8A8 linear-layer
 * arithmetic (bitemyapp/inferrous, crates/inferrous-qwen3/).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load this library, and only as the checker or
 * as the timed CPU baseline.  The product library never links or calls it.
 *
 * Build flags are part of the contract: -O2 -ffp-contract=off (no FMA
 * contraction: the reference is compiled --no-fmad and every product here is
 * a separate round-to-nearest operation), default round-to-nearest-even FP
 * environment.  See oracle/Makefile.
 *
 * Parity pinning (what checks each function, see tests/test_oracle.py):
 *   orc_bf16_rne      all 2^16 BF16 encodings + random f32 vs numpy/torch RNE
 *   orc_round_i8      the 1,328,443-input set of src/conformance.rs:841-871
 *                     vs f64 clamp + round-half-even (closed form)
 *   orc_quantize_*    fixture KATs (tools/operator_fixtures.py:36-45 recipe,
 *                     torch CPU), zero-row floor, tie row, NaN/inf cases
 *   orc_linear_*      brute-force int64 numpy GEMM, worst-case accumulator
 *                     +-198,193,152, fixture cases of
 *                     tools/operator_fixtures.py:47-55 (torch CPU)
 *   orc_epilogue      torch/numpy f32 RN multiply order + bf16 cast
 *   orc_argmax        src/conformance.rs:684-698 cases + src/model.rs:268-272
 *   orc_synth_*       SplitMix64 published test vectors for orc_mix64's
 *                     finaliser; range/uniformity invariants
 */
#include "w8a8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* src/kernels.rs:11-15: (u + 0x7fff + ((u >> 16) & 1)) & 0xffff0000,
 * wrapping u32 arithmetic. */
float orc_bf16_rne(float x) {
  uint32_t u = f2u(x);
  u = (uint32_t)(u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  return u2f(u);
}

uint16_t orc_bf16_bits(float x) { return (uint16_t)(f2u(orc_bf16_rne(x)) >> 16); }

/* src/kernels.rs:24-34.  Round-half-even written out explicitly so the
 * result does not depend on the FP environment: for |x| <= 127 both
 * floor(x) and x - floor(x) are exact in binary32. */
int8_t orc_round_i8(float x) {
  if (x != x) return 0; /* cvt.rni of NaN gives 0 */
  if (x < -127.0f) x = -127.0f;
  if (x > 127.0f) x = 127.0f;
  float r = floorf(x);
  float d = x - r;
  int i = (int)r;
  if (d > 0.5f || (d == 0.5f && (i & 1))) i += 1;
  return (int8_t)i;
}

void orc_round_many(const float *x, size_t n, int8_t *out) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_round_i8(x[i]);
}

/* Non-negative f32 values order like their bit patterns; NaN (bits above
 * 0x7f800000 after clearing the sign) is skipped, as f32::max skips it
 * (src/kernels.rs:433-438, src/kernels.rs:133-139). */
uint32_t orc_absmax_bits(const float *x, size_t n) {
  uint32_t m = f2u(1e-8f);
  for (size_t j = 0; j < n; ++j) {
    uint32_t b = f2u(x[j]) & 0x7fffffffu;
    if (b > 0x7f800000u) continue;
    if (b > m) m = b;
  }
  return m;
}

static void quant_row_with(const float *x, size_t width, float m, int8_t *q,
                           float *scale) {
  float s = m / 127.0f; /* IEEE binary32 RN division, src/kernels.rs:439 */
  *scale = s;
  for (size_t j = 0; j < width; ++j) q[j] = orc_round_i8(x[j] / s);
}

void orc_quantize_rows(const float *x, size_t rows, size_t width, int8_t *q,
                       float *scales) {
  for (size_t r = 0; r < rows; ++r) {
    const float *row = x + r * width;
    quant_row_with(row, width, u2f(orc_absmax_bits(row, width)),
                   q + r * width, scales + r);
  }
}

void orc_quantize_rows_bf16(const uint16_t *x, size_t rows, size_t width,
                            int8_t *q, float *scales) {
  float buf[4096];
  for (size_t r = 0; r < rows; ++r) {
    /* widen exactly (src/kernels.rs:16-19), then as orc_quantize_rows.
     * Processed in 4096-wide pieces to keep the stack bounded. */
    const uint16_t *row = x + r * width;
    uint32_t mb = f2u(1e-8f);
    for (size_t j = 0; j < width; ++j) {
      uint32_t b = ((uint32_t)row[j] << 16) & 0x7fffffffu;
      if (b > 0x7f800000u) continue;
      if (b > mb) mb = b;
    }
    float s = u2f(mb) / 127.0f;
    scales[r] = s;
    for (size_t j0 = 0; j0 < width; j0 += 4096) {
      size_t len = width - j0 < 4096 ? width - j0 : 4096;
      for (size_t j = 0; j < len; ++j) buf[j] = u2f((uint32_t)row[j0 + j] << 16);
      for (size_t j = 0; j < len; ++j) q[r * width + j0 + j] = orc_round_i8(buf[j] / s);
    }
  }
}

void orc_quantize_rows_with_max(const float *x, size_t rows, size_t width,
                                const uint32_t *maxima, int8_t *q,
                                float *scales) {
  for (size_t r = 0; r < rows; ++r)
    quant_row_with(x + r * width, width, u2f(maxima[r]), q + r * width,
                   scales + r);
}

/* Exact: |acc| <= 12288 * 127^2 = 198,193,152 < 2^31 for admitted widths;
 * accumulate in int32 like the reference (src/kernels.rs:839). */
static int32_t dot_i8(const int8_t *a, const int8_t *b, size_t k) {
  int32_t acc = 0;
  for (size_t j = 0; j < k; ++j) acc += (int32_t)a[j] * (int32_t)b[j];
  return acc;
}

void orc_linear_i32(const int8_t *q, size_t m, const int8_t *w, size_t n,
                    size_t k, int32_t *acc, int nthreads) {
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
  for (long long c = 0; c < (long long)n; ++c)
    for (size_t r = 0; r < m; ++r)
      acc[r * n + (size_t)c] = dot_i8(q + r * k, w + (size_t)c * k, k);
}

void orc_epilogue(const int32_t *acc, const float *asc, size_t m,
                  const float *ws, size_t n, float *out_f32,
                  uint16_t *out_bf16) {
  for (size_t r = 0; r < m; ++r)
    for (size_t c = 0; c < n; ++c) {
      float a = (float)acc[r * n + c]; /* RNE int -> f32 */
      float t = a * asc[r];            /* RN */
      float v = orc_bf16_rne(t * ws[c]);
      if (out_f32) out_f32[r * n + c] = v;
      if (out_bf16) out_bf16[r * n + c] = (uint16_t)(f2u(v) >> 16);
    }
}

void orc_linear(const int8_t *q, const float *asc, size_t m, const int8_t *w,
                const float *ws, size_t n, size_t k, int32_t *acc_out,
                float *out_f32, uint16_t *out_bf16, int nthreads) {
  if (nthreads <= 0) nthreads = 1;
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
  for (long long c = 0; c < (long long)n; ++c) {
    for (size_t r = 0; r < m; ++r) {
      int32_t acc = dot_i8(q + r * k, w + (size_t)c * k, k);
      size_t o = r * n + (size_t)c;
      if (acc_out) acc_out[o] = acc;
      float v = orc_bf16_rne(((float)acc * asc[r]) * ws[c]);
      if (out_f32) out_f32[o] = v;
      if (out_bf16) out_bf16[o] = (uint16_t)(f2u(v) >> 16);
    }
  }
}

void orc_residual(const float *residual, const float *out, size_t n,
                  float *combined) {
  for (size_t i = 0; i < n; ++i) combined[i] = orc_bf16_rne(residual[i] + out[i]);
}

float orc_silu_mul(float g, float u) {
  float d = 1.0f + expf(-g); /* RN add (built with -ffp-contract=off) */
  float s = g / d;           /* RN division */
  return orc_bf16_rne(s * u);
}

uint32_t orc_swiglu(const float *gate, const float *up, size_t n, float *act) {
  for (size_t i = 0; i < n; ++i) act[i] = orc_silu_mul(gate[i], up[i]);
  return orc_absmax_bits(act, n); /* fold(1e-8, max |act|), NaN ignored */
}

/* src/kernels.rs:354-392: 256 partial sums, each a sequential RN sum over
 * the thread's 16 coordinates (stride 256), then the halving tree. */
float orc_norm_sum_sq(const float *x) {
  float p[256];
  for (int t = 0; t < 256; ++t) {
    float s = 0.0f;
    for (int i = 0; i < 16; ++i) {
      const float v = x[t + 256 * i];
      s = s + v * v; /* RN multiply, then RN add (-ffp-contract=off) */
    }
    p[t] = s;
  }
  for (int d = 128; d > 0; d /= 2)
    for (int t = 0; t < d; ++t) p[t] = p[t] + p[t + d];
  return p[0];
}

static float norm_inv(const float *x) {
  const float mean = orc_norm_sum_sq(x) / 4096.0f; /* RN division */
  const float a = mean + 1e-6f;                    /* RN add */
  return (float)(1.0 / sqrt((double)a));
}

void orc_norm_rows(const float *x, const float *gain, size_t rows, float *out) {
  for (size_t r = 0; r < rows; ++r) {
    const float *row = x + r * 4096;
    const float inv = norm_inv(row);
    for (int j = 0; j < 4096; ++j) {
      const float a = row[j] * inv;
      out[r * 4096 + j] = orc_bf16_rne(a * gain[j]);
    }
  }
}

void orc_norm_quantize(const float *x, const float *gain, size_t rows,
                       float *out, int8_t *q, float *scales, uint32_t *maxima) {
  orc_norm_rows(x, gain, rows, out);
  orc_quantize_rows(out, rows, 4096, q, scales);
  for (size_t r = 0; r < rows; ++r) maxima[r] = f2u(1e-8f);
}

size_t orc_bf16_pack(const uint16_t *in, size_t n, uint32_t *words,
                     uint32_t *offsets, uint16_t *exceptions) {
  size_t nexc = 0;
  memset(words, 0, n / 8 * 3 * sizeof(uint32_t));
  for (size_t c = 0; c < n / 256; ++c) {
    const size_t base = nexc;
    offsets[c] = (uint32_t)base;
    for (size_t local = 0; local < 256; ++local) {
      const uint16_t v = in[c * 256 + local];
      const uint32_t e = (v >> 7) & 255u;
      uint32_t code;
      if (e >= 109 && e < 124) {
        code = ((e - 109) << 8) | ((v >> 8) & 128u) | (v & 127u);
      } else {
        code = 0xf00u | (uint32_t)(nexc - base);
        exceptions[nexc++] = v;
      }
      const size_t step = local / 32; /* which of the lane's eight codes */
      const size_t word = c * 96 + local % 32 + (step * 12 / 32) * 32;
      const unsigned shift = (unsigned)(step * 12 % 32);
      words[word] |= code << shift;
      if (shift > 20) words[word + 32] |= code >> (32 - shift);
    }
  }
  if (nexc == 0) exceptions[nexc++] = 0; /* keep the list nonempty */
  return nexc;
}

uint16_t orc_bf16_unpack_at(const uint32_t *words, const uint32_t *offsets,
                            const uint16_t *exceptions, size_t i) {
  const size_t step = i % 256 / 32;
  const size_t word = i / 256 * 96 + i % 32 + (step * 12 / 32) * 32;
  const unsigned shift = (unsigned)(step * 12 % 32);
  uint32_t code = words[word] >> shift;
  if (shift > 20) code |= words[word + 32] << (32 - shift);
  code &= 4095u;
  if (code >> 8 == 15) return exceptions[offsets[i / 256] + (code & 255u)];
  return (uint16_t)(((code & 128u) << 8) | (((code >> 8) + 109u) << 7) | (code & 127u));
}

void orc_head_bf16(const float *x4096, const uint16_t *w, size_t rows, float *out) {
  for (size_t r = 0; r < rows; ++r) {
    float lane[32];
    for (int l = 0; l < 32; ++l) {
      float s = 0.0f;
      for (int j = l; j < 4096; j += 32) {
        const float wv = u2f((uint32_t)w[r * 4096 + j] << 16);
        s = s + x4096[j] * wv;
      }
      lane[l] = s;
    }
    for (int d = 16; d > 0; d /= 2)
      for (int l = 0; l < d; ++l) lane[l] = lane[l] + lane[l + d];
    out[r] = orc_bf16_rne(lane[0]);
  }
}

/* src/kernels.rs:2196-2229: scan with (v > best) || (v == best && i < idx);
 * a sequential ascending scan with strict '>' keeps the lowest index, and
 * IEEE '==' makes -0 and +0 tie (src/model.rs:210-215). */
uint32_t orc_argmax(const float *x, size_t n) {
  if (n == 0) return 0xFFFFFFFFu;
  size_t best = 0;
  for (size_t i = 0; i < n; ++i) {
    if (!isfinite(x[i])) return 0xFFFFFFFFu;
    if (x[i] > x[best]) best = i;
  }
  return (uint32_t)best;
}

uint32_t orc_linear_argmax(const int8_t *q, const float *asc, const int8_t *w,
                           const float *ws, size_t n, size_t k,
                           float *logits_f32, int nthreads) {
  float *logits = logits_f32 ? logits_f32 : (float *)malloc(n * sizeof(float) + 4);
  if (!logits) return 0xFFFFFFFFu;
  orc_linear(q, asc, 1, w, ws, n, k, NULL, logits, NULL, nthreads);
  uint32_t t = orc_argmax(logits, n);
  if (!logits_f32) free(logits);
  return t;
}

/* SplitMix64 output finaliser (Steele, Lea & Flood, "Fast splittable
 * pseudorandom number generators", OOPSLA 2014; constants as in Vigna's
 * public-domain splitmix64.c). */
uint64_t orc_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/* Counter-based generator: a per-(seed, stream) key, then one finaliser per
 * index.  The device generator computes the identical function. */
uint64_t orc_synth_hash(uint64_t seed, uint64_t stream, uint64_t index) {
  uint64_t key = orc_mix64(seed * 0x9E3779B97F4A7C15ULL +
                           stream * 0xD1B54A32D192ED03ULL +
                           0x632BE59BD9B4E019ULL);
  return orc_mix64(key ^ (index * 0x9E3779B97F4A7C15ULL));
}

/* Element i uses 16 bits (i % 4) of hash(i / 4): v = (h16 * 255) >> 16
 * lies in [0, 254]; minus 127 gives the 255 admitted weights [-127, 127]
 * (src/model.rs:143 forbids -128). */
void orc_synth_i8(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                  int8_t *out) {
  /* element-wise, so the parallel split cannot change a value */
#pragma omp parallel for schedule(static) if (n >= (1u << 20))
  for (size_t j = 0; j < n; ++j) {
    uint64_t i = first + j;
    uint64_t h = orc_synth_hash(seed, stream, i >> 2);
    uint32_t h16 = (uint32_t)(h >> (16 * (i & 3))) & 0xffffu;
    out[j] = (int8_t)((int)((h16 * 255u) >> 16) - 127);
  }
}

void orc_synth_f32(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                   float lo, float hi, float *out) {
  float d = hi - lo;
  for (size_t j = 0; j < n; ++j) {
    uint64_t h = orc_synth_hash(seed, stream, first + j);
    float u = (float)(uint32_t)(h >> 40) * 5.9604644775390625e-8f; /* 2^-24 */
    float t = u * d;
    out[j] = lo + t;
  }
}
