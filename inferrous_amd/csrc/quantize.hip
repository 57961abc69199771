// quantize.hip -- dynamic per-token symmetric INT8 activation quantization.
//
// Reference semantics (crates/inferrous-qwen3/):
//   quantize           src/kernels.rs:414-452
//   quantize_with_max  src/kernels.rs:453-475
//   norm_quantize      src/kernels.rs:476-575 (sum tree of `norm` :354-392,
//                      maxima reset at :566)
//   rounding_probe     src/kernels.rs:325-333
//
// MI355X design: one 256-thread workgroup (4 waves) per token row.  Each
// thread loads its share of the row with 16-byte loads and keeps it in
// registers (rows up to 16384 wide), so the row is read from HBM once: a
// wave-level max over ordered |x| bits, a 4-entry LDS exchange, one RN
// division for the scale, then RN divisions + clamp + round-half-even per
// element and packed 4/8-byte stores of the int8 codes.
#include "device_common.hpp"
#include "internal.hpp"

namespace w8a8 {

constexpr int kQThreads = 256;

// f32 rows, width % 4 == 0, 16-byte aligned rows.  NV = float4 per thread
// held in registers (NV * 256 * 4 >= width), or 0: the row is streamed
// twice (the second pass hits L2).  The NV loads are issued unconditionally
// (indices clamped to the row) so they are all in flight at once; a load
// guarded by its own branch would be waited for before the next is issued.
// FULL (width == NV * 1024, the decode widths 4096 and 12288): no index
// clamps and no per-element range branches.  Measured on MI355X in a graph
// of quantize -> GEMV pairs, the checked form cost ~0.2 us per call.
template <int NV, bool FULL = false>
__global__ __launch_bounds__(kQThreads) void quantize_f32_vec(
    const float* __restrict__ x, uint32_t width, int8_t* __restrict__ q,
    float* __restrict__ scales, uint32_t* __restrict__ maxima_reset) {
  __shared__ uint32_t red[4];
  const size_t r = blockIdx.x;
  const uint32_t nvec = width >> 2;
  const v4f* row = reinterpret_cast<const v4f*>(x + r * width);
  uint32_t* qrow = reinterpret_cast<uint32_t*>(q + r * width);
  const uint32_t t = threadIdx.x;
  auto absmax4 = [](v4f a) {
    return max(max(abs_bits_no_nan(a.x), abs_bits_no_nan(a.y)), max(abs_bits_no_nan(a.z), abs_bits_no_nan(a.w)));
  };
  v4f v[NV > 0 ? NV : 1];
  uint32_t m = kFloorBits;
  if (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = row[FULL ? t + i * kQThreads : min(t + i * kQThreads, nvec - 1)];
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (FULL || t + i * kQThreads < nvec) m = max(m, absmax4(v[i]));
  } else {
    for (uint32_t j = t; j < nvec; j += kQThreads) m = max(m, absmax4(row[j]));
  }
  m = block_max_256(m, red);
  const float s = __uint_as_float(m) / 127.0f;
  if (t == 0) {
    scales[r] = s;
    if (maxima_reset) maxima_reset[r] = kFloorBits;
  }
  if (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t j = t + i * kQThreads;
      if (FULL || j < nvec) qrow[j] = pack4(v[i].x, v[i].y, v[i].z, v[i].w, s);
    }
  } else {
    for (uint32_t j = t; j < nvec; j += kQThreads) {
      v4f a = row[j];
      qrow[j] = pack4(a.x, a.y, a.z, a.w, s);
    }
  }
}

__device__ __forceinline__ float widen(uint32_t h) { return __uint_as_float(h << 16); }

// BF16 rows, width % 8 == 0, 16-byte aligned rows: 8 values per 16 bytes;
// NV as above (16-byte vectors per thread).
template <int NV>
__global__ __launch_bounds__(kQThreads) void quantize_bf16_vec(
    const uint16_t* __restrict__ x, uint32_t width, int8_t* __restrict__ q,
    float* __restrict__ scales, uint32_t* __restrict__ maxima_reset) {
  __shared__ uint32_t red[4];
  const size_t r = blockIdx.x;
  const uint32_t nvec = width >> 3;
  const v4i* row = reinterpret_cast<const v4i*>(x + r * width);
  v2i* qrow = reinterpret_cast<v2i*>(q + r * width);
  const uint32_t t = threadIdx.x;

  v4i v[NV > 0 ? NV : 1];
  uint32_t m = kFloorBits;
  auto absmax8 = [](v4i a) {
    uint32_t mm = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t w = (uint32_t)a[e];
      mm = max(mm, max(abs_bits_no_nan(widen(w & 0xffffu)), abs_bits_no_nan(widen(w >> 16))));
    }
    return mm;
  };
  auto quant8 = [](v4i a, float s) {
    v2i o;
    o.x = (int)pack4(widen((uint32_t)a.x & 0xffffu), widen((uint32_t)a.x >> 16),
                     widen((uint32_t)a.y & 0xffffu), widen((uint32_t)a.y >> 16), s);
    o.y = (int)pack4(widen((uint32_t)a.z & 0xffffu), widen((uint32_t)a.z >> 16),
                     widen((uint32_t)a.w & 0xffffu), widen((uint32_t)a.w >> 16), s);
    return o;
  };
  if (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = row[min(t + i * kQThreads, nvec - 1)];
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (t + i * kQThreads < nvec) m = max(m, absmax8(v[i]));
  } else {
    for (uint32_t j = t; j < nvec; j += kQThreads) m = max(m, absmax8(row[j]));
  }
  m = block_max_256(m, red);
  const float s = __uint_as_float(m) / 127.0f;
  if (t == 0) {
    scales[r] = s;
    if (maxima_reset) maxima_reset[r] = kFloorBits;
  }
  if (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t j = t + i * kQThreads;
      if (j < nvec) qrow[j] = quant8(v[i], s);
    }
  } else {
    for (uint32_t j = t; j < nvec; j += kQThreads) qrow[j] = quant8(row[j], s);
  }
}

// Any width / alignment: scalar two-pass fallback (second pass hits L2).
template <bool BF16>
__global__ __launch_bounds__(kQThreads) void quantize_scalar(
    const void* __restrict__ xv, uint32_t width, int8_t* __restrict__ q,
    float* __restrict__ scales, uint32_t* __restrict__ maxima_reset) {
  __shared__ uint32_t red[4];
  const size_t r = blockIdx.x;
  auto load = [&](uint32_t j) -> float {
    if (BF16) return widen(reinterpret_cast<const uint16_t*>(xv)[r * width + j]);
    return reinterpret_cast<const float*>(xv)[r * width + j];
  };
  uint32_t m = kFloorBits;
  for (uint32_t j = threadIdx.x; j < width; j += kQThreads) m = max(m, abs_bits_no_nan(load(j)));
  m = block_max_256(m, red);
  const float s = __uint_as_float(m) / 127.0f;
  if (threadIdx.x == 0) {
    scales[r] = s;
    if (maxima_reset) maxima_reset[r] = kFloorBits;
  }
  for (uint32_t j = threadIdx.x; j < width; j += kQThreads) q[r * width + j] = round_i8(load(j) / s);
}

// quantize_with_max: elementwise, 4 per thread when width % 4 == 0.
__global__ __launch_bounds__(256) void quantize_with_max_vec(
    const float* __restrict__ x, uint32_t width, size_t total_vec,
    const uint32_t* __restrict__ maxima, int8_t* __restrict__ q, float* __restrict__ scales) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total_vec) return;
  const size_t e = i * 4;
  const size_t r = e / width;
  const float s = __uint_as_float(maxima[r]) / 127.0f;
  v4f a = reinterpret_cast<const v4f*>(x)[i];
  reinterpret_cast<uint32_t*>(q)[i] = pack4(a.x, a.y, a.z, a.w, s);
  if (e % width == 0) scales[r] = s;
}

__global__ __launch_bounds__(256) void quantize_with_max_scalar(
    const float* __restrict__ x, uint32_t width, size_t total,
    const uint32_t* __restrict__ maxima, int8_t* __restrict__ q, float* __restrict__ scales) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const size_t r = i / width;
  const float s = __uint_as_float(maxima[r]) / 127.0f;
  q[i] = round_i8(x[i] / s);
  if (i % width == 0) scales[r] = s;
}

__global__ __launch_bounds__(256) void rounding_probe_kernel(const float* __restrict__ in, size_t n,
                                                              int8_t* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = round_i8(in[i]);
}

// ------------------------------------------------------------------ launchers
// RMSNorm of one 4096-wide row per workgroup (norm_inv_4096: the
// reference's sum order), then the row's quantization.  `out` matches the
// reference within its tolerance, while (q, scale) are exactly the
// quantization of `out`.
__global__ __launch_bounds__(256) void norm_quantize_4096(
    const float* __restrict__ x, const float* __restrict__ gain, float* __restrict__ out,
    int8_t* __restrict__ q, float* __restrict__ scales, uint32_t* __restrict__ maxima) {
  __shared__ float part[256];
  __shared__ float inv_shared;
  __shared__ uint32_t red[4];
  const size_t r = blockIdx.x;
  const int t = threadIdx.x;
  const float* row = x + r * 4096;
  float v[16], g[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    v[i] = row[t + 256 * i];
    g[i] = gain[t + 256 * i];
  }
  const float inv = norm_inv_4096(v, part, &inv_shared);
  float* orow = out + r * 4096;
  uint32_t mb = kFloorBits;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float o = bf16_rne((v[i] * inv) * g[i]);
    v[i] = o;
    orow[t + 256 * i] = o;
    mb = max(mb, abs_bits_no_nan(o));
  }
  mb = block_max_256(mb, red);
  const float sc = __uint_as_float(mb) / 127.0f;
  int8_t* qrow = q + r * 4096;
#pragma unroll
  for (int i = 0; i < 16; ++i) qrow[t + 256 * i] = round_i8(v[i] / sc);
  if (t == 0) {
    scales[r] = sc;
    maxima[r] = kFloorBits;
  }
}

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t launch_quantize(hipStream_t st, const void* x, bool bf16, uint32_t width, size_t rows,
                           int8_t* q, float* scales, uint32_t* maxima_reset) {
  if (rows == 0 || width == 0) return hipSuccess;
  dim3 grid((unsigned)rows), block(kQThreads);
  if (!bf16 && width % 4 == 0 && aligned16(x) && ((uintptr_t)q & 3u) == 0) {
    const uint32_t nv = (width / 4 + kQThreads - 1) / kQThreads;  // float4 per thread
    auto k = width == 4096    ? quantize_f32_vec<4, true>
           : width == 12288   ? quantize_f32_vec<12, true>
           : nv <= 1 ? quantize_f32_vec<1> : nv <= 2 ? quantize_f32_vec<2> : nv <= 4 ? quantize_f32_vec<4>
           : nv <= 8 ? quantize_f32_vec<8> : nv <= 12 ? quantize_f32_vec<12>
           : nv <= 16 ? quantize_f32_vec<16> : quantize_f32_vec<0>;
    hipLaunchKernelGGL(k, grid, block, 0, st, (const float*)x, width, q, scales, maxima_reset);
  } else if (bf16 && width % 8 == 0 && aligned16(x) && ((uintptr_t)q & 7u) == 0) {
    const uint32_t nv = (width / 8 + kQThreads - 1) / kQThreads;  // 16-byte vectors per thread
    auto k = nv <= 1 ? quantize_bf16_vec<1> : nv <= 2 ? quantize_bf16_vec<2> : nv <= 4 ? quantize_bf16_vec<4>
           : nv <= 6 ? quantize_bf16_vec<6> : nv <= 8 ? quantize_bf16_vec<8> : quantize_bf16_vec<0>;
    hipLaunchKernelGGL(k, grid, block, 0, st, (const uint16_t*)x, width, q, scales, maxima_reset);
  }
  else if (bf16)
    hipLaunchKernelGGL(quantize_scalar<true>, grid, block, 0, st, x, width, q, scales, maxima_reset);
  else
    hipLaunchKernelGGL(quantize_scalar<false>, grid, block, 0, st, x, width, q, scales,
                       maxima_reset);
  return hipGetLastError();
}

hipError_t launch_quantize_with_max(hipStream_t st, const float* x, uint32_t width, size_t rows,
                                    const uint32_t* maxima, int8_t* q, float* scales) {
  const size_t total = rows * (size_t)width;
  if (total == 0) return hipSuccess;
  if (width % 4 == 0 && aligned16(x) && ((uintptr_t)q & 3u) == 0) {
    const size_t nv = total / 4;
    hipLaunchKernelGGL(quantize_with_max_vec, dim3((unsigned)((nv + 255) / 256)), dim3(256), 0, st,
                       x, width, nv, maxima, q, scales);
  } else {
    hipLaunchKernelGGL(quantize_with_max_scalar, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, st, x, width, total, maxima, q, scales);
  }
  return hipGetLastError();
}

hipError_t launch_norm_quantize(hipStream_t st, const float* x, const float* gain, size_t rows,
                                float* out, int8_t* q, float* scales, uint32_t* maxima) {
  constexpr size_t kChunk = size_t(1) << 30;  // rows per launch (grid x limit)
  for (size_t r0 = 0; r0 < rows; r0 += kChunk) {
    const size_t n = rows - r0 < kChunk ? rows - r0 : kChunk;
    hipLaunchKernelGGL(norm_quantize_4096, dim3((unsigned)n), dim3(256), 0, st, x + r0 * 4096, gain,
                       out + r0 * 4096, q + r0 * 4096, scales + r0, maxima + r0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_rounding_probe(hipStream_t st, const float* in, size_t n, int8_t* out) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rounding_probe_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     in, n, out);
  return hipGetLastError();
}

}  // namespace w8a8
