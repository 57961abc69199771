// synth.hip -- seeded synthetic tensors generated on the device, plus a
// graph-safe zero fill.
//
// The generator is a pure function of (seed, stream, index) so a host
// checker can regenerate any row: key = mix64(seed * G + stream * H + C),
// h(i) = mix64(key ^ (i * G)) with mix64 the SplitMix64 output finaliser
// (Steele, Lea & Flood, OOPSLA 2014).  int8 element i takes 16 bits
// (i % 4) of h(i / 4): ((h16 * 255) >> 16) - 127 in [-127, 127] (the
// reference's admitted weight range, src/model.rs:143).  f32 element i is
// lo + RN(u * RN(hi - lo)) with u = (h(i) >> 40) * 2^-24.
#include "device_common.hpp"
#include "internal.hpp"

namespace w8a8 {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t synth_key(uint64_t seed, uint64_t stream) {
  return mix64(seed * 0x9E3779B97F4A7C15ull + stream * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull);
}

// Each thread writes 16 bytes (4 hashes) per iteration; grid-stride.
__global__ __launch_bounds__(256) void synth_i8_kernel(int8_t* __restrict__ out, size_t n, uint64_t key) {
  const size_t nvec = n / 16;
  for (size_t v = (size_t)blockIdx.x * 256 + threadIdx.x; v < nvec; v += (size_t)gridDim.x * 256) {
    v4i o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t h = mix64(key ^ ((v * 4 + j) * 0x9E3779B97F4A7C15ull));
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t h16 = (uint32_t)(h >> (16 * b)) & 0xffffu;
        word |= (uint32_t)(uint8_t)(int8_t)((int)((h16 * 255u) >> 16) - 127) << (8 * b);
      }
      o[j] = (int)word;
    }
    reinterpret_cast<v4i*>(out)[v] = o;
  }
  // tail bytes (n % 16), done by the first threads of block 0
  if (blockIdx.x == 0) {
    const size_t i = nvec * 16 + threadIdx.x;
    if (i < n) {
      const uint64_t h = mix64(key ^ ((i >> 2) * 0x9E3779B97F4A7C15ull));
      const uint32_t h16 = (uint32_t)(h >> (16 * (i & 3))) & 0xffffu;
      out[i] = (int8_t)((int)((h16 * 255u) >> 16) - 127);
    }
  }
}

__global__ __launch_bounds__(256) void synth_f32_kernel(float* __restrict__ out, size_t n, uint64_t key,
                                                        float lo, float d) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const uint64_t h = mix64(key ^ (i * 0x9E3779B97F4A7C15ull));
    const float u = (float)(uint32_t)(h >> 40) * 5.9604644775390625e-8f;
    const float t = u * d;
    out[i] = lo + t;
  }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(uint8_t* __restrict__ p, size_t bytes) {
  const size_t nvec = bytes / 16;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t v = (size_t)blockIdx.x * 256 + threadIdx.x; v < nvec; v += stride)
    reinterpret_cast<v4i*>(p)[v] = v4i{0, 0, 0, 0};
  if (blockIdx.x == 0 && threadIdx.x < 16) {
    const size_t i = nvec * 16 + threadIdx.x;
    if (i < bytes) p[i] = 0;
  }
}

static unsigned grid_for(size_t items) {
  const size_t b = (items + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

hipError_t launch_synth_i8(hipStream_t st, int8_t* out, size_t n, uint64_t seed, uint64_t stream_id) {
  if (n == 0) return hipSuccess;
  // the host key uses the same wrapping 64-bit arithmetic
  const uint64_t g = 0x9E3779B97F4A7C15ull, h = 0xD1B54A32D192ED03ull, c = 0x632BE59BD9B4E019ull;
  uint64_t z = seed * g + stream_id * h + c;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  const uint64_t key = z ^ (z >> 31);
  hipLaunchKernelGGL(synth_i8_kernel, dim3(grid_for(n / 16 + 1)), dim3(256), 0, st, out, n, key);
  return hipGetLastError();
}

hipError_t launch_synth_f32(hipStream_t st, float* out, size_t n, uint64_t seed, uint64_t stream_id,
                            float lo, float hi) {
  if (n == 0) return hipSuccess;
  const uint64_t g = 0x9E3779B97F4A7C15ull, h = 0xD1B54A32D192ED03ull, c = 0x632BE59BD9B4E019ull;
  uint64_t z = seed * g + stream_id * h + c;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  const uint64_t key = z ^ (z >> 31);
  volatile float vhi = hi, vlo = lo;  // RN(hi - lo) on the host, no contraction
  const float d = vhi - vlo;
  hipLaunchKernelGGL(synth_f32_kernel, dim3(grid_for(n)), dim3(256), 0, st, out, n, key, lo, d);
  return hipGetLastError();
}

hipError_t launch_fill_zero(hipStream_t st, void* dst, size_t bytes) {
  if (bytes == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(bytes / 16 + 1)), dim3(256), 0, st,
                     (uint8_t*)dst, bytes);
  return hipGetLastError();
}

}  // namespace w8a8
