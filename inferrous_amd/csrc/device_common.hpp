// device_common.hpp -- gfx950 device helpers shared by the W8A8 kernels.
//
// Exactness contract (restated from the reference, crates/inferrous-qwen3/):
//   bf16_rne:  src/kernels.rs:11-15, bit formula including its wrap-around
//   round_i8:  src/kernels.rs:24-34, clamp then round-half-even, NaN -> 0
//   dequant:   src/kernels.rs:290, bf(RN(RN(f32(acc) * asc) * ws))
// All HIP sources are built with -ffp-contract=off so no multiply is fused
// with a neighbouring add, and f32 division / conversion stay IEEE RN.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w8a8 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr uint32_t kFloorBits = 0x322bcc77u;  // bits of 1e-8f

__device__ __forceinline__ float bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  return __uint_as_float(u);
}

__device__ __forceinline__ int8_t round_i8(float v) {
  if (v != v) return 0;
  v = __builtin_fminf(__builtin_fmaxf(v, -127.0f), 127.0f);
  return (int8_t)(int)__builtin_rintf(v);  // v_rndne_f32: ties to even
}

// round_i8(RN(v / s)) from r = RN(1 / s), for a scale s = RN(m / 127) of a
// maximum m >= |v| (so |v / s| <= 128): the code of quantize
// (src/kernels.rs:441-449) without a division per element.  y = RN(v * r)
// lies within |v / s| * 2^-23 <= 2^-16 of v / s, and RN(v / s) within 2^-18
// of it, so y and RN(v / s) are less than 2^-15 apart: unless y is within
// that distance of a half-integer they round to the same integer (and the
// clamp to +-127 commutes with the rounding, its bounds being integers).
// Those cases, and NaN, take the division itself.  About 2^-11 of uniformly
// spread values do.  Used where a workgroup recomputes a row's codes that
// another kernel would compute once (the folded producers).
__device__ __forceinline__ int8_t quant_code(float v, float s, float r) {
  const float y = v * r;
  const float ry = __builtin_rintf(y);
  if (__builtin_fabsf(y - ry) < 0.5f - 0x1p-12f) return (int8_t)(int)__builtin_fminf(__builtin_fmaxf(ry, -127.0f), 127.0f);
  return round_i8(v / s);
}

// quant_code of N values with one branch per thread: the fast product for
// every value and, when any of them lies within quant_code's margin of a
// rounding boundary (or is NaN), the division for all of them -- the same
// integers as quant_code value by value.
template <int N>
__device__ __forceinline__ void quant_codes(const float (&v)[N], float s, float r, int (&code)[N]) {
  bool slow = false;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float y = v[i] * r;
    const float ry = __builtin_rintf(y);
    slow |= !(__builtin_fabsf(y - ry) < 0.5f - 0x1p-12f);
    code[i] = (int)__builtin_amdgcn_fmed3f(ry, -127.0f, 127.0f);
  }
  if (slow) {
#pragma unroll
    for (int i = 0; i < N; ++i) code[i] = round_i8(v[i] / s);
  }
}

// |x| as ordered bits with NaN mapped to 0 (f32::max ignores NaN,
// src/kernels.rs:133-139); non-negative floats order like unsigned ints.
__device__ __forceinline__ uint32_t abs_bits_no_nan(float x) {
  uint32_t b = __float_as_uint(x) & 0x7fffffffu;
  return b > 0x7f800000u ? 0u : b;
}

__device__ __forceinline__ float dequant(int32_t acc, float asc, float ws) {
  float a = (float)acc;  // v_cvt_f32_i32, round to nearest even
  float t = a * asc;
  return bf16_rne(t * ws);
}

// Four quantized codes round(RN(v / s)) packed little-endian into one word
// (src/kernels.rs:449-451: RN division, then the clamp / ties-even round).
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d, float s) {
  uint32_t q0 = (uint8_t)round_i8(a / s), q1 = (uint8_t)round_i8(b / s);
  uint32_t q2 = (uint8_t)round_i8(c / s), q3 = (uint8_t)round_i8(d / s);
  return q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);
}

// SiLU(g) * u in the reference's operation order (src/kernels.rs:681,
// :2181): bf(RN(RN(g / RN(1 + exp(-g))) * u)).  exp is the ROCm device
// library's expf (accurate to about 1 ulp); the reference uses an
// approximate exp2, so this one value is tolerance-checked, not bit-exact.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float d = 1.0f + expf(-g);
  const float s = g / d;
  return bf16_rne(s * u);
}

__device__ __forceinline__ int dot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

__device__ __forceinline__ int dot16(v4i a, v4i b, int c) {
  c = dot4(a.x, b.x, c);
  c = dot4(a.y, b.y, c);
  c = dot4(a.z, b.z, c);
  c = dot4(a.w, b.w, c);
  return c;
}

// Wave maximum, returned wave-uniform; every lane of the wave must be active.
// Within each 16-lane row DPP quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror and row_mirror leave the row's maximum in every lane (no
// LDS traffic); v_readlane of the four rows and scalar maxima combine them.
// The max is order-free, so any combining pattern gives the same value.
// Against six LDS-permute rounds, measured on MI355X per call in a graph:
// quantize (K = 4096) 2.50 -> 2.20 us, norm_quantize 3.31 -> 3.11 us.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// Maximum over 256 threads (four whole waves, every thread active): the wave
// maxima, then one LDS round through red[4].  The quantizers' row maximum.
// t is the thread's index among the 256; sync() makes the four waves' LDS
// writes visible to all of them (a workgroup barrier when they are the whole
// workgroup).
template <class Sync>
__device__ __forceinline__ uint32_t block_max_256_with(uint32_t m, uint32_t* red, int t, Sync sync) {
  m = wave_max_u32(m);
  if ((t & 63) == 0) red[t >> 6] = m;
  sync();
  return max(max(red[0], red[1]), max(red[2], red[3]));
}

__device__ __forceinline__ uint32_t block_max_256(uint32_t m, uint32_t* red) {
  return block_max_256_with(m, red, (int)threadIdx.x, [] { __syncthreads(); });
}

// RMSNorm scale of one 4096-wide row over 256 threads (four whole waves),
// thread t holding v[i] = x[t + 256 i] (i < 16).  The sum of squares keeps the
// reference's order exactly (src/kernels.rs:509-538, the tree of `norm`
// :354-392): thread t sums RN(x^2) over its coordinates (sequential RN
// adds), then the halving tree p[t] = RN(p[t] + p[t + d]), d = 128, 64, ...,
// 1 -- here the first two levels in one wave from LDS, the rest with
// cross-lane moves with the same pairs (v_permlane32_swap: lanes 0-31
// receive lanes 32-63; ds_swizzle xor 16; DPP row_shl 8/4/2/1 inside each
// 16-lane row; lane 0 ends with the sum, the other lanes' values past each
// level are unused).  inv = 1 / sqrt(mean + 1e-6) is evaluated in binary64
// and rounded once to binary32; the reference uses an approximate rsqrt
// (src/kernels.rs:5-6), so normalised values match it within its tolerance.
// Returns inv to every thread, after the sync that publishes it.  t and
// sync as for block_max_256_with.
template <class Sync>
__device__ __forceinline__ float norm_inv_4096_with(const float (&v)[16], float* part, float* inv, int t,
                                                    Sync sync) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s = s + v[i] * v[i];
  part[t] = s;
  sync();
  if (t < 64) {
    float a = part[t] + part[t + 128];           // d = 128 (t < 64)
    const float b = part[t + 64] + part[t + 192];  // d = 128 (t + 64 < 128)
    a = a + b;                                   // d = 64
    a = a + __int_as_float((int)__builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a),
                                                                  false, false)[1]);
    a = a + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(a), 0x401F));
    a = a + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x108, 0xF, 0xF, false));
    a = a + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x104, 0xF, 0xF, false));
    a = a + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x102, 0xF, 0xF, false));
    a = a + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x101, 0xF, 0xF, false));
    if (t == 0) {
      const float m = a / 4096.0f + 1e-6f;  // RN division, RN add
      *inv = (float)(1.0 / __builtin_sqrt((double)m));
    }
  }
  sync();
  return *inv;
}

__device__ __forceinline__ float norm_inv_4096(const float (&v)[16], float* part, float* inv) {
  return norm_inv_4096_with(v, part, inv, (int)threadIdx.x, [] { __syncthreads(); });
}

// The 64-bit maximum keeps the cross-lane shuffle form.  Its users are the
// fused selection's wave publish and its finalize: measured on MI355X, the
// DPP form above made the 151,936 x 4096 head's fused-selection GEMV slower
// (98.9-99.4 against 93.6-94.6 us per launch), while it made every
// quantizer faster.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, kWave);
    uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, kWave);
    uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  }
  return v;
}

// Greedy-selection key: orderable value in the high word, ~index in the low
// word, so one unsigned max picks the largest value and, among equal values,
// the lowest index (src/kernels.rs:2206-2209).  -0 is folded onto +0 so the
// two tie (src/conformance.rs:685-686).  Any non-finite value yields the
// all-ones key, which no finite value can produce (largest finite high word
// is 0xff7fffff), and which maps to the u32::MAX sentinel.
__device__ __forceinline__ uint64_t select_key(float v, uint32_t index) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7f800000u) == 0x7f800000u) return ~0ull;
  if ((u & 0x7fffffffu) == 0u) u = 0u;
  uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(~index);
}

__device__ __forceinline__ uint32_t key_to_token(uint64_t key) {
  if (key == ~0ull || key == 0ull) return 0xffffffffu;
  return ~(uint32_t)key;
}

// 16-byte loads.  Weights are streamed once per call: the non-temporal hint
// keeps them from displacing the reused activations in L2 / MALL.
__device__ __forceinline__ v4i load_nt16(const int8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}
__device__ __forceinline__ v4i load16(const int8_t* p) {
  return *reinterpret_cast<const v4i*>(p);
}

}  // namespace w8a8
