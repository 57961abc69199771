// head.hip -- the reference's BF16 lm_head, stored losslessly packed.
//
// Reference semantics (crates/inferrous-qwen3/):
//   PackedBf16::new    src/packing.rs:8-46 (host packer)
//   unpack_code        src/kernels.rs:295-302, unpack_bf16 :304-314
//   head               src/kernels.rs:2233-2257
//   head_packed        src/kernels.rs:2258-2373 (bit-identical to head)
//   unpack_head        src/kernels.rs:2376-2388
//
// Format: BF16 values in chunks of 256.  A value whose exponent lies in
// [109, 124) is coded in 12 bits as ((e - 109) << 8) | sign << 7 | mantissa;
// any other value escapes to 0xF00 | k, the k-th entry of that chunk's
// exception list (offsets[chunk] is where the list starts).  The 256 codes of
// a chunk form 32 lane streams of eight codes, 96 bits each; stream l sits
// in words l, l + 32 and l + 64 of the chunk's 96 words, so a 4096-wide row
// is 16 chunks = 6144 contiguous bytes.
//
// The logit keeps the reference's FP32 order: lane l of a 32-lane group sums
// RN(x[j] * w[j]) for j = l, l + 32, ..., 4064 in that order, then the group
// reduces with the halving tree d = 16, 8, 4, 2, 1; out = bf(sum).
//
// MI355X design: one 32-lane half-wave per row, so lane l of the half-wave is
// the reference's lane l.  Each half-wave issues all 48 of its word loads
// (6 KiB of row, three contiguous 128-byte segments per chunk) and the
// exception-list offsets up front; the activation row is staged in LDS once
// per workgroup and read back with the two halves of a wave hitting the same
// addresses (broadcast).  The kernel is bound by vector-ALU issue, so the
// decode is held to four instructions per value (plus three shifts per
// chunk).  Escapes are rare for trained head weights (|w| in [2^-18, 2^-3)
// codes directly): every code is decoded as if direct, and only in a chunk
// whose exception list is non-empty (in either row of the wave) is each code
// position tested -- one ballot per position -- and the escaped values
// loaded.
#include <algorithm>
#include <vector>

#include "device_common.hpp"
#include "internal.hpp"

namespace w8a8 {

constexpr int kHeadThreads = 256;  // 8 rows per workgroup

__device__ __forceinline__ float unpack_value(uint32_t code, const uint16_t* __restrict__ exceptions,
                                              uint32_t offset) {
  code &= 4095u;
  uint32_t bits;
  if ((code >> 8) == 15u)
    bits = exceptions[offset + (code & 255u)];
  else
    bits = ((code & 128u) << 8) | (((code >> 8) + 109u) << 7) | (code & 127u);
  return __uint_as_float(bits << 16);
}
// The eight codes of one lane stream (96 bits w2:w1:w0, code t at bits
// [12t, 12t + 12)), each taken as direct, straight to f32 bits:
//   B = (exponent nibble + 109) << 23          bit-field extract, shift-add
//   A = sign/mantissa byte copied to bytes 3, 2 byte permute (sign at bit 31,
//                                              mantissa at bits 22..16)
//   f = (A & 0x807F0000) | B                   and-or
// The sign/mantissa bytes of the odd codes are nibble-aligned; three funnel
// shifts of the stream by 4 bits make all four byte-aligned.  The
// instructions are written out so that the compiler keeps this selection
// (it otherwise re-forms the expressions into five or six operations).
__device__ __forceinline__ void decode_chunk(uint32_t w0, uint32_t w1, uint32_t w2, float (&v)[8]) {
  const uint32_t y0 = __builtin_amdgcn_alignbit(w1, w0, 4);  // stream bits 4..35
  const uint32_t y1 = __builtin_amdgcn_alignbit(w2, w1, 4);  // stream bits 36..67
  const uint32_t y2 = w2 >> 4;                               // stream bits 68..95
  const uint32_t smw[8] = {w0, y0, w0, y1, w1, y1, w2, y2};  // word holding code t's sign/mantissa byte
  constexpr uint32_t smb[8] = {0, 1, 3, 0, 2, 3, 1, 2};      // its byte index there
  const uint32_t ew[8] = {w0, w0, w1, w1, w1, w2, w2, w2};   // word holding code t's exponent nibble
  constexpr uint32_t eb[8] = {8, 20, 0, 12, 24, 4, 16, 28};  // its bit offset there
  const uint32_t cexp = 109u << 23, cmask = 0x807F0000u;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t sel = (smb[t] << 24) | (smb[t] << 16) | 0x0C0Cu;
    uint32_t e, B, A, f;
    asm("v_bfe_u32 %0, %1, %2, 4" : "=v"(e) : "v"(ew[t]), "i"(eb[t]));
    asm("v_lshl_add_u32 %0, %1, 23, %2" : "=v"(B) : "v"(e), "s"(cexp));
    asm("v_perm_b32 %0, 0, %1, %2" : "=v"(A) : "v"(smw[t]), "s"(sel));
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(f) : "v"(A), "s"(cmask), "v"(B));
    v[t] = __uint_as_float(f);
  }
}

__global__ __launch_bounds__(kHeadThreads) void head_packed_kernel(
    const float* __restrict__ x4096, const uint32_t* __restrict__ words,
    const uint32_t* __restrict__ offsets, const uint16_t* __restrict__ exceptions, uint32_t n_exceptions,
    uint32_t rows, float* __restrict__ out) {
  __shared__ __attribute__((aligned(1024))) float xs[4096];
  const int lane = threadIdx.x & 31;
  const int wlane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * (kHeadThreads / 32) + (threadIdx.x >> 5);
  const uint32_t r = min(row, rows - 1);  // tail half-waves recompute the last row
  // Loads complete in issue order: first the activation row into LDS (DMA,
  // 1 KiB per wave instruction), then the exception-list offsets, then the
  // 48 words -- so after one wait for the first five the row's words keep
  // streaming while chunk 0 is decoded.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = i * 4 + wave;
    __builtin_amdgcn_global_load_lds((const void*)(x4096 + blk * 256 + wlane * 4),
                                     (void __attribute__((address_space(3)))*)(xs + blk * 256 + wlane * 4), 16,
                                     0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t* wp = words + (size_t)r * 1536 + lane;
  // one unconditional load (the wait counter stays exact): lanes 0..15 take
  // chunk lane's offset, the others the next row's first offset, or the list
  // length after the last row
  const bool past_end = lane >= 16 && r + 1 >= rows;
  const size_t oidx = lane < 16 ? (size_t)r * 16 + lane : (past_end ? (size_t)r * 16 : (size_t)(r + 1) * 16);
  uint32_t my_off = offsets[oidx];
  uint32_t w[16][3];
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    w[g][0] = __builtin_nontemporal_load(wp + g * 96);
    w[g][1] = __builtin_nontemporal_load(wp + g * 96 + 32);
    w[g][2] = __builtin_nontemporal_load(wp + g * 96 + 64);
  }
  __builtin_amdgcn_sched_barrier(0);
  // vmcnt(48): the activation DMA and the offset load have landed, the 48
  // words may still be in flight
  __builtin_amdgcn_s_waitcnt((48 & 15) | ((48 >> 4) << 14) | (7 << 4) | (15 << 8));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  if (past_end) my_off = n_exceptions;
  // chunk g has escapes iff offsets[g + 1] != offsets[g]; the mask ORs the
  // wave's two rows, so every branch below is uniform over the wave
  const uint32_t o_next = (uint32_t)__shfl_down((int)my_off, 1, 32);
  const unsigned long long bal = __ballot(lane < 16 && o_next != my_off);
  const uint32_t wmask = ((uint32_t)bal | (uint32_t)(bal >> 32)) & 0xffffu;
  const float* xl = xs + lane;
  float sum = 0.f;
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    const uint32_t w0 = w[g][0], w1 = w[g][1], w2 = w[g][2];
    float xv[8], v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) xv[t] = xl[g * 256 + 32 * t];
    decode_chunk(w0, w1, w2, v);
    if ((wmask >> g) & 1u) {  // rare: replace the escaped codes' values
      const uint32_t og = (uint32_t)__shfl((int)my_off, g, 32);
      const uint32_t code[8] = {w0, w0 >> 12, (w0 >> 24) | (w1 << 8), w1 >> 4,
                                w1 >> 16, (w1 >> 28) | (w2 << 4), w2 >> 8, w2 >> 20};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t c = code[t] & 4095u;
        const bool esc = c >= 0xf00u;
        if (__ballot(esc) != 0) {
          if (esc) v[t] = __uint_as_float((uint32_t)exceptions[min(og + (c & 255u), n_exceptions - 1)] << 16);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) sum = sum + xv[t] * v[t];
    // keeps this chunk's products here: left alone, the compiler sinks the
    // whole sum chain below the last branch and holds all 128 values live
    asm volatile("" : "+v"(sum));
  }
  // The row's half-wave tree, lane t adding lane t + d for d = 16 .. 1 (the
  // reference's pairs; lane 0 of each half ends with the sum): ds_swizzle
  // xor 16 inside each 32-lane half, then DPP row_shl:8/4/2/1 inside each
  // 16-lane row -- no LDS traffic.
  sum = sum + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(sum), 0x401F));
  sum = sum + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x108, 0xF, 0xF, false));
  sum = sum + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x104, 0xF, 0xF, false));
  sum = sum + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x102, 0xF, 0xF, false));
  sum = sum + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x101, 0xF, 0xF, false));
  if (lane == 0 && row < rows) out[row] = bf16_rne(sum);
}

__global__ __launch_bounds__(256) void unpack_bf16_kernel(const uint32_t* __restrict__ words,
                                                          const uint32_t* __restrict__ offsets,
                                                          const uint16_t* __restrict__ exceptions,
                                                          size_t n, uint16_t* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint32_t step = (uint32_t)(i % 256 / 32);
  const size_t word = i / 256 * 96 + i % 32 + (step * 12 / 32) * 32;
  const uint32_t shift = step * 12 % 32;
  uint32_t code = words[word] >> shift;
  if (shift > 20) code |= words[word + 32] << (32 - shift);
  out[i] = (uint16_t)(__float_as_uint(unpack_value(code, exceptions, offsets[i / 256])) >> 16);
}

hipError_t launch_head_packed(hipStream_t st, const float* x4096, const uint32_t* words,
                              const uint32_t* offsets, const uint16_t* exceptions, uint32_t n_exceptions,
                              uint32_t rows, float* out) {
  const uint32_t per = kHeadThreads / 32;
  hipLaunchKernelGGL(head_packed_kernel, dim3((rows + per - 1) / per), dim3(kHeadThreads), 0, st, x4096,
                     words, offsets, exceptions, n_exceptions, rows, out);
  return hipGetLastError();
}

hipError_t launch_unpack_bf16(hipStream_t st, const uint32_t* words, const uint32_t* offsets,
                              const uint16_t* exceptions, size_t n, uint16_t* out) {
  hipLaunchKernelGGL(unpack_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, words,
                     offsets, exceptions, n, out);
  return hipGetLastError();
}

// Host packer.  Each chunk is coded lane stream by lane stream: the eight
// values l, l + 32, ..., l + 224 of stream l become one 96-bit little-endian
// field whose three 32-bit words land at l, l + 32, l + 64.
size_t pack_bf16_host(const uint16_t* in, size_t n, uint32_t* words, uint32_t* offsets,
                      uint16_t* exceptions) {
  size_t nexc = 0;
  for (size_t c = 0; c < n / 256; ++c) {
    offsets[c] = (uint32_t)nexc;
    const uint16_t* v = in + c * 256;
    uint16_t escaped = 0;  // index within this chunk's list
    uint32_t codes[256];
    for (int i = 0; i < 256; ++i) {
      const uint32_t e = (v[i] >> 7) & 255u;
      if (e >= 109u && e < 124u) {
        codes[i] = ((e - 109u) << 8) | ((v[i] >> 8) & 128u) | (v[i] & 127u);
      } else {
        codes[i] = 0xf00u | escaped++;
        exceptions[nexc++] = v[i];
      }
    }
    uint32_t* cw = words + c * 96;
    for (int l = 0; l < 32; ++l) {
      unsigned __int128 field = 0;
      for (int t = 0; t < 8; ++t) field |= (unsigned __int128)codes[l + 32 * t] << (12 * t);
      cw[l] = (uint32_t)field;
      cw[l + 32] = (uint32_t)(field >> 32);
      cw[l + 64] = (uint32_t)(field >> 64);
    }
  }
  if (nexc == 0) exceptions[nexc++] = 0;  // the device list is never empty
  return nexc;
}

}  // namespace w8a8
