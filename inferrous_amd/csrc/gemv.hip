// gemv.hip -- memory-bound INT8 GEMV for decode (M = 1) and ragged small M.
//
// Reference semantics (crates/inferrous-qwen3/):
//   linear           src/kernels.rs:807-845 (+ scaled_dot :268-291)
//   linear_pair      src/kernels.rs:696-735
//   linear_triple    src/kernels.rs:736-806
//   linear_swiglu    src/kernels.rs:619-695 (gate/up projections)
//   linear_residual  src/kernels.rs:577-618
//   select_token     src/kernels.rs:2191-2231 (fused onto the lm_head GEMV)
//
// MI355X design.  Weights W[n, k] stream from HBM exactly once, in 16-byte
// non-temporal loads: one wave (64 lanes) owns R consecutive output rows and
// splits k into 1 KiB chunks, lane l reading bytes [l*16, l*16+16) of each
// chunk, so every wave-wide load is one contiguous, fully coalesced 1 KiB
// segment.  All R x chunks loads of a row group are issued before the first
// v_dot4_i32_i8, which keeps 16-24 KiB in flight per wave.  For M = 1 and
// the Qwen3 widths (4096, 12288) the activation row lives in registers
// (loaded once per wave from L2), so HBM traffic is the weights plus a few
// bytes per row.  Partial sums are folded across lanes with a transposing
// butterfly: R rows need log2(R) exchange steps that halve the values per
// lane, then 6 - log2(R) plain steps -- instead of 6 R shuffles.
//
// INT32 sums are exact (|acc| <= 12288 * 127^2 < 2^31), so the lane/chunk
// order is free; the epilogue keeps the reference's two RN multiplies and
// BF16 RNE (device_common.hpp `dequant`).
#include "device_common.hpp"
#include "internal.hpp"

namespace w8a8 {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

enum { EPI_PLAIN = 0, EPI_RESIDUAL = 1, EPI_ARGMAX = 2 };

// Reduce V values per lane (V a power of two <= 64) across the wave.  On
// return v[0] holds the full sum for value index lane / (64 / V) in every
// lane whose low log2(64/V) bits are zero.
template <int V>
__device__ __forceinline__ int fold_reduce(int (&v)[V], int lane) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
#pragma unroll
  for (int width = V, off = 32; width > 1; width >>= 1, off >>= 1) {
    const int half = width >> 1;
    const bool upper = (lane & off) != 0;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      const int send = upper ? v[j] : v[j + half];
      const int keep = upper ? v[j + half] : v[j];
      v[j] = keep + __shfl_xor(send, off, kWave);
    }
  }
#pragma unroll
  for (int off = 32 / V; off >= 1; off >>= 1) v[0] += __shfl_xor(v[0], off, kWave);
  return v[0];
}

__device__ __forceinline__ void store_out(void* out, size_t idx, int dtype, int32_t acc, float value) {
  if (dtype == W8A8_OUT_F32)
    reinterpret_cast<float*>(out)[idx] = value;
  else if (dtype == W8A8_OUT_BF16)
    reinterpret_cast<uint16_t*>(out)[idx] = (uint16_t)(__float_as_uint(value) >> 16);
  else
    reinterpret_cast<int32_t*>(out)[idx] = acc;
}

// Which sibling matrix owns row group g (wave-uniform).
__device__ __forceinline__ int owner(const GemvArgs& a, uint32_t g) {
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i)
    if (i < a.count && g >= a.gbegin[i]) mi = i;
  return mi;
}

// Last-workgroup reduction of per-workgroup selection keys.  `key` is this
// thread's best key (0 = none).  Every thread of every workgroup must call it.
__device__ __forceinline__ void select_finish(uint64_t key, uint64_t* partials, uint32_t* counter,
                                              uint32_t* token) {
  __shared__ uint64_t wbest[kGemvWaves];
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  key = wave_max_u64(key);
  if (lane == 0) wbest[wave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = wbest[0];
#pragma unroll
    for (int i = 1; i < kGemvWaves; ++i) b = wbest[i] > b ? wbest[i] : b;
    __hip_atomic_store(&partials[blockIdx.x], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __threadfence();
    const uint32_t prev = atomicAdd(counter, 1u);
    last = (prev == gridDim.x - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  uint64_t b = 0;
  for (uint32_t i = threadIdx.x; i < gridDim.x; i += kGemvThreads) {
    const uint64_t p = __hip_atomic_load(&partials[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    b = p > b ? p : b;
  }
  b = wave_max_u64(b);
  if (lane == 0) wbest[wave] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t f = wbest[0];
#pragma unroll
    for (int i = 1; i < kGemvWaves; ++i) f = wbest[i] > f ? wbest[i] : f;
    *token = key_to_token(f);
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// M = 1, k = KC * 1024 known at compile time: activations held in registers.
template <int R, int KC, int EPI>
__global__ __launch_bounds__(kGemvThreads) void gemv_m1(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t g = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  const bool live = g < a.gbegin[a.count];
  const int mi = live ? owner(a, g) : 0;
  const uint32_t n = a.n[mi];
  const uint32_t row0 = live ? (g - a.gbegin[mi]) * R : 0;
  constexpr uint32_t K = KC * 1024;

  int acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0;
  if (live) {
    const int8_t* __restrict__ W = a.w[mi];
    v4i x[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) x[c] = load16(a.q + c * 1024 + lane * 16);
    v4i wv[R][KC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t row = min(row0 + r, n - 1);  // tail rows recompute the last row
      const int8_t* p = W + (size_t)row * K + lane * 16;
#pragma unroll
      for (int c = 0; c < KC; ++c) wv[r][c] = load_nt16(p + c * 1024);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int c = 0; c < KC; ++c) acc[r] = dot16(x[c], wv[r][c], acc[r]);
  }
  const int total = fold_reduce<R>(acc, lane);
  constexpr int kSpan = 64 / R;
  const uint32_t row = row0 + lane / kSpan;
  const bool writer = live && (lane % kSpan) == 0 && row < n;
  float value = 0.f;
  if (writer) {
    value = dequant(total, a.asc[0], a.ws[mi][row]);
    if (a.out[mi]) store_out(a.out[mi], row, a.out_dtype, total, value);
    if (EPI == EPI_RESIDUAL) {
      const float comb = bf16_rne(a.residual[row] + value);
      store_out(a.combined, row, a.out_dtype, total, comb);
    }
  }
  if (EPI == EPI_ARGMAX)
    select_finish(writer ? select_key(value, row) : 0ull, a.partials, a.counter, a.token);
}

// Any m (blockIdx.y selects MT activation rows), any k % 16 == 0.
template <int R, int MT, int U, int EPI>
__global__ __launch_bounds__(kGemvThreads) void gemv_mt(GemvArgs a) {
  constexpr int V = R * MT;
  const int lane = threadIdx.x & 63;
  const uint32_t g = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  const bool live = g < a.gbegin[a.count];
  const int mi = live ? owner(a, g) : 0;
  const uint32_t n = a.n[mi];
  const uint32_t row0 = live ? (g - a.gbegin[mi]) * R : 0;
  const uint32_t m0 = blockIdx.y * MT;
  const uint32_t K = a.k;

  int acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0;
  if (live) {
    const int8_t* __restrict__ W = a.w[mi];
    size_t wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = (size_t)min(row0 + r, n - 1) * K;
    const int8_t* xrow[MT];
    bool xok[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      xok[t] = m0 + t < a.m;
      xrow[t] = a.q + (size_t)(xok[t] ? m0 + t : 0) * K;
    }
    const uint32_t nch = (K + 1023) / 1024;
    for (uint32_t c = 0; c < nch; c += U) {
      v4i wv[U][R], xv[U][MT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t kk = (c + u) * 1024 + lane * 16;
        const bool ok = (c + u < nch) && kk < K;
#pragma unroll
        for (int r = 0; r < R; ++r) wv[u][r] = ok ? load_nt16(W + wrow[r] + kk) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < MT; ++t) xv[u][t] = (ok && xok[t]) ? load16(xrow[t] + kk) : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int r = 0; r < R; ++r) acc[t * R + r] = dot16(xv[u][t], wv[u][r], acc[t * R + r]);
    }
  }
  const int total = fold_reduce<V>(acc, lane);
  constexpr int kSpan = 64 / V;
  const int idx = lane / kSpan;
  const uint32_t t = m0 + idx / R;
  const uint32_t row = row0 + idx % R;
  const bool writer = live && (lane % kSpan) == 0 && row < n && t < a.m;
  float value = 0.f;
  if (writer) {
    value = dequant(total, a.asc[t], a.ws[mi][row]);
    const size_t o = (size_t)t * n + row;
    if (a.out[mi]) store_out(a.out[mi], o, a.out_dtype, total, value);
    if (EPI == EPI_RESIDUAL) {
      const float comb = bf16_rne(a.residual[o] + value);
      store_out(a.combined, o, a.out_dtype, total, comb);
    }
  }
  if (EPI == EPI_ARGMAX)
    select_finish(writer ? select_key(value, row) : 0ull, a.partials, a.counter, a.token);
}

// Standalone greedy selection over f32 values.
__global__ __launch_bounds__(kGemvThreads) void select_kernel(const float* __restrict__ x, size_t n,
                                                               uint64_t* partials, uint32_t* counter,
                                                               uint32_t* token) {
  uint64_t best = 0;
  for (size_t i = (size_t)blockIdx.x * kGemvThreads + threadIdx.x; i < n;
       i += (size_t)gridDim.x * kGemvThreads) {
    const uint64_t k = select_key(x[i], (uint32_t)i);
    best = k > best ? k : best;
  }
  select_finish(best, partials, counter, token);
}

__global__ void write_sentinel(uint32_t* token) {
  if (threadIdx.x == 0) *token = 0xffffffffu;
}

// ------------------------------------------------------------------ launchers
template <int R>
static uint32_t count_groups(GemvArgs& a, const uint32_t* n, int count) {
  uint32_t g = 0;
  for (int i = 0; i < count; ++i) {
    a.gbegin[i] = g;
    g += (n[i] + R - 1) / R;
  }
  for (int i = count; i <= kMaxGroup; ++i) a.gbegin[i] = g;
  return g;
}

template <int EPI>
static hipError_t dispatch(hipStream_t st, GemvArgs& a) {
  uint32_t nn[kMaxGroup];
  for (int i = 0; i < a.count; ++i) nn[i] = a.n[i];
  // M = 1 at the Qwen3 widths: activation row register-resident.
  if (a.m == 1 && a.k == 4096) {
    const uint32_t groups = count_groups<4>(a, nn, a.count);
    if (groups == 0) return hipSuccess;
    hipLaunchKernelGGL((gemv_m1<4, 4, EPI>), dim3((groups + kGemvWaves - 1) / kGemvWaves),
                       dim3(kGemvThreads), 0, st, a);
    return hipGetLastError();
  }
  if (a.m == 1 && a.k == 12288) {
    const uint32_t groups = count_groups<2>(a, nn, a.count);
    if (groups == 0) return hipSuccess;
    hipLaunchKernelGGL((gemv_m1<2, 12, EPI>), dim3((groups + kGemvWaves - 1) / kGemvWaves),
                       dim3(kGemvThreads), 0, st, a);
    return hipGetLastError();
  }
  if (a.m == 1 || EPI == EPI_ARGMAX) {
    const uint32_t groups = count_groups<4>(a, nn, a.count);
    if (groups == 0) return hipSuccess;
    hipLaunchKernelGGL((gemv_mt<4, 1, 4, EPI>), dim3((groups + kGemvWaves - 1) / kGemvWaves),
                       dim3(kGemvThreads), 0, st, a);
    return hipGetLastError();
  }
  if (a.m <= 2) {
    const uint32_t groups = count_groups<4>(a, nn, a.count);
    if (groups == 0) return hipSuccess;
    hipLaunchKernelGGL((gemv_mt<4, 2, 4, EPI>), dim3((groups + kGemvWaves - 1) / kGemvWaves, 1),
                       dim3(kGemvThreads), 0, st, a);
    return hipGetLastError();
  }
  if (a.m <= 4) {
    const uint32_t groups = count_groups<4>(a, nn, a.count);
    if (groups == 0) return hipSuccess;
    hipLaunchKernelGGL((gemv_mt<4, 4, 2, EPI>), dim3((groups + kGemvWaves - 1) / kGemvWaves, 1),
                       dim3(kGemvThreads), 0, st, a);
    return hipGetLastError();
  }
  const uint32_t groups = count_groups<4>(a, nn, a.count);
  if (groups == 0) return hipSuccess;
  hipLaunchKernelGGL((gemv_mt<4, 8, 2, EPI>),
                     dim3((groups + kGemvWaves - 1) / kGemvWaves, (a.m + 7) / 8), dim3(kGemvThreads),
                     0, st, a);
  return hipGetLastError();
}

hipError_t launch_gemv(hipStream_t st, GemvArgs& a) {
  if (a.residual) return dispatch<EPI_RESIDUAL>(st, a);
  return dispatch<EPI_PLAIN>(st, a);
}

// Number of workgroups the fused lm_head launch uses for n rows at width k.
uint32_t gemv_argmax_blocks(size_t n, uint32_t k) {
  const uint32_t R = (k == 12288) ? 2 : 4;
  const uint64_t groups = (n + R - 1) / R;
  return (uint32_t)((groups + kGemvWaves - 1) / kGemvWaves);
}

hipError_t launch_gemv_argmax(hipStream_t st, GemvArgs& a) {
  if (a.n[0] == 0) {
    hipLaunchKernelGGL(write_sentinel, dim3(1), dim3(64), 0, st, a.token);
    return hipGetLastError();
  }
  return dispatch<EPI_ARGMAX>(st, a);
}

uint32_t select_blocks(size_t n) {
  const uint64_t b = (n + kGemvThreads * 16 - 1) / (kGemvThreads * 16);
  return (uint32_t)(b < 1 ? 1 : (b > 1024 ? 1024 : b));
}

hipError_t launch_select(hipStream_t st, const float* x, size_t n, uint64_t* partials,
                         uint32_t* counter, uint32_t* token) {
  if (n == 0) {
    hipLaunchKernelGGL(write_sentinel, dim3(1), dim3(64), 0, st, token);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(select_kernel, dim3(select_blocks(n)), dim3(kGemvThreads), 0, st, x, n,
                     partials, counter, token);
  return hipGetLastError();
}

}  // namespace w8a8
