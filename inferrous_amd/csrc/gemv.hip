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
// segment.  A wave issues the loads of its whole row group (one or two rows,
// 4-12 KiB) up front, reduces, writes and exits; the hardware dispatcher then
// walks the matrix in address order.  For M = 1 and
// the Qwen3 widths (4096, 12288) the activation row lives in registers
// (loaded once per wave from L2), so HBM traffic is the weights plus a few
// bytes per row.  Row-group indices are wave-uniform (scalar registers), so
// sibling selection and row addressing cost scalar loads only.  Partial sums
// are reduced with DPP row operations and v_readlane (no LDS round trips);
// lanes 0..R-1 then write R consecutive outputs.
//
// INT32 sums are exact (|acc| <= 12288 * 127^2 < 2^31), so the lane/chunk
// order is free; the epilogue keeps the reference's two RN multiplies and
// BF16 RNE (device_common.hpp `dequant`).
#include <algorithm>

#include "device_common.hpp"
#include "internal.hpp"

namespace w8a8 {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

enum { EPI_PLAIN = 0, EPI_RESIDUAL = 1, EPI_ARGMAX = 2 };

// Sum of one int over the wave, returned wave-uniform (in an SGPR).  Within
// each 16-lane row: quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror (DPP, no LDS traffic) leave the row sum in every
// lane of the row; four v_readlane and scalar adds combine the rows.  i32
// adds wrap, and every partial and final sum fits in i32, so it is exact.
__device__ __forceinline__ int wave_sum_uniform(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, true);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

// Reduce V per-lane partial sums; lane i < V receives total i.
template <int V>
__device__ __forceinline__ int reduce_to_lanes(const int (&v)[V], int lane) {
  static_assert(V >= 1 && V <= 64, "at most one value per lane");
  int out = 0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int t = wave_sum_uniform(v[i]);
    out = lane == i ? t : out;
  }
  return out;
}

// Wave index inside the workgroup as a wave-uniform (scalar) value, so that
// everything derived from it -- the owning sibling matrix, row addresses --
// is computed and loaded through the scalar unit.
__device__ __forceinline__ uint32_t wave_id() {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ void store_out(void* out, size_t idx, int dtype, int32_t acc, float value) {
  if (dtype == W8A8_OUT_F32)
    reinterpret_cast<float*>(out)[idx] = value;
  else if (dtype == W8A8_OUT_BF16)
    reinterpret_cast<uint16_t*>(out)[idx] = (uint16_t)(__float_as_uint(value) >> 16);
  else
    reinterpret_cast<int32_t*>(out)[idx] = acc;
}

// Which sibling matrix owns row group g (wave-uniform).  The launcher sets
// gbegin[i] to the total for every i >= count, and gbegin is nondecreasing, so
// the owner is the number of boundaries at or below g.  Every operand sits at
// a fixed kernel-argument offset: the kernel's argument loads issue as one
// batch instead of a chain of dependent scalar round trips.
__device__ __forceinline__ int owner(const GemvArgs& a, uint32_t g) {
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i) mi += g >= a.gbegin[i] ? 1 : 0;
  return mi;
}

// v[mi] by selects over fixed offsets (no argument load indexed by mi).
template <typename T, int N>
__device__ __forceinline__ T pick(const T (&v)[N], int mi) {
  static_assert(N >= kMaxGroup, "one entry per sibling matrix");
  T r = v[0];
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i) r = mi == i ? v[i] : r;
  return r;
}

// Rows covered by a launch: one past the last row group.
__device__ __forceinline__ uint32_t total_groups(const GemvArgs& a) { return a.gbegin[kMaxGroup]; }

// Greedy selection across workgroups, in two kernels and with no atomics on
// device memory.  The producer's workgroup b writes the largest key of its
// rows to keys[b]: its waves meet in LDS, and the wave that arrives last (an
// LDS counter, zeroed behind a barrier at the workgroup's start) writes.  A
// one-workgroup kernel, stream-ordered after the producer, reduces the keys
// and writes the token.  Each call writes every key it reads, so the
// workspace needs no initialisation and carries nothing between calls.
template <int W = kGemvWaves>
struct SelectLds {
  uint64_t key[W];
  uint32_t arrived;
};

template <int W>
__device__ __forceinline__ void select_lds_init(SelectLds<W>& s) {
  if (threadIdx.x == 0) s.arrived = 0;
  __syncthreads();
}

// Every lane of every wave calls this once, with its key (0 for no row).
template <int W>
__device__ __forceinline__ void select_publish_wave(uint64_t key, SelectLds<W>& s, uint64_t* keys) {
  key = wave_max_u64(key);
  if ((threadIdx.x & 63) == 0) {
    s.key[threadIdx.x >> 6] = key;
    const uint32_t before =
        __hip_atomic_fetch_add(&s.arrived, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (before == W - 1) {
      uint64_t b = s.key[0];
#pragma unroll
      for (int i = 1; i < W; ++i) b = s.key[i] > b ? s.key[i] : b;
      keys[blockIdx.x] = b;
    }
  }
}

constexpr int kFinalizeThreads = 1024;

// Latency-bound: each round issues all its loads before the first use (the
// index is clamped rather than tested, so no load waits behind a branch).
// B keys per thread per round, chosen by the launcher from the key count so
// that a small key set is not re-read B times over.
template <int B>
__global__ __launch_bounds__(kFinalizeThreads) void select_finalize(const uint64_t* __restrict__ keys,
                                                                    uint32_t nkeys, uint32_t* token) {
  __shared__ uint64_t wbest[kFinalizeThreads / 64];
  uint64_t b = 0;
  for (uint32_t base = 0; base < nkeys; base += kFinalizeThreads * B) {
    uint64_t v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) v[u] = keys[min(base + u * kFinalizeThreads + threadIdx.x, nkeys - 1)];
#pragma unroll
    for (int u = 0; u < B; ++u) b = v[u] > b ? v[u] : b;
  }
  b = wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < kFinalizeThreads / 64; ++i) b = wbest[i] > b ? wbest[i] : b;
    *token = key_to_token(b);
  }
}

// Operands of one M = 1 row-group wave, resolved by the kernel entry.
struct M1Operands {
  const int8_t* q;
  const float* asc;
  const int8_t* w;
  const float* ws;
  uint32_t n;     // rows of the owning matrix (>= 1 when live)
  uint32_t row0;  // first row of this wave's group
  bool live;
  void* out;
  int dtype;
  const float* residual;  // EPI_RESIDUAL
  void* combined;
};

// M = 1, k = KC * 1024 known at compile time: activations held in registers.
// R consecutive rows per wave; `sel` and `slots` serve the fused selection.
// TIMED (diagnostics only): the wave also records the 100 MHz device clock
// at its start, once all its loads have landed, and once its store is
// acknowledged, into stamps[3 g .. 3 g + 2] (g: the wave's index in the grid).
template <int R, int KC, int EPI, int WV, bool TIMED = false>
__device__ __forceinline__ void gemv_m1_body(const M1Operands& o, SelectLds<WV>* sel, uint64_t* slots,
                                             uint64_t* stamps = nullptr) {
  uint64_t t0 = 0, t1 = 0;
  if constexpr (TIMED) t0 = __builtin_amdgcn_s_memrealtime();
  const int lane = threadIdx.x & 63;
  constexpr uint32_t K = KC * 1024;
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0;
  float wsc = 0.f;  // ws of this lane's output row (writer lanes)
  float asc = 0.f;
  float resid = 0.f;
  if (o.live) {
    v4i x[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) x[c] = load16(o.q + c * 1024 + lane * 16);
    // The epilogue's operands are loaded ahead of the weight stream, so that
    // their latency hides under it instead of extending the wave's life.
    const uint32_t erow = min(o.row0 + (uint32_t)min(lane, R - 1), o.n - 1);
    wsc = o.ws[erow];
    asc = o.asc[0];
    if (EPI == EPI_RESIDUAL) resid = o.residual[erow];
    v4i wv[R][KC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t row = min(o.row0 + r, o.n - 1);  // tail rows recompute the last row
      const int8_t* p = o.w + (size_t)row * K + lane * 16;
#pragma unroll
      for (int c = 0; c < KC; ++c) wv[r][c] = load_nt16(p + c * 1024);
    }
    if constexpr (TIMED) {
      __builtin_amdgcn_s_waitcnt(0);
      t1 = __builtin_amdgcn_s_memrealtime();
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int c = 0; c < KC; ++c) acc[r] = dot16(x[c], wv[r][c], acc[r]);
  }
  const int total = reduce_to_lanes<R>(acc, lane);
  const uint32_t row = o.row0 + lane;
  const bool writer = o.live && lane < R && row < o.n;
  // Computed on every lane and pinned here, so the compiler cannot sink the
  // operand loads above into the writer branch, behind the weight stream.
  const float value = dequant(total, asc, wsc);
  const float comb = EPI == EPI_RESIDUAL ? bf16_rne(resid + value) : 0.f;
  const int dtype = o.dtype;
  asm volatile("" ::"v"(value), "v"(comb), "s"(dtype));
  if (writer) {
    if (o.out) store_out(o.out, row, dtype, total, value);
    if (EPI == EPI_RESIDUAL) store_out(o.combined, row, dtype, total, comb);
  }
  if (EPI == EPI_ARGMAX) select_publish_wave(writer ? select_key(value, row) : 0ull, *sel, slots);
  if constexpr (TIMED) {
    __builtin_amdgcn_s_waitcnt(0);
    const uint64_t t2 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
      const size_t g = (size_t)blockIdx.x * WV + wave_id();
      stamps[3 * g] = t0;
      stamps[3 * g + 1] = t1;
      stamps[3 * g + 2] = t2;
    }
  }
}

// Generic entry: up to kMaxGroup sibling matrices, and the fused selection.
template <int R, int KC, int EPI, int WV = kGemvWaves>
__global__ __launch_bounds__(64 * WV) void gemv_m1(GemvArgs a) {
  const uint32_t g = blockIdx.x * WV + wave_id();
  __shared__ SelectLds<WV> sel;
  M1Operands o;
  o.live = g < total_groups(a);
  const int mi = o.live ? owner(a, g) : 0;
  o.q = a.q;
  o.asc = a.asc;
  o.w = pick(a.w, mi);
  o.ws = pick(a.ws, mi);
  o.n = pick(a.n, mi);
  o.row0 = o.live ? (g - pick(a.gbegin, mi)) * R : 0;
  o.out = pick(a.out, mi);
  o.dtype = a.out_dtype;
  o.residual = a.residual;
  o.combined = a.combined;
  if (EPI == EPI_ARGMAX) {
    // The selection's LDS counter is zeroed behind a barrier.  The barrier
    // follows the argument loads (pinned here), so that the waves leave it
    // together and go straight to the weight stream: measured on MI355X for
    // the 151,936 x 4096 head, 88.9-89.1 us per launch this way against
    // 92.4-96.0 with the barrier first.
    asm volatile("" ::"s"(o.n), "s"(o.w), "s"(o.row0));
    select_lds_init(sel);
  }
  gemv_m1_body<R, KC, EPI, WV>(o, &sel, a.slots);
}

// One matrix (plain or residual epilogue), with scalar kernel arguments:
// the build preloads the first 16 argument dwords -- all of these -- into
// SGPRs, so the waves issue their loads without a kernel-argument load.
// The grid's tail waves clamp their rows rather than branch.  Measured on
// MI355X against the generic entry, the sibling lookup's chain of dependent
// argument loads cost 0.3-0.7 us per decode launch.
template <int R, int KC, int EPI, int WV = kGemvWaves>
__global__ __launch_bounds__(64 * WV) void gemv_m1_one(const int8_t* w, const int8_t* q, const float* ws,
                                                       const float* asc, void* out, uint32_t n, int dtype,
                                                       const float* residual, void* combined) {
  static_assert(EPI != EPI_ARGMAX, "the fused selection takes the generic entry");
  M1Operands o;
  o.q = q;
  o.asc = asc;
  o.w = w;
  o.ws = ws;
  o.n = n;
  o.row0 = (blockIdx.x * WV + wave_id()) * R;
  o.live = true;
  o.out = out;
  o.dtype = dtype;
  o.residual = residual;
  o.combined = combined;
  gemv_m1_body<R, KC, EPI, WV>(o, nullptr, nullptr);
}

// Diagnostics: gemv_m1_one (plain epilogue) with the per-wave clock stamps.
template <int R, int KC>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_m1_timed(const int8_t* w, const int8_t* q, const float* ws,
                                                                 const float* asc, void* out, uint32_t n, int dtype,
                                                                 uint64_t* stamps) {
  M1Operands o;
  o.q = q;
  o.asc = asc;
  o.w = w;
  o.ws = ws;
  o.n = n;
  o.row0 = (blockIdx.x * kGemvWaves + wave_id()) * R;
  o.live = true;
  o.out = out;
  o.dtype = dtype;
  o.residual = nullptr;
  o.combined = nullptr;
  gemv_m1_body<R, KC, EPI_PLAIN, kGemvWaves, true>(o, nullptr, nullptr, stamps);
}

// The producer of the activation codes folded into the prologue of the M = 1
// GEMV that consumes them: norm_quantize (src/kernels.rs:476-575) or
// quantize (src/kernels.rs:433-451) of one 4096-wide f32 row, then linear /
// linear_residual (src/kernels.rs:577-618, :807-845) on one matrix.  Every
// workgroup loads the row (and the gains) ahead of its weight stream and
// recomputes the row's scale with the producer's own arithmetic and order,
// and its codes with quant_code (the same integers as the producer's
// division), so every workgroup holds the same bits the producer kernel
// would have written; they reach the dot products through LDS.  Workgroup 0
// also writes the producer's outputs (codes, scale, the normalised row when
// asked for, the maxima reset).  One launch instead of two: measured on
// MI355X in graphs of 36 distinct-weight pairs, norm_quantize + qkv
// (6144 x 4096) 8.45 -> 7.43 us, quantize + o (4096 x 4096) 6.64 -> 5.30 us.
// The SwiGLU GEMV takes the same fold with two coordinates per wave
// (gemv_swiglu_norm, below).
enum { PROD_QUANT = 1, PROD_NORM = 2 };

struct ProducerLds {
  float part[256];
  float inv;
  uint32_t red[4];
  alignas(16) int8_t qs[4096];
};

// The producer's half of a folded kernel, over the workgroup's 256 threads,
// thread t holding v[i] = x[t + 256 i] (and g[i] = gain[t + 256 i]): the
// row's codes into L.qs (visible after the next barrier) and its scale,
// returned.  v is left holding the normalised values (PROD_NORM).
template <int PROD>
__device__ __forceinline__ float producer_codes(float (&v)[16], const float (&g)[16], ProducerLds& L) {
  static_assert(kGemvThreads == 256, "the producers' element order is laid out over 256 threads");
  const int t = threadIdx.x;
  uint32_t mb = kFloorBits;
  if (PROD == PROD_NORM) {
    const float inv = norm_inv_4096(v, L.part, &L.inv);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      v[i] = bf16_rne((v[i] * inv) * g[i]);
      mb = max(mb, abs_bits_no_nan(v[i]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) mb = max(mb, abs_bits_no_nan(v[i]));
  }
  mb = block_max_256(mb, L.red);
  const float sc = __uint_as_float(mb) / 127.0f, rc = 1.0f / sc;
#pragma unroll
  for (int i = 0; i < 16; ++i) L.qs[t + 256 * i] = quant_code(v[i], sc, rc);
  return sc;
}

// Workgroup 0 writes what the producer kernel would have written: the
// normalised row (when asked for), the scale and the maxima reset now, the
// codes after the barrier that publishes L.qs (producer_codes_out).
template <int PROD>
__device__ __forceinline__ void producer_outputs(const float (&v)[16], float sc, float* normed, float* scale_out,
                                                 uint32_t* maxima) {
  if (blockIdx.x != 0) return;
  const int t = threadIdx.x;
  if (PROD == PROD_NORM && normed)
#pragma unroll
    for (int i = 0; i < 16; ++i) normed[t + 256 * i] = v[i];
  if (t == 0) {
    scale_out[0] = sc;
    if (maxima) maxima[0] = kFloorBits;
  }
}

__device__ __forceinline__ void producer_codes_out(const ProducerLds& L, int8_t* q_out) {
  if (blockIdx.x == 0)
    *reinterpret_cast<v4i*>(q_out + threadIdx.x * 16) = *reinterpret_cast<const v4i*>(L.qs + threadIdx.x * 16);
}

template <int R, int EPI, int PROD>
__global__ __launch_bounds__(kGemvThreads) void gemv_m1_produce(
    const float* x, const float* gain, const int8_t* w, const float* ws, uint32_t n, int dtype,
    const float* residual, void* out, void* combined, int8_t* q_out, float* scale_out, uint32_t* maxima,
    float* normed) {
  __shared__ ProducerLds L;
  const int t = threadIdx.x, lane = t & 63;
  const uint32_t row0 = (blockIdx.x * kGemvWaves + wave_id()) * R;
  // The producer's operands are loaded first: loads complete in issue order,
  // so its math then waits for them alone while the weights are in flight.
  float v[16], g[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    v[i] = x[t + 256 * i];
    g[i] = PROD == PROD_NORM ? gain[t + 256 * i] : 0.f;
  }
  // The epilogue's operands and the weight stream; tail rows recompute the
  // last row (n >= 1).
  const uint32_t erow = min(row0 + (uint32_t)min(lane, R - 1), n - 1);
  const float wsc = ws[erow];
  const float resid = EPI == EPI_RESIDUAL ? residual[erow] : 0.f;
  v4i wv[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int8_t* p = w + (size_t)min(row0 + r, n - 1) * 4096 + lane * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) wv[r][c] = load_nt16(p + c * 1024);
  }
  const float sc = producer_codes<PROD>(v, g, L);
  producer_outputs<PROD>(v, sc, normed, scale_out, maxima);
  __syncthreads();
  v4i xq[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) xq[c] = *reinterpret_cast<const v4i*>(L.qs + c * 1024 + lane * 16);
  producer_codes_out(L, q_out);
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r] = dot16(xq[c], wv[r][c], acc[r]);
  }
  const int total = reduce_to_lanes<R>(acc, lane);
  const uint32_t row = row0 + lane;
  const bool writer = lane < R && row < n;
  // computed on every lane and pinned, as in gemv_m1_body
  const float value = dequant(total, sc, wsc);
  const float comb = EPI == EPI_RESIDUAL ? bf16_rne(resid + value) : 0.f;
  asm volatile("" ::"v"(value), "v"(comb), "s"(dtype));
  if (writer) {
    if (out) store_out(out, row, dtype, total, value);
    if (EPI == EPI_RESIDUAL) store_out(combined, row, dtype, total, comb);
  }
}

// Any m (blockIdx.y selects MT activation rows), any k % 16 == 0.
template <int R, int MT, int U, int EPI>
__global__ __launch_bounds__(kGemvThreads) void gemv_mt(GemvArgs a) {
  constexpr int V = R * MT;
  const int lane = threadIdx.x & 63;
  const uint32_t g = blockIdx.x * kGemvWaves + wave_id();
  const bool live = g < total_groups(a);
  const int mi = live ? owner(a, g) : 0;
  const uint32_t n = pick(a.n, mi);
  const uint32_t row0 = live ? (g - pick(a.gbegin, mi)) * R : 0;
  void* const out = pick(a.out, mi);
  const float* const ws = pick(a.ws, mi);
  const uint32_t m0 = blockIdx.y * MT;
  const uint32_t K = a.k;
  __shared__ SelectLds<> sel;
  if (EPI == EPI_ARGMAX) select_lds_init(sel);

  int acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0;
  if (live) {
    const int8_t* __restrict__ W = pick(a.w, mi);
    const int8_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = W + (size_t)min(row0 + r, n - 1) * K;
    const int8_t* xrow[MT];
    bool xok[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      xok[t] = m0 + t < a.m;
      xrow[t] = a.q + (size_t)(xok[t] ? m0 + t : 0) * K;
    }
    const uint32_t nch = (K + 1023) / 1024;
    // Up to 4 activation rows per pass, the row group's chunk order starts at
    // chunk g mod nch (exact sums in any order), so the waves of a launch do
    // not all read the same 1 KiB column of their rows at once.  Measured on
    // MI355X: gate_up 24576 x 4096 at M = 2 5.13 -> 5.65-5.76 TB/s, at M = 4
    // 4.58 -> 4.81-4.85; down 4096 x 12288 at M = 4 3.34 -> 3.48-3.51.  The
    // 8-row form (M >= 8, where the MFMA family is routed) lost 5-9% rotated.
    const uint32_t rot = MT <= 4 ? g % nch : 0;
    for (uint32_t c = 0; c < nch; c += U) {
      v4i wv[U][R], xv[U][MT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint32_t ci = c + u + rot;
        ci = ci >= nch ? ci - nch : ci;
        const uint32_t kk = ci * 1024 + lane * 16;
        const bool ok = (c + u < nch) && kk < K;
#pragma unroll
        for (int r = 0; r < R; ++r) wv[u][r] = ok ? load_nt16(wrow[r] + kk) : v4i{0, 0, 0, 0};
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
  const int total = reduce_to_lanes<V>(acc, lane);
  const uint32_t t = m0 + lane / R;
  const uint32_t row = row0 + lane % R;
  const bool writer = live && lane < V && row < n && t < a.m;
  float value = 0.f;
  if (writer) {
    value = dequant(total, a.asc[t], ws[row]);
    const size_t o = (size_t)t * n + row;
    if (out) store_out(out, o, a.out_dtype, total, value);
    if (EPI == EPI_RESIDUAL) {
      const float comb = bf16_rne(a.residual[o] + value);
      store_out(a.combined, o, a.out_dtype, total, comb);
    }
  }
  if (EPI == EPI_ARGMAX) select_publish_wave(writer ? select_key(value, row) : 0ull, sel, a.slots);
}

// Producer side of the maxima protocol (publish_absmax, src/kernels.rs:133-147):
// the workgroup's largest bits(|v|) (NaN -> 0) is folded into *p with one
// atomicMax.  *p only grows while producers run, so the thread first reads
// it (device-coherent relaxed load) and skips the atomic when not larger.
// Every thread of the workgroup must call this (it has a barrier).
__device__ __forceinline__ void publish_absmax_block(uint32_t bits, uint32_t* p) {
  __shared__ uint32_t wmax[kGemvWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  bits = wave_max_u32(bits);
  if (lane == 0) wmax[wave] = bits;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t b = wmax[0];
#pragma unroll
    for (int i = 1; i < kGemvWaves; ++i) b = wmax[i] > b ? wmax[i] : b;
    if (b > __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(p, b);
  }
}

// linear_swiglu (src/kernels.rs:619-695) at M = 1: one wave owns output
// coordinate c and streams gate row c and up row c (2 x k bytes) against the
// activation row held in registers; lane 0 writes gate, up (bit-exact
// linear epilogues) and act = silu_mul(gate, up).  The row's largest |act|
// is published by row_absmax_kernel, launched after this one.
template <int KC>
__global__ __launch_bounds__(kGemvThreads) void gemv_swiglu(SwigluArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t c = blockIdx.x * kGemvWaves + wave_id();
  // The grid's tail waves recompute the last row (the launcher requires
  // n >= 1) instead of branching, so the kernel-argument loads issue as one
  // batch ahead of the weight stream.
  const uint32_t cr = min(c, a.n - 1);
  constexpr uint32_t K = KC * 1024;
  int ag = 0, au = 0;
  v4i x[KC], wg[KC], wu[KC];
#pragma unroll
  for (int i = 0; i < KC; ++i) x[i] = load16(a.q + i * 1024 + lane * 16);
  // epilogue operands ahead of the weight stream (latency hidden under it)
  const float wsg = a.wsg[cr];
  const float wsu = a.wsu[cr];
  const float asc = a.asc[0];
  const int8_t* pg = a.wg + (size_t)cr * K + lane * 16;
  const int8_t* pu = a.wu + (size_t)cr * K + lane * 16;
#pragma unroll
  for (int i = 0; i < KC; ++i) {
    wg[i] = load_nt16(pg + i * 1024);
    wu[i] = load_nt16(pu + i * 1024);
  }
#pragma unroll
  for (int i = 0; i < KC; ++i) {
    ag = dot16(x[i], wg[i], ag);
    au = dot16(x[i], wu[i], au);
  }
  const int tg = wave_sum_uniform(ag);
  const int tu = wave_sum_uniform(au);
  const float g = dequant(tg, asc, wsg);
  const float u = dequant(tu, asc, wsu);
  const float v = silu_mul(g, u);
  // pinned on every lane: the operand loads stay ahead of the weight stream
  const int dtype = a.out_dtype;
  asm volatile("" ::"v"(v), "s"(dtype));
  if (c < a.n && lane == 0) {
    store_out(a.gate, c, dtype, tg, g);
    store_out(a.up, c, dtype, tu, u);
    store_out(a.act, c, dtype, 0, v);
  }
}

// norm_quantize folded into the M = 1 SwiGLU GEMV (K = 4096), as
// gemv_m1_produce folds it into linear: every workgroup recomputes the row's
// codes.  Each wave owns RC consecutive coordinates (their gate and up rows):
// with one coordinate per wave the 3,072 workgroups' repeated norm did not
// hide behind the weight stream (norm_quantize + SwiGLU GEMV 19.8 us as two
// launches, 20.0-20.3 as one); with two, 18.7 us.  The plain GEMV keeps one
// coordinate per wave (16.5 against 17.3 us with two).
template <int RC>
__global__ __launch_bounds__(kGemvThreads) void gemv_swiglu_norm(
    const float* x, const float* gain, const int8_t* wg, const float* wsg, const int8_t* wu, const float* wsu,
    uint32_t n, int dtype, void* gate, void* up, void* act, int8_t* q_out, float* scale_out, uint32_t* maxima,
    float* normed) {
  __shared__ ProducerLds L;
  const int t = threadIdx.x, lane = t & 63;
  const uint32_t c0 = (blockIdx.x * kGemvWaves + wave_id()) * RC;
  float v[16], g[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    v[i] = x[t + 256 * i];
    g[i] = gain[t + 256 * i];
  }
  // epilogue operands and weights; tail coordinates recompute the last (n >= 1)
  float sg[RC], su[RC];
  v4i wgv[RC][4], wuv[RC][4];
#pragma unroll
  for (int rc = 0; rc < RC; ++rc) {
    const uint32_t cr = min(c0 + rc, n - 1);
    sg[rc] = wsg[cr];
    su[rc] = wsu[cr];
    const int8_t* pg = wg + (size_t)cr * 4096 + lane * 16;
    const int8_t* pu = wu + (size_t)cr * 4096 + lane * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wgv[rc][i] = load_nt16(pg + i * 1024);
      wuv[rc][i] = load_nt16(pu + i * 1024);
    }
  }
  const float sc = producer_codes<PROD_NORM>(v, g, L);
  producer_outputs<PROD_NORM>(v, sc, normed, scale_out, maxima);
  __syncthreads();
  v4i xq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xq[i] = *reinterpret_cast<const v4i*>(L.qs + i * 1024 + lane * 16);
  producer_codes_out(L, q_out);
#pragma unroll
  for (int rc = 0; rc < RC; ++rc) {
    int ag = 0, au = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ag = dot16(xq[i], wgv[rc][i], ag);
      au = dot16(xq[i], wuv[rc][i], au);
    }
    const int tg = wave_sum_uniform(ag);
    const int tu = wave_sum_uniform(au);
    const float gv = dequant(tg, sc, sg[rc]);
    const float uv = dequant(tu, sc, su[rc]);
    const float av = silu_mul(gv, uv);
    asm volatile("" ::"v"(av), "s"(dtype));
    const uint32_t c = c0 + rc;
    if (c < n && lane == 0) {
      store_out(gate, c, dtype, tg, gv);
      store_out(up, c, dtype, tu, uv);
      store_out(act, c, dtype, 0, av);
    }
  }
}

__device__ __forceinline__ float load_val(const void* p, size_t i, int dtype) {
  if (dtype == W8A8_OUT_BF16)
    return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
  return reinterpret_cast<const float*>(p)[i];
}

// SwiGLU row tail, one workgroup per act row (blockIdx.x).  FOLD: the row's
// largest bits(|act|) (NaN -> 0) is folded into maxima[row] with one
// atomicMax -- the producer half of the quantize_with_max protocol
// (src/kernels.rs:133-147) for the fused M = 1 GEMV, which publishes
// nothing itself.  Publishing from each of that GEMV's 3,072 workgroups
// instead, right after the maximum was reset to its floor, made most of them
// atomics on the same word: 32.2 us per gate/up GEMV against 16.5 us
// without.  With q != null the row is then quantized exactly as
// quantize_with_max (src/kernels.rs:453-475) does with the folded maximum:
// s = RN(from_bits(maxima[row]) / 127), q_j = round(RN(act_j / s)).  A row
// of up to 16,384 values is loaded once, all loads issued before the first
// use (indices clamped), and kept in registers for both passes.
constexpr int kRowTailThreads = 1024;
constexpr int kRowTailCache = 16;  // act values per thread held in registers (rows up to 16,384 wide)

template <bool FOLD>
__global__ __launch_bounds__(kRowTailThreads) void swiglu_row_tail(const void* act, uint32_t n, int dtype,
                                                                    uint32_t* maxima, int8_t* q, float* scales) {
  __shared__ uint32_t wmax[kRowTailThreads / 64];
  __shared__ uint32_t row_max;
  const size_t r = blockIdx.x, base_i = r * (size_t)n;
  // Only this workgroup folds into maxima[r] during the call, so the value
  // before the fold can be read up front, and the fold needs no return.
  uint32_t before = 0;
  if (threadIdx.x == 0) before = maxima[r];
  const bool cached = n <= (uint32_t)(kRowTailThreads * kRowTailCache);
  float v[kRowTailCache];
  if (cached) {
#pragma unroll
    for (int u = 0; u < kRowTailCache; ++u)
      v[u] = load_val(act, base_i + min(u * kRowTailThreads + threadIdx.x, n - 1), dtype);
  }
  if (FOLD) {
    uint32_t bits = 0;
    if (cached) {
#pragma unroll
      for (int u = 0; u < kRowTailCache; ++u) bits = max(bits, abs_bits_no_nan(v[u]));
    } else {
      for (uint32_t j = threadIdx.x; j < n; j += kRowTailThreads)
        bits = max(bits, abs_bits_no_nan(load_val(act, base_i + j, dtype)));
    }
    bits = wave_max_u32(bits);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = bits;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 0; i < kRowTailThreads / 64; ++i) bits = max(bits, wmax[i]);
      atomicMax(maxima + r, bits);
      row_max = max(before, bits);
    }
  } else if (threadIdx.x == 0) {
    row_max = before;
  }
  if (!q) return;
  __syncthreads();
  const float s = __uint_as_float(row_max) / 127.0f;
  if (threadIdx.x == 0) scales[r] = s;
  if (cached) {
#pragma unroll
    for (int u = 0; u < kRowTailCache; ++u) {
      const uint32_t j = u * kRowTailThreads + threadIdx.x;
      if (j < n) q[base_i + j] = round_i8(v[u] / s);
    }
  } else {
    for (uint32_t j = threadIdx.x; j < n; j += kRowTailThreads)
      q[base_i + j] = round_i8(load_val(act, base_i + j, dtype) / s);
  }
}

// The SwiGLU row tail folded into the M = 1 down GEMV that consumes its
// codes (gemv_m1_rowtail): swiglu_row_tail<true>'s work -- the act row's
// largest bits(|act|) (NaN -> 0) folded into maxima[0], then
// quantize_with_max (src/kernels.rs:453-475) with that maximum, s =
// RN(from_bits(max(m0, row max)) / 127), q_j = round(RN(act_j / s)) -- then
// linear / linear_residual (src/kernels.rs:577-618) on one matrix of
// K = 12,288.  Every workgroup loads the act row ahead of its weights,
// reduces the row maximum with the row tail's expressions and quantizes the
// row to the row tail's codes (quant_code: the same integers without a
// division per element), so it holds the codes and scale the row tail would
// have written; they reach the dot products through LDS.  m0 is maxima[0] as a
// workgroup reads it: the call's value, or that value with the row maximum
// folded in by workgroup 0's atomicMax -- max(m0, row max) is the same
// either way.  Workgroup 0 also writes the codes and the scale (when asked
// for) and folds the maximum, so the state after the call is the row
// tail's.  Sixteen waves per workgroup, one row each: every workgroup
// repeats the row's 12,288 divisions, so fewer, larger workgroups pay less
// for them.  Measured on MI355X, graphs of 36 distinct-weight launches,
// row tail + down with residual: 14.46 us per layer as two launches, 11.88
// folded with 16 waves, 13.05 with 8, 16.85 with 4.
constexpr int kRowtailWaves = 16;
constexpr uint32_t kRowtailWidth = 12288;

template <int EPI>
__global__ __launch_bounds__(kRowtailWaves * kWave) void gemv_m1_rowtail(
    const void* act, int act_dtype, uint32_t* maxima, const int8_t* w, const float* ws, uint32_t n, int dtype,
    const float* residual, void* out, void* combined, int8_t* q_out, float* scale_out) {
  constexpr int T = kRowtailWaves * kWave, PER = kRowtailWidth / T, KC = kRowtailWidth / 1024;
  static_assert(kRowtailWidth % T == 0, "the row splits evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) int8_t qs[kRowtailWidth];
  __shared__ uint32_t wmax[kRowtailWaves];
  const int t = threadIdx.x, lane = t & 63, wv = wave_id();
  // The producer's operands first: loads complete in issue order, so its
  // math waits for them alone while the weights are in flight.
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = load_val(act, t + (size_t)T * i, act_dtype);
  const uint32_t m0 = maxima[0];
  const uint32_t row0 = blockIdx.x * kRowtailWaves + wv;
  const uint32_t erow = min(row0, n - 1);  // tail rows recompute the last row (n >= 1)
  const float wsc = ws[erow];
  const float resid = EPI == EPI_RESIDUAL ? residual[erow] : 0.f;
  v4i wt[KC];
  const int8_t* p = w + (size_t)erow * kRowtailWidth + lane * 16;
#pragma unroll
  for (int c = 0; c < KC; ++c) wt[c] = load_nt16(p + c * 1024);
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) bits = max(bits, abs_bits_no_nan(v[i]));
  bits = wave_max_u32(bits);
  if (lane == 0) wmax[wv] = bits;
  __syncthreads();
  uint32_t rmax = 0;
#pragma unroll
  for (int j = 0; j < kRowtailWaves; ++j) rmax = max(rmax, wmax[j]);
  const float sc = __uint_as_float(max(m0, rmax)) / 127.0f, rc = 1.0f / sc;
#pragma unroll
  for (int i = 0; i < PER; ++i) qs[t + T * i] = quant_code(v[i], sc, rc);
  if (blockIdx.x == 0 && t == 0) {
    atomicMax(maxima, rmax);
    if (scale_out) scale_out[0] = sc;
  }
  __syncthreads();
  if (blockIdx.x == 0 && q_out && t < (int)(kRowtailWidth / 16))
    *reinterpret_cast<v4i*>(q_out + t * 16) = *reinterpret_cast<const v4i*>(qs + t * 16);
  v4i xq[KC];
#pragma unroll
  for (int c = 0; c < KC; ++c) xq[c] = *reinterpret_cast<const v4i*>(qs + c * 1024 + lane * 16);
  int acc[1] = {0};
#pragma unroll
  for (int c = 0; c < KC; ++c) acc[0] = dot16(xq[c], wt[c], acc[0]);
  const int total = reduce_to_lanes<1>(acc, lane);
  const bool writer = lane == 0 && row0 < n;
  // computed on every lane and pinned, as in gemv_m1_body
  const float value = dequant(total, sc, wsc);
  const float comb = EPI == EPI_RESIDUAL ? bf16_rne(resid + value) : 0.f;
  asm volatile("" ::"v"(value), "v"(comb), "s"(dtype));
  if (writer) {
    if (out) store_out(out, row0, dtype, total, value);
    if (EPI == EPI_RESIDUAL) store_out(combined, row0, dtype, total, comb);
  }
}

// swiglu (src/kernels.rs:2172-2190): act = silu_mul(gate, up) elementwise
// over rows x width (blockIdx.y = row); with maxima, each row's largest
// |act| is published into maxima[row].
__global__ __launch_bounds__(kGemvThreads) void swiglu_kernel(const void* gate, const void* up,
                                                               uint32_t width, void* act, int dtype,
                                                               uint32_t* maxima) {
  const size_t r = blockIdx.y;
  uint32_t bits = 0;
  for (uint32_t j = blockIdx.x * kGemvThreads + threadIdx.x; j < width;
       j += gridDim.x * kGemvThreads) {
    const size_t i = r * width + j;
    const float v = silu_mul(load_val(gate, i, dtype), load_val(up, i, dtype));
    store_out(act, i, dtype, 0, v);
    bits = max(bits, abs_bits_no_nan(v));
  }
  if (maxima) publish_absmax_block(bits, maxima + r);
}

// Standalone greedy selection over f32 values.  Each thread takes
// kSelectPer values per pass, all loaded before any is compared (indices
// clamped), so a pass costs one load round trip.
constexpr int kSelectPer = 16;

__global__ __launch_bounds__(kGemvThreads) void select_kernel(const float* __restrict__ x, size_t n,
                                                               uint64_t* keys) {
  __shared__ SelectLds<> sel;
  select_lds_init(sel);
  uint64_t best = 0;
  for (size_t base = (size_t)blockIdx.x * kGemvThreads * kSelectPer; base < n;
       base += (size_t)gridDim.x * kGemvThreads * kSelectPer) {
    float v[kSelectPer];
#pragma unroll
    for (int u = 0; u < kSelectPer; ++u) v[u] = x[min(base + u * kGemvThreads + threadIdx.x, n - 1)];
#pragma unroll
    for (int u = 0; u < kSelectPer; ++u) {
      const size_t i = base + u * kGemvThreads + threadIdx.x;
      const uint64_t k = i < n ? select_key(v[u], (uint32_t)i) : 0ull;
      best = k > best ? k : best;
    }
  }
  select_publish_wave(best, sel, keys);
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

// Each launcher reports its grid's x extent in *blocks: the fused selection
// publishes one key per workgroup, and the one-workgroup finalize reads them
// all.  Its M = 1 workgroups carry 16 waves, a quarter of the keys of the
// plain GEMV's 4-wave workgroups.
template <int R, int KC, int EPI>
static hipError_t launch_m1(hipStream_t st, GemvArgs& a, const uint32_t* nn, uint32_t* blocks) {
  constexpr int W = EPI == EPI_ARGMAX ? 16 : kGemvWaves;
  const uint32_t groups = count_groups<R>(a, nn, a.count);
  *blocks = (groups + W - 1) / W;
  if (groups == 0) return hipSuccess;
  // The fused selection keeps the generic entry, which orders its barrier
  // after the argument loads.
  if constexpr (EPI != EPI_ARGMAX) {
    if (a.count == 1) {
      hipLaunchKernelGGL((gemv_m1_one<R, KC, EPI, W>), dim3(*blocks), dim3(64 * W), 0, st, a.w[0], a.q,
                         a.ws[0], a.asc, a.out[0], a.n[0], a.out_dtype, a.residual, a.combined);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv_m1<R, KC, EPI, W>), dim3(*blocks), dim3(64 * W), 0, st, a);
  return hipGetLastError();
}

template <int MT, int U, int EPI>
static hipError_t launch_mt(hipStream_t st, GemvArgs& a, const uint32_t* nn, uint32_t* blocks) {
  const uint32_t groups = count_groups<4>(a, nn, a.count);
  *blocks = (groups + kGemvWaves - 1) / kGemvWaves;
  if (groups == 0) return hipSuccess;
  hipLaunchKernelGGL((gemv_mt<4, MT, U, EPI>), dim3(*blocks, (a.m + MT - 1) / MT), dim3(kGemvThreads), 0,
                     st, a);
  return hipGetLastError();
}

// Row-group shape: measured on MI355X, waves that issue one short batch
// (one or two 4 KiB rows) and exit stream HBM better than longer batches or
// grid-stride sweeps; two rows per wave helps only the small matrices.
template <int EPI>
static hipError_t dispatch(hipStream_t st, GemvArgs& a, uint32_t* blocks) {
  uint32_t nn[kMaxGroup];
  uint64_t total = 0;
  for (int i = 0; i < a.count; ++i) {
    nn[i] = a.n[i];
    total += a.n[i];
  }
  if (a.m == 1 && a.k == 4096)
    return total <= 8192 ? launch_m1<2, 4, EPI>(st, a, nn, blocks) : launch_m1<1, 4, EPI>(st, a, nn, blocks);
  if (a.m == 1 && a.k == 12288) return launch_m1<1, 12, EPI>(st, a, nn, blocks);
  if (a.m == 1 || EPI == EPI_ARGMAX) return launch_mt<1, 4, EPI>(st, a, nn, blocks);
  if (a.m <= 2) return launch_mt<2, 4, EPI>(st, a, nn, blocks);
  if (a.m <= 4) return launch_mt<4, 2, EPI>(st, a, nn, blocks);
  return launch_mt<8, 2, EPI>(st, a, nn, blocks);
}

// The one-matrix M = 1 launch shape of `dispatch` (rows per wave by total N,
// four waves per workgroup), for the timed diagnostics kernel.
size_t gemv_timeline_waves(size_t n, uint32_t k) {
  if (n == 0 || (k != 4096 && k != 12288)) return 0;
  const size_t r = (k == 4096 && n <= 8192) ? 2 : 1;
  const size_t groups = (n + r - 1) / r;
  return (groups + kGemvWaves - 1) / kGemvWaves * kGemvWaves;
}

hipError_t launch_gemv_timeline(hipStream_t st, const int8_t* q, const float* asc, const int8_t* w,
                                const float* ws, uint32_t n, uint32_t k, void* out, int dtype,
                                uint64_t* stamps) {
  const uint32_t blocks = (uint32_t)(gemv_timeline_waves(n, k) / kGemvWaves);
  if (blocks == 0) return hipErrorInvalidValue;
  if (k == 12288)
    hipLaunchKernelGGL((gemv_m1_timed<1, 12>), dim3(blocks), dim3(kGemvThreads), 0, st, w, q, ws, asc, out, n,
                       dtype, stamps);
  else if (n <= 8192)
    hipLaunchKernelGGL((gemv_m1_timed<2, 4>), dim3(blocks), dim3(kGemvThreads), 0, st, w, q, ws, asc, out, n,
                       dtype, stamps);
  else
    hipLaunchKernelGGL((gemv_m1_timed<1, 4>), dim3(blocks), dim3(kGemvThreads), 0, st, w, q, ws, asc, out, n,
                       dtype, stamps);
  return hipGetLastError();
}

hipError_t launch_gemv(hipStream_t st, GemvArgs& a) {
  uint32_t blocks = 0;
  if (a.residual) return dispatch<EPI_RESIDUAL>(st, a, &blocks);
  return dispatch<EPI_PLAIN>(st, a, &blocks);
}

template <int R, int EPI, int PROD>
static hipError_t launch_produce(hipStream_t st, const ProduceArgs& p) {
  const uint32_t blocks = (p.n + R * kGemvWaves - 1) / (R * kGemvWaves);
  hipLaunchKernelGGL((gemv_m1_produce<R, EPI, PROD>), dim3(blocks), dim3(kGemvThreads), 0, st, p.x, p.gain, p.w,
                     p.ws, p.n, p.out_dtype, p.residual, p.out, p.combined, p.q, p.scale, p.maxima, p.normed);
  return hipGetLastError();
}

template <int PROD>
static hipError_t launch_produce_epi(hipStream_t st, const ProduceArgs& p) {
  // Four rows per wave up to N = 8192, one beyond.  Each workgroup repeats
  // the producer, so fewer workgroups pay less for it than the plain GEMV's
  // two rows per wave would: measured on MI355X, graphs of 24 distinct-weight
  // launches, two -> four rows, quantize + o with residual (4096 x 4096)
  // 5.50 -> 4.90 us, norm_quantize + qkv (6144 x 4096) 7.75 -> 7.56.
  if (p.residual)
    return p.n <= 8192 ? launch_produce<4, EPI_RESIDUAL, PROD>(st, p) : launch_produce<1, EPI_RESIDUAL, PROD>(st, p);
  return p.n <= 8192 ? launch_produce<4, EPI_PLAIN, PROD>(st, p) : launch_produce<1, EPI_PLAIN, PROD>(st, p);
}

hipError_t launch_gemv_produce(hipStream_t st, const ProduceArgs& p) {
  if (p.n == 0) return hipErrorInvalidValue;
  return p.gain ? launch_produce_epi<PROD_NORM>(st, p) : launch_produce_epi<PROD_QUANT>(st, p);
}

static hipError_t launch_finalize(hipStream_t st, const uint64_t* keys, uint32_t nkeys, uint32_t* token) {
  const uint32_t per = (nkeys + kFinalizeThreads - 1) / kFinalizeThreads;  // keys per thread
  if (per <= 1)
    hipLaunchKernelGGL(select_finalize<1>, dim3(1), dim3(kFinalizeThreads), 0, st, keys, nkeys, token);
  else if (per <= 8)
    hipLaunchKernelGGL(select_finalize<8>, dim3(1), dim3(kFinalizeThreads), 0, st, keys, nkeys, token);
  else if (per <= 16)
    hipLaunchKernelGGL(select_finalize<16>, dim3(1), dim3(kFinalizeThreads), 0, st, keys, nkeys, token);
  else
    hipLaunchKernelGGL(select_finalize<48>, dim3(1), dim3(kFinalizeThreads), 0, st, keys, nkeys, token);
  return hipGetLastError();
}

hipError_t launch_gemv_argmax(hipStream_t st, GemvArgs& a) {
  if (a.n[0] == 0) {
    hipLaunchKernelGGL(write_sentinel, dim3(1), dim3(64), 0, st, a.token);
    return hipGetLastError();
  }
  uint32_t blocks = 0;
  hipError_t e = dispatch<EPI_ARGMAX>(st, a, &blocks);
  if (e != hipSuccess) return e;
  return launch_finalize(st, a.slots, blocks, a.token);
}

size_t argmax_keys_bound(size_t n) {
  // every route puts at least one row per wave and at least kGemvWaves waves
  // per workgroup
  static_assert(kGemvWaves == kArgmaxRowsPerKey, "selection key bound");
  return argmax_keys_for(n);
}

hipError_t launch_gemv_swiglu(hipStream_t st, const SwigluArgs& a) {
  if (a.n == 0) return hipSuccess;
  const dim3 grid((a.n + kGemvWaves - 1) / kGemvWaves);
  if (a.k == 4096)
    hipLaunchKernelGGL(gemv_swiglu<4>, grid, dim3(kGemvThreads), 0, st, a);
  else if (a.k == 12288)
    hipLaunchKernelGGL(gemv_swiglu<12>, grid, dim3(kGemvThreads), 0, st, a);
  else
    return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !a.maxima) return e;
  hipLaunchKernelGGL(swiglu_row_tail<true>, dim3(1), dim3(kRowTailThreads), 0, st, a.act, a.n, a.out_dtype,
                     a.maxima, a.q_out, a.scales_out);
  return hipGetLastError();
}

hipError_t launch_gemv_swiglu_norm(hipStream_t st, const ProduceArgs& p, const SwigluArgs& a, bool row_tail) {
  if (a.n == 0 || a.k != 4096 || !a.maxima) return hipErrorInvalidValue;
  constexpr int RC = 2;  // four coordinates per wave: 20.5 us against 18.8 (gate_up 2 x 12288 x 4096)
  const dim3 grid((a.n + RC * kGemvWaves - 1) / (RC * kGemvWaves));
  hipLaunchKernelGGL(gemv_swiglu_norm<RC>, grid, dim3(kGemvThreads), 0, st, p.x, p.gain, a.wg, a.wsg, a.wu, a.wsu,
                     a.n, a.out_dtype, a.gate, a.up, a.act, p.q, p.scale, p.maxima, p.normed);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !row_tail) return e;
  // the norm reset maxima[0] inside the GEMV; the row tail folds into it
  hipLaunchKernelGGL(swiglu_row_tail<true>, dim3(1), dim3(kRowTailThreads), 0, st, a.act, a.n, a.out_dtype,
                     a.maxima, a.q_out, a.scales_out);
  return hipGetLastError();
}

hipError_t launch_gemv_rowtail(hipStream_t st, const RowtailArgs& d) {
  if (d.n == 0 || !d.maxima) return hipErrorInvalidValue;
  const dim3 grid((d.n + kRowtailWaves - 1) / kRowtailWaves), block(kRowtailWaves * kWave);
  if (d.residual)
    hipLaunchKernelGGL(gemv_m1_rowtail<EPI_RESIDUAL>, grid, block, 0, st, d.act, d.act_dtype, d.maxima, d.w, d.ws,
                       d.n, d.out_dtype, d.residual, d.out, d.combined, d.q_out, d.scale_out);
  else
    hipLaunchKernelGGL(gemv_m1_rowtail<EPI_PLAIN>, grid, block, 0, st, d.act, d.act_dtype, d.maxima, d.w, d.ws,
                       d.n, d.out_dtype, nullptr, d.out, nullptr, d.q_out, d.scale_out);
  return hipGetLastError();
}

hipError_t launch_swiglu_quantize_rows(hipStream_t st, const void* act, size_t rows, uint32_t width, int dtype,
                                       const uint32_t* maxima, int8_t* q, float* scales) {
  if (rows == 0 || width == 0) return hipSuccess;
  if (rows > 0x7fffffffu) return hipErrorInvalidValue;
  hipLaunchKernelGGL(swiglu_row_tail<false>, dim3((unsigned)rows), dim3(kRowTailThreads), 0, st, act, width, dtype,
                     const_cast<uint32_t*>(maxima), q, scales);
  return hipGetLastError();
}

hipError_t launch_swiglu(hipStream_t st, const void* gate, const void* up, size_t rows,
                         uint32_t width, void* act, int dtype, uint32_t* maxima) {
  if (rows == 0 || width == 0) return hipSuccess;
  const uint32_t bx = std::min<uint32_t>((width + kGemvThreads - 1) / kGemvThreads, 64u);
  const size_t esz = dtype == W8A8_OUT_BF16 ? 2 : 4;
  for (size_t r0 = 0; r0 < rows; r0 += 65535) {
    const uint32_t ry = (uint32_t)std::min<size_t>(rows - r0, 65535);
    const size_t off = r0 * width * esz;
    hipLaunchKernelGGL(swiglu_kernel, dim3(bx, ry), dim3(kGemvThreads), 0, st,
                       (const char*)gate + off, (const char*)up + off, width, (char*)act + off,
                       dtype, maxima ? maxima + r0 : nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_select(hipStream_t st, const float* x, size_t n, uint64_t* keys, uint32_t* token) {
  if (n == 0) {
    hipLaunchKernelGGL(write_sentinel, dim3(1), dim3(64), 0, st, token);
    return hipGetLastError();
  }
  const uint64_t b = (n + kGemvThreads * kSelectPer - 1) / (kGemvThreads * kSelectPer);
  const unsigned blocks = (unsigned)(b > kSelectBlocks ? kSelectBlocks : b);
  hipLaunchKernelGGL(select_kernel, dim3(blocks), dim3(kGemvThreads), 0, st, x, n, keys);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_finalize(st, keys, blocks, token);
}

}  // namespace w8a8
