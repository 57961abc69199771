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

// The row slot of workgroup b among G.  The dispatcher deals workgroups to
// the eight XCDs in turn (b on XCD b mod 8); slot (b mod 8) (G / 8) + b / 8
// gives each XCD a contiguous range of slots, so that at each step an XCD's
// streaming waves read consecutive rows, spread over the HBM channels,
// instead of every eighth row.  Measured on MI355X with per-workgroup clock
// stamps: with slot = b, one XCD's workgroups ended up to 2 us after
// another's in the 12,288-coordinate SwiGLU GEMV.  (The dispatcher-ordered
// GEMVs keep slot = b: this mapping made the decode chain of gemv_m1_one
// launches 1.306 -> 1.327 ms.)
__device__ __forceinline__ uint32_t xcd_slot(uint32_t b, uint32_t G) {
  return G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
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

// ------------------------------------------------ folded producers, split roles
// The producer of a GEMV's activation codes folded into the GEMV launch:
// norm_quantize (src/kernels.rs:476-575) or quantize (:433-451) of one
// 4096-wide f32 row before linear / linear_residual (src/kernels.rs:577-618,
// :807-845) or linear_swiglu (:619-695), and the SwiGLU row tail
// (quantize_with_max with the act row's maximum folded in, :453-475 and
// :133-147) before the down projection of K = 12,288.  Every workgroup
// derives the codes itself, with the producer kernel's arithmetic and
// order, so it holds the bits the producer would have written; workgroup 0
// also writes the producer's outputs.  One launch instead of two.
//
// Roles.  A CU holds back the issue of further vector-memory loads while
// many of its requests are in flight: measured on MI355X with per-wave clock
// stamps, of sixteen waves that each stream a 12 KiB row, the k-th wave on
// each SIMD finished issuing its loads about k x 1.7 us after the launch.  A
// producer whose waves also stream weights, meeting at workgroup barriers,
// therefore waits for the last wave to issue its weights -- near the end of
// the stream -- before its codes exist (2-3 us of the 9-19 us launches).  So
// the roles are split: four producer waves load the row, and a barrier
// orders those loads ahead of every weight load of the workgroup; the NS
// streaming waves then issue their weights and meet the producers once
// more, at the hand-off barrier, which publishes the codes and the scale.
// The producers meet among themselves through an LDS counter (prod_sync),
// never at a workgroup barrier, so the streamers' held-back issue does not
// delay them.  One workgroup per CU at the decode shapes.
enum { PROD_QUANT = 1, PROD_NORM = 2 };
constexpr int kProdWaves = 4;
// KiB of its first row each streaming wave requests before the first
// barrier.  Measured on MI355X: two KiB delayed the barrier (the producer's
// row loads then queue behind them) and gained nothing, so none.
constexpr int kSplitLead = 0;

template <int K>
struct SplitLds {
  float part[256];
  float inv;
  uint32_t red[4];
  uint32_t count;  // producer-wave arrivals (prod_sync)
  float scale;
  alignas(16) int8_t qs[K];
};

// Workgroup barrier that orders the LDS operations before it and nothing
// else: a wave's outstanding global loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The producer waves' own barrier: each adds one to *count and waits until
// the count reaches the next multiple of kProdWaves.  Every producer wave
// arrives (none of them waits on anything but its own row loads), so the
// waits end; the other waves never touch the counter.
__device__ __forceinline__ void prod_sync(uint32_t* count, uint32_t& target) {
  target += kProdWaves;
  __builtin_amdgcn_wave_barrier();
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(count, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target)
    __builtin_amdgcn_s_sleep(1);
}

// The K = 4096 producer, run by the producer waves (pt = 0..255) holding
// v[i] = x[pt + 256 i] and g[i] = gain[pt + 256 i]: the codes into L.qs and
// the scale into L.scale, with norm_quantize's / quantize's arithmetic
// (norm_inv_4096's order, the same maximum, quant_code's integers).
// Workgroup 0 also writes the normalised row (when asked for), the scale
// and the maxima reset.
template <int PROD>
__device__ __forceinline__ void split_producer_4096(float (&v)[16], const float (&g)[16], SplitLds<4096>& L,
                                                    int pt, float* normed, float* scale_out,
                                                    uint32_t* maxima) {
  uint32_t target = 0;
  auto sync = [&] { prod_sync(&L.count, target); };
  uint32_t mb = kFloorBits;
  if (PROD == PROD_NORM) {
    const float inv = norm_inv_4096_with(v, L.part, &L.inv, pt, sync);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      v[i] = bf16_rne((v[i] * inv) * g[i]);
      mb = max(mb, abs_bits_no_nan(v[i]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) mb = max(mb, abs_bits_no_nan(v[i]));
  }
  mb = block_max_256_with(mb, L.red, pt, sync);
  const float sc = __uint_as_float(mb) / 127.0f, rc = 1.0f / sc;
  int code[16];
  quant_codes(v, sc, rc, code);
#pragma unroll
  for (int i = 0; i < 16; ++i) L.qs[pt + 256 * i] = (int8_t)code[i];
  if (pt == 0) L.scale = sc;
  if (blockIdx.x != 0) return;
  if (PROD == PROD_NORM && normed)
#pragma unroll
    for (int i = 0; i < 16; ++i) normed[pt + 256 * i] = v[i];
  if (pt == 0) {
    scale_out[0] = sc;
    if (maxima) maxima[0] = kFloorBits;
  }
}

// The producer waves' row loads (thread pt of the four).
template <int PROD>
__device__ __forceinline__ void split_load_4096(const float* x, const float* gain, int pt, float (&v)[16],
                                                float (&g)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    v[i] = x[pt + 256 * i];
    g[i] = PROD == PROD_NORM ? gain[pt + 256 * i] : 0.f;
  }
}

// Workgroup 0's producer waves copy the codes out after the hand-off.
template <int K>
__device__ __forceinline__ void split_codes_out(const SplitLds<K>& L, int pt, int8_t* q_out) {
  if (blockIdx.x != 0 || !q_out) return;
  for (int i = pt; i < K / 16; i += kProdWaves * kWave)
    *reinterpret_cast<v4i*>(q_out + i * 16) = *reinterpret_cast<const v4i*>(L.qs + i * 16);
}

// linear / linear_residual with the K = 4096 producer folded in: NS
// streaming waves of RS consecutive rows each (workgroup b: rows
// [b NS RS, (b + 1) NS RS)), four producer waves.  Tail rows recompute the
// last row (n >= 1).
template <int NS, int RS, int EPI, int PROD>
__global__ __launch_bounds__((NS + kProdWaves) * kWave) void gemv_m1_split(
    const float* x, const float* gain, const int8_t* w, const float* ws, uint32_t n, int dtype,
    const float* residual, void* out, void* combined, int8_t* q_out, float* scale_out, uint32_t* maxima,
    float* normed) {
  __shared__ SplitLds<4096> L;
  const int t = threadIdx.x, lane = t & 63;
  const uint32_t wv = wave_id();
  const int pt = t - NS * kWave;
  const bool producer = wv >= NS;
  if (t == 0) L.count = 0;
  // row r of a streaming wave: (r NS + wave) G + workgroup, so that the
  // streamers of all workgroups sweep one window of the matrix together
  const uint32_t G = gridDim.x;
  auto row_of = [&](int r) -> uint32_t { return ((uint32_t)r * NS + wv) * G + xcd_slot(blockIdx.x, G); };
  auto wrow = [&](int r) { return w + (size_t)min(row_of(r), n - 1) * 4096 + lane * 16; };
  float v[16], g[16];
  v4i wt[RS][4];
  if (producer)
    split_load_4096<PROD>(x, gain, pt, v, g);
  else
#pragma unroll
    for (int c = 0; c < kSplitLead; ++c) wt[0][c] = load_nt16(wrow(0) + c * 1024);
  lds_barrier();  // the row loads ahead of the weight stream; L.count zeroed
  if (producer) {
    split_producer_4096<PROD>(v, g, L, pt, normed, scale_out, maxima);
    lds_barrier();  // hand-off
    split_codes_out(L, pt, q_out);
    return;
  }
  float wsr[RS], rsr[RS];
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const uint32_t er = min(row_of(r), n - 1);
    wsr[r] = ws[er];
    rsr[r] = EPI == EPI_RESIDUAL ? residual[er] : 0.f;
#pragma unroll
    for (int c = r == 0 ? kSplitLead : 0; c < 4; ++c) wt[r][c] = load_nt16(wrow(r) + c * 1024);
  }
  lds_barrier();  // hand-off: codes and scale
  const float sc = L.scale;
  v4i xq[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) xq[c] = *reinterpret_cast<const v4i*>(L.qs + c * 1024 + lane * 16);
  int acc[RS];
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    acc[r] = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r] = dot16(xq[c], wt[r][c], acc[r]);
  }
  const int total = reduce_to_lanes<RS>(acc, lane);
  float wl = wsr[0], rl = rsr[0];
  uint32_t row = row_of(0);
#pragma unroll
  for (int r = 1; r < RS; ++r) {
    wl = lane == r ? wsr[r] : wl;
    rl = lane == r ? rsr[r] : rl;
    row = lane == r ? row_of(r) : row;
  }
  const float value = dequant(total, sc, wl);
  const float comb = EPI == EPI_RESIDUAL ? bf16_rne(rl + value) : 0.f;
  asm volatile("" ::"v"(value), "v"(comb), "s"(dtype));
  if (lane < RS && row < n) {
    if (out) store_out(out, row, dtype, total, value);
    if (EPI == EPI_RESIDUAL) store_out(combined, row, dtype, total, comb);
  }
}

// linear_swiglu with norm_quantize folded in: NS streaming waves of CS
// consecutive coordinates each (a coordinate: its gate row and its up row,
// 8 KiB), two coordinates in flight per wave, four producer waves.  Lane 0
// writes gate, up (bit-exact linear epilogues) and act = silu_mul(gate, up).
template <int NS, int CS>
__global__ __launch_bounds__((NS + kProdWaves) * kWave) void gemv_swiglu_split(
    const float* x, const float* gain, const int8_t* wg, const float* wsg, const int8_t* wu, const float* wsu,
    uint32_t n, int dtype, void* gate, void* up, void* act, int8_t* q_out, float* scale_out, uint32_t* maxima,
    float* normed) {
  static_assert(CS % 2 == 0, "coordinates go through two register slots");
  __shared__ SplitLds<4096> L;
  const int t = threadIdx.x, lane = t & 63;
  const uint32_t wv = wave_id();
  const int pt = t - NS * kWave;
  if (t == 0) L.count = 0;
  // coordinate k of a streaming wave: (k NS + wave) G + workgroup, so that
  // the streamers of all workgroups sweep one window of the matrices together
  const uint32_t G = gridDim.x;
  auto coord = [&](int k) -> uint32_t { return ((uint32_t)k * NS + wv) * G + xcd_slot(blockIdx.x, G); };
  auto grow = [&](int k) { return wg + (size_t)min(coord(k), n - 1) * 4096 + lane * 16; };
  auto urow = [&](int k) { return wu + (size_t)min(coord(k), n - 1) * 4096 + lane * 16; };
  float v[16], g[16];
  v4i ga[4], ua[4], gb[4], ub[4];
  if (wv >= NS)
    split_load_4096<PROD_NORM>(x, gain, pt, v, g);
  else
#pragma unroll
    for (int i = 0; i < kSplitLead; ++i) ga[i] = load_nt16(grow(0) + i * 1024);
  lds_barrier();
  if (wv >= NS) {
    split_producer_4096<PROD_NORM>(v, g, L, pt, normed, scale_out, maxima);
    lds_barrier();
    split_codes_out(L, pt, q_out);
    return;
  }
  float sg[CS], su[CS];
#pragma unroll
  for (int k = 0; k < CS; ++k) {
    const uint32_t cr = min(coord(k), n - 1);
    sg[k] = wsg[cr];
    su[k] = wsu[cr];
  }
  auto issue = [&](v4i (&gv)[4], v4i (&uv)[4], int k, int from) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i >= from) gv[i] = load_nt16(grow(k) + i * 1024);
      uv[i] = load_nt16(urow(k) + i * 1024);
    }
  };
  issue(ga, ua, 0, kSplitLead);
  issue(gb, ub, 1, 0);
  lds_barrier();  // hand-off
  const float sc = L.scale;
  v4i xq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xq[i] = *reinterpret_cast<const v4i*>(L.qs + i * 1024 + lane * 16);
  auto finish = [&](const v4i (&gv)[4], const v4i (&uv)[4], int k) {
    int ag = 0, au = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ag = dot16(xq[i], gv[i], ag);
      au = dot16(xq[i], uv[i], au);
    }
    const int tg = wave_sum_uniform(ag);
    const int tu = wave_sum_uniform(au);
    const float gv_ = dequant(tg, sc, sg[k]);
    const float uv_ = dequant(tu, sc, su[k]);
    const float av = silu_mul(gv_, uv_);
    asm volatile("" ::"v"(av), "s"(dtype));
    const uint32_t c = coord(k);
    if (c < n && lane == 0) {
      store_out(gate, c, dtype, tg, gv_);
      store_out(up, c, dtype, tu, uv_);
      store_out(act, c, dtype, 0, av);
    }
  };
#pragma unroll
  for (int k = 0; k < CS; k += 2) {
    finish(ga, ua, k);
    if (k + 2 < CS) issue(ga, ua, k + 2, 0);
    finish(gb, ub, k + 1);
    if (k + 3 < CS) issue(gb, ub, k + 3, 0);
  }
}

// The SwiGLU row tail folded into the down GEMV (K = 12,288) that consumes
// its codes: swiglu_row_tail<true>'s work -- the act row's largest
// bits(|act|) (NaN -> 0) folded into maxima[0], then quantize_with_max
// (src/kernels.rs:453-475) with that maximum, s = RN(from_bits(max(m0, row
// max)) / 127), q_j = round(RN(act_j / s)) -- then linear / linear_residual
// on one matrix.  m0 is maxima[0] as a workgroup reads it: the call's value,
// or that value with the row maximum folded in by workgroup 0's atomicMax
// -- max(m0, row max) is the same either way.  Producer thread pt holds
// elements 4 (pt + 256 j) .. + 3 (j < 12): one 16-byte (F32) or 8-byte
// (BF16) load each.  NS streaming waves of RS rows.
constexpr uint32_t kRowtailWidth = 12288;

template <int NS, int RS, int EPI, bool BF16_ACT>
__global__ __launch_bounds__((NS + kProdWaves) * kWave) void gemv_rowtail_split(
    const void* act, uint32_t* maxima, const int8_t* w, const float* ws, uint32_t n, int dtype,
    const float* residual, void* out, void* combined, int8_t* q_out, float* scale_out) {
  constexpr int KC = kRowtailWidth / 1024, J = kRowtailWidth / (4 * kProdWaves * kWave);
  __shared__ SplitLds<kRowtailWidth> L;
  const int t = threadIdx.x, lane = t & 63;
  const uint32_t wv = wave_id();
  const int pt = t - NS * kWave;
  if (t == 0) L.count = 0;
  const uint32_t G = gridDim.x;
  auto row_of = [&](int r) -> uint32_t { return ((uint32_t)r * NS + wv) * G + xcd_slot(blockIdx.x, G); };
  auto wrow = [&](int r) { return w + (size_t)min(row_of(r), n - 1) * kRowtailWidth + lane * 16; };
  uint32_t raw[BF16_ACT ? 2 * J : 4 * J];  // the thread's act values as loaded
  uint32_t m0 = 0;
  v4i wt[RS][KC];
  if (wv < NS) {
#pragma unroll
    for (int c = 0; c < kSplitLead; ++c) wt[0][c] = load_nt16(wrow(0) + c * 1024);
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (BF16_ACT) {
        const v2i d = reinterpret_cast<const v2i*>(act)[pt + 256 * j];
        raw[2 * j] = (uint32_t)d.x;
        raw[2 * j + 1] = (uint32_t)d.y;
      } else {
        const v4i d = reinterpret_cast<const v4i*>(act)[pt + 256 * j];
        raw[4 * j] = (uint32_t)d.x;
        raw[4 * j + 1] = (uint32_t)d.y;
        raw[4 * j + 2] = (uint32_t)d.z;
        raw[4 * j + 3] = (uint32_t)d.w;
      }
    }
    m0 = maxima[0];
  }
  lds_barrier();
  if (wv >= NS) {
    // element i of the thread (i < 4 J): act[4 (pt + 256 (i / 4)) + i % 4]
    auto val = [&](int i) -> float {
      if (!BF16_ACT) return __uint_as_float(raw[i]);
      const uint32_t d = raw[i >> 1];
      return __uint_as_float((i & 1) ? (d & 0xffff0000u) : (d << 16));
    };
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < 4 * J; ++i) bits = max(bits, abs_bits_no_nan(val(i)));
    uint32_t target = 0;
    const uint32_t rmax = block_max_256_with(bits, L.red, pt, [&] { prod_sync(&L.count, target); });
    const float sc = __uint_as_float(max(m0, rmax)) / 127.0f, rc = 1.0f / sc;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float e[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) e[u] = val(4 * j + u);
      int code[4];
      quant_codes(e, sc, rc, code);
      reinterpret_cast<uint32_t*>(L.qs)[pt + 256 * j] = (uint32_t)(code[0] & 0xff) |
                                                          ((uint32_t)(code[1] & 0xff) << 8) |
                                                          ((uint32_t)(code[2] & 0xff) << 16) |
                                                          ((uint32_t)code[3] << 24);
    }
    if (pt == 0) {
      L.scale = sc;
      if (blockIdx.x == 0) {
        atomicMax(maxima, rmax);
        if (scale_out) scale_out[0] = sc;
      }
    }
    lds_barrier();  // hand-off
    split_codes_out(L, pt, q_out);
    return;
  }
  float wsr[RS], rsr[RS];
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const uint32_t er = min(row_of(r), n - 1);
    wsr[r] = ws[er];
    rsr[r] = EPI == EPI_RESIDUAL ? residual[er] : 0.f;
#pragma unroll
    for (int c = r == 0 ? kSplitLead : 0; c < KC; ++c) wt[r][c] = load_nt16(wrow(r) + c * 1024);
  }
  lds_barrier();  // hand-off
  const float sc = L.scale;
  int acc[RS];
#pragma unroll
  for (int r = 0; r < RS; ++r) acc[r] = 0;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    const v4i xq = *reinterpret_cast<const v4i*>(L.qs + c * 1024 + lane * 16);
#pragma unroll
    for (int r = 0; r < RS; ++r) acc[r] = dot16(xq, wt[r][c], acc[r]);
  }
  const int total = reduce_to_lanes<RS>(acc, lane);
  float wl = wsr[0], rl = rsr[0];
  uint32_t row = row_of(0);
#pragma unroll
  for (int r = 1; r < RS; ++r) {
    wl = lane == r ? wsr[r] : wl;
    rl = lane == r ? rsr[r] : rl;
    row = lane == r ? row_of(r) : row;
  }
  const float value = dequant(total, sc, wl);
  const float comb = EPI == EPI_RESIDUAL ? bf16_rne(rl + value) : 0.f;
  asm volatile("" ::"v"(value), "v"(comb), "s"(dtype));
  if (lane < RS && row < n) {
    if (out) store_out(out, row, dtype, total, value);
    if (EPI == EPI_RESIDUAL) store_out(combined, row, dtype, total, comb);
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
// grid-stride sweeps; two rows per wave helps only the small matrices.  M = 1
// at K = 4096 / 12288: gemv_m1_one (one matrix) or gemv_m1 (siblings, or the
// fused selection, whose workgroups carry 16 waves: a quarter of the keys of
// the plain GEMV's 4-wave workgroups).  Otherwise gemv_mt with 4-row groups.
GemvRoute gemv_route(uint32_t m, uint32_t k, const uint32_t* n, int count, bool argmax) {
  GemvRoute r{};
  uint64_t total = 0;
  for (int i = 0; i < count; ++i) total += n[i];
  r.grid_y = 1;
  if (m == 1 && (k == 4096 || k == 12288)) {
    r.family = argmax || count != 1 ? kRouteGemvM1 : kRouteGemvM1One;
    r.rows = k == 4096 && total <= 8192 ? 2 : 1;
    r.kc = (int)(k / 1024);
    r.waves = argmax ? 16 : kGemvWaves;
  } else {
    r.family = kRouteGemvMt;
    r.rows = 4;
    r.mt = (m == 1 || argmax) ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    r.u = r.mt <= 2 ? 4 : 2;
    r.waves = kGemvWaves;
    r.grid_y = (m + r.mt - 1) / r.mt;
  }
  uint64_t groups = 0;
  for (int i = 0; i < count; ++i) groups += (n[i] + r.rows - 1) / r.rows;
  r.grid_x = (uint32_t)((groups + r.waves - 1) / r.waves);
  return r;
}

template <int EPI>
static hipError_t dispatch(hipStream_t st, GemvArgs& a, uint32_t* blocks) {
  const GemvRoute r = gemv_route(a.m, a.k, a.n, a.count, EPI == EPI_ARGMAX);
  uint32_t nn[kMaxGroup];
  for (int i = 0; i < a.count; ++i) nn[i] = a.n[i];
  if (r.family != kRouteGemvMt) {
    if (r.kc == 12) return launch_m1<1, 12, EPI>(st, a, nn, blocks);
    return r.rows == 2 ? launch_m1<2, 4, EPI>(st, a, nn, blocks) : launch_m1<1, 4, EPI>(st, a, nn, blocks);
  }
  if (r.mt == 1) return launch_mt<1, 4, EPI>(st, a, nn, blocks);
  if (r.mt == 2) return launch_mt<2, 4, EPI>(st, a, nn, blocks);
  if (r.mt == 4) return launch_mt<4, 2, EPI>(st, a, nn, blocks);
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

template <int NS, int RS, int EPI, int PROD>
static hipError_t launch_split(hipStream_t st, const ProduceArgs& p) {
  const uint32_t blocks = (p.n + NS * RS - 1) / (NS * RS);
  hipLaunchKernelGGL((gemv_m1_split<NS, RS, EPI, PROD>), dim3(blocks), dim3((NS + kProdWaves) * kWave), 0, st, p.x,
                     p.gain, p.w, p.ws, p.n, p.out_dtype, p.residual, p.out, p.combined, p.q, p.scale, p.maxima,
                     p.normed);
  return hipGetLastError();
}

// Rows per workgroup: 16 (8 streaming waves) up to N = 4096, 24 (12) beyond,
// so that the o (4096) and qkv (6144) projections run one workgroup per CU.
template <int PROD>
static hipError_t launch_produce_epi(hipStream_t st, const ProduceArgs& p) {
  if (p.residual)
    return p.n <= 4096 ? launch_split<8, 2, EPI_RESIDUAL, PROD>(st, p) : launch_split<12, 2, EPI_RESIDUAL, PROD>(st, p);
  return p.n <= 4096 ? launch_split<8, 2, EPI_PLAIN, PROD>(st, p) : launch_split<12, 2, EPI_PLAIN, PROD>(st, p);
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
  // 12 streaming waves of 4 coordinates: one workgroup per CU for 12,288
  constexpr int NS = 12, CS = 4;
  const dim3 grid((a.n + NS * CS - 1) / (NS * CS));
  hipLaunchKernelGGL((gemv_swiglu_split<NS, CS>), grid, dim3((NS + kProdWaves) * kWave), 0, st, p.x, p.gain, a.wg,
                     a.wsg, a.wu, a.wsu, a.n, a.out_dtype, a.gate, a.up, a.act, p.q, p.scale, p.maxima, p.normed);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !row_tail) return e;
  // the norm reset maxima[0] inside the GEMV; the row tail folds into it
  hipLaunchKernelGGL(swiglu_row_tail<true>, dim3(1), dim3(kRowTailThreads), 0, st, a.act, a.n, a.out_dtype,
                     a.maxima, a.q_out, a.scales_out);
  return hipGetLastError();
}

template <int EPI, bool BF16_ACT>
static hipError_t launch_rowtail(hipStream_t st, const RowtailArgs& d) {
  // 8 streaming waves of 2 rows: one workgroup per CU for N = 4096
  constexpr int NS = 8, RS = 2;
  const dim3 grid((d.n + NS * RS - 1) / (NS * RS)), block((NS + kProdWaves) * kWave);
  hipLaunchKernelGGL((gemv_rowtail_split<NS, RS, EPI, BF16_ACT>), grid, block, 0, st, d.act, d.maxima, d.w, d.ws,
                     d.n, d.out_dtype, d.residual, d.out, d.combined, d.q_out, d.scale_out);
  return hipGetLastError();
}

hipError_t launch_gemv_rowtail(hipStream_t st, const RowtailArgs& d) {
  if (d.n == 0 || !d.maxima) return hipErrorInvalidValue;
  const bool bf16 = d.act_dtype == W8A8_OUT_BF16;
  if (d.residual)
    return bf16 ? launch_rowtail<EPI_RESIDUAL, true>(st, d) : launch_rowtail<EPI_RESIDUAL, false>(st, d);
  return bf16 ? launch_rowtail<EPI_PLAIN, true>(st, d) : launch_rowtail<EPI_PLAIN, false>(st, d);
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
