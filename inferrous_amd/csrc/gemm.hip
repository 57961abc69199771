// gemm.hip -- INT8 MFMA GEMM (exact i32 accumulate) for prefill and small
// batches, with the fused per-token x per-channel dequant epilogue.
//
// Reference semantics (crates/inferrous-qwen3/): the M > 1 projections
//   linear_prefill src/kernels.rs:846-931, linear_splitk :932-1034,
//   linear_tiled :1035-1141, linear_large :1142-1289, epilogues
//   :918-930, :1008-1033, :1123-1140, :1249-1288:
//   out[r][c] = bf(RN(RN(f32(sum_k q[r][k] w[c][k]) * asc[r]) * ws[c]))
//
// gfx950 design.  Any k permutation applied identically to A and B leaves
// the exact integer sum unchanged, so each kernel reads both operands with
// one lane -> k map of its own choosing.  Layouts of the two matrix-core
// ops used:
//   v_mfma_i32_16x16x64_i8: per lane a 16-byte A fragment (row lane%16) and
//     a 16-byte B fragment (column lane%16); the 4 x i32 result of lane l
//     holds rows 4*(l/16)+v, column l%16.
//   v_mfma_i32_32x32x32_i8: 16-byte fragments, row / column lane%32; the
//     16 x i32 result of lane l holds rows 8*(v/4)+4*(l/32)+v%4, column l%32.
//
// Kernels:
//  * gemm_dma (k % 128 == 0 and M > 64, or 8 <= M <= 64 when n gives >= 128
//    tiles of 128 columns, wherever gemm_tall's plan does not apply): the
//    prefill GEMM, built on
//    v_mfma_i32_32x32x32_i8 (on gfx950 the 16x16x64 int8 form issues at half
//    its rate), eight waves per workgroup (two per SIMD, so one wave's LDS
//    reads overlap the other's MFMAs).  Operands move global -> LDS with
//    global_load_lds_dwordx4 (no VGPR staging) in 128-byte K stages (whole
//    cache lines) through two rings, activations and weights, the weights
//    requested further ahead; one barrier per stage; the 16-byte chunks of
//    each LDS row are XOR-swizzled so fragment reads spread over the banks.
//    Workgroups are numbered XCD-aware (below).  Tile shape per problem is
//    chosen by the host from the tile count.  With a caller workspace, some
//    shapes run split-K (i32 slabs + splitk_epilogue).
//  * gemm_tall (M <= 256, k % 128 == 0, where its plan applies; M tiles of
//    64, 160 or 256 rows): one M tile holds every activation row, so each
//    weight tile streams from HBM once; the waves hold 32 x 32 output blocks
//    one each (M <= 64) or 32-row slices of all BN columns, and those
//    holding none only move data; activation rows past M are never loaded;
//    split-K on narrow n.
//  * gemm_narrow (M <= 16, or M <= 32 on n <= 4096 at k <= 4096, where the
//    n / 96 tiles are fewer than 224 and k splits into S slices of 128-byte
//    stages): one workgroup owns 16 weight rows; its S waves split K
//    (contiguous slices at S = 4, interleaved 128-byte chunks at S = 8), and
//    each wave streams its share through its own global -> LDS ring (16 weight rows and the live activation rows of a 128-byte stage,
//    global_load_lds_dwordx4: eight whole lines per instruction), so the K
//    loop has no workgroup barrier and no split-K slabs leave the CU.  The S
//    partial 16 x 16 tiles are summed through LDS (exact) and stored by the
//    fused epilogue.
//  * gemm_skinny (small M on narrow n, HBM-bound, 16x16x64 MFMA): one
//    workgroup owns 16 weight rows; its S waves split K and stream their
//    weight fragments straight from HBM into MFMA B operands (no LDS round
//    trip), activation fragments come from L1/L2.  Partial i32 tiles are
//    summed through LDS -- exact.
//  * gemm_tiled (M > 64 with k % 128 != 0): BM x BN output tile, 4 waves,
//    128-byte K stages double-buffered in LDS (row pitch 144 B: a 16-lane
//    ds_read_b128 column touches every bank once), global loads of stage
//    k+1 in flight while stage k feeds the MFMAs.  Workgroups are numbered
//    so that the M tiles sharing one weight panel run on the same XCD
//    (workgroup id mod 8 picks the XCD), so the panel is fetched into that
//    XCD's L2 once.
#include <algorithm>
#include <type_traits>

#include "device_common.hpp"
#include "internal.hpp"

namespace w8a8 {

__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void epilogue_store(const GemmArgs& a, uint32_t r, uint32_t c, int32_t acc) {
  const size_t o = (size_t)r * a.n + c;
  if (a.out_dtype == W8A8_OUT_I32) {
    reinterpret_cast<int32_t*>(a.out)[o] = acc;
    return;
  }
  const float v = dequant(acc, a.asc[r], a.ws[c]);
  if (a.out_dtype == W8A8_OUT_F32) {
    if (a.out) reinterpret_cast<float*>(a.out)[o] = v;
    if (a.residual) reinterpret_cast<float*>(a.combined)[o] = bf16_rne(a.residual[o] + v);
  } else {
    if (a.out) reinterpret_cast<uint16_t*>(a.out)[o] = (uint16_t)(__float_as_uint(v) >> 16);
    if (a.residual)
      reinterpret_cast<uint16_t*>(a.combined)[o] =
          (uint16_t)(__float_as_uint(bf16_rne(a.residual[o] + v)) >> 16);
  }
}

// ---------------------------------------------------------------- skinny
template <int MT, int S, int U>
__global__ __launch_bounds__(64 * S) void gemm_skinny(GemmArgs a) {
  __shared__ int red[S][MT][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t n0 = blockIdx.x * 16;
  const uint32_t m0 = blockIdx.y * 16 * MT;
  const uint32_t K = a.k;
  const uint32_t steps = (K + 63) / 64;
  const uint32_t per = (steps + S - 1) / S;
  const uint32_t s0 = min(wave * per, steps), s1 = min(s0 + per, steps);
  const uint32_t koff = (lane >> 4) * 16;
  const int8_t* wp = a.w + (size_t)min(n0 + (lane & 15), a.n - 1) * K + koff;
  const int8_t* ap[MT];
  bool aok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const uint32_t r = m0 + t * 16 + (lane & 15);
    aok[t] = r < a.m;
    ap[t] = a.q + (size_t)(aok[t] ? r : 0) * K + koff;
  }
  v4i acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = v4i{0, 0, 0, 0};
  for (uint32_t s = s0; s < s1; s += U) {
    v4i wv[U], av[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t kk = (s + u) * 64;
      const bool ok = (s + u < s1) && (kk + koff < K);
      wv[u] = ok ? load_nt16(wp + kk) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < MT; ++t) av[u][t] = (ok && aok[t]) ? load16(ap[t] + kk) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = mfma16(av[u][t], wv[u], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][t][v][lane] = acc[t][v];
  __syncthreads();
  for (int i = threadIdx.x; i < MT * 4 * 64; i += 64 * S) {
    const int l = i & 63, v = (i >> 6) & 3, t = i >> 8;
    int sum = 0;
#pragma unroll
    for (int w = 0; w < S; ++w) sum += red[w][t][v][l];
    const uint32_t r = m0 + t * 16 + 4 * (l >> 4) + v;
    const uint32_t c = n0 + (l & 15);
    if (r < a.m && c < a.n) epilogue_store(a, r, c, sum);
  }
}

// ---------------------------------------------------------------- tiled
template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void gemm_tiled(GemmArgs a, uint32_t tiles_m, uint32_t tiles_n) {
  constexpr int BK = 128;
  constexpr int PITCH = BK + 16;
  constexpr int WAVES_N = BN / WN;
  static_assert((BM / WM) * (BN / WN) == 4, "four waves per workgroup");
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int ACH = BM * (BK / 16) / 256, BCH = BN * (BK / 16) / 256;
  static_assert(ACH >= 1 && BCH >= 1, "tile too small for 256 loaders");
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * PITCH];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * PITCH];

  // XCD-aware numbering: workgroups id, id+8, id+16, ... share an XCD; give
  // each XCD a contiguous run of (n tile, m tile) pairs, m fastest.
  const uint32_t T = tiles_m * tiles_n;
  uint32_t L = blockIdx.x;
  if (T % 8 == 0) L = (blockIdx.x % 8) * (T / 8) + blockIdx.x / 8;
  const uint32_t mt = L % tiles_m, nt = L / tiles_m;
  const uint32_t m0 = mt * BM, n0 = nt * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
  const uint32_t K = a.k, M = a.m, N = a.n;
  const uint32_t KT = (K + BK - 1) / BK;

  v4i ra[ACH], rb[BCH];
  auto gload = [&](uint32_t kt) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int id = tid + i * 256, row = id >> 3, kc = id & 7;
      const uint32_t gm = m0 + row, kk = kt * BK + kc * 16;
      ra[i] = (gm < M && kk < K) ? load16(a.q + (size_t)gm * K + kk) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int id = tid + i * 256, row = id >> 3, kc = id & 7;
      const uint32_t gn = n0 + row, kk = kt * BK + kc * 16;
      rb[i] = (gn < N && kk < K) ? load16(a.w + (size_t)gn * K + kk) : v4i{0, 0, 0, 0};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int id = tid + i * 256, row = id >> 3, kc = id & 7;
      *reinterpret_cast<v4i*>(&As[buf][row * PITCH + kc * 16]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int id = tid + i * 256, row = id >> 3, kc = id & 7;
      *reinterpret_cast<v4i*>(&Bs[buf][row * PITCH + kc * 16]) = rb[i];
    }
  };

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  gload(0);
  sstore(0);
  __syncthreads();
  const int frow = lane & 15, fk = (lane >> 4) * 16;
  for (uint32_t kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      v4i af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const v4i*>(&As[buf][(wm0 + i * 16 + frow) * PITCH + ks * 64 + fk]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const v4i*>(&Bs[buf][(wn0 + j * 16 + frow) * PITCH + ks * 64 + fk]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < KT) sstore(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t r = m0 + wm0 + i * 16 + 4 * (lane >> 4) + v;
        const uint32_t c = n0 + wn0 + j * 16 + (lane & 15);
        if (r < M && c < N) epilogue_store(a, r, c, acc[i][j][v]);
      }
}

// ---------------------------------------------------------------- dma
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// s_waitcnt with vmcnt = N and the other counters left at their maximum
// (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}


#define W8A8_LDS_PTR(p) ((void __attribute__((address_space(3)))*)(p))

// Epilogue modes, resolved at compile time so the unrolled store loop stays
// branch-free: raw accumulators, f32 or BF16 outputs, each optionally with
// the residual sum bf(residual + out).  EP_SLAB is EP_I32 for a split-K slab
// that is streamed: non-temporal stores, read back once by the slab epilogue.
enum { EP_I32 = 0, EP_F32 = 1, EP_BF16 = 2, EP_F32_RES = 3, EP_BF16_RES = 4, EP_SLAB = 5 };
constexpr bool raw_i32(int ep) { return ep == EP_I32 || ep == EP_SLAB; }

// ---------------------------------------------------------------- narrow
// Workgroup b owns output columns [16 b, 16 b + 16) and all M rows (MB
// 16-row blocks).  Wave w sums ST = K / (128 S) of the 128-byte K chunks
// (the host guarantees K % (128 S) == 0): with S = 4 the contiguous slice
// w ST .. w ST + ST - 1, stage s reading chunk w ST + s; with S = 8 the
// waves interleave, stage s reading chunk ((s + b) mod ST) S + w, so that a
// workgroup's eight waves read eight consecutive chunks of every row and
// workgroups start at different chunks (down 4096 x 12288 at M = 2 / 8 / 16,
// graphs of 36 launches on MI355X: 10.90 / 10.93 / 11.98 us against 11.03 /
// 11.27 / 12.32 for contiguous slices; at K = 4096 with S = 4 the
// interleaved order was 0.4-0.8 us slower on qkv and o).  Each wave streams
// its chunks through its own ring of R stages: a stage holds 16 weight rows,
// then 16 MB activation
// rows, 128 bytes each; DMA instruction j fills rows 8j .. 8j + 7, lane l
// chunk l % 8 of row 8j + l / 8 with global chunk (l % 8) ^ (row % 8), so
// that the 16-row fragment reads (lane l: row l % 16) meet eight distinct
// bank groups.  Only the first LAL activation instructions are issued (the
// host picks LAL = ceil(M / 8)); lanes of rows >= M load nothing, so those
// LDS rows hold stale bytes whose products reach only accumulator rows >= M,
// which are never stored.  Weight rows past N re-read row N - 1.  A wave
// reads only its own ring, so the K loop needs no workgroup barrier: each
// stage is waited for with vmcnt (every issued instruction has a live lane,
// so the count is exact), and a slot is refilled only after the previous
// stage's fragment reads have returned.
template <int MB, int LAL, int S, int R>
__global__ __launch_bounds__(64 * S) void gemm_narrow(GemmArgs a) {
  constexpr int ROWS = 16 * (1 + MB);
  constexpr int STAGE = ROWS * 128;
  constexpr int L = 2 + LAL;  // DMA instructions per stage
  constexpr int RING = R * STAGE;
  static_assert(MB >= 1 && LAL >= 1 && LAL <= 2 * MB, "live activation loads");
  static_assert(R >= 2 && (R - 1) * L < 64, "ring depth");
  static_assert(S * RING <= 160 * 1024, "LDS");
  static_assert(S * MB * 4 * 64 * (int)sizeof(int) <= S * RING, "the reduction reuses the rings");
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * RING];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const uint32_t n0 = blockIdx.x * 16, K = a.k, M = a.m, N = a.n;
  const uint32_t ST = K / (128 * S);
  int8_t* const ring = lds + wave * RING;

  const int8_t* src[L];
  bool live[L];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int row = 8 * j + (lane >> 3);
    const size_t chunk = (size_t)(((lane & 7) ^ (row & 7)) * 16);
    if (row < 16) {
      const uint32_t g = n0 + row;
      src[j] = a.w + (size_t)(g < N ? g : N - 1) * K + chunk;
      live[j] = true;
    } else {
      const uint32_t g = (uint32_t)(row - 16);
      live[j] = g < M;
      src[j] = a.q + (size_t)(live[j] ? g : 0) * K + chunk;
    }
  }
  auto load = [&](uint32_t s) {
    int8_t* const base = ring + (s % R) * STAGE;
    const size_t kc = S >= 8 ? (size_t)((s + blockIdx.x) % ST) * S + wave : (size_t)wave * ST + s;
#pragma unroll
    for (int j = 0; j < L; ++j)
      if (live[j])
        __builtin_amdgcn_global_load_lds((const void*)(src[j] + kc * 128),
                                         W8A8_LDS_PTR(base + j * 1024 + lane * 16), 16, 0, 0);
  };

  const int fr = lane & 15, fq = lane >> 4;
  v4i acc[MB];
#pragma unroll
  for (int t = 0; t < MB; ++t) acc[t] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < R - 1; ++s)
    if ((uint32_t)s < ST) load(s);
  for (uint32_t s = 0; s < ST; ++s) {
    if (s + R - 1 < ST) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage s - 1's fragment reads returned
      load(s + R - 1);                                     // into stage s - 1's slot
      wait_vmcnt<(R - 1) * L>();                           // stage s landed
    } else {
      wait_vmcnt<0>();
    }
    const int8_t* const base = ring + (s % R) * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // the stage's two 64-byte k steps
      const int c = 4 * h + fq;
      const v4i b = *(const v4i*)(base + fr * 128 + ((c ^ (fr & 7)) * 16));
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        const int row = 16 + 16 * t + fr;
        const v4i av = *(const v4i*)(base + row * 128 + ((c ^ (row & 7)) * 16));
        acc[t] = mfma16(av, b, acc[t]);
      }
    }
  }
  __syncthreads();  // every wave is done with its ring
  int* const red = reinterpret_cast<int*>(lds);
#pragma unroll
  for (int t = 0; t < MB; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[((wave * MB + t) * 4 + v) * 64 + lane] = acc[t][v];
  __syncthreads();
  // value v of lane l of block t: row 16 t + 4 (l / 16) + v, column n0 + l % 16
  for (int i = threadIdx.x; i < MB * 4 * 64; i += 64 * S) {
    const int l = i & 63, v = (i >> 6) & 3, t = i >> 8;
    int sum = 0;
#pragma unroll
    for (int w = 0; w < S; ++w) sum += red[((w * MB + t) * 4 + v) * 64 + l];
    const uint32_t r = 16 * t + 4 * (l >> 4) + v;
    const uint32_t c = n0 + (l & 15);
    if (r < M && c < N) epilogue_store(a, r, c, sum);
  }
}

// Epilogue of a wave's FM x FN grid of 32x32 accumulator blocks whose top
// left corner is (row0, col0).  Lane l, value v of block (i, j) is row
// row0 + 32i + 8(v / 4) + 4(l / 32) + v % 4, column col0 + 32j + l % 32.
// Every operand the epilogue reads (row scales, column scales, residuals)
// is loaded first, at clamped, always valid addresses, and every store comes
// after the last use of a load: stores count in the same in-order counter
// as loads, so a load issued after a store would wait for the store too.
template <int EP, int FM, int FN>
__device__ __forceinline__ void store_blocks(const GemmArgs& a, const v16i (&acc)[FM][FN], uint32_t row0,
                                             uint32_t col0, int lane) {
  constexpr bool RES = EP == EP_F32_RES || EP == EP_BF16_RES;
  uint32_t rows[FM][16];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) rows[i][v] = row0 + 32 * i + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
  if (raw_i32(EP)) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t c = col0 + 32 * j + (lane & 31);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (rows[i][v] < a.m && c < a.n) {
            int32_t* o = reinterpret_cast<int32_t*>(a.out) + (size_t)rows[i][v] * a.n + c;
            if (EP == EP_SLAB) __builtin_nontemporal_store(acc[i][j][v], o);
            else *o = acc[i][j][v];
          }
    }
    return;
  }
  float asc[FM][16], wsc[FN];
  float res[RES ? FM : 1][RES ? FN : 1][16];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) asc[i][v] = a.asc[min(rows[i][v], a.m - 1)];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const uint32_t cc = min(col0 + 32 * j + (lane & 31), a.n - 1);
    wsc[j] = a.ws[cc];
    if (RES)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) res[i][j][v] = a.residual[(size_t)min(rows[i][v], a.m - 1) * a.n + cc];
  }
  // one wait for every load above, taken unconditionally: a wait first met
  // inside a guarded store would be repeated in each guarded store after it
  wait_vmcnt<0>();
  // The outputs are written non-temporally (no line of them is re-read by
  // this kernel).  Measured on MI355X, graphs of 16 distinct-weight launches
  // with random operands: o at M = 512 16.8 against 17.2-17.4 us, qkv
  // 22.5-22.7 against 23.0-23.3, gate_up at M = 129 30.9 against 31.2-31.4.
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const uint32_t c = col0 + 32 * j + (lane & 31);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t r = rows[i][v];
        const float val = dequant(acc[i][j][v], asc[i][v], wsc[j]);
        if (r >= a.m || c >= a.n) continue;
        const size_t o = (size_t)r * a.n + c;
        if (EP == EP_F32 || EP == EP_F32_RES) {
          if (a.out) __builtin_nontemporal_store(val, reinterpret_cast<float*>(a.out) + o);
          if (RES) reinterpret_cast<float*>(a.combined)[o] = bf16_rne(res[RES ? i : 0][RES ? j : 0][v] + val);
        } else {
          if (a.out)
            __builtin_nontemporal_store((uint16_t)(__float_as_uint(val) >> 16), reinterpret_cast<uint16_t*>(a.out) + o);
          if (RES)
            reinterpret_cast<uint16_t*>(a.combined)[o] =
                (uint16_t)(__float_as_uint(bf16_rne(res[RES ? i : 0][RES ? j : 0][v] + val)) >> 16);
        }
      }
  }
}

// Prefill GEMM.  Workgroup = 8 waves (two per SIMD: while one wave waits on
// LDS the other keeps the matrix core busy), output tile BM x BN, wave tile
// WM x WN built from 32x32 MFMA blocks.  K advances in 128-byte stages, so
// every DMA row request is one whole 128-byte cache line.
//
// LDS holds two rings: activations (A, BM rows of 128 bytes per stage, SA
// slots) and weights (B, BN rows, SB >= SA slots).  Weight lines mostly miss
// L2, so they can be requested further ahead than the activation lines,
// which every workgroup shares.  Batch(kt) = {A(kt + SA - 1), B(kt + SB - 1)}
// is issued during stage kt (A first) into the slots stage kt - 1 released.
// Loads complete in issue order, so at the end of stage kt "A(kt + 1) and
// B(kt + 1) have landed" means: at most the loads issued after A(kt + 1)
// remain -- the B half of its batch when SB > SA (when SB == SA that half is
// B(kt + 1) itself and must land too), plus the SA - 2 whole batches after
// it.
//
// 16-byte chunk c of LDS row r sits at chunk c ^ ((r >> 1) & 7): sixteen
// consecutive rows (two per 256-byte bank window) of one fragment read then
// hit sixteen different 16-byte bank groups.  Sub-step i of a stage covers
// k bytes [32i, 32i + 32): lane l (row / column l % 32, half h = l / 32)
// reads chunk 2i + h -- the same lane -> k map for A and B.
template <int BM, int BN, int WM, int WN, int SA, int SB, int EP, bool ROT = false>
__global__ __launch_bounds__(512) void gemm_dma(GemmArgs a, uint32_t tiles_m, uint32_t tiles_n,
                                                uint32_t splits) {
  constexpr int WAVES_N = BN / WN;
  static_assert((BM / WM) * (BN / WN) == 8, "eight waves per workgroup");
  static_assert(WM % 32 == 0 && WN % 32 == 0 && BM % 64 == 0 && BN % 64 == 0, "tile shape");
  static_assert(SA >= 2 && SB >= SA && SB >= 3 && SB <= 8, "ring depths");
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int LA = BM / 64, LB = BN / 64;  // DMA loads (8 rows x 128 B) per wave per stage
  constexpr int L = LA + LB;
  constexpr int ASL = BM * 128, BSL = BN * 128;
  static_assert(SA * ASL + SB * BSL <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) int8_t lds[SA * ASL + SB * BSL];
  int8_t* const ldsA = lds;
  int8_t* const ldsB = lds + SA * ASL;

  // Split-K (splits > 1, EP_SLAB or EP_I32): workgroup (tile, split) sums K range
  // [split * K / splits, (split + 1) * K / splits) into i32 slab `split` of
  // a.out; a separate epilogue kernel adds the slabs (exact) and dequantizes.
  const uint32_t T = tiles_m * tiles_n, G = T * splits;
  uint32_t Lt = blockIdx.x;
  if (G % 8 == 0) Lt = (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8;
  const uint32_t split = Lt / T;
  Lt %= T;
  const uint32_t m0 = (Lt % tiles_m) * BM, n0 = (Lt / tiles_m) * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
  const uint32_t K = a.k, KT = K / 128 / splits;
  const size_t kbase = (size_t)split * KT * 128;
  if (raw_i32(EP)) a.out = reinterpret_cast<int32_t*>(a.out) + (size_t)split * a.m * a.n;

  // Sources of this wave's DMA loads (8 rows each); rows past M / N re-read
  // row 0 (their products only reach accumulator cells that are never
  // stored).  Lane l fills LDS chunk l % 8 of row l / 8 with global chunk
  // (l % 8) ^ key(row).
  const int8_t* srcA[LA];
  const int8_t* srcB[LB];
#pragma unroll
  for (int j = 0; j < LA; ++j) {
    const int row = 8 * (wave * LA + j) + (lane >> 3);
    const uint32_t g = m0 + row;
    srcA[j] = a.q + (size_t)(g < a.m ? g : 0) * K + kbase + ((lane & 7) ^ ((row >> 1) & 7)) * 16;
  }
#pragma unroll
  for (int j = 0; j < LB; ++j) {
    const int row = 8 * (wave * LB + j) + (lane >> 3);
    const uint32_t g = n0 + row;
    srcB[j] = a.w + (size_t)(g < a.n ? g : 0) * K + kbase + ((lane & 7) ^ ((row >> 1) & 7)) * 16;
  }
  // ROT: stage kt reads global K chunk (kt + rot) mod KT, rot = tile mod KT.
  const uint32_t rot = ROT ? Lt % KT : 0;
  auto kc = [&](uint32_t kt) -> size_t {
    const uint32_t c = kt + rot;
    return (size_t)(c >= KT ? c - KT : c) * 128;
  };
  auto loadA = [&](uint32_t kt, int j) {
    __builtin_amdgcn_global_load_lds((const void*)(srcA[j] + kc(kt)),
                                     W8A8_LDS_PTR(ldsA + (kt % SA) * ASL + (wave * LA + j) * 1024 + lane * 16),
                                     16, 0, 0);
  };
  auto loadB = [&](uint32_t kt, int j) {
    __builtin_amdgcn_global_load_lds((const void*)(srcB[j] + kc(kt)),
                                     W8A8_LDS_PTR(ldsB + (kt % SB) * BSL + (wave * LB + j) * 1024 + lane * 16),
                                     16, 0, 0);
  };
  // Batch(kt), A first.
  auto batch = [&](uint32_t kt) {
    if (kt + SA - 1 < KT)
#pragma unroll
      for (int j = 0; j < LA; ++j) loadA(kt + SA - 1, j);
    if (kt + SB - 1 < KT)
#pragma unroll
      for (int j = 0; j < LB; ++j) loadB(kt + SB - 1, j);
  };

  const int fr = lane & 31, fh = lane >> 5;
  int off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) off[i] = fr * 128 + (((2 * i + fh) ^ ((fr >> 1) & 7)) * 16);
  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};
  auto rd = [&](uint32_t kt, int i, v4i (&af)[FM], v4i (&bf)[FN]) {
    const int8_t* ba = ldsA + (kt % SA) * ASL;
    const int8_t* bb = ldsB + (kt % SB) * BSL;
#pragma unroll
    for (int f = 0; f < FM; ++f) af[f] = *(const v4i*)(ba + (wm0 + 32 * f) * 128 + off[i]);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *(const v4i*)(bb + (wn0 + 32 * j) * 128 + off[i]);
  };
  auto mm = [&](const v4i (&af)[FM], const v4i (&bf)[FN]) {
#pragma unroll
    for (int f = 0; f < FM; ++f)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[f][j] = mfma32(af[f], bf[j], acc[f][j]);
  };

  // Prologue: stages 0 .. SB - 2 (A only up to SA - 2), stage by stage, A
  // before B; then wait for stage 0.
#pragma unroll
  for (int s = 0; s < SB - 1; ++s) {
    if (s >= (int)KT) break;
    if (s < SA - 1)
#pragma unroll
      for (int j = 0; j < LA; ++j) loadA(s, j);
#pragma unroll
    for (int j = 0; j < LB; ++j) loadB(s, j);
  }
  if (KT >= (uint32_t)SB - 1) wait_vmcnt<(SA - 2) * LA + (SB - 2) * LB>();
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  v4i a0[FM], b0[FN], a1[FM], b1[FN];
  batch(0);
  rd(0, 0, a0, b0);
  // Fragments of the next sub-step are read while the current one's MFMAs
  // run.  The loop body has no branch between a read and its use, so the
  // compiler's LDS waits keep the newest reads in flight.
  for (uint32_t kt = 0; kt + 1 < KT; ++kt) {
    rd(kt, 1, a1, b1);
    mm(a0, b0);
    rd(kt, 2, a0, b0);
    mm(a1, b1);
    rd(kt, 3, a1, b1);
    mm(a0, b0);
    // A(kt + 1), B(kt + 1) landed (every load counted here exists while batch
    // kt was complete)
    if (kt + SB - 1 < KT) wait_vmcnt<(SB > SA ? LB : 0) + (SA - 2) * L>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's reads of stage kt returned
    __builtin_amdgcn_s_barrier();         // all waves: stage kt + 1 landed, stage kt read
    batch(kt + 1);                        // into the slots stage kt released
    rd(kt + 1, 0, a0, b0);
    mm(a1, b1);
  }
  rd(KT - 1, 1, a1, b1);
  mm(a0, b0);
  rd(KT - 1, 2, a0, b0);
  mm(a1, b1);
  rd(KT - 1, 3, a1, b1);
  mm(a0, b0);
  mm(a1, b1);

  store_blocks<EP, FM, FN>(a, acc, m0 + wm0, n0 + wn0, lane);
}

// Unsplit launches rotate each workgroup's K order (stage kt reads K chunk
// (kt + tile) mod KT; the i32 sums are exact in any order, so outputs are
// bit-identical).  Otherwise every workgroup reads the same 128-byte column
// of its 4 KiB weight rows at the same time.  Measured on MI355X (graphs of 16
// distinct-weight launches): gate_up 24576 x 4096 at M = 64 22.2 against
// 25.1 us, M = 100 33.8 against 35.2, M = 129 29.4-29.7 against 30.3-31.4,
// M = 193 32.8 against 34.5-35.0, M = 300 51.7-53.3 against 54.2-54.8,
// M = 512 54.6-56.1 against 56.0-58.8; qkv at M = 512 21.9-22.5 against
// 22.3-22.7; o level.  In the 36-layer prefill graphs, where each gate_up
// follows qkv and o, the M = 512 and M = 129 totals came out level (A/B on
// one box) while the ragged gate_up at M = 16 went from 4.20 to 4.85 TB/s.
// Split-K launches, whose slabs already start at different K offsets,
// measured level or up to 1.3% slower rotated, and keep the order.
constexpr bool kRotateK = true;

// The residual epilogue holds a residual per accumulator; with a 64 x 96
// wave tile that is 96 more registers than the kernel has, and it spills.
// Such tiles take no residual (launch_gemm routes residual outputs to
// 128-row tiles).
template <int WM, int WN>
constexpr bool kResidualTile = WM * WN <= 32 * 96;

template <int BM, int BN, int WM, int WN, int SA, int SB>
static hipError_t launch_dma(hipStream_t st, const GemmArgs& a) {
  const uint32_t tm = (a.m + BM - 1) / BM, tn = (a.n + BN - 1) / BN;
  const dim3 grid(tm * tn), block(512);
  if (a.out_dtype == W8A8_OUT_I32) {
    hipLaunchKernelGGL((gemm_dma<BM, BN, WM, WN, SA, SB, EP_I32, kRotateK>), grid, block, 0, st, a, tm, tn, 1u);
  } else if (a.residual) {
    if constexpr (kResidualTile<WM, WN>) {
      if (a.out_dtype == W8A8_OUT_F32)
        hipLaunchKernelGGL((gemm_dma<BM, BN, WM, WN, SA, SB, EP_F32_RES, kRotateK>), grid, block, 0, st, a, tm, tn, 1u);
      else
        hipLaunchKernelGGL((gemm_dma<BM, BN, WM, WN, SA, SB, EP_BF16_RES, kRotateK>), grid, block, 0, st, a, tm, tn, 1u);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (a.out_dtype == W8A8_OUT_F32) {
    hipLaunchKernelGGL((gemm_dma<BM, BN, WM, WN, SA, SB, EP_F32, kRotateK>), grid, block, 0, st, a, tm, tn, 1u);
  } else {
    hipLaunchKernelGGL((gemm_dma<BM, BN, WM, WN, SA, SB, EP_BF16, kRotateK>), grid, block, 0, st, a, tm, tn, 1u);
  }
  return hipGetLastError();
}

// Cache policy of a load streamed once (the weights of a single M tile): the
// non-temporal bit, so the lines do not displace the activations that every
// workgroup re-reads from L2.
constexpr int kCpolNT = 2;

// s_waitcnt vmcnt(n) for a wave-uniform n known only at run time (n <= 20).
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    case 8: wait_vmcnt<8>(); break;
    case 9: wait_vmcnt<9>(); break;
    case 10: wait_vmcnt<10>(); break;
    case 11: wait_vmcnt<11>(); break;
    case 12: wait_vmcnt<12>(); break;
    case 13: wait_vmcnt<13>(); break;
    case 14: wait_vmcnt<14>(); break;
    case 15: wait_vmcnt<15>(); break;
    case 16: wait_vmcnt<16>(); break;
    case 17: wait_vmcnt<17>(); break;
    case 18: wait_vmcnt<18>(); break;
    case 19: wait_vmcnt<19>(); break;
    default: wait_vmcnt<20>(); break;
  }
}

// Prefill / small-batch GEMM for M <= MA (gemm_tall, MA = 64, 160 or 256).  One M tile
// of MA rows holds every activation row, so each weight tile is read from
// HBM once, and no DMA or MFMA goes to a second M tile holding a few rows.
// MA = 160 and 256: the eight waves are stacked along M (wave w: rows
// 32w .. 32w + 31, all BN columns), so a wave reads one activation fragment
// per k step for its BN / 32 MFMAs.  MA = 64 (M <= 64, one or two 32-row
// blocks): the 32 x 32 output blocks are dealt to the waves one each (block
// b = row block * BN / 32 + column block goes to wave b), so the SIMDs (wave
// w runs on SIMD w % 4) share the MFMAs instead of one or two waves holding
// them all.  Measured on MI355X, graphs of 16 distinct-weight launches with
// random operands, rows-per-wave -> one block per wave: at M = 16 qkv 11.7
// -> 10.6 us, o 9.3 -> 8.6, gate_up 21.0-21.4 -> 18.1, down 15.6 -> 13.8;
// at M = 64 qkv 13.0 -> 12.0, o 10.9 -> 10.4, gate_up 22.1-23.3 -> 20.0-20.4,
// down 17.6-18.2 -> 16.3.  With more row blocks the same dealing reads twice
// the LDS fragment bytes per MFMA for no better balance (M = 129: level;
// M = 200: gate_up 33.0 -> 37.8), so those tiles keep rows per wave.
// A wave that holds no block only moves data.
//
// Rings as in gemm_dma: activations (SA slots of MA rows; the lines are
// shared by every workgroup and come from L2 or MALL) and weights (SB slots;
// the lines come from HBM and are read once, non-temporal).  With few MFMAs
// per stage the stage is short, so both rings look several stages ahead.
// Loads complete in issue order, so a weight load issued before an
// activation load has to land before that activation's wait: weight slots
// beyond the activation ring's depth add no lookahead, and most plans use
// equal depths.
//
// A stage's DMA instructions (8 rows x 128 bytes each) are dealt to the
// waves round-robin, separately for the ceil(M / 8) activation row groups --
// rows past the last group are never loaded -- and the BN / 8 weight row
// groups, so a wave issues na activation and nb weight instructions per stage
// and counts its waits with its own na, nb.  During stage kt it issues
// A(kt + SA - 1), then B(kt + SB - 1).
// Split-K as in gemm_dma: workgroup (tile, split) writes i32 slab `split`.
// TIMED (diagnostics only, w8a8_diag_gemm_timeline): every wave also
// records the 100 MHz device clock at its start, once stage 0 has landed
// (the prologue), after its last MFMA / DMA issue, and once its stores are
// acknowledged, into stamps[4 g .. 4 g + 3] (g = workgroup * 8 + wave).
template <int BN, int SA, int SB, int MA, int EP, bool ROT = false, bool TIMED = false>
__global__ __launch_bounds__(512) void gemm_tall(GemmArgs a, uint32_t tiles_n, uint32_t splits,
                                                 uint64_t* stamps) {
  uint64_t ts[4] = {0, 0, 0, 0};
  if constexpr (TIMED) ts[0] = __builtin_amdgcn_s_memrealtime();
  constexpr int FN = BN / 32;
  constexpr int ASL = MA * 128, BSL = BN * 128;
  constexpr uint32_t NB = BN / 8;
  constexpr int kMaxA = (MA / 8 + 7) / 8, kMaxB = (NB + 7) / 8;
  static_assert(BN % 32 == 0 && BN <= 128 && MA % 32 == 0 && MA <= 256, "tile");
  static_assert(SA >= 2 && SB >= SA && SA * ASL + SB * BSL <= 160 * 1024, "LDS");
  static_assert((SB > SA ? kMaxB : 0) + (SA - 2) * (kMaxA + kMaxB) <= 20 &&
                    (SA - 2) * kMaxA + (SB - 2) * kMaxB <= 20,
                "wait range");
  __shared__ __attribute__((aligned(1024))) int8_t lds[SA * ASL + SB * BSL];
  int8_t* const ldsA = lds;
  int8_t* const ldsB = lds + SA * ASL;

  const uint32_t G = tiles_n * splits;
  uint32_t Lt = blockIdx.x;
  if (G % 8 == 0) Lt = (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8;
  const uint32_t split = Lt / tiles_n;
  const uint32_t n0 = (Lt % tiles_n) * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const uint32_t K = a.k, KT = K / 128 / splits;
  const size_t kbase = (size_t)split * KT * 128;
  if (raw_i32(EP)) a.out = reinterpret_cast<int32_t*>(a.out) + (size_t)split * a.m * a.n;

  // This wave's DMA instructions: activation row groups w, w + 8, ... below
  // ceil(M / 8), weight row groups w, w + 8, ... below BN / 8.  Lane l fills
  // LDS chunk l % 8 of row l / 8 with global chunk (l % 8) ^ key(row).
  const uint32_t NA = (a.m + 7) / 8;
  const int na = (int)((NA + 7 - (uint32_t)wave) / 8);
  const int nb = (int)((NB + 7 - (uint32_t)wave) / 8);
  const int8_t* srcA[kMaxA];
  const int8_t* srcB[kMaxB];
#pragma unroll
  for (int j = 0; j < kMaxA; ++j) {
    const uint32_t row = 8 * (wave + 8 * j) + (lane >> 3);
    srcA[j] = a.q + (size_t)min(row, a.m - 1) * K + kbase + ((lane & 7) ^ ((row >> 1) & 7)) * 16;
  }
#pragma unroll
  for (int j = 0; j < kMaxB; ++j) {
    const uint32_t br = 8 * (wave + 8 * j) + (lane >> 3);  // row within the weight tile
    srcB[j] = a.w + (size_t)min(n0 + br, a.n - 1) * K + kbase + ((lane & 7) ^ ((br >> 1) & 7)) * 16;
  }
  // ROT: stage kt reads global K chunk (kt + rot) mod KT, rot = Lt mod KT, so
  // the workgroups do not all read the same 128-byte column of their weight
  // rows at once.
  const uint32_t rot = ROT ? Lt % KT : 0;
  auto kc = [&](uint32_t kt) -> size_t {
    const uint32_t c = kt + rot;
    return (size_t)(c >= KT ? c - KT : c) * 128;
  };
  auto issueA = [&](uint32_t kt) {
#pragma unroll
    for (int j = 0; j < kMaxA; ++j)
      if (j < na)
        __builtin_amdgcn_global_load_lds((const void*)(srcA[j] + kc(kt)),
                                         W8A8_LDS_PTR(ldsA + (kt % SA) * ASL + 1024 * (wave + 8 * j) + lane * 16),
                                         16, 0, 0);
  };
  auto issueB = [&](uint32_t kt) {
#pragma unroll
    for (int j = 0; j < kMaxB; ++j)
      if (j < nb)
        __builtin_amdgcn_global_load_lds((const void*)(srcB[j] + kc(kt)),
                                         W8A8_LDS_PTR(ldsB + (kt % SB) * BSL + 1024 * (wave + 8 * j) + lane * 16),
                                         16, 0, kCpolNT);
  };
  auto batch = [&](uint32_t kt) {
    if (kt + SA - 1 < KT) issueA(kt + SA - 1);
    if (kt + SB - 1 < KT) issueB(kt + SB - 1);
  };
  // end of stage kt: A(kt + 1) and B(kt + 1) landed; in flight may remain the
  // B half of A(kt + 1)'s batch (when SB > SA) and the SA - 2 whole batches
  // after it
  auto wait_next = [&](uint32_t kt) {
    if (kt + SB - 1 < KT) wait_vmcnt_dyn((SB > SA ? nb : 0) + (SA - 2) * (na + nb));
    else wait_vmcnt<0>();
  };

  const int fr = lane & 31, fh = lane >> 5;
  int off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) off[i] = fr * 128 + (((2 * i + fh) ^ ((fr >> 1) & 7)) * 16);
  // Stage pipeline shared by both mappings: fragments of sub-step i + 1 are
  // read while the MFMAs of sub-step i issue.  rd(kt, i, f) reads sub-step i
  // of stage kt into f; mm(f) issues its MFMAs.
  auto pipeline = [&](auto& f0, auto& f1, auto rd, auto mm) {
    batch(0);
    rd(0, 0, f0);
    for (uint32_t kt = 0; kt + 1 < KT; ++kt) {
      rd(kt, 1, f1);
      mm(f0);
      rd(kt, 2, f0);
      mm(f1);
      rd(kt, 3, f1);
      mm(f0);
      wait_next(kt);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's reads of stage kt returned
      __builtin_amdgcn_s_barrier();
      batch(kt + 1);
      rd(kt + 1, 0, f0);
      mm(f1);
    }
    rd(KT - 1, 1, f1);
    mm(f0);
    rd(KT - 1, 2, f0);
    mm(f1);
    rd(KT - 1, 3, f1);
    mm(f0);
    mm(f1);
  };
  // rows past M, or no block: this wave only moves its share of the data
  auto move_only = [&]() {
    batch(0);
    for (uint32_t kt = 0; kt + 1 < KT; ++kt) {
      wait_next(kt);
      __builtin_amdgcn_s_barrier();
      batch(kt + 1);
    }
  };

  // Prologue: stages 0 .. SB - 2 (activations up to SA - 2), stage by stage;
  // then wait for A(0) and B(0).
  for (int s = 0; s < SB - 1; ++s) {
    if (s >= (int)KT) break;
    if (s < SA - 1) issueA(s);
    issueB(s);
  }
  if (KT >= (uint32_t)SB - 1) wait_vmcnt_dyn((SA - 2) * na + (SB - 2) * nb);
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  if constexpr (TIMED) ts[1] = __builtin_amdgcn_s_memrealtime();
  auto stamp_stream_end = [&]() {
    if constexpr (TIMED) ts[2] = __builtin_amdgcn_s_memrealtime();
  };

  if constexpr (MA == 64) {
    // one 32 x 32 block per wave: block `wave` of the (M / 32) x FN grid
    const uint32_t T = (a.m + 31) / 32 * FN;
    static_assert(2 * FN <= 8, "one block per wave");
    if ((uint32_t)wave < T) {
      const uint32_t mb = (uint32_t)wave / FN, nbk = (uint32_t)wave % FN;
      const int8_t* const aa = ldsA + mb * 32 * 128;
      const int8_t* const bb = ldsB + nbk * 32 * 128;
      struct Frag { v4i a, b; };
      v16i acc = v16i{};
      Frag f0, f1;
      pipeline(f0, f1,
               [&](uint32_t kt, int i, Frag& f) {
                 f.a = *(const v4i*)(aa + (kt % SA) * ASL + off[i]);
                 f.b = *(const v4i*)(bb + (kt % SB) * BSL + off[i]);
               },
               [&](const Frag& f) { acc = mfma32(f.a, f.b, acc); });
      stamp_stream_end();
      const v16i blocks[1][1] = {{acc}};
      store_blocks<EP, 1, 1>(a, blocks, 32 * mb, n0 + 32 * nbk, lane);
    } else {
      move_only();
      stamp_stream_end();
    }
  } else {
    if (32u * wave < a.m) {
      struct Frag { v4i a, b[FN]; };
      v16i acc[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[j] = v16i{};
      Frag f0, f1;
      pipeline(f0, f1,
               [&](uint32_t kt, int i, Frag& f) {
                 f.a = *(const v4i*)(ldsA + (kt % SA) * ASL + (32 * wave) * 128 + off[i]);
                 const int8_t* bb = ldsB + (kt % SB) * BSL;
#pragma unroll
                 for (int j = 0; j < FN; ++j) f.b[j] = *(const v4i*)(bb + (32 * j) * 128 + off[i]);
               },
               [&](const Frag& f) {
#pragma unroll
                 for (int j = 0; j < FN; ++j) acc[j] = mfma32(f.a, f.b[j], acc[j]);
               });
      stamp_stream_end();
      const v16i (&blocks)[1][FN] = *reinterpret_cast<const v16i(*)[1][FN]>(&acc);
      store_blocks<EP, 1, FN>(a, blocks, 32 * wave, n0, lane);
    } else {
      move_only();
      stamp_stream_end();
    }
  }
  if constexpr (TIMED) {
    __builtin_amdgcn_s_waitcnt(0);
    ts[3] = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
      uint64_t* o = stamps + ((size_t)blockIdx.x * 8 + wave) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = ts[i];
    }
  }
}

constexpr uint32_t kMaxSplits = 4;  // split-K plans use 2 or 4 slabs

// A slab quad; NT: the slabs were streamed (EP_SLAB) and are read once.
template <bool NT>
__device__ __forceinline__ v4i load_slab(const int32_t* p) {
  if (NT) return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
  return *reinterpret_cast<const v4i*>(p);
}

// Split-K epilogue: out[r][c] = epilogue(sum over slabs of partials[s][r][c]).
// The i32 sum is exact in any order.  blockIdx.y walks rows (the row scale is
// one scalar load), each thread four consecutive columns (n % 4 == 0), so the
// slab, weight-scale and residual loads are all issued up front.
template <int EP, bool NT>
__global__ __launch_bounds__(256) void splitk_epilogue(GemmArgs a, const int32_t* __restrict__ partials,
                                                        uint32_t splits) {
  constexpr bool RES = EP == EP_F32_RES || EP == EP_BF16_RES;
  const size_t mn = (size_t)a.m * a.n;
  const uint32_t c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= a.n) return;
  float wsc[4] = {0.f, 0.f, 0.f, 0.f};
  if (EP != EP_I32)
#pragma unroll
    for (int j = 0; j < 4; ++j) wsc[j] = a.ws[c + j];
  for (uint32_t r = blockIdx.y; r < a.m; r += gridDim.y) {
    const size_t i = (size_t)r * a.n + c;
    // every operand of the row first -- up to kMaxSplits slabs (slab index
    // clamped, surplus slabs masked), the row scale, the residuals -- so one
    // load round trip covers them; the stores come last
    v4i part[kMaxSplits];
#pragma unroll
    for (uint32_t s = 0; s < kMaxSplits; ++s)
      part[s] = load_slab<NT>(partials + min(s, splits - 1) * mn + i);
    const float asc = EP != EP_I32 ? a.asc[r] : 0.f;
    float res[4] = {0.f, 0.f, 0.f, 0.f};
    if (RES)
#pragma unroll
      for (int j = 0; j < 4; ++j) res[j] = a.residual[i + j];
    v4i acc = part[0];
#pragma unroll
    for (uint32_t s = 1; s < kMaxSplits; ++s)
      if (s < splits) acc += part[s];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const size_t o = i + j;
      if (EP == EP_I32) {
        reinterpret_cast<int32_t*>(a.out)[o] = acc[j];
        continue;
      }
      const float v = dequant(acc[j], asc, wsc[j]);
      if (EP == EP_F32 || EP == EP_F32_RES) {
        if (a.out) reinterpret_cast<float*>(a.out)[o] = v;
        if (RES) reinterpret_cast<float*>(a.combined)[o] = bf16_rne(res[j] + v);
      } else {
        if (a.out) reinterpret_cast<uint16_t*>(a.out)[o] = (uint16_t)(__float_as_uint(v) >> 16);
        if (RES)
          reinterpret_cast<uint16_t*>(a.combined)[o] = (uint16_t)(__float_as_uint(bf16_rne(res[j] + v)) >> 16);
      }
    }
  }
}

// The same epilogue with 8 columns per thread, for n % 8 == 0 and 16-byte
// aligned scales, residuals and outputs: every operand moves in 16-byte
// loads and stores (one store of 8 BF16 values), so a row costs a quarter of
// the 4-column kernel's store instructions.
template <int EP, bool NT>
__global__ __launch_bounds__(256) void splitk_epilogue8(GemmArgs a, const int32_t* __restrict__ partials,
                                                         uint32_t splits) {
  constexpr bool RES = EP == EP_F32_RES || EP == EP_BF16_RES;
  constexpr bool F32 = EP == EP_F32 || EP == EP_F32_RES;
  const size_t mn = (size_t)a.m * a.n;
  const uint32_t c = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= a.n) return;
  float wsc[8] = {};
  if (EP != EP_I32) {
    const v4i w0 = *reinterpret_cast<const v4i*>(a.ws + c), w1 = *reinterpret_cast<const v4i*>(a.ws + c + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wsc[j] = __int_as_float(w0[j]);
      wsc[4 + j] = __int_as_float(w1[j]);
    }
  }
  for (uint32_t r = blockIdx.y; r < a.m; r += gridDim.y) {
    const size_t i = (size_t)r * a.n + c;
    // every operand of the row first (slab index clamped, surplus slabs
    // masked), the stores last
    v4i p0[kMaxSplits], p1[kMaxSplits];
#pragma unroll
    for (uint32_t s = 0; s < kMaxSplits; ++s) {
      const int32_t* ps = partials + min(s, splits - 1) * mn + i;
      p0[s] = load_slab<NT>(ps);
      p1[s] = load_slab<NT>(ps + 4);
    }
    const float asc = EP != EP_I32 ? a.asc[r] : 0.f;
    v4i r0 = {0, 0, 0, 0}, r1 = {0, 0, 0, 0};
    if (RES) {
      r0 = *reinterpret_cast<const v4i*>(a.residual + i);
      r1 = *reinterpret_cast<const v4i*>(a.residual + i + 4);
    }
    v4i s0 = p0[0], s1 = p1[0];
#pragma unroll
    for (uint32_t s = 1; s < kMaxSplits; ++s)
      if (s < splits) {
        s0 += p0[s];
        s1 += p1[s];
      }
    if (EP == EP_I32) {
      int32_t* o = reinterpret_cast<int32_t*>(a.out) + i;
      *reinterpret_cast<v4i*>(o) = s0;
      *reinterpret_cast<v4i*>(o + 4) = s1;
      continue;
    }
    float v[8], cmb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = dequant(j < 4 ? s0[j] : s1[j - 4], asc, wsc[j]);
      if (RES) cmb[j] = bf16_rne(__int_as_float(j < 4 ? r0[j] : r1[j - 4]) + v[j]);
    }
    if (F32) {
      if (a.out) {
        float* o = reinterpret_cast<float*>(a.out) + i;
        *reinterpret_cast<v4i*>(o) = v4i{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]),
                                         __float_as_int(v[3])};
        *reinterpret_cast<v4i*>(o + 4) = v4i{__float_as_int(v[4]), __float_as_int(v[5]), __float_as_int(v[6]),
                                             __float_as_int(v[7])};
      }
      if (RES) {
        float* o = reinterpret_cast<float*>(a.combined) + i;
        *reinterpret_cast<v4i*>(o) = v4i{__float_as_int(cmb[0]), __float_as_int(cmb[1]), __float_as_int(cmb[2]),
                                         __float_as_int(cmb[3])};
        *reinterpret_cast<v4i*>(o + 4) = v4i{__float_as_int(cmb[4]), __float_as_int(cmb[5]),
                                             __float_as_int(cmb[6]), __float_as_int(cmb[7])};
      }
    } else {
      // BF16 values are the high halves of the BF16-valued floats
      v4i ob, cb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ob[j] = (int)((__float_as_uint(v[2 * j]) >> 16) | (__float_as_uint(v[2 * j + 1]) & 0xFFFF0000u));
        cb[j] = (int)((__float_as_uint(cmb[2 * j]) >> 16) | (__float_as_uint(cmb[2 * j + 1]) & 0xFFFF0000u));
      }
      if (a.out) *reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(a.out) + i) = ob;
      if (RES) *reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(a.combined) + i) = cb;
    }
  }
}

// gemm_dma's split-K plan (128 x 128 tiles, two slabs): M > 256 at K >= 8192,
// the down projection's few, long tiles (measured on MI355X at M = 300 and
// 512).  gemm_tall's plan covers M <= 256.
static bool split_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t& splits) {
  if (m <= 256 || k < 8192 || k % 128 != 0 || n % 4 != 0) return false;
  const uint32_t kt = k / 128;
  splits = 2;
  return kt % splits == 0 && kt / splits >= 4;
}

// gemm_narrow's plan: S = 4 waves below K = 8192 and 8 from there (each wave
// keeps eight or more 128-byte stages), R-deep rings, MB 16-row blocks, LAL
// = ceil(M / 8) activation DMA loads per stage.  It takes M <= 16 on the
// narrow shapes, and M <= 32 where one workgroup per 16 columns fits the
// CUs once at K <= 4096; the wide shapes (n / 96 >= 224 tiles) keep
// gemm_tall's unsplit 96-column tiles.  Measured on MI355X, graphs of 36
// distinct-weight launches, random operands, against the routes it
// replaced (gemm_tall split-K 4 with its slab epilogue launch, gemm_skinny),
// bit-identical outputs: down 4096 x 12288 at M = 2 / 4 / 8 / 12 / 16
// 10.98 / 11.06 / 11.23 / 11.68 / 12.25 us against 12.64 / 12.72 / 12.77 /
// 13.17 / 13.17 (S = 8); o 4096 x 4096 at M = 2 / 8 / 16 / 24 / 32 5.53 /
// 5.63 / 5.73 / 6.63 / 7.01 against 6.94 / 7.46 / 7.84 / 8.36 / 8.77 (S = 4);
// qkv 6144 x 4096 at M = 2 / 8 / 16 6.98 / 7.48 / 8.09 against 8.30 / 8.98 /
// 9.25 (S = 4; 8.50 / 9.17 / 9.59 with S = 8).  At M = 24 and 32 down and
// qkv are level or slower than gemm_tall (down 13.78 / 15.12 against 13.59 /
// 14.03) and keep it.  gate_up (24576 x 4096, 1,536 workgroups) measured
// slower on it (M = 4 / 8 / 16 19.31 / 19.86 / 21.74 us against 18.23 /
// 18.01 / 17.41 on the 96-column tiles).  Deeper rings (5) and 16 waves
// measured level or slower.  These down figures are for contiguous K slices;
// the interleaved order the kernel now takes at S = 8 runs 2-3% faster.
static bool narrow_plan(uint32_t m, uint32_t n, uint32_t k, int& S, int& R, int& MB, int& LAL) {
  if (m == 0 || m > 32 || (n + 95) / 96 >= 224) return false;
  S = k >= 8192 ? 8 : 4;
  if (k % (128u * S) != 0) return false;
  if (m > 16 && !(k <= 4096 && (n + 15) / 16 <= 256)) return false;
  MB = m <= 16 ? 1 : 2;  // two blocks only at S = 4 (K <= 4096)
  LAL = (int)((m + 7) / 8);
  R = 4;
  return true;
}


// gemm_tall plan for 1 <= m <= 256 (measured on MI355X on the Qwen3-8B
// projection shapes at M = 16, 64, 65, 80, 100, 128 and 129): 96-column
// tiles when they alone give about one tile per CU; otherwise split K four
// ways (two when K is short), with 96- or 64-column tiles, to reach about one
// workgroup per CU.  For 64 < m <= 128 one 160-row tile streams the weights
// once where gemm_dma's two 64-row tiles stream them twice (gate_up at
// M = 100 24.6-24.9 against 33.3-34.1 us, down 20.7 against 23.3-23.5), and
// with streamed slabs the split route also beats gemm_dma's split-K 2 on
// qkv and o (qkv at M = 65 / 100 / 128 12.6 / 14.1 / 14.5 against
// 13.2-13.3 / 14.6 / 15.5, o 10.9 / 11.6 / 12.7 against 12.0 / 12.7 / 13.2).
// At small m the plan applies to the wide shapes and to long K at any m,
// where it beats gemm_skinny (graphs of 16 distinct-weight launches, random
// operands, m = 1..6: gate_up 17.9-18.1 against 21.2-24.0 us, down at
// K = 12288 13.1-13.5 against 16.7-17.1).  At K = 4096 on narrow N the
// skinny kernel (one workgroup per 16 columns) led while its grid fits the
// CUs once: o (4096 columns) at m = 2 / 4 / 8 / 12 / 16 / 24 7.1 / 7.2 /
// 7.4 / 7.6 / 7.9 / 9.6 us against 7.8 / 7.8 / 8.0 / 8.0 / 8.2 / 9.0; qkv
// (6144 columns) 8.4 / 8.8 / 9.6 / 10.5 / 11.5 against 8.6 / 8.8 / 9.0 /
// 9.1 / 9.3, so it takes this plan from m = 8, o from m = 24.  gemm_narrow's
// plan, checked first, now takes the small batches on narrow N.
// Returns false when no plan applies (the gemm_dma or gemm_skinny routes
// then run).  ma: the M tile (64, 160 or 256 rows).
static bool tall_plan(uint32_t m, uint32_t n, uint32_t k, int& bn, uint32_t& splits, int& ma) {
  if (m == 0 || m > 256 || k % 128 != 0) return false;
  ma = m <= 64 ? 64 : m <= 160 ? 160 : 256;
  const uint32_t kt = k / 128, t96 = (n + 95) / 96;
  if (t96 >= 224) {
    bn = 96;
    splits = 1;
    return true;
  }
  if (n % 4 != 0) return false;  // the split-K epilogue works on column quads
  if (k < 8192 && (m < 8 || (m < 24 && (n + 15) / 16 <= 256))) return false;
  splits = (kt % 4 == 0 && kt / 4 >= 4) ? 4 : (kt % 2 == 0 && kt / 2 >= 4) ? 2 : 1;
  if (splits == 1) return false;
  bn = t96 * splits >= 224 ? 96 : 64;
  return true;
}

size_t gemm_workspace_bytes(uint32_t m, uint32_t n, uint32_t k) {
  int tile;
  uint32_t splits;
  int ma;
  {
    int S, R, MB, LAL;
    if (narrow_plan(m, n, k, S, R, MB, LAL)) return 0;
  }
  if (tall_plan(m, n, k, tile, splits, ma)) return splits > 1 ? (size_t)splits * m * n * sizeof(int32_t) : 0;
  if (!split_plan(m, n, k, splits)) return 0;
  return (size_t)splits * m * n * sizeof(int32_t);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// gemm_tall's split-K slab sets of at least this many bytes are streamed:
// written with non-temporal stores (EP_SLAB) and read back non-temporally.
// Measured on MI355X (graphs of 16 distinct-weight launches, GEMM + slab
// epilogue, plain -> streamed): qkv at M = 255 23.6 -> 19.7-20.2 us, o at
// M = 255 19.1 -> 15.9, down at M = 200 26.3 -> 25.1, qkv at M = 129
// 19.4 -> 16.0, o at M = 129 14.4 -> 13.8-14.1, qkv at M = 40 13.6 -> 12.9.
// The streamed GEMM itself runs 1.2-1.3 us faster (no dirty slab lines left
// in L2 at its end).  Smaller sets, whose epilogue is latency-bound, lose
// (down at M = 32, 2 MiB: 16.6 -> 17.0; at M = 16, 1 MiB: 15.4 -> 15.9), and
// so does gemm_dma's split route (down at M = 512 38.3 -> 41.0, at M = 300
// 32.0 -> 33.2): both keep the default policy.
constexpr size_t kSlabStreamBytes = size_t(3) << 20;

static bool stream_slabs(const GemmArgs& a, uint32_t splits) {
  return (size_t)splits * a.m * a.n * sizeof(int32_t) >= kSlabStreamBytes;
}

template <int EP, bool NT>
static void launch_epilogue(hipStream_t st, const GemmArgs& a, uint32_t splits, bool wide) {
  const uint32_t rows = std::min<uint32_t>(a.m, 65535);
  if (wide)
    hipLaunchKernelGGL((splitk_epilogue8<EP, NT>), dim3((a.n / 8 + 255) / 256, rows), dim3(256), 0, st, a,
                       a.partials, splits);
  else
    hipLaunchKernelGGL((splitk_epilogue<EP, NT>), dim3((a.n / 4 + 255) / 256, rows), dim3(256), 0, st, a,
                       a.partials, splits);
}

// 8 columns per split-K epilogue thread above M = 200 when every row of
// every operand starts 16-byte aligned (n % 8 == 0 and aligned bases); 4
// otherwise.  The epilogue is latency-bound: up to M = 200 twice the threads
// with half the loads each finish sooner.  Measured on MI355X, graphs of 16
// distinct-weight launches, GEMM + epilogue, 8 -> 4 columns: M = 64 o
// 10.3 -> 9.7 us, M = 100 qkv 14.4 -> 13.5, M = 129 qkv 15.6-15.8 -> 14.9,
// o 13.5-13.9 -> 13.1, down 22.6-24.1 -> 22.0, M = 200 qkv 18.7 -> 17.7;
// but M = 255 o 15.9-16.1 -> 17.1, and level on gemm_dma's split route at
// M = 300 and 512.  Two columns per thread (256- or 512-thread workgroups)
// and four with 1,024-thread workgroups measured level or slower from M = 24
// to 200 (M = 129 o 12.28-12.44 against 12.24 us, down 21.6-21.8 against
// 21.5).
static bool wide_epilogue(const GemmArgs& a) {
  return a.m > 200 && a.n % 8 == 0 && aligned16(a.partials) && aligned16(a.out) &&
         (a.out_dtype == W8A8_OUT_I32 || aligned16(a.ws)) &&
         (!a.residual || (aligned16(a.residual) && aligned16(a.combined)));
}

template <bool NT>
static hipError_t launch_splitk_epilogue(hipStream_t st, const GemmArgs& a, uint32_t splits) {
  if (splits < 1 || splits > kMaxSplits) return hipErrorInvalidValue;
  const bool wide = wide_epilogue(a);
  if (a.out_dtype == W8A8_OUT_I32)
    launch_epilogue<EP_I32, NT>(st, a, splits, wide);
  else if (a.out_dtype == W8A8_OUT_F32 && a.residual)
    launch_epilogue<EP_F32_RES, NT>(st, a, splits, wide);
  else if (a.out_dtype == W8A8_OUT_F32)
    launch_epilogue<EP_F32, NT>(st, a, splits, wide);
  else if (a.residual)
    launch_epilogue<EP_BF16_RES, NT>(st, a, splits, wide);
  else
    launch_epilogue<EP_BF16, NT>(st, a, splits, wide);
  return hipGetLastError();
}

// Split-K launch: `gemm` launches the split GEMM into a.partials, given the
// slab mode as a compile-time constant; the slab epilogue follows.  Both
// take the same slab policy (nt: streamed).
template <typename Launch>
static hipError_t launch_slabs(hipStream_t st, const GemmArgs& a, uint32_t splits, bool nt, Launch gemm) {
  GemmArgs p = a;
  p.out = a.partials;
  p.out_dtype = W8A8_OUT_I32;
  if (nt) gemm(std::integral_constant<int, EP_SLAB>{}, p);
  else gemm(std::integral_constant<int, EP_I32>{}, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return nt ? launch_splitk_epilogue<true>(st, a, splits) : launch_splitk_epilogue<false>(st, a, splits);
}

template <int BM, int BN, int WM, int WN, int SA, int SB>
static hipError_t launch_split(hipStream_t st, const GemmArgs& a, uint32_t splits) {
  const uint32_t tm = (a.m + BM - 1) / BM, tn = (a.n + BN - 1) / BN;
  return launch_slabs(st, a, splits, false, [&](auto ep, const GemmArgs& p) {
    hipLaunchKernelGGL((gemm_dma<BM, BN, WM, WN, SA, SB, decltype(ep)::value, false>), dim3(tm * tn * splits),
                       dim3(512), 0, st, p, tm, tn, splits);
  });
}

template <int BN, int SA, int SB, int MA>
static hipError_t launch_tall(hipStream_t st, const GemmArgs& a, uint32_t splits) {
  const uint32_t tn = (a.n + BN - 1) / BN;
  const dim3 grid(tn * splits), block(512);
  if (splits > 1)
    return launch_slabs(st, a, splits, stream_slabs(a, splits), [&](auto ep, const GemmArgs& p) {
      hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, decltype(ep)::value, false>), grid, block, 0, st, p, tn, splits,
                         nullptr);
    });
  if (a.out_dtype == W8A8_OUT_I32)
    hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, EP_I32, kRotateK>), grid, block, 0, st, a, tn, 1u, nullptr);
  else if (a.out_dtype == W8A8_OUT_F32 && a.residual)
    hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, EP_F32_RES, kRotateK>), grid, block, 0, st, a, tn, 1u, nullptr);
  else if (a.out_dtype == W8A8_OUT_F32)
    hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, EP_F32, kRotateK>), grid, block, 0, st, a, tn, 1u, nullptr);
  else if (a.residual)
    hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, EP_BF16_RES, kRotateK>), grid, block, 0, st, a, tn, 1u, nullptr);
  else
    hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, EP_BF16, kRotateK>), grid, block, 0, st, a, tn, 1u, nullptr);
  return hipGetLastError();
}

// Diagnostics: gemm_tall with the per-wave clock stamps (TIMED), BF16
// outputs without a residual; the split-K epilogue follows as in launch_tall.
template <int BN, int SA, int SB, int MA>
static hipError_t launch_tall_timed(hipStream_t st, const GemmArgs& a, uint32_t splits, uint64_t* stamps) {
  const uint32_t tn = (a.n + BN - 1) / BN;
  const dim3 grid(tn * splits), block(512);
  if (splits > 1)
    return launch_slabs(st, a, splits, stream_slabs(a, splits), [&](auto ep, const GemmArgs& p) {
      hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, decltype(ep)::value, false, true>), grid, block, 0, st, p, tn,
                         splits, stamps);
    });
  hipLaunchKernelGGL((gemm_tall<BN, SA, SB, MA, EP_BF16, kRotateK, true>), grid, block, 0, st, a, tn, 1u, stamps);
  return hipGetLastError();
}

// ---------------------------------------------------------------- dispatch
// The route of one GEMM call (see GemmRoute).
GemmRoute gemm_route(const GemmArgs& a) {
  GemmRoute r{};
  r.splits = 1;
  r.epi_cols = 4;
  r.grid_y = 1;
  r.block = 512;
  if (a.m == 0 || a.n == 0) return r;
  {
    int S, R, MB, LAL;
    if (narrow_plan(a.m, a.n, a.k, S, R, MB, LAL)) {
      r.family = kRouteNarrow;
      r.mt = MB;
      r.s = S;
      r.u = LAL;
      r.sa = R;
      r.grid_x = (a.n + 15) / 16;
      r.block = 64 * S;
      return r;
    }
  }
  // m <= 256 goes to gemm_tall when its plan applies.
  // Otherwise, for small m: from m = 8 the 8-wave kernel with 64-row tiles
  // streams the weights faster when n gives at least 128 tiles; below that
  // the skinny kernel's split-K keeps more CUs busy.
  const bool wide = a.m >= 8 && a.k % 128 == 0 && (a.n + 127) / 128 >= 128;
  {
    int tile, ma;
    uint32_t splits;
    if (tall_plan(a.m, a.n, a.k, tile, splits, ma) &&
        (splits == 1 || (a.partials && a.partial_bytes >= (size_t)splits * a.m * a.n * sizeof(int32_t)))) {
      // Ring depths four and four for the 64- and 160-row tiles.  Measured on
      // MI355X, graphs of 16 distinct-weight launches (split routes: GEMM +
      // epilogue), from 8 / 8 and 4 / 8 (64 rows) and 5 / 5 and 4 / 6 (160
      // rows): M = 16 qkv 10.25 -> 9.3 us, o 8.56 -> 8.24, down 13.7 -> 13.2,
      // gate_up 18.1 -> 17.3; M = 64 qkv 11.6-11.8 -> 10.4, o 9.6-9.8 -> 8.8,
      // down 15.4-16.0 -> 14.9, gate_up 19.7-20.0 -> 19.0-19.2; M = 80 down
      // 18.7-19.5 -> 16.9; M = 100 qkv 13.2 -> 12.4-12.6, o 11.2 -> 10.4,
      // down 19.6-19.8 -> 17.7-18.1; M = 129 qkv 14.7-14.8 -> 14.0-14.3, o
      // 13.1-13.2 -> 12.4-12.6, gate_up 28.7-28.9 -> 27.0-28.1; M = 160 down
      // level.  6 / 6, 5 / 5, 4 / 5, 3 / 4 and 3 / 3 measured in between.  The
      // 256-row tile: 2 / 4 for the unsplit 96-column tiles (gate_up at
      // M = 200 33.7-35.1 -> 31.5-32.9 us, M = 255 37.6-37.9 -> 36.1-37.1
      // from 3 / 3), 3 / 3 and 4 / 4 for the split routes (2 / 3, 2 / 4 and
      // 3 / 4 level or slower there).
      r.family = kRouteTall;
      r.bn = tile;
      r.ma = ma;
      r.splits = splits;
      r.sa = r.sb = 4;
      if (ma == 256 && tile == 96) {
        r.sa = splits > 1 ? 3 : 2;
        r.sb = splits > 1 ? 3 : 4;
      }
      r.grid_x = (a.n + tile - 1) / tile * splits;
      if (splits > 1) {
        r.nt_slabs = stream_slabs(a, splits);
        r.epi_cols = wide_epilogue(a) ? 8 : 4;
      }
      return r;
    }
  }
  const uint32_t nb16 = (a.n + 15) / 16;
  if (a.m <= 64 && !wide) {
    r.family = kRouteSkinny;
    r.mt = a.m <= 16 ? 1 : a.m <= 32 ? 2 : 4;
    r.s = 4;
    r.u = a.m <= 32 ? 4 : 2;
    r.grid_x = nb16;
    r.block = 64 * r.s;
    return r;
  }
  if (a.k % 128 == 0) {
    r.family = kRouteDma;
    uint32_t splits;
    if (a.partials && split_plan(a.m, a.n, a.k, splits) &&
        a.partial_bytes >= (size_t)splits * a.m * a.n * sizeof(int32_t)) {
      r.bm = 128, r.bn = 128, r.wm = 32, r.wn = 64, r.sa = 4, r.sb = 4;
      r.splits = splits;
      r.epi_cols = wide_epilogue(a) ? 8 : 4;
    } else {
      // Tile per problem, measured on MI355X at M = 129 / 512 on the Qwen3-8B
      // projection shapes: the largest tile that still gives about one tile
      // per CU, smaller tiles for narrow N.  Residual outputs skip the
      // 256 x 192 tile (kResidualTile); t128 is then at least 480.
      const uint64_t t256 = (uint64_t)((a.m + 255) / 256) * ((a.n + 191) / 192);
      const uint64_t t128 = (uint64_t)((a.m + 127) / 128) * ((a.n + 191) / 192);
      if (t256 >= 240 && !a.residual) r.bm = 256, r.bn = 192, r.wm = 64, r.wn = 96, r.sa = 2, r.sb = 3;
      else if (t128 >= 240) r.bm = 128, r.bn = 192, r.wm = 32, r.wn = 96, r.sa = 2, r.sb = 4;
      else if (a.n >= 6144 && a.m >= 256) r.bm = 128, r.bn = 128, r.wm = 32, r.wn = 64, r.sa = 4, r.sb = 4;
      else if (a.m >= 128) r.bm = 128, r.bn = 64, r.wm = 32, r.wn = 32, r.sa = 4, r.sb = 4;
      else r.bm = 64, r.bn = 128, r.wm = 32, r.wn = 32, r.sa = 4, r.sb = 4;
    }
    r.grid_x = (a.m + r.bm - 1) / r.bm * ((a.n + r.bn - 1) / r.bn) * r.splits;
    return r;
  }
  r.family = kRouteTiled;
  r.bm = 128, r.bn = 128, r.wm = 64, r.wn = 64;
  r.grid_x = (a.m + r.bm - 1) / r.bm * ((a.n + r.bn - 1) / r.bn);
  r.block = 256;
  return r;
}

size_t gemm_timeline_waves(const GemmArgs& a) {
  const GemmRoute r = gemm_route(a);
  return r.family == kRouteTall ? (size_t)r.grid_x * 8 : 0;
}

hipError_t launch_gemm_timeline(hipStream_t st, const GemmArgs& a, uint64_t* stamps) {
  const GemmRoute r = gemm_route(a);
  if (r.family != kRouteTall || a.out_dtype != W8A8_OUT_BF16 || a.residual) return hipErrorInvalidValue;
  if (r.ma == 64)
    return r.bn == 96 ? launch_tall_timed<96, 4, 4, 64>(st, a, r.splits, stamps)
                      : launch_tall_timed<64, 4, 4, 64>(st, a, r.splits, stamps);
  if (r.ma == 160)
    return r.bn == 96 ? launch_tall_timed<96, 4, 4, 160>(st, a, r.splits, stamps)
                      : launch_tall_timed<64, 4, 4, 160>(st, a, r.splits, stamps);
  if (r.bn == 96)
    return r.splits > 1 ? launch_tall_timed<96, 3, 3, 256>(st, a, r.splits, stamps)
                        : launch_tall_timed<96, 2, 4, 256>(st, a, r.splits, stamps);
  return launch_tall_timed<64, 4, 4, 256>(st, a, r.splits, stamps);
}

template <int MB, int LAL, int S, int R>
static hipError_t launch_narrow_as(hipStream_t st, const GemmArgs& a, uint32_t grid) {
  hipLaunchKernelGGL((gemm_narrow<MB, LAL, S, R>), dim3(grid), dim3(64 * S), 0, st, a);
  return hipGetLastError();
}

// The instantiations narrow_plan can ask for: S = 4 with one or two 16-row
// blocks, S = 8 (K >= 8192) with one; LAL = ceil(M / 8); R = 4.
static hipError_t launch_narrow(hipStream_t st, const GemmArgs& a, const GemmRoute& r) {
  const uint32_t g = r.grid_x;
  if (r.s == 4) {
    switch (r.u) {
      case 1: return launch_narrow_as<1, 1, 4, 4>(st, a, g);
      case 2: return launch_narrow_as<1, 2, 4, 4>(st, a, g);
      case 3: return launch_narrow_as<2, 3, 4, 4>(st, a, g);
      case 4: return launch_narrow_as<2, 4, 4, 4>(st, a, g);
    }
  } else if (r.s == 8) {
    switch (r.u) {
      case 1: return launch_narrow_as<1, 1, 8, 4>(st, a, g);
      case 2: return launch_narrow_as<1, 2, 8, 4>(st, a, g);
    }
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm(hipStream_t st, const GemmArgs& a) {
  const GemmRoute r = gemm_route(a);
  auto is = [&](int bm, int bn, int wm, int wn, int sa, int sb) {
    return r.bm == bm && r.bn == bn && r.wm == wm && r.wn == wn && r.sa == sa && r.sb == sb;
  };
  switch (r.family) {
    case kRouteNone:
      return hipSuccess;
    case kRouteTall:
      if (r.ma == 64)
        return r.bn == 96 ? launch_tall<96, 4, 4, 64>(st, a, r.splits) : launch_tall<64, 4, 4, 64>(st, a, r.splits);
      if (r.ma == 160)
        return r.bn == 96 ? launch_tall<96, 4, 4, 160>(st, a, r.splits) : launch_tall<64, 4, 4, 160>(st, a, r.splits);
      if (r.bn == 96)
        return r.splits > 1 ? launch_tall<96, 3, 3, 256>(st, a, r.splits) : launch_tall<96, 2, 4, 256>(st, a, r.splits);
      return launch_tall<64, 4, 4, 256>(st, a, r.splits);
    case kRouteNarrow:
      return launch_narrow(st, a, r);
    case kRouteSkinny:
      if (r.mt == 1) hipLaunchKernelGGL((gemm_skinny<1, 4, 4>), dim3(r.grid_x, 1), dim3(r.block), 0, st, a);
      else if (r.mt == 2) hipLaunchKernelGGL((gemm_skinny<2, 4, 4>), dim3(r.grid_x, 1), dim3(r.block), 0, st, a);
      else hipLaunchKernelGGL((gemm_skinny<4, 4, 2>), dim3(r.grid_x, 1), dim3(r.block), 0, st, a);
      return hipGetLastError();
    case kRouteDma:
      if (r.splits > 1) return launch_split<128, 128, 32, 64, 4, 4>(st, a, r.splits);
      if (is(256, 192, 64, 96, 2, 3)) return launch_dma<256, 192, 64, 96, 2, 3>(st, a);
      if (is(128, 192, 32, 96, 2, 4)) return launch_dma<128, 192, 32, 96, 2, 4>(st, a);
      if (is(128, 128, 32, 64, 4, 4)) return launch_dma<128, 128, 32, 64, 4, 4>(st, a);
      if (is(128, 64, 32, 32, 4, 4)) return launch_dma<128, 64, 32, 32, 4, 4>(st, a);
      return launch_dma<64, 128, 32, 32, 4, 4>(st, a);
    case kRouteTiled: {
      const uint32_t tm = (a.m + 127) / 128, tn = (a.n + 127) / 128;
      hipLaunchKernelGGL((gemm_tiled<128, 128, 64, 64>), dim3(tm * tn), dim3(256), 0, st, a, tm, tn);
      return hipGetLastError();
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace w8a8
