// gemm.hip -- INT8 MFMA GEMM (exact i32 accumulate) for prefill and small
// batches, with the fused per-token x per-channel dequant epilogue.
//
// Reference semantics (crates/inferrous-qwen3/): the M > 1 projections
//   linear_prefill src/kernels.rs:846-931, linear_splitk :932-1034,
//   linear_tiled :1035-1141, linear_large :1142-1289, epilogues
//   :918-930, :1008-1033, :1123-1140, :1249-1288:
//   out[r][c] = bf(RN(RN(f32(sum_k q[r][k] w[c][k]) * asc[r]) * ws[c]))
//
// gfx950 design.  The matrix core op is v_mfma_i32_16x16x64_i8: per lane a
// 16-byte A fragment (row lane%16) and a 16-byte B fragment (column
// lane%16), both taken at k offset (lane/16)*16 within the 64-wide step.
// Any k permutation applied identically to A and B leaves the exact integer
// sum unchanged, so both operands are read with the same lane -> k map; the
// 4 x i32 result of lane l holds rows 4*(l/16)+v, column l%16.
//
// Two kernels:
//  * gemm_skinny (M <= 64, HBM-bound): one workgroup owns 16 weight rows;
//    its S waves split K and stream their weight fragments straight from
//    HBM into MFMA B operands (no LDS round trip), activation fragments come
//    from L1/L2.  Partial i32 tiles are summed through LDS -- exact.
//  * gemm_tiled (M > 64): BM x BN output tile, 4 waves, 128-byte K stages
//    double-buffered in LDS (row pitch 144 B: a 16-lane ds_read_b128 column
//    touches every bank once), global loads of stage k+1 in flight while
//    stage k feeds the MFMAs.  Workgroups are numbered so that the M tiles
//    sharing one weight panel run on the same XCD (workgroup id mod 8 picks
//    the XCD), so the panel is fetched into that XCD's L2 once.
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

// ---------------------------------------------------------------- dispatch
hipError_t launch_gemm(hipStream_t st, const GemmArgs& a) {
  if (a.m == 0 || a.n == 0) return hipSuccess;
  const unsigned nb16 = (a.n + 15) / 16;
  if (a.m <= 16) {
    hipLaunchKernelGGL((gemm_skinny<1, 4, 4>), dim3(nb16, 1), dim3(256), 0, st, a);
  } else if (a.m <= 32) {
    hipLaunchKernelGGL((gemm_skinny<2, 4, 4>), dim3(nb16, 1), dim3(256), 0, st, a);
  } else if (a.m <= 64) {
    hipLaunchKernelGGL((gemm_skinny<4, 4, 2>), dim3(nb16, 1), dim3(256), 0, st, a);
  } else {
    constexpr int BM = 128, BN = 128;
    const uint32_t tm = (a.m + BM - 1) / BM, tn = (a.n + BN - 1) / BN;
    hipLaunchKernelGGL((gemm_tiled<BM, BN, 64, 64>), dim3(tm * tn), dim3(256), 0, st, a, tm, tn);
  }
  return hipGetLastError();
}

}  // namespace w8a8
