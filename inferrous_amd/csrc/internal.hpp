// internal.hpp -- host-side launch interface between the C ABI layer
// (abi.hip) and the kernel files.  Not installed; not part of the ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/inferrous_w8a8.h"

namespace w8a8 {

constexpr int kMaxGroup = 4;
constexpr int kSelectBlocks = 1024;  // stand-alone selection: at most this many workgroups (one u64 key each)
// The fused lm_head selection writes one u64 key per workgroup; every route
// gives a workgroup at least this many vocabulary rows.
constexpr size_t kArgmaxRowsPerKey = 4;
constexpr size_t argmax_keys_for(size_t n) { return (n + kArgmaxRowsPerKey - 1) / kArgmaxRowsPerKey; }

// One GEMV launch: up to kMaxGroup sibling projections sharing q/asc.
struct GemvArgs {
  const int8_t* q;
  const float* asc;
  uint32_t m, k;
  int count;
  const int8_t* w[kMaxGroup];
  const float* ws[kMaxGroup];
  uint32_t n[kMaxGroup];
  uint32_t gbegin[kMaxGroup + 1];  // first row group of each projection (set by the launcher)
  void* out[kMaxGroup];
  int out_dtype;
  const float* residual;  // EPI residual (count == 1)
  void* combined;
  uint64_t* slots;  // fused selection (count == 1, m == 1): one u64 key per workgroup
  uint32_t* token;
};

// Fused gate/up GEMV with the SiLU product (M = 1).
struct SwigluArgs {
  const int8_t* q;
  const float* asc;
  uint32_t k, n;
  const int8_t* wg;
  const float* wsg;
  const int8_t* wu;
  const float* wsu;
  void* gate;
  void* up;
  void* act;
  int out_dtype;      // F32 or BF16
  uint32_t* maxima;   // optional: atomicMax of bits(|act|)
  int8_t* q_out;      // optional (with maxima): act quantized with the folded maximum
  float* scales_out;
};

struct GemmArgs {
  const int8_t* q;
  const float* asc;
  uint32_t m;
  const int8_t* w;
  const float* ws;
  uint32_t n, k;
  void* out;
  int out_dtype;
  const float* residual;
  void* combined;
  int32_t* partials;     // optional split-K workspace (i32 slabs), may be null
  size_t partial_bytes;
};

// Bytes of split-K workspace launch_gemm would use for this shape (0: none).
size_t gemm_workspace_bytes(uint32_t m, uint32_t n, uint32_t k);

// The launch a GEMM call makes, decided on the host: the kernel family, its
// compile-time shape and its grid.  launch_gemm runs exactly this route; the
// diagnostics export it so that host-side checks can replay each kernel's
// index arithmetic over its grid.
enum { kRouteNone = 0, kRouteGemvM1One = 1, kRouteGemvM1 = 2, kRouteGemvMt = 3, kRouteSkinny = 11,
       kRouteTall = 12, kRouteDma = 13, kRouteTiled = 14, kRouteNarrow = 15 };
struct GemmRoute {
  int family;                       // kRouteSkinny, kRouteTall, kRouteDma, kRouteTiled, kRouteNarrow
                                    // (kRouteNone: m or n is 0)
  int bm, bn, wm, wn, sa, sb, ma;   // dma / tiled tile; tall: bn, sa, sb, ma; narrow: sa = ring stages
  int mt, s, u;                     // skinny: 16-row tiles, waves, unroll; narrow: 16-row tiles, waves,
                                    // live activation DMA loads per stage
  uint32_t splits;                  // split-K slabs (1: none)
  int nt_slabs;                     // slabs streamed (EP_SLAB)
  int epi_cols;                     // split-K epilogue columns per thread (4 or 8)
  uint32_t grid_x, grid_y, block;   // the GEMM launch
};
GemmRoute gemm_route(const GemmArgs& a);
// Diagnostics: the gemm_tall route with per-wave clock stamps (4 per wave).
size_t gemm_timeline_waves(const GemmArgs& a);
hipError_t launch_gemm_timeline(hipStream_t st, const GemmArgs& a, uint64_t* stamps);

// The launch a GEMV call makes (launch_gemv / launch_gemv_argmax): family
// kRouteGemvM1One, kRouteGemvM1 or kRouteGemvMt; `rows` rows per row group
// (one wave's), kc = K / 1024 (M = 1 families), mt activation rows and u
// chunks per pass (gemv_mt), waves per workgroup and the grid.
struct GemvRoute {
  int family;
  int rows, kc, mt, u, waves;
  uint32_t grid_x, grid_y;
};
GemvRoute gemv_route(uint32_t m, uint32_t k, const uint32_t* n, int count, bool argmax);

hipError_t launch_quantize(hipStream_t st, const void* x, bool bf16, uint32_t width, size_t rows,
                           int8_t* q, float* scales, uint32_t* maxima_reset);
hipError_t launch_quantize_with_max(hipStream_t st, const float* x, uint32_t width, size_t rows,
                                    const uint32_t* maxima, int8_t* q, float* scales);
hipError_t launch_rounding_probe(hipStream_t st, const float* in, size_t n, int8_t* out);
hipError_t launch_head_packed(hipStream_t st, const float* x4096, const uint32_t* words,
                              const uint32_t* offsets, const uint16_t* exceptions, uint32_t n_exceptions,
                              uint32_t rows, float* out);
hipError_t launch_unpack_bf16(hipStream_t st, const uint32_t* words, const uint32_t* offsets,
                              const uint16_t* exceptions, size_t n, uint16_t* out);
size_t pack_bf16_host(const uint16_t* in, size_t n, uint32_t* words, uint32_t* offsets,
                      uint16_t* exceptions);
hipError_t launch_norm_quantize(hipStream_t st, const float* x, const float* gain, size_t rows,
                                float* out, int8_t* q, float* scales, uint32_t* maxima);  // width 4096

hipError_t launch_gemv(hipStream_t st, GemvArgs& a);

// A producer of one 4096-wide f32 row's codes -- norm_quantize when gain is
// set, quantize otherwise -- and the M = 1 linear (or linear_residual) on
// those codes, in one launch.
struct ProduceArgs {
  const float* x;
  const float* gain;
  float* normed;          // optional: norm_quantize's normalised row
  int8_t* q;              // the row's codes (16-byte aligned)
  float* scale;
  uint32_t* maxima;       // optional: reset to the floor, as the producers do
  const int8_t* w;
  const float* ws;
  uint32_t n;             // >= 1
  const float* residual;  // with combined: linear_residual
  void* out;
  void* combined;
  int out_dtype;
};
hipError_t launch_gemv_produce(hipStream_t st, const ProduceArgs& p);
// norm_quantize (p: x, gain, normed, q, scale; p.maxima == a.maxima) folded
// into the M = 1 SwiGLU GEMV (a: k = 4096, maxima required), then the row
// tail that folds the act maximum (and quantizes act when a.q_out is set).
// row_tail: also run swiglu_row_tail<true> (maximum fold, and the codes when
// a.q_out is set); without it maxima[0] is left as the norm reset it.
hipError_t launch_gemv_swiglu_norm(hipStream_t st, const ProduceArgs& p, const SwigluArgs& a, bool row_tail);
// The SwiGLU row tail folded into the M = 1, K = 12288 GEMV that consumes
// its codes (gemv_rowtail_split).
struct RowtailArgs {
  const void* act;   // [12288], act_dtype (F32 or BF16)
  int act_dtype;
  uint32_t* maxima;  // maxima[0]: read, the row maximum folded in
  int8_t* q_out;     // optional: the row's codes
  float* scale_out;  // optional: its scale
  const int8_t* w;   // [n, 12288]
  const float* ws;
  uint32_t n;
  const float* residual;  // optional, with combined
  void* out;
  void* combined;
  int out_dtype;  // F32 or BF16
};
hipError_t launch_gemv_rowtail(hipStream_t st, const RowtailArgs& d);
// Diagnostics: the one-matrix M = 1 GEMV with per-wave clock stamps.
size_t gemv_timeline_waves(size_t n, uint32_t k);
hipError_t launch_gemv_timeline(hipStream_t st, const int8_t* q, const float* asc, const int8_t* w,
                                const float* ws, uint32_t n, uint32_t k, void* out, int dtype,
                                uint64_t* stamps);
hipError_t launch_gemv_argmax(hipStream_t st, GemvArgs& a);
hipError_t launch_gemv_swiglu(hipStream_t st, const SwigluArgs& a);  // m == 1, k in {4096, 12288}
hipError_t launch_swiglu(hipStream_t st, const void* gate, const void* up, size_t rows,
                         uint32_t width, void* act, int dtype, uint32_t* maxima);
// act rows quantized as quantize_with_max does with maxima (F32 or BF16 act)
hipError_t launch_swiglu_quantize_rows(hipStream_t st, const void* act, size_t rows, uint32_t width, int dtype,
                                       const uint32_t* maxima, int8_t* q, float* scales);
hipError_t launch_select(hipStream_t st, const float* x, size_t n, uint64_t* keys, uint32_t* token);
// u64 keys the fused selection of an n-row lm_head writes (an upper bound)
size_t argmax_keys_bound(size_t n);

hipError_t launch_gemm(hipStream_t st, const GemmArgs& a);

// One entry of a decode-sequence table (device memory, 64 bytes).
struct SeqEntry {
  const int8_t* w;         // [n, k]
  const float* ws;         // [n]
  const int8_t* q;         // [k]
  const float* asc;        // [1]
  void* out;               // [n], or null (selecting entry without logits)
  const float* residual;   // [n], with combined
  void* combined;          // [n]
  uint32_t n;
  uint32_t meta;           // bits 0-1: k / 4096; bit 2: BF16 out (else F32); bit 3: residual; bit 4: selection
};
static_assert(sizeof(SeqEntry) == 64, "one scalar cache line pair per entry");
constexpr int kSeqGroups = 8;              // arrival counters of the sequence barrier
constexpr size_t kSeqCtlBytes = 4096;      // uncached control block: counters, status
// Workgroups of a sequence launch on the current device (one per CU; 0 when
// a CU cannot hold one), and the largest n an entry may have for that grid.
uint32_t seq_grid();
uint32_t seq_max_rows(uint32_t grid);
hipError_t launch_sequence(hipStream_t st, const SeqEntry* tab, uint32_t count, uint32_t base, uint32_t* ctl,
                           uint64_t* keys, uint32_t* token, uint64_t spin, uint32_t grid);

hipError_t launch_synth_i8(hipStream_t st, int8_t* out, size_t n, uint64_t seed, uint64_t stream_id);
hipError_t launch_synth_f32(hipStream_t st, float* out, size_t n, uint64_t seed, uint64_t stream_id,
                            float lo, float hi);
hipError_t launch_fill_zero(hipStream_t st, void* dst, size_t bytes);

}  // namespace w8a8
