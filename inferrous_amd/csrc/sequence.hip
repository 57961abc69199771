// sequence.hip -- a dependent sequence of M = 1 projections in one launch.
//
// Reference: the decode step replays its projections as a captured graph
// whose kernel edges are programmatic (crates/inferrous-qwen3/src/graph.rs:
// 56-110): each kernel issues its weight stream, then waits at
// griddepcontrol.wait for its predecessor (src/kernels.rs:173-184), which
// kept DRAM busy across kernel boundaries (docs/qwen3-8b-w8a8/optimization/
// round-6.md:63-73).  The per-projection arithmetic is linear /
// linear_residual (src/kernels.rs:577-618, :807-845) and, for a selecting
// last entry, the lm_head GEMV with select_token (src/kernels.rs:2191-2231).
//
// MI355X design.  HIP has no dependent-launch edge: between two dependent
// kernels the queue leaves every CU idle (~1.1 us), and each kernel then
// waits a memory latency for its first bytes.  Here one workgroup per CU
// runs the whole sequence.  Entry p+1 starts only after every workgroup
// has finished entry p: each workgroup announces an entry with one atomic
// add on its group's arrival counter (8 counters, workgroups dealt by
// blockIdx mod 8), and reads entry p+1's activation row only once all
// counters have reached the entry's epoch.  What does not depend on
// entry p -- the weights, which no entry writes -- is requested ahead of
// that barrier, like the reference's prefetch before griddepcontrol.wait.
//
// Per workgroup: wave 0 is the control wave (barrier, arrival, the
// selection's reduction); waves 1-15 stream weights.  Every compute wave
// keeps kSeqRing units of 4 KiB (one row of K = 4096, a third of a row of
// K = 12288) in flight, across entry boundaries, in its own LDS ring
// filled by global -> LDS DMA (120 KiB per CU).  A CU's
// vector-memory returns come back in issue order, so anything requested
// through that path waits behind the ring; the barrier is therefore polled
// with scalar loads of uncached memory, and the activation row is fetched
// with scalar loads (one slice per wave) into LDS.  Row r of an entry goes
// to compute wave g = r mod (15 G), g = (wave - 1) * G + blockIdx.x, so at
// any moment the machine streams a contiguous window of each matrix, as the
// one-shot GEMV's dispatch order does.
//
// The i32 sums are exact, so every output equals w8a8_linear's bit for bit
// (same dequant epilogue and BF16 rounding).  Waits are bounded: a wait
// that exceeds the caller's tick limit marks the sequence state aborted in
// the control block, every wave then leaves, and the host reads the status.
#include "device_common.hpp"
#include "internal.hpp"

namespace w8a8 {

constexpr int kSeqWaves = 16;               // 1 control + 15 compute waves
constexpr int kSeqCompute = kSeqWaves - 1;
constexpr uint32_t kSeqRing = 4;            // 4 KiB units in flight per compute wave
constexpr uint32_t kSeqUnit = 4096;         // bytes of a row per unit
constexpr uint32_t kSeqMaxUnits = 3;        // K <= 12288
constexpr uint32_t kSeqActBytes = kSeqUnit * kSeqMaxUnits;

static_assert(kSeqGroups == 8, "the poll reads eight counters");

struct SeqLds {
  alignas(16) int8_t act[kSeqActBytes];  // activation row of the open entry
  uint32_t released;   // entries whose activation may be loaded (control wave)
  uint32_t slices;     // activation slices written, 16 per entry
  uint32_t done;       // compute waves done with an entry, 15 per entry
  uint32_t abort;
  uint64_t wkey[kSeqCompute];
};

__device__ __forceinline__ uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

__device__ __forceinline__ uint32_t lds_get(uint32_t* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)__hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP));
}

// Wait until *p >= target (wrap-safe); false on abort or time-out (the
// wave then sets the workgroup's abort flag).
__device__ __forceinline__ bool lds_wait(uint32_t* p, uint32_t target, SeqLds& L, uint64_t spin) {
  const uint64_t t0 = now_ticks();
  for (;;) {
    if ((int32_t)(lds_get(p) - target) >= 0) return true;
    if (lds_get(&L.abort)) return false;
    if (now_ticks() - t0 > spin) {
      __hip_atomic_store(&L.abort, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Scalar read of the arrival counters and the status word, bypassing the
// scalar cache (glc); the control block is uncached device memory, so the
// values come from memory, not from a stale cache line.

struct CtlView {
  uint32_t c[kSeqGroups];
  uint32_t status;
};

__device__ __forceinline__ CtlView read_ctl(const uint32_t* ctl) {
  CtlView v;
  asm volatile(
      "s_load_dword %0, %9, 0x0 glc\n\t"
      "s_load_dword %1, %9, 0x100 glc\n\t"
      "s_load_dword %2, %9, 0x200 glc\n\t"
      "s_load_dword %3, %9, 0x300 glc\n\t"
      "s_load_dword %4, %9, 0x400 glc\n\t"
      "s_load_dword %5, %9, 0x500 glc\n\t"
      "s_load_dword %6, %9, 0x600 glc\n\t"
      "s_load_dword %7, %9, 0x700 glc\n\t"
      "s_load_dword %8, %9, 0x800 glc\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(v.c[0]), "=&s"(v.c[1]), "=&s"(v.c[2]), "=&s"(v.c[3]), "=&s"(v.c[4]), "=&s"(v.c[5]),
        "=&s"(v.c[6]), "=&s"(v.c[7]), "=&s"(v.status)
      : "s"(ctl)
      : "memory");
  return v;
}

// Workgroups of arrival group c (blockIdx mod 8 == c) among G.
__device__ __forceinline__ uint32_t group_size(uint32_t c, uint32_t G) {
  return G / kSeqGroups + (c < G % kSeqGroups ? 1u : 0u);
}

// Wait until every workgroup has announced `epoch` entries of the call
// (counter c >= epoch * |group c|, wrap-safe).  false on abort / time-out.
__device__ __forceinline__ bool global_wait(const uint32_t* ctl, uint32_t epoch, uint32_t G, SeqLds& L,
                                          uint64_t spin) {
  const uint64_t t0 = now_ticks();
  for (;;) {
    const CtlView v = read_ctl(ctl);
    bool ok = true;
#pragma unroll
    for (uint32_t c = 0; c < kSeqGroups; ++c) ok = ok && (int32_t)(v.c[c] - epoch * group_size(c, G)) >= 0;
    if (ok) return true;
    if (v.status != 0 || lds_get(&L.abort)) return false;
    if (now_ticks() - t0 > spin) return false;
    __builtin_amdgcn_s_sleep(1);
  }
}

typedef int v16i __attribute__((ext_vector_type(16)));

// Read-only, wave-uniform data (the entry table, scales, residuals) is read
// through the constant address space, which the compiler turns into scalar
// loads: they do not queue behind the weight ring on the vector path.  The
// caller does not write any of it during the call.
template <typename T>
using Const = const __attribute__((address_space(4))) T*;
template <typename T>
__device__ __forceinline__ Const<T> cptr(const T* p) {
  return (Const<T>)(const __attribute__((address_space(4))) void*)p;
}

__device__ __forceinline__ const int8_t* uniform_ptr(const int8_t* p) {
  const uint64_t u = (uint64_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
  return (const int8_t*)(((uint64_t)hi << 32) | lo);
}

// 256 bytes at p (wave-uniform, 64-byte aligned) by four scalar loads, then
// written to LDS at dst: lane l stores dword l.  The activation row is an
// input of the call, unchanged while it runs, and the scalar cache starts
// each launch invalidated, so the loads may hit it.  (With the cache-bypass
// bit every load went to L2 one after another: 10.3 against 3.6 us per
// entry for a sequence of one-row entries on MI355X.)
__device__ __forceinline__ void slice256_to_lds(const int8_t* p, int8_t* dst, int lane) {
  p = uniform_ptr(p);
  v16i a, b, c, d;
  asm volatile(
      "s_load_dwordx16 %0, %4, 0x0\n\t"
      "s_load_dwordx16 %1, %4, 0x40\n\t"
      "s_load_dwordx16 %2, %4, 0x80\n\t"
      "s_load_dwordx16 %3, %4, 0xc0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(a), "=&s"(b), "=&s"(c), "=&s"(d)
      : "s"(p)
      : "memory");
  int v = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(a[i]), "i"(i));
    asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(b[i]), "i"(16 + i));
    asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(c[i]), "i"(32 + i));
    asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(d[i]), "i"(48 + i));
  }
  reinterpret_cast<int*>(dst)[lane] = v;
}

// This wave's slice (1/16) of an entry's activation row into L.act.  One
// buffer is enough: entry p + 1's row is written only after the barrier
// that follows every wave's last read of entry p's.
__device__ __forceinline__ void load_act_slice(const int8_t* q, uint32_t kc, uint32_t wave, SeqLds& L, int lane) {
  const uint32_t slice = kc * 256;  // K / 16 bytes
  const int8_t* src = q + (size_t)wave * slice;
  int8_t* dst = &L.act[wave * slice];
  for (uint32_t b = 0; b < kc; ++b) slice256_to_lds(src + b * 256, dst + b * 256, lane);
  // One count per wave: from one lane (an atomic on every lane adds 64).
  if (lane == 0) __hip_atomic_fetch_add(&L.slices, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ uint32_t entry_units(uint32_t meta) { return meta & 3u; }

// Where a compute wave's unit stream stands: entry p, row, unit of the row.
struct Cursor {
  uint32_t p = 0, row = 0, sub = 0, kc = 1, n = 0;
  const int8_t* w = nullptr;
  bool live = false;
};

// First entry at or after p with a row for wave g; live = false past the end.
__device__ __forceinline__ void seek(Cursor& c, Const<SeqEntry> tab, uint32_t count, uint32_t p,
                                     uint32_t g) {
  c.live = false;
  for (; p < count; ++p) {
    const uint32_t n = tab[p].n;
    if (g < n) {
      c.p = p;
      c.row = g;
      c.sub = 0;
      c.n = n;
      c.kc = entry_units(tab[p].meta);
      c.w = tab[p].w;
      c.live = true;
      return;
    }
  }
  c.p = count;
}

__device__ __forceinline__ void step_cursor(Cursor& c, Const<SeqEntry> tab, uint32_t count, uint32_t g,
                                            uint32_t NW) {
  if (++c.sub < c.kc) return;
  c.sub = 0;
  c.row += NW;
  if (c.row < c.n) return;
  seek(c, tab, count, c.p + 1, g);
}

// One unit (4 KiB of a weight row) into a register slot: four wave-wide
// 1 KiB non-temporal loads, lane l holding bytes [16 l, 16 l + 16) of each
// KiB.  A spent cursor reloads `spare` (4 KiB that stay in L2), so every
// slot is refilled on every pass and no slot's registers depend on a branch.
__device__ __forceinline__ void issue_unit(v4i (&r)[4], const Cursor& c, const int8_t* spare, int lane) {
  const int8_t* p = c.live ? c.w + (size_t)c.row * (c.kc * kSeqUnit) + c.sub * kSeqUnit : spare;
  p += lane * 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = load_nt16(p + i * 1024);
}

// Each compute wave's scales and residuals of its rows of the open entry,
// brought in by global -> LDS DMA (lane l: row g + l NW).
__shared__ __attribute__((aligned(16))) float seq_rowv[kSeqCompute][2][64];

// M0 carries the LDS address of a DMA request; nothing else in this file
// uses it, and the compiler emits no M0 use of its own here.  The request
// is written as an instruction, so the compiler does not count it: the
// wave waits for it with wait_vm_dyn below, and the compiler's waits for
// its own loads, which count fewer requests than are outstanding, only
// wait longer.
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void issue_row_values(float* dst, const float* src) {
  const uint32_t lds = (uint32_t)(uintptr_t)(void __attribute__((address_space(3)))*)dst;
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dword %0, off"
      :
      : "v"(src), "s"(lds)
      : "memory", "m0");
}

// vmcnt(n) with the other counters left open (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// vmcnt(min(n, 15)) for a wave-uniform n known at run time (a smaller
// count only waits longer).
__device__ __forceinline__ void wait_vm_dyn(uint32_t n) {
  switch (n < 15 ? n : 15) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<1>(); break;
    case 2: wait_vm<2>(); break;
    case 3: wait_vm<3>(); break;
    case 4: wait_vm<4>(); break;
    case 5: wait_vm<5>(); break;
    case 6: wait_vm<6>(); break;
    case 7: wait_vm<7>(); break;
    case 8: wait_vm<8>(); break;
    case 9: wait_vm<9>(); break;
    case 10: wait_vm<10>(); break;
    case 11: wait_vm<11>(); break;
    case 12: wait_vm<12>(); break;
    case 13: wait_vm<13>(); break;
    case 14: wait_vm<14>(); break;
    default: wait_vm<15>(); break;
  }
}

__device__ __forceinline__ void store_val(void* out, size_t i, bool bf16, float v) {
  if (bf16)
    reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)(__float_as_uint(v) >> 16);
  else
    reinterpret_cast<float*>(out)[i] = v;
}

struct SeqArgs {
  const SeqEntry* tab;
  uint32_t count;
  uint32_t base;  // entries announced by every workgroup before this call
  uint32_t* ctl;  // uncached control block: counters at u32 index c * 64, status at 8 * 64
  uint64_t* keys;  // selecting last entry: one key per workgroup
  uint32_t* token;
  uint64_t spin;  // wait limit in 100 MHz ticks
};

// The compute side: waves 1..15.  Four register slots r0..r3 hold units
// u, u + 1, u + 2, u + 3 of the wave's stream; the loop body is unrolled
// over them, so each slot's registers are named statically.  Slot s is
// refilled with unit u + 4 right after its products, unconditionally, and
// the compiler's own waits count the loads issued after each slot's.  A
// row's sum stays in lane j (the wave's j-th row of the entry); the
// epilogue runs once per entry, over every row of the wave, with the rows'
// scales (and residuals) loaded when the entry opens.
__device__ __forceinline__ void seq_compute(const SeqArgs& a, SeqLds& L, uint32_t wave, int lane) {
  Const<SeqEntry> tab = cptr(a.tab);
  const uint32_t count = a.count;
  const uint32_t G = gridDim.x, NW = kSeqCompute * G;
  const uint32_t g = (wave - 1) * G + blockIdx.x;
  const uint32_t cw = wave - 1;
  const int8_t* spare = tab[count - 1].q;  // k >= 4096 bytes

  Cursor is, cs;  // issue and consume cursors
  seek(is, tab, count, 0, g);
  seek(cs, tab, count, 0, g);
  v4i r0[4], r1[4], r2[4], r3[4];
  issue_unit(r0, is, spare, lane);
  if (is.live) step_cursor(is, tab, count, g, NW);
  issue_unit(r1, is, spare, lane);
  if (is.live) step_cursor(is, tab, count, g, NW);
  issue_unit(r2, is, spare, lane);
  if (is.live) step_cursor(is, tab, count, g, NW);
  issue_unit(r3, is, spare, lane);
  if (is.live) step_cursor(is, tab, count, g, NW);

  float* rowws = &seq_rowv[cw][0][0];
  float* rowres = &seq_rowv[cw][1][0];
  uint32_t vm_ops = 16;  // vector-memory requests issued so far (vmcnt order)
  uint32_t rows_at = 0;  // vm_ops right after the open entry's row-value requests
  uint32_t open = 0;     // next entry whose boundary this wave has not passed
  uint32_t j = 0;        // rows of the open entry summed by this wave
  int tots = 0;          // lane j: the sum of row g + j NW
  int acc = 0;
  uint32_t cmeta = 0;
  bool ok = true;

  // Boundary of entry e: wait for its release, write this wave's slice of
  // its activation, wait for all sixteen slices.
  auto boundary = [&](uint32_t e) -> bool {
    if (!lds_wait(&L.released, e + 1, L, a.spin)) return false;
    load_act_slice(tab[e].q, entry_units(tab[e].meta), wave, L, lane);
    return lds_wait(&L.slices, kSeqWaves * (e + 1), L, a.spin);
  };
  // Close entry e: the epilogue of this wave's `rows` rows (lane i: row
  // g + i NW), the outputs, the selection key, then done.
  auto finish = [&](uint32_t e, uint32_t rows, uint32_t meta) {
    const bool bf16 = (meta >> 2) & 1u, res = (meta >> 3) & 1u, sel = (meta >> 4) & 1u;
    if (rows > 0) {
      wait_vm_dyn(vm_ops - rows_at);  // the row values have landed
      const float asc = *cptr(tab[e].asc);
      const float value = dequant(tots, asc, rowws[lane]);
      const size_t row = g + (size_t)lane * NW;
      const bool mine = (uint32_t)lane < rows;
      void* out = tab[e].out;
      if (mine) {
        if (out) store_val(out, row, bf16, value);
        if (res) store_val(tab[e].combined, row, bf16, bf16_rne(rowres[lane] + value));
      }
      if (sel) {
        const uint64_t k = wave_max_u64(mine ? select_key(value, (uint32_t)row) : 0ull);
        if (lane == 0) L.wkey[cw] = k;
      }
    } else if (sel && lane == 0) {
      L.wkey[cw] = 0ull;
    }
    if (lane == 0) __hip_atomic_fetch_add(&L.done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  // Open every entry up to the consume cursor's (those before it hold no
  // row of this wave: they close at once), then set up the cursor's entry.
  auto open_upto = [&]() -> bool {
    for (; open < cs.p; ++open) {
      if (!boundary(open)) return false;
      finish(open, 0, tab[open].meta);
    }
    if (!boundary(open)) return false;
    cmeta = tab[open].meta;
    const uint32_t n = tab[open].n;
    const uint32_t rows = (n - g + NW - 1) / NW;
    const uint32_t r = g + ((uint32_t)lane < rows ? (uint32_t)lane : 0u) * NW;
    issue_row_values(rowws, tab[open].ws + r);
    ++vm_ops;
    if ((cmeta >> 3) & 1u) {
      issue_row_values(rowres, tab[open].residual + r);
      ++vm_ops;
    }
    rows_at = vm_ops;
    j = 0;
    tots = 0;
    ++open;
    return true;
  };

#define W8A8_SEQ_STEP(R)                                                   \
  if (cs.live && ok && open <= cs.p) ok = open_upto();                     \
  if (cs.live && ok) {                                                     \
    if (cs.sub == 0) acc = 0;                                              \
    {                                                                      \
      const int8_t* xa = &L.act[cs.sub * kSeqUnit + lane * 16];            \
      _Pragma("unroll") for (int i = 0; i < 4; ++i)                       \
        acc = dot16(*reinterpret_cast<const v4i*>(xa + i * 1024), R[i], acc); \
    }                                                                      \
    if (cs.sub + 1 == cs.kc) { /* row complete: its sum into lane j */    \
      int s_ = acc;                                                        \
      s_ += __builtin_amdgcn_update_dpp(0, s_, 0xB1, 0xF, 0xF, true);      \
      s_ += __builtin_amdgcn_update_dpp(0, s_, 0x4E, 0xF, 0xF, true);      \
      s_ += __builtin_amdgcn_update_dpp(0, s_, 0x141, 0xF, 0xF, true);     \
      s_ += __builtin_amdgcn_update_dpp(0, s_, 0x140, 0xF, 0xF, true);     \
      const int tot_ = __builtin_amdgcn_readlane(s_, 0) + __builtin_amdgcn_readlane(s_, 16) + \
                       __builtin_amdgcn_readlane(s_, 32) + __builtin_amdgcn_readlane(s_, 48); \
      tots = (uint32_t)lane == j ? tot_ : tots;                            \
      ++j;                                                                 \
    }                                                                      \
    const uint32_t pe_ = cs.p;                                             \
    step_cursor(cs, tab, count, g, NW);                                    \
    if (!cs.live || cs.p != pe_) finish(pe_, j, cmeta);                    \
  }                                                                        \
  /* the slot's refill may not move above the products that read it */   \
  __builtin_amdgcn_sched_barrier(0);                                       \
  issue_unit(R, is, spare, lane);                                          \
  vm_ops += 4;                                                             \
  if (is.live) step_cursor(is, tab, count, g, NW);
  for (;;) {
    W8A8_SEQ_STEP(r0)
    W8A8_SEQ_STEP(r1)
    W8A8_SEQ_STEP(r2)
    W8A8_SEQ_STEP(r3)
    if (!cs.live || !ok) break;
  }
#undef W8A8_SEQ_STEP
  if (!ok) return;
  for (; open < count; ++open) {  // entries past this wave's last row
    if (!boundary(open)) return;
    finish(open, 0, tab[open].meta);
  }
}

// The control side: wave 0.  Entry p's activation is released once every
// workgroup has announced entry p - 1; entry p is announced once this
// workgroup's compute waves are done with it.
__device__ __forceinline__ void seq_control(const SeqArgs& a, SeqLds& L, int lane) {
  Const<SeqEntry> tab = cptr(a.tab);
  const uint32_t G = gridDim.x;
  uint32_t* counter = a.ctl + (blockIdx.x % kSeqGroups) * 64;
  bool ok = true;
  for (uint32_t p = 0; ok && p < a.count; ++p) {
    if (p > 0 && !global_wait(a.ctl, a.base + p, G, L, a.spin)) {
      ok = false;
      break;
    }
    if (lane == 0) __hip_atomic_store(&L.released, p + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    const uint32_t meta = tab[p].meta;
    load_act_slice(tab[p].q, entry_units(meta), 0, L, lane);
    if (!lds_wait(&L.done, kSeqCompute * (p + 1), L, a.spin)) {
      ok = false;
      break;
    }
    const bool select = (meta >> 4) & 1u;
    if (select) {
      // The workgroup's selection key, acknowledged before the arrival so
      // that the reducing workgroup reads it after the barrier.
      uint64_t b = lane < kSeqCompute ? L.wkey[lane] : 0ull;
      b = wave_max_u64(b);
      if (lane == 0) __hip_atomic_store(&a.keys[blockIdx.x], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wait_vm<0>();
    }
    if (lane == 0) __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (select && p + 1 == a.count && blockIdx.x == 0) {
      if (!global_wait(a.ctl, a.base + a.count, G, L, a.spin)) {
        ok = false;
        break;
      }
      uint64_t b = 0;
      for (uint32_t i = lane; i < G; i += 64) {
        const uint64_t k = __hip_atomic_load(&a.keys[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        b = k > b ? k : b;
      }
      b = wave_max_u64(b);
      if (lane == 0) *a.token = key_to_token(b);
    }
  }
  if (!ok) {
    // Stop this workgroup's compute waves and mark the state aborted.
    if (lane == 0) {
      __hip_atomic_store(&L.abort, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_store(a.ctl + kSeqGroups * 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

__global__ __launch_bounds__(64 * kSeqWaves) void seq_kernel(SeqArgs a) {
  __shared__ SeqLds L;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (threadIdx.x == 0) {
    L.released = 0;
    L.slices = 0;
    L.done = 0;
    L.abort = 0;
  }
  __syncthreads();
  // A state left aborted by an earlier call: do nothing (the host resets it).
  if (read_ctl(a.ctl).status != 0) return;
  if (wave == 0)
    seq_control(a, L, lane);
  else
    seq_compute(a, L, wave, lane);
}

uint32_t seq_grid() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, seq_kernel, 64 * kSeqWaves, 0) != hipSuccess)
    return 0;
  return per_cu >= 1 ? (uint32_t)cus : 0u;
}

uint32_t seq_max_rows(uint32_t grid) { return 64u * kSeqCompute * grid; }

hipError_t launch_sequence(hipStream_t st, const SeqEntry* tab, uint32_t count, uint32_t base, uint32_t* ctl,
                           uint64_t* keys, uint32_t* token, uint64_t spin, uint32_t grid) {
  SeqArgs a{tab, count, base, ctl, keys, token, spin};
  hipLaunchKernelGGL(seq_kernel, dim3(grid), dim3(64 * kSeqWaves), 0, st, a);
  return hipGetLastError();
}

}  // namespace w8a8
