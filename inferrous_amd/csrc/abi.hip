// abi.hip -- the extern "C" boundary (include/inferrous_w8a8.h): runtime
// primitives, host-side argument validation and kernel dispatch.
//
// Every entry validates its arguments on the host before any HIP call and
// returns a negative W8A8_E* code on a violation, so misuse never reaches a
// kernel.  HIP failures are returned as the positive hipError_t.  Ops only
// launch kernels on the caller's stream: no allocation, no synchronisation,
// no hipMemsetAsync (zeroing uses a fill kernel), hence graph-capturable.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/inferrous_w8a8.h"
#include "../../include/inferrous_w8a8_diag.h"
#include "internal.hpp"

using namespace w8a8;

// Selection keys of w8a8_linear_argmax_noalloc: a file-scope device array,
// one copy per GPU, held until the process ends.  In host code `scratch` is
// only a stand-in for the symbol; w8a8_init looks up each device's own
// address once (hipGetSymbolAddress, with that device current) and every
// launch uses that address.
static constexpr size_t kNoallocKeys = argmax_keys_for(W8A8_NOALLOC_MAX_ROWS);
static __device__ __align__(256) uint64_t scratch[kNoallocKeys];

namespace {

std::mutex g_init_mu;
std::atomic<uint64_t> g_ready_mask{0};  // devices that passed w8a8_init
std::atomic<void*> g_scratch[64];  // per device: the address of `scratch` below

inline int hip_status(hipError_t e) { return e == hipSuccess ? W8A8_OK : (int)e; }

inline bool ready() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  return (g_ready_mask.load(std::memory_order_acquire) >> dev) & 1u;
}

inline bool al(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

constexpr size_t kU32Max = 0xffffffffu;

int out_align(int dtype) { return dtype == W8A8_OUT_BF16 ? 2 : 4; }

bool valid_dtype(int dtype) {
  return dtype == W8A8_OUT_F32 || dtype == W8A8_OUT_BF16 || dtype == W8A8_OUT_I32;
}

// Common checks of a single projection (q[m,k], asc[m], w[n,k], ws[n]).
int check_linear(const int8_t* q, const float* asc, size_t m, const int8_t* w, const float* ws,
                 size_t n, uint32_t k, const void* out, int out_dtype) {
  if (!valid_dtype(out_dtype)) return W8A8_EARG;
  if (m > kU32Max || n > kU32Max || k == 0 || k % 16 != 0) return W8A8_ESHAPE;
  if (m > 0 && m * (size_t)k / k != m) return W8A8_ESHAPE;
  if (m == 0 || n == 0) return W8A8_OK;
  if (!q || !asc || !w || !ws || !out) return W8A8_ENULL;
  if (!al(q, 16) || !al(w, 16) || !al(asc, 4) || !al(ws, 4) || !al(out, out_align(out_dtype)))
    return W8A8_EALIGN;
  return W8A8_OK;
}

// AUTO route of one projection: the dot4 GEMV at m = 1; at m = 2 the MFMA
// family where it runs gemm_narrow or an unsplit gemm_tall, the dot4 GEMV
// otherwise; the MFMA family from m = 3.  Measured on MI355X through this ABI (graphs of
// 36 distinct-weight launches, random operands), dot4 against MFMA at
// m = 1 / 2 / 3 / 4: qkv 5.46 / 7.35 / 8.58 / 9.00 against 6.92 / 7.00 /
// 7.05 / 7.17 us, o 4.36 / 5.71 / 7.13 / 7.26 against 5.50 / 5.49 / 5.51 /
// 5.54, gate_up 15.85 / 17.58 / 19.69 / 20.59 against 17.15 / 17.16 / 17.19
// / 17.21, down 8.81 / 11.55 / 13.90 / 14.28 against 10.96 / 11.01 / 11.05 /
// 11.09 (gemm_narrow on qkv, o and down, gemm_tall on gate_up).  The other
// MFMA routes at m = 2 (gemm_skinny at K not a multiple of 512, split-K) were
// not measured to lead and keep the GEMV.  A split-K route needs the
// caller's workspace; without it m = 3 and 4 keep the dot4 GEMV.  The grouped
// projections keep one dot4 launch for every matrix up to m = 4 (kDot4MaxM).
constexpr size_t kDot4MaxM = 4;
constexpr size_t kDot4AutoMaxM = 2;
constexpr size_t kRowtailWidthAbi = 12288;  // the down projection's K (the MLP width)

static int auto_path(size_t m, size_t n, uint32_t k, size_t workspace_bytes) {
  if (m < kDot4AutoMaxM) return W8A8_PATH_DOT4;
  if (m > kDot4MaxM) return W8A8_PATH_MFMA;
  const size_t need = gemm_workspace_bytes((uint32_t)m, (uint32_t)n, k);
  if (need != 0 && workspace_bytes < need) return W8A8_PATH_DOT4;
  if (m == kDot4AutoMaxM) {
    GemmArgs g{};
    g.m = (uint32_t)m;
    g.n = (uint32_t)n;
    g.k = k;
    const int family = gemm_route(g).family;
    return family == kRouteNarrow || (family == kRouteTall && need == 0) ? W8A8_PATH_MFMA : W8A8_PATH_DOT4;
  }
  return W8A8_PATH_MFMA;
}

int run_linear(hipStream_t st, const int8_t* q, const float* asc, size_t m, const int8_t* w,
               const float* ws, size_t n, uint32_t k, void* out, int out_dtype, int path,
               const float* residual, void* combined, void* workspace = nullptr,
               size_t workspace_bytes = 0) {
  if (m == 0 || n == 0) return W8A8_OK;
  if (path == W8A8_PATH_AUTO) path = auto_path(m, n, k, workspace ? workspace_bytes : 0);
  if (path == W8A8_PATH_DOT4) {
    GemvArgs a{};
    a.q = q;
    a.asc = asc;
    a.m = (uint32_t)m;
    a.k = k;
    a.count = 1;
    a.w[0] = w;
    a.ws[0] = ws;
    a.n[0] = (uint32_t)n;
    a.out[0] = out;
    a.out_dtype = out_dtype;
    a.residual = residual;
    a.combined = combined;
    return hip_status(launch_gemv(st, a));
  }
  GemmArgs g{};
  g.q = q;
  g.asc = asc;
  g.m = (uint32_t)m;
  g.w = w;
  g.ws = ws;
  g.n = (uint32_t)n;
  g.k = k;
  g.out = out;
  g.out_dtype = out_dtype;
  g.residual = residual;
  g.combined = combined;
  g.partials = static_cast<int32_t*>(workspace);
  g.partial_bytes = workspace ? workspace_bytes : 0;
  return hip_status(launch_gemm(st, g));
}


int check_argmax(const int8_t* q, const float* asc, const int8_t* w, const float* ws, size_t n,
                 uint32_t k, const uint32_t* token, const void* logits, int logits_dtype) {
  if (logits && logits_dtype != W8A8_OUT_F32 && logits_dtype != W8A8_OUT_BF16) return W8A8_EARG;
  if (!token) return W8A8_ENULL;
  if (n > 0) {
    // validate as a 1-row projection; logits are optional
    int s = check_linear(q, asc, 1, w, ws, n, k, logits ? logits : (const void*)token,
                         logits ? logits_dtype : W8A8_OUT_F32);
    if (s != W8A8_OK) return s;
  }
  if (!al(token, 4)) return W8A8_EALIGN;
  return W8A8_OK;
}

int run_argmax(hipStream_t st, const int8_t* q, const float* asc, const int8_t* w, const float* ws,
               size_t n, uint32_t k, uint32_t* token, void* logits, int logits_dtype, uint64_t* keys) {
  GemvArgs a{};
  a.q = q;
  a.asc = asc;
  a.m = 1;
  a.k = k;
  a.count = 1;
  a.w[0] = w;
  a.ws[0] = ws;
  a.n[0] = (uint32_t)n;
  a.out[0] = logits;
  a.out_dtype = logits ? logits_dtype : W8A8_OUT_F32;
  a.slots = keys;
  a.token = token;
  return hip_status(launch_gemv_argmax(st, a));
}

}  // namespace

extern "C" {

int w8a8_abi_version(void) { return W8A8_ABI_VERSION; }

const char* w8a8_status_string(int status) {
  switch (status) {
    case W8A8_OK: return "ok";
    case W8A8_ENULL: return "required pointer is NULL";
    case W8A8_ESHAPE: return "inconsistent or unsupported dimensions";
    case W8A8_EALIGN: return "pointer alignment below requirement";
    case W8A8_EINIT: return "w8a8_init has not succeeded on the current device";
    case W8A8_EWORKSPACE: return "workspace missing or too small";
    case W8A8_EARG: return "invalid enum or flag value";
    case W8A8_ENODEV: return "no usable gfx950 device";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

// ------------------------------------------------------------------ runtime
int w8a8_device_count(int* count) {
  if (!count) return W8A8_ENULL;
  *count = 0;
  int c = 0;
  if (hipGetDeviceCount(&c) != hipSuccess) {
    (void)hipGetLastError();
    return W8A8_OK;
  }
  *count = c;
  return W8A8_OK;
}

int w8a8_init(int device) {
  if (device < 0 || device >= 64) return W8A8_EARG;
  std::lock_guard<std::mutex> lk(g_init_mu);
  int c = 0;
  if (hipGetDeviceCount(&c) != hipSuccess || device >= c) {
    (void)hipGetLastError();
    return W8A8_ENODEV;
  }
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return hip_status(e);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_status(e);
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return W8A8_ENODEV;
  // force code-object load now (device::load) rather than at first launch
  e = hipFree(nullptr);
  if (e != hipSuccess) return hip_status(e);
  if (!g_scratch[device].load(std::memory_order_acquire)) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e);
    if (!p) return W8A8_ENODEV;
    g_scratch[device].store(p, std::memory_order_release);
  }
  g_ready_mask.fetch_or(1ull << device, std::memory_order_acq_rel);
  return W8A8_OK;
}

int w8a8_device_clock_khz(int* khz) {
  if (!khz) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  e = hipDeviceGetAttribute(khz, hipDeviceAttributeClockRate, dev);
  return hip_status(e);
}

int w8a8_device_info(int* cu_count, char* arch_name, size_t arch_len) {
  if (!ready()) return W8A8_EINIT;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return hip_status(e);
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (arch_name && arch_len) {
    std::strncpy(arch_name, prop.gcnArchName, arch_len - 1);
    arch_name[arch_len - 1] = 0;
  }
  return W8A8_OK;
}

int w8a8_stream_create(void** stream) {
  if (!stream) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_status(e);
  *stream = (void*)s;
  return W8A8_OK;
}

int w8a8_stream_destroy(void* stream) {
  if (!stream) return W8A8_ENULL;
  return hip_status(hipStreamDestroy((hipStream_t)stream));
}

int w8a8_stream_synchronize(void* stream) {
  if (!ready()) return W8A8_EINIT;
  return hip_status(hipStreamSynchronize((hipStream_t)stream));
}

int w8a8_malloc(void** ptr, size_t bytes) {
  if (!ptr) return W8A8_ENULL;
  *ptr = nullptr;
  if (!ready()) return W8A8_EINIT;
  if (bytes == 0) bytes = 16;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return hip_status(e);
  e = hipMemset(p, 0, bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_status(e);
  }
  *ptr = p;
  return W8A8_OK;
}

int w8a8_free(void* ptr) {
  if (!ptr) return W8A8_OK;
  return hip_status(hipFree(ptr));
}

int w8a8_host_malloc(void** ptr, size_t bytes) {
  if (!ptr) return W8A8_ENULL;
  *ptr = nullptr;
  if (!ready()) return W8A8_EINIT;
  if (bytes == 0) bytes = 16;
  return hip_status(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
}

int w8a8_host_free(void* ptr) {
  if (!ptr) return W8A8_OK;
  return hip_status(hipHostFree(ptr));
}

int w8a8_memcpy_htod(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return W8A8_OK;
  if (!dst || !src) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
}

int w8a8_memcpy_dtoh(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return W8A8_OK;
  if (!dst || !src) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
}

int w8a8_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return W8A8_OK;
  if (!dst || !src) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
}

int w8a8_fill_zero(void* dst, size_t bytes, void* stream) {
  if (bytes == 0) return W8A8_OK;
  if (!dst) return W8A8_ENULL;
  if (!al(dst, 16)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_fill_zero((hipStream_t)stream, dst, bytes));
}

int w8a8_event_create(void** event) {
  if (!event) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  hipEvent_t e = nullptr;
  hipError_t r = hipEventCreate(&e);
  if (r != hipSuccess) return hip_status(r);
  *event = (void*)e;
  return W8A8_OK;
}

int w8a8_event_destroy(void* event) {
  if (!event) return W8A8_ENULL;
  return hip_status(hipEventDestroy((hipEvent_t)event));
}

int w8a8_event_record(void* event, void* stream) {
  if (!event) return W8A8_ENULL;
  return hip_status(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
}

int w8a8_event_synchronize(void* event) {
  if (!event) return W8A8_ENULL;
  return hip_status(hipEventSynchronize((hipEvent_t)event));
}

int w8a8_event_elapsed_ms(float* ms, void* start, void* stop) {
  if (!ms || !start || !stop) return W8A8_ENULL;
  return hip_status(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
}

int w8a8_graph_capture_begin(void* stream) {
  if (!stream) return W8A8_ENULL;  // the legacy default stream cannot be captured
  if (!ready()) return W8A8_EINIT;
  return hip_status(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
}

int w8a8_graph_capture_end(void* stream, void** graph_exec) {
  if (!stream || !graph_exec) return W8A8_ENULL;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
  if (e != hipSuccess) return hip_status(e);
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_status(e);
  *graph_exec = (void*)x;
  return W8A8_OK;
}

int w8a8_graph_launch(void* graph_exec, void* stream) {
  if (!graph_exec) return W8A8_ENULL;
  return hip_status(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream));
}

int w8a8_graph_destroy(void* graph_exec) {
  if (!graph_exec) return W8A8_ENULL;
  return hip_status(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
}

// ------------------------------------------------------------------ ops
int w8a8_rounding_probe(void* stream, const float* input, size_t n, int8_t* out) {
  if (n == 0) return W8A8_OK;
  if (!input || !out) return W8A8_ENULL;
  if (!al(input, 4)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_rounding_probe((hipStream_t)stream, input, n, out));
}

static int quantize_common(void* stream, const void* x, bool bf16, uint32_t width, size_t rows,
                           int8_t* q, float* scales, uint32_t* maxima_reset) {
  if (rows == 0) return W8A8_OK;
  if (width == 0 || rows > 0x7fffffffu) return W8A8_ESHAPE;
  if (rows * (size_t)width / width != rows) return W8A8_ESHAPE;
  if (!x || !q || !scales) return W8A8_ENULL;
  if (!al(x, bf16 ? 2 : 4) || !al(scales, 4) || !al(maxima_reset, 4)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_quantize((hipStream_t)stream, x, bf16, width, rows, q, scales, maxima_reset));
}

int w8a8_quantize(void* stream, const float* x, uint32_t width, size_t rows, int8_t* q,
                  float* scales, uint32_t* maxima_reset) {
  return quantize_common(stream, x, false, width, rows, q, scales, maxima_reset);
}

int w8a8_quantize_bf16(void* stream, const uint16_t* x, uint32_t width, size_t rows, int8_t* q,
                       float* scales, uint32_t* maxima_reset) {
  return quantize_common(stream, x, true, width, rows, q, scales, maxima_reset);
}

int w8a8_quantize_with_max(void* stream, const float* x, uint32_t width, size_t rows,
                           const uint32_t* maxima, int8_t* q, float* scales) {
  if (rows == 0) return W8A8_OK;
  if (width == 0 || rows * (size_t)width / width != rows) return W8A8_ESHAPE;
  if ((rows * (size_t)width) >> 40) return W8A8_ESHAPE;
  if (!x || !maxima || !q || !scales) return W8A8_ENULL;
  if (!al(x, 4) || !al(maxima, 4) || !al(scales, 4)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_quantize_with_max((hipStream_t)stream, x, width, rows, maxima, q, scales));
}

int w8a8_norm_quantize(void* stream, const float* x, const float* gain, size_t rows, uint32_t width,
                       float* out, int8_t* q, float* scales, uint32_t* maxima) {
  if (width != 4096) return W8A8_ESHAPE;
  if (rows == 0) return W8A8_OK;
  if (rows > kU32Max) return W8A8_ESHAPE;
  if (!x || !gain || !out || !q || !scales || !maxima) return W8A8_ENULL;
  if (!al(x, 4) || !al(gain, 4) || !al(out, 4) || !al(scales, 4) || !al(maxima, 4))
    return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_norm_quantize((hipStream_t)stream, x, gain, rows, out, q, scales, maxima));
}

int w8a8_bf16_pack(const uint16_t* in, size_t n, uint32_t* words, uint32_t* offsets,
                   uint16_t* exceptions, size_t exceptions_cap, size_t* exceptions_len) {
  if (n % 256 != 0 || n > kU32Max) return W8A8_ESHAPE;
  if (!exceptions_len) return W8A8_ENULL;
  if (n > 0 && (!in || !words || !offsets)) return W8A8_ENULL;
  if (!exceptions) return W8A8_ENULL;
  // worst case: every value escapes (and the list holds at least one entry)
  size_t need = 1;
  for (size_t i = 0; i < n; ++i) {
    const uint32_t e = (in[i] >> 7) & 255u;
    need += (e < 109u || e >= 124u);
  }
  if (need > 1) --need;
  if (exceptions_cap < need) return W8A8_EWORKSPACE;
  *exceptions_len = pack_bf16_host(in, n, words, offsets, exceptions);
  return W8A8_OK;
}

int w8a8_head_packed(void* stream, const float* x, size_t x_len, const uint32_t* words,
                     const uint32_t* offsets, const uint16_t* exceptions, size_t exceptions_len,
                     size_t rows, float* out) {
  if (x_len < 4096 || rows > kU32Max / 16 || exceptions_len == 0 || exceptions_len > kU32Max)
    return W8A8_ESHAPE;
  if (rows == 0) return W8A8_OK;
  if (!x || !words || !offsets || !exceptions || !out) return W8A8_ENULL;
  if (!al(x + (x_len - 4096), 16) || !al(words, 4) || !al(offsets, 4) || !al(exceptions, 2) ||
      !al(out, 4))
    return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_head_packed((hipStream_t)stream, x + (x_len - 4096), words, offsets, exceptions,
                                       (uint32_t)exceptions_len, (uint32_t)rows, out));
}

int w8a8_unpack_bf16(void* stream, const uint32_t* words, const uint32_t* offsets,
                     const uint16_t* exceptions, size_t n, uint16_t* out) {
  if (n % 256 != 0) return W8A8_ESHAPE;
  if (n == 0) return W8A8_OK;
  if (!words || !offsets || !exceptions || !out) return W8A8_ENULL;
  if (!al(words, 4) || !al(offsets, 4) || !al(exceptions, 2) || !al(out, 2)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_unpack_bf16((hipStream_t)stream, words, offsets, exceptions, n, out));
}

int w8a8_linear_path(void* stream, const int8_t* q, const float* asc, size_t m, const int8_t* w,
                     const float* ws, size_t n, uint32_t k, void* out, int out_dtype, int path) {
  if (path != W8A8_PATH_AUTO && path != W8A8_PATH_DOT4 && path != W8A8_PATH_MFMA) return W8A8_EARG;
  int s = check_linear(q, asc, m, w, ws, n, k, out, out_dtype);
  if (s != W8A8_OK || m == 0 || n == 0) return s;
  if (!ready()) return W8A8_EINIT;
  return run_linear((hipStream_t)stream, q, asc, m, w, ws, n, k, out, out_dtype, path, nullptr,
                    nullptr);
}

int w8a8_linear(void* stream, const int8_t* q, const float* asc, size_t m, const int8_t* w,
                const float* ws, size_t n, uint32_t k, void* out, int out_dtype) {
  return w8a8_linear_path(stream, q, asc, m, w, ws, n, k, out, out_dtype, W8A8_PATH_AUTO);
}

int w8a8_linear_residual(void* stream, const int8_t* q, const float* asc, size_t m,
                         const int8_t* w, const float* ws, size_t n, uint32_t k,
                         const float* residual, void* out, void* combined, int out_dtype) {
  if (out_dtype != W8A8_OUT_F32 && out_dtype != W8A8_OUT_BF16) return W8A8_EARG;
  int s = check_linear(q, asc, m, w, ws, n, k, out, out_dtype);
  if (s != W8A8_OK || m == 0 || n == 0) return s;
  if (!residual || !combined) return W8A8_ENULL;
  if (!al(residual, 4) || !al(combined, out_align(out_dtype))) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return run_linear((hipStream_t)stream, q, asc, m, w, ws, n, k, out, out_dtype, W8A8_PATH_AUTO,
                    residual, combined);
}

size_t w8a8_linear_workspace_bytes(size_t m, size_t n, uint32_t k) {
  if (m == 0 || m > kU32Max || n > kU32Max) return 0;
  return gemm_workspace_bytes((uint32_t)m, (uint32_t)n, k);
}

size_t w8a8_linear_workspace_bytes_path(size_t m, size_t n, uint32_t k, int path) {
  if (path == W8A8_PATH_DOT4) return 0;
  if (path == W8A8_PATH_AUTO && m <= kDot4AutoMaxM && auto_path(m, n, k, 0) == W8A8_PATH_DOT4)
    return 0;  // AUTO runs the dot4 GEMV there
  if (path != W8A8_PATH_AUTO && path != W8A8_PATH_MFMA) return 0;
  return w8a8_linear_workspace_bytes(m, n, k);
}

size_t w8a8_linear_workspace_bytes_upto(size_t max_m, size_t n, uint32_t k) {
  // The split plans depend on M in both directions (gemm_tall's split-K
  // slabs peak below M = 256 on narrow N), so take every M.
  size_t most = 0;
  if (max_m > kU32Max) max_m = kU32Max;
  for (size_t m = 1; m <= max_m; ++m) most = std::max(most, w8a8_linear_workspace_bytes(m, n, k));
  return most;
}

int w8a8_linear_ex(void* stream, const int8_t* q, const float* asc, size_t m, const int8_t* w,
                   const float* ws, size_t n, uint32_t k, const float* residual, void* out,
                   void* combined, int out_dtype, int path, void* workspace, size_t workspace_bytes) {
  if (path != W8A8_PATH_AUTO && path != W8A8_PATH_DOT4 && path != W8A8_PATH_MFMA) return W8A8_EARG;
  if (residual && out_dtype != W8A8_OUT_F32 && out_dtype != W8A8_OUT_BF16) return W8A8_EARG;
  int s = check_linear(q, asc, m, w, ws, n, k, out, out_dtype);
  if (s != W8A8_OK || m == 0 || n == 0) return s;
  if ((residual == nullptr) != (combined == nullptr)) return W8A8_ENULL;
  if (!al(residual, 4) || !al(combined, out_align(out_dtype)) || !al(workspace, 16))
    return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return run_linear((hipStream_t)stream, q, asc, m, w, ws, n, k, out, out_dtype, path, residual,
                    combined, workspace, workspace_bytes);
}

int w8a8_linear_quantize_with_max(void* stream, const float* x, const uint32_t* maxima, size_t m,
                                  uint32_t k, int8_t* q, float* scales, const int8_t* w,
                                  const float* ws, size_t n, const float* residual, void* out,
                                  void* combined, int out_dtype) {
  if (residual && out_dtype != W8A8_OUT_F32 && out_dtype != W8A8_OUT_BF16) return W8A8_EARG;
  int s = check_linear(q, scales, m, w, ws, n, k, out, out_dtype);
  if (s != W8A8_OK) return s;
  if (m == 0) return W8A8_OK;
  if (!x || !maxima || !q || !scales) return W8A8_ENULL;
  if ((residual == nullptr) != (combined == nullptr)) return W8A8_ENULL;
  if (!al(x, 16) || !al(maxima, 4) || !al(residual, 4) || !al(combined, out_align(out_dtype)))
    return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  // Two stream-ordered launches.  A variant that quantized inside the M = 1
  // GEMV (one launch) measured slower on MI355X: 12.05 us against
  // 9.49 + 1.87 us for the 4096 x 12288 down projection.
  hipStream_t st = (hipStream_t)stream;
  s = hip_status(launch_quantize_with_max(st, x, k, m, maxima, q, scales));
  if (s != W8A8_OK || n == 0) return s;
  return run_linear(st, q, scales, m, w, ws, n, k, out, out_dtype, W8A8_PATH_AUTO, residual, combined);
}

int w8a8_linear_grouped(void* stream, const int8_t* q, const float* asc, size_t m, uint32_t k,
                        int count, const int8_t* const* w, const float* const* ws, const size_t* n,
                        void* const* out, int out_dtype) {
  if (count < 1 || count > kMaxGroup) return W8A8_EARG;
  if (!w || !ws || !n || !out) return W8A8_ENULL;
  for (int i = 0; i < count; ++i) {
    int s = check_linear(q, asc, m, w[i], ws[i], n[i], k, out[i], out_dtype);
    if (s != W8A8_OK) return s;
  }
  if (m == 0) return W8A8_OK;
  if (!ready()) return W8A8_EINIT;
  hipStream_t st = (hipStream_t)stream;
  if (m <= kDot4MaxM) {
    GemvArgs a{};
    a.q = q;
    a.asc = asc;
    a.m = (uint32_t)m;
    a.k = k;
    a.count = count;
    for (int i = 0; i < count; ++i) {
      a.w[i] = w[i];
      a.ws[i] = ws[i];
      a.n[i] = (uint32_t)n[i];
      a.out[i] = out[i];
    }
    a.out_dtype = out_dtype;
    return hip_status(launch_gemv(st, a));
  }
  for (int i = 0; i < count; ++i) {
    int s = run_linear(st, q, asc, m, w[i], ws[i], n[i], k, out[i], out_dtype, W8A8_PATH_MFMA,
                       nullptr, nullptr);
    if (s != W8A8_OK) return s;
  }
  return W8A8_OK;
}

int w8a8_swiglu(void* stream, const void* gate, const void* up, size_t rows, uint32_t width,
                void* act, uint32_t* maxima, int dtype) {
  if (dtype != W8A8_OUT_F32 && dtype != W8A8_OUT_BF16) return W8A8_EARG;
  if (rows == 0 || width == 0) return W8A8_OK;
  if (!gate || !up || !act) return W8A8_ENULL;
  if (rows > SIZE_MAX / width) return W8A8_ESHAPE;
  const size_t a = out_align(dtype);
  if (!al(gate, a) || !al(up, a) || !al(act, a) || !al(maxima, 4)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_swiglu((hipStream_t)stream, gate, up, rows, width, act, dtype, maxima));
}

// linear_swiglu, and with q_out the quantize_with_max of its act that the
// decode chain runs next (src/gpu.rs:377-390).
static int run_swiglu(void* stream, const int8_t* q, const float* asc, size_t m, uint32_t k,
                      const int8_t* w_gate, const float* ws_gate, const int8_t* w_up, const float* ws_up, size_t n,
                      void* gate, void* up, void* act, uint32_t* maxima, int8_t* q_out, float* scales_out,
                      int out_dtype) {
  if (out_dtype != W8A8_OUT_F32 && out_dtype != W8A8_OUT_BF16) return W8A8_EARG;
  int s = check_linear(q, asc, m, w_gate, ws_gate, n, k, gate, out_dtype);
  if (s != W8A8_OK) return s;
  s = check_linear(q, asc, m, w_up, ws_up, n, k, up, out_dtype);
  if (s != W8A8_OK) return s;
  if (m == 0 || n == 0) return W8A8_OK;
  if (!act) return W8A8_ENULL;
  if (q_out && (!maxima || !scales_out)) return W8A8_ENULL;
  if (n > 0xffffffffu) return W8A8_ESHAPE;
  if (!al(act, out_align(out_dtype)) || !al(maxima, 4) || !al(scales_out, 4)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  hipStream_t st = (hipStream_t)stream;
  if (m == 1 && (k == 4096 || k == 12288)) {
    SwigluArgs a{};
    a.q = q;
    a.asc = asc;
    a.k = k;
    a.n = (uint32_t)n;
    a.wg = w_gate;
    a.wsg = ws_gate;
    a.wu = w_up;
    a.wsu = ws_up;
    a.gate = gate;
    a.up = up;
    a.act = act;
    a.out_dtype = out_dtype;
    a.maxima = maxima;
    a.q_out = q_out;
    a.scales_out = scales_out;
    return hip_status(launch_gemv_swiglu(st, a));
  }
  const int8_t* w[2] = {w_gate, w_up};
  const float* ws[2] = {ws_gate, ws_up};
  const size_t nn[2] = {n, n};
  void* out[2] = {gate, up};
  s = w8a8_linear_grouped(stream, q, asc, m, k, 2, w, ws, nn, out, out_dtype);
  if (s != W8A8_OK) return s;
  s = hip_status(launch_swiglu(st, gate, up, m, (uint32_t)n, act, out_dtype, maxima));
  if (s != W8A8_OK || !q_out) return s;
  return hip_status(launch_swiglu_quantize_rows(st, act, m, (uint32_t)n, out_dtype, maxima, q_out, scales_out));
}

int w8a8_linear_swiglu(void* stream, const int8_t* q, const float* asc, size_t m, uint32_t k,
                       const int8_t* w_gate, const float* ws_gate, const int8_t* w_up,
                       const float* ws_up, size_t n, void* gate, void* up, void* act,
                       uint32_t* maxima, int out_dtype) {
  return run_swiglu(stream, q, asc, m, k, w_gate, ws_gate, w_up, ws_up, n, gate, up, act, maxima, nullptr,
                    nullptr, out_dtype);
}

int w8a8_linear_swiglu_quantize(void* stream, const int8_t* q, const float* asc, size_t m, uint32_t k,
                                const int8_t* w_gate, const float* ws_gate, const int8_t* w_up,
                                const float* ws_up, size_t n, void* gate, void* up, void* act,
                                uint32_t* maxima, int8_t* q_out, float* scales_out, int out_dtype) {
  if (!maxima || !q_out || !scales_out) return W8A8_ENULL;
  return run_swiglu(stream, q, asc, m, k, w_gate, ws_gate, w_up, ws_up, n, gate, up, act, maxima, q_out,
                    scales_out, out_dtype);
}

namespace {

bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
  if (!a || !b) return false;
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  return a0 < b0 + bbytes && b0 < a0 + abytes;
}

// The producer (norm_quantize when gain is set, quantize otherwise) of one
// 4096-wide row and the M = 1 linear on its codes, in one launch.
int produce_linear(void* stream, const float* x, const float* gain, float* out_norm, int8_t* q, float* scale,
                   uint32_t* maxima, const int8_t* w, const float* ws, size_t n, const float* residual, void* out,
                   void* combined, int out_dtype) {
  if (!valid_dtype(out_dtype) || (residual && out_dtype == W8A8_OUT_I32)) return W8A8_EARG;
  if (n == 0 || n > kU32Max) return W8A8_ESHAPE;
  if (!x || !q || !scale || !w || !ws || !out) return W8A8_ENULL;
  if ((residual == nullptr) != (combined == nullptr)) return W8A8_ENULL;
  if (!al(x, 4) || !al(gain, 4) || !al(out_norm, 4) || !al(q, 16) || !al(scale, 4) || !al(maxima, 4) ||
      !al(w, 16) || !al(ws, 4) || !al(out, out_align(out_dtype)) || !al(residual, 4) ||
      !al(combined, out_align(out_dtype)))
    return W8A8_EALIGN;
  // Every workgroup reads the row (and the gains) while workgroup 0 and the
  // GEMV write the outputs, so no output may share their bytes.
  const size_t ob = n * (size_t)out_align(out_dtype);
  const struct {
    const void* p;
    size_t bytes;
  } outs[] = {{out_norm, 4096 * 4}, {q, 4096}, {scale, 4}, {maxima, 4}, {out, ob}, {combined, ob}};
  for (const auto& o : outs)
    if (overlaps(x, 4096 * 4, o.p, o.bytes) || overlaps(gain, 4096 * 4, o.p, o.bytes)) return W8A8_EARG;
  if (!ready()) return W8A8_EINIT;
  ProduceArgs p{};
  p.x = x;
  p.gain = gain;
  p.normed = out_norm;
  p.q = q;
  p.scale = scale;
  p.maxima = maxima;
  p.w = w;
  p.ws = ws;
  p.n = (uint32_t)n;
  p.residual = residual;
  p.out = out;
  p.combined = combined;
  p.out_dtype = out_dtype;
  return hip_status(launch_gemv_produce((hipStream_t)stream, p));
}

}  // namespace

int w8a8_norm_quantize_linear(void* stream, const float* x, const float* gain, float* out_norm, int8_t* q,
                              float* scale, uint32_t* maxima, const int8_t* w, const float* ws, size_t n,
                              const float* residual, void* out, void* combined, int out_dtype) {
  if (!gain) return W8A8_ENULL;
  return produce_linear(stream, x, gain, out_norm, q, scale, maxima, w, ws, n, residual, out, combined,
                        out_dtype);
}

int w8a8_norm_quantize_linear_swiglu(void* stream, const float* x, const float* gain, float* out_norm, int8_t* q,
                                     float* scale, const int8_t* w_gate, const float* ws_gate, const int8_t* w_up,
                                     const float* ws_up, size_t n, void* gate, void* up, void* act,
                                     uint32_t* maxima, int8_t* q_out, float* scales_out, int out_dtype) {
  if (out_dtype != W8A8_OUT_F32 && out_dtype != W8A8_OUT_BF16) return W8A8_EARG;
  if (n == 0 || n > kU32Max) return W8A8_ESHAPE;
  if (!x || !gain || !q || !scale || !w_gate || !ws_gate || !w_up || !ws_up || !gate || !up || !act || !maxima)
    return W8A8_ENULL;
  if ((q_out == nullptr) != (scales_out == nullptr)) return W8A8_ENULL;
  const int oa = out_align(out_dtype);
  if (!al(x, 4) || !al(gain, 4) || !al(out_norm, 4) || !al(q, 16) || !al(scale, 4) || !al(w_gate, 16) ||
      !al(ws_gate, 4) || !al(w_up, 16) || !al(ws_up, 4) || !al(gate, oa) || !al(up, oa) || !al(act, oa) ||
      !al(maxima, 4) || !al(scales_out, 4))
    return W8A8_EALIGN;
  const size_t ob = n * (size_t)oa;
  const struct {
    const void* p;
    size_t bytes;
  } outs[] = {{out_norm, 4096 * 4}, {q, 4096}, {scale, 4}, {gate, ob},  {up, ob},
              {act, ob},            {maxima, 4}, {q_out, n}, {scales_out, 4}};
  for (const auto& o : outs)
    if (overlaps(x, 4096 * 4, o.p, o.bytes) || overlaps(gain, 4096 * 4, o.p, o.bytes)) return W8A8_EARG;
  if (!ready()) return W8A8_EINIT;
  ProduceArgs p{};
  p.x = x;
  p.gain = gain;
  p.normed = out_norm;
  p.q = q;
  p.scale = scale;
  p.maxima = maxima;
  SwigluArgs a{};
  a.k = 4096;
  a.n = (uint32_t)n;
  a.wg = w_gate;
  a.wsg = ws_gate;
  a.wu = w_up;
  a.wsu = ws_up;
  a.gate = gate;
  a.up = up;
  a.act = act;
  a.out_dtype = out_dtype;
  a.maxima = maxima;
  a.q_out = q_out;
  a.scales_out = scales_out;
  return hip_status(launch_gemv_swiglu_norm((hipStream_t)stream, p, a, true));
}

int w8a8_norm_quantize_mlp(void* stream, const float* x, const float* gain, float* out_norm, int8_t* q, float* scale,
                           const int8_t* w_gate, const float* ws_gate, const int8_t* w_up, const float* ws_up,
                           size_t n_ff, void* gate, void* up, void* act, int act_dtype, uint32_t* maxima,
                           int8_t* q_act, float* scale_act, const int8_t* w_down, const float* ws_down, size_t n,
                           const float* residual, void* out, void* combined, int out_dtype) {
  if ((act_dtype != W8A8_OUT_F32 && act_dtype != W8A8_OUT_BF16) ||
      (out_dtype != W8A8_OUT_F32 && out_dtype != W8A8_OUT_BF16))
    return W8A8_EARG;
  if (n_ff != kRowtailWidthAbi || n == 0 || n > kU32Max) return W8A8_ESHAPE;
  if (!x || !gain || !q || !scale || !w_gate || !ws_gate || !w_up || !ws_up || !gate || !up || !act || !maxima ||
      !w_down || !ws_down || !out)
    return W8A8_ENULL;
  if ((q_act == nullptr) != (scale_act == nullptr) || (residual == nullptr) != (combined == nullptr))
    return W8A8_ENULL;
  const int aa = out_align(act_dtype), oa = out_align(out_dtype);
  if (!al(x, 4) || !al(gain, 4) || !al(out_norm, 4) || !al(q, 16) || !al(scale, 4) || !al(w_gate, 16) ||
      !al(ws_gate, 4) || !al(w_up, 16) || !al(ws_up, 4) || !al(gate, aa) || !al(up, aa) || !al(act, aa) ||
      !al(maxima, 4) || !al(q_act, 16) || !al(scale_act, 4) || !al(w_down, 16) || !al(ws_down, 4) ||
      !al(residual, 4) || !al(out, oa) || !al(combined, oa))
    return W8A8_EALIGN;
  const size_t ab = n_ff * (size_t)aa, ob = n * (size_t)oa;
  struct Span {
    const void* p;
    size_t bytes;
  };
  // written by the SwiGLU GEMV, and by the down GEMV (which reads act in
  // every workgroup while others write these)
  const Span first[] = {{out_norm, 4096 * 4}, {q, 4096}, {scale, 4}, {gate, ab}, {up, ab}, {act, ab}};
  const Span second[] = {{maxima, 4}, {q_act, n_ff}, {scale_act, 4}, {out, ob}, {combined, ob}};
  for (const Span& o : first)
    if (overlaps(x, 4096 * 4, o.p, o.bytes) || overlaps(gain, 4096 * 4, o.p, o.bytes)) return W8A8_EARG;
  for (const Span& o : second)
    if (overlaps(x, 4096 * 4, o.p, o.bytes) || overlaps(gain, 4096 * 4, o.p, o.bytes) ||
        overlaps(act, ab, o.p, o.bytes))
      return W8A8_EARG;
  if (!ready()) return W8A8_EINIT;
  hipStream_t st = (hipStream_t)stream;
  ProduceArgs p{};
  p.x = x;
  p.gain = gain;
  p.normed = out_norm;
  p.q = q;
  p.scale = scale;
  p.maxima = maxima;
  SwigluArgs a{};
  a.k = 4096;
  a.n = (uint32_t)n_ff;
  a.wg = w_gate;
  a.wsg = ws_gate;
  a.wu = w_up;
  a.wsu = ws_up;
  a.gate = gate;
  a.up = up;
  a.act = act;
  a.out_dtype = act_dtype;
  a.maxima = maxima;
  int s = hip_status(launch_gemv_swiglu_norm(st, p, a, false));
  if (s != W8A8_OK) return s;
  RowtailArgs d{};
  d.act = act;
  d.act_dtype = act_dtype;
  d.maxima = maxima;
  d.q_out = q_act;
  d.scale_out = scale_act;
  d.w = w_down;
  d.ws = ws_down;
  d.n = (uint32_t)n;
  d.residual = residual;
  d.out = out;
  d.combined = combined;
  d.out_dtype = out_dtype;
  return hip_status(launch_gemv_rowtail(st, d));
}

int w8a8_quantize_linear(void* stream, const float* x, uint32_t width, int8_t* q, float* scale,
                         uint32_t* maxima_reset, const int8_t* w, const float* ws, size_t n,
                         const float* residual, void* out, void* combined, int out_dtype) {
  if (width != 4096) return W8A8_ESHAPE;
  return produce_linear(stream, x, nullptr, nullptr, q, scale, maxima_reset, w, ws, n, residual, out, combined,
                        out_dtype);
}

size_t w8a8_select_workspace_bytes(size_t n) {
  (void)n;
  return kSelectBlocks * sizeof(uint64_t);
}

int w8a8_select_token(void* stream, const float* x, size_t n, uint32_t* token, void* workspace,
                      size_t workspace_bytes) {
  if (n > kU32Max) return W8A8_ESHAPE;
  if (!token) return W8A8_ENULL;
  if (n > 0 && !x) return W8A8_ENULL;
  if (!workspace || workspace_bytes < w8a8_select_workspace_bytes(n)) return W8A8_EWORKSPACE;
  if (!al(x, 4) || !al(token, 4) || !al(workspace, 8)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_select((hipStream_t)stream, x, n, (uint64_t*)workspace, token));
}

size_t w8a8_linear_argmax_workspace_bytes(size_t n) {
  return std::max<size_t>(1, argmax_keys_bound(n)) * sizeof(uint64_t);
}


int w8a8_linear_argmax(void* stream, const int8_t* q, const float* asc, const int8_t* w,
                       const float* ws, size_t n, uint32_t k, uint32_t* token, void* logits,
                       int logits_dtype, void* workspace, size_t workspace_bytes) {
  int s = check_argmax(q, asc, w, ws, n, k, token, logits, logits_dtype);
  if (s != W8A8_OK) return s;
  if (!workspace || workspace_bytes < w8a8_linear_argmax_workspace_bytes(n)) return W8A8_EWORKSPACE;
  if (!al(workspace, 8)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return run_argmax((hipStream_t)stream, q, asc, w, ws, n, k, token, logits, logits_dtype,
                    (uint64_t*)workspace);
}

int w8a8_linear_argmax_noalloc(void* stream, const int8_t* q, const float* asc, const int8_t* w,
                               const float* ws, size_t n, uint32_t k, uint32_t* token, void* logits,
                               int logits_dtype) {
  if (n > W8A8_NOALLOC_MAX_ROWS) return W8A8_ESHAPE;
  int s = check_argmax(q, asc, w, ws, n, k, token, logits, logits_dtype);
  if (s != W8A8_OK) return s;
  if (!ready()) return W8A8_EINIT;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return W8A8_EINIT;
  void* keys = g_scratch[dev].load(std::memory_order_acquire);
  if (!keys) return W8A8_EINIT;
  static_assert(kNoallocKeys >= argmax_keys_for(W8A8_NOALLOC_MAX_ROWS), "scratch holds every key");
  return run_argmax((hipStream_t)stream, q, asc, w, ws, n, k, token, logits, logits_dtype,
                    static_cast<uint64_t*>(keys));
}


size_t w8a8_diag_linear_timeline_stamps(size_t n, uint32_t k) {
  if (n > kU32Max) return 0;
  return 3 * gemv_timeline_waves(n, k);
}

int w8a8_diag_linear_timeline(void* stream, const int8_t* q, const float* asc, const int8_t* w,
                              const float* ws, size_t n, uint32_t k, void* out, int out_dtype,
                              uint64_t* stamps, size_t stamps_len) {
  const int c = check_linear(q, asc, 1, w, ws, n, k, out, out_dtype);
  if (c != W8A8_OK) return c;
  if (n == 0) return W8A8_OK;
  const size_t need = w8a8_diag_linear_timeline_stamps(n, k);
  if (need == 0) return W8A8_ESHAPE;  // k other than 4096 / 12288
  if (!stamps) return W8A8_ENULL;
  if (!al(stamps, 8)) return W8A8_EALIGN;
  if (stamps_len < need) return W8A8_EWORKSPACE;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_gemv_timeline((hipStream_t)stream, q, asc, w, ws, (uint32_t)n, k, out, out_dtype,
                                         stamps));
}

static GemmArgs timeline_args(const int8_t* q, const float* asc, size_t m, const int8_t* w, const float* ws,
                               size_t n, uint32_t k, void* out, void* workspace, size_t workspace_bytes) {
  GemmArgs g{};
  g.q = q;
  g.asc = asc;
  g.m = (uint32_t)m;
  g.w = w;
  g.ws = ws;
  g.n = (uint32_t)n;
  g.k = k;
  g.out = out;
  g.out_dtype = W8A8_OUT_BF16;
  g.partials = static_cast<int32_t*>(workspace);
  g.partial_bytes = workspace ? workspace_bytes : 0;
  return g;
}

size_t w8a8_diag_gemm_timeline_stamps(size_t m, size_t n, uint32_t k, size_t workspace_bytes) {
  if (m == 0 || n == 0 || m > kU32Max || n > kU32Max || k == 0 || k % 16 != 0) return 0;
  static const float kDummy[4] = {0.f, 0.f, 0.f, 0.f};
  GemmArgs g = timeline_args(nullptr, nullptr, m, nullptr, nullptr, n, k, nullptr,
                             workspace_bytes ? (void*)kDummy : nullptr, workspace_bytes);
  return 4 * gemm_timeline_waves(g);
}

int w8a8_diag_gemm_timeline(void* stream, const int8_t* q, const float* asc, size_t m, const int8_t* w,
                            const float* ws, size_t n, uint32_t k, void* out, void* workspace,
                            size_t workspace_bytes, uint64_t* stamps, size_t stamps_len) {
  const int c = check_linear(q, asc, m, w, ws, n, k, out, W8A8_OUT_BF16);
  if (c != W8A8_OK) return c;
  if (m == 0 || n == 0) return W8A8_OK;
  if (workspace && !al(workspace, 16)) return W8A8_EALIGN;
  const size_t need = w8a8_diag_gemm_timeline_stamps(m, n, k, workspace ? workspace_bytes : 0);
  if (need == 0) return W8A8_ESHAPE;  // not a gemm_tall route
  if (!stamps) return W8A8_ENULL;
  if (!al(stamps, 8)) return W8A8_EALIGN;
  if (stamps_len < need) return W8A8_EWORKSPACE;
  if (!ready()) return W8A8_EINIT;
  const GemmArgs g = timeline_args(q, asc, m, w, ws, n, k, out, workspace, workspace_bytes);
  return hip_status(launch_gemm_timeline((hipStream_t)stream, g, stamps));
}

// Fixed layout of a route record (include/inferrous_w8a8_diag.h).
static void put_route(int32_t* r, int family, uint32_t gx, uint32_t gy, uint32_t block) {
  for (size_t i = 0; i < W8A8_DIAG_ROUTE_LEN; ++i) r[i] = 0;
  r[0] = family;
  r[1] = (int32_t)gx;
  r[2] = (int32_t)gy;
  r[3] = (int32_t)block;
}

static void put_gemv_route(int32_t* r, const GemvRoute& g) {
  put_route(r, g.family, g.grid_x, g.grid_y, 64u * (uint32_t)g.waves);
  r[11] = g.mt;
  r[13] = g.u;
  r[17] = g.rows;
  r[18] = g.kc;
  r[19] = g.waves;
}

int w8a8_diag_linear_route(size_t m, size_t n, uint32_t k, int out_dtype, int residual, int path,
                           size_t workspace_bytes, int32_t* route, size_t route_len) {
  if (!route) return W8A8_ENULL;
  if (route_len < W8A8_DIAG_ROUTE_LEN) return W8A8_EWORKSPACE;
  if (out_dtype != W8A8_OUT_I32 && out_dtype != W8A8_OUT_F32 && out_dtype != W8A8_OUT_BF16) return W8A8_EARG;
  if (path != W8A8_PATH_AUTO && path != W8A8_PATH_DOT4 && path != W8A8_PATH_MFMA) return W8A8_EARG;
  if (k == 0 || k % 16 != 0 || m > kU32Max || n > kU32Max) return W8A8_ESHAPE;
  if (residual && out_dtype == W8A8_OUT_I32) return W8A8_EARG;
  put_route(route, kRouteNone, 0, 0, 0);
  if (m == 0 || n == 0) return W8A8_OK;
  if (path == W8A8_PATH_AUTO) path = auto_path(m, n, k, workspace_bytes);
  if (path == W8A8_PATH_DOT4) {
    const uint32_t nn = (uint32_t)n;
    put_gemv_route(route, gemv_route((uint32_t)m, k, &nn, 1, false));
    return W8A8_OK;
  }
  // the route taken with 16-byte aligned operands and a workspace of
  // workspace_bytes (a non-null stand-in: only its presence and size count)
  static const float kDummy[4] = {0.f, 0.f, 0.f, 0.f};
  GemmArgs a{};
  a.m = (uint32_t)m;
  a.n = (uint32_t)n;
  a.k = k;
  a.out_dtype = out_dtype;
  a.residual = residual ? kDummy : nullptr;
  a.partials = workspace_bytes ? (int32_t*)kDummy : nullptr;
  a.partial_bytes = workspace_bytes;
  const GemmRoute g = gemm_route(a);
  put_route(route, g.family, g.grid_x, g.grid_y, g.block);
  route[4] = g.bm;
  route[5] = g.bn;
  route[6] = g.wm;
  route[7] = g.wn;
  route[8] = g.sa;
  route[9] = g.sb;
  route[10] = g.ma;
  route[11] = g.mt;
  route[12] = g.s;
  route[13] = g.u;
  route[14] = (int32_t)g.splits;
  route[15] = g.nt_slabs;
  route[16] = g.epi_cols;
  return W8A8_OK;
}

int w8a8_diag_argmax_route(size_t n, uint32_t k, int32_t* route, size_t route_len) {
  if (!route) return W8A8_ENULL;
  if (route_len < W8A8_DIAG_ROUTE_LEN) return W8A8_EWORKSPACE;
  if (k == 0 || k % 16 != 0 || n > kU32Max) return W8A8_ESHAPE;
  put_route(route, kRouteNone, 0, 0, 0);
  if (n == 0) return W8A8_OK;
  const uint32_t nn = (uint32_t)n;
  put_gemv_route(route, gemv_route(1, k, &nn, 1, true));
  return W8A8_OK;
}

int w8a8_synth_i8(void* stream, int8_t* out, size_t n, uint64_t seed, uint64_t stream_id) {
  if (n == 0) return W8A8_OK;
  if (!out) return W8A8_ENULL;
  if (!al(out, 16)) return W8A8_EALIGN;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_synth_i8((hipStream_t)stream, out, n, seed, stream_id));
}

int w8a8_synth_f32(void* stream, float* out, size_t n, uint64_t seed, uint64_t stream_id, float lo,
                   float hi) {
  if (n == 0) return W8A8_OK;
  if (!out) return W8A8_ENULL;
  if (!al(out, 4)) return W8A8_EALIGN;
  if (!(lo <= hi)) return W8A8_EARG;
  if (!ready()) return W8A8_EINIT;
  return hip_status(launch_synth_f32((hipStream_t)stream, out, n, seed, stream_id, lo, hi));
}


// ------------------------------------------------------------ decode sequence
namespace {

struct SeqDevice {
  uint32_t* ctl = nullptr;  // uncached control block (never freed)
  uint32_t base = 0;        // entries every workgroup announced in earlier calls
  uint32_t grid = 0;
};
struct SeqTableInfo {
  size_t count;
  int device;
  bool select;
};
std::mutex g_seq_mu;
SeqDevice g_seq[64];
std::vector<std::pair<const void*, SeqTableInfo>> g_seq_tables;  // prepared tables

constexpr uint64_t kSeqDefaultWaitUs = 100000;
constexpr size_t kSeqStatusIndex = kSeqGroups * 64;  // u32 index of the status word
constexpr size_t kSeqMaxCount = 1u << 20;

int current_device(int* dev) {
  const hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_status(e);
  return *dev >= 0 && *dev < 64 ? W8A8_OK : W8A8_ENODEV;
}

// The device's control block, allocated (uncached, zeroed) on first use.
// Caller holds g_seq_mu.
int seq_device(int dev, SeqDevice** out) {
  SeqDevice& d = g_seq[dev];
  if (!d.ctl) {
    const uint32_t grid = seq_grid();
    if (grid == 0) return W8A8_ENODEV;
    void* p = nullptr;
    hipError_t e = hipExtMallocWithFlags(&p, kSeqCtlBytes, hipDeviceMallocUncached);
    if (e != hipSuccess) return hip_status(e);
    e = hipMemset(p, 0, kSeqCtlBytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_status(e);  // the block stays allocated: uncached memory is never freed
    d.ctl = (uint32_t*)p;
    d.grid = grid;
    d.base = 0;
  }
  *out = &d;
  return W8A8_OK;
}

}  // namespace

size_t w8a8_linear_sequence_table_bytes(size_t count) { return count * sizeof(SeqEntry); }

size_t w8a8_linear_sequence_workspace_bytes(void) {
  if (!ready()) return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return (size_t)cus * sizeof(uint64_t);
}

int w8a8_linear_sequence_prepare(const w8a8_seq_entry* entries, size_t count, void* table, size_t table_bytes) {
  if (!entries || !table) return W8A8_ENULL;
  if (count == 0 || count > kSeqMaxCount) return W8A8_ESHAPE;
  if (table_bytes < w8a8_linear_sequence_table_bytes(count)) return W8A8_EWORKSPACE;
  if (!al(table, 16)) return W8A8_EALIGN;
  // host-side checks of every entry first
  for (size_t i = 0; i < count; ++i) {
    const w8a8_seq_entry& e = entries[i];
    if (e.flags & ~W8A8_SEQ_SELECT) return W8A8_EARG;
    const bool select = e.flags & W8A8_SEQ_SELECT;
    if (select && i + 1 != count) return W8A8_EARG;  // only the last entry selects
    if (e.out_dtype != W8A8_OUT_F32 && e.out_dtype != W8A8_OUT_BF16) return W8A8_EARG;
    if (e.k != 4096 && e.k != 8192 && e.k != 12288) return W8A8_ESHAPE;
    if (e.n == 0 || e.n > kU32Max) return W8A8_ESHAPE;
    if (!e.w || !e.ws || !e.q || !e.asc) return W8A8_ENULL;
    if (!e.out && !select) return W8A8_ENULL;
    if ((e.residual == nullptr) != (e.combined == nullptr)) return W8A8_ENULL;
    if (select && e.residual) return W8A8_EARG;
    if (!al(e.w, 16) || !al(e.q, 16) || !al(e.ws, 4) || !al(e.asc, 4) || !al(e.out, out_align(e.out_dtype)) ||
        !al(e.residual, 4) || !al(e.combined, out_align(e.out_dtype)))
      return W8A8_EALIGN;
  }
  if (!ready()) return W8A8_EINIT;
  int dev = 0;
  int st = current_device(&dev);
  if (st != W8A8_OK) return st;
  std::lock_guard<std::mutex> lk(g_seq_mu);
  SeqDevice* d = nullptr;
  st = seq_device(dev, &d);
  if (st != W8A8_OK) return st;
  std::vector<SeqEntry> host(count);
  for (size_t i = 0; i < count; ++i) {
    const w8a8_seq_entry& e = entries[i];
    if (e.n > seq_max_rows(d->grid)) return W8A8_ESHAPE;  // 64 rows per wave at most
    SeqEntry& t = host[i];
    t.w = e.w;
    t.ws = e.ws;
    t.q = e.q;
    t.asc = e.asc;
    t.out = e.out;
    t.residual = e.residual;
    t.combined = e.combined;
    t.n = (uint32_t)e.n;
    t.meta = (e.k / 4096) | (e.out_dtype == W8A8_OUT_BF16 ? 4u : 0u) | (e.residual ? 8u : 0u) |
             ((e.flags & W8A8_SEQ_SELECT) ? 16u : 0u);
  }
  const hipError_t e = hipMemcpy(table, host.data(), count * sizeof(SeqEntry), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_status(e);
  const SeqTableInfo info{count, dev, (entries[count - 1].flags & W8A8_SEQ_SELECT) != 0};
  for (auto& t : g_seq_tables)
    if (t.first == table) {
      t.second = info;
      return W8A8_OK;
    }
  g_seq_tables.emplace_back(table, info);
  return W8A8_OK;
}

int w8a8_linear_sequence(void* stream, const void* table, size_t count, uint32_t* token, void* workspace,
                         size_t workspace_bytes, uint32_t wait_us) {
  if (!table) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  int dev = 0;
  int st = current_device(&dev);
  if (st != W8A8_OK) return st;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing((hipStream_t)stream, &cap);
  if (e != hipSuccess) return hip_status(e);
  if (cap != hipStreamCaptureStatusNone) return W8A8_EARG;  // the launch argument `base` changes per call
  std::lock_guard<std::mutex> lk(g_seq_mu);
  const SeqTableInfo* info = nullptr;
  for (const auto& t : g_seq_tables)
    if (t.first == table) info = &t.second;
  if (!info || info->count != count || info->device != dev) return W8A8_EARG;  // not prepared here
  SeqDevice* d = nullptr;
  st = seq_device(dev, &d);
  if (st != W8A8_OK) return st;
  if (info->select) {
    if (!token || !workspace) return W8A8_ENULL;
    if (!al(token, 4) || !al(workspace, 8)) return W8A8_EALIGN;
    if (workspace_bytes < (size_t)d->grid * sizeof(uint64_t)) return W8A8_EWORKSPACE;
  }
  const uint64_t ticks = (wait_us ? (uint64_t)wait_us : kSeqDefaultWaitUs) * 100;  // 100 MHz clock
  e = launch_sequence((hipStream_t)stream, (const SeqEntry*)table, (uint32_t)count, d->base, d->ctl,
                      (uint64_t*)workspace, token, ticks, d->grid);
  if (e != hipSuccess) return hip_status(e);
  d->base += (uint32_t)count;
  return W8A8_OK;
}

int w8a8_linear_sequence_status(uint32_t* status) {
  if (!status) return W8A8_ENULL;
  if (!ready()) return W8A8_EINIT;
  int dev = 0;
  int st = current_device(&dev);
  if (st != W8A8_OK) return st;
  std::lock_guard<std::mutex> lk(g_seq_mu);
  *status = 0;
  if (!g_seq[dev].ctl) return W8A8_OK;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(status, g_seq[dev].ctl + kSeqStatusIndex, 4, hipMemcpyDeviceToHost);
  return hip_status(e);
}

int w8a8_linear_sequence_reset(void) {
  if (!ready()) return W8A8_EINIT;
  int dev = 0;
  int st = current_device(&dev);
  if (st != W8A8_OK) return st;
  std::lock_guard<std::mutex> lk(g_seq_mu);
  SeqDevice& d = g_seq[dev];
  if (!d.ctl) return W8A8_OK;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemset(d.ctl, 0, kSeqCtlBytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_status(e);
  d.base = 0;
  return W8A8_OK;
}

}  // extern "C"
