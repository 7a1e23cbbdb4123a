// awq_api.hip -- host side of libcube_awq_gfx950: the reference's launch-time
// validation, the m_valid / decode-prefill dispatch rule, the module-level
// tile selection, a per-stream workspace, and the extern "C" ABI of awq.h.
#include <atomic>
#include <map>
#include <mutex>
#include <set>
#include <sstream>
#include <vector>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <utility>

#include "awq_common.h"

namespace cube_awq {

// ---------------------------------------------------------------------------
// Errors
// ---------------------------------------------------------------------------
static thread_local std::string g_last_error;

[[noreturn]] void panic(const std::string& msg) { throw Panic{msg}; }

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::ostringstream os;
    os << what << ": " << hipGetErrorString(e) << " (" << (int)e << ")";
    throw HipFailure{os.str()};
  }
}

std::string assert_eq_text(const std::string& msg, long long left, long long right) {
  std::ostringstream os;
  os << "assertion `left == right` failed: " << msg << "\n  left: " << left << "\n right: " << right;
  return os.str();
}

template <class Fn>
static int guarded(Fn&& fn) {
  try {
    fn();
    g_last_error.clear();
    return AWQ_OK;
  } catch (const Panic& p) {
    g_last_error = p.msg;
    return AWQ_ERR_INVALID;
  } catch (const HipFailure& h) {
    g_last_error = h.msg;
    return AWQ_ERR_HIP;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return AWQ_ERR_HIP;
  }
}

// ---------------------------------------------------------------------------
// Constants of the reference (src/kernel/awq_kernel_gemm.rs:81-87,
// src/modules/awq_gemm.rs:12-18).
// ---------------------------------------------------------------------------
constexpr int64_t kDecodeMThreshold = 8;
constexpr int64_t kDecodeTileM = 8;
constexpr int64_t kRowsPerThread = 2;
constexpr int64_t kNLinesPerThread = 2;
constexpr int64_t kRowsPerThreadDecode = 1;
constexpr int64_t kNLinesPerThreadDecode = 4;
constexpr int64_t kTileNBase = 32, kTileNMedium = 64, kTileNLarge = 128;
constexpr int64_t kInnerK = 64;
constexpr int64_t kTileMSmall = 16, kTileMLarge = 32;

// Rust usize divisibility with `is_multiple_of` semantics (x % 0 is "multiple"
// only for x == 0).
static bool multiple_of(int64_t x, int64_t d) { return d == 0 ? x == 0 : x % d == 0; }

// validate_launch_params_impl, src/kernel/awq_kernel_gemm.rs:89-158, same
// order and messages. Negative sizes (impossible with Rust usize) are rejected
// first.
static void validate_impl(const awq_shape_config& s, int64_t group_size, int64_t rows_per_thread,
                          int64_t n_lines_per_thread) {
  AWQ_ASSERT(s.k >= 0 && s.n >= 0 && s.m_valid >= 0, "shape sizes must be non-negative");
  AWQ_ASSERT(s.m > 0, "m must be > 0");
  AWQ_ASSERT(s.line_size > 0, "line_size must be > 0");
  AWQ_ASSERT(s.tile_m > 0, "m_tile_size must be > 0");
  AWQ_ASSERT(s.tile_n > 0, "n_tile_size must be > 0");
  AWQ_ASSERT(s.inner_k > 0, "inner_k_size must be > 0");
  AWQ_ASSERT(group_size > 0, "group_size must be > 0");

  AWQ_ASSERT(multiple_of(s.k, s.line_size), "k must be divisible by line_size");
  AWQ_ASSERT(multiple_of(s.n, s.line_size), "n must be divisible by line_size");
  AWQ_ASSERT(multiple_of(s.inner_k, s.line_size), "inner_k_size must be divisible by line_size");

  AWQ_ASSERT(multiple_of(s.n, s.tile_n), "n must be divisible by n_tile_size");
  AWQ_ASSERT(multiple_of(s.k, s.inner_k), "k must be divisible by inner_k_size");

  AWQ_ASSERT(multiple_of(s.tile_n, s.line_size * 8), "n_tile_size must be divisible by line_size*8");
  AWQ_ASSERT(multiple_of(s.n, s.line_size * 8), "n must be divisible by line_size*8");

  AWQ_ASSERT(multiple_of(s.k, group_size), "k must be divisible by group_size");
  AWQ_ASSERT(group_size >= s.inner_k && multiple_of(group_size, s.inner_k),
             "fast path requires group_size >= inner_k_size and divisible by inner_k_size");
  AWQ_ASSERT(s.m_valid <= s.m, "m_valid must be <= m");

  AWQ_ASSERT(multiple_of(s.tile_n, s.line_size * n_lines_per_thread),
             "tile_n must be divisible by line_size * N_LINES_PER_THREAD");
  AWQ_ASSERT(multiple_of(s.tile_m, rows_per_thread),
             "m_tile_size must be divisible by ROWS_PER_THREAD");
}

static void validate_prefill(const awq_shape_config& s, int64_t g) {
  validate_impl(s, g, kRowsPerThread, kNLinesPerThread);
}
static void validate_decode(const awq_shape_config& s, int64_t g) {
  validate_impl(s, g, kRowsPerThreadDecode, kNLinesPerThreadDecode);
}

// ---------------------------------------------------------------------------
// Tuning overrides, read once per process (and by awq_tuning_reload()).
// ---------------------------------------------------------------------------
static const char* const kTuneNames[kTuneCount] = {
    "AWQ_GEMM_TILE",  "AWQ_GEMM_SPLITS", "AWQ_GEMM_GROUP_M", "AWQ_F32_SLICES",  "AWQ_GEMV_WAVES",
    "AWQ_GEMV_RPW",   "AWQ_MFMA_WAVES",  "AWQ_MFMA_RPW",     "AWQ_M4_WAVES",    "AWQ_M4_RPW",
    "AWQ_DECODE_MFMA", "AWQ_DECODE_M4",  "AWQ_SMALLM_MFMA",  "AWQ_SKINNY",      "AWQ_SKINNY_SPLITS",
    "AWQ_SKINNY_COLS", "AWQ_DECODE_TREE", "AWQ_SKINNY_TREE"};
static std::atomic<int> g_tune_val[kTuneCount];
static std::atomic<bool> g_tune_set[kTuneCount];
static std::once_flag g_tune_once;

// Rust's char::is_whitespace (the Unicode White_Space property), which
// str::trim strips from both ends.
static bool rust_whitespace(uint32_t c) {
  return (c >= 0x09 && c <= 0x0D) || c == 0x20 || c == 0x85 || c == 0xA0 || c == 0x1680 ||
         (c >= 0x2000 && c <= 0x200A) || c == 0x2028 || c == 0x2029 || c == 0x202F ||
         c == 0x205F || c == 0x3000;
}

// Decode UTF-8 (strictly: no overlongs, surrogates or values past U+10FFFF);
// false for bytes that std::env::var would reject as not Unicode.
static bool utf8_decode(const char* s, std::vector<uint32_t>& out) {
  const unsigned char* p = reinterpret_cast<const unsigned char*>(s);
  while (*p) {
    uint32_t c = *p, need = 0, min = 0;
    if (c < 0x80) { need = 0; }
    else if ((c & 0xE0) == 0xC0) { c &= 0x1F; need = 1; min = 0x80; }
    else if ((c & 0xF0) == 0xE0) { c &= 0x0F; need = 2; min = 0x800; }
    else if ((c & 0xF8) == 0xF0) { c &= 0x07; need = 3; min = 0x10000; }
    else return false;
    ++p;
    for (uint32_t i = 0; i < need; ++i, ++p) {
      if ((*p & 0xC0) != 0x80) return false;
      c = (c << 6) | (*p & 0x3F);
    }
    if (need && c < min) return false;
    if (c > 0x10FFFF || (c >= 0xD800 && c <= 0xDFFF)) return false;
    out.push_back(c);
  }
  return true;
}

// AWQ_GEMM_FORCE_TILE_M as the reference reads it (src/modules/awq_gemm.rs:
// 20-28): std::env::var (absent or not Unicode -> no override), then
// raw.trim().parse::<usize>() (an optional '+', ASCII digits, no overflow of
// a 64-bit usize), kept only if it is 8, 16 or 32.
static int64_t parse_forced_tile_m(const char* raw) {
  if (!raw) return 0;
  std::vector<uint32_t> cp;
  if (!utf8_decode(raw, cp)) return 0;
  size_t b = 0, e = cp.size();
  while (b < e && rust_whitespace(cp[b])) ++b;
  while (e > b && rust_whitespace(cp[e - 1])) --e;
  if (b < e && cp[b] == '+') ++b;
  if (b == e) return 0;
  uint64_t v = 0;
  for (size_t i = b; i < e; ++i) {
    if (cp[i] < '0' || cp[i] > '9') return 0;
    const uint64_t d = cp[i] - '0';
    if (v > (UINT64_MAX - d) / 10) return 0;  // usize overflow: parse error
    v = v * 10 + d;
  }
  return (v == 8 || v == 16 || v == 32) ? (int64_t)v : 0;
}

static void tuning_read() {
  for (int i = 0; i < kTuneCount; ++i) {
    const char* e = std::getenv(kTuneNames[i]);
    g_tune_val[i].store(e ? std::atoi(e) : 0, std::memory_order_relaxed);
    g_tune_set[i].store(e != nullptr, std::memory_order_relaxed);
  }
}

int tuning(TuneKey key, int dflt) {
  std::call_once(g_tune_once, tuning_read);
  return g_tune_set[key].load(std::memory_order_relaxed) ? g_tune_val[key].load(std::memory_order_relaxed)
                                                         : dflt;
}

// Read once per process, like the reference's OnceLock (awq_tuning_reload()
// does not re-read it).
static int64_t forced_tile_m() {
  static const int64_t forced = parse_forced_tile_m(std::getenv("AWQ_GEMM_FORCE_TILE_M"));
  return forced;
}

// select_tile_m / select_tile_n, src/modules/awq_gemm.rs:20-52.
static int64_t select_tile_m(int64_t m) {
  if (int64_t f = forced_tile_m()) return f;
  if (m <= kDecodeMThreshold) return kDecodeTileM;
  if (m <= kTileMSmall) return kTileMSmall;
  return kTileMLarge;
}

static int64_t select_tile_n(int64_t n) {
  if (n >= kTileNLarge && n % kTileNLarge == 0) return kTileNLarge;
  if (n >= kTileNMedium && n % kTileNMedium == 0) return kTileNMedium;
  return kTileNBase;
}

static void check_aligned(const void* p, const char* what) {
  if (p && (reinterpret_cast<uintptr_t>(p) & 15u) != 0) {
    panic(std::string(what) + " must be 16-byte aligned");
  }
}

static void check_float_dtype(int32_t t, const char* what) {
  if (!is_float_dtype(t)) panic(std::string(what) + " must have f32/f16/bf16 dtype");
}

// Run the GEMM over validated sizes: rows = m_valid; M <= 8 (and 9..16 when
// the matrix-core decode kernel takes them) -> GEMV, else the prefill kernels.
static void run_gemm(GemmProblem p, int64_t launch_m) {
  check_aligned(p.x, "input");
  check_aligned(p.qweight, "qweight");
  check_aligned(p.qzeros, "qzeros");
  check_aligned(p.scales, "scales");
  check_aligned(p.y, "output");
  if (p.bias) check_aligned(p.bias, "bias");
  if (p.rows <= 0 || p.N == 0) return;
  if (launch_m <= kDecodeMThreshold || small_m_mfma_ok(p, launch_m)) {
    launch_gemv(p);
  } else {
    launch_gemm(p);
  }
}

// ---------------------------------------------------------------------------
// Workspace: one device buffer per (device, stream, slot). Calls on one
// stream are ordered, so reuse within a stream is safe; calls on different
// streams get different buffers. A graph captured on a stream keeps the
// buffers that stream had at capture time, so a buffer is never freed: when
// a call needs more, a new buffer (at least twice the old size) replaces it
// for later calls and the old one is retired, alive until the process ends.
// ---------------------------------------------------------------------------
struct WsKey {
  int device;
  hipStream_t stream;
  int slot;
  bool operator<(const WsKey& o) const {
    if (device != o.device) return device < o.device;
    if (stream != o.stream) return std::less<void*>()(stream, o.stream);
    return slot < o.slot;
  }
};
struct WsBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
};
static std::mutex g_ws_mu;
static std::map<WsKey, WsBuf>& ws_map() {
  static auto* m = new std::map<WsKey, WsBuf>();  // never destroyed: no frees at exit
  return *m;
}
static std::vector<void*>& ws_retired() {
  static auto* v = new std::vector<void*>();  // superseded buffers, kept for captured graphs
  return *v;
}

int64_t device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (!v) {
    check_hip(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    if (v <= 0) v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

void ensure_dyn_smem(const void* kernel, int bytes, const char* what) {
  static std::mutex mu;
  static auto* done = new std::set<std::pair<int, const void*>>();
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lk(mu);
  if (done->count({dev, kernel})) return;
  check_hip(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes), what);
  done->insert({dev, kernel});
}

void* workspace_get(hipStream_t stream, size_t bytes, int slot) {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  WsBuf& b = ws_map()[WsKey{dev, stream, slot}];
  if (b.bytes < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    check_hip(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
      panic("the split-K workspace of this stream must be allocated before graph capture: "
            "make one call of the same or a larger shape on this stream outside the capture");
    size_t want = bytes < (1u << 16) ? (size_t)(1u << 16) : bytes;
    if (want < 2 * b.bytes) want = 2 * b.bytes;
    want = (want + 4095) & ~(size_t)4095;
    void* fresh = nullptr;
    check_hip(hipMalloc(&fresh, want), "workspace hipMalloc");
    if (slot == kWsCounters) {
      // Arrival counters must start at zero; every kernel leaves them at zero.
      check_hip(hipMemsetAsync(fresh, 0, want, stream), "workspace hipMemsetAsync");
    }
    // Work already queued (or captured) with the old buffer keeps using it.
    if (b.ptr) ws_retired().push_back(b.ptr);
    b.ptr = fresh;
    b.bytes = want;
  }
  return b.ptr;
}

// ---------------------------------------------------------------------------
// Static split-K scratch of awq_gemm_noalloc: a file-scope device array,
// one copy per GPU, held for the life of the process: 1 MiB of arrival
// counters (zero between calls: every split-K kernel re-arms the counters it
// uses), 63 MiB of fp32 partial sums, and 64 MiB for fp32 activations split
// into f16 hi + lo rows (the fp32 prefill's prepass). Host code never names the
// array itself (its host-side name is not a device address): its address on
// each device comes from hipGetSymbolAddress, looked up once per device on
// the first awq_gemm_noalloc call there, which also clears the counters with
// a fill kernel on the caller's stream.
// ---------------------------------------------------------------------------
constexpr size_t kScratchCounterBytes = size_t(1) << 20;
constexpr size_t kScratchPartialBytes = (size_t(63) << 20);
constexpr size_t kScratchXSplitBytes = size_t(64) << 20;
constexpr size_t kScratchBytes = kScratchCounterBytes + kScratchPartialBytes + kScratchXSplitBytes;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void fill_zero_u32(uint32_t* p, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

static void* scratch_on_device(hipStream_t stream) {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) panic("awq_gemm_noalloc: device index out of range (0..63)");
  std::lock_guard<std::mutex> lk(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "awq_gemm_noalloc: hipGetSymbolAddress(scratch)");
    if (!ptr) panic("awq_gemm_noalloc: hipGetSymbolAddress(scratch) returned null");
    const uint32_t words = (uint32_t)(kScratchCounterBytes / 4);
    hipLaunchKernelGGL(fill_zero_u32, dim3(256), dim3(256), 0, stream, static_cast<uint32_t*>(ptr), words);
    check_hip(hipGetLastError(), "awq_gemm_noalloc: clearing the scratch counters");
    ptrs[dev] = ptr;
  }
  return ptrs[dev];
}

void* ws_get(const GemmProblem& p, size_t bytes, int slot) {
  if (!p.scratch) return workspace_get(p.stream, bytes, slot);
  const size_t cap = slot == kWsCounters ? kScratchCounterBytes
                   : slot == kWsPartials ? kScratchPartialBytes : kScratchXSplitBytes;
  const size_t off = slot == kWsCounters ? 0
                   : slot == kWsPartials ? kScratchCounterBytes : kScratchCounterBytes + kScratchPartialBytes;
  if (bytes > cap) {
    std::ostringstream os;
    os << "awq_gemm_noalloc: this call needs " << bytes << " bytes of "
       << (slot == kWsCounters ? "split-K counters" : slot == kWsPartials ? "split-K partial sums"
                                                                          : "split fp32 activations")
       << ", more than the " << cap << " bytes of the static scratch (awq_gemm has no such limit)";
    panic(os.str());
  }
  return static_cast<char*>(p.scratch) + off;
}

static int64_t numel(const awq_tensor_ref& t) {
  int64_t n = 1;
  for (int i = 0; i < t.rank; ++i) n *= t.shape[i];
  return n;
}

static void check_ref(const awq_tensor_ref* t, const char* what) {
  if (!t) panic(std::string(what) + " tensor reference is null");
  if (t->rank < 0 || t->rank > 8 || (t->rank > 0 && !t->shape))
    panic(std::string(what) + " tensor reference has an invalid shape");
  for (int i = 0; i < t->rank; ++i)
    if (t->shape[i] < 0) panic(std::string(what) + " tensor shape must be non-negative");
}

}  // namespace cube_awq

using namespace cube_awq;

extern "C" {

awq_shape_config awq_shape_config_new(int64_t m, int64_t n, int64_t k, int64_t m_tile_size,
                                      int64_t n_tile_size, int64_t inner_k_size) {
  return awq_shape_config_new_with_valid_m(m, n, k, m_tile_size, n_tile_size, inner_k_size, m);
}

awq_shape_config awq_shape_config_new_with_valid_m(int64_t m, int64_t n, int64_t k,
                                                   int64_t m_tile_size, int64_t n_tile_size,
                                                   int64_t inner_k_size, int64_t m_valid) {
  awq_shape_config s;
  s.m = m;
  s.k = k;
  s.n = n;
  s.tile_m = m_tile_size;
  s.tile_n = n_tile_size;
  s.inner_k = inner_k_size;
  s.line_size = 4;
  s.m_valid = m_valid;
  return s;
}

int awq_validate_launch_params(const awq_shape_config* shape, int64_t group_size) {
  return guarded([&] {
    if (!shape) panic("shape is null");
    validate_prefill(*shape, group_size);
  });
}

int awq_validate_decode_launch_params(const awq_shape_config* shape, int64_t group_size) {
  return guarded([&] {
    if (!shape) panic("shape is null");
    validate_decode(*shape, group_size);
  });
}

// awq_gemm_linear, src/kernel/awq_kernel_gemm.rs:626-771.
int awq_gemm_linear(const awq_tensor_ref* input, const awq_tensor_ref* qweight,
                    const awq_tensor_ref* qzeros, const awq_tensor_ref* scales,
                    const awq_tensor_ref* output, const awq_shape_config* shape,
                    int64_t group_size, void* stream) {
  return guarded([&] {
    check_ref(input, "input");
    check_ref(qweight, "qweight");
    check_ref(qzeros, "qzeros");
    check_ref(scales, "scales");
    check_ref(output, "output");
    if (!shape) panic("shape is null");

    AWQ_ASSERT(input->rank >= 2, "input must have shape [.., M, K] or [M, K]");
    AWQ_ASSERT(qweight->rank >= 2, "qweight must have shape [K, N/8]");
    AWQ_ASSERT(qzeros->rank >= 2, "qzeros must have shape [K/G, N/8]");
    AWQ_ASSERT(scales->rank >= 2, "scales must have shape [K/G, N]");
    AWQ_ASSERT(output->rank >= 2, "output must have shape [.., M, N] or [M, N]");

    const int64_t input_k = input->shape[input->rank - 1];
    AWQ_ASSERT(input_k > 0, "input K must be > 0");
    AWQ_ASSERT_EQ(input_k, shape->k, "input K must match shape.k");

    const int64_t input_numel = numel(*input);
    const int64_t launch_m = input_numel / input_k;
    AWQ_ASSERT_EQ(input_numel % input_k, 0, "input elements must be divisible by K");

    const int64_t output_n = output->shape[output->rank - 1];
    AWQ_ASSERT(output_n > 0, "output N must be > 0");
    AWQ_ASSERT_EQ(output_n, shape->n, "output N must match shape.n");
    const int64_t output_numel = numel(*output);
    const int64_t output_rows = output_numel / output_n;
    AWQ_ASSERT_EQ(output_numel % output_n, 0, "output elements must be divisible by N");
    AWQ_ASSERT_EQ(output_rows, launch_m, "output rows must match flattened input rows");

    // m_valid rule, :675-690.
    int64_t launch_m_valid;
    if (shape->m == launch_m) {
      launch_m_valid = shape->m_valid;
    } else if (shape->m > 0 && launch_m % shape->m == 0 && shape->m_valid == shape->m) {
      launch_m_valid = launch_m;
    } else {
      launch_m_valid = launch_m < shape->m_valid ? launch_m : shape->m_valid;
    }
    awq_shape_config ls = awq_shape_config_new_with_valid_m(
        launch_m, shape->n, shape->k, shape->tile_m, shape->tile_n, shape->inner_k, launch_m_valid);
    ls.line_size = shape->line_size;
    const bool use_decode = ls.m <= kDecodeMThreshold;
    if (use_decode) validate_decode(ls, group_size);
    else validate_prefill(ls, group_size);

    const int64_t num_groups = ls.k / group_size;
    AWQ_ASSERT_EQ(qweight->shape[0], ls.k, "qweight K must match shape.k");
    AWQ_ASSERT_EQ(qweight->shape[1], ls.n / 8, "qweight packed N must be N/8");
    AWQ_ASSERT_EQ(qzeros->shape[0], num_groups, "qzeros rows must be K/group_size");
    AWQ_ASSERT_EQ(qzeros->shape[1], ls.n / 8, "qzeros packed N must be N/8");
    AWQ_ASSERT_EQ(scales->shape[0], num_groups, "scales rows must be K/group_size");
    AWQ_ASSERT_EQ(scales->shape[1], ls.n, "scales N must match shape.n");
    // The reference reads these through linear views of the whole buffer; a
    // rank > 2 packed tensor would alias, so require exactly the 2-D sizes.
    AWQ_ASSERT_EQ(numel(*qweight), ls.k * (ls.n / 8), "qweight must have shape [K, N/8]");
    AWQ_ASSERT_EQ(numel(*qzeros), num_groups * (ls.n / 8), "qzeros must have shape [K/G, N/8]");
    AWQ_ASSERT_EQ(numel(*scales), num_groups * ls.n, "scales must have shape [K/G, N]");

    // Element types (the reference's module checks these, src/modules/awq_gemm.rs:177-184).
    AWQ_ASSERT(qweight->dtype == AWQ_U32 || qweight->dtype == AWQ_I32,
               "qweight must have i32/u32 dtype");
    AWQ_ASSERT(qzeros->dtype == AWQ_U32 || qzeros->dtype == AWQ_I32,
               "qzeros must have i32/u32 dtype");
    check_float_dtype(input->dtype, "input");
    check_float_dtype(scales->dtype, "scales");
    check_float_dtype(output->dtype, "output");
    AWQ_ASSERT_EQ(input->elem_size, dtype_size(input->dtype), "input elem_size must match dtype");
    AWQ_ASSERT_EQ(scales->elem_size, dtype_size(scales->dtype), "scales elem_size must match dtype");
    AWQ_ASSERT_EQ(output->elem_size, dtype_size(output->dtype), "output elem_size must match dtype");

    GemmProblem p{};
    p.x = input->data;
    p.xt = input->dtype;
    p.qweight = static_cast<const uint32_t*>(qweight->data);
    p.qzeros = static_cast<const uint32_t*>(qzeros->data);
    p.scales = scales->data;
    p.st = scales->dtype;
    p.bias = nullptr;
    p.bt = AWQ_F32;
    p.y = const_cast<void*>(output->data);
    p.yt = output->dtype;
    p.rows = ls.m_valid;
    p.K = ls.k;
    p.N = ls.n;
    p.group = group_size;
    p.stream = static_cast<hipStream_t>(stream);
    run_gemm(p, ls.m);
  });
}

// dequantize_native, src/kernel/awq_kernel.rs:63-111.
int awq_dequantize_native(const awq_tensor_ref* q_weight, const awq_tensor_ref* q_zeros,
                          const awq_tensor_ref* q_scales, const awq_tensor_ref* output,
                          int64_t group_size, void* stream) {
  return guarded([&] {
    check_ref(q_weight, "q_weight");
    check_ref(q_zeros, "q_zeros");
    check_ref(q_scales, "q_scales");
    check_ref(output, "output");
    {
      std::ostringstream os;
      os << "AWQ packed q_weight must use 32-bit elements (i32/u32), got elem_size="
         << q_weight->elem_size << ".";
      AWQ_ASSERT_EQ(q_weight->elem_size, 4, os.str());
    }
    {
      std::ostringstream os;
      os << "AWQ packed q_zeros must use 32-bit elements (i32/u32), got elem_size="
         << q_zeros->elem_size << ".";
      AWQ_ASSERT_EQ(q_zeros->elem_size, 4, os.str());
    }
    AWQ_ASSERT(output->rank >= 1, "output must have at least one dimension");
    const int64_t out_width = output->shape[output->rank - 1];
    AWQ_ASSERT(out_width % 32 == 0, "assertion failed: out_width % 32 == 0");

    // The reference reads every tensor through a linear view (any rank) and
    // runs one unit per 4-word line of q_weight (numel / 4, rounded down):
    // line i covers output columns 32 (i % (N/32)) .. +31 of row i / (N/32),
    // whose group is row / group_size; nothing else about the shapes is
    // asserted. The same lines are computed here. What the reference leaves
    // unchecked and this library rejects: lines that would read or write past
    // the end of q_zeros, q_scales or output (out-of-bounds access there),
    // and group_size or out_width of 0 with work to do (a division by zero).
    const int64_t N = out_width;
    const int64_t lines = numel(*q_weight) / 4;
    if (lines > 0) {
      AWQ_ASSERT(N > 0, "dequantize: out_width must be > 0 when q_weight is not empty");
      AWQ_ASSERT(group_size > 0, "group_size must be > 0");
    }
    const int64_t lines_per_row = N / 32;
    const int64_t K = lines_per_row > 0 ? lines / lines_per_row : 0;        // complete rows
    const int64_t tail_cols = lines_per_row > 0 ? (lines % lines_per_row) * 32 : 0;  // last, partial row
    if (lines > 0) {
      // Highest zero word / scale / output element any line touches, + 1.
      int64_t need_z = 0, need_s = 0;
      if (K > 0) {
        const int64_t gl = (K - 1) / group_size;
        need_z = gl * (N / 8) + N / 8;
        need_s = gl * N + N;
      }
      if (tail_cols > 0) {
        const int64_t gt = K / group_size;
        need_z = std::max(need_z, gt * (N / 8) + tail_cols / 8);
        need_s = std::max(need_s, gt * N + tail_cols);
      }
      AWQ_ASSERT(numel(*q_zeros) >= need_z,
                 "dequantize: q_zeros is too small for q_weight, out_width and group_size");
      AWQ_ASSERT(numel(*q_scales) >= need_s,
                 "dequantize: q_scales is too small for q_weight, out_width and group_size");
      AWQ_ASSERT(numel(*output) >= K * N + tail_cols,
                 "dequantize: output is too small for q_weight");
    }
    check_float_dtype(q_scales->dtype, "scales");
    check_float_dtype(output->dtype, "output");

    DequantProblem p{};
    p.qweight = static_cast<const uint32_t*>(q_weight->data);
    p.qzeros = static_cast<const uint32_t*>(q_zeros->data);
    p.scales = q_scales->data;
    p.st = q_scales->dtype;
    p.out = const_cast<void*>(output->data);
    p.ot = output->dtype;
    p.K = K;
    p.N = N;
    p.group = group_size;
    p.tail_cols = tail_cols;
    p.order = AWQ_ORDER_SEQUENTIAL;
    p.stream = static_cast<hipStream_t>(stream);
    check_aligned(p.qweight, "qweight");
    check_aligned(p.qzeros, "qzeros");
    check_aligned(p.scales, "scales");
    check_aligned(p.out, "output");
    if (lines > 0) launch_dequant(p);
  });
}

// Module-level forward (AWQGEMMLinear::forward, src/modules/awq_gemm.rs:146-232)
// on plain pointers: tile choice by select_tile_m/n, INNER_K = 64.
static int gemm_entry(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
                      const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
                      int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size,
                      int32_t order, int32_t act, void* stream, bool noalloc = false) {
  return guarded([&] {
    AWQ_ASSERT(M >= 0 && K >= 0 && N >= 0, "shape sizes must be non-negative");
    awq_shape_config s = awq_shape_config_new(M, N, K, select_tile_m(M), select_tile_n(N), kInnerK);
    if (M <= kDecodeMThreshold) validate_decode(s, group_size);
    else validate_prefill(s, group_size);
    AWQ_ASSERT(order == AWQ_ORDER_AUTOAWQ || order == AWQ_ORDER_SEQUENTIAL,
               "order must be AWQ_ORDER_AUTOAWQ or AWQ_ORDER_SEQUENTIAL");
    check_float_dtype(x_t, "input");
    check_float_dtype(s_t, "scales");
    check_float_dtype(y_t, "output");
    if (bias) check_float_dtype(b_t, "bias");
    if (order == AWQ_ORDER_SEQUENTIAL)
      AWQ_ASSERT(s_t == x_t, "sequential-order GEMM needs scales in the input dtype");
    if (act) AWQ_ASSERT(N % 64 == 0, "gate/up GEMM: N (gate and up interleaved) must be a multiple of 64");
    GemmProblem p{};
    p.x = x;
    p.xt = x_t;
    p.qweight = qweight;
    p.qzeros = qzeros;
    p.scales = scales;
    p.st = s_t;
    p.bias = bias;
    p.bt = b_t;
    p.y = y;
    p.yt = y_t;
    p.rows = M;
    p.K = K;
    p.N = N;
    p.group = group_size;
    p.order = order;
    p.act = act;
    p.stream = static_cast<hipStream_t>(stream);
    if (noalloc && M > 0 && N > 0) p.scratch = scratch_on_device(p.stream);
    run_gemm(p, M);
  });
}

int awq_gemm(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
             const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
             int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size, void* stream) {
  return gemm_entry(x, x_t, qweight, qzeros, scales, s_t, bias, b_t, y, y_t, M, K, N, group_size,
                    AWQ_ORDER_AUTOAWQ, 0, stream);
}

int awq_gemm_noalloc(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
                     const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
                     int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size, void* stream) {
  return gemm_entry(x, x_t, qweight, qzeros, scales, s_t, bias, b_t, y, y_t, M, K, N, group_size,
                    AWQ_ORDER_AUTOAWQ, 0, stream, true);
}

int awq_gemm_silu_mul(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
                      const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
                      int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size,
                      void* stream) {
  return gemm_entry(x, x_t, qweight, qzeros, scales, s_t, bias, b_t, y, y_t, M, K, N, group_size,
                    AWQ_ORDER_AUTOAWQ, 1, stream);
}

int awq_gemm_ordered(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
                     const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
                     int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size,
                     int32_t order, void* stream) {
  return gemm_entry(x, x_t, qweight, qzeros, scales, s_t, bias, b_t, y, y_t, M, K, N, group_size,
                    order, 0, stream);
}

int awq_validate_gemm(int64_t M, int64_t K, int64_t N, int64_t group_size) {
  return guarded([&] {
    AWQ_ASSERT(M >= 0 && K >= 0 && N >= 0, "shape sizes must be non-negative");
    awq_shape_config s = awq_shape_config_new(M, N, K, select_tile_m(M), select_tile_n(N), kInnerK);
    if (M <= kDecodeMThreshold) validate_decode(s, group_size);
    else validate_prefill(s, group_size);
  });
}

int awq_dequantize(const uint32_t* qweight, const uint32_t* qzeros, const void* scales,
                   int32_t s_t, void* out, int32_t o_t, int64_t K, int64_t N,
                   int64_t group_size, int32_t order, void* stream) {
  return guarded([&] {
    AWQ_ASSERT(K >= 0 && N >= 0, "shape sizes must be non-negative");
    AWQ_ASSERT(N % 32 == 0, "assertion failed: out_width % 32 == 0");
    AWQ_ASSERT(group_size > 0, "group_size must be > 0");
    AWQ_ASSERT(K % group_size == 0, "k must be divisible by group_size");
    AWQ_ASSERT(order == AWQ_ORDER_AUTOAWQ || order == AWQ_ORDER_SEQUENTIAL,
               "order must be AWQ_ORDER_AUTOAWQ or AWQ_ORDER_SEQUENTIAL");
    check_float_dtype(s_t, "scales");
    check_float_dtype(o_t, "output");
    check_aligned(qweight, "qweight");
    check_aligned(qzeros, "qzeros");
    check_aligned(scales, "scales");
    check_aligned(out, "output");
    DequantProblem p{};
    p.qweight = qweight;
    p.qzeros = qzeros;
    p.scales = scales;
    p.st = s_t;
    p.out = out;
    p.ot = o_t;
    p.K = K;
    p.N = N;
    p.group = group_size;
    p.order = order;
    p.stream = static_cast<hipStream_t>(stream);
    if (K > 0 && N > 0) launch_dequant(p);
  });
}

int64_t awq_select_tile_m(int64_t m) { return select_tile_m(m); }
int64_t awq_select_tile_n(int64_t n) { return select_tile_n(n); }
int64_t awq_decode_m_threshold(void) { return kDecodeMThreshold; }

const char* awq_last_error(void) { return g_last_error.c_str(); }

void awq_tuning_reload(void) {
  std::call_once(g_tune_once, tuning_read);
  tuning_read();
}

int32_t awq_version(void) { return 100; /* 0.1.0 */ }

}  // extern "C"
