// awq_common.h -- shared host/device definitions of the gfx950 AWQ library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/awq.h"

namespace cube_awq {

// ---------------------------------------------------------------------------
// Host-side error plumbing. A failed assertion throws Panic carrying the exact
// text the reference panics with; the C ABI turns it into AWQ_ERR_INVALID and
// awq_last_error().
// ---------------------------------------------------------------------------
struct Panic {
  std::string msg;
};
struct HipFailure {
  std::string msg;
};

[[noreturn]] void panic(const std::string& msg);
void check_hip(hipError_t e, const char* what);

// Rust `assert!(cond, "msg")` -> panics with "msg".
#define AWQ_ASSERT(cond, msg)                  \
  do {                                         \
    if (!(cond)) ::cube_awq::panic((msg));     \
  } while (0)

// Rust `assert_eq!(a, b, "msg")` -> "assertion `left == right` failed: msg\n  left: a\n right: b".
std::string assert_eq_text(const std::string& msg, long long left, long long right);
#define AWQ_ASSERT_EQ(a, b, msg)                                                         \
  do {                                                                                  \
    long long _l = (long long)(a), _r = (long long)(b);                                 \
    if (_l != _r) ::cube_awq::panic(::cube_awq::assert_eq_text((msg), _l, _r));         \
  } while (0)

constexpr int dtype_size_ct(int32_t t) {
  switch (t) {
    case AWQ_F32: return 4;
    case AWQ_F16: return 2;
    case AWQ_BF16: return 2;
    case AWQ_U32: return 4;
    case AWQ_I32: return 4;
    case AWQ_I16: return 2;
    case AWQ_I64: return 8;
    default: return 0;
  }
}
inline int dtype_size(int32_t t) { return dtype_size_ct(t); }
inline bool is_float_dtype(int32_t t) { return t == AWQ_F32 || t == AWQ_F16 || t == AWQ_BF16; }

// ---------------------------------------------------------------------------
// Device element helpers.
// ---------------------------------------------------------------------------
typedef _Float16 f16_t;
typedef __bf16 bf16_t;

template <int T> struct Elem;
template <> struct Elem<AWQ_F32> { typedef float type; };
template <> struct Elem<AWQ_F16> { typedef f16_t type; };
template <> struct Elem<AWQ_BF16> { typedef bf16_t type; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16_t v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
  // bf16 -> f32 is exact: the bf16 bits are the high half of the f32.
  return __builtin_bit_cast(float, ((uint32_t)__builtin_bit_cast(uint16_t, v)) << 16);
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float v) {
  return (f16_t)v;  // v_cvt_f16_f32, round to nearest even
}
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
  return (bf16_t)v;  // v_cvt_pk_bf16_f32 on gfx950, round to nearest even
}

// Runtime-typed scalar load/store for data touched outside the hot loops.
__device__ __forceinline__ float load_f32_any(const void* p, int64_t i, int32_t t) {
  if (t == AWQ_F32) return ((const float*)p)[i];
  if (t == AWQ_F16) return to_f32(((const f16_t*)p)[i]);
  return to_f32(((const bf16_t*)p)[i]);
}
__device__ __forceinline__ void store_f32_any(void* p, int64_t i, int32_t t, float v) {
  if (t == AWQ_F32) ((float*)p)[i] = v;
  else if (t == AWQ_F16) ((f16_t*)p)[i] = from_f32<f16_t>(v);
  else ((bf16_t*)p)[i] = from_f32<bf16_t>(v);
}

// Fused gate/up epilogue: the weights interleave the two projections by
// column (column 2j = gate j, column 2j + 1 = up j); output j is SiLU(gate j)
// * up j, SiLU(g) = g / (1 + e^-g), in a [rows, N/2] output.
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.f + __expf(-g)) * u; }

// Final store of output (m, n) of a width-N GEMM: v itself, or with the
// activation (act != 0) SiLU(v) * partner from the lane of the even column
// of a pair, to (m, n / 2); the odd column's lane stores nothing.
__device__ __forceinline__ void store_out(void* y, int32_t yt, int32_t act, int64_t m, int64_t n,
                                          int64_t N, float v, float partner) {
  if (!act) store_f32_any(y, m * N + n, yt, v);
  else if ((n & 1) == 0) store_f32_any(y, m * (N >> 1) + (n >> 1), yt, silu_mul(v, partner));
}

// The activation outputs of 4 consecutive GEMM columns n .. n + 3 (n % 4 ==
// 0: gate/up pairs (n, n + 1) and (n + 2, n + 3)), two consecutive outputs
// of row m, written as one 8-byte (f32) or 4-byte (f16, bf16) store.
__device__ __forceinline__ void store_act_quad(void* y, int32_t yt, int64_t m, int64_t n, int64_t N, float g0,
                                               float u0, float g1, float u1) {
  const int64_t i = m * (N >> 1) + (n >> 1);
  const float o0 = silu_mul(g0, u0), o1 = silu_mul(g1, u1);
  if (yt == AWQ_F32) {
    typedef float f2_t __attribute__((ext_vector_type(2)));
    *reinterpret_cast<f2_t*>(static_cast<float*>(y) + i) = f2_t{o0, o1};
  } else if (yt == AWQ_F16) {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    *reinterpret_cast<h2_t*>(static_cast<f16_t*>(y) + i) = h2_t{(_Float16)o0, (_Float16)o1};
  } else {
    store_f32_any(y, i, yt, o0);
    store_f32_any(y, i + 1, yt, o1);
  }
}

// Packed lane L of two words as f16x2 magic numbers: the byte holding lane L
// of w0 and of w1 goes to the two halves (v_perm_b32), then one v_bitop3
// keeps the nibble and ORs in the exponent: low nibble (even L) -> 0x6400 | q
// = 1024 + q, high nibble (odd L) -> 0x5400 | q << 4 = 64 + q (mantissa unit
// 1/16 at exponent 6). L must be a compile-time constant after inlining.
__device__ __forceinline__ uint32_t nib_f16x2(uint32_t w0, uint32_t w1, int L) {
  const uint32_t b = (uint32_t)L >> 1;
  const uint32_t h = __builtin_amdgcn_perm(w1, w0, b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24));
  return (L & 1) ? __builtin_amdgcn_bitop3_b32(h, 0x00F000F0u, 0x54005400u, 0xEA)
                 : __builtin_amdgcn_bitop3_b32(h, 0x000F000Fu, 0x64006400u, 0xEA);
}

// Raw buffer access: a 128-bit resource (base, byte size) in SGPRs plus a
// per-lane byte offset (VGPR) and a wave-uniform byte offset (SGPR), so a
// strided walk over rows costs no per-load VALU address arithmetic.
// 0x00020000 is the gfx9-family dword3 (32-bit raw data format).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint32_t buf_load_u32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
// Same with the nontemporal (nt) cache policy: for data read exactly once
// (the weight stream), so it does not displace reused lines in L2.
constexpr int kCachePolicyNT = 2;
// Device-coherent (agent scope) access: sc1, as agent-scope atomic loads and
// stores use, so data written by other workgroups' sc1 stores is seen.
constexpr int kCachePolicySC1 = 16;

// Split-K handshake (decode, skinny and large-tile kernels). Each workgroup
// of a K split writes its fp32 partials, then counts its arrival on a
// per-chunk counter; the workgroup that arrives last sums every split's
// partials and re-arms the counter. Why relaxed agent-scope atomics and a
// vmcnt wait are enough, without the L2 writeback / invalidate that a
// release / acquire pair would add on gfx950 (one L2 per XCD):
//  * Writer. Every partial is stored with an agent-scope atomic store or a
//    buffer store with the same sc1 policy (kCachePolicySC1; 16-byte pieces
//    in the skinny and 2..16-row decode kernels), which is written through
//    its XCD's L2 to the device's point of
//    coherence instead of staying dirty there; that writeback is what an
//    agent-scope release adds, for plain stores only. Each wave then waits
//    for its stores to complete (s_waitcnt vmcnt(0): a store's count drops
//    once the write is acknowledged at its scope), and a workgroup barrier
//    follows, so every partial of the workgroup is visible device-wide
//    before thread 0 issues the counter's fetch_add. The asm statement's
//    "memory" clobber and the barrier also keep the compiler from moving
//    the stores past the fetch_add.
//  * Reader. Only the workgroup whose fetch_add returned splits - 1 reads
//    the partials, and its loads are issued after that value has returned
//    (a barrier and a branch on it). They are agent-scope atomic loads, or
//    buffer loads with the same sc1 policy (kCachePolicySC1), which do not
//    return a stale line of this XCD's L2; the invalidate an agent-scope
//    acquire adds is for plain loads only. The reader never reads partials
//    it did not wait for, since every writer's fetch_add follows its
//    stores.
//  * Re-arm. The last workgroup stores 0 to the counter; the next call on
//    the stream starts after this kernel ends (stream order), so no
//    arrival of the next call races with the reset.
// The counters are zeroed once when their buffer is allocated and are back
// at zero after every complete launch.
__device__ __forceinline__ uint32_t buf_load_u32_nt(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kCachePolicyNT);
}

// AutoAWQ interleave: logical column c of a pack sits in packed lane
// kAwqLaneOfCol[c]; packed lane p holds column kAwqColOfLane[p].
// (Same table as the reference, src/kernel/awq_kernel_gemm.rs:7-30.)
__host__ __device__ constexpr int awq_lane_of_col(int c) {
  return (c == 0) ? 0 : (c == 1) ? 4 : (c == 2) ? 1 : (c == 3) ? 5
       : (c == 4) ? 2 : (c == 5) ? 6 : (c == 6) ? 3 : 7;
}
__host__ __device__ constexpr int awq_col_of_lane(int p) {
  return (p == 0) ? 0 : (p == 1) ? 2 : (p == 2) ? 4 : (p == 3) ? 6
       : (p == 4) ? 1 : (p == 5) ? 3 : (p == 6) ? 5 : 7;
}

// ---------------------------------------------------------------------------
// Launch descriptors shared by the API layer and the kernels.
// ---------------------------------------------------------------------------
struct GemmProblem {
  const void* x;
  int32_t xt;
  const uint32_t* qweight;
  const uint32_t* qzeros;
  const void* scales;
  int32_t st;
  const void* bias;  // nullable, [N]
  int32_t bt;
  void* y;
  int32_t yt;
  int64_t rows;  // rows to compute and write (m_valid)
  int64_t K, N, group;
  int32_t order;  // AWQ_ORDER_AUTOAWQ (awq_gemm) or AWQ_ORDER_SEQUENTIAL (AWQLinear's weights)
  int32_t act;    // 1: gate/up interleaved by column, y [rows, N/2] = SiLU(gate) * up
  hipStream_t stream;
  void* scratch;  // static split-K scratch (awq_gemm_noalloc), or null: library workspace
  const float* xrowfac;  // fp32 activations split into f16 hi + lo: row factors (else null)
};

struct DequantProblem {
  const uint32_t* qweight;
  const uint32_t* qzeros;
  const void* scales;
  int32_t st;
  void* out;
  int32_t ot;
  int64_t K, N, group;  // K complete rows of N columns
  int64_t tail_cols;    // then this many columns (a multiple of 32) of row K
  int32_t order;
  hipStream_t stream;
};

// Kernel launchers (defined in the .hip translation units).
void launch_dequant(const DequantProblem& p);
void launch_gemv(const GemmProblem& p);   // rows <= 8, and 9..16 when small_m_mfma_ok
void launch_gemm(const GemmProblem& p);   // rows > 8
// 9..16 rows run on the matrix-core decode kernel (16-row tile) when its
// constraints hold (group % 32, K % 32); AWQ_SMALLM_MFMA=0 turns it off.
bool small_m_mfma_ok(const GemmProblem& p, int64_t launch_m);
// 9..128 rows of f16/bf16 activations (wide outputs, or narrower ones up
// to 64..128 rows): the skinny kernel (awq_skinny.hip); AWQ_SKINNY=0/1
// forces the choice.
bool skinny_ok(const GemmProblem& p);
void launch_skinny(const GemmProblem& p);

// Compute units of the current device (queried once per device).
int64_t device_cus();

// Tuning overrides (AWQ_* environment variables that force a route or a
// launch configuration). They are read from the environment once per process
// (and again by awq_tuning_reload()), never on the launch path.
enum TuneKey {
  kTuneGemmTile,      // AWQ_GEMM_TILE
  kTuneGemmSplits,    // AWQ_GEMM_SPLITS
  kTuneGemmGroupM,    // AWQ_GEMM_GROUP_M
  kTuneF32Slices,     // AWQ_F32_SLICES
  kTuneGemvWaves,     // AWQ_GEMV_WAVES
  kTuneGemvRpw,       // AWQ_GEMV_RPW
  kTuneMfmaWaves,     // AWQ_MFMA_WAVES
  kTuneMfmaRpw,       // AWQ_MFMA_RPW
  kTuneM4Waves,       // AWQ_M4_WAVES
  kTuneM4Rpw,         // AWQ_M4_RPW
  kTuneDecodeMfma,    // AWQ_DECODE_MFMA
  kTuneDecodeM4,      // AWQ_DECODE_M4
  kTuneSmallMMfma,    // AWQ_SMALLM_MFMA
  kTuneSkinny,        // AWQ_SKINNY
  kTuneSkinnySplits,  // AWQ_SKINNY_SPLITS
  kTuneSkinnyCols,    // AWQ_SKINNY_COLS
  kTuneDecodeTree,    // AWQ_DECODE_TREE
  kTuneSkinnyTree,    // AWQ_SKINNY_TREE
  kTuneCount
};
// The override's value (atoi of the variable), or dflt when it is unset.
int tuning(TuneKey key, int dflt);

// Opt a kernel in to `bytes` of dynamic LDS on the current device (once per
// device and kernel; thread-safe).
void ensure_dyn_smem(const void* kernel, int bytes, const char* what);

// Split-K workspace of a launch: kWsCounters (arrival counters, zero between
// calls: every kernel that takes one re-arms it) and kWsPartials (fp32
// partial sums, contents undefined between calls). workspace_get returns a
// per-(device, stream, slot) library buffer of at least `bytes`; a buffer is
// never freed once handed out (a graph captured on the stream may still
// hold it), so growth allocates a new one and retires the old one for the
// life of the process. Growth is refused during stream capture.
// kWsXSplit holds fp32 activations split into f16 hi and lo rows and their
// row factors (M K 4 + M 4 bytes), written by a prepass of the same call.
enum { kWsCounters = 0, kWsPartials = 1, kWsXSplit = 2 };
void* workspace_get(hipStream_t stream, size_t bytes, int slot);
// The split-K buffer of one launch of problem p: a region of p.scratch when
// it is set (awq_gemm_noalloc; sizes past the region are an error, nothing is
// allocated), else workspace_get on p.stream.
void* ws_get(const GemmProblem& p, size_t bytes, int slot);

}  // namespace cube_awq
