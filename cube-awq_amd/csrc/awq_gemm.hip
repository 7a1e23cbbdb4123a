// awq_gemm.hip -- prefill path (M > 8) of the fused AWQ dequant-GEMM for gfx950.
//
// Y[M, N] = X[M, K] . W[K, N], W[k, n] = (q - z) * s (AutoAWQ nibble order),
// the operation of the reference's gemm_awq (src/kernel/awq_kernel_gemm.rs:
// 181-439), which runs it as scalar vector-FMA in the activation type. Here it
// runs on CDNA4 matrix cores with fp32 accumulation:
//   f16  activations: v_mfma_f32_32x32x16_f16, W dequantised to f16
//   bf16 activations: v_mfma_f32_32x32x16_bf16, W dequantised to bf16
//   f32  activations: v_mfma_f32_32x32x2_f32, W dequantised in f32 exactly as
//                     the reference's F = f32 kernel does
//
// Tiling: a 256-thread workgroup (4 waves as 2 x 2) owns a 128 x 128 tile of Y
// and walks K in 64-row stages. Per stage it loads the X tile (row-major) and
// the packed 64 x 16-word W tile, dequantises W in registers and writes it to
// LDS transposed, n-major with k contiguous, so that both MFMA operands are
// single 16-byte LDS reads (lane l of a 32x32xK MFMA needs 8 consecutive k of
// one row of X and of one column of W). LDS is double buffered: global loads
// of stage s+1 are in flight while stage s feeds the matrix cores, one
// barrier per stage.
//
// f16 dequant (2.25 VALU ops per weight): for column c (packed lane L) and
// rows r, r+1, one v_perm_b32 gathers the byte holding lane L of both words
// into the two 16-bit halves, one v_and_or_b32 turns the nibbles into f16
// 1024+q (0x6400 | q), one v_pk_add_f16 subtracts 1024+z exactly and one
// v_pk_mul_f16 applies the scale: the result is the correctly rounded f16 of
// (q - z) * s, the value the reference computes with F = f16. Odd packed
// lanes (high nibble of the byte) take one extra shift.
#include <type_traits>

#include "awq_common.h"

namespace cube_awq {
namespace {

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kThreads = 256;

enum { MODE_F16 = 0, MODE_BF16 = 1, MODE_F32 = 2 };

template <int MODE> struct ModeT;
template <> struct ModeT<MODE_F16> {
  typedef f16_t T;
  static constexpr int kPad = 8;
};
template <> struct ModeT<MODE_BF16> {
  typedef bf16_t T;
  static constexpr int kPad = 8;
};
template <> struct ModeT<MODE_F32> {
  typedef float T;
  static constexpr int kPad = 4;
};

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef f16_t f16x8 __attribute__((ext_vector_type(8)));
typedef bf16_t bf16x8 __attribute__((ext_vector_type(8)));
typedef f16_t f16x2 __attribute__((ext_vector_type(2)));

struct GemmArgs {
  const void* x;
  const uint32_t* qweight;
  const uint32_t* qzeros;
  const void* scales;
  const void* bias;
  void* y;
  int32_t st, bt, yt;
  int32_t M, K, N, group;
  int32_t tiles_n;
};

template <int MODE>
struct Smem {
  typedef typename ModeT<MODE>::T T;
  static constexpr int kPitch = kBK + ModeT<MODE>::kPad;  // elements per LDS row
  T a[2][kBM][kPitch];  // X tile, row-major
  T b[2][kBN][kPitch];  // W tile, n-major (k contiguous)
};

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Two consecutive-k f16 weights (rows r, r+1) of the column held in packed
// lane L, as f16x2 bits: (q - z) * s correctly rounded.
template <int L>
__device__ __forceinline__ uint32_t deq_pair_f16(uint32_t w0, uint32_t w1, uint32_t zc, uint32_t sc) {
  constexpr uint32_t b = L / 2;
  constexpr uint32_t sel = b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
  uint32_t h = perm_b32(w1, w0, sel);  // byte b of w0 -> bits 0..7, of w1 -> bits 16..23
  if (L & 1) h >>= 4;
  const uint32_t v = (h & 0x000F000Fu) | 0x64006400u;  // f16 1024 + q per half
  f16x2 fv = __builtin_bit_cast(f16x2, v);
  f16x2 fz = __builtin_bit_cast(f16x2, zc);            // 1024 + z in both halves
  f16x2 fs = __builtin_bit_cast(f16x2, sc);            // s in both halves
  f16x2 r = (fv - fz) * fs;                            // exact subtract, one rounding
  return __builtin_bit_cast(uint32_t, r);
}

template <int MODE, int ST>
__global__ __launch_bounds__(kThreads, (MODE == MODE_F32) ? 1 : 2) void gemm_kernel(GemmArgs a) {
  typedef typename ModeT<MODE>::T T;
  using S = typename Elem<ST>::type;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Smem<MODE>& sm = *reinterpret_cast<Smem<MODE>*>(smem_raw);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave position in the 2 x 2 grid
  const int tile_m = blockIdx.x / a.tiles_n;
  const int tile_n = blockIdx.x - tile_m * a.tiles_n;
  const int m0 = tile_m * kBM, n0 = tile_n * kBN;
  const int np = a.N >> 3;
  const int stages = (a.K + kBK - 1) / kBK;

  // ---- per-thread load assignment -----------------------------------------
  // X tile: kBM rows x kBK elements; thread t covers row t/2, half (t%2).
  constexpr int kXElems = kBK / 2;                          // elements per thread
  constexpr int kXVec = 16 / (int)sizeof(T);                // elements per 16 B
  constexpr int kXLoads = kXElems / kXVec;                  // 16 B loads per thread
  using XIn = typename std::conditional<MODE == MODE_F32, float, T>::type;
  const int xr = tid >> 1;
  const int xk = (tid & 1) * kXElems;
  const bool x_row_ok = (m0 + xr) < a.M;
  const XIn* xsrc = static_cast<const XIn*>(a.x) + (int64_t)(x_row_ok ? m0 + xr : 0) * a.K + xk;

  // W tile: 16 packed words per row x 64 rows; thread t covers word t%16 of
  // rows 4*(t/16) .. +3.
  const int wp = tid & 15;
  const int wq = tid >> 4;
  const int pack = (n0 >> 3) + wp;
  const bool w_ok = pack < np;
  const uint32_t* wsrc = a.qweight + (w_ok ? pack : 0);

  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 xreg[kXLoads];
  uint32_t wreg[4];

  // 16-byte X loads need 16-byte aligned rows: K a multiple of the vector.
  const bool x_vec = (a.K % kXVec) == 0;

  auto load_stage = [&](int s) {
    const int k0 = s * kBK;
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
      const int k = k0 + xk + i * kXVec;
      if (x_row_ok && x_vec && k + kXVec <= a.K) {
        xreg[i] = *reinterpret_cast<const u32x4*>(xsrc + k0 + i * kXVec);
      } else if (x_row_ok && k < a.K) {
        // K is a multiple of 4 only: the last vector of a row may be partial.
        typedef XIn xv_t __attribute__((ext_vector_type(kXVec)));
        xv_t v;
#pragma unroll
        for (int e = 0; e < kXVec; ++e) v[e] = (k + e < a.K) ? xsrc[k0 + i * kXVec + e] : (XIn)0.0f;
        xreg[i] = __builtin_bit_cast(u32x4, v);
      } else {
        xreg[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = k0 + wq * 4 + r;
      wreg[r] = (w_ok && k < a.K) ? wsrc[(int64_t)k * np] : 0u;
    }
  };

  auto store_stage = [&](int s, int buf) {
    // X: straight copy into row-major LDS.
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      *reinterpret_cast<u32x4*>(&sm.a[buf][xr][xk + i * kXVec]) = xreg[i];
    // W: dequantise 4 rows x 8 columns, write k-contiguous per column.
    const int k0 = s * kBK + wq * 4;
    if (!w_ok || k0 >= a.K) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        T* dst = &sm.b[buf][wp * 8 + c][wq * 4];
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = (T)0.0f;
      }
      return;
    }
    const int grp = k0 / a.group;
    const uint32_t zw = a.qzeros[(int64_t)grp * np + pack];
    const S* srow = static_cast<const S*>(a.scales) + (int64_t)grp * a.N + (int64_t)pack * 8;
    if constexpr (MODE == MODE_F16) {
      uint32_t out[8][2];
#define AWQ_DEQ_COL(C)                                                                 \
  {                                                                                     \
    constexpr int L = awq_lane_of_col(C);                                               \
    const uint32_t z = (zw >> (4 * L)) & 0xFu;                                          \
    const f16_t zf = (f16_t)(1024.0f + (float)z);                                       \
    const f16_t sf = (f16_t)to_f32(srow[C]);                                            \
    const uint32_t zc = (uint32_t)__builtin_bit_cast(uint16_t, zf) * 0x10001u;          \
    const uint32_t scc = (uint32_t)__builtin_bit_cast(uint16_t, sf) * 0x10001u;         \
    out[C][0] = deq_pair_f16<L>(wreg[0], wreg[1], zc, scc);                             \
    out[C][1] = deq_pair_f16<L>(wreg[2], wreg[3], zc, scc);                             \
  }
      AWQ_DEQ_COL(0) AWQ_DEQ_COL(1) AWQ_DEQ_COL(2) AWQ_DEQ_COL(3)
      AWQ_DEQ_COL(4) AWQ_DEQ_COL(5) AWQ_DEQ_COL(6) AWQ_DEQ_COL(7)
#undef AWQ_DEQ_COL
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(&sm.b[buf][wp * 8 + c][wq * 4]) = u32x2{out[c][0], out[c][1]};
      }
    } else {
      // bf16 / f32: (float(q) - float(z)) * s in f32 (the reference's F = f32
      // arithmetic), then one rounding to T.
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int L = awq_lane_of_col(c);
        const int z = (int)((zw >> (4 * L)) & 0xFu);
        const float s = to_f32(srow[c]);
        T v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q = (int)((wreg[r] >> (4 * L)) & 0xFu);
          v[r] = from_f32<T>((float)(q - z) * s);
        }
        T* dst = &sm.b[buf][wp * 8 + c][wq * 4];
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = v[r];
      }
    }
  };

  // ---- accumulators: wave tile 64 x 64 = 2 x 2 blocks of 32 x 32 ------------
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int arow = wm * 64 + (lane & 31);  // + 32*i
  const int bcol = wn * 64 + (lane & 31);  // + 32*j
  const int kofs = (lane >> 5);            // which half of the MFMA k-slice

  auto compute_stage = [&](int buf) {
    if constexpr (MODE == MODE_F32) {
#pragma unroll 4
      for (int kk = 0; kk < kBK; kk += 2) {
        float av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) av[i] = sm.a[buf][arow + 32 * i][kk + kofs];
#pragma unroll
        for (int j = 0; j < 2; ++j) bv[j] = sm.b[buf][bcol + 32 * j][kk + kofs];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    } else {
      typedef typename std::conditional<MODE == MODE_F16, f16x8, bf16x8>::type V8;
#pragma unroll
      for (int kk = 0; kk < kBK; kk += 16) {
        V8 av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          av[i] = *reinterpret_cast<const V8*>(&sm.a[buf][arow + 32 * i][kk + kofs * 8]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          bv[j] = *reinterpret_cast<const V8*>(&sm.b[buf][bcol + 32 * j][kk + kofs * 8]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if constexpr (MODE == MODE_F16)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
            else
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
          }
      }
    }
  };

  // ---- main loop --------------------------------------------------------------
  load_stage(0);
  store_stage(0, 0);
  __syncthreads();
  for (int s = 0; s < stages; ++s) {
    const int buf = s & 1;
    const bool has_next = (s + 1) < stages;
    if (has_next) load_stage(s + 1);
    compute_stage(buf);
    if (has_next) store_stage(s + 1, buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: D layout of a 32x32 MFMA: lane l, register r ->
  //      row 8*(r/4) + 4*(l/32) + r%4, column l%32 ----------------------------
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + bcol + 32 * j;
    if (n >= a.N) continue;
    const float bias = a.bias ? load_f32_any(a.bias, n, a.bt) : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < a.M) store_f32_any(a.y, (int64_t)m * a.N + n, a.yt, acc[i][j][r] + bias);
      }
    }
  }
}

template <int MODE, int ST>
void launch_typed(const GemmProblem& p) {
  GemmArgs a{};
  a.x = p.x;
  a.qweight = p.qweight;
  a.qzeros = p.qzeros;
  a.scales = p.scales;
  a.bias = p.bias;
  a.y = p.y;
  a.st = p.st;
  a.bt = p.bt;
  a.yt = p.yt;
  a.M = (int32_t)p.rows;
  a.K = (int32_t)p.K;
  a.N = (int32_t)p.N;
  a.group = (int32_t)p.group;
  const int tiles_m = (int)((p.rows + kBM - 1) / kBM);
  const int tiles_n = (int)((p.N + kBN - 1) / kBN);
  a.tiles_n = tiles_n;
  const size_t smem = sizeof(Smem<MODE>);
  static bool attr_set = false;  // one-time opt-in above 64 KiB of LDS
  if (!attr_set) {
    check_hip(hipFuncSetAttribute((const void*)gemm_kernel<MODE, ST>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem),
              "hipFuncSetAttribute(gemm)");
    attr_set = true;
  }
  hipLaunchKernelGGL((gemm_kernel<MODE, ST>), dim3(tiles_m * tiles_n), dim3(kThreads), smem,
                     p.stream, a);
  check_hip(hipGetLastError(), "gemm kernel launch");
}

template <int MODE>
void launch_mode(const GemmProblem& p) {
  switch (p.st) {
    case AWQ_F32: launch_typed<MODE, AWQ_F32>(p); break;
    case AWQ_F16: launch_typed<MODE, AWQ_F16>(p); break;
    default: launch_typed<MODE, AWQ_BF16>(p); break;
  }
}

}  // namespace

void launch_gemm(const GemmProblem& p) {
  AWQ_ASSERT(p.rows < (1ll << 31) && p.K < (1ll << 31) && p.N < (1ll << 31) &&
                 p.rows * p.K < (1ll << 40) && p.K * (p.N / 8) < (1ll << 31),
             "prefill GEMM: tensor too large");
  const int64_t tiles = ((p.rows + kBM - 1) / kBM) * ((p.N + kBN - 1) / kBN);
  AWQ_ASSERT(tiles < (1ll << 31), "prefill GEMM: too many tiles");
  switch (p.xt) {
    case AWQ_F16: launch_mode<MODE_F16>(p); break;
    case AWQ_BF16: launch_mode<MODE_BF16>(p); break;
    default: launch_mode<MODE_F32>(p); break;
  }
}

}  // namespace cube_awq
