// awq_gemm.hip -- prefill path (M > 8) of the fused AWQ dequant-GEMM for gfx950.
//
// Y[M, N] = X[M, K] . W[K, N], W[k, n] = (q - z) * s, the operation of the
// reference's gemm_awq (src/kernel/awq_kernel_gemm.rs:181-439), which runs it
// as scalar vector-FMA in the activation type. Here it runs on CDNA4 matrix
// cores with fp32 accumulation. Nibbles are read in AutoAWQ order, or in
// sequential order (SEQ, the layout AWQLinear's weights use): the order only
// changes which packed lane a column is taken from.
//
// gemm_big_kernel (f16/bf16 activations, K % 64 == 0, group = 64 * 2^j):
//  * A workgroup of WGM x WGN waves owns a BM x BN tile of Y (256x224,
//    256x256, 128x256, 128x128, ...; v_mfma_f32_32x32x16 or, for 256x224,
//    v_mfma_f32_16x16x32 blocks) and walks its K range in 64-row stages.
//  * X goes global -> LDS directly (buffer_load_dwordx4 ... lds, no VGPR
//    staging), two stages ahead in three LDS buffers when they fit. Each LDS
//    row is 128 bytes of eight 16-byte granules at slot g ^ swz<MS>(row),
//    which keeps both the MFMA operand reads and the dequantised-W writes
//    free of bank conflicts without padding.
//  * Packed W, zeros and scales of stage s+2 are loaded into registers while
//    W of stage s+1 is dequantised between the MFMAs of stage s (scheduling
//    groups interleave a few VALU ops after each MFMA) and written to LDS
//    n-major with k contiguous. One s_barrier per stage; waits are explicit
//    vmcnt/lgkmcnt counts, so loads of later stages stay in flight.
//  * 256x224 runs ping-pong (PP) by default: the two halves of the waves
//    (one half of the rows each) run one phase apart, one half multiplying
//    while the other reads its operands from LDS, issues the next loads and
//    dequantises; two barriers per stage. Each accumulator's MFMAs keep the
//    single-phase order, so both schedules give the same bits.
//  * f16 dequant: one v_perm_b32 gathers the byte holding the column's lane
//    from two rows, one v_bitop3_b32 forms f16 1024 + q (low nibble) or
//    64 + q (high nibble), then an exact v_pk_add_f16 of the zero and one
//    v_pk_mul_f16 of the scale: the correctly rounded f16 of (q - z) * s,
//    the reference's F = f16 value. bf16: (q - z) * s exact in f32, rounded
//    once to bf16.
//  * Tiles are rastered in groups of a few row tiles and remapped so each
//    XCD runs a contiguous block of them, sharing X and W in its L2.
//  * Problems with fewer tiles than CUs split K across workgroups; partials
//    are summed in split order by the last workgroup to arrive on its tile.
//    (9..128 rows of f16/bf16 take the skinny kernel where it is faster,
//    awq_skinny.hip.)
// gemm_kernel (generic, 128x128, padded LDS, VGPR-staged loads) takes fp32
// activations (v_mfma_f32_32x32x2_f32, W dequantised in f32 exactly as the
// reference's F = f32 kernel) and every shape the large-tile kernel does not.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "awq_common.h"

namespace cube_awq {
namespace {

constexpr int kBK = 64;

// MODE_F32S: fp32 activations on the f16 matrix cores. A prepass
// (x_split_kernel) writes each row of x, scaled by the power of two 2^e that
// puts its largest |x| in [2^14, 2^15), as f16 hi + lo (hi = f16(x 2^e),
// lo = f16(x 2^e - hi)) and the row factor 2^-e. The large-tile kernel
// multiplies both halves with the exact f16 integers q - z (no rounding of
// the weight at all), sums each quantisation group in fp32, applies the
// group's scale s to that sum in fp32, and the row factor at the end: fp32
// accuracy at about half the f16 rate.
enum { MODE_F16 = 0, MODE_BF16 = 1, MODE_F32 = 2, MODE_F32S = 3 };

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
template <> struct ModeT<MODE_F32S> {
  typedef f16_t T;
};

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef f16_t f16x8 __attribute__((ext_vector_type(8)));
typedef bf16_t bf16x8 __attribute__((ext_vector_type(8)));
typedef f16_t f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct GemmArgs {
  const void* x;
  const uint32_t* qweight;
  const uint32_t* qzeros;
  const void* scales;
  const void* bias;
  void* y;
  int32_t st, bt, yt;
  int32_t M, K, N, group;
  int32_t tiles_m, tiles_n;
  int32_t swizzled_tiles;  // leading tiles covered by the XCD mapping (multiple of 8)
  int32_t group_m;         // row tiles per raster group (large-tile kernel)
  int32_t grp_shift;       // large-tile kernel: group = 64 << grp_shift
  // Large-tile kernel split-K (grid.y = splits): workgroup y covers stages
  // [y * stages_per_split, ...); partials [splits][M][N] and one arrival
  // counter per tile (kTileCtrStride apart, zero between calls).
  int32_t splits, stages_per_split;
  float* partial;
  uint32_t* counters;
  // MODE_F32S: x is the prepass output, hi [M][K] f16 then lo [M][K] f16
  // (lo_off = M K 2 bytes after hi), and rowfac [M] the row factors 2^-e.
  const float* rowfac;
  uint32_t lo_off;
};

constexpr int kTileCtrStride = 64;  // u32 words between per-tile counters (256 B)

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

// Packed lane holding column c of a pack: AutoAWQ interleave, or lane c in
// sequential order (the order AWQLinear's weights use).
template <bool SEQ>
__host__ __device__ constexpr int lane_of_col(int c) { return SEQ ? c : awq_lane_of_col(c); }

template <int MODE, int BM, int BN, int WGM, int WGN>
struct Tile {
  typedef typename ModeT<MODE>::T T;
  static constexpr int kThreads = 64 * WGM * WGN;
  static constexpr int kPitch = kBK + ModeT<MODE>::kPad;  // elements per LDS row
  static constexpr int kWTM = BM / WGM, kWTN = BN / WGN;  // wave tile
  static constexpr int kI = kWTM / 32, kJ = kWTN / 32;    // 32 x 32 blocks per wave
  static constexpr int kXVec = 16 / (int)sizeof(T);       // elements per 16-byte load
  static constexpr int kXChunksPerRow = kBK / kXVec;
  static constexpr int kXLoads = BM * kXChunksPerRow / kThreads;
  static constexpr size_t kSmem = (size_t)2 * (BM + BN) * kPitch * sizeof(T);
  static_assert(kThreads == 2 * BN, "W tile mapping: each thread dequantises 4 rows x 8 columns");
  static_assert(kWTM % 32 == 0 && kWTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert((BM * kXChunksPerRow) % kThreads == 0, "X tile must split evenly");
};

// Hint for the register allocator: the 256x256 tile runs one workgroup per CU.
constexpr int min_blocks(int tile_elems) { return tile_elems >= 256 * 256 ? 1 : 2; }

// ACT: the gate/up SiLU epilogue (store_out). A template parameter, not a
// kernel argument: as a runtime flag its epilogue code changed the register
// allocation of the main loop and cost 2.5-6 % on every prefill GEMM.
template <int MODE, int ST, int BM, int BN, int WGM, int WGN, bool SEQ, bool ACT>
__global__ __launch_bounds__(64 * WGM * WGN, min_blocks(BM * BN)) void gemm_kernel(GemmArgs a) {
  using C = Tile<MODE, BM, BN, WGM, WGN>;
  typedef typename C::T T;
  using S = typename Elem<ST>::type;
  constexpr int P = C::kPitch;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* sa = reinterpret_cast<T*>(smem_raw);                 // [2][BM][P]
  T* sb = sa + 2 * BM * P;                                // [2][BN][P]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  // Tile index: consecutive workgroups are dispatched to different XCDs, so
  // remap them to give each XCD a contiguous run of tiles (tile_m fastest:
  // the run shares a few columns of W and so hits that XCD's L2).
  int t = blockIdx.x;
  if (t < a.swizzled_tiles) {
    const int per_xcd = a.swizzled_tiles >> 3;
    t = (t & 7) * per_xcd + (t >> 3);
  }
  const int tile_m = t % a.tiles_m;
  const int tile_n = t / a.tiles_m;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int np = a.N >> 3;
  const int stages = (a.K + kBK - 1) / kBK;

  // ---- X tile loads: 16-byte chunks, chunk c = tid + i*T: row c/8, k 8*(c%8)
  using XIn = typename std::conditional<MODE == MODE_F32, float, T>::type;
  constexpr int XV = C::kXVec;
  const XIn* xsrc[C::kXLoads];
  int xrow[C::kXLoads], xk[C::kXLoads];
  bool xrow_ok[C::kXLoads];
#pragma unroll
  for (int i = 0; i < C::kXLoads; ++i) {
    const int c = tid + i * C::kThreads;
    xrow[i] = c / C::kXChunksPerRow;
    xk[i] = (c % C::kXChunksPerRow) * XV;
    xrow_ok[i] = (m0 + xrow[i]) < a.M;
    xsrc[i] = static_cast<const XIn*>(a.x) + (int64_t)(xrow_ok[i] ? m0 + xrow[i] : 0) * a.K + xk[i];
  }
  // 16-byte X loads need 16-byte aligned rows: K a multiple of the vector.
  const bool x_vec = (a.K % XV) == 0;

  // ---- W tile: thread covers packed word wp of rows 4*wq .. 4*wq+3
  const int wp = tid % (BN / 8);
  const int wq = tid / (BN / 8);
  const int pack = (n0 >> 3) + wp;
  const bool w_ok = pack < np;
  const uint32_t* wsrc = a.qweight + (w_ok ? pack : 0);

  u32x4 xreg[C::kXLoads];
  uint32_t wreg[4];

  auto load_stage = [&](int s) {
    const int k0 = s * kBK;
#pragma unroll
    for (int i = 0; i < C::kXLoads; ++i) {
      const int k = k0 + xk[i];
      if (xrow_ok[i] && x_vec && k + XV <= a.K) {
        xreg[i] = *reinterpret_cast<const u32x4*>(xsrc[i] + k0);
      } else if (xrow_ok[i] && k < a.K) {
        // K is a multiple of 4 only: the last vector of a row may be partial.
        typedef XIn xv_t __attribute__((ext_vector_type(XV)));
        xv_t v;
#pragma unroll
        for (int e = 0; e < XV; ++e) v[e] = (k + e < a.K) ? xsrc[i][k0 + e] : (XIn)0.0f;
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
    for (int i = 0; i < C::kXLoads; ++i)
      *reinterpret_cast<u32x4*>(&sa[(buf * BM + xrow[i]) * P + xk[i]]) = xreg[i];
    // W: dequantise 4 rows x 8 columns, write k-contiguous per column.
    T* bdst = &sb[(buf * BN + wp * 8) * P + wq * 4];
    const int k0 = s * kBK + wq * 4;
    if (!w_ok || k0 >= a.K) {
#pragma unroll
      for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) bdst[c * P + r] = (T)0.0f;
      return;
    }
    const int grp = k0 / a.group;
    const uint32_t zw = a.qzeros[(int64_t)grp * np + pack];
    const S* srow = static_cast<const S*>(a.scales) + (int64_t)grp * a.N + (int64_t)pack * 8;
    if constexpr (MODE == MODE_F16) {
      uint32_t out[8][2];
#define AWQ_DEQ_COL(CC)                                                                \
  {                                                                                     \
    constexpr int L = lane_of_col<SEQ>(CC);                                             \
    const uint32_t z = (zw >> (4 * L)) & 0xFu;                                          \
    const f16_t zf = (f16_t)(1024.0f + (float)z);                                       \
    const f16_t sf = (f16_t)to_f32(srow[CC]);                                           \
    const uint32_t zc = (uint32_t)__builtin_bit_cast(uint16_t, zf) * 0x10001u;          \
    const uint32_t scc = (uint32_t)__builtin_bit_cast(uint16_t, sf) * 0x10001u;         \
    out[CC][0] = deq_pair_f16<L>(wreg[0], wreg[1], zc, scc);                            \
    out[CC][1] = deq_pair_f16<L>(wreg[2], wreg[3], zc, scc);                            \
  }
      AWQ_DEQ_COL(0) AWQ_DEQ_COL(1) AWQ_DEQ_COL(2) AWQ_DEQ_COL(3)
      AWQ_DEQ_COL(4) AWQ_DEQ_COL(5) AWQ_DEQ_COL(6) AWQ_DEQ_COL(7)
#undef AWQ_DEQ_COL
#pragma unroll
      for (int c = 0; c < 8; ++c)
        *reinterpret_cast<u32x2*>(&bdst[c * P]) = u32x2{out[c][0], out[c][1]};
    } else {
      // bf16 / f32: (float(q) - float(z)) * s in f32 (the reference's F = f32
      // arithmetic), then one rounding to T.
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int L = lane_of_col<SEQ>(c);
        const int z = (int)((zw >> (4 * L)) & 0xFu);
        const float sv = to_f32(srow[c]);
        T v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q = (int)((wreg[r] >> (4 * L)) & 0xFu);
          v[r] = from_f32<T>((float)(q - z) * sv);
        }
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<u32x2*>(&bdst[c * P]) =
              u32x2{(uint32_t)__builtin_bit_cast(uint16_t, v[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, v[1]) << 16),
                    (uint32_t)__builtin_bit_cast(uint16_t, v[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, v[3]) << 16)};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) bdst[c * P + r] = v[r];
        }
      }
    }
  };

  // ---- accumulators: kI x kJ blocks of 32 x 32 per wave ------------------------
  f32x16 acc[C::kI][C::kJ];
#pragma unroll
  for (int i = 0; i < C::kI; ++i)
#pragma unroll
    for (int j = 0; j < C::kJ; ++j) acc[i][j] = f32x16{};

  const int arow = wm * C::kWTM + (lane & 31);  // + 32*i
  const int bcol = wn * C::kWTN + (lane & 31);  // + 32*j
  const int kofs = (lane >> 5);                  // which half of the MFMA k-slice

  auto compute_stage = [&](int buf) {
    const T* A = sa + buf * BM * P;
    const T* B = sb + buf * BN * P;
    if constexpr (MODE == MODE_F32) {
#pragma unroll 4
      for (int kk = 0; kk < kBK; kk += 2) {
        float av[C::kI], bv[C::kJ];
#pragma unroll
        for (int i = 0; i < C::kI; ++i) av[i] = A[(arow + 32 * i) * P + kk + kofs];
#pragma unroll
        for (int j = 0; j < C::kJ; ++j) bv[j] = B[(bcol + 32 * j) * P + kk + kofs];
#pragma unroll
        for (int i = 0; i < C::kI; ++i)
#pragma unroll
          for (int j = 0; j < C::kJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    } else {
      typedef typename std::conditional<MODE == MODE_F16, f16x8, bf16x8>::type V8;
#pragma unroll
      for (int kk = 0; kk < kBK; kk += 16) {
        V8 av[C::kI], bv[C::kJ];
#pragma unroll
        for (int i = 0; i < C::kI; ++i)
          av[i] = *reinterpret_cast<const V8*>(&A[(arow + 32 * i) * P + kk + kofs * 8]);
#pragma unroll
        for (int j = 0; j < C::kJ; ++j)
          bv[j] = *reinterpret_cast<const V8*>(&B[(bcol + 32 * j) * P + kk + kofs * 8]);
#pragma unroll
        for (int i = 0; i < C::kI; ++i)
#pragma unroll
          for (int j = 0; j < C::kJ; ++j) {
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
  // Column lane % 32: a gate/up pair is this lane and its xor-1 neighbour
  // (N is even, so both are in range or neither).
#pragma unroll
  for (int j = 0; j < C::kJ; ++j) {
    const int n = n0 + bcol + 32 * j;
    if (n >= a.N) continue;
    const float bias = a.bias ? load_f32_any(a.bias, n, a.bt) : 0.f;
#pragma unroll
    for (int i = 0; i < C::kI; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * C::kWTM + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const float v = acc[i][j][r] + bias;
        const float pv = ACT ? __shfl_xor(v, 1, 64) : 0.f;
        if (m < a.M) store_out(a.y, a.yt, ACT, m, n, a.N, v, pv);
      }
    }
  }
}

// ===========================================================================
// Large-tile f16/bf16 kernel: one workgroup per CU, 128 KB of LDS.
//
// Requirements (checked by the launcher): K % 64 == 0, group = 64 * 2^j, X
// and W small enough for 32-bit buffer offsets. Each wave owns a (BM/WGM) x
// (BN/WGN) block of Y in 32 x 32 MFMA tiles.
//
// LDS rows are 128 bytes (64 k of one row of X or one column of W) made of
// eight 16-byte granules; granule g of row r is stored in slot g ^ swz<MS>(r).
// The swizzle makes the MFMA operand reads and the dequantised-W writes (rows
// 8 apart, one granule) bank-conflict free without padding.
//
// Software pipeline per 64-row stage s (buffers s & 1):
//   issue LDS-direct X loads for s+1 and packed W / zeros / scales for s+2,
//   per 16-k slice: MFMAs of stage s, then dequantise two columns of W(s+1)
//   (loaded a stage ago) into the other buffer; one barrier.
// ===========================================================================
// s_waitcnt immediate (gfx9 encoding): vmcnt in bits 3:0 and 15:14, expcnt
// 6:4 (left at its maximum), lgkmcnt 11:8.
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | ((lgkm & 0xF) << 8);
}
// Two swizzles, chosen by the MFMA shape; each measured free of bank
// conflicts (SQ_LDS_BANK_CONFLICT, gfx950) for its operand reads and for the
// dequantised-W writes: 32x32x16 reads (32 rows x 2 granules per instruction)
// with (r ^ (r >> 3)) & 7, 16x16x32 reads (16 rows x 4 granules) with
// ((r >> 1) ^ (r >> 4)) & 7 -- the first costs 4 conflict cycles per
// 16x16x32 operand read.
template <int MS> __device__ __forceinline__ int swz(int row) {
  if constexpr (MS == 16) return ((row >> 1) ^ (row >> 4)) & 7;
  else return (row ^ (row >> 3)) & 7;
}
// Both are w_slot_base(wp) ^ w_slot_flip(c) on W column 8 wp + c (c < 8).
template <int MS> __device__ __forceinline__ int w_slot_base(int wp) {
  if constexpr (MS == 16) return ((wp & 1) << 2) ^ ((wp >> 1) & 7);
  else return wp & 7;
}
template <int MS> __device__ __forceinline__ uint32_t w_slot_flip(int c) {
  return MS == 16 ? (uint32_t)(c >> 1) : (uint32_t)c;
}

// 16 bytes per lane from a buffer straight into LDS: lane l's data lands at
// dst + 16 l (dst is wave-uniform; it goes through M0).
__device__ __forceinline__ void lds_dma16(rsrc_t r, unsigned char* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

template <int MODE, int BM, int BN, int WGM, int WGN, int MS>
struct BigTile {
  typedef typename ModeT<MODE>::T T;
  static constexpr int kThreads = 64 * WGM * WGN;
  static constexpr int kRowBytes = kBK * 2;
  static constexpr int kWTM = BM / WGM, kWTN = BN / WGN;
  // MFMA shape: MS = 32 -> 32x32x16 (16 k per slice), MS = 16 -> 16x16x32.
  static constexpr int kI = kWTM / MS, kJ = kWTN / MS;
  static constexpr int kSliceK = MS == 32 ? 16 : 32;
  static constexpr int kSlices = kBK / kSliceK;
  static constexpr int kColsPerSlice = 8 / kSlices;  // W columns dequantised per slice
  static constexpr int kPacks = BN / 8;                         // packed words per W row
  static constexpr int kRW = (64 * kPacks / kThreads >= 8) ? 8 : 4;  // W rows per thread
  static constexpr int kWThreads = kPacks * (kBK / kRW);
  static constexpr int kXParts = MODE == MODE_F32S ? 2 : 1;  // hi and lo rows
  static constexpr int kABytes = BM * kRowBytes * kXParts;  // one X buffer
  static constexpr int kBBytes = BN * kRowBytes;  // one W buffer
  // X is prefetched two stages ahead: three X buffers when they fit in the
  // 160 KB of LDS next to the two W buffers.
  static constexpr int kNA = (3 * kABytes + 2 * kBBytes <= 160 * 1024) ? 3 : 2;
  // Layout: X buffers 0..kNA-1, then W buffers 0, 1.
  static constexpr size_t kSmem = (size_t)kNA * kABytes + 2 * (size_t)kBBytes;
  static_assert(MODE != MODE_F32, "large-tile kernel is f16/bf16 (or fp32 split into f16 hi + lo)");
  static_assert(kWThreads <= kThreads, "W tile needs more threads");
  static_assert((BM / 8) % (kThreads / 64) == 0, "X tile must split evenly over the waves");
  static_assert(MS == 32 || MS == 16, "MFMA shape");
  static_assert(kWTM % MS == 0 && kWTN % MS == 0, "wave tile must be whole MFMA blocks");
};

template <int MODE, int ST, int BM, int BN, int WGM, int WGN, int MS, bool SEQ, bool ACT, bool PP>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_big_kernel(GemmArgs a) {
  using C = BigTile<MODE, BM, BN, WGM, WGN, MS>;
  using S = typename Elem<ST>::type;
  constexpr bool F32S = MODE == MODE_F32S;
  static_assert(!F32S || (!PP && MS == 32), "fp32 split mode runs the single-phase 32x32 schedule");
  constexpr int RW = C::kRW;
  constexpr int kSW = (sizeof(S) * 8) / 4;  // dwords holding a pack's 8 scales
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  int t = blockIdx.x;
  if (t < a.swizzled_tiles) {
    const int per_xcd = a.swizzled_tiles >> 3;
    t = (t & 7) * per_xcd + (t >> 3);
  }
  // Raster in groups of group_m row tiles, row tiles fastest inside a group:
  // the tiles an XCD runs at one time then cover a few row tiles by several
  // column tiles, so X and W are each fetched into its L2 by few of them.
  const int gsz = a.group_m * a.tiles_n;
  const int grp = t / gsz;
  const int gm = min(a.group_m, a.tiles_m - grp * a.group_m);
  const int r = t - grp * gsz;
  const int tile_m = grp * a.group_m + r % gm;
  const int tile_n = r / gm;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int np = a.N >> 3;
  // K range of this workgroup: all of K, or its split's run of stages.
  const int split = blockIdx.y;
  const int s_begin = split * a.stages_per_split;
  const int stages = min(a.stages_per_split, a.K / kBK - s_begin);

  // ---- X: copied global -> LDS directly (buffer_load ... lds). One
  // instruction moves 64 x 16 bytes into 1 KB of LDS, lane l landing in row
  // l >> 3, slot l & 7 of an 8-row chunk; so lane l fetches the granule that
  // belongs in that slot, (l & 7) ^ swz(row). Wave w fills chunks w + i*NW.
  constexpr int NW = C::kThreads / 64;
  // PP (ping-pong): the two halves of the waves own the two halves of the
  // rows, and each half loads only its own rows of X: wave w of half h fills
  // chunks (BM/16) h + (w mod NW/2) + i NW/2.
  constexpr int kXIns = BM / 8 / NW;
  auto xchunk = [&](int i) {
    if constexpr (PP) return (wave / (NW / 2)) * (BM / 16) + wave % (NW / 2) + i * (NW / 2);
    else return wave + i * NW;
  };
  const rsrc_t xres = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.K * 2 * C::kXParts));
  uint32_t xvoff[kXIns];
#pragma unroll
  for (int i = 0; i < kXIns; ++i) {
    const int row = 8 * xchunk(i) + (lane >> 3);
    const int grow = min(m0 + row, a.M - 1);  // rows past M read row M-1; never stored
    const int gran = (lane & 7) ^ swz<MS>(row);
    xvoff[i] = (uint32_t)(grow * a.K + gran * 8) * 2u;
  }

  // ---- W: thread covers pack wp, rows wq*RW .. wq*RW+RW-1 of each stage ----
  // RW = 8: consecutive lanes take consecutive packs; their 16-byte LDS
  // writes land in 8 distinct slots. RW = 4: lane bit 0 picks the half
  // granule (k 0-3 or 4-7) and the next bits the pack, so 16 consecutive
  // lanes' 8-byte writes cover all 32 banks once.
  const bool w_act = tid < C::kWThreads;
  const int wp = (RW == 8) ? tid % C::kPacks : (tid >> 1) % C::kPacks;
  const int wq = !w_act ? 0 : (RW == 8) ? tid / C::kPacks : 2 * (tid / (2 * C::kPacks)) + (tid & 1);
  const int pack = min((n0 >> 3) + wp, np - 1);  // ragged N: clamp, never stored
  const rsrc_t wres = make_rsrc(a.qweight, (uint32_t)((int64_t)a.K * np * 4));
  const rsrc_t zres = make_rsrc(a.qzeros, (uint32_t)((int64_t)(a.K / a.group) * np * 4));
  const rsrc_t sres = make_rsrc(a.scales, (uint32_t)((int64_t)(a.K / a.group) * a.N * sizeof(S)));
  const uint32_t wvoff = (uint32_t)((wq * RW) * np + pack) * 4u;
  const uint32_t row_bytes = (uint32_t)np * 4u;
  // LDS byte offset (within a W buffer) of this thread's k-run in column 8 wp:
  // column 8 wp + c uses this slot ^ w_slot_flip(c).
  const uint32_t wl0 = (uint32_t)(wp * 8 * C::kRowBytes) +
                       (uint32_t)((((wq * RW) >> 3) ^ w_slot_base<MS>(wp)) << 4) + (((wq * RW) & 7) ? 8u : 0u);

  // Two register sets for packed W / zeros / scales, used alternately: one
  // being dequantised, the other in flight two stages ahead.
  // F32S: cs holds this lane's output-column scales (one per block column
  // j) of the stage's group, applied to the group's sums.
  constexpr int kCS = F32S ? C::kJ : 0;
  struct WRegs {
    uint32_t w[RW];
    uint32_t z;
    uint32_t sv[kSW];
    float cs[kCS > 0 ? kCS : 1];
  };
  // W(j) lives in wr[j % 2]: loaded two stages ahead of its MFMAs.
  WRegs wr[2];

  auto load_w = [&](int s, WRegs& r_) {
    s += s_begin;
    const int k0 = s * kBK;
#pragma unroll
    // Plain (cached) loads: every row tile of the grid re-reads this W block,
    // from L2 when the tiles sharing it run close together.
    for (int r = 0; r < RW; ++r) r_.w[r] = buf_load_u32(wres, wvoff, (uint32_t)(k0 + r) * row_bytes);
    const int grp = s >> a.grp_shift;  // a 64-row stage lies in one group
    r_.z = buf_load_u32(zres, (uint32_t)(grp * np + pack) * 4u, 0);
    const uint32_t soff = (uint32_t)(grp * a.N + pack * 8) * (uint32_t)sizeof(S);
#pragma unroll
    for (int v = 0; v < kSW; v += 4) {
      const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(sres, soff + v * 4, 0, 0);
      r_.sv[v] = q[0]; r_.sv[v + 1] = q[1]; r_.sv[v + 2] = q[2]; r_.sv[v + 3] = q[3];
    }
    if constexpr (F32S) {
      // One VMEM load per block column, issued with the stage's other loads
      // (the explicit vmcnt counts below include them).
#pragma unroll
      for (int j = 0; j < kCS; ++j) {
        const int col = min(n0 + wn * C::kWTN + 32 * j + (lane & 31), a.N - 1);
        const uint32_t o = (uint32_t)(grp * a.N + col) * (uint32_t)sizeof(S);
        if constexpr (sizeof(S) == 4) {
          r_.cs[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sres, o, 0, 0));
        } else {
          const uint16_t hbits = __builtin_amdgcn_raw_buffer_load_b16(sres, o, 0, 0);
          r_.cs[j] = to_f32(__builtin_bit_cast(S, hbits));
        }
      }
    }
  };
  auto scale_of = [&](const uint32_t (&sv)[kSW], int c) -> float {
    if constexpr (sizeof(S) == 4) return __builtin_bit_cast(float, sv[c]);
    else {
      const uint16_t h = (uint16_t)(sv[c >> 1] >> (16 * (c & 1)));
      return to_f32(__builtin_bit_cast(S, h));
    }
  };

  auto load_x = [&](int s, int buf) {
    const uint32_t koff = (uint32_t)((s_begin + s) * kBK) * 2u;
#pragma unroll
    for (int i = 0; i < kXIns; ++i) {
      lds_dma16(xres, smem_raw + buf * C::kABytes + xchunk(i) * 1024, xvoff[i], koff);
    }
    if constexpr (F32S) {  // the lo rows, BM rows after the hi rows in LDS
#pragma unroll
      for (int i = 0; i < kXIns; ++i)
        lds_dma16(xres, smem_raw + buf * C::kABytes + BM * C::kRowBytes + xchunk(i) * 1024, xvoff[i],
                  koff + a.lo_off);
    }
  };

  // Dequantise column c of the pack (RW k values) and write it to W buffer
  // buf: LDS column 8 wp + c, whose slot is that of column 8 wp flipped by c.
  auto deq_store_col = [&](const WRegs& r_, int c, int buf) {
    uint32_t dq[RW / 2];
    const int L = lane_of_col<SEQ>(c);
    const uint32_t zw = r_.z;
    if constexpr (F32S) {
      // Exact f16 integers q - z: magic numbers of the nibble and the zero,
      // one exact v_pk_add_f16; the scale is applied to the group's sums.
      const f16x2 fz = __builtin_bit_cast(f16x2, nib_f16x2(zw, zw, L));
#pragma unroll
      for (int r = 0; r < RW / 2; ++r) {
        const f16x2 fv = __builtin_bit_cast(f16x2, nib_f16x2(r_.w[2 * r], r_.w[2 * r + 1], L));
        dq[r] = __builtin_bit_cast(uint32_t, fv - fz);
      }
    } else if constexpr (MODE == MODE_F16) {
      // Nibbles of packed lane L as f16 magic numbers (1024 + q or 64 + q),
      // zero likewise; (v - zc) is exact and * sc rounds once.
      const uint32_t zc = nib_f16x2(zw, zw, L);
      uint32_t scc;
      if constexpr (ST == AWQ_F16) {
        scc = __builtin_amdgcn_perm(r_.sv[c >> 1], r_.sv[c >> 1], (c & 1) ? 0x03020302u : 0x01000100u);
      } else {
        const f16_t sf = (f16_t)scale_of(r_.sv, c);
        scc = (uint32_t)__builtin_bit_cast(uint16_t, sf) * 0x10001u;
      }
      const f16x2 fz = __builtin_bit_cast(f16x2, zc);
      const f16x2 fs = __builtin_bit_cast(f16x2, scc);
#pragma unroll
      for (int r = 0; r < RW / 2; ++r) {
        const f16x2 fv = __builtin_bit_cast(f16x2, nib_f16x2(r_.w[2 * r], r_.w[2 * r + 1], L));
        dq[r] = __builtin_bit_cast(uint32_t, (fv - fz) * fs);
      }
    } else {
      // bf16: (q - z) * s is exact in f32 (5-bit by at most 24-bit
      // significand); one rounding to bf16 gives the bf16 product.
      const int z = (int)((zw >> (4 * L)) & 0xFu);
      const float sv_ = scale_of(r_.sv, c);
      // 16-bit scales: z s is exact, so fma(q, s, -z s) is (q - z) s exactly
      // in one op after the conversion of q (v_bfe_u32, v_cvt_f32_ubyte0,
      // v_fma_f32). f32 scales: (q - z) converted, then multiplied.
      const float nzs = -(float)z * sv_;
#pragma unroll
      for (int r = 0; r < RW / 2; ++r) {
        const uint32_t q0 = (r_.w[2 * r] >> (4 * L)) & 0xFu;
        const uint32_t q1 = (r_.w[2 * r + 1] >> (4 * L)) & 0xFu;
        float d0, d1;
        if constexpr (sizeof(S) == 4) {
          d0 = (float)((int)q0 - z) * sv_;
          d1 = (float)((int)q1 - z) * sv_;
        } else {
          d0 = __builtin_fmaf((float)q0, sv_, nzs);
          d1 = __builtin_fmaf((float)q1, sv_, nzs);
        }
        const bf16_t v0 = from_f32<bf16_t>(d0);
        const bf16_t v1 = from_f32<bf16_t>(d1);
        dq[r] = (uint32_t)__builtin_bit_cast(uint16_t, v0) | ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
      }
    }
    if constexpr (C::kWThreads < C::kThreads) {
      if (!w_act) return;
    }
    uint32_t off = wl0;
    asm volatile("" : "+v"(off));  // recompute per use: keeps 8 addresses out of the register file
    unsigned char* dst = smem_raw + ((off ^ (w_slot_flip<MS>(c) << 4)) + (uint32_t)(C::kNA * C::kABytes + buf * C::kBBytes + c * C::kRowBytes));
    if constexpr (RW == 8)
      *reinterpret_cast<u32x4*>(dst) = u32x4{dq[0], dq[1], dq[2], dq[3]};
    else
      *reinterpret_cast<u32x2*>(dst) = u32x2{dq[0], dq[1]};
  };

  // ---- MFMA operand addressing -------------------------------------------
  typedef float AccT __attribute__((ext_vector_type(MS == 32 ? 16 : 4)));
  AccT acc[C::kI][C::kJ];
  // F32S: the current group's sums (MFMA target), folded into acc with the
  // group's column scales gsc at the group's end.
  constexpr int kPI = F32S ? C::kI : 1, kPJ = F32S ? C::kJ : 1;
  AccT pacc[kPI][kPJ];
  float gsc[kPJ];
#pragma unroll
  for (int i = 0; i < C::kI; ++i)
#pragma unroll
    for (int j = 0; j < C::kJ; ++j) acc[i][j] = AccT{};
#pragma unroll
  for (int i = 0; i < kPI; ++i)
#pragma unroll
    for (int j = 0; j < kPJ; ++j) pacc[i][j] = AccT{};
  // 16x16x32: lane l reads row (l & 15) of a block, granule 4 kq + (l >> 4);
  // the slice kq flips granule bit 2 (kq << 6 in bytes), so one base per
  // block row plus an XOR.
  uint32_t a16[C::kI], b16[C::kJ];
  if constexpr (MS == 16) {
    const int l16 = lane & 15, h4 = lane >> 4;
#pragma unroll
    for (int i = 0; i < C::kI; ++i) {
      const int row = wm * C::kWTM + 16 * i + l16;
      a16[i] = (uint32_t)(row * C::kRowBytes + ((h4 ^ swz<MS>(row)) << 4));
    }
#pragma unroll
    for (int j = 0; j < C::kJ; ++j) {
      const int col = wn * C::kWTN + 16 * j + l16;
      b16[j] = (uint32_t)(C::kNA * C::kABytes + col * C::kRowBytes + ((h4 ^ swz<MS>(col)) << 4));
    }
  }
  const int h = lane >> 5;  // which 8-k half of the 16-k MFMA slice
  // Row wm*WTM + 32 i + (lane & 31): its swizzle is swz(lane & 31) with bit 2
  // flipped by (4 i + wm*WTM/8) & 4, so two base registers per operand and
  // the 32-row step as an immediate. k-slice kq flips slot bits 1-2 (kq << 5).
  const uint32_t lr = (uint32_t)(lane & 31);
  const uint32_t a_base = (uint32_t)((wm * C::kWTM) * C::kRowBytes) + lr * C::kRowBytes +
                          (uint32_t)((h ^ swz<MS>((int)lr)) << 4);
  const uint32_t b_base = (uint32_t)(C::kNA * C::kABytes) + (uint32_t)((wn * C::kWTN) * C::kRowBytes) +
                          lr * C::kRowBytes + (uint32_t)((h ^ swz<MS>((int)lr)) << 4);
  const uint32_t a_fl = (uint32_t)(((wm * (C::kWTM / 8)) & 4) << 4);
  const uint32_t b_fl = (uint32_t)(((wn * (C::kWTN / 8)) & 4) << 4);
  const uint32_t a_par[2] = {a_base ^ a_fl, a_base ^ a_fl ^ 64u};
  const uint32_t b_par[2] = {b_base ^ b_fl, b_base ^ b_fl ^ 64u};
  typedef typename std::conditional<MODE == MODE_BF16, bf16x8, f16x8>::type V8;
  // X fragments (kI), W fragments (kJ), and for F32S the lo X fragments (kI).
  constexpr int kFA2 = F32S ? C::kI : 0;
  typedef V8 Frags[C::kI + C::kJ + kFA2];
  auto read_frags = [&](int abuf, int bbuf, int kq, Frags& f) {
    if constexpr (MS == 16) {
#pragma unroll
      for (int i = 0; i < C::kI; ++i)
        f[i] = *reinterpret_cast<const V8*>(smem_raw + (a16[i] ^ (uint32_t)(kq << 6)) + abuf * C::kABytes);
#pragma unroll
      for (int j = 0; j < C::kJ; ++j)
        f[C::kI + j] = *reinterpret_cast<const V8*>(smem_raw + (b16[j] ^ (uint32_t)(kq << 6)) + bbuf * C::kBBytes);
      return;
    }
#pragma unroll
    for (int i = 0; i < C::kI; ++i)
      f[i] = *reinterpret_cast<const V8*>(smem_raw + (a_par[i & 1] ^ (uint32_t)(kq << 5)) +
                                          (abuf * C::kABytes + i * 32 * C::kRowBytes));
#pragma unroll
    for (int j = 0; j < C::kJ; ++j)
      f[C::kI + j] = *reinterpret_cast<const V8*>(smem_raw + (b_par[j & 1] ^ (uint32_t)(kq << 5)) +
                                                  (bbuf * C::kBBytes + j * 32 * C::kRowBytes));
    if constexpr (F32S) {
      // lo rows: BM rows further; (BM + r) has the swizzle of r (BM % 64 == 0).
#pragma unroll
      for (int i = 0; i < C::kI; ++i)
        f[C::kI + C::kJ + i] = *reinterpret_cast<const V8*>(
            smem_raw + (a_par[i & 1] ^ (uint32_t)(kq << 5)) +
            (abuf * C::kABytes + (BM + i * 32) * C::kRowBytes));
    }
  };
  auto mfmas = [&](const Frags& f) {
    if constexpr (F32S) {
#pragma unroll
      for (int i = 0; i < C::kI; ++i)
#pragma unroll
        for (int j = 0; j < C::kJ; ++j) {
          pacc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i], f[C::kI + j], pacc[i][j], 0, 0, 0);
          pacc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[C::kI + C::kJ + i], f[C::kI + j], pacc[i][j],
                                                               0, 0, 0);
        }
      return;
    }
#pragma unroll
    for (int i = 0; i < C::kI; ++i)
#pragma unroll
      for (int j = 0; j < C::kJ; ++j) {
        if constexpr (MS == 16 && MODE == MODE_F16)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f[i], f[C::kI + j], acc[i][j], 0, 0, 0);
        else if constexpr (MS == 16)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f[i], f[C::kI + j], acc[i][j], 0, 0, 0);
        else if constexpr (MODE == MODE_F16)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i], f[C::kI + j], acc[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], f[C::kI + j], acc[i][j], 0, 0, 0);
      }
  };
  // Output element r of block (i, j) for this lane: 32x32 blocks hold rows
  // 8 (r / 4) + 4 (lane / 32) + r % 4 of column lane % 32; 16x16 blocks rows
  // 4 (lane / 16) + r of column lane % 16.
  constexpr int kAccN = MS == 32 ? 16 : 4;
  auto out_row = [&](int i, int r) -> int {
    if constexpr (MS == 32) return m0 + wm * C::kWTM + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    else return m0 + wm * C::kWTM + 16 * i + 4 * (lane >> 4) + r;
  };
  auto out_col = [&](int j) -> int {
    if constexpr (MS == 32) return n0 + wn * C::kWTN + 32 * j + (lane & 31);
    else return n0 + wn * C::kWTN + 16 * j + (lane & 15);
  };

  // VMEM instructions one stage issues: packed W rows, the zero word, the
  // scales (16 bytes each), the LDS-direct X granules.
  constexpr int kVmPerStage = RW + 1 + (kSW + 3) / 4 + kCS + kXIns * C::kXParts;
  static_assert(kVmPerStage < 64, "vmcnt range");
  constexpr int kNA = C::kNA;
  // End-of-stage wait: with three X buffers the X loads of stage s+1 were
  // issued a stage earlier, so this stage's loads may stay in flight; with
  // two they were issued last in this stage and everything must land.
  constexpr int kVmWait = (kNA == 3) ? kVmPerStage : 0;

  if constexpr (PP) {
    // ---- ping-pong schedule ------------------------------------------------
    // Half 0 (waves 0..NW/2-1, rows 0..BM/2-1) and half 1 (the other rows)
    // run one phase apart: while one half multiplies, the other reads its
    // operands from LDS, issues the loads of stage s+2 and dequantises
    // W(s+1). Every stage is two phases, each closed by a barrier; half 1
    // takes one extra barrier before its loop and half 0 one after, so the
    // counts match. A memory phase of stage s of one half and the compute
    // phase of stage s-1 (half 1) or s (half 0) of the other run together.
    //   X: each half loads and reads only its own rows, three buffers, two
    //      stages ahead (buffer (s+2) % 3 last held X(s-1), read by this half
    //      in its memory phase s-1).
    //   W: both halves dequantise W(s+1) into buffer (s+1) % 2 in memory
    //      phase s. Its previous contents W(s-1) were read by half 0 before
    //      the barrier that half 1's memory phase s-1 ends with, and by half 1
    //      before its memory phase s-1 ended; W(s+1) is complete at the end of
    //      half 1's memory phase s, before either half reads it in memory
    //      phase s+1. So a stage's W operands are all read in its memory
    //      phase; X of its second k-slice is read in the compute phase.
    static_assert(kNA == 3 && WGM % 2 == 0 && (BM / 16) % (NW / 2) == 0 && MS == 16 && C::kSlices == 2,
                  "ping-pong layout");
    const bool h1 = wave >= NW / 2;
    WRegs& wq_ = wr[0];  // one register set: W(s+2) is loaded once W(s+1) is dequantised
    load_w(0, wq_);
    load_x(0, 0);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
#pragma unroll
    for (int c = 0; c < 8; ++c) deq_store_col(wq_, c, 0);
    load_x(min(1, stages - 1), 1);
    load_w(min(1, stages - 1), wq_);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(kVmPerStage, 0));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (h1) __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    auto read_a = [&](int xb, int kq, int i) {
      return *reinterpret_cast<const V8*>(smem_raw + (a16[i] ^ (uint32_t)(kq << 6)) + xb * C::kABytes);
    };
    auto read_b = [&](int wb, int kq, int j) {
      return *reinterpret_cast<const V8*>(smem_raw + (b16[j] ^ (uint32_t)(kq << 6)) + wb * C::kBBytes);
    };
    auto mma = [&](const V8& x, const V8& w, AccT& d) {
      if constexpr (MODE == MODE_F16) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, w, d, 0, 0, 0);
      else d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, w, d, 0, 0, 0);
    };
    auto step_pp = [&](int s, int xb, int wb) {
      V8 fa[C::kI], fb0[C::kJ], fb1[C::kJ];
      // Memory phase: W operands of both k-slices and X of the first.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < C::kJ; ++j) fb0[j] = read_b(wb, 0, j);
#pragma unroll
      for (int j = 0; j < C::kJ; ++j) fb1[j] = read_b(wb, 1, j);
#pragma unroll
      for (int i = 0; i < C::kI; ++i) fa[i] = read_a(xb, 0, i);
      load_x(min(s + 2, stages - 1), (xb + 2) % 3);
      // X(s+1) and W(s+1), issued in the previous memory phase, have landed.
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(kXIns, 15));
#pragma unroll
      for (int c = 0; c < 8; ++c) deq_store_col(wq_, c, wb ^ 1);
      load_w(min(s + 2, stages - 1), wq_);
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(kVmPerStage, 0));
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      // Compute phase: X of the second k-slice (rows private to this half)
      // is read row block by row block into the registers the first slice
      // has finished with. Raised wave priority: the multiplying half wins
      // issue over the half in its memory phase.
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < C::kI; ++i) {
#pragma unroll
        for (int j = 0; j < C::kJ; ++j) mma(fa[i], fb0[j], acc[i][j]);
        fa[i] = read_a(xb, 1, i);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < C::kI; ++i)
#pragma unroll
        for (int j = 0; j < C::kJ; ++j) mma(fa[i], fb1[j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    for (int s = 0; s < stages; s += 6) {
#pragma unroll
      for (int u = 0; u < 6; ++u) {
        if (u == 0 || s + u < stages) step_pp(s + u, u % 3, u % 2);
      }
    }
    if (!h1) __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  } else {
  // ---- prologue ------------------------------------------------------------
  load_w(0, wr[0]);
  load_x(0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
#pragma unroll
  for (int c = 0; c < 8; ++c) deq_store_col(wr[0], c, 0);
  if constexpr (F32S) {
#pragma unroll
    for (int j = 0; j < kPJ; ++j) gsc[j] = wr[0].cs[j];
  }
  load_w(min(1, stages - 1), wr[1]);
  if constexpr (kNA == 3) load_x(min(1, stages - 1), 1);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(kVmWait, 0));
  __builtin_amdgcn_s_barrier();

  // ---- main loop -----------------------------------------------------------
  // Stage s reads X buffer s % kNA and W buffer s % 2. It issues the packed
  // W / zeros / scales of stage s+2 (registers) and then the LDS-direct X
  // loads of stage s+2 (buffer (s+2) % kNA; with kNA == 2 X goes one stage
  // ahead instead), dequantises W(s+1) into W buffer (s+1) % 2 while its
  // MFMAs run, and ends with an explicit wait: vmcnt(loads issued in this
  // stage) leaves this stage's prefetches in flight but guarantees the X of
  // stage s+1 has landed, lgkmcnt(0) completes this wave's LDS writes; then
  // the barrier. (A plain s_barrier, not __syncthreads(): the latter would
  // also wait for the X loads just issued.) The body is branch-free: at the
  // tail the prefetches clamp to the last stage and land in buffers nobody
  // reads any more.
  auto interleave = [&]() {
    constexpr int kM = C::kI * C::kJ * (F32S ? 2 : 1);
    constexpr int kValu = F32S ? 2 : MS == 32 ? 4 : 3;  // VALU ops after each MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, C::kI + C::kJ + kFA2, 0);  // DS read
#pragma unroll
    for (int q = 0; q < kM; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);  // VALU
    }
    __builtin_amdgcn_sched_group_barrier(0x200, 2 * C::kColsPerSlice, 0);  // DS write
  };
  constexpr int kXAhead = (kNA == 3) ? 2 : 1;
  auto step = [&](int s, int abuf, int bbuf, WRegs& deq, WRegs& next) {
    Frags f0, f1;
    read_frags(abuf, bbuf, 0, f0);
    load_w(min(s + 2, stages - 1), next);
    __builtin_amdgcn_sched_barrier(0);
    load_x(min(s + kXAhead, stages - 1), (abuf + kXAhead) % kNA);
    constexpr int kCPS = C::kColsPerSlice;
#pragma unroll
    for (int kq = 0; kq < C::kSlices; kq += 2) {
      __builtin_amdgcn_sched_barrier(0);
      read_frags(abuf, bbuf, kq + 1, f1);
      mfmas(f0);
#pragma unroll
      for (int c = 0; c < kCPS; ++c) deq_store_col(deq, kq * kCPS + c, bbuf ^ 1);
      interleave();
      __builtin_amdgcn_sched_barrier(0);
      if (kq + 2 < C::kSlices) read_frags(abuf, bbuf, kq + 2, f0);
      mfmas(f1);
#pragma unroll
      for (int c = 0; c < kCPS; ++c) deq_store_col(deq, (kq + 1) * kCPS + c, bbuf ^ 1);
      interleave();
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (F32S) {
      // End of the group (or of this workgroup's K run): fold the group's
      // sums into acc with its column scales. Then take the scales of stage
      // s+1 (its W registers have landed: they were just dequantised).
      const int gs = s_begin + s;
      if (((gs + 1) & ((1 << a.grp_shift) - 1)) == 0 || s + 1 == stages) {
#pragma unroll
        for (int i = 0; i < C::kI; ++i)
#pragma unroll
          for (int j = 0; j < C::kJ; ++j) {
#pragma unroll
            for (int r = 0; r < kAccN; ++r) acc[i][j][r] = __builtin_fmaf(gsc[j], pacc[i][j][r], acc[i][j][r]);
            pacc[i][j] = AccT{};
          }
      }
#pragma unroll
      for (int j = 0; j < kPJ; ++j) gsc[j] = deq.cs[j];
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(kVmWait, 0));
    __builtin_amdgcn_s_barrier();
  };
  // Unrolled over lcm(kNA, 2) stages so buffers and register sets are
  // compile-time: step s dequantises W(s+1) from wr[(s+1) % 2] and loads
  // W(s+2) into wr[s % 2], whose W(s) was dequantised in step s-1.
  constexpr int kU = (kNA == 3) ? 6 : 2;
  for (int s = 0; s < stages; s += kU) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (u == 0 || s + u < stages) step(s + u, u % kNA, u % 2, wr[(u + 1) % 2], wr[u % 2]);
    }
  }
  }

  // ---- epilogue --------------------------------------------------------------
  if constexpr (F32S) {
    // Undo the row scaling 2^e of the prepass (exact: a power of two).
#pragma unroll
    for (int i = 0; i < C::kI; ++i)
#pragma unroll
      for (int r = 0; r < kAccN; ++r) {
        const float rf = a.rowfac[min(out_row(i, r), a.M - 1)];
#pragma unroll
        for (int j = 0; j < C::kJ; ++j) acc[i][j][r] *= rf;
      }
  }
  if (a.splits > 1) {
    // Split-K: publish this split's tile with agent-scope (write-through)
    // stores, wait for them, count the arrival; the last workgroup of the tile
    // re-reads all splits' partials (agent-scope loads, split order, in a
    // coalesced row-major walk of the tile), adds the bias and writes y, and
    // re-arms the counter.
    // The partial tile passes through the (idle) LDS in row passes and leaves
    // as 16-byte pieces of whole rows with the sc1 policy: a wave store
    // instruction moves 1 KB instead of 256 scattered bytes (the vector
    // memory path takes about 16 clocks per instruction whatever its width).
    const rsrc_t pres = make_rsrc(a.partial, (uint32_t)((int64_t)a.splits * a.M * a.N * 4));
    const uint32_t sstride = (uint32_t)((int64_t)a.M * a.N * 4);
    {
      constexpr int pitch = BN * 4 + 16;  // bytes per staged row (bank spread)
      constexpr int fit = (int)(C::kSmem / pitch) & ~(MS - 1);
      constexpr int rows_pass = fit < BM ? fit : BM;
      constexpr int gran = BN / 4;  // 16-byte pieces per tile row
      static_assert(rows_pass >= MS, "staged rows");
      // LDS-direct prefetches of clamped tail stages may still be landing.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      for (int p0 = 0; p0 < BM; p0 += rows_pass) {
        __syncthreads();
#pragma unroll
        for (int j = 0; j < C::kJ; ++j) {
          const int lc = out_col(j) - n0;
#pragma unroll
          for (int i = 0; i < C::kI; ++i) {
#pragma unroll
            for (int r = 0; r < kAccN; ++r) {
              const int lr = out_row(i, r) - m0 - p0;
              if (rows_pass < BM && (lr < 0 || lr >= rows_pass)) continue;
              *reinterpret_cast<float*>(smem_raw + lr * pitch + lc * 4) = acc[i][j][r];
            }
          }
        }
        __syncthreads();
        const int rows = min(rows_pass, BM - p0);
        for (int g = tid; g < rows * gran; g += C::kThreads) {
          const int row = g / gran, gc = g % gran;
          const int m = m0 + p0 + row;
          const int n = n0 + gc * 4;  // N % 32 == 0: a piece is all in or all out
          if (m < a.M && n < a.N)
            __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4*>(smem_raw + row * pitch + gc * 16),
                                                   pres, (uint32_t)(((int64_t)m * a.N + n) * 4),
                                                   (uint32_t)split * sstride, kCachePolicySC1);
        }
      }
    }
    // Partials complete before the arrival (split-K handshake, awq_common.h).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // The flag lives in the (now idle) tile buffers: a static __shared__
    // variable would push the 160 KB configuration over the LDS limit.
    volatile int* s_last = reinterpret_cast<volatile int*>(smem_raw);
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&a.counters[t * kTileCtrStride], 1u,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_last = (prev == (uint32_t)(a.splits - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!*s_last) return;
    // 4 consecutive columns per thread and step (N % 8 == 0 keeps a group of
    // 4 inside the row) as one 16-byte agent-scope (sc1) load per split, kG
    // steps at a time with 8 splits each: 8 kG loads in flight per thread.
    // (One step at a time left this single workgroup latency-bound on the
    // splits x tile partials: ~30 us for a 128 x 128 tile and 8 splits.)
    // Every slot is loaded (indices clamped into the workspace) and only the
    // valid ones are added and stored, so nothing read is ever undefined.
    constexpr int kG = 4;
    constexpr int kStep4 = C::kThreads * 4;
    for (int e0 = tid * 4; e0 < BM * BN; e0 += kG * kStep4) {
      uint32_t off[kG];
      bool ok[kG];
      float v[kG][4];
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        const int e = e0 + g * kStep4;
        const int m = m0 + e / BN, n = n0 + e % BN;
        ok[g] = e < BM * BN && m < a.M && n < a.N;
        off[g] = (uint32_t)(((int64_t)min(m, a.M - 1) * a.N + min(n, a.N - 4)) * 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[g][q] = 0.f;
      }
      for (int s0 = 0; s0 < a.splits; s0 += 8) {
        float t8[kG][8][4];
#pragma unroll
        for (int g = 0; g < kG; ++g)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const u32x4 w4 = __builtin_amdgcn_raw_buffer_load_b128(
                pres, off[g], (uint32_t)min(s0 + j, a.splits - 1) * sstride, kCachePolicySC1);
            // Elements through plain scalars: __builtin_bit_cast applied to
            // a vector element directly reads the wrong element (hipcc 7.2).
            const uint32_t e0 = w4[0], e1 = w4[1], e2 = w4[2], e3 = w4[3];
            t8[g][j][0] = __uint_as_float(e0);
            t8[g][j][1] = __uint_as_float(e1);
            t8[g][j][2] = __uint_as_float(e2);
            t8[g][j][3] = __uint_as_float(e3);
          }
#pragma unroll
        for (int g = 0; g < kG; ++g)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const bool live = s0 + j < a.splits;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[g][q] += live ? t8[g][j][q] : 0.f;
          }
      }
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        if (!ok[g]) continue;
        const int e = e0 + g * kStep4;
        const int m = m0 + e / BN, n = n0 + e % BN;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (a.bias) v[g][q] += load_f32_any(a.bias, n + q, a.bt);
        // n % 4 == 0: the gate/up pairs are (q, q ^ 1) of this thread; plain
        // outputs leave as one 16- or 8-byte store of the 4 columns.
        if (ACT) {
          store_act_quad(a.y, a.yt, m, n, a.N, v[g][0], v[g][1], v[g][2], v[g][3]);
        } else if (a.yt == AWQ_F32) {
          *reinterpret_cast<u32x4*>(static_cast<float*>(a.y) + (int64_t)m * a.N + n) =
              u32x4{__float_as_uint(v[g][0]), __float_as_uint(v[g][1]), __float_as_uint(v[g][2]),
                    __float_as_uint(v[g][3])};
        } else if (a.yt == AWQ_F16) {
          typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
          *reinterpret_cast<h4_t*>(static_cast<f16_t*>(a.y) + (int64_t)m * a.N + n) =
              h4_t{(_Float16)v[g][0], (_Float16)v[g][1], (_Float16)v[g][2], (_Float16)v[g][3]};
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) store_out(a.y, a.yt, 0, m, n + q, a.N, v[g][q], 0.f);
        }
      }
    }
    if (tid == 0)
      __hip_atomic_store(&a.counters[t * kTileCtrStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if constexpr (!ACT) {
    // The tile goes through LDS (idle now) so that Y is written in 16-byte
    // pieces of whole rows. Stored straight from the MFMA layout, a wave's
    // store instruction covers 16 or 32 columns of several rows, pieces of
    // 128-byte lines that were each written back in parts (HBM writes 1.75x
    // the output bytes at 2048 x 4096 -> 14336 with f16 output; staged: 1.0x,
    // 240 -> 222 us). Rows of the staged tile are BN * es + 16 bytes apart
    // (bank spread); an f32 tile that does not fit goes in row passes.
    auto staged = [&](auto es_c) {
      constexpr int es = decltype(es_c)::value;
      constexpr int pitch = BN * es + 16;
      constexpr int rows_pass = ((int)(C::kSmem / pitch) & ~(MS - 1)) < BM ? ((int)(C::kSmem / pitch) & ~(MS - 1)) : BM;
      constexpr int gran = BN * es / 16;  // 16-byte pieces per tile row
      static_assert(rows_pass >= MS, "staged rows");
      char* yb = static_cast<char*>(a.y);
      for (int p0 = 0; p0 < BM; p0 += rows_pass) {
        __syncthreads();
#pragma unroll
        for (int j = 0; j < C::kJ; ++j) {
          const int n = out_col(j);
          const float bias = (a.bias && n < a.N) ? load_f32_any(a.bias, n, a.bt) : 0.f;
          const int lc = n - n0;
#pragma unroll
          for (int i = 0; i < C::kI; ++i) {
#pragma unroll
            for (int r = 0; r < kAccN; ++r) {
              const int lr = out_row(i, r) - m0 - p0;
              if (rows_pass < BM && (lr < 0 || lr >= rows_pass)) continue;
              const float v = acc[i][j][r] + bias;
              unsigned char* d = smem_raw + lr * pitch + lc * es;
              if constexpr (es == 4) *reinterpret_cast<float*>(d) = v;
              else if (a.yt == AWQ_BF16) *reinterpret_cast<bf16_t*>(d) = from_f32<bf16_t>(v);
              else *reinterpret_cast<f16_t*>(d) = from_f32<f16_t>(v);
            }
          }
        }
        __syncthreads();
        const int rows = min(rows_pass, BM - p0);
        for (int g = tid; g < rows * gran; g += C::kThreads) {
          const int row = g / gran, gc = g % gran;
          const int m = m0 + p0 + row;
          const int n = n0 + gc * 16 / es;  // N % 32 == 0: a piece is all in or all out
          const u32x4 v = *reinterpret_cast<const u32x4*>(smem_raw + row * pitch + gc * 16);
          if (m < a.M && n < a.N) *reinterpret_cast<u32x4*>(yb + ((int64_t)m * a.N + n) * es) = v;
        }
      }
    };
    // LDS-direct prefetches of clamped tail stages may still be landing.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (a.yt == AWQ_F32) staged(std::integral_constant<int, 4>{});
    else staged(std::integral_constant<int, 2>{});
    return;
  }
  // SiLU(gate) * up: column lane % 32 (or % 16) and its xor-1 neighbour are
  // a gate/up pair; the even lane's output (column n / 2 of the half-width
  // Y) goes into the staged half-width tile (it fits the LDS in one pass),
  // which leaves as 16-byte pieces of whole rows.
  auto staged_act = [&](auto es_c) {
    constexpr int es = decltype(es_c)::value;
    constexpr int kHW = BN / 2;
    constexpr int pitch = kHW * es + 16;
    constexpr int gran = kHW * es / 16;  // 16-byte pieces per half-width row
    static_assert((size_t)BM * pitch <= C::kSmem && (kHW * es) % 16 == 0, "staged half-width tile");
    char* yb = static_cast<char*>(a.y);
    const int64_t hn = a.N >> 1;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < C::kJ; ++j) {
      const int n = out_col(j);
      const float bias = (a.bias && n < a.N) ? load_f32_any(a.bias, n, a.bt) : 0.f;
      const int lc = (n - n0) >> 1;
      const bool even = (n & 1) == 0;
#pragma unroll
      for (int i = 0; i < C::kI; ++i) {
#pragma unroll
        for (int r = 0; r < kAccN; ++r) {
          const float v = acc[i][j][r] + bias;
          const float pv = __shfl_xor(v, 1, 64);
          if (even) {
            const float o = silu_mul(v, pv);
            unsigned char* d = smem_raw + (out_row(i, r) - m0) * pitch + lc * es;
            if constexpr (es == 4) *reinterpret_cast<float*>(d) = o;
            else if (a.yt == AWQ_BF16) *reinterpret_cast<bf16_t*>(d) = from_f32<bf16_t>(o);
            else *reinterpret_cast<f16_t*>(d) = from_f32<f16_t>(o);
          }
        }
      }
    }
    __syncthreads();
    for (int g = tid; g < BM * gran; g += C::kThreads) {
      const int row = g / gran, gc = g % gran;
      const int m = m0 + row;
      const int64_t n2 = (n0 >> 1) + gc * 16 / es;  // N / 2 % 16 == 0: a piece is all in or all out
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem_raw + row * pitch + gc * 16);
      if (m < a.M && n2 < hn) *reinterpret_cast<u32x4*>(yb + ((int64_t)m * hn + n2) * es) = v;
    }
  };
  // LDS-direct prefetches of clamped tail stages may still be landing.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (a.yt == AWQ_F32) staged_act(std::integral_constant<int, 4>{});
  else staged_act(std::integral_constant<int, 2>{});
}

// Prepass of MODE_F32S: one workgroup per row of x [M, K] f32 (K % 4 == 0).
// The row's largest finite |x| gives e with max |x| 2^e in [2^14, 2^15)
// (e = 0 for a row of zeros or with no finite value, clamped to +-126 so
// 2^-e stays a normal float); then hi = f16(x 2^e), lo = f16(x 2^e - hi)
// (x 2^e is exact, and so is x 2^e - hi: both lie in one binade of f32), so
// |x - (hi + lo) 2^-e| <= 2^-22 max |x|. Outputs: hi [M][K], lo [M][K]
// (f16), rowfac [M] = 2^-e. Non-finite values stay non-finite.
__global__ __launch_bounds__(256) void x_split_kernel(const float* __restrict__ x, f16_t* __restrict__ hi,
                                                      f16_t* __restrict__ lo, float* __restrict__ rowfac,
                                                      int K) {
  __shared__ float wmax[4];
  const int64_t row = (int64_t)blockIdx.x * K;
  const float4* xr = reinterpret_cast<const float4*>(x + row);
  const int n4 = K >> 2;
  float mx = 0.f;
  for (int i = threadIdx.x; i < n4; i += 256) {
    const float4 v = xr[i];
    const float m4 = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    mx = (m4 <= 3.4028234e38f) ? fmaxf(mx, m4) : mx;  // finite values only (NaN, inf skipped)
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  int e = 0;
  if (mx > 0.f) {
    int E;
    frexpf(mx, &E);  // mx in [2^(E-1), 2^E)
    e = min(max(15 - E, -126), 126);
  }
  if (threadIdx.x == 0) rowfac[blockIdx.x] = ldexpf(1.f, -e);
  typedef f16_t h4_t __attribute__((ext_vector_type(4)));
  for (int i = threadIdx.x; i < n4; i += 256) {
    const float4 v = xr[i];
    const float t[4] = {ldexpf(v.x, e), ldexpf(v.y, e), ldexpf(v.z, e), ldexpf(v.w, e)};
    h4_t h, l;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      h[q] = (f16_t)t[q];
      l[q] = (f16_t)(t[q] - (float)h[q]);
    }
    *reinterpret_cast<h4_t*>(hi + row + 4 * i) = h;
    *reinterpret_cast<h4_t*>(lo + row + 4 * i) = l;
  }
}

// Row tiles per raster group. An XCD runs about CUs/8 tiles at once; with a
// rows by b columns of them (a*b fixed) it fetches a*BM + b*BN/4 row-bytes of
// X and W per K step (f16 X, 4-bit W), least near a = sqrt(CUs/8 * BN / (4 BM)).
int raster_group_m(int tiles_m, int bm, int bn) {
  if (const int v = tuning(kTuneGemmGroupM, 0); v > 0) return std::min(v, tiles_m);
  const double conc = (double)std::max<int64_t>(1, device_cus() / 8);
  const double best = std::sqrt(conc * bn / (4.0 * bm));
  int a = 1;
  while (a * 2 <= tiles_m && a * 2 <= best * 1.41421356) a *= 2;
  return a;
}

template <int MODE, int ST, int BM, int BN, int WGM, int WGN, int MS, bool SEQ, bool ACT, bool PP>
void launch_big_act(const GemmProblem& p, int splits) {
  using C = BigTile<MODE, BM, BN, WGM, WGN, MS>;
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
  a.tiles_m = (int)((p.rows + BM - 1) / BM);
  a.tiles_n = (int)((p.N + BN - 1) / BN);
  const int tiles = a.tiles_m * a.tiles_n;
  a.swizzled_tiles = tiles & ~7;
  a.group_m = raster_group_m(a.tiles_m, BM, BN);
  a.grp_shift = __builtin_ctzll(p.group / kBK);
  a.rowfac = p.xrowfac;
  a.lo_off = (uint32_t)(p.rows * p.K * 2);
  const int total_stages = (int)(p.K / kBK);
  // Partials are addressed through a 32-bit buffer range.
  while (splits > 1 && (int64_t)splits * p.rows * p.N * 4 >= (1ll << 32)) --splits;
  a.stages_per_split = (total_stages + splits - 1) / splits;
  a.splits = (total_stages + a.stages_per_split - 1) / a.stages_per_split;  // no empty split
  if (a.splits > 1) {
    a.counters = static_cast<uint32_t*>(
        ws_get(p, (size_t)tiles * kTileCtrStride * sizeof(uint32_t), kWsCounters));
    a.partial = static_cast<float*>(
        ws_get(p, (size_t)a.splits * p.rows * p.N * sizeof(float), kWsPartials));
  }
  ensure_dyn_smem((const void*)gemm_big_kernel<MODE, ST, BM, BN, WGM, WGN, MS, SEQ, ACT, PP>, (int)C::kSmem,
                  "hipFuncSetAttribute(gemm_big)");
  hipLaunchKernelGGL((gemm_big_kernel<MODE, ST, BM, BN, WGM, WGN, MS, SEQ, ACT, PP>), dim3(tiles, a.splits),
                     dim3(C::kThreads), C::kSmem, p.stream, a);
  check_hip(hipGetLastError(), "gemm kernel launch");
}

// The SiLU epilogue exists for the AutoAWQ order only (awq_gemm_silu_mul).
template <int MODE, int ST, int BM, int BN, int WGM, int WGN, int MS, bool SEQ, bool PP = false>
void launch_big(const GemmProblem& p, int splits) {
  if constexpr (!SEQ) {
    if (p.act) return launch_big_act<MODE, ST, BM, BN, WGM, WGN, MS, SEQ, true, PP>(p, splits);
  }
  launch_big_act<MODE, ST, BM, BN, WGM, WGN, MS, SEQ, false, PP>(p, splits);
}

template <int MODE, int ST, int BM, int BN, int WGM, int WGN, bool SEQ, bool ACT>
void launch_cfg_act(const GemmProblem& p) {
  using C = Tile<MODE, BM, BN, WGM, WGN>;
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
  a.tiles_m = (int)((p.rows + BM - 1) / BM);
  a.tiles_n = (int)((p.N + BN - 1) / BN);
  const int tiles = a.tiles_m * a.tiles_n;
  a.swizzled_tiles = tiles & ~7;
  a.splits = 1;
  const size_t smem = C::kSmem;
  ensure_dyn_smem((const void*)gemm_kernel<MODE, ST, BM, BN, WGM, WGN, SEQ, ACT>, (int)smem,
                  "hipFuncSetAttribute(gemm)");
  hipLaunchKernelGGL((gemm_kernel<MODE, ST, BM, BN, WGM, WGN, SEQ, ACT>), dim3(tiles), dim3(C::kThreads),
                     smem, p.stream, a);
  check_hip(hipGetLastError(), "gemm kernel launch");
}

template <int MODE, int ST, int BM, int BN, int WGM, int WGN, bool SEQ>
void launch_cfg(const GemmProblem& p) {
  if constexpr (!SEQ) {
    if (p.act) return launch_cfg_act<MODE, ST, BM, BN, WGM, WGN, SEQ, true>(p);
  }
  launch_cfg_act<MODE, ST, BM, BN, WGM, WGN, SEQ, false>(p);
}


// Tile choice. f16/bf16 problems with K % 64 == 0 and group = 64 * 2^j use the
// large-tile kernel with the largest tile that still yields a full wave of
// workgroups; anything else (fp32, K % 64 != 0, tiny problems) the generic
// 128x128 kernel.
template <int MODE, int ST, bool SEQ>
void launch_mode(const GemmProblem& p) {
  int cfg = tuning(kTuneGemmTile, 0);  // tuning override: 1 generic, 2.. large tiles
  const int64_t gs = p.group / kBK;
  const bool big_ok = MODE != MODE_F32 && p.K % kBK == 0 && p.group % kBK == 0 && (gs & (gs - 1)) == 0 &&
                      p.rows * p.K * 2 < (1ll << 32) && p.K * (p.N / 8) * 4 < (1ll << 32) &&
                      (p.K / p.group) * p.N * 4 < (1ll << 32);
  if (!big_ok) cfg = 1;
  auto tiles = [&](int bm, int bn) { return ((p.rows + bm - 1) / bm) * ((p.N + bn - 1) / bn); };
  int splits = 1;
  if (cfg == 0) {
    // Whole waves of workgroups over the CUs matter at these sizes. A wave
    // of 256 x 224 tiles (16x16 MFMA blocks, ping-pong schedule) costs about
    // 0.85 of a wave of 256 x 256 tiles (measured 211 against 250 us per
    // wave at 4096 x 8192 -> 28672), so they are taken when 0.85 x their
    // waves is below the 256 x 256 waves: e.g. 2048 x 14336 = 2 waves of
    // either, 4096 x 28672 8 against 7; not 4096 x 8192 (3 against 2).
    auto waves = [&](int64_t t) {
      const int64_t cus = device_cus();
      return (double)((t + cus - 1) / cus);
    };
    if (tiles(256, 224) >= 240 && 0.85 * waves(tiles(256, 224)) < waves(tiles(256, 256))) cfg = 10;
    else if (tiles(256, 256) >= 240) cfg = 2;
    // 128 x 256 tiles run 16x16x32 MFMA blocks (12): against 32x32x16 (3)
    // 2048 x 4096 -> 4096 82.5 -> 78.4 us, 2048 x 14336 -> 4096 265 -> 254 us,
    // 0-4 % faster on 11 of 12 split-K shapes at M = 129..1024 (the 12th,
    // 768 x 4096 -> 6144, 1.3 % slower); a ping-pong 128 x 256 (11) was not
    // faster than 3.
    else if (tiles(128, 256) >= 200) cfg = 12;
    else {
      cfg = 4;  // 128 x 128 tiles, two workgroups per CU
      const int64_t t = tiles(128, 128);
      const int64_t stages = p.K / kBK;
      // Fewer tiles than CUs: double the K splits while the workgroups still
      // fit one per CU (at most 8, at least 4 stages each); odd split counts
      // and more than one workgroup per CU measured slower.
      auto pow2_splits = [&](int64_t tl) {
        int sp = 1;
        while (sp < 8 && tl * sp * 2 <= device_cus() && stages / (sp * 2) >= 4) sp *= 2;
        return sp;
      };
      if (p.rows <= 128) {
        // Skinny problems: split K across workgroups until ~320 are in
        // flight (at most 8 splits, at least 4 stages each).
        splits = (int)std::min<int64_t>({(320 + t - 1) / t, 8, std::max<int64_t>(stages / 4, 1)});
      } else {
        // 128 x 128 or 128 x 256 tiles, each with its split count. Time in
        // units of one 128 x 128 x K tile: waves of workgroups over the CUs
        // times the work of one (1/splits, or 2/splits for the wider tile).
        // The wider tiles when that is no longer and they either need at most
        // 4 splits or give each split >= 16 stages (8 splits of short K lose
        // to the last workgroup's sum of 8 partial tiles). Measured at
        // M = 129..768, K 4096..28672, N 1024..14336: e.g. 14336 -> 4096 at
        // M = 256 175 -> 62 us, 28672 -> 8192 at M = 256 218 -> 180 us.
        // On equal time the wider tile wins if it needs no more K splits; if
        // it needs more, only with enough stages per split to amortise the
        // extra partial tile its last workgroup sums: >= 24, or >= 48 when
        // the narrower tile needs no split at all. Measured (narrower wins):
        // 1024 x 8192 -> 1024 42.1 -> 39.3 us, 1024 x 4096 -> 4096 59.5 ->
        // 56.9, 512 x 4096 -> 4096 42.1 -> 41.1, 256 x 4096 -> 14336 59.4 ->
        // 57.1, 768 x 4096 -> 4096 54.2 -> 52.2; (wider wins) 256 x 14336 ->
        // 4096 (28 stages per split) 54.2 against 56.4, 512 x 28672 -> 8192
        // (224) 278 against 346, 384 x 4096 -> 14336 (one split either way)
        // 72.5 against 100.5.
        splits = pow2_splits(t);
        const int64_t t3 = tiles(128, 256);
        const int s3 = pow2_splits(t3);
        const int64_t cus = device_cus();
        const int64_t waves4 = (t * splits + cus - 1) / cus, waves3 = (t3 * s3 + cus - 1) / cus;
        const bool wider = 2 * waves3 * splits < waves4 * s3 ||
                           (2 * waves3 * splits == waves4 * s3 &&
                            (s3 <= splits || stages / s3 >= (splits > 1 ? 24 : 48)));
        if (wider && (s3 <= 4 || stages / s3 >= 16)) {
          cfg = 12;
          splits = s3;
        }
      }
    }
    // 257..1024 rows with too few 256-row tiles for the first two rules: a
    // cost model fitted to a sweep of M 384..1024, K 4096..28672, N
    // 4096..28672 (tiles 256x224, 256x256, 128x256; 1 or 2 K splits). Time =
    // waves of workgroups (one per CU) x stages per split x per-stage time
    // (1.9 / 2.1 / 1.2 us), plus for K splits the partials' round trip
    // (splits x M x N x 8 bytes at 4 TB/s, + 10 us). The 256-row tiles
    // replace the choice above only when the model puts them 10 % ahead of
    // the best 128 x 256 option: e.g. 4096 -> 14336 at M = 768 169 -> 136 us,
    // 28672 -> 8192 at M = 768 516 -> 451 us; no swept point got slower.
    if (p.rows > 256 && p.rows <= 1024 && p.N >= 4096 && tiles(256, 224) < 240) {
      const int64_t cus = device_cus();
      const int64_t stages = p.K / kBK;
      auto est = [&](int bm, int bn, int sp, double per_stage) {
        const int64_t waves = (tiles(bm, bn) * sp + cus - 1) / cus;
        const int64_t st = (stages + sp - 1) / sp;
        const double partials = sp > 1 ? (double)sp * (double)p.rows * (double)p.N * 8.0 / 4e6 + 10.0 : 0.0;
        return (double)(waves * st) * per_stage + partials;
      };
      struct Cand { int cfg, sp; double t; };
      const Cand big[4] = {{10, 1, est(256, 224, 1, 1.9)}, {10, 2, est(256, 224, 2, 1.9)},
                           {2, 1, est(256, 256, 1, 2.1)}, {2, 2, est(256, 256, 2, 2.1)}};
      Cand b = big[0];
      for (const Cand& c : big)
        if (c.t < b.t) b = c;
      const double mid = std::min(est(128, 256, 1, 1.2), est(128, 256, 2, 1.2));
      if (b.t < 0.9 * mid) {
        cfg = b.cfg;
        splits = b.sp;
      }
    }
  }
  if (int v = tuning(kTuneGemmSplits, 0); v >= 1) splits = v;
  if constexpr (MODE == MODE_F32S) {
    // X tiles hold hi and lo rows, so 256-row tiles do not fit the LDS: the
    // 128 x 256 tile (8 waves) where a 256-row or wide tile was chosen,
    // else 128 x 128 (4 waves), with the split count chosen above.
    if (cfg == 3 || cfg == 2 || cfg == 6 || cfg == 7 || cfg == 8 || cfg == 9 || cfg == 10 || cfg == 11 ||
        cfg == 12)
      return launch_big<MODE, ST, 128, 256, 2, 4, 32, SEQ>(p, splits);
    return launch_big<MODE, ST, 128, 128, 2, 2, 32, SEQ>(p, splits);
  } else if constexpr (MODE != MODE_F32) {
    switch (cfg) {
      case 2: return launch_big<MODE, ST, 256, 256, 2, 4, 32, SEQ>(p, splits);
      case 3: return launch_big<MODE, ST, 128, 256, 2, 4, 32, SEQ>(p, splits);
      case 4: return launch_big<MODE, ST, 128, 128, 2, 2, 32, SEQ>(p, splits);
      case 6: return launch_big<MODE, ST, 256, 128, 4, 2, 32, SEQ>(p, splits);
      case 7: return launch_big<MODE, ST, 256, 256, 2, 2, 32, SEQ>(p, splits);
      case 8: return launch_big<MODE, ST, 64, 256, 1, 8, 32, SEQ>(p, splits);
      case 9: return launch_big<MODE, ST, 256, 224, 4, 2, 16, SEQ>(p, splits);  // single-phase
      case 10: return launch_big<MODE, ST, 256, 224, 4, 2, 16, SEQ, true>(p, splits);  // ping-pong
      case 11: return launch_big<MODE, ST, 128, 256, 2, 4, 16, SEQ, true>(p, splits);  // ping-pong
      case 12: return launch_big<MODE, ST, 128, 256, 2, 4, 16, SEQ>(p, splits);  // single-phase
      default: break;
    }
  }
  if constexpr (MODE != MODE_F32S) launch_cfg<MODE, ST, 128, 128, 2, 2, SEQ>(p);
}

template <int MODE>
void launch_st(const GemmProblem& p) {
  if (p.order == AWQ_ORDER_SEQUENTIAL) {
    // Sequential order (AWQLinear): scales in the activations' dtype, as the
    // reference's single float type F has them.
    constexpr int kST = MODE == MODE_F16 ? AWQ_F16 : MODE == MODE_BF16 ? AWQ_BF16 : AWQ_F32;
    AWQ_ASSERT(p.st == kST, "sequential-order GEMM needs scales in the input dtype");
    launch_mode<MODE, kST, true>(p);
    return;
  }
  switch (p.st) {
    case AWQ_F32: launch_mode<MODE, AWQ_F32, false>(p); break;
    case AWQ_F16: launch_mode<MODE, AWQ_F16, false>(p); break;
    default: launch_mode<MODE, AWQ_BF16, false>(p); break;
  }
}

}  // namespace

void launch_gemm(const GemmProblem& p) {
  AWQ_ASSERT(p.rows < (1ll << 31) && p.K < (1ll << 31) && p.N < (1ll << 31) &&
                 p.rows * p.K < (1ll << 40) && p.K * (p.N / 8) < (1ll << 31),
             "prefill GEMM: tensor too large");
  const int64_t tiles = ((p.rows + 127) / 128) * ((p.N + 127) / 128);
  AWQ_ASSERT(tiles < (1ll << 31), "prefill GEMM: too many tiles");
  // fp32 activations, 17 or more rows: 16-row slices, each one launch of the
  // decode kernels' 16-row matrix-core tile (x split as hi + lo in f16 with a
  // per-row power-of-two scale, exact q - z operands: fp32-level accuracy),
  // in order on the stream, where that beats the 128 x 128 fp32-MFMA kernel.
  // That kernel runs about 6.1 us per 64-row stage of K per wave of tiles
  // over the CUs (no K split), so with few tiles it is slow however few rows
  // there are: 4096 -> 14336 at M = 17 373 us, 14336 -> 4096 1287 us. A slice
  // costs about 12 us + its weight bytes at 2.4 TB/s. Slices for <= 256 rows
  // (faster at every measured shape) and up to 1024 when that estimate is
  // lower (measured 10-35 % faster up to 1024 rows at 4096 -> 14336 and
  // 8192 -> 28672, up to 768 at 14336 -> 4096; slower past 256 at
  // 4096 -> 4096, where the fp32 kernel's time stays flat).
  const int f32_slices = tuning(kTuneF32Slices, 1);  // 0: never, 2: at any row count
  auto slices_win = [&]() {
    if (p.rows <= 256 || f32_slices == 2) return true;
    if (p.rows > 1024) return false;
    const int64_t cus = device_cus();
    const double generic = (double)((tiles + cus - 1) / cus) * (double)(p.K / 64) * 6.1;
    const double slice = 12.0 + (double)p.K * (double)p.N / 2.0 / 2.4e6;
    return (double)((p.rows + 15) / 16) * slice < generic;
  };
  // fp32 activations on the f16 matrix cores (MODE_F32S), where the
  // large-tile kernel takes the shape, from 33 rows: at 17..32 two 16-row
  // slices are faster (4096 -> 14336: 32 against 74 us at M = 17; 79 us
  // against 95 for four slices at M = 64, 522 us at M = 2048 against
  // ~2.4 ms on the fp32-MFMA kernel). AWQ_F32_SLICES=2 forces slices.
  const int64_t gsz = p.group / kBK;
  const bool f32s_ok = p.xt == AWQ_F32 && p.rows > 32 && p.K % kBK == 0 && p.group % kBK == 0 &&
                       (gsz & (gsz - 1)) == 0 && p.rows * p.K * 4 < (1ll << 32) &&
                       p.K * (p.N / 8) * 4 < (1ll << 32) && (p.K / p.group) * p.N * 4 < (1ll << 32) &&
                       f32_slices != 2 && tuning(kTuneGemmTile, 0) != 1;
  if (f32s_ok) {
    const size_t split_bytes = (size_t)p.rows * p.K * 4;
    char* xs = static_cast<char*>(ws_get(p, split_bytes + (size_t)p.rows * 4, kWsXSplit));
    GemmProblem q = p;
    q.x = xs;
    q.xrowfac = reinterpret_cast<const float*>(xs + split_bytes);
    hipLaunchKernelGGL(x_split_kernel, dim3((unsigned)p.rows), dim3(256), 0, p.stream,
                       static_cast<const float*>(p.x), reinterpret_cast<f16_t*>(xs),
                       reinterpret_cast<f16_t*>(xs + split_bytes / 2), reinterpret_cast<float*>(xs + split_bytes),
                       (int)p.K);
    check_hip(hipGetLastError(), "x split kernel launch");
    if (p.order == AWQ_ORDER_SEQUENTIAL) {
      AWQ_ASSERT(p.st == AWQ_F32, "sequential-order GEMM needs scales in the input dtype");
      return launch_mode<MODE_F32S, AWQ_F32, true>(q);
    }
    switch (p.st) {
      case AWQ_F32: return launch_mode<MODE_F32S, AWQ_F32, false>(q);
      case AWQ_F16: return launch_mode<MODE_F32S, AWQ_F16, false>(q);
      default: return launch_mode<MODE_F32S, AWQ_BF16, false>(q);
    }
  }
  if (p.xt == AWQ_F32 && p.rows > 16 && p.group % 32 == 0 && p.K % 32 == 0 && f32_slices != 0 &&
      slices_win()) {
    const int64_t y_row = (p.act ? p.N / 2 : p.N) * dtype_size(p.yt);
    for (int64_t r0 = 0; r0 < p.rows; r0 += 16) {
      GemmProblem q = p;
      q.rows = std::min<int64_t>(16, p.rows - r0);
      q.x = static_cast<const char*>(p.x) + r0 * p.K * 4;
      q.y = static_cast<char*>(p.y) + r0 * y_row;
      launch_gemv(q);
    }
    return;
  }
  if (skinny_ok(p)) return launch_skinny(p);
  switch (p.xt) {
    case AWQ_F16: launch_st<MODE_F16>(p); break;
    case AWQ_BF16: launch_st<MODE_BF16>(p); break;
    default: launch_st<MODE_F32>(p); break;
  }
}

}  // namespace cube_awq
