// awq_gemv.hip -- decode path (M <= 8, and 9..16 rows on the matrix cores) of
// the fused AWQ dequant-GEMM for gfx950: gemv_kernel (VALU, 1 row and small
// 2-row problems), gemv_m4_kernel (2..4 rows, 4x4x4 matrix-core blocks),
// gemv_mfma_kernel (5..16 rows, 16x16x32 matrix-core tile).
//
// y[m, n] = sum_k x[m, k] * (q[k, n] - z[k/g, n]) * s[k/g, n]   (AutoAWQ nibble order)
// The reference's gemm_awq_decode (src/kernel/awq_kernel_gemm.rs:445-624) runs
// one thread per (row, 16 columns) over the whole K in 64 threads per
// workgroup, 112 workgroups for N = 14336. Here the kernel is shaped for HBM
// bandwidth on 256 CUs:
//
//  * qweight is read row-contiguously: lane l of a wave owns packed word
//    chunk*64 + l (8 columns), so a wave load reads 256 contiguous bytes of a
//    row; a wave walks RPW consecutive rows of one quantisation group, which
//    makes x[m, k] wave-uniform (scalar loads, SGPR operand of the FMAs).
//    Every load a wave needs (its RPW weight words, one x value per lane for
//    the activation sum, the zero word and the 8 scales) is issued up front,
//    so a workgroup's whole share of qweight is in flight at once.
//  * Per wave segment a[m, n] = sum_k x[m, k] * (q[k, n] - z[g, n]) is
//    accumulated with the exact integer q - z as the weight operand, and the
//    scale applied once: acc[m, n] += s[g, n] * a[m, n] (the reference's sum
//    of x * (q - z) * s, one FMA per weight, with no cancellation however
//    large the mean of x).
//  * Nibbles reach the FMA as f16 integers without a conversion: AutoAWQ
//    packs columns (0,1), (2,3), (4,5), (6,7) in packed lanes (0,4), (1,5),
//    (2,6), (3,7), i.e. in the low nibble of the two 16-bit halves at bit
//    offsets 0, 4, 8, 12. v_bitop3_b32 keeps one nibble per half and ORs in
//    an exponent: 0x6400 | q is the f16 1024 + q, 0x5400 | 16q is 64 + q
//    (mantissa unit 1/16). v_pk_add_f16 of the group's -(1024 + z) (or
//    -(64 + z)) leaves q - z exactly in both halves, which v_fma_mix_f32
//    widens and accumulates as x * (q - z) in f32. Per 8 weights: 1 shift +
//    4 bitop3 + 4 pk_add + 8 v_fma_mix_f32.
//  * The waves of a workgroup (stacked along K) are summed through LDS in a
//    fixed order. When K needs more than one workgroup per column chunk
//    (grid.y = splits), each writes its partial and the last to arrive sums
//    them in a fixed order (split order; with more than 8 splits, contiguous
//    split ranges per thread group, then the groups in order:
//    grouped_split_sum; on the matrix-core kernels with deep K over few
//    chunks, two levels: groups of about sqrt(splits) splits summed by their
//    last workgroup, then the groups, finish_chunk); arrival counters sit on
//    separate 256-byte lines so chunks do not serialise on one line.
//
// Algorithmic HBM bytes per call: K*N/2 (qweight) + (K/g)*(N/8)*4 (qzeros) +
// (K/g)*N*sizeof(scale) + M*K*sizeof(x) + M*N*sizeof(y).
#include <cstdlib>
#include <type_traits>

#include "awq_common.h"

namespace cube_awq {
namespace {

struct GemvArgs {
  const void* x;
  const uint32_t* qweight;
  const uint32_t* qzeros;
  const void* scales;
  const void* bias;
  void* y;
  float* partial;     // [splits (+ ngroups)][MT][N] when splits > 1
  uint32_t* counters; // per chunk (ngroups + 1 with the tree), kCounterStride apart, zero between calls
  int32_t st, bt, yt;
  int32_t rows;       // valid rows (<= MT)
  int32_t K, N, group;
  int32_t splits;
  int32_t seq;        // sequential nibble order (packed lane j = column j)
  int32_t gsize;      // two-level split sum: splits per group (finish_chunk, when ngroups > 1)
  int32_t ngroups;    // groups of gsize splits; 0 or 1: one level
};

template <int XT>
__device__ __forceinline__ float load_x(const void* x, int64_t i) {
  using X = typename Elem<XT>::type;
  return to_f32(static_cast<const X*>(x)[i]);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Raw bytes of the 8 scales of one packed word: 32 bytes for f32 scales, 16
// for f16/bf16 (the second load then repeats the first). Issued without any
// dtype branch so no wait is placed before the weight stream.
struct RawScales {
  u32x4_t lo, hi;
};
__device__ __forceinline__ RawScales load_scales_raw(const void* scales, int32_t st, int64_t off) {
  const int es = st == AWQ_F32 ? 4 : 2;
  const char* p = static_cast<const char*>(scales) + off * es;
  RawScales r;
  r.lo = *reinterpret_cast<const u32x4_t*>(p);
  r.hi = *reinterpret_cast<const u32x4_t*>(p + (es == 4 ? 16 : 0));
  return r;
}
// Convert once the weights are consumed: column order, as floats. All three
// interpretations are formed and one selected, so no branch (and no early
// wait on the loads) is introduced.
__device__ __forceinline__ void scales_to_f32(const RawScales& r, int32_t st, float (&sc)[8]) {
  const bool is32 = st == AWQ_F32, is16 = st == AWQ_F16;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t word = r.lo[j >> 1];
    const uint32_t half = (j & 1) ? (word >> 16) : (word & 0xFFFFu);
    const float v32 = __builtin_bit_cast(float, (j < 4) ? r.lo[j] : r.hi[j - 4]);
    const float v16 = (float)__builtin_bit_cast(f16_t, (uint16_t)half);
    const float vb16 = __builtin_bit_cast(float, half << 16);
    sc[j] = is32 ? v32 : (is16 ? v16 : vb16);
  }
}

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// The 4 magic views of a packed word: element j holds the two packed lanes
// of accumulator slots (2j, 2j+1) as f16 1024 + q (j = 0, 2: low nibble of
// each half) or 64 + q (j = 1, 3: high nibble, mantissa unit 1/16).
__device__ __forceinline__ void magic_word(uint32_t w, uint32_t (&mk)[4]) {
  const uint32_t w8 = w >> 8;
  mk[0] = __builtin_amdgcn_bitop3_b32(w, 0x000F000Fu, 0x64006400u, 0xEA);   // (w & m) | e
  mk[1] = __builtin_amdgcn_bitop3_b32(w, 0x00F000F0u, 0x54005400u, 0xEA);
  mk[2] = __builtin_amdgcn_bitop3_b32(w8, 0x000F000Fu, 0x64006400u, 0xEA);
  mk[3] = __builtin_amdgcn_bitop3_b32(w8, 0x00F000F0u, 0x54005400u, 0xEA);
}

// The negated magic views of a zero word: -(1024 + z) / -(64 + z) per half.
__device__ __forceinline__ void neg_magic_zero(uint32_t zw, h2_t (&nz)[4]) {
  uint32_t mk[4];
  magic_word(zw, mk);
#pragma unroll
  for (int j = 0; j < 4; ++j) nz[j] = __builtin_bit_cast(h2_t, mk[j] ^ 0x80008000u);
}

// Exact q - z of the 8 slots of a word, as 4 f16 pairs (v_pk_add_f16: both
// operands are integers below 2048 of one binade, so the sum is exact).
__device__ __forceinline__ void qz_word(uint32_t w, const h2_t (&nz)[4], h2_t (&d)[4]) {
  uint32_t mk[4];
  magic_word(w, mk);
#pragma unroll
  for (int j = 0; j < 4; ++j) d[j] = __builtin_bit_cast(h2_t, mk[j]) + nz[j];
}

// acc[c] += x * (q - z) of slot c for the 8 slots of one word.
__device__ __forceinline__ void fma_word(float (&acc)[8], float x, const h2_t (&d)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc[2 * j] = fmaf(x, (float)d[j][0], acc[2 * j]);          // v_fma_mix_f32, low half
    acc[2 * j + 1] = fmaf(x, (float)d[j][1], acc[2 * j + 1]);  // v_fma_mix_f32, high half
  }
}



constexpr int kCounterStride = 64;  // u32 words between arrival counters (256 B)

// Partial planes of the split-K workspace: one per split, plus one per group
// with the two-level sum.
__device__ __forceinline__ int partial_planes(const GemvArgs& a) {
  return a.splits + (a.ngroups > 1 ? a.ngroups : 0);
}

// Split-K sums with more splits than a single batch of loads: the last
// workgroup of a chunk sums the partials of its kQ 4-column pieces with kG
// thread groups (threads kG * kQ of the workgroup; piece q = tid % kQ, group
// h = tid / kQ, uniform per wave since kQ is a multiple of 64). Of the np
// planes from p0 (of `planes` in the workspace), group h sums [h per,
// (h + 1) per) in order with all of its 16-byte loads in flight; the kG
// group sums meet in lds (kG * kQ 16-byte entries) and are added in group
// order. Returns the piece's total in threads tid < kQ; every thread of the
// workgroup calls it (it holds a barrier). The partials are laid out
// [plane][MV][N] f32.
template <int MV, int kQ, int kG>
__device__ __forceinline__ f32x4_t grouped_split_sum(const GemvArgs& a, f32x4_t* lds, int rows, int col_base,
                                                     int planes, int p0, int np) {
  const int tid = threadIdx.x;
  const int q = tid % kQ, h = tid / kQ;
  const int m = q / 128, c0 = 4 * (q % 128);
  const rsrc_t pres = make_rsrc(a.partial, (uint32_t)((int64_t)planes * MV * a.N * 4));
  const uint32_t sstride = (uint32_t)((int64_t)MV * a.N * 4);
  const uint32_t off = (uint32_t)(((int64_t)min(m, rows - 1) * a.N + min(col_base + c0, a.N - 4)) * 4);
  const int per = (np + kG - 1) / kG;
  const int sb = p0 + min(h * per, np), se = min(sb + per, p0 + np);
  f32x4_t v = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto run = [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    for (int s0 = sb; s0 < se; s0 += NB) {
      f32x4_t t[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int sj = min(s0 + j, se - 1);  // clamped: stays in the group's range
        const u32x4_t w4 = __builtin_amdgcn_raw_buffer_load_b128(pres, off, (uint32_t)sj * sstride, kCachePolicySC1);
        // through plain scalars (hipcc 7.2 misreads a bit cast of a vector element)
        const uint32_t e0 = w4[0], e1 = w4[1], e2 = w4[2], e3 = w4[3];
        t[j] = f32x4_t{__uint_as_float(e0), __uint_as_float(e1), __uint_as_float(e2), __uint_as_float(e3)};
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const bool live = s0 + j < se;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += live ? t[j][e] : 0.f;
      }
    }
  };
  if (per <= 2) run(std::integral_constant<int, 2>{});
  else run(std::integral_constant<int, 4>{});
  lds[tid] = v;
  __syncthreads();
  f32x4_t r = v;
  if (tid < kQ) {
    r = lds[tid];
#pragma unroll
    for (int g = 1; g < kG; ++g) {
      const f32x4_t r4 = lds[g * kQ + tid];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] += r4[e];
    }
  }
  return r;
}

// Bias, then the store of 4 consecutive columns n0 .. n0 + 3 of row m (one
// vector store for f32 and f16 outputs; with ACT the 2 SiLU outputs of the
// gate/up pairs (n0, n0 + 1), (n0 + 2, n0 + 3)).
template <bool ACT>
__device__ __forceinline__ void store_cols4(const GemvArgs& a, int64_t m, int64_t n0, float (&v)[4]) {
  if (a.bias) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += load_f32_any(a.bias, n0 + e, a.bt);
  }
  if (ACT) {
    store_act_quad(a.y, a.yt, m, n0, a.N, v[0], v[1], v[2], v[3]);
  } else if (a.yt == AWQ_F32) {
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.y) + m * a.N + n0) = f32x4_t{v[0], v[1], v[2], v[3]};
  } else if (a.yt == AWQ_F16) {
    typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
    *reinterpret_cast<h4_t*>(static_cast<f16_t*>(a.y) + m * a.N + n0) =
        h4_t{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) store_out(a.y, a.yt, 0, m, n0 + e, a.N, v[e], 0.f);
  }
}

// ACT (all decode kernels): the gate/up SiLU epilogue, a template parameter
// so the plain kernels' code is untouched by it.
template <int XT, int MT, int WAVES, int RPW, bool ACT>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(GemvArgs a) {
  constexpr int kChunkCols = 512;  // 64 lanes x 8 columns
  __shared__ float red[WAVES][MT][kChunkCols];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  // Wave-uniform by construction; readfirstlane lets the compiler know, so the
  // K range, x addresses and group index live in SGPRs (x via scalar loads).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunk = blockIdx.x;
  const int split = blockIdx.y;
  const int np = a.N >> 3;
  const int pack = chunk * 64 + lane;
  const bool lane_ok = pack < np;
  const int pack_c = lane_ok ? pack : np - 1;  // clamped: loads stay in bounds
  const int rows = a.rows;

  // This wave's rows [k0, k0 + RPW): one run inside one quantisation group
  // (RPW divides the group size, K is a multiple of the group size), so a
  // wave's run is either entirely inside K or entirely past it.
  const int k0 = (split * WAVES + wave) * RPW;
  const bool live = k0 < a.K;
  const int kc = live ? k0 : 0;  // row base for loads (row 0 for waves past K)
  const int grp = kc / a.group;

  int64_t xrow[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) xrow[m] = (int64_t)min(m, rows - 1) * a.K + kc;

  // ---- loads, in the order they are consumed (vmcnt retires in issue order) ----
  // 1. zero word and scales of the group, 2. the RPW weight words (batches of
  // RB, the next batch requested before the current one is consumed).
  const uint32_t zw = a.qzeros[(int64_t)grp * np + pack_c];
  const RawScales sraw = load_scales_raw(a.scales, a.st, (int64_t)grp * a.N + (int64_t)pack_c * 8);
  constexpr int RB = RPW < 32 ? RPW : 32;
  constexpr int NB = RPW / RB;
  const rsrc_t wr = make_rsrc(a.qweight, (uint32_t)a.K * (uint32_t)np * 4u);
  const uint32_t voff = (uint32_t)pack_c * 4u;
  const uint32_t row_bytes = (uint32_t)np * 4u;
  uint32_t w[2][RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) w[0][r] = buf_load_u32_nt(wr, voff, (uint32_t)(kc + r) * row_bytes);

  // ---- accumulate sum_k x * (q - z) ---------------------------------------------
  h2_t nz[4];
  neg_magic_zero(zw, nz);
  float part[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 8; ++c) part[m][c] = 0.f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b + 1 < NB) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
        w[(b + 1) & 1][r] = buf_load_u32_nt(wr, voff, (uint32_t)(kc + (b + 1) * RB + r) * row_bytes);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if constexpr (MT >= 4) {
        // Many rows: widen each nibble once (v_cvt_f32_f16 of the same
        // denormal halves, half rate) and reuse it in MT full-rate FMAs,
        // instead of MT half-rate v_fma_mix_f32 per weight.
        h2_t d[4];
        qz_word(w[b & 1][r], nz, d);
        float v[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = (float)d[c >> 1][c & 1];
        // Opaque: otherwise the widening is folded back into v_fma_mix_f32.
#pragma unroll
        for (int c = 0; c < 8; ++c) asm("" : "+v"(v[c]));
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float xv = load_x<XT>(a.x, xrow[m] + b * RB + r);
#pragma unroll
          for (int c = 0; c < 8; ++c) part[m][c] = fmaf(xv, v[c], part[m][c]);
        }
      } else {
        h2_t d[4];
        qz_word(w[b & 1][r], nz, d);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          fma_word(part[m], load_x<XT>(a.x, xrow[m] + b * RB + r), d);
        }
      }
    }
  }

  // ---- apply the scale -----------------------------------------------------------
  // Accumulator slot c holds the packed lane that magic_word puts there: lane
  // kAwqLaneOfCol[c], which is column c in AutoAWQ order and column
  // seq_col(c) = (c >> 1) + 4 (c & 1) in sequential order. Zero points come
  // through the same views; scales (and, below, outputs) are per column, so in
  // sequential order they are permuted to slot order (once per wave).
  float sl[8];
  scales_to_f32(sraw, a.st, sl);
  const bool seq = a.seq != 0;
  {
    float t[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) t[c] = seq ? sl[(c >> 1) + 4 * (c & 1)] : sl[c];
#pragma unroll
    for (int c = 0; c < 8; ++c) sl[c] = t[c];
  }
  float acc[MT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    // Waves past K read row 0 and contribute nothing (uniform, once per wave).
    if (!live) {
#pragma unroll
      for (int c = 0; c < 8; ++c) part[m][c] = 0.f;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[m][c] = sl[c] * part[m][c];
  }

  // ---- sum the waves of the workgroup (fixed order) ------------------------------
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float o[8];  // column order: column j is slot j (AutoAWQ) or slot 2 (j & 3) + (j >> 2)
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = seq ? acc[m][2 * (j & 3) + (j >> 2)] : acc[m][j];
    float4* dst = reinterpret_cast<float4*>(&red[wave][m][lane * 8]);
    dst[0] = make_float4(o[0], o[1], o[2], o[3]);
    dst[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
  __syncthreads();
  constexpr int kOut = MT * kChunkCols;
  constexpr int kPer = (kOut + 64 * WAVES - 1) / (64 * WAVES);
  float res[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int o = threadIdx.x + i * 64 * WAVES;
    float v = 0.f;
    if (o < kOut) {
      const int m = o / kChunkCols, c = o % kChunkCols;
#pragma unroll
      for (int ww = 0; ww < WAVES; ++ww) v += red[ww][m][c];
    }
    res[i] = v;
  }

  const int col_base = chunk * kChunkCols;
  if (a.splits > 1) {
    // Split-K handshake (the memory-ordering argument is in awq_common.h):
    // partials written with agent-scope (write-through, sc1) stores, the wave
    // waits for their completion (vmcnt 0), and only then the workgroup's
    // arrival is counted. The last workgroup to arrive for this chunk reads
    // all partials with agent-scope (sc1) loads, sums them in a fixed order,
    // and re-arms the counter for the next call.
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int o = threadIdx.x + i * 64 * WAVES;
      const int m = o / kChunkCols, c = o % kChunkCols;
      if (o < kOut && m < rows && col_base + c < a.N)
        __hip_atomic_store(&a.partial[((int64_t)split * MT + m) * a.N + col_base + c], res[i],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Partials complete before the arrival (split-K handshake, awq_common.h).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&a.counters[chunk * kCounterStride], 1u,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (prev == (uint32_t)(a.splits - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    // The counter is re-armed after the sum: issued earlier, the agent-scope
    // store would sit ahead of the sum's loads in wave 0's in-order vmcnt.
    auto rearm = [&]() {
      if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[chunk * kCounterStride], 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    };
    // More than 8 splits (deep K): 4-column pieces, the splits shared by
    // thread groups (grouped_split_sum), one round of loads instead of one
    // per 8 splits (14336 -> 4096 at one row: 28 splits).
    constexpr int kQ = MT * kChunkCols / 4;
    if constexpr (kQ < 64 * WAVES) {
      if (a.splits > 8) {
        // The slots are free: every thread read its slots before the arrival barrier.
        const f32x4_t r = grouped_split_sum<MT, kQ, 64 * WAVES / kQ>(
            a, reinterpret_cast<f32x4_t*>(&red[0][0][0]), rows, col_base, a.splits, 0, a.splits);
        rearm();
        const int q = threadIdx.x;
        const int m = q / (kChunkCols / 4), n0 = col_base + 4 * (q % (kChunkCols / 4));
        if (q < kQ && m < rows && n0 < a.N) {
          float v[4] = {r[0], r[1], r[2], r[3]};
          store_cols4<ACT>(a, m, n0, v);
        }
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int o = threadIdx.x + i * 64 * WAVES;
      const int m = o / kChunkCols, c = o % kChunkCols;
      if (o < kOut && m < rows && col_base + c < a.N) {
        const float* src = a.partial + (int64_t)m * a.N + col_base + c;
        const int64_t stride = (int64_t)MT * a.N;
        float v = 0.f;
        int s = 0;
        for (; s + 8 <= a.splits; s += 8) {  // 8 loads in flight, summed in split order
          float t[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            t[j] = __hip_atomic_load(src + (s + j) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
          for (int j = 0; j < 8; ++j) v += t[j];
        }
        for (; s < a.splits; ++s)
          v += __hip_atomic_load(src + s * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        res[i] = v;
      }
    }
    rearm();
  }

  // Adjacent threads hold adjacent columns, so a gate/up pair is this lane
  // and its xor-1 neighbour.
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int o = threadIdx.x + i * 64 * WAVES;
    const int m = o / kChunkCols, c = o % kChunkCols;
    const int n = col_base + c;
    float v = res[i];
    if (a.bias && n < a.N) v += load_f32_any(a.bias, n, a.bt);
    const float pv = ACT ? __shfl_xor(v, 1, 64) : 0.f;
    if (o < kOut && m < rows && n < a.N) store_out(a.y, a.yt, ACT, m, n, a.N, v, pv);
  }
}

// ---------------------------------------------------------------------------
// Small-M path on the matrix cores (2 <= rows <= 16 per launch).
//
// The VALU path above spends one FMA per weight per activation row, so its
// cost grows with M. Here the weights feed v_mfma_f32_16x16x32_f16 as exact
// f16 integers q - z (|q - z| <= 15) and each group's partial sums are scaled
// once, so the arithmetic per weight is the same for every M <= 16:
//   acc[m, n] = sum_k x[m, k] * (q[k, n] - z[n]);  y[m, n] += s[n] * acc[m, n]
// Activations that are not f16 are first scaled, per activation row and
// wave, by the power of two that puts the row's largest |x| in [2^14, 2^15)
// (exact; undone when the scale s is applied), then split as x = hi + lo with
// hi = f16(x), lo = f16(x - hi): |x - hi - lo| <= 2^-22 max|x|, and no f16
// overflow or denormal loss whatever the magnitude of x. Both halves run
// through the MFMA; products of f16 values with 4-bit integers are exact in
// the fp32 accumulators, so the result keeps fp32 accuracy. (Non-finite
// activations give non-finite outputs, NaN where an fp32 sum might give inf.)
//
// Weights are read exactly as in the VALU path (lane l owns packed word
// chunk*64 + l, one 256-byte row segment per load), then a 4x4 transpose of
// 16-lane groups (v_permlane32_swap, v_permlane16_swap) gives lane group b
// rows 8b..8b+7 of 16 packs: the B operand layout of the 16x16x32 MFMA
// (lane l supplies 8 consecutive k of column l % 16). Reading the weights in
// that layout directly (4 rows x 64 bytes per load) measured 30 % slower.
// One 32-row step of a wave: 32 transposes, 4 x 8 MFMA operands (packed lane
// c of 16 packs, 1.5 VALU ops per weight: v_perm_b32, v_bitop3_b32, exact
// v_pk_add_f16 of -(1024 + z)), 32 MFMAs (64 with the low half of x).
// Waves of a workgroup are summed through LDS in a fixed order, K splits
// through the workspace exactly as in the VALU path.
// ---------------------------------------------------------------------------
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef h2_t f16x2;

__device__ __forceinline__ void tr4(uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
  // In: r_b's 16-lane group a holds block (a, b). Out: r_a's group b holds it.
  auto s02 = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
  auto s13 = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
  auto t01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  auto t23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  r0 = t01[0];
  r1 = t01[1];
  r2 = t23[0];
  r3 = t23[1];
}

template <int XT>
__device__ __forceinline__ void load_x8(const void* x, int64_t i, float (&v)[8]) {
  if constexpr (XT == AWQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + i);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    using X = typename Elem<XT>::type;
    const u32x4_t r = *reinterpret_cast<const u32x4_t*>(static_cast<const X*>(x) + i);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t h = (uint16_t)(r[e >> 1] >> (16 * (e & 1)));
      v[e] = to_f32(__builtin_bit_cast(X, h));
    }
  }
}

// Sum a workgroup's slot-order partials over its LDS slots (fixed order),
// publish them across K splits (16-byte sc1 stores, completion wait, arrival
// count; the last workgroup of the chunk sums the splits in a fixed order:
// split order, or, with more threads than pieces, contiguous split ranges
// per thread group, then the groups in order), add the bias and store rows <
// rows of the chunk's 512 columns. red[w][m][8 p + c]
// holds packed lane c of pack p (column c in sequential order,
// kAwqColOfLane[c] in AutoAWQ order). Each thread owns pieces of 4
// consecutive slots of one row, kept in slot order until the final store
// (the split partials too): 16-byte LDS reads without bank conflicts, and
// 16-byte partial stores and loads (the vector memory path takes about 16
// clocks per wave instruction whatever its width).
template <int MV, int WAVES, int kSlots, bool ACT>
__device__ __forceinline__ void finish_chunk(const GemvArgs& a, float (*red)[MV][512], int* s_last_p, int rows,
                                             bool seq) {
  constexpr int kChunkCols = 512;
  constexpr int kQ = MV * kChunkCols / 4;  // 4-slot pieces of the chunk's outputs
  constexpr int kTh = 64 * WAVES;
  constexpr int kPer = (kQ + kTh - 1) / kTh;  // pieces per thread
  // Thread groups that share the last workgroup's sum over the K splits when
  // the workgroup has more threads than pieces (grouped_split_sum).
  constexpr int kG = kQ >= kTh ? 1 : kTh / kQ;
  static_assert(kG == 1 || kSlots * kQ >= kTh, "LDS slots too small for the grouped split sum");
  const int chunk = blockIdx.x;
  const int split = blockIdx.y;
  const int tid = threadIdx.x;
  int& s_last = *s_last_p;
  const int col_base = chunk * kChunkCols;
  // piece q: row q / 128, slots 4 (q % 128) .. + 3 of the chunk
  f32x4_t res[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int q = tid + i * kTh;
    f32x4_t v = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (q < kQ) {
      const int m = q / (kChunkCols / 4), s0 = 4 * (q % (kChunkCols / 4));
#pragma unroll
      for (int ww = 0; ww < kSlots; ++ww) {
        const f32x4_t r4 = *reinterpret_cast<const f32x4_t*>(&red[ww][m][s0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += r4[e];
      }
    }
    res[i] = v;
  }

  if (a.splits > 1) {
    // Same handshake as the VALU path, with sc1 buffer stores and loads
    // (split-K handshake, awq_common.h). One level: the last workgroup of
    // the chunk sums the splits in order. Two levels (ngroups > 1, deep K):
    // the splits form groups of gsize; the last workgroup of a group sums
    // the group's splits in order and publishes that sum as plane splits +
    // group through the same handshake, and the last group sums the group
    // planes in order. Both orders are fixed, so results stay deterministic;
    // the last workgroup's serial sum (bound by one CU's loads) shrinks from
    // splits planes to about 2 sqrt(splits).
    const bool tree = a.ngroups > 1;
    const int cpc = tree ? a.ngroups + 1 : 1;  // counters per chunk
    const rsrc_t pres = make_rsrc(a.partial, (uint32_t)((int64_t)partial_planes(a) * MV * a.N * 4));
    const uint32_t sstride = (uint32_t)((int64_t)MV * a.N * 4);
    auto store_plane = [&](int plane) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int q = tid + i * kTh;
        const int m = q / (kChunkCols / 4), c0 = 4 * (q % (kChunkCols / 4));
        if (q < kQ && m < rows && col_base + c0 < a.N) {
          const float f0 = res[i][0], f1 = res[i][1], f2 = res[i][2], f3 = res[i][3];
          const u32x4_t w4 =
              u32x4_t{__float_as_uint(f0), __float_as_uint(f1), __float_as_uint(f2), __float_as_uint(f3)};
          __builtin_amdgcn_raw_buffer_store_b128(w4, pres, (uint32_t)(((int64_t)m * a.N + col_base + c0) * 4),
                                                 (uint32_t)plane * sstride, kCachePolicySC1);
        }
      }
    };
    // Publish the stored plane and count the arrival on counter ci of this
    // chunk; true in the last of `expect` arrivals.
    auto arrive = [&](int ci, int expect) -> bool {
      // Partials complete before the arrival (split-K handshake, awq_common.h).
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      uint32_t* ctr = &a.counters[(chunk * cpc + ci) * kCounterStride];
      if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (uint32_t)(expect - 1)) ? 1 : 0;
      }
      __syncthreads();
      return s_last != 0;
    };
    // Re-arm counter ci for the next call, after the sum (issued earlier, the
    // agent-scope store would sit ahead of the sum's loads in wave 0's
    // in-order vmcnt).
    auto rearm = [&](int ci) {
      if (tid == 0)
        __hip_atomic_store(&a.counters[(chunk * cpc + ci) * kCounterStride], 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    };
    // res = the sum of planes p0 .. p0 + np - 1, in order.
    auto sum_planes = [&](int p0, int np) {
      bool grouped = false;
      if constexpr (kG > 1) grouped = np > 8;
      if (grouped) {
        // More threads than pieces and more than 8 planes: one round of
        // loads shared by kG thread groups (the slots are free: every thread
        // read its slots before the first arrival barrier).
        if constexpr (kG > 1)
          res[0] = grouped_split_sum<MV, kQ, kG>(a, reinterpret_cast<f32x4_t*>(&red[0][0][0]), rows, col_base,
                                                 partial_planes(a), p0, np);
      } else {
        // Each thread's kPer pieces, kSB planes at a time: kPer * kSB loads
        // in flight; every output still sums its planes in order.
        constexpr int kSB = kPer >= 4 ? 4 : 8;
        uint32_t off[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          const int q = min(tid + i * kTh, kQ - 1);
          const int m = q / (kChunkCols / 4), c0 = 4 * (q % (kChunkCols / 4));
          // Rows past M read row M-1's partials (cached, discarded): unconditional
          // loads keep the batch in flight.
          off[i] = (uint32_t)(((int64_t)min(m, rows - 1) * a.N + min(col_base + c0, a.N - 4)) * 4);
          res[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        for (int s0 = 0; s0 < np; s0 += kSB) {
          f32x4_t t[kPer][kSB];
#pragma unroll
          for (int i = 0; i < kPer; ++i)
#pragma unroll
            for (int j = 0; j < kSB; ++j) {
              const int sj = p0 + min(s0 + j, np - 1);  // clamped: stays in the range
              const u32x4_t w4 = __builtin_amdgcn_raw_buffer_load_b128(pres, off[i], (uint32_t)sj * sstride,
                                                                       kCachePolicySC1);
              // through plain scalars (hipcc 7.2 misreads a bit cast of a vector element)
              const uint32_t e0 = w4[0], e1 = w4[1], e2 = w4[2], e3 = w4[3];
              t[i][j] = f32x4_t{__uint_as_float(e0), __uint_as_float(e1), __uint_as_float(e2), __uint_as_float(e3)};
            }
#pragma unroll
          for (int i = 0; i < kPer; ++i)
#pragma unroll
            for (int j = 0; j < kSB; ++j) {
              const bool live = s0 + j < np;
#pragma unroll
              for (int e = 0; e < 4; ++e) res[i][e] += live ? t[i][j][e] : 0.f;
            }
        }
      }
    };
    store_plane(split);
    if (tree) {
      const int grp = split / a.gsize, gbeg = grp * a.gsize, gn = min(a.gsize, a.splits - gbeg);
      if (!arrive(grp, gn)) return;
      sum_planes(gbeg, gn);
      rearm(grp);
      store_plane(a.splits + grp);
      if (!arrive(a.ngroups, a.ngroups)) return;
      sum_planes(a.splits, a.ngroups);
      rearm(a.ngroups);
    } else {
      if (!arrive(0, a.splits)) return;
      sum_planes(0, a.splits);
      rearm(0);
    }
  }

  // Slots to columns. Sequential order: slot = column. AutoAWQ: the even
  // lane of a pack holds slots 0..3 = columns 0, 2, 4, 6 and the odd lane
  // slots 4..7 = columns 1, 3, 5, 7; one exchange leaves columns 0..3 in the
  // even lane and 4..7 in the odd one. Then each lane stores 4 consecutive
  // columns (a gate/up pair is elements 2 j, 2 j + 1).
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int q = tid + i * kTh;
    const int m = q / (kChunkCols / 4), n0 = col_base + 4 * (q % (kChunkCols / 4));
    float v[4];
    if (seq) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = res[i][e];
    } else {
      float x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = __shfl_xor(res[i][e], 1, 64);
      const bool odd = (tid & 1) != 0;
      v[0] = odd ? x[2] : res[i][0];
      v[1] = odd ? res[i][2] : x[0];
      v[2] = odd ? x[3] : res[i][1];
      v[3] = odd ? res[i][3] : x[1];
    }
    if (q >= kQ || m >= rows || n0 >= a.N) continue;
    store_cols4<ACT>(a, m, n0, v);
  }
}

template <int XT, int MV, int WAVES, int RPW, bool ACT>
__global__ __launch_bounds__(64 * WAVES) void gemv_mfma_kernel(GemvArgs a) {
  constexpr int kChunkCols = 512;
  constexpr bool kLo = XT != AWQ_F16;
  constexpr int kSteps = RPW / 32;
  static_assert(RPW == 32 || RPW == 64, "rows per wave: whole 32-row MFMA steps");
  static_assert(MV == 2 || MV == 4 || MV == 8 || MV == 16, "rows kept (the MFMA tile has 16)");
  // LDS partial slots: one per wave for 8 rows; for 16 rows (128 KB for 4
  // slots) waves w and w + 4 share slot w: the upper waves store, the lower
  // ones add after a barrier (per pack set, so the compute stays parallel).
  constexpr int kSlots = MV == 16 ? WAVES / 2 : WAVES;
  constexpr bool kTwoRounds = kSlots < WAVES;
  static_assert(WAVES == 4 || WAVES == 8, "waves per workgroup");
  __shared__ float red[kSlots][MV][kChunkCols];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunk = blockIdx.x;
  const int split = blockIdx.y;
  const int np = a.N >> 3;
  const int rows = a.rows;
  const int lg = lane >> 4, lj = lane & 15;
  const int slot = wave % kSlots;
  const int pack_c = min(chunk * 64 + lane, np - 1);  // clamped: loads stay in bounds

  const int k0 = (split * WAVES + wave) * RPW;  // one run inside one group
  const bool live = k0 < a.K;
  const int kc = live ? k0 : 0;
  const int grp = kc / a.group;

  // ---- loads: the activations, then the zero words and scales of the 4
  // packs this lane feeds (pack chunk*64 + 16 s + lj), then the wave's RPW
  // weight rows (activations first: 16 rows at 4096 -> 14336 23.9 -> 23.3 us).
  // A operand: lane (lg, lj) holds x[lj, k + 8 lg .. k + 8 lg + 7] of each step.
  const bool xrow_ok = lj < rows;
  const int64_t xbase = (int64_t)min(lj, rows - 1) * a.K + kc + 8 * lg;
  float xv[kSteps][8];
#pragma unroll
  for (int b = 0; b < kSteps; ++b) load_x8<XT>(a.x, xbase + 32 * b, xv[b]);
  uint32_t zq[4];
  RawScales sraw[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int pk = min(chunk * 64 + 16 * s + lj, np - 1);
    zq[s] = a.qzeros[(int64_t)grp * np + pk];
    sraw[s] = load_scales_raw(a.scales, a.st, (int64_t)grp * a.N + (int64_t)pk * 8);
  }
  // Issued before the weight rows (a compiler barrier: otherwise the row
  // mask below turns the activation loads into predicated loads placed
  // after the weights, and the activations' row scale waits for every row).
  asm volatile("" ::: "memory");
  const rsrc_t wr = make_rsrc(a.qweight, (uint32_t)a.K * (uint32_t)np * 4u);
  const uint32_t voff = (uint32_t)pack_c * 4u;
  const uint32_t row_bytes = (uint32_t)np * 4u;
  uint32_t w[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) w[r] = buf_load_u32_nt(wr, voff, (uint32_t)(kc + r) * row_bytes);
#pragma unroll
  for (int b = 0; b < kSteps; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[b][e] = xrow_ok ? xv[b][e] : 0.f;
  // Row scale (not for f16 activations, which are exact as they are): the
  // largest |x| of row lj over this wave's rows goes to [2^14, 2^15).
  float xdown[4] = {1.f, 1.f, 1.f, 1.f};  // undo factor of D rows 4 lg + r
  if constexpr (kLo) {
    float mx = 0.f;
#pragma unroll
    for (int b = 0; b < kSteps; ++b)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(xv[b][e]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    int ex;
    (void)frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
    const int up = min(max(15 - ex, -126), 127);
    const float fup = ldexpf(1.f, up);
#pragma unroll
    for (int b = 0; b < kSteps; ++b)
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[b][e] *= fup;
    const float down = ldexpf(1.f, -up);
    // Row 4 lg + r of the D layout is row lj = 4 lg + r of the A layout.
#pragma unroll
    for (int r = 0; r < 4; ++r) xdown[r] = __shfl(down, 4 * lg + r, 64);
  }
  f16x8_t ahi[kSteps], alo[kSteps];
#pragma unroll
  for (int b = 0; b < kSteps; ++b)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 h = (_Float16)xv[b][e];
      ahi[b][e] = h;
      alo[b][e] = (_Float16)(xv[b][e] - (float)h);
    }

  // ---- transpose of step b: w[32 b + 8 s + u] becomes, in lane group lg,
  // row 32 b + 8 lg + u of pack chunk*64 + 16 s + lj. Then per pack set s:
  // MFMAs over the wave's rows (acc[c][r] is row 4 lg + r of packed lane c
  // of pack chunk*64 + 16 s + lj; columns of a pack in order take packed
  // lane kAwqLaneOfCol[j] (AutoAWQ) or j (sequential)), scaled and written
  // to this wave's LDS slot. s is a compile-time constant in each body
  // (every register index must be static).
  const bool seq = a.seq != 0;
  auto transpose = [&](int b) {
#pragma unroll
    for (int u = 0; u < 8; ++u) tr4(w[32 * b + u], w[32 * b + 8 + u], w[32 * b + 16 + u], w[32 * b + 24 + u]);
  };
  auto mfmas = [&](auto s_const, int b, f32x4_t (&acc)[8]) {
    constexpr int s = decltype(s_const)::value;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const f16x2 fz = __builtin_bit_cast(f16x2, nib_f16x2(zq[s], zq[s], c));
      f16x8_t bq;
#pragma unroll
      for (int u = 0; u < 8; u += 2) {
        const f16x2 d = __builtin_bit_cast(f16x2, nib_f16x2(w[32 * b + 8 * s + u], w[32 * b + 8 * s + u + 1], c)) - fz;
        bq[u] = d[0];
        bq[u + 1] = d[1];
      }
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[b], bq, acc[c], 0, 0, 0);
      if constexpr (kLo) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[b], bq, acc[c], 0, 0, 0);
    }
  };
  // Scaled sums of pack set s; into this wave's slot (add: onto what it holds).
  auto store_set = [&](auto s_const, const f32x4_t (&acc)[8], bool add) {
    constexpr int s = decltype(s_const)::value;
    float sl[8], slp[8];
    scales_to_f32(sraw[s], a.st, sl);  // column order
    // Partial sums stay in packed-lane (slot) order; the scale of slot c is
    // that of its column (c in sequential order, kAwqColOfLane[c] in AutoAWQ).
#pragma unroll
    for (int c = 0; c < 8; ++c) slp[c] = seq ? sl[c] : sl[awq_col_of_lane(c)];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * lg + r;
      if (m < MV) {
        float o[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) o[c] = acc[c][r] * slp[c] * xdown[r];
        float4* d4 = reinterpret_cast<float4*>(&red[slot][m][8 * (16 * s + lj)]);
        float4 v0 = make_float4(o[0], o[1], o[2], o[3]);
        float4 v1 = make_float4(o[4], o[5], o[6], o[7]);
        if (add) {
          const float4 p0 = d4[0], p1 = d4[1];
          v0 = make_float4(v0.x + p0.x, v0.y + p0.y, v0.z + p0.z, v0.w + p0.w);
          v1 = make_float4(v1.x + p1.x, v1.y + p1.y, v1.z + p1.z, v1.w + p1.w);
        }
        d4[0] = v0;
        d4[1] = v1;
      }
    }
  };
  if (live) {
#pragma unroll
    for (int b = 0; b < kSteps; ++b) transpose(b);
  }
  // Per pack set, all steps' MFMAs, then the store. (Step by step instead,
  // step 0's MFMAs starting while step 1's rows are in flight and each
  // step's sums added into the slot, measured 5-13 % slower at 5..8 rows.)
  // 16 rows: waves w and w + 4 share slot w (the upper waves store, the
  // lower ones add after a barrier, per pack set).
  auto pack_set = [&](auto s_const) {
    f32x4_t acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (live) {
#pragma unroll
      for (int b = 0; b < kSteps; ++b) mfmas(s_const, b, acc);
    }
    if constexpr (kTwoRounds) {
      if (wave >= kSlots) store_set(s_const, acc, false);
      __syncthreads();
      if (wave < kSlots) store_set(s_const, acc, true);
    } else {
      store_set(s_const, acc, false);
    }
  };
  pack_set(std::integral_constant<int, 0>{});
  pack_set(std::integral_constant<int, 1>{});
  pack_set(std::integral_constant<int, 2>{});
  pack_set(std::integral_constant<int, 3>{});
  __syncthreads();

  finish_chunk<MV, WAVES, kSlots, ACT>(a, red, &s_last, rows, seq);
}

// ---------------------------------------------------------------------------
// 2..8 rows on 4x4x4 matrix-core blocks (v_mfma_f32_4x4x4_16b_f16), in the
// VALU path's own layout: lane l owns packed word chunk*64 + l of each of
// the wave's RPW rows, one 256-byte row segment per load, and keeps it. The
// 16 blocks of one instruction are lanes 4b .. 4b + 3: lane 4b + i supplies
// row i of A (4 consecutive k of activation row i, the same for every
// block) and column i of B (4 consecutive k of its own packed lane c, exact
// f16 integers q - z: v_perm_b32 + v_bitop3_b32 + exact v_pk_add_f16 for
// each pair of rows), and receives rows 0..3 of that column. So every lane
// accumulates its own 8 columns for 4 activation rows with no transpose and
// no padding: per 4 rows of W, 8 MFMAs per 4-row set of activations (twice
// that with the low half of non-f16 activations), 1.5 VALU ops per weight.
// Activations that are not f16 are scaled per row and wave by a power of two
// and split as hi + lo in f16 exactly as in the 16x16x32 path above; the
// scale is applied once per wave (its rows lie in one group).
// ---------------------------------------------------------------------------
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

template <int XT, int MV, int WAVES, int RPW, bool ACT>
__global__ __launch_bounds__(64 * WAVES) void gemv_m4_kernel(GemvArgs a) {
  constexpr int kChunkCols = 512;
  constexpr bool kLo = XT != AWQ_F16;
  constexpr int kSets = MV / 4;  // 4-row activation sets
  constexpr int kQ = RPW / 4;    // 4-row steps of W per wave
  static_assert(MV == 4 || MV == 8, "rows kept");
  static_assert(RPW == 16 || RPW == 32 || RPW == 64, "rows per wave");
  __shared__ float red[WAVES][MV][kChunkCols];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunk = blockIdx.x;
  const int split = blockIdx.y;
  const int np = a.N >> 3;
  const int rows = a.rows;
  const int pack_c = min(chunk * 64 + lane, np - 1);  // clamped: loads stay in bounds

  const int k0 = (split * WAVES + wave) * RPW;  // one run inside one group
  const bool live = k0 < a.K;
  const int kc = live ? k0 : 0;
  const int grp = kc / a.group;

  // ---- loads: the wave's RPW weight words, the zero word and scales of the
  // lane's pack, then activation row (lane & 3) + 4 t over the same k.
  const rsrc_t wr = make_rsrc(a.qweight, (uint32_t)a.K * (uint32_t)np * 4u);
  const uint32_t voff = (uint32_t)pack_c * 4u;
  const uint32_t row_bytes = (uint32_t)np * 4u;
  uint32_t w[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) w[r] = buf_load_u32_nt(wr, voff, (uint32_t)(kc + r) * row_bytes);
  const uint32_t zw = a.qzeros[(int64_t)grp * np + pack_c];
  const RawScales sraw = load_scales_raw(a.scales, a.st, (int64_t)grp * a.N + (int64_t)pack_c * 8);
  const int ai = lane & 3;
  float xv[kSets][RPW];
#pragma unroll
  for (int t = 0; t < kSets; ++t) {
    const int m = ai + 4 * t;
    const int64_t base = (int64_t)min(m, rows - 1) * a.K + kc;
#pragma unroll
    for (int j = 0; j < RPW; j += 8) {
      float v8[8];
      load_x8<XT>(a.x, base + j, v8);
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[t][j + e] = m < rows ? v8[e] : 0.f;
    }
  }
  // Row scale (non-f16 activations): this row's largest |x| over the wave's
  // rows to [2^14, 2^15); D row r of every block is A row r, held by lane r.
  float xdown[kSets][4];
#pragma unroll
  for (int t = 0; t < kSets; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) xdown[t][r] = 1.f;
  if constexpr (kLo) {
#pragma unroll
    for (int t = 0; t < kSets; ++t) {
      float mx = 0.f;
#pragma unroll
      for (int j = 0; j < RPW; ++j) mx = fmaxf(mx, fabsf(xv[t][j]));
      int ex;
      (void)frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
      const int up = min(max(15 - ex, -126), 127);
      const float fup = ldexpf(1.f, up);
#pragma unroll
      for (int j = 0; j < RPW; ++j) xv[t][j] *= fup;
      const float down = ldexpf(1.f, -up);
#pragma unroll
      for (int r = 0; r < 4; ++r) xdown[t][r] = __shfl(down, r, 64);
    }
  }
  f16x4_t ahi[kSets][kQ], alo[kSets][kQ];
#pragma unroll
  for (int t = 0; t < kSets; ++t)
#pragma unroll
    for (int q = 0; q < kQ; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = xv[t][4 * q + e];
        const _Float16 h = (_Float16)v;
        ahi[t][q][e] = h;
        if constexpr (kLo) alo[t][q][e] = (_Float16)(v - (float)h);
      }

  // ---- MFMAs: acc[t][c][r] = sum_k x[r + 4 t, k] * (q - z)[k, packed lane c]
  f32x4_t acc[kSets][8];
#pragma unroll
  for (int t = 0; t < kSets; ++t)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[t][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f16x2 fz[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) fz[c] = __builtin_bit_cast(f16x2, nib_f16x2(zw, zw, c));
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const f16x2 d01 = __builtin_bit_cast(f16x2, nib_f16x2(w[4 * q], w[4 * q + 1], c)) - fz[c];
      const f16x2 d23 = __builtin_bit_cast(f16x2, nib_f16x2(w[4 * q + 2], w[4 * q + 3], c)) - fz[c];
      const f16x4_t bq = f16x4_t{d01[0], d01[1], d23[0], d23[1]};
#pragma unroll
      for (int t = 0; t < kSets; ++t) {
        acc[t][c] = __builtin_amdgcn_mfma_f32_4x4x4f16(ahi[t][q], bq, acc[t][c], 0, 0, 0);
        if constexpr (kLo) acc[t][c] = __builtin_amdgcn_mfma_f32_4x4x4f16(alo[t][q], bq, acc[t][c], 0, 0, 0);
      }
    }
  }

  // ---- scale (slot c takes the scale of its column), this wave's LDS slot ----
  const bool seq = a.seq != 0;
  float sl[8], slp[8];
  scales_to_f32(sraw, a.st, sl);
#pragma unroll
  for (int c = 0; c < 8; ++c) slp[c] = seq ? sl[c] : sl[awq_col_of_lane(c)];
#pragma unroll
  for (int t = 0; t < kSets; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) o[c] = live ? acc[t][c][r] * slp[c] * xdown[t][r] : 0.f;
      float4* d4 = reinterpret_cast<float4*>(&red[wave][4 * t + r][8 * lane]);
      d4[0] = make_float4(o[0], o[1], o[2], o[3]);
      d4[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
  __syncthreads();

  finish_chunk<MV, WAVES, WAVES, ACT>(a, red, &s_last, rows, seq);
}

// Two-level split sum of the matrix-core decode kernels (finish_chunk): groups
// of g splits (the smallest g with g * g >= splits) where the last
// workgroups' serial sums (splits planes of MV x 2 KB, bound by one CU's
// loads) end the call: 24 or more splits over at most 16 column chunks (and
// 4 or more at 4 rows). Measured (us, one level / two, f32 x): 8 rows
// 14336 -> 4096 / 13824 -> 5120 / 28672 -> 8192 / 8192 -> 1024 (28 / 54 /
// 112 / 32 splits) 20.4 / 31.0 / 57.6 / 15.0 -> 19.6 / 27.4 / 51.1 / 14.2;
// 4 rows on the first three 16.8 / 21.2 / 44.5 -> 16.3 / 20.0 / 43.9; 12 and
// 16 rows 14336 -> 4096 / 28672 -> 8192 25.5 / 75.5 -> 23.5 / 66.6. Slower
// at 16 or 20 splits (3-17 %), on 56 chunks (8192 -> 28672, 32 splits:
// 3 %) and at 4 rows over 2 chunks (3 %). AWQ_DECODE_TREE=0 / 1 forces one
// level / two (3 or more splits). Then the split-K workspace: partial
// planes and arrival counters.
void set_split_sum(const GemmProblem& p, GemvArgs& a, int mv, int chunks) {
  a.gsize = a.splits;
  a.ngroups = 1;
  const int force = tuning(kTuneDecodeTree, -1);
  const bool deep = a.splits >= 24 && chunks <= 16 && (mv >= 8 || chunks >= 4);
  if (force != 0 && a.splits >= 3 && (force == 1 || deep)) {
    int g = 1;
    while (g * g < a.splits) ++g;
    const int ng = (a.splits + g - 1) / g;
    if (ng > 1) {
      a.gsize = g;
      a.ngroups = ng;
    }
  }
  const int planes = a.splits + (a.ngroups > 1 ? a.ngroups : 0);
  const int cpc = a.ngroups > 1 ? a.ngroups + 1 : 1;
  const size_t part_bytes = (size_t)planes * mv * p.N * sizeof(float);
  const size_t ctr_bytes = (size_t)chunks * cpc * kCounterStride * sizeof(uint32_t);
  a.counters = static_cast<uint32_t*>(ws_get(p, ctr_bytes, kWsCounters));
  a.partial = static_cast<float*>(ws_get(p, part_bytes, kWsPartials));
}

template <int XT, int MT, int WAVES, int RPW>
void launch_cfg(const GemmProblem& p) {
  const int np = (int)(p.N / 8);
  const int chunks = (np + 63) / 64;
  const int rows_per_wg = WAVES * RPW;
  const int splits = (int)((p.K + rows_per_wg - 1) / rows_per_wg);

  GemvArgs a{};
  a.x = p.x;
  a.qweight = p.qweight;
  a.qzeros = p.qzeros;
  a.scales = p.scales;
  a.bias = p.bias;
  a.y = p.y;
  a.st = p.st;
  a.bt = p.bt;
  a.yt = p.yt;
  a.rows = (int32_t)p.rows;
  a.K = (int32_t)p.K;
  a.N = (int32_t)p.N;
  a.group = (int32_t)p.group;
  a.splits = splits;
  a.seq = p.order == AWQ_ORDER_SEQUENTIAL ? 1 : 0;
  if (splits > 1) {
    const size_t part_bytes = (size_t)splits * MT * p.N * sizeof(float);
    const size_t ctr_bytes = (size_t)chunks * kCounterStride * sizeof(uint32_t);
    a.counters = static_cast<uint32_t*>(ws_get(p, ctr_bytes, kWsCounters));
    a.partial = static_cast<float*>(ws_get(p, part_bytes, kWsPartials));
  }
  if (p.act)
    hipLaunchKernelGGL((gemv_kernel<XT, MT, WAVES, RPW, true>), dim3(chunks, splits), dim3(64 * WAVES), 0,
                       p.stream, a);
  else
    hipLaunchKernelGGL((gemv_kernel<XT, MT, WAVES, RPW, false>), dim3(chunks, splits), dim3(64 * WAVES), 0,
                       p.stream, a);
  check_hip(hipGetLastError(), "gemv kernel launch");
}

// Largest rows-per-wave a (x dtype, rows, waves) instantiation holds in
// registers without spilling: two batches of up to 32 weight words per lane
// plus the row accumulators, within 512 / waves-per-SIMD VGPRs (f16/bf16
// activations need a few more for the conversions).
constexpr int rpw_max(int xt, int mt, int waves) {
  const bool f32 = xt == AWQ_F32;
  return mt == 1 ? (waves >= 16 ? (f32 ? 96 : 64) : 128)
       : mt == 2 ? (waves >= 16 ? 8 : waves == 8 ? (f32 ? 16 : 8) : 32)
       : mt == 4 ? (waves >= 8 ? 16 : 32)
       : (waves >= 8 ? (f32 ? 16 : 8) : (f32 ? 32 : 16));
}

// Rows per wave (dividing the group size) and waves per workgroup: enough
// workgroups to occupy the CUs with as few K splits as possible (one row:
// one round of workgroups over the CUs where a shape allows it); never a
// configuration that spills.
template <int XT, int MT, int WMAX>
void launch_rpw(const GemmProblem& p) {
  const int g = (int)p.group;
  const int chunks = (int)((p.N / 8 + 63) / 64);
  int rpw = g % 32 == 0 ? 32 : g % 16 == 0 ? 16 : g % 8 == 0 ? 8 : 4;
  int waves = WMAX;
  auto wgs = [&](int w, int r) {
    return (int64_t)chunks * ((p.K + (int64_t)w * r - 1) / ((int64_t)w * r));
  };
  auto cap = [&](int w, int r) {
    while (r > rpw_max(XT, MT, w)) r >>= 1;
    return r;
  };
  if (MT == 1 && WMAX >= 16 && g % 32 == 0) {
    // One row: one round of workgroups over the CUs (3/4 C .. C of them, C =
    // CUs), since a partial second round finishes late. 16 waves x 32 rows
    // when that gives such a round; fewer, shorter runs (down to 8 rows, more
    // K splits) when it gives fewer; beyond C, 16 x 64 if that gives one
    // round, else 8 waves x 32 rows (several rounds of small workgroups).
    // Measured, us (one row, f32 x), chosen against the next best:
    // 4096 -> 14336 / 14336 -> 4096 / 8192 -> 8192: 16 x 32 (224 / 224 / 256
    // workgroups) 9.8 / 10.2 / 10.4 against 10.5 / 11.6 / 11.0 with 16 x 16;
    // 4096 -> 4096 / 1024 -> 4096 / 8192 -> 1024: 16 x 8 6.3 / 5.2 / 6.7
    // against 6.7 / 6.2 / 7.0 (16 x 16) and 6.8 / 6.5 / 7.4 (8 x 32);
    // 4096 -> 6144: 16 x 16 7.3; 4096 -> 28672, 8192 -> 14336 and
    // 14336 -> 8192: 16 x 64 (224) 17.1 / 17.1 / 17.3, 16 x 32 (448) up to
    // 4 % slower; 5120 -> 13824 / 13824 -> 5120: 8 x 32 (540) 13.3 / 14.5
    // against 15.9 / 16.3 with 16 x 32 (270); 8192 -> 28672 / 28672 -> 8192:
    // 8 x 32 (1792) 29.1 / 30.2 against 31.3 / 31.6 with 16 x 64 (448).
    const int64_t cus = device_cus(), lo = cus * 3 / 4;
    waves = 16;
    rpw = 32;
    const int64_t w32 = wgs(16, 32);
    if (w32 < lo) {
      while (rpw > 8 && wgs(16, rpw) < lo) rpw >>= 1;
    } else if (w32 > cus) {
      const int64_t w64 = wgs(16, 64);
      if (g % 64 == 0 && rpw_max(XT, 1, 16) >= 64 && w64 >= lo && w64 <= cus) rpw = 64;
      else waves = 8;
    }
  } else {
    while (waves > 4 && wgs(waves, cap(waves, rpw)) < 192) waves >>= 1;
    // Small matrices keep more waves even below 192 workgroups: two rows 16
    // waves of 8 (4096 x 1024: 12.8 us with 4 waves, 8.4 with 16).
    if (MT == 2) waves = WMAX;
    rpw = cap(waves, rpw);
    // Long runs per wave (fewer splits) while the workgroup count stays high.
    while (rpw < 128 && 2 * rpw <= rpw_max(XT, MT, waves) && g % (2 * rpw) == 0 &&
           wgs(waves, 2 * rpw) >= 192)
      rpw *= 2;
  }
  if (int v = tuning(kTuneGemvWaves, 0); (v == 4 || v == 8 || v == 16) && v <= WMAX) waves = v;
  if (int v = tuning(kTuneGemvRpw, 0); v >= 4 && g % v == 0) rpw = v;
  rpw = cap(waves, rpw);
  while (g % rpw != 0) rpw >>= 1;
#define AWQ_GEMV_CASE(W, R) \
  if constexpr (R <= rpw_max(XT, MT, W)) { if (waves == W && rpw == R) return launch_cfg<XT, MT, W, R>(p); }
#define AWQ_GEMV_WCASES(W)                                                                    \
  AWQ_GEMV_CASE(W, 4) AWQ_GEMV_CASE(W, 8) AWQ_GEMV_CASE(W, 16) AWQ_GEMV_CASE(W, 32)          \
  AWQ_GEMV_CASE(W, 64) AWQ_GEMV_CASE(W, 96) AWQ_GEMV_CASE(W, 128)
  if constexpr (WMAX >= 16) { AWQ_GEMV_WCASES(16) }
  AWQ_GEMV_WCASES(8)
  AWQ_GEMV_WCASES(4)
#undef AWQ_GEMV_WCASES
#undef AWQ_GEMV_CASE
  panic("decode GEMV: no kernel configuration for this shape");
}

template <int XT, int MV, int WAVES, int RPW>
void launch_mfma_cfg(const GemmProblem& p) {
  const int np = (int)(p.N / 8);
  const int chunks = (np + 63) / 64;
  const int splits = (int)((p.K + WAVES * RPW - 1) / (WAVES * RPW));
  GemvArgs a{};
  a.x = p.x;
  a.qweight = p.qweight;
  a.qzeros = p.qzeros;
  a.scales = p.scales;
  a.bias = p.bias;
  a.y = p.y;
  a.st = p.st;
  a.bt = p.bt;
  a.yt = p.yt;
  a.rows = (int32_t)p.rows;
  a.K = (int32_t)p.K;
  a.N = (int32_t)p.N;
  a.group = (int32_t)p.group;
  a.splits = splits;
  a.seq = p.order == AWQ_ORDER_SEQUENTIAL ? 1 : 0;
  if (splits > 1) set_split_sum(p, a, MV, chunks);
  if (p.act)
    hipLaunchKernelGGL((gemv_mfma_kernel<XT, MV, WAVES, RPW, true>), dim3(chunks, splits), dim3(64 * WAVES),
                       0, p.stream, a);
  else
    hipLaunchKernelGGL((gemv_mfma_kernel<XT, MV, WAVES, RPW, false>), dim3(chunks, splits), dim3(64 * WAVES),
                       0, p.stream, a);
  check_hip(hipGetLastError(), "gemv mfma kernel launch");
}

// Small-M matrix-core path: 8 waves per workgroup, 64 rows per wave when the
// group allows and that still gives >= 192 workgroups, else 32. Also 32 for
// 2..4 rows when 64 would already give two workgroups per CU: those
// configurations hold two 8-wave workgroups per CU (<= 128 VGPRs), and the
// second hides the first's loads (8192 -> 28672 at M = 2/4: 51/56 -> 39/45
// us); with 8 rows the registers allow one, and the extra K splits only cost.
// (Fewer waves per workgroup measured slower at every shape tried: more K
// splits cost more in the final reduction than the extra workgroups gain.)
template <int XT, int MV>
void launch_mfma(const GemmProblem& p) {
  const int chunks = (int)((p.N / 8 + 63) / 64);
  auto wgs = [&](int w, int r) {
    return (int64_t)chunks * ((p.K + (int64_t)w * r - 1) / ((int64_t)w * r));
  };
  int rpw = p.group % 64 == 0 ? 64 : 32;
  int waves = 8;
  if (rpw == 64 && wgs(8, 64) < 192) rpw = 32;
  if (rpw == 64 && MV <= 4 && wgs(8, 64) >= 2 * device_cus()) rpw = 32;
  // 8 rows past one round of workgroups over the CUs: 4 waves x 64 rows
  // (twice the workgroups, two per CU). 5120 -> 13824 / 8192 -> 28672 /
  // 28672 -> 8192 (270 / 896 / 896 workgroups of 8 x 64): 29.3 / 55.4 / 60.2
  // -> 25.7 / 49.3 / 57.3 us; within one round (224, 256) 4 x 64 measured
  // 13-18 % slower.
  if (MV == 8 && rpw == 64 && wgs(8, 64) > device_cus()) waves = 4;
  if (int v = tuning(kTuneMfmaWaves, 0); v == 4 || v == 8) waves = v;
  if (int v = tuning(kTuneMfmaRpw, 0); (v == 32 || v == 64) && p.group % v == 0) rpw = v;
  if (waves == 8 && rpw == 64) return launch_mfma_cfg<XT, MV, 8, 64>(p);
  if (waves == 8) return launch_mfma_cfg<XT, MV, 8, 32>(p);
  if (rpw == 64) return launch_mfma_cfg<XT, MV, 4, 64>(p);
  return launch_mfma_cfg<XT, MV, 4, 32>(p);
}

template <int XT, int MV, int WAVES, int RPW>
void launch_m4_cfg(const GemmProblem& p) {
  const int np = (int)(p.N / 8);
  const int chunks = (np + 63) / 64;
  const int splits = (int)((p.K + WAVES * RPW - 1) / (WAVES * RPW));
  GemvArgs a{};
  a.x = p.x;
  a.qweight = p.qweight;
  a.qzeros = p.qzeros;
  a.scales = p.scales;
  a.bias = p.bias;
  a.y = p.y;
  a.st = p.st;
  a.bt = p.bt;
  a.yt = p.yt;
  a.rows = (int32_t)p.rows;
  a.K = (int32_t)p.K;
  a.N = (int32_t)p.N;
  a.group = (int32_t)p.group;
  a.splits = splits;
  a.seq = p.order == AWQ_ORDER_SEQUENTIAL ? 1 : 0;
  if (splits > 1) set_split_sum(p, a, MV, chunks);
  if (p.act)
    hipLaunchKernelGGL((gemv_m4_kernel<XT, MV, WAVES, RPW, true>), dim3(chunks, splits), dim3(64 * WAVES), 0,
                       p.stream, a);
  else
    hipLaunchKernelGGL((gemv_m4_kernel<XT, MV, WAVES, RPW, false>), dim3(chunks, splits), dim3(64 * WAVES), 0,
                       p.stream, a);
  check_hip(hipGetLastError(), "gemv m4 kernel launch");
}

// 4x4x4 matrix-core decode. 512 rows per workgroup (16 waves x 32 rows, or
// 8 x 64) when that gives one round of workgroups over the CUs (3/4 C .. C,
// C = CUs): 16 x 32 for f16 activations (the only case whose registers,
// <= 128 VGPRs, and LDS slots, 16 x 4 rows x 2 KB, allow 16 waves), else
// 8 x 64 (if the group allows 64); otherwise 8 waves of 32 rows. Measured at
// 4 rows, us: 8 x 64 at 4096 -> 14336 / 14336 -> 4096 (224 workgroups) 5-12 %
// faster than 8 x 32 with f32 activations, 16 x 32 at 14336 -> 4096 /
// 8192 -> 8192 (224 / 256) 13.4 / 12.6 against 15.0 / 13.3 with 8 waves for
// f16; 8 x 32 where 512 rows give a partial or several rounds: 5120 -> 13824
// / 13824 -> 5120 (270) f32 25.3 / 26.3 -> 19.9 / 21.0 (against 8 x 64),
// f16 19.3 / 20.2 -> 15.8 / 17.9 (against 16 x 32); 8192 -> 28672 (896) f16
// 38.1 -> 33.7; 4096 -> 4096 (64) f16 10.0 -> 8.3.
template <int XT, int MV>
void launch_m4(const GemmProblem& p) {
  constexpr bool k16 = MV == 4 && XT == AWQ_F16;
  const int64_t chunks = (p.N / 8 + 63) / 64;
  const int64_t wgs64 = chunks * ((p.K + 511) / 512);
  const int64_t cus = device_cus();
  const bool one_round = wgs64 >= cus * 3 / 4 && wgs64 <= cus;
  int waves = k16 && one_round ? 16 : 8;
  int rpw = (waves == 8 && p.group % 64 == 0 && one_round) ? 64 : 32;
  if (int v = tuning(kTuneM4Waves, 0); v == 8 || (v == 16 && k16)) waves = v;
  if (int v = tuning(kTuneM4Rpw, 0); (v == 32 || v == 64) && p.group % v == 0) rpw = v;
  if constexpr (k16) {
    if (waves == 16) return launch_m4_cfg<XT, MV, 16, 32>(p);
  }
  if (rpw == 64) return launch_m4_cfg<XT, MV, 8, 64>(p);
  return launch_m4_cfg<XT, MV, 8, 32>(p);
}

template <int XT>
void launch_xt(const GemmProblem& p) {
  // 2..8 rows: matrix cores, whose cost per weight does not grow with M,
  // except 2 rows of a small matrix (K x N <= 4096 x 4096), where the VALU
  // kernel with 16 waves measured faster (4096 x 4096 / 4096 x 1024 /
  // 8192 x 1024: 8.4 / 8.4 / 10.3 us against 10.5 / 10.2 / 11.7).
  // AWQ_DECODE_MFMA=0/1 forces the choice.
  const int force = tuning(kTuneDecodeMfma, -1);
  const bool small2 = p.rows == 2 && p.K * p.N <= 4096ll * 4096ll;
  const bool mfma_ok = p.rows >= 2 && p.group % 32 == 0 && p.K % 32 == 0 &&
                       (force == 1 || (force != 0 && !small2));
  if (p.rows > 8) return launch_mfma<XT, 16>(p);  // accepted by small_m_mfma_ok
  // 2..4 rows: the 4x4x4 blocks (no padding to 16 rows, no transposes):
  // 4096 -> 14336 at M = 4 15.2 -> 11.4 us with f16 activations, 16.3 ->
  // 14.6 with f32; 5..8 rows stay on the 16x16x32 kernel (at 8 rows the
  // 4x4x4 MFMAs, twice as many, measured 5-45 % slower). AWQ_DECODE_M4=0
  // forces the 16x16x32 kernel.
  if (mfma_ok && p.rows <= 4 && tuning(kTuneDecodeM4, 1) != 0) return launch_m4<XT, 4>(p);
  if (mfma_ok) {
    // Rows kept in LDS, the workspace and the final reduction (the MFMA
    // tile always computes 16).
    if (p.rows <= 2) return launch_mfma<XT, 2>(p);
    if (p.rows <= 4) return launch_mfma<XT, 4>(p);
    return launch_mfma<XT, 8>(p);
  }
  if (p.rows <= 1) launch_rpw<XT, 1, 16>(p);
  else if (p.rows <= 2) launch_rpw<XT, 2, 16>(p);
  else if (p.rows <= 4) launch_rpw<XT, 4, 8>(p);
  else launch_rpw<XT, 8, 8>(p);
}

}  // namespace

// 9..16 rows (prefill by the reference's M > 8 rule) on the decode kernels'
// 16-row tile, unless the skinny kernel takes them (f16/bf16 activations on
// outputs it suits). AWQ_SMALLM_MFMA=0 sends them to the prefill kernels.
bool small_m_mfma_ok(const GemmProblem& p, int64_t launch_m) {
  return launch_m > 8 && launch_m <= 16 && p.rows <= 16 && p.group % 32 == 0 && p.K % 32 == 0 &&
         tuning(kTuneSmallMMfma, 1) != 0 && !skinny_ok(p);
}

void launch_gemv(const GemmProblem& p) {
  AWQ_ASSERT(p.K < (1ll << 31) && p.N < (1ll << 31) && p.K * (p.N / 8) < (1ll << 30),
             "decode GEMV: tensor too large");
  switch (p.xt) {
    case AWQ_F32: launch_xt<AWQ_F32>(p); break;
    case AWQ_F16: launch_xt<AWQ_F16>(p); break;
    default: launch_xt<AWQ_BF16>(p); break;
  }
}

}  // namespace cube_awq
