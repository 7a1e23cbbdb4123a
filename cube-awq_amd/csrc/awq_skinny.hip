// awq_skinny.hip -- fused AWQ dequant-GEMM for skinny problems (9..128 rows,
// f16 or bf16 activations) on gfx950.
//
// Y[M, N] = X[M, K] . W[K, N], W[k, n] = F((q - z) * s) for F = f16 or bf16,
// the reference's F-typed dequantised weight (gemm_awq,
// src/kernel/awq_kernel_gemm.rs:181-439), accumulated in fp32 on
// v_mfma_f32_16x16x32_f16 / _bf16.
//
// With few activation rows the large-tile kernel (awq_gemm.hip) is latency
// bound: every 64-row stage of a 128..256-column tile is a load, dequantise,
// barrier, MFMA round trip, and on wide outputs its tiles already fill the
// CUs, so K splits cannot hide that. Here the weights stream as in the decode
// kernels:
//  * A workgroup owns a chunk of 256 columns (32 packed words = 128 bytes of
//    each row; 8 waves of 32 columns) or, on outputs narrower than 6144
//    columns, 64 (8 packed words; 4 waves of 16 columns, one MFMA tile each,
//    chunks placed so each XCD runs a contiguous run of them and their
//    32-byte row pieces share 128-byte lines in its L2), and a run of K;
//    32-row steps of W, the matching 32 columns of X and,
//    up front, the zeros and scales of the run's groups go global -> LDS
//    directly (buffer_load ... lds, 16 bytes per lane for W and X, 4 for the
//    zeros and scales) into a ring of kRing steps, kRing - 2 steps ahead,
//    with explicit vmcnt waits and one s_barrier per two steps.
//  * 256 columns: wave w takes packs 4 w .. 4 w + 3 (32 columns, two
//    16-column MFMA tiles) for every 16-row tile, so each weight is
//    dequantised once. Lane (lg = lane / 16, lj = lane % 16) reads the 8
//    words of rows 8 lg .. 8 lg + 7 of pack 4 w + (lj & 3) from LDS and
//    builds the B operands of tiles 0 and 1 from packed lanes 2 (lj >> 2)
//    and 2 (lj >> 2) + 1, the two nibbles of one byte (64 columns: pack
//    2 w + (lj & 1), packed lane lj >> 1): one v_perm_b32 gathers that byte
//    of two rows, one v_bitop3_b32 per nibble makes the f16 magic 1024 + q
//    (64 + q for the high nibble), then an exact v_pk_add_f16 of -(1024 + z)
//    and one v_pk_mul_f16 by s: 1.75 VALU ops per weight. bf16 (no packed bf16
//    arithmetic on gfx950): after the same v_perm_b32, one v_and_b32 leaves
//    q (or 16 q) in bytes 0 and 2, v_cvt_f32_ubyte0/2 convert them, one
//    v_fma_f32 per weight forms q s' - z s = (q - z) s exactly (s' = s or
//    s / 16; exact for 16-bit scales), and v_cvt_pk_bf16_f32 rounds each pair
//    once: 3.5 VALU ops per weight.
//  * Waves never share outputs, so there is no cross-wave reduction; K
//    splits (grid.y) publish fp32 partials and the last workgroup to arrive on
//    a chunk sums them in split order (deterministic), adds the bias and
//    writes Y.
// Algorithmic HBM bytes per call: K*N/2 + (K/g)*(N/8)*4 + (K/g)*N*sizeof(s) +
// M*K*2 + M*N*sizeof(y).
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "awq_common.h"

namespace cube_awq {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kStep = 32;           // K rows per step (one MFMA k-block)
constexpr int kRing = 8;            // steps held in LDS
constexpr int kCtrStride = 64;      // u32 words between arrival counters

// Layout constants of a chunk width CW (columns per workgroup) over WV waves:
// 256 columns on 4 waves (64 columns, four 16-column MFMA tiles each) or on
// 8 (32 columns, two tiles), 64 columns on 4 waves (16 columns, one tile).
template <int CW, int WV>
struct Chunk {
  static constexpr int kWaves = WV;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kPacks = CW / 8;               // packed words per row
  static constexpr int kPPW = kPacks / kWaves;         // packs per wave (8, 4 or 2)
  static constexpr int kT = kPPW / 2;                  // 16-column MFMA tiles per wave
  static constexpr int kRowBytes = CW / 2;             // one packed W row
  // W: wave i < 4 moves rows 8 i .. 8 i + 7 of a step (one DMA: 16 bytes per
  // lane for 128-byte rows, 4 for 32-byte rows) into a padded 8-row block
  // (the pad spreads the blocks over the LDS banks).
  static constexpr int kWBlock = 8 * kRowBytes + (CW == 256 ? 32 : 16);
  static constexpr int kWSlot = (kStep / 8) * kWBlock;
  static constexpr int kMaxGroups = CW == 256 ? 36 : 128;  // groups a K run may touch
  static constexpr int kXWave0 = kWaves - 4;           // first wave loading X
  static_assert(kWaves >= 4 && kT >= 1 && kT <= 4 && kPPW * kWaves == kPacks, "chunk layout");
};

// Dynamic LDS of skinny_kernel<MT, *, *, CW>: the W and X rings, then the
// zero words and scales of up to kMaxGroups groups.
template <int MT, int CW>
constexpr int skinny_smem_bytes() {
  using C = Chunk<CW, 4>;  // the memory layout does not depend on the wave count
  return kRing * C::kWSlot + kRing * 16 * MT * 64 + C::kMaxGroups * C::kPacks * 4 + C::kMaxGroups * CW * 4;
}

struct SkinnyArgs {
  const void* x;
  const uint32_t* qweight;
  const uint32_t* qzeros;
  const void* scales;
  const void* bias;
  void* y;
  float* partial;      // [splits (+ ngroups)][M][N] when splits > 1
  uint32_t* counters;  // per chunk (ngroups + 1 with the two-level sum), kCtrStride apart, zero between calls
  int32_t st, bt, yt;
  int32_t M, K, N, group;
  int32_t splits, steps_per_split;
  int32_t seq;         // sequential nibble order
  int32_t chunks;      // column chunks (grid.x)
  int32_t xcd_chunks;  // leading chunks covered by the XCD mapping (multiple of 8)
  int32_t gsize;       // two-level split sum: splits per group (when ngroups > 1)
  int32_t ngroups;     // groups of gsize splits; 0 or 1: one level
};

constexpr int waitcnt_vm(int vm) { return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

__device__ __forceinline__ void dma4(rsrc_t r, unsigned char* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, soff, 0, 0);
}
// 16 bytes per lane: lane l's data lands at dst + 16 l.
__device__ __forceinline__ void dma16(rsrc_t r, unsigned char* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

// Granule swizzle of an X row in LDS (64 bytes = four 16-byte granules):
// granule g of row r sits in slot g ^ xswz(r), so the 16 rows one A-operand
// read touches spread over all banks. Chosen among 22 candidates with a
// probe kernel under SQ_LDS_BANK_CONFLICT: (r >> 1) & 3 reads conflict-free,
// (r >> 2) & 3 cost 4 conflict cycles per ds_read_b128 (gfx950 serves a
// 16-byte read in lane groups other than 16 consecutive lanes).
__device__ __forceinline__ int xswz(int r) { return (r >> 1) & 3; }

// ACT: the gate/up SiLU epilogue (store_out; AutoAWQ order only), a template
// parameter so the plain kernel's code is untouched by it. BF: bf16
// activations (16-bit scales), W dequantised through f32 (see compute).
template <int MT, bool ACT, bool BF, int CW, int WV>
__global__ __launch_bounds__(64 * WV) void skinny_kernel(SkinnyArgs a) {
  using C = Chunk<CW, WV>;
  typedef typename std::conditional<BF, bf16x8_t, f16x8_t>::type XV;
  constexpr int kT = C::kT;
  constexpr int kPacks = C::kPacks;
  constexpr int kXRows = 16 * MT;
  constexpr int kXSlot = kXRows * 64;          // 32 f16 columns of X per row
  // 16-byte DMAs per step for X: rows 16 j .. 16 j + 15 by X wave j % 4.
  constexpr int kXPerWave = (MT + 3) / 4;
  static_assert(MT >= 1 && MT <= 8, "row tiles");
  constexpr int kSmem = skinny_smem_bytes<MT, CW>();
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* wring = smem;                               // kRing W slots
  unsigned char* xring = smem + kRing * C::kWSlot;           // kRing X slots
  uint32_t* zlds = reinterpret_cast<uint32_t*>(xring + kRing * kXSlot);  // [groups][kPacks] zero words
  unsigned char* slds = reinterpret_cast<unsigned char*>(zlds + C::kMaxGroups * kPacks);  // [groups][CW] scales

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4, lj = lane & 15;
  // Consecutive workgroups go to different XCDs: remap so each XCD runs a
  // contiguous run of chunks, whose rows share 128-byte lines in its L2.
  int chunk = blockIdx.x;
  if (chunk < a.xcd_chunks) chunk = (chunk & 7) * (a.xcd_chunks >> 3) + (chunk >> 3);
  const int split = blockIdx.y;
  const int np = a.N >> 3;
  const int s0 = split * a.steps_per_split;
  const int steps = min(a.steps_per_split, a.K / kStep - s0);
  const int k_begin = s0 * kStep;
  const int g_first = k_begin / a.group;
  const int es = a.st == AWQ_F32 ? 4 : 2;

  // ---- prologue DMAs: zeros and scales of the run's groups (wave 0 and 1),
  // then the first kRing - 2 steps of W and X (every wave) ---------------------
  const int ngroups = (k_begin + steps * kStep - 1) / a.group - g_first + 1;
  const int ngroups_all = a.K / a.group;
  const rsrc_t zres = make_rsrc(a.qzeros, (uint32_t)(ngroups_all * np * 4));
  const rsrc_t sres = make_rsrc(a.scales, (uint32_t)((int64_t)ngroups_all * a.N * es));
  if (wave == 0) {
    // lane l: zero word of pack l % kPacks of group gi + l / kPacks
    constexpr int kGpi = 64 / kPacks;  // groups per instruction
    for (int gi = 0; gi < ngroups; gi += kGpi) {
      const int pk = min(chunk * kPacks + (lane % kPacks), np - 1);
      const int grc = min(g_first + gi + lane / kPacks, ngroups_all - 1);
      dma4(zres, reinterpret_cast<unsigned char*>(zlds + gi * kPacks), (uint32_t)(grc * np + pk) * 4u, 0);
    }
  } else if (wave == 1) {
    // scales of the chunk's CW columns per group, CW * es bytes, stored at a
    // CW * 4-byte pitch
    const int row_bytes = CW * es;
    if (row_bytes >= 256) {
      for (int gi = 0; gi < ngroups; ++gi) {
        const int grc = min(g_first + gi, ngroups_all - 1);
        for (int o = 0; o < row_bytes; o += 256) {
          const int col_byte = min(chunk * CW * es + o + lane * 4, a.N * es - 4);
          dma4(sres, slds + gi * CW * 4 + o, (uint32_t)((int64_t)grc * a.N * es + col_byte), 0);
        }
      }
    } else {
      // one instruction covers 256 / row_bytes groups: lane l -> group
      // gi + l / (row_bytes / 4), byte 4 (l % (row_bytes / 4)); each group's
      // row lands at its CW * 4 pitch only if 256 / row_bytes == 1, so the
      // lanes of later groups go through separate instructions.
      const int lpg = row_bytes / 4;  // lanes per group row
      for (int gi = 0; gi < ngroups; ++gi) {
        const int grc = min(g_first + gi, ngroups_all - 1);
        const int col_byte = min(chunk * CW * es + (lane % lpg) * 4, a.N * es - 4);
        if (lane < lpg)
          dma4(sres, slds + gi * CW * 4, (uint32_t)((int64_t)grc * a.N * es + col_byte), 0);
      }
    }
  }

  const rsrc_t wres = make_rsrc(a.qweight, (uint32_t)a.K * (uint32_t)np * 4u);
  const rsrc_t xres = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.K * 2));
  const uint32_t row_bytes_w = (uint32_t)np * 4u;
  // W (waves 0..3): wave i moves rows 8 i .. 8 i + 7 of a step. CW = 256:
  // lane l -> row 8 i + (l >> 3), packs 4 (l & 7) .. + 3 (16 bytes; clamped
  // at the last pack). CW = 64: lane l -> row 8 i + (l >> 3), pack l & 7.
  const uint32_t wvoff = CW == 256
      ? (uint32_t)(lane >> 3) * row_bytes_w + (uint32_t)min(chunk * kPacks + 4 * (lane & 7), np - 4) * 4u
      : (uint32_t)(lane >> 3) * row_bytes_w + (uint32_t)min(chunk * kPacks + (lane & 7), np - 1) * 4u;
  // X (waves kXWave0 ..): rows 16 j .. 16 j + 15; lane l -> row + (l >> 2),
  // slot l & 3 holding granule (l & 3) ^ xswz(row) (16 bytes = 8 f16 columns).
  const int xw = wave - C::kXWave0;
  const int n_xins = xw < 0 ? 0 : (MT - xw + 3) / 4;  // tiles xw, xw + 4, ... below MT
  uint32_t xvoff[kXPerWave];
#pragma unroll
  for (int i = 0; i < kXPerWave; ++i) {
    const int j = (xw < 0 ? 0 : xw) + 4 * i;
    const int r = 16 * j + (lane >> 2);
    const int g = (lane & 3) ^ xswz(r);
    const int rc = min(r, a.M - 1);  // rows past M read row M - 1 (never stored)
    xvoff[i] = (uint32_t)(((int64_t)rc * a.K) * 2 + g * 16);
  }
  auto issue = [&](int s) {
    const int slot = s % kRing;
    const uint32_t k = (uint32_t)((s0 + s) * kStep);
    if (wave < 4) {
      if constexpr (CW == 256) dma16(wres, wring + slot * C::kWSlot + wave * C::kWBlock, wvoff, (k + 8 * wave) * row_bytes_w);
      else dma4(wres, wring + slot * C::kWSlot + wave * C::kWBlock, wvoff, (k + 8 * wave) * row_bytes_w);
    }
    if (xw >= 0) {
#pragma unroll
      for (int i = 0; i < kXPerWave; ++i)
        if (i < n_xins) dma16(xres, xring + slot * kXSlot + (xw + 4 * i) * 1024, xvoff[i], k * 2u);
    }
  };
  // VMEM instructions this wave issues per step (uniform per wave): 1..3.
  const int per_step = (wave < 4 ? 1 : 0) + n_xins;
  const int pre = min(kRing - 2, steps);
  for (int s = 0; s < pre; ++s) issue(s);

  // ---- per-lane constants: wave w owns packs kPPW w .. kPPW w + kPPW - 1
  // (16 kT columns) for every row tile; lane lj is pack kPPW w + lj % kPPW
  // and in tile t packed lane c = kT (lj / kPPW) + t (byte c / 2, nibble
  // c & 1), so each weight is dequantised once, and with two or more tiles
  // tiles 2p and 2p + 1 are the two nibbles of one byte: one v_perm_b32
  // serves both. Packed lanes c and c + 4 (AutoAWQ columns 2j and 2j + 1)
  // sit in lanes lj and lj ^ 8, same tile.
  constexpr int kP = (kT + 1) / 2;                 // bytes (v_perm selectors) per lane
  const int pl = C::kPPW * wave + (lj % C::kPPW);  // pack within the chunk
  const int c0 = kT * (lj / C::kPPW);              // packed lane of tile 0
  const bool seq = a.seq != 0;
  int colt[kT];
#pragma unroll
  for (int t = 0; t < kT; ++t) colt[t] = seq ? c0 + t : awq_col_of_lane(c0 + t);
  uint32_t selp[kP];
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    const uint32_t b = (uint32_t)((c0 + 2 * p) >> 1);
    selp[p] = b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
  }
  // Nibble of tile t: t & 1 with two or more tiles, c0 & 1 with one.
  auto nib = [&](int t) { return kT >= 2 ? (t & 1) : (c0 & 1); };
  // This lane's scale of tile t within a group's row of scales in LDS: the
  // aligned 32-bit word holding it and the shift that brings it to bit 0.
  uint32_t soff[kT], sshift[kT];
#pragma unroll
  for (int t = 0; t < kT; ++t) {
    const int col = 8 * pl + colt[t];
    soff[t] = es == 4 ? (uint32_t)col * 4u : ((uint32_t)col * 2u) & ~3u;
    sshift[t] = es == 4 ? 0u : 16u * (uint32_t)(col & 1);
  }
  auto hmask = [&](int t) { return nib(t) ? 0x00F000F0u : 0x000F000Fu; };
  auto hexp = [&](int t) { return nib(t) ? 0x54005400u : 0x64006400u; };

  f32x4_t acc[MT][kT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < kT; ++t) acc[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  f16x2_t fz[kT], fs[kT];
  float bs[kT], bzs[kT];  // BF: s (s / 16 for the high nibble) and -z s
  // Group of the zeros and scales, counted per step instead of divided out
  // (the run starts g_skip steps into group g_first). fetch() reads a new
  // group's zero word and scales from LDS together with the step's W and X
  // (one wait for all of them); compute() converts them when the step
  // starts that group.
  const int g_steps = a.group / kStep;
  const int g_skip = (k_begin % a.group) / kStep;
  int fg = -1, fg_left = 0;

  struct StepRegs {
    uint32_t w[8];     // the 8 W words of this lane's pack (rows 8 lg ..)
    XV x[MT];          // A operands of every row tile
    uint32_t zw;       // zero word of a new group
    uint32_t sb[kT];   // the 32-bit LDS word holding each tile's scale of a new group
    bool newg;
  };

  auto fetch = [&](int s, StepRegs& r) {
    const unsigned char* wsl = wring + (s % kRing) * C::kWSlot;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int rr = 8 * lg + u;
      r.w[u] = *reinterpret_cast<const uint32_t*>(wsl + (rr >> 3) * C::kWBlock + (rr & 7) * C::kRowBytes + pl * 4);
    }
    const unsigned char* xsl = xring + (s % kRing) * kXSlot;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int rr = 16 * i + lj;
      r.x[i] = *reinterpret_cast<const XV*>(xsl + rr * 64 + ((lg ^ xswz(rr)) << 4));
    }
    r.newg = fg_left == 0;
    if (r.newg) {
      ++fg;
      fg_left = fg == 0 ? g_steps - g_skip : g_steps;
      r.zw = zlds[fg * kPacks + pl];
      const unsigned char* srow = slds + fg * CW * 4;
#pragma unroll
      for (int t = 0; t < kT; ++t) r.sb[t] = *reinterpret_cast<const uint32_t*>(srow + soff[t]);
    }
    --fg_left;
  };

  // One step (steps are computed in order): the zero points and scales when
  // a group starts, then per byte the B operands of its tiles and their
  // MT MFMAs each.
  auto compute = [&](const StepRegs& r) {
    if (r.newg) {
#pragma unroll
      for (int t = 0; t < kT; ++t) {
        const uint32_t zh = __builtin_amdgcn_perm(r.zw, r.zw, selp[kT >= 2 ? t / 2 : 0]);
        // Branch-free on the scale type (selects, not branches, so the
        // loads above need no wait of their own).
        const uint32_t bits = r.sb[t] >> sshift[t];
        const float s32 = __builtin_bit_cast(float, bits);
        const float s16 = (float)__builtin_bit_cast(f16_t, (uint16_t)bits);
        const float sbf = __builtin_bit_cast(float, bits << 16);
        const float sv = es == 4 ? s32 : (a.st == AWQ_F16 ? s16 : sbf);
        if constexpr (BF) {
          // z s is exact in f32 for 16-bit scales (4 by at most 11 bits).
          const int z = (int)((zh >> (4 * nib(t))) & 0xFu);
          bs[t] = nib(t) ? sv * 0.0625f : sv;
          bzs[t] = -(float)z * sv;
        } else {
          fz[t] = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_bitop3_b32(zh, hmask(t), hexp(t), 0xEA));
          const _Float16 sh = (_Float16)sv;
          fs[t] = f16x2_t{sh, sh};
        }
      }
    }
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      constexpr int kTP = kT >= 2 ? 2 : 1;  // tiles of this byte
      XV bq[kTP];
#pragma unroll
      for (int u = 0; u < 8; u += 2) {
        const uint32_t h = __builtin_amdgcn_perm(r.w[u + 1], r.w[u], selp[p]);
#pragma unroll
        for (int e = 0; e < kTP; ++e) {
          const int t = kTP * p + e;
          if constexpr (BF) {
            // Bytes 0 and 2 hold q (or 16 q): v_cvt_f32_ubyte0/2, then one fma
            // gives (q - z) s exactly (q s and z s are exact, so is their
            // difference), rounded once to bf16 (v_cvt_pk_bf16_f32).
            const uint32_t hm = h & hmask(t);
            const float q0 = (float)(hm & 0xFFu), q1 = (float)((hm >> 16) & 0xFFu);
            bq[e][u] = (__bf16)__builtin_fmaf(q0, bs[t], bzs[t]);
            bq[e][u + 1] = (__bf16)__builtin_fmaf(q1, bs[t], bzs[t]);
          } else {
            const f16x2_t v = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_bitop3_b32(h, hmask(t), hexp(t), 0xEA));
            const f16x2_t d = (v - fz[t]) * fs[t];
            bq[e][u] = d[0];
            bq[e][u + 1] = d[1];
          }
        }
      }
#pragma unroll
      for (int e = 0; e < kTP; ++e) {
        const int t = kTP * p + e;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          if constexpr (BF) acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.x[i], bq[e], acc[i][t], 0, 0, 0);
          else acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.x[i], bq[e], acc[i][t], 0, 0, 0);
        }
      }
    }
  };

  // Two steps per barrier. With up to 3 row tiles both are fetched from LDS
  // before either is computed (the second step's LDS latency hides under the
  // first's dequantisation; measured 2-7 % faster, not with 4 or more tiles).
  for (int s = 0; s < steps; s += 2) {
    // Steps s and s + 1 have landed once no more than the later steps' DMAs
    // are in flight.
    if (s + kRing - 3 < steps) {
      if (per_step == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm((kRing - 4) * 1));
      else if (per_step == 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm((kRing - 4) * 2));
      else __builtin_amdgcn_s_waitcnt(waitcnt_vm((kRing - 4) * 3));
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
    __builtin_amdgcn_s_barrier();
    // into the slots steps s - 2 and s - 1 used
    if (s + kRing - 2 < steps) issue(s + kRing - 2);
    if (s + kRing - 1 < steps) issue(s + kRing - 1);
    StepRegs ra, rb;
    const bool two = s + 1 < steps;
    if constexpr (MT * kT <= 6 || WV == 4) {
      fetch(s, ra);
      if (two) fetch(s + 1, rb);
      compute(ra);
      if (two) compute(rb);
    } else {  // many MFMAs per step: enough to cover the LDS latency
      fetch(s, ra);
      compute(ra);
      if (two) {
        fetch(s + 1, rb);
        compute(rb);
      }
    }
  }

  // ---- epilogue: element r of acc[i][t] is row 16 i + 4 lg + r, column
  // 8 (chunk kPacks + pl) + colt[t] ----------------------------------------------
  const int nbase = chunk * CW + 8 * pl;
  if (a.splits > 1) {
    const int planes = a.splits + (a.ngroups > 1 ? a.ngroups : 0);
    const rsrc_t pres = make_rsrc(a.partial, (uint32_t)((int64_t)planes * a.M * a.N * 4));
    constexpr int kQuads = CW / 4;
    // 256-column chunks stage the partial tile in LDS (idle once every wave
    // has left the main loop) and store it as whole 16-byte row pieces with
    // the agent-scope (sc1) policy: full 128-byte lines instead of 4-byte
    // stores scattered over the MFMA layout, which wrote each line in halves
    // (4096 -> 14336 at M = 64: the store phase 4.9 -> 2.4 us, the call
    // 29.8 -> 26.7 us; M = 128 44.9 -> 39.4 us). 64-column chunks keep the
    // direct stores (staged, 4096 -> 4096 at M = 64 measured 15.6 -> 16.8 us;
    // reading the own split back from LDS in the sum was slower too).
    constexpr bool kStage = CW == 256;
    constexpr int kPitch = CW * 4 + 16;  // bytes per staged row (the pad spreads the banks)
    static_assert(!kStage || 16 * MT * kPitch + 16 <= kSmem, "the partial tile fits the LDS");
    volatile int* s_last = reinterpret_cast<volatile int*>(smem + kSmem - 16);  // past the staged tile
    if constexpr (kStage) {
      __syncthreads();  // every wave is done with the ring
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < kT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            *reinterpret_cast<float*>(smem + (16 * i + 4 * lg + r) * kPitch + (8 * pl + colt[t]) * 4) =
                acc[i][t][r];
      __syncthreads();
      const uint32_t split_off = (uint32_t)((int64_t)split * a.M * a.N * 4);
      for (int e = tid; e < a.M * kQuads; e += C::kThreads) {
        const int m = e / kQuads, q = e % kQuads;
        const int n = chunk * CW + 4 * q;
        if (n < a.N) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(smem + m * kPitch + q * 16);
          __builtin_amdgcn_raw_buffer_store_b128(v, pres, (uint32_t)(((int64_t)m * a.N + n) * 4), split_off,
                                                 kCachePolicySC1);
        }
      }
    } else {
      float* part = a.partial + (int64_t)split * a.M * a.N;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < kT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 16 * i + 4 * lg + r;
            const int n = nbase + colt[t];
            if (m < a.M && n < a.N)
              __hip_atomic_store(&part[(int64_t)m * a.N + n], acc[i][t][r], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
          }
    }
    // One level: the last workgroup of the chunk sums the splits in order.
    // Two levels (ngroups > 1, deep K): the splits form groups of gsize; the
    // last workgroup of a group sums the group's splits in order and
    // publishes that sum as plane splits + group through the same handshake
    // (one more arrival counter per group), and the last group sums the
    // group planes in order. Both trees are fixed, so results stay
    // deterministic. 256-column chunks only (the deep-K shapes that reach
    // 12 splits; 64-column chunks stay at 8 or fewer).
    const bool tree = CW == 256 && a.ngroups > 1;
    const int cpc = tree ? a.ngroups + 1 : 1;  // counters per chunk
    auto arrive = [&](int ci, int expect) -> bool {
      // Partials complete before the arrival (split-K handshake, awq_common.h).
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      uint32_t* ctr = &a.counters[(chunk * cpc + ci) * kCtrStride];
      if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_last = (prev == (uint32_t)(expect - 1)) ? 1 : 0;
      }
      __syncthreads();
      return *s_last != 0;
    };
    // Re-arm counter ci for the next call, after the sum (issued earlier, the
    // agent-scope store would sit ahead of the sum's loads in wave 0's
    // in-order vmcnt).
    auto rearm = [&](int ci) {
      if (tid == 0)
        __hip_atomic_store(&a.counters[(chunk * cpc + ci) * kCtrStride], 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    };
    // Sum planes p0 .. p0 + np - 1 of this chunk in order: 4 consecutive
    // columns per 16-byte load (N % 32 == 0 keeps them inside a row), kG
    // column groups per thread per round, kSB planes deep -- kG kSB loads in
    // flight, so most chunks take one round. Slots past the chunk, M or the
    // planes are loaded clamped and not used. The sums go to plane
    // out_plane (>= 0) or, with the bias and epilogue, to Y.
    const uint32_t sstride = (uint32_t)((int64_t)a.M * a.N * 4);
    constexpr int kG = 4, kSB = 4;
    constexpr int kTh = C::kThreads;
    const int total4 = a.M * kQuads;
    auto reduce = [&](int p0, int np, int out_plane) {
      for (int base = 0; base < total4; base += kTh * kG) {
        uint32_t off[kG];
        bool ok[kG];
        float v[kG][4];
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          const int e4 = base + g * kTh + tid;
          const int m = e4 / kQuads, n = chunk * CW + 4 * (e4 % kQuads);
          ok[g] = e4 < total4 && n < a.N;
          off[g] = (uint32_t)(((int64_t)min(m, a.M - 1) * a.N + min(n, a.N - 4)) * 4);
#pragma unroll
          for (int q = 0; q < 4; ++q) v[g][q] = 0.f;
        }
        for (int sp = 0; sp < np; sp += kSB) {
          float t[kG][kSB][4];
#pragma unroll
          for (int g = 0; g < kG; ++g)
#pragma unroll
            for (int b = 0; b < kSB; ++b) {
              const u32x4_t w4 = __builtin_amdgcn_raw_buffer_load_b128(
                  pres, off[g], (uint32_t)(p0 + min(sp + b, np - 1)) * sstride, kCachePolicySC1);
              // through plain scalars: __builtin_bit_cast of a vector element
              // directly reads the wrong element (hipcc 7.2)
              const uint32_t e0 = w4[0], e1 = w4[1], e2 = w4[2], e3 = w4[3];
              t[g][b][0] = __uint_as_float(e0);
              t[g][b][1] = __uint_as_float(e1);
              t[g][b][2] = __uint_as_float(e2);
              t[g][b][3] = __uint_as_float(e3);
            }
#pragma unroll
          for (int g = 0; g < kG; ++g)
#pragma unroll
            for (int b = 0; b < kSB; ++b) {
              const bool live = sp + b < np;
#pragma unroll
              for (int q = 0; q < 4; ++q) v[g][q] += live ? t[g][b][q] : 0.f;
            }
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          if (!ok[g]) continue;
          const int e4 = base + g * kTh + tid;
          const int m = e4 / kQuads, n = chunk * CW + 4 * (e4 % kQuads);
          if (out_plane >= 0) {
            const u32x4_t w4 = u32x4_t{__float_as_uint(v[g][0]), __float_as_uint(v[g][1]),
                                       __float_as_uint(v[g][2]), __float_as_uint(v[g][3])};
            __builtin_amdgcn_raw_buffer_store_b128(w4, pres, off[g], (uint32_t)out_plane * sstride,
                                                   kCachePolicySC1);
            continue;
          }
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (a.bias) v[g][q] += load_f32_any(a.bias, n + q, a.bt);
          // n % 4 == 0: the gate/up pairs are (q, q ^ 1) of this thread; plain
          // outputs leave as one 16- or 8-byte store of the 4 columns.
          if (ACT) {
            store_act_quad(a.y, a.yt, m, n, a.N, v[g][0], v[g][1], v[g][2], v[g][3]);
          } else if (a.yt == AWQ_F32) {
            *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.y) + (int64_t)m * a.N + n) =
                f32x4_t{v[g][0], v[g][1], v[g][2], v[g][3]};
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
    };
    if (tree) {
      const int grp = split / a.gsize, gbeg = grp * a.gsize, gn = min(a.gsize, a.splits - gbeg);
      if (!arrive(grp, gn)) return;
      reduce(gbeg, gn, a.splits + grp);
      rearm(grp);
      if (!arrive(a.ngroups, a.ngroups)) return;
      reduce(a.splits, a.ngroups, -1);
      rearm(a.ngroups);
    } else {
      // One level: the loop kept in this form (the shared sum above, used
      // here too, changed the 64-column kernels' register allocation and put
      // a vmcnt(0) wait before each partial store: 20-39 % slower at 64..128
      // rows).
      if (!arrive(0, a.splits)) return;
      // Sum the splits of this chunk in split order: 4 consecutive columns per
      // 16-byte load (N % 32 == 0 keeps them inside a row), kG column groups
      // per thread per round, kSB splits deep -- kG kSB loads in flight, so
      // most chunks take one round. Slots past the chunk, M or the splits are
      // loaded clamped and not used.
      for (int base = 0; base < total4; base += kTh * kG) {
        uint32_t off[kG];
        bool ok[kG];
        float v[kG][4];
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          const int e4 = base + g * kTh + tid;
          const int m = e4 / kQuads, n = chunk * CW + 4 * (e4 % kQuads);
          ok[g] = e4 < total4 && n < a.N;
          off[g] = (uint32_t)(((int64_t)min(m, a.M - 1) * a.N + min(n, a.N - 4)) * 4);
#pragma unroll
          for (int q = 0; q < 4; ++q) v[g][q] = 0.f;
        }
        for (int sp = 0; sp < a.splits; sp += kSB) {
          float t[kG][kSB][4];
#pragma unroll
          for (int g = 0; g < kG; ++g)
#pragma unroll
            for (int b = 0; b < kSB; ++b) {
              const u32x4_t w4 = __builtin_amdgcn_raw_buffer_load_b128(
                  pres, off[g], (uint32_t)min(sp + b, a.splits - 1) * sstride, kCachePolicySC1);
              // through plain scalars: __builtin_bit_cast of a vector element
              // directly reads the wrong element (hipcc 7.2)
              const uint32_t e0 = w4[0], e1 = w4[1], e2 = w4[2], e3 = w4[3];
              t[g][b][0] = __uint_as_float(e0);
              t[g][b][1] = __uint_as_float(e1);
              t[g][b][2] = __uint_as_float(e2);
              t[g][b][3] = __uint_as_float(e3);
            }
#pragma unroll
          for (int g = 0; g < kG; ++g)
#pragma unroll
            for (int b = 0; b < kSB; ++b) {
              const bool live = sp + b < a.splits;
#pragma unroll
              for (int q = 0; q < 4; ++q) v[g][q] += live ? t[g][b][q] : 0.f;
            }
        }
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          if (!ok[g]) continue;
          const int e4 = base + g * kTh + tid;
          const int m = e4 / kQuads, n = chunk * CW + 4 * (e4 % kQuads);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (a.bias) v[g][q] += load_f32_any(a.bias, n + q, a.bt);
          // n % 4 == 0: the gate/up pairs are (q, q ^ 1) of this thread; plain
          // outputs leave as one 16- or 8-byte store of the 4 columns.
          if (ACT) {
            store_act_quad(a.y, a.yt, m, n, a.N, v[g][0], v[g][1], v[g][2], v[g][3]);
          } else if (a.yt == AWQ_F32) {
            *reinterpret_cast<f32x4_t*>(static_cast<float*>(a.y) + (int64_t)m * a.N + n) =
                f32x4_t{v[g][0], v[g][1], v[g][2], v[g][3]};
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
      rearm(0);
    }
    return;
  }
  if constexpr (ACT) {
    // AutoAWQ order: packed lanes c and c + 4 of a pack are columns 2 j and
    // 2 j + 1 -- a gate/up pair: lanes lj (c < 4, lj < 8) and lj ^ 8, same tile.
    const bool even = (lj & 8) == 0;
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      const int n = nbase + colt[t];
      const float b0 = (a.bias && n < a.N) ? load_f32_any(a.bias, n, a.bt) : 0.f;
      const float b1 = (a.bias && n + 1 < a.N) ? load_f32_any(a.bias, n + 1, a.bt) : 0.f;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * i + 4 * lg + r;
          const float g = acc[i][t][r];
          const float u = __shfl_xor(g, 8, 64);
          if (even && m < a.M && n < a.N) store_out(a.y, a.yt, 1, m, n, a.N, g + b0, u + b1);
        }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < kT; ++t) {
    const int n = nbase + colt[t];
    if (n >= a.N) continue;
    const float b = a.bias ? load_f32_any(a.bias, n, a.bt) : 0.f;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * i + 4 * lg + r;
        if (m < a.M) store_f32_any(a.y, (int64_t)m * a.N + n, a.yt, acc[i][t][r] + b);
      }
  }
}

template <int MT, bool BF, int CW, int WV>
void launch_mt(const GemmProblem& p) {
  using C = Chunk<CW, WV>;
  const size_t smem = (size_t)skinny_smem_bytes<MT, CW>();
  const int chunks = (int)((p.N + CW - 1) / CW);
  const int total_steps = (int)(p.K / kStep);
  // About one workgroup per CU, each run at least 16 steps and touching at
  // most kMaxGroups groups; fp32 partials (splits x M x N x 4 bytes) at most
  // the packed weights (K x N / 2 bytes), and at most 1024 partial rows per
  // chunk for the last workgroup to sum (splits x M): beyond those the split-K
  // traffic and the serial reduction cost more than the extra workgroups gain
  // (measured on 4096..14336-deep, 4096..28672-wide problems, 32..128 rows).
  // 64-column chunks of up to 64 rows fit two workgroups per CU (LDS and
  // registers), and the second hides the first's latencies: twice the splits
  // (4096 -> 4096 at M = 17 / 32 / 64: 13.6 / 13.9 / 15.4 -> 11.4 / 11.5 /
  // 14.9 us; 14336 -> 4096 at M = 64: 36.2 -> 31.2; not at M = 128, where
  // only one fits: 21.4 -> 25.8).
  const int per_cu = (CW == 64 && MT <= 4) ? 2 : 1;
  int splits = (int)std::max<int64_t>(1, per_cu * device_cus() / chunks);
  // A grid that those limits would leave under one workgroup per CU (few
  // chunks) takes runs down to 8 steps and partials up to twice the packed
  // weights instead (4096 -> 1024 at M = 64: 8 -> 16 splits, 10.6 -> 10.0 us).
  const bool few = (int64_t)chunks * std::min(splits, std::max(1, total_steps / 16)) < device_cus();
  splits = std::min(splits, std::max(1, total_steps / (few ? 8 : 16)));
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, p.K / ((few ? 4 : 8) * p.rows)));
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, 1024 / p.rows));
  if (int v = tuning(kTuneSkinnySplits, 0); v >= 1) splits = std::min(v, total_steps);
  int sps = (total_steps + splits - 1) / splits;
  while ((int64_t)sps * kStep / p.group + 2 > C::kMaxGroups) {
    ++splits;
    sps = (total_steps + splits - 1) / splits;
  }
  splits = (total_steps + sps - 1) / sps;
  // (planes, with the two-level sum's extra ones, below 4 GB: splits + 2 sqrt(splits) < 2 splits)
  while (splits > 1 && (int64_t)2 * splits * p.rows * p.N * 4 >= (1ll << 32)) {
    --splits;
    sps = (total_steps + splits - 1) / splits;
    splits = (total_steps + sps - 1) / sps;
  }
  SkinnyArgs a{};
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
  a.splits = splits;
  a.steps_per_split = sps;
  a.seq = p.order == AWQ_ORDER_SEQUENTIAL ? 1 : 0;
  a.chunks = chunks;
  // XCD mapping only where grid.x keeps the XCD of a workgroup independent of
  // its split (chunks % 8 == 0) and each XCD's run covers whole 128-byte lines.
  a.xcd_chunks = (CW == 64 && chunks % 8 == 0 && (chunks / 8) % 4 == 0) ? chunks : 0;
  a.gsize = splits;
  a.ngroups = 1;
  if (splits > 1) {
    // Two-level split sum (groups of g splits, g the smallest with g * g >=
    // splits) on deep K: 12 or more splits, 256-column chunks. Measured (us,
    // one level / two):
    // 14336 -> 4096 at M = 17 / 24 / 64 (16 splits) 20.8 / 21.6 / 29.6 ->
    // 20.2 / 20.7 / 27.5; 28672 -> 4096 at M = 64 41.5 -> 40.6. (More
    // splits stay slower with it: 20..32 splits at 14336 -> 4096, M = 64,
    // 37..43 us.) AWQ_SKINNY_TREE=0 / 1 forces one level / two (3 or more
    // splits).
    const int force = tuning(kTuneSkinnyTree, -1);
    if (CW == 256 && force != 0 && splits >= 3 && (force == 1 || splits >= 12)) {
      int g = 1;
      while (g * g < splits) ++g;
      const int ng = (splits + g - 1) / g;
      if (ng > 1) {
        a.gsize = g;
        a.ngroups = ng;
      }
    }
    const int planes = splits + (a.ngroups > 1 ? a.ngroups : 0);
    const int cpc = a.ngroups > 1 ? a.ngroups + 1 : 1;
    a.counters = static_cast<uint32_t*>(
        ws_get(p, (size_t)chunks * cpc * kCtrStride * sizeof(uint32_t), kWsCounters));
    a.partial = static_cast<float*>(
        ws_get(p, (size_t)planes * p.rows * p.N * sizeof(float), kWsPartials));
  }
  ensure_dyn_smem((const void*)skinny_kernel<MT, false, BF, CW, WV>, (int)smem, "hipFuncSetAttribute(skinny)");
  ensure_dyn_smem((const void*)skinny_kernel<MT, true, BF, CW, WV>, (int)smem, "hipFuncSetAttribute(skinny)");
  if (p.act)
    hipLaunchKernelGGL((skinny_kernel<MT, true, BF, CW, WV>), dim3(chunks, splits), dim3(C::kThreads), smem, p.stream,
                       a);
  else
    hipLaunchKernelGGL((skinny_kernel<MT, false, BF, CW, WV>), dim3(chunks, splits), dim3(C::kThreads), smem,
                       p.stream, a);
  check_hip(hipGetLastError(), "skinny kernel launch");
}

template <bool BF, int CW, int WV>
void launch_rows_cw(const GemmProblem& p) {
  // One 16-row tile up to 16 rows (against two, half of them padding: 9..16
  // rows of f16 3-6 % faster at K 4096..28672, N 1024..28672, e.g.
  // 4096 -> 14336 at M = 16 18.6 -> 17.6 us, 8192 -> 28672 55.3 -> 51.8).
  if (p.rows <= 16) return launch_mt<1, BF, CW, WV>(p);
  if (p.rows <= 32) return launch_mt<2, BF, CW, WV>(p);
  if (p.rows <= 48) return launch_mt<3, BF, CW, WV>(p);
  if (p.rows <= 64) return launch_mt<4, BF, CW, WV>(p);
  // 5 and 7 tiles for 65..80 and 97..112 rows (against 6 and 8: 2-5 %
  // faster, e.g. 4096 -> 14336 at M = 72 / 100 27.6 / 32.1 -> 26.4 / 31.0 us).
  if (p.rows <= 80) return launch_mt<5, BF, CW, WV>(p);
  if (p.rows <= 96) return launch_mt<6, BF, CW, WV>(p);
  if (p.rows <= 112) return launch_mt<7, BF, CW, WV>(p);
  return launch_mt<8, BF, CW, WV>(p);
}

template <bool BF>
void launch_rows(const GemmProblem& p) {
  // Chunk width: 256 columns on wide outputs, 64 below 6144 columns. Measured
  // (us, f16, g128, 64 / 256 columns / large tiles): 4096 -> 4096 at M = 17 /
  // 64 / 128: 13.6 / 16.0 / 22.0 (15.0 / 22.3 / 36.4; 18.9 / 21.6 / 24.6);
  // 4096 -> 1024 at M = 32 / 64: 10.0 / 11.5 (15.2 / 20.6; 17.9 / 20.1); but
  // 4096 -> 14336 at M = 64: 40.0 against 28.9 -- with narrow chunks every
  // workgroup streams all of X, and wide outputs need no K splits to fill
  // the CUs anyway. AWQ_SKINNY_COLS=64/256 forces the width.
  const int cols = tuning(kTuneSkinnyCols, 0);
  // 256 columns over 8 waves: on 4 waves of 64 columns (half the X reads
  // from LDS, one wave per SIMD) 4096 -> 14336 at M = 64 measured 33.9
  // against 26.1 us, the LDS and dependency latencies no longer hidden.
  // Very deep K also favours the wide chunks (their K splits keep long
  // runs): 14336 -> 4096 at M = 17 / 32 / 64 22.5 / 22.8 / 30.8 -> 20.7 /
  // 21.4 / 29.9 us, 28672 -> 4096 at M = 64 53.0 -> 41.7; not at 33..48 rows
  // (three row tiles: 26.8 -> 28.6) or at K = 8192 / 11008 (the 64-column
  // chunks stay 5-19 % ahead).
  const bool deep = p.K >= 14336 && (p.rows <= 32 || p.rows > 48);
  if (cols == 256 || (cols != 64 && (p.N >= 6144 || deep))) return launch_rows_cw<BF, 256, 8>(p);
  return launch_rows_cw<BF, 64, 4>(p);
}

}  // namespace

bool skinny_ok(const GemmProblem& p) {
  // Where it beats the split-K tiles of the large-tile kernel (measured at
  // K 4096..28672, N 1024..28672, 17..128 rows): wide outputs (N >= 6144,
  // 256-column chunks: 1.1-2.7x), and narrower ones (64-column chunks) up to
  // 128 rows when K <= 8192 and up to 64 rows beyond. 9..16 rows of f16/bf16
  // also come here instead of the decode kernels' 16-row tile (f16 0-28 %
  // faster at K 4096..28672, N 1024..28672; bf16 -8..+20 %). AWQ_SKINNY=0/1
  // forces the choice.
  const int force = tuning(kTuneSkinny, -1);
  // Narrower outputs run 64-column chunks (see launch_rows), which beat the
  // split-K tiles up to 128 rows when K <= 8192 and up to 64 rows beyond
  // (14336 -> 4096 at M = 64: 37.7 against 37.6 us; at M = 128 51.3 against
  // 39.5).
  const bool wins = p.N >= 6144 || (p.N >= 1024 && (p.K <= 8192 || p.rows <= 64));
  if (force == 0 || (force != 1 && !wins)) return false;
  // bf16 activations need 16-bit scales (z s exact in f32, see the kernel).
  const bool types = p.xt == AWQ_F16 || (p.xt == AWQ_BF16 && p.st != AWQ_F32);
  return types && p.rows > 8 && p.rows <= 128 && p.K % kStep == 0 && p.group % kStep == 0 &&
         p.N % 32 == 0 && p.K * (p.N / 8) * 4 < (1ll << 32) && p.rows * p.K * 2 < (1ll << 32) &&
         (p.K / p.group) * p.N * 4 < (1ll << 32);
}

void launch_skinny(const GemmProblem& p) {
  if (p.xt == AWQ_BF16) return launch_rows<true>(p);
  launch_rows<false>(p);
}

}  // namespace cube_awq
