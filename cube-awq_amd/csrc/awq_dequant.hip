// awq_dequant.hip -- standalone AWQ dequantize for gfx950 (pure streaming).
//
// Computes out[k, n] = (q - z) * s for a [K, N] output, the operation of the
// reference's dequantize_awq_symmetric (src/kernel/awq_kernel.rs:23-61):
// F(q) - F(z) is exact (both are integers in [0, 15]), so evaluating it in
// f32 and multiplying once by the f32-widened scale gives the same single
// rounding as the reference's (F(q) - F(z)) * s in F, bit for bit, whether the
// output is f32, f16 or bf16 (the f32 product of a <=4-bit integer and an
// f16/bf16 scale is exact; the cast to the output type is its one rounding).
//
// HBM layout and work split. The output is written as a flat stream: one
// thread item is 16 bytes of consecutive output columns (4 f32 or 8 f16/bf16)
// of R consecutive rows of the same quantisation group, so every wave store
// instruction writes 1 KiB of contiguous output, every packed word is read by
// adjacent lanes in one coalesced load, and the group's zero word and scales
// are loaded once per R rows. Bytes per output element (f32 out, g >= 4):
// 4 written + 0.5 packed weight + (0.5 + 4) / g zeros and scales.
#include "awq_common.h"

namespace cube_awq {
namespace {

template <bool kSeq>
__device__ __forceinline__ uint32_t nibble(uint32_t w, int col) {
  const int lane = kSeq ? col : awq_lane_of_col(col);
  return (w >> (4 * lane)) & 0xFu;
}

template <typename S, int V>
__device__ __forceinline__ void load_scales(const S* p, float (&s)[V]) {
  // V consecutive scales starting at a V-aligned column; read in 16-byte (or
  // smaller) chunks so no access assumes more than 16-byte alignment.
  constexpr int kBytes = V * (int)sizeof(S);
  if constexpr (kBytes >= 16) {
    constexpr int kPer = 16 / (int)sizeof(S);
#pragma unroll
    for (int c = 0; c < V / kPer; ++c) {
      typedef S chunk_t __attribute__((ext_vector_type(kPer)));
      chunk_t v = *reinterpret_cast<const chunk_t*>(p + c * kPer);
#pragma unroll
      for (int j = 0; j < kPer; ++j) s[c * kPer + j] = to_f32(v[j]);
    }
  } else {
    typedef S chunk_t __attribute__((ext_vector_type(V)));
    chunk_t v = *reinterpret_cast<const chunk_t*>(p);
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] = to_f32(v[j]);
  }
}

template <typename O, int V, bool kNT>
__device__ __forceinline__ void store_out(O* p, const float (&v)[V]) {
  typedef O vec_t __attribute__((ext_vector_type(V)));
  vec_t o;
#pragma unroll
  for (int j = 0; j < V; ++j) o[j] = from_f32<O>(v[j]);
  if constexpr (kNT) {
    __builtin_nontemporal_store(o, reinterpret_cast<vec_t*>(p));
  } else {
    *reinterpret_cast<vec_t*>(p) = o;
  }
}

template <bool kSeq, int ST, int OT, int R, bool kNT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ qweight,
                                                      const uint32_t* __restrict__ qzeros,
                                                      const void* __restrict__ scales_v,
                                                      void* __restrict__ out_v, uint32_t N,
                                                      uint32_t group, uint32_t items_per_row,
                                                      uint32_t n_items) {
  using S = typename Elem<ST>::type;
  using O = typename Elem<OT>::type;
  constexpr int V = 16 / (int)sizeof(O);  // output columns per item
  const S* __restrict__ scales = static_cast<const S*>(scales_v);
  O* __restrict__ out = static_cast<O*>(out_v);
  const uint32_t np = N / 8;

  for (uint32_t it = blockIdx.x * 256u + threadIdx.x; it < n_items; it += gridDim.x * 256u) {
    const uint32_t rb = it / items_per_row;
    const uint32_t ci = it - rb * items_per_row;
    const uint32_t k0 = rb * R;
    const uint32_t col0 = ci * V;
    const uint32_t pack = col0 / 8;
    const int cin = (int)(col0 % 8);  // 0 or 4 for f32 output, 0 otherwise
    const uint32_t grp = k0 / group;

    const uint32_t zw = qzeros[(size_t)grp * np + pack];
    float s[V];
    load_scales<S, V>(scales + (size_t)grp * N + col0, s);
    int z[V];
#pragma unroll
    for (int j = 0; j < V; ++j) z[j] = (int)nibble<kSeq>(zw, cin + j);

    uint32_t w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = qweight[(size_t)(k0 + r) * np + pack];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float o[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        // (q - z) is an exact small integer; one rounding in the multiply.
        o[j] = (float)((int)nibble<kSeq>(w[r], cin + j) - z[j]) * s[j];
      }
      store_out<O, V, kNT>(out + (size_t)(k0 + r) * N + col0, o);
    }
  }
}

template <bool kSeq, int ST, int OT>
void launch_typed(const DequantProblem& p) {
  constexpr int V = 16 / dtype_size_ct(OT);
  // 4 rows per item when they always share a group and every item is whole;
  // a partial last row (tail_cols) is walked one row per item.
  const int R = (p.group % 4 == 0 && p.K % 4 == 0 && p.tail_cols == 0) ? 4 : 1;
  const uint32_t items_per_row = (uint32_t)(p.N / V);
  const uint64_t n_items64 = (uint64_t)(p.K / R) * items_per_row + (uint64_t)(p.tail_cols / V);
  AWQ_ASSERT(n_items64 < (1ull << 32) && (uint64_t)(p.K + 1) * (uint64_t)p.N < (1ull << 40),
             "dequantize: tensor too large for one launch");
  const uint32_t n_items = (uint32_t)n_items64;
  if (n_items == 0) return;
  uint32_t blocks = (n_items + 255u) / 256u;
  const uint32_t max_blocks = 256u * 16u;  // 256 CUs x 16 resident blocks
  if (blocks > max_blocks) blocks = max_blocks;
  // Nontemporal stores: the output is written once and is larger than the
  // caches; streaming it past them measured 5.7 -> 6.9 TB/s at 14336 x 4096.
  if (R == 4) {
    hipLaunchKernelGGL((dequant_kernel<kSeq, ST, OT, 4, true>), dim3(blocks), dim3(256), 0,
                       p.stream, p.qweight, p.qzeros, p.scales, p.out, (uint32_t)p.N,
                       (uint32_t)p.group, items_per_row, n_items);
  } else {
    hipLaunchKernelGGL((dequant_kernel<kSeq, ST, OT, 1, true>), dim3(blocks), dim3(256), 0,
                       p.stream, p.qweight, p.qzeros, p.scales, p.out, (uint32_t)p.N,
                       (uint32_t)p.group, items_per_row, n_items);
  }
  check_hip(hipGetLastError(), "dequantize kernel launch");
}

template <bool kSeq, int ST>
void launch_out(const DequantProblem& p) {
  switch (p.ot) {
    case AWQ_F32: launch_typed<kSeq, ST, AWQ_F32>(p); break;
    case AWQ_F16: launch_typed<kSeq, ST, AWQ_F16>(p); break;
    default: launch_typed<kSeq, ST, AWQ_BF16>(p); break;
  }
}

template <bool kSeq>
void launch_order(const DequantProblem& p) {
  switch (p.st) {
    case AWQ_F32: launch_out<kSeq, AWQ_F32>(p); break;
    case AWQ_F16: launch_out<kSeq, AWQ_F16>(p); break;
    default: launch_out<kSeq, AWQ_BF16>(p); break;
  }
}

}  // namespace

void launch_dequant(const DequantProblem& p) {
  if (p.order == AWQ_ORDER_SEQUENTIAL) launch_order<true>(p);
  else launch_order<false>(p);
}

}  // namespace cube_awq
