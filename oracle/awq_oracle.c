/*
 * awq_oracle.c -- CPU restatement of the reference's AWQ algorithms.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker (or the reported CPU baseline), never as a product path.
 * The product library (cube-awq_amd/csrc) does not link or call it.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the reference repository root). How each one is pinned:
 *   awqo_nibble_seq / awqo_dequant_f32(order=SEQ): golden vectors from the
 *     reference's own dequantize tests (tests/awq_test.rs:117-221,
 *     src/modules/awq_dequantize.rs:133-237) plus an exhaustive sweep of all
 *     256 (q, z) pairs against the closed form (q - z) * s.
 *   awqo_nibble_awq: the reference's pack_i4/AWQ_ORDER test helper
 *     (src/modules/awq_gemm.rs:248-282) round trip and the module decode
 *     golden case (src/modules/awq_gemm.rs:517-559).
 *   awqo_gemm_f32 / awqo_gemm_f64: the closed-form kernel cases of
 *     src/kernel/awq_kernel_gemm.rs:1125-1391 (exact integers), brute force
 *     against an independent exact-rational evaluation on tiny shapes, and
 *     the module golden cases.
 * Build: cc -O2 -fPIC -shared -ffp-contract=off -fopenmp (oracle/Makefile).
 * -ffp-contract=off keeps `acc += x * w` as a rounded multiply followed by a
 * rounded add, which is what the reference's CPU test loops compute.
 */
#include <stdint.h>
#include <stddef.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define AWQO_ORDER_AUTOAWQ 0
#define AWQO_ORDER_SEQUENTIAL 1

/* Sequential nibble order: column c of a pack is bits 4c..4c+3.
 * src/kernel/awq_kernel.rs:8-19 (unpack_u32: `(packed_value >> idx*4) & 0x0f`). */
uint32_t awqo_nibble_seq(uint32_t word, int col) { return (word >> (4 * col)) & 0xFu; }

/* AutoAWQ order: logical column c sits in packed lane [0,4,1,5,2,6,3,7][c].
 * src/kernel/awq_kernel_gemm.rs:10-30 (unpack_u32_to_i4_0_4 shifts {0,16,4,20},
 * unpack_u32_to_i4_4_8 shifts {8,24,12,28}) and the test-side
 * AWQ_REVERSE_ORDER at src/kernel/awq_kernel_gemm.rs:809. */
uint32_t awqo_nibble_awq(uint32_t word, int col) {
  static const int lane_of_col[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  return (word >> (4 * lane_of_col[col & 7])) & 0xFu;
}

static inline uint32_t nib(uint32_t word, int col, int order) {
  return order == AWQO_ORDER_SEQUENTIAL ? awqo_nibble_seq(word, col) : awqo_nibble_awq(word, col);
}

/* Dequantize one element as the reference does in F = f32:
 * (F::cast_from(q) - F::cast_from(z)) * s  -- src/kernel/awq_kernel.rs:52-59
 * (sequential order) and src/kernel/awq_kernel_gemm.rs:355-362 (AWQ order). */
static inline float deq1(uint32_t q, uint32_t z, float s) {
  float d = (float)q - (float)z; /* exact: both are integers in [0, 15] */
  return d * s;                  /* the one rounding */
}

/* out[k, n] for k < K, n < N; scales is [K/g, N] f32.
 * Index math of src/kernel/awq_kernel.rs:41-59: row = k, group = k / g,
 * pack = n / 8, column-in-pack = n % 8. */
void awqo_dequant_f32(const uint32_t* qweight, const uint32_t* qzeros, const float* scales,
                      float* out, int64_t K, int64_t N, int64_t g, int order) {
  const int64_t np = N / 8;
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < K; ++k) {
    const int64_t grp = k / g;
    for (int64_t n = 0; n < N; ++n) {
      uint32_t q = nib(qweight[k * np + n / 8], (int)(n % 8), order);
      uint32_t z = nib(qzeros[grp * np + n / 8], (int)(n % 8), order);
      out[k * N + n] = deq1(q, z, scales[grp * N + n]);
    }
  }
}

/* y[m, n] = sum_k x[m, k] * w[k, n] in f32, one accumulator per output, k in
 * increasing order, multiply and add rounded separately; bias (nullable) added
 * afterwards. Rows m >= m_valid are not written.
 * Restates the per-thread loop of gemm_awq / gemm_awq_decode
 * (src/kernel/awq_kernel_gemm.rs:346-399, :553-606: each output owned by one
 * thread, acc += a_k * deq_k sequentially over K) and the CPU references
 * src/kernel/awq_kernel_gemm.rs:793-829, src/modules/awq_gemm.rs:322-341;
 * bias after the GEMM as src/modules/awq_gemm.rs:225-228. */
void awqo_gemm_f32(const float* x, const uint32_t* qweight, const uint32_t* qzeros,
                   const float* scales, const float* bias, float* y, int64_t M, int64_t K,
                   int64_t N, int64_t g, int64_t m_valid, int order) {
  const int64_t np = N / 8;
  if (m_valid > M) m_valid = M;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < m_valid; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      const int col = (int)(n % 8);
      for (int64_t k = 0; k < K; ++k) {
        const int64_t grp = k / g;
        uint32_t q = nib(qweight[k * np + n / 8], col, order);
        uint32_t z = nib(qzeros[grp * np + n / 8], col, order);
        float w = deq1(q, z, scales[grp * N + n]);
        acc = acc + x[m * K + k] * w; /* not contracted: -ffp-contract=off */
      }
      if (bias) acc = acc + bias[n];
      y[m * N + n] = acc;
    }
  }
}

/* Same sum with f64 products and accumulation (the dequantized weight is the
 * exact f32 (q - z) * s of the reference, widened): the high-precision truth
 * against which the fp32 and fp16/bf16 paths' relative L2 error is measured. */
void awqo_gemm_f64(const float* x, const uint32_t* qweight, const uint32_t* qzeros,
                   const float* scales, const float* bias, double* y, int64_t M, int64_t K,
                   int64_t N, int64_t g, int order) {
  const int64_t np = N / 8;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      const int col = (int)(n % 8);
      for (int64_t k = 0; k < K; ++k) {
        const int64_t grp = k / g;
        uint32_t q = nib(qweight[k * np + n / 8], col, order);
        uint32_t z = nib(qzeros[grp * np + n / 8], col, order);
        double w = (double)deq1(q, z, scales[grp * N + n]);
        acc += (double)x[m * K + k] * w;
      }
      if (bias) acc += (double)bias[n];
      y[m * N + n] = acc;
    }
  }
}

/* Threads OpenMP will use for the parallel loops above (reported as the CPU
 * baseline's core count). */
int awqo_num_threads(void) {
  int t = 1;
#pragma omp parallel
  {
#pragma omp single
    {
#ifdef _OPENMP
      t = omp_get_num_threads();
#endif
    }
  }
  return t;
}
