/*
 * awq.h -- C ABI of libcube_awq_gfx950.so, the MI355X (gfx950) AWQ INT4
 * dequant-GEMM / dequantize library.
 *
 * Every pointer named qweight/qzeros/scales/x/y/out/bias is a DEVICE pointer to
 * caller-owned, row-major, contiguous memory. Calls are stream-ordered and
 * asynchronous: they enqueue work on `stream` (a hipStream_t passed as void*,
 * NULL = the legacy default stream) and never synchronise the host.
 *
 * Workspace. The GEMM entry points allocate device memory in one case: a
 * launch that splits K over several workgroups keeps fp32 partial sums
 * (splits x rows x N x 4 bytes) and arrival counters (<= 256 bytes per
 * column chunk or tile) in a workspace owned by the library, one per
 * (device, stream). Routes that split K: the decode kernels (M <= 16) when K
 * spans more than one workgroup's rows, the 9..128-row f16/bf16 kernel, the
 * large-tile kernel when it has few tiles (about M <= 1024), and fp32
 * activations run as 16-row slices. The workspace is allocated on first need
 * and grown when a call needs more; a superseded buffer is never freed (it is
 * retired and kept until the process ends), so work queued or captured
 * earlier stays valid. Growth during stream capture is refused with an
 * error: before capturing, make one eager call on the capture stream with
 * the largest shape the graph will hold. A graph keeps the workspace its
 * capture stream had: replays of graphs captured on one stream, and eager
 * calls on that stream, share it and must not overlap in time (replay them
 * on the capture stream, or order them with events).
 *
 * Return value: 0 on success, a negative AWQ_ERR_* code otherwise. On error the
 * thread-local string returned by awq_last_error() holds the message; for shape
 * and dtype problems it is the exact assertion text the reference panics with,
 * so a Rust wrapper can do `panic!("{}", awq_last_error())` and keep the
 * reference's `#[should_panic(expected = ...)]` behaviour.
 *
 * Layout (AutoAWQ, reference README.md:60-70):
 *   qweight [K, N/8] u32/i32 : 8 x 4-bit weights per word, one K row, 8 N columns
 *   qzeros  [K/g, N/8] u32/i32
 *   scales  [K/g, N]  f32/f16/bf16
 * Nibble orders:
 *   AWQ_ORDER_AUTOAWQ    packed lane p (bits 4p..4p+3) holds column [0,2,4,6,1,3,5,7][p]
 *                        (reference src/kernel/awq_kernel_gemm.rs:7-30, used by the GEMM)
 *   AWQ_ORDER_SEQUENTIAL column c is bits 4c..4c+3
 *                        (reference src/kernel/awq_kernel.rs:8-19, used by dequantize)
 */
#ifndef CUBE_AWQ_AWQ_H
#define CUBE_AWQ_AWQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. F32/F16/BF16 for activations, scales, outputs and bias;
 * U32/I32 for packed tensors. I16/I64 exist only so a caller can describe a
 * wrongly-typed packed tensor and get the reference's rejection message. */
typedef enum {
  AWQ_F32 = 0,
  AWQ_F16 = 1,
  AWQ_BF16 = 2,
  AWQ_U32 = 3,
  AWQ_I32 = 4,
  AWQ_I16 = 5,
  AWQ_I64 = 6
} awq_dtype;

typedef enum { AWQ_ORDER_AUTOAWQ = 0, AWQ_ORDER_SEQUENTIAL = 1 } awq_order;

enum {
  AWQ_OK = 0,
  AWQ_ERR_INVALID = -1, /* a constraint / shape / dtype assertion failed     */
  AWQ_ERR_HIP = -2,     /* a HIP runtime call or kernel launch failed         */
  AWQ_ERR_UNSUPPORTED = -3
};

/* Mirror of the reference's ShapeConfig (src/kernel/awq_kernel_gemm.rs:35-79).
 * tile_m/tile_n/inner_k/line_size are validated exactly as the reference does
 * (they decide which shapes are accepted) but do not pick the kernels' own
 * tiling, which is internal. m_valid: rows >= m_valid are neither computed nor
 * written. */
typedef struct {
  int64_t m, k, n;
  int64_t tile_m, tile_n, inner_k;
  int64_t line_size;
  int64_t m_valid;
} awq_shape_config;

/* Mirror of CubeCL's TensorHandleRef as the reference's launchers read it:
 * device pointer, row-major contiguous shape, element size in bytes, dtype. */
typedef struct {
  const void* data;
  const int64_t* shape;
  int32_t rank;
  int32_t elem_size;
  int32_t dtype; /* awq_dtype */
} awq_tensor_ref;

/* ShapeConfig::new(m, n, k, m_tile_size, n_tile_size, inner_k_size)
 * (src/kernel/awq_kernel_gemm.rs:48-57; note the m, n, k argument order). */
awq_shape_config awq_shape_config_new(int64_t m, int64_t n, int64_t k, int64_t m_tile_size,
                                      int64_t n_tile_size, int64_t inner_k_size);
/* ShapeConfig::new_with_valid_m (src/kernel/awq_kernel_gemm.rs:59-78). */
awq_shape_config awq_shape_config_new_with_valid_m(int64_t m, int64_t n, int64_t k,
                                                   int64_t m_tile_size, int64_t n_tile_size,
                                                   int64_t inner_k_size, int64_t m_valid);

/* validate_launch_params / validate_decode_launch_params
 * (src/kernel/awq_kernel_gemm.rs:89-171). Host only; no GPU needed. */
int awq_validate_launch_params(const awq_shape_config* shape, int64_t group_size);
int awq_validate_decode_launch_params(const awq_shape_config* shape, int64_t group_size);

/* awq_gemm_linear (src/kernel/awq_kernel_gemm.rs:626-771):
 *   output[M, N] = input[M, K] . dequant(qweight, qzeros, scales)  (AutoAWQ order)
 * with M = numel(input) / K. Same rank/shape assertions and messages, the same
 * m_valid rule (:675-690) and the same decode/prefill split: M <= 8 runs the
 * dequant-GEMV, M > 8 the MFMA GEMM. input/output dtype: F32, F16 or BF16;
 * scales: F32, F16 or BF16 (may differ from input). F32 input computes in
 * fp32; F16/BF16 input runs fp16/bf16 MFMA with fp32 accumulation. */
int awq_gemm_linear(const awq_tensor_ref* input, const awq_tensor_ref* qweight,
                    const awq_tensor_ref* qzeros, const awq_tensor_ref* scales,
                    const awq_tensor_ref* output, const awq_shape_config* shape,
                    int64_t group_size, void* stream);

/* dequantize_native (src/kernel/awq_kernel.rs:63-111): sequential nibble order,
 * out[k, n] = (F(q) - F(z)) * s, bit-exact. Rejects non-4-byte packed tensors
 * and out_width % 32 != 0 with the reference's messages. */
int awq_dequantize_native(const awq_tensor_ref* q_weight, const awq_tensor_ref* q_zeros,
                          const awq_tensor_ref* q_scales, const awq_tensor_ref* output,
                          int64_t group_size, void* stream);

/* Pointer-level fused linear with the module's constraints
 * (AWQGEMMLinear::forward, src/modules/awq_gemm.rs:146-232): tile_m/tile_n
 * picked by awq_select_tile_m/n, INNER_K = 64, so K % 64, N % 32, g % 64,
 * g >= 64. bias (nullable, [N], dtype b_t) is added in the epilogue before the
 * cast to y_t; the reference adds it afterwards as a separate op (:225-228). */
int awq_gemm(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
             const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
             int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size, void* stream);

/* awq_gemm with the nibble order of qweight/qzeros as a parameter.
 * AWQ_ORDER_AUTOAWQ is awq_gemm. AWQ_ORDER_SEQUENTIAL is AWQLinear's layout:
 * the reference's AWQLinear::forward (src/modules/awq_dequantize.rs:74-108)
 * dequantizes in that order (src/kernel/awq_kernel.rs:23-61) and then runs a
 * matmul; here the two are one fused launch, with scales in the input dtype
 * (the reference's single F). Same shape constraints as awq_gemm. */
int awq_gemm_ordered(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
                     const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
                     int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size,
                     int32_t order, void* stream);

/* awq_gemm without any device allocation, for callers that cannot allocate
 * (code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc). No counterpart in the reference (whose launcher allocates
 * nothing because it never splits K). Same arguments, constraints, kernels
 * and results as awq_gemm; split-K partial sums and arrival counters, and
 * the f16 hi/lo split of fp32 activations that the fp32 prefill makes, go
 * to a static scratch array in device memory (128 MiB per GPU: 1 MiB of
 * counters, 63 MiB of fp32 partials, 64 MiB for the split activations,
 * M x K x 4 + M x 4 bytes; held by every GPU the library runs on until the
 * process ends) instead of the per-stream workspace. A call whose route
 * needs more than a region holds (partials: splits x rows x N x 4 bytes)
 * fails with AWQ_ERR_INVALID before launching anything. The first call on a
 * device looks the array up (hipGetSymbolAddress) and clears its counters
 * with a kernel on `stream`: make that call outside graph capture. Every
 * call on one GPU shares that GPU's scratch: calls that overlap in time on
 * one GPU (other streams, concurrent graph replays) race and must be
 * serialised by the caller. */
int awq_gemm_noalloc(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
                     const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
                     int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size,
                     void* stream);

/* Fused gate/up projection with its activation in the GEMM epilogue: the
 * weights hold the gate and up projections interleaved by column (column 2j
 * of qweight/qzeros/scales/bias is gate column j, column 2j + 1 is up column
 * j; N = 2 x the intermediate width, N % 64 == 0) in AutoAWQ nibble order,
 * and y [M, N/2] receives SiLU(x.Wg + bg) * (x.Wu + bu), SiLU(g) = g / (1 +
 * exp(-g)). No reference counterpart: its GEMM path has no activation and
 * adds the bias as a separate op (src/modules/awq_gemm.rs:225-228), so gate,
 * up and SiLU * up there are separate launches. Otherwise the constraints and
 * dispatch of awq_gemm. */
int awq_gemm_silu_mul(const void* x, int32_t x_t, const uint32_t* qweight, const uint32_t* qzeros,
                      const void* scales, int32_t s_t, const void* bias, int32_t b_t, void* y,
                      int32_t y_t, int64_t M, int64_t K, int64_t N, int64_t group_size,
                      void* stream);

/* Host-only check of an awq_gemm problem: the same shape validation awq_gemm
 * applies (the module's constraints through validate_launch_params_impl,
 * src/kernel/awq_kernel_gemm.rs:89-171, with the M <= 8 decode split of :691),
 * without touching the GPU. 0 if awq_gemm would accept the shapes, else the
 * error code with awq_last_error() set to the reference's panic text. */
int awq_validate_gemm(int64_t M, int64_t K, int64_t N, int64_t group_size);

/* Pointer-level dequantize: out[K, N] in o_t from scales in s_t (s_t == o_t is
 * the reference's single-F case), either nibble order. N % 32 == 0, K % g == 0. */
int awq_dequantize(const uint32_t* qweight, const uint32_t* qzeros, const void* scales,
                   int32_t s_t, void* out, int32_t o_t, int64_t K, int64_t N,
                   int64_t group_size, int32_t order, void* stream);

/* select_tile_m / select_tile_n (src/modules/awq_gemm.rs:30-52), including the
 * AWQ_GEMM_FORCE_TILE_M environment override (:20-28). */
int64_t awq_select_tile_m(int64_t m);
int64_t awq_select_tile_n(int64_t n);

/* DECODE_M_THRESHOLD (src/kernel/awq_kernel_gemm.rs:81): M <= this runs the GEMV. */
int64_t awq_decode_m_threshold(void);

/* Re-read the AWQ_* tuning overrides (environment variables that force a
 * kernel route or launch configuration, used by tests and tuning sweeps).
 * The library reads them once per process, on its first launch, so that no
 * launch pays for a getenv(); call this after changing one. No reference
 * counterpart (the reference has no such overrides besides
 * AWQ_GEMM_FORCE_TILE_M, which, as there, is read once and not re-read). */
void awq_tuning_reload(void);

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* awq_last_error(void);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int32_t awq_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CUBE_AWQ_AWQ_H */
