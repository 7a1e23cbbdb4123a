// awq_bench_stream.hip -- measurement helper for bench.py, not part of the
// AWQ library or its ABI: a plain streaming read of a device buffer, so the
// benchmark can report the read bandwidth this GPU reaches on a buffer of the
// decode call's size, next to the decode kernel's own rate.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Every thread streams 16-byte words with a grid stride (nontemporal: the
// data is read once); one word per workgroup is written only if an
// impossible value turns up, so the loads cannot be removed.
__global__ __launch_bounds__(256) void read_stream(const u32x4* __restrict__ p, int64_t n16,
                                                   uint32_t* sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
#pragma unroll 8
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, buffer 16-byte aligned) with `grid`
// workgroups of 256 threads on `stream`; `sink` must hold `grid` words.
// Returns 0, or the HIP error code of the launch.
int awqbench_read_stream(const void* p, int64_t bytes, uint32_t* sink, int grid, void* stream) {
  if (bytes % 16 != 0 || grid <= 0) return -1;
  hipLaunchKernelGGL(read_stream, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(p), bytes / 16, sink);
  return (int)hipGetLastError();
}

}  // extern "C"
