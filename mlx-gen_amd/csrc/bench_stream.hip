// bench_stream.hip — measurement reference for bench.py, built into libmlxq_bench.so (not part of
// libmlxq_hip.so or its ABI).
//
// stream_kernel has quantize_kernel's memory pattern with trivial arithmetic: each thread reads
// a 64-byte chunk (four 16-byte loads, consecutive threads consecutive chunks) and writes `WORDS`
// 4-byte words for it (4: the Q4 codes of 32 bf16 weights, 8: Q8).  With one workgroup of 256
// threads per 256 chunks (quantize's grid) each thread takes one chunk; a smaller grid walks the
// chunks at a stride of the whole grid, the next chunk's loads in flight.  The time it takes on
// the same buffers is the floor the quantize pass is compared against.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int WORDS>
__global__ __launch_bounds__(256) void stream_kernel(const u32x4* __restrict__ src, int64_t n_chunks,
                                                     u32x4* __restrict__ dst) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t chunk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  u32x4 cur[4], nxt[4];
  const int64_t c0 = chunk < n_chunks ? chunk : 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) cur[i] = src[c0 * 4 + i];
  for (; chunk - lane < n_chunks; chunk += stride) {
    const int64_t next = chunk + stride < n_chunks ? chunk + stride : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) nxt[i] = src[next * 4 + i];
    if (chunk < n_chunks) {
#pragma unroll
      for (int q = 0; q < WORDS / 4; ++q) {
        u32x4 o = cur[0] ^ cur[1] ^ cur[2] ^ cur[3];
        o += (uint32_t)q;
        dst[chunk * (WORDS / 4) + q] = o;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
  }
}

}  // namespace

// src: n_chunks x 64 bytes; dst: n_chunks x 4 * words bytes (words 4 or 8); blocks: grid size
// (quantize's is ceil(n_chunks / 256)).
extern "C" int mlxq_bench_stream(const void* src, int64_t n_chunks, void* dst, int words, int64_t blocks,
                                 void* stream) {
  if (n_chunks <= 0 || blocks <= 0 || (words != 4 && words != 8)) return 1;
  hipStream_t st = (hipStream_t)stream;
  if (words == 4)
    hipLaunchKernelGGL(stream_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, (const u32x4*)src, n_chunks,
                       (u32x4*)dst);
  else
    hipLaunchKernelGGL(stream_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, st, (const u32x4*)src, n_chunks,
                       (u32x4*)dst);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
