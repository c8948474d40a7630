// qmv.hip — small-M quantized GEMV (y[M,N] = x[M,K] . W^T, M <= 8) for gfx950.
//
// The path is HBM-bound: each packed weight byte is read once and used M times, so the kernel
// is built around wide coalesced weight loads and cheap per-weight arithmetic rather than MFMA.
// Weights are dequantized exactly in f32 through the factored per-group form
//     sum_k x[k] * (s*c[k] + b) = s * sum_k x[k]*c[k] + b * sum_k x[k]
// so each weight costs one int->float conversion and one FMA per activation row.
//
// Work split: a wave owns ROWS consecutive weight rows (output columns n); its 64 lanes stride
// over K in 32-element chunks (16 B of Q4 codes / 32 B of Q8 codes per row per chunk), each chunk
// inside a single group (group_size >= 32).  Lane partial sums are reduced across the wave at
// the end.  x (M rows) is re-read per chunk from L1/L2 and shared by the ROWS weight rows.
#include <type_traits>

#include "mlxq_common.h"

namespace mlxq {

template <typename XT>
__device__ __forceinline__ void load_x32(const XT* p, float (&v)[32]);

template <>
__device__ __forceinline__ void load_x32<uint16_t>(const uint16_t* p, float (&v)[32]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    u32x4 r = reinterpret_cast<const u32x4*>(p)[q];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[q * 8 + 2 * i] = __uint_as_float(r[i] << 16);
      v[q * 8 + 2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
}

template <>
__device__ __forceinline__ void load_x32<float>(const float* p, float (&v)[32]) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    f32x4 r = reinterpret_cast<const f32x4*>(p)[q];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[q * 4 + i] = r[i];
  }
}

template <>
__device__ __forceinline__ void load_x32<_Float16>(const _Float16* p, float (&v)[32]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    u32x4 r = reinterpret_cast<const u32x4*>(p)[q];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[q * 8 + 2 * i] = f16_lo(r[i]);
      v[q * 8 + 2 * i + 1] = f16_hi(r[i]);
    }
  }
}

// dot of 32 codes (one chunk of a weight row) with 32 activations.
template <int BITS>
__device__ __forceinline__ float dot_chunk(const uint32_t (&w)[BITS], const float (&x)[32]) {
  float acc = 0.0f;
  if constexpr (BITS == 4) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = w[q] & 0x0f0f0f0fu, hi = (w[q] >> 4) & 0x0f0f0f0fu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc = fmaf(x[q * 8 + 2 * i], (float)((lo >> (8 * i)) & 0xffu), acc);
        acc = fmaf(x[q * 8 + 2 * i + 1], (float)((hi >> (8 * i)) & 0xffu), acc);
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = fmaf(x[q * 4 + i], (float)((w[q] >> (8 * i)) & 0xffu), acc);
    }
  }
  return acc;
}

// The result dtype is MLX's promote(x, scales): bf16 only when both are bf16 (uint16_t storage);
// fp16 x against bf16 or f32 scales promotes to f32.
template <typename XT, typename SB>
using QmvOut = typename std::conditional<std::is_same<XT, uint16_t>::value && std::is_same<SB, uint16_t>::value,
                                         uint16_t, float>::type;

template <typename XT, typename SB, int BITS, int GS, int MR, int ROWS>
__global__ __launch_bounds__(256) void qmv_kernel(const XT* __restrict__ x, int M, int64_t K,
                                                  const uint32_t* __restrict__ wq,
                                                  const SB* __restrict__ scales,
                                                  const SB* __restrict__ biases, int64_t N,
                                                  QmvOut<XT, SB>* __restrict__ y) {
  constexpr int WPC = BITS;  // uint32 words per 32-element chunk: 4 (Q4) or 8 (Q8)
  const int lane = threadIdx.x & 63;
  const int64_t n0 = ((int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)) * ROWS;
  const int m0 = blockIdx.y * MR;
  if (n0 >= N) return;
  const int64_t chunks = K / 32;
  const int64_t words_per_row = K * BITS / 32;
  const int64_t groups = K / GS;

  float acc[ROWS][MR];
#pragma unroll
  for (int r = 0; r < ROWS; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;

  for (int64_t c = lane; c < chunks; c += 64) {
    float xs[MR][32];
    float xsum[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m0 + m < M) {
        load_x32<XT>(x + (int64_t)(m0 + m) * K + c * 32, xs[m]);
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) xs[m][i] = 0.0f;
      }
      float t = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; ++i) t += xs[m][i];
      xsum[m] = t;
    }
    const int64_t g = c * 32 / GS;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const int64_t n = n0 + r;
      if (n < N) {
        uint32_t w[WPC];
        const u32x4* wp = reinterpret_cast<const u32x4*>(wq + n * words_per_row + c * WPC);
#pragma unroll
        for (int q = 0; q < WPC / 4; ++q) {
          u32x4 v = wp[q];
#pragma unroll
          for (int i = 0; i < 4; ++i) w[q * 4 + i] = v[i];
        }
        const float s = SBLoad<SB>::ld(scales, n * groups + g);
        const float b = SBLoad<SB>::ld(biases, n * groups + g);
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = fmaf(s, dot_chunk<BITS>(w, xs[m]), fmaf(b, xsum[m], acc[r][m]));
      }
    }
  }
#pragma unroll
  for (int r = 0; r < ROWS; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = acc[r][m];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
      acc[r][m] = v;
    }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (n0 + r < N && m0 + m < M) Act<QmvOut<XT, SB>>::st(y, (int64_t)(m0 + m) * N + n0 + r, acc[r][m]);
  }
}

template <typename XT, typename SB, int BITS, int GS, int MR>
static int launch_qmv(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                      const void* b, int64_t N, void* y, hipStream_t st) {
  constexpr int ROWS = 4;
  const int64_t rows_per_block = 4 * ROWS;
  const int64_t gx = (N + rows_per_block - 1) / rows_per_block;
  const int64_t gy = (M + MR - 1) / MR;
  if (gx == 0 || gy == 0) return MLXQ_OK;
  if (gy > 65535) return set_error(MLXQ_EINVAL, "qmv: M=%lld too large for the f32 kernel", (long long)M);
  hipLaunchKernelGGL((qmv_kernel<XT, SB, BITS, GS, MR, ROWS>), dim3((unsigned)gx, (unsigned)gy),
                     dim3(256), 0, st, (const XT*)x, (int)M, K, wq, (const SB*)s, (const SB*)b, N,
                     (QmvOut<XT, SB>*)y);
  return check_launch("qmv");
}

template <typename XT, typename SB, int BITS, int GS>
static int qmv_rows(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                    const void* b, int64_t N, void* y, hipStream_t st) {
  if (M <= 1) return launch_qmv<XT, SB, BITS, GS, 1>(x, M, K, wq, s, b, N, y, st);
  if (M <= 2) return launch_qmv<XT, SB, BITS, GS, 2>(x, M, K, wq, s, b, N, y, st);
  if (M <= 4) return launch_qmv<XT, SB, BITS, GS, 4>(x, M, K, wq, s, b, N, y, st);
  return launch_qmv<XT, SB, BITS, GS, 8>(x, M, K, wq, s, b, N, y, st);
}

template <typename XT, typename SB>
static int qmv_bits_gs(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                       const void* b, int64_t N, int gs, int bits, void* y, hipStream_t st) {
#define MLXQ_V(B, G) \
  if (bits == B && gs == G) return qmv_rows<XT, SB, B, G>(x, M, K, wq, s, b, N, y, st);
  MLXQ_V(4, 32) MLXQ_V(4, 64) MLXQ_V(4, 128) MLXQ_V(8, 32) MLXQ_V(8, 64) MLXQ_V(8, 128)
#undef MLXQ_V
  return set_error(MLXQ_EINVAL, "qmv: unsupported bits=%d group_size=%d", bits, gs);
}

int run_qmv_valu(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                 const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y, hipStream_t st) {
  // bf16 decode shapes at M = 1: the one-row kernel's loads with VALU dot products, so the A/B
  // against the matrix cores compares the arithmetic alone.
  if (qmv_row_valu_applicable(x_dtype, sb_dtype, M, K, N, gs, bits))
    return run_qmv_row_valu(x, K, wq, s, b, N, gs, y, st);
  if (x_dtype == MLXQ_BFLOAT16) {
    if (sb_dtype == MLXQ_BFLOAT16) return qmv_bits_gs<uint16_t, uint16_t>(x, M, K, wq, s, b, N, gs, bits, y, st);
    return qmv_bits_gs<uint16_t, float>(x, M, K, wq, s, b, N, gs, bits, y, st);
  }
  if (x_dtype == MLXQ_FLOAT16) {
    if (sb_dtype == MLXQ_BFLOAT16) return qmv_bits_gs<_Float16, uint16_t>(x, M, K, wq, s, b, N, gs, bits, y, st);
    return qmv_bits_gs<_Float16, float>(x, M, K, wq, s, b, N, gs, bits, y, st);
  }
  if (sb_dtype == MLXQ_BFLOAT16) return qmv_bits_gs<float, uint16_t>(x, M, K, wq, s, b, N, gs, bits, y, st);
  return qmv_bits_gs<float, float>(x, M, K, wq, s, b, N, gs, bits, y, st);
}

// The f32-dequant product for any M: the decode GEMV for M <= 8, the split-bf16 matrix-core GEMM
// (qmm_f32.hip) above that.
int run_qmv(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq, const void* s,
            const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y, hipStream_t st) {
  if (M > 8) {
    if (x_dtype == MLXQ_BFLOAT16 && sb_dtype == MLXQ_BFLOAT16)
      return set_error(MLXQ_EINVAL, "qmv: M=%lld exceeds the GEMV limit of 8", (long long)M);
    return run_qmm_f32(x, x_dtype, M, K, wq, s, b, sb_dtype, N, gs, bits, y, st);
  }
  // bf16 activations with 64/128 groups take the matrix-core GEMV; f32 activations and
  // group_size 32 take the VALU kernel above (same exact-f32 dequant semantics).
  if (qmv_mfma_applicable(x_dtype, sb_dtype, M, K, N, gs, bits))
    return run_qmv_mfma(x, M, K, wq, s, b, N, gs, bits, y, st);
  return run_qmv_valu(x, x_dtype, M, K, wq, s, b, sb_dtype, N, gs, bits, y, st);
}

}  // namespace mlxq
