// epilogue.hip — LoRA prologue and the unfused linear epilogue.
//
// The adapter residual of the reference (Adapter::residual: scale * (x.A).B, each matmul and the
// scale multiply rounded to the activation dtype) needs x.A once per call.  lora_prep computes it
// together with the transposed, zero-padded up-projection so the GEMM epilogue can run the
// rank-R product as one more MFMA K-step.  linear_epilogue applies bias / LoRA / activation to an
// already computed y for the paths that do not fuse them (GEMV and f32 activations).
#include "mlxq_common.h"

namespace mlxq {

// xa[M,R] = round(x[M,K] . A[K,rank]) (zero for r >= rank); lbt[N,R] = B[rank,N]^T (zero padded).
// One thread per output element: the general form (f32 activations, K not a multiple of 32).
template <typename XT>
__global__ void lora_prep_kernel(const XT* __restrict__ x, int64_t M, int64_t K,
                                 const XT* __restrict__ A, const XT* __restrict__ B, int64_t N,
                                 int rank, int R, XT* __restrict__ xa, XT* __restrict__ lbt) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nxa = M * R;
  if (t < nxa) {
    const int64_t m = t / R;
    const int r = (int)(t % R);
    float acc = 0.0f;
    if (r < rank) {
      for (int64_t k = 0; k < K; ++k) acc = fmaf(Act<XT>::ld(x, m * K + k), Act<XT>::ld(A, k * rank + r), acc);
    }
    Act<XT>::st(xa, t, acc);
  } else if (t < nxa + N * R) {
    const int64_t u = t - nxa;
    const int64_t n = u / R;
    const int r = (int)(u % R);
    lbt[u] = r < rank ? B[(int64_t)r * N + n] : (XT)0;
  }
}

// bf16 x.A on the matrix cores: xa[M,R] = round_bf16(x[M,K] . A[K,rank]), columns >= rank zero.
// A workgroup owns 16 rows of x and 16 columns of xa; its 8 waves split K (32 per MFMA step,
// K % 32 == 0 because K is a multiple of the group size) and reduce through LDS.  The MFMA's B
// operand needs 8 consecutive k of one column of the k-major A: 8 two-byte loads per lane and
// step, L1/L2 hits (A is at most K x 256 x 2 bytes and every workgroup reads it).  Each wave
// walks its K range in chunks of kXaChunk steps, double-buffered: a chunk's loads are issued
// before the previous chunk's MFMAs, so a wave waits for memory about once instead of once per
// step (the x rows come from HBM).
constexpr int kXaWaves = 8;
constexpr int kXaChunk = 4;
// Workgroups past the x.A grid (blockIdx.x >= xa_blocks) write lbt[N,R] = B[rank,N]^T instead
// (zero padded, the GEMM epilogue's operand), so the LoRA preparation is one launch.
// A16 (rank 16, one 16-column block): a chunk of A (4 steps x 32 rows x 16 columns) is 4 KB of
// contiguous memory, fetched with four 16-byte loads per lane and transposed through the wave's
// 4 KB LDS buffer, instead of 32 two-byte gathers per lane.
template <bool A16>
__global__ __launch_bounds__(kXaWaves * 64) void lora_xa_kernel(const uint16_t* __restrict__ x, int M,
                                                                int K, const uint16_t* __restrict__ A,
                                                                int rank, int R, uint16_t* __restrict__ xa,
                                                                int xa_blocks, const uint16_t* __restrict__ B,
                                                                int64_t N, uint16_t* __restrict__ lbt) {
  __shared__ float red[kXaWaves][16 * 16];
  __shared__ __attribute__((aligned(16))) uint16_t abuf[A16 ? kXaWaves * 2048 : 8];
  // wave is made scalar so the K-range branches below are uniform scalar branches.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if ((int)blockIdx.x >= xa_blocks) {
    if (blockIdx.y != 0) return;
    const int64_t u = ((int64_t)blockIdx.x - xa_blocks) * (kXaWaves * 64) + tid;
    if (u < N * R) {
      const int64_t n = u / R;
      const int rr = (int)(u % R);
      lbt[u] = rr < rank ? B[(int64_t)rr * N + n] : (uint16_t)0;
    }
    return;
  }
  const int c16 = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.x * 16, r0 = blockIdx.y * 16;
  const int xrow = m0 + c16 < M ? m0 + c16 : M - 1;
  const int r = r0 + c16;
  const bool rvalid = r < rank;
  const int KS = K / 32, per = (KS + kXaWaves - 1) / kXaWaves;
  const int ks0 = __builtin_amdgcn_readfirstlane(wave * per);
  const int ks1 = __builtin_amdgcn_readfirstlane(ks0 + per < KS ? ks0 + per : KS);
  const uint16_t* xp = x + (int64_t)xrow * K + 8 * q;
  const uint16_t* ap = A + (int64_t)(8 * q) * rank + (rvalid ? r : 0);
  struct Chunk {
    bf16x8 a[kXaChunk];
    uint16_t w[A16 ? 1 : kXaChunk][8];
    u32x4 araw[A16 ? kXaChunk : 1];  // A16: lane l's 64 bytes of the chunk (rows 2l, 2l+1)
  };
  uint16_t* const wbuf = abuf + (A16 ? wave * 2048 : 0);
  // Steps past the wave's range repeat its last step (in bounds) and are not accumulated.  Every
  // load is unconditional (lanes of columns >= rank read column 0 and zero it afterwards): a
  // conditional load made the compiler wait for each one before the next.
  auto load = [&](int ks, Chunk& c) {
#pragma unroll
    for (int u = 0; u < kXaChunk; ++u) {
      const int k = ks + u < ks1 ? ks + u : ks1 - 1;
      c.a[u] = *reinterpret_cast<const bf16x8*>(xp + k * 32);
      if constexpr (!A16) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c.w[u][j] = ap[(int64_t)(k * 32 + j) * rank];  // column 0 if !rvalid
      }
    }
    if constexpr (A16) {
#pragma unroll
      for (int p = 0; p < kXaChunk; ++p) {  // row ks*32 + 2 lane + p/2, columns 8 (p&1) .. +8
        const int row = ks * 32 + 2 * lane + (p >> 1);
        c.araw[p] = *reinterpret_cast<const u32x4*>(A + (int64_t)(row < K ? row : K - 1) * 16 + 8 * (p & 1));
      }
    }
  };
  // A16: the chunk's rows into the wave's buffer, [128 rows][16 columns] bf16 (after this wave's
  // reads of the previous chunk, LDS being in order within a wave).
  auto stage = [&](const Chunk& c) {
    if constexpr (A16) {
#pragma unroll
      for (int p = 0; p < kXaChunk; ++p) *reinterpret_cast<u32x4*>(wbuf + lane * 32 + p * 8) = c.araw[p];
    }
  };
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  // Every MFMA of a chunk is issued; steps past the wave's range and padding columns get a zero B
  // operand through a mask the compiler cannot see through.  MFMA does not honour the EXEC mask:
  // given a visible "operand is zero" condition the compiler predicated the MFMA on EXEC without
  // a branch, and with one step per wave it then added the repeated step a second time.
  auto compute = [&](int ks, const Chunk& c) {
#pragma unroll
    for (int u = 0; u < kXaChunk; ++u) {
      uint32_t keep = rvalid && ks + u < ks1 ? 0xffffffffu : 0u;
      asm volatile("" : "+v"(keep));
      u32x4 bw;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t lo, hi;
        if constexpr (A16) {
          lo = wbuf[(u * 32 + 8 * q + 2 * j) * 16 + c16];
          hi = wbuf[(u * 32 + 8 * q + 2 * j + 1) * 16 + c16];
        } else {
          lo = c.w[u][2 * j];
          hi = c.w[u][2 * j + 1];
        }
        bw[j] = (lo | (hi << 16)) & keep;
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c.a[u], __builtin_bit_cast(bf16x8, bw), acc, 0, 0, 0);
    }
  };
  if (ks0 < ks1) {
    Chunk c0, c1;
    load(ks0, c0);
    for (int ks = ks0; ks < ks1; ks += 2 * kXaChunk) {
      load(ks + kXaChunk, c1);
      stage(c0);
      compute(ks, c0);
      if (ks + kXaChunk < ks1) {
        load(ks + 2 * kXaChunk, c0);
        stage(c1);
        compute(ks + kXaChunk, c1);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) red[wave][(4 * q + e) * 16 + c16] = acc[e];
  __syncthreads();
  if (tid < 256) {
    const int m = tid >> 4, n = tid & 15;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kXaWaves; ++w) v += red[w][m * 16 + n];
    if (m0 + m < M) xa[(int64_t)(m0 + m) * R + r0 + n] = f32_to_bf16_bits(v);
  }
}

int run_lora_prep(const void* x, int x_dtype, int64_t M, int64_t K, const void* A, const void* B,
                  int64_t N, int rank, int R, void* xa, void* lbt, hipStream_t st) {
  const int64_t total = M * R + N * R;
  if (total == 0) return MLXQ_OK;
  const int64_t blocks = (total + 255) / 256;
  const int64_t bt_blocks = (N * R + kXaWaves * 64 - 1) / (kXaWaves * 64);
  if (x_dtype == MLXQ_BFLOAT16 && K % 32 == 0 && M < (1LL << 31) / 16 && K < (1LL << 31) &&
      bt_blocks < (1LL << 30)) {
    // x.A workgroups (16 rows x 16 columns each), then the B^T workgroups.
    const int xa_blocks = (int)((M + 15) / 16);
    const dim3 grid((unsigned)(xa_blocks + bt_blocks), (unsigned)(R / 16));
    if (rank == 16 && R == 16)
      hipLaunchKernelGGL(lora_xa_kernel<true>, grid, dim3(kXaWaves * 64), 0, st, (const uint16_t*)x,
                         (int)M, (int)K, (const uint16_t*)A, rank, R, (uint16_t*)xa, xa_blocks,
                         (const uint16_t*)B, N, (uint16_t*)lbt);
    else
      hipLaunchKernelGGL(lora_xa_kernel<false>, grid, dim3(kXaWaves * 64), 0, st, (const uint16_t*)x,
                         (int)M, (int)K, (const uint16_t*)A, rank, R, (uint16_t*)xa, xa_blocks,
                         (const uint16_t*)B, N, (uint16_t*)lbt);
  } else if (x_dtype == MLXQ_BFLOAT16) {
    hipLaunchKernelGGL(lora_prep_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint16_t*)x, M, K, (const uint16_t*)A, (const uint16_t*)B, N, rank, R,
                       (uint16_t*)xa, (uint16_t*)lbt);
  } else {
    hipLaunchKernelGGL(lora_prep_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const float*)x, M, K, (const float*)A, (const float*)B, N, rank, R,
                       (float*)xa, (float*)lbt);
  }
  return check_launch("lora_prep");
}

// In place on y[M,N]: y = act(rnd(rnd(y + bias) + rnd(rnd(xa . lbt^T) * scale))).
template <typename XT>
__global__ void linear_epilogue_kernel(XT* __restrict__ y, int64_t M, int64_t N,
                                       const XT* __restrict__ bias, const XT* __restrict__ xa,
                                       const XT* __restrict__ lbt, int R, float scale, int act) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * N) return;
  const int64_t m = t / N, n = t % N;
  float o = Act<XT>::ld(y, t);
  if (bias) o = Act<XT>::rnd(o + Act<XT>::ld(bias, n));
  if (R > 0) {
    float r = 0.0f;
    for (int k = 0; k < R; ++k) r = fmaf(Act<XT>::ld(xa, m * R + k), Act<XT>::ld(lbt, n * R + k), r);
    o = Act<XT>::rnd(o + Act<XT>::rnd(Act<XT>::rnd(r) * scale));
  }
  if (act == MLXQ_ACT_GELU) o = gelu_erf(o);
  else if (act == MLXQ_ACT_GELU_TANH) o = gelu_tanh<sizeof(XT) == 2>(o);
  Act<XT>::st(y, t, o);
}

int run_linear_epilogue(void* y, int x_dtype, int64_t M, int64_t N, const void* bias, const void* xa,
                        const void* lbt, int R, float scale, int act, hipStream_t st) {
  const int64_t total = M * N;
  if (total == 0) return MLXQ_OK;
  const int64_t blocks = (total + 255) / 256;
  if (x_dtype == MLXQ_BFLOAT16) {
    hipLaunchKernelGGL(linear_epilogue_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (uint16_t*)y, M, N, (const uint16_t*)bias, (const uint16_t*)xa,
                       (const uint16_t*)lbt, R, scale, act);
  } else {
    hipLaunchKernelGGL(linear_epilogue_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (float*)y, M, N, (const float*)bias, (const float*)xa, (const float*)lbt, R,
                       scale, act);
  }
  return check_launch("linear_epilogue");
}

// dst[i] = src[i] converted between f32 and bf16 (round to nearest even) or copied.
template <typename ST, typename DT>
__global__ void cast_kernel(const ST* __restrict__ src, DT* __restrict__ dst, int64_t n) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) Act<DT>::st(dst, t, Act<ST>::ld(src, t));
}

int run_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, hipStream_t st) {
  if (n == 0) return MLXQ_OK;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return set_error(MLXQ_EINVAL, "cast: %lld elements is too many", (long long)n);
  const dim3 g((unsigned)blocks), b(256);
  if (src_dtype == MLXQ_BFLOAT16 && dst_dtype == MLXQ_BFLOAT16)
    hipLaunchKernelGGL((cast_kernel<uint16_t, uint16_t>), g, b, 0, st, (const uint16_t*)src, (uint16_t*)dst, n);
  else if (src_dtype == MLXQ_BFLOAT16)
    hipLaunchKernelGGL((cast_kernel<uint16_t, float>), g, b, 0, st, (const uint16_t*)src, (float*)dst, n);
  else if (dst_dtype == MLXQ_BFLOAT16)
    hipLaunchKernelGGL((cast_kernel<float, uint16_t>), g, b, 0, st, (const float*)src, (uint16_t*)dst, n);
  else
    hipLaunchKernelGGL((cast_kernel<float, float>), g, b, 0, st, (const float*)src, (float*)dst, n);
  return check_launch("cast");
}

}  // namespace mlxq
