// epilogue.hip — LoRA prologue and the unfused linear epilogue.
//
// The adapter residual of the reference (Adapter::residual: scale * (x.A).B, each matmul and the
// scale multiply rounded to the activation dtype) needs x.A once per call.  lora_prep computes it
// together with the transposed, zero-padded up-projection so the GEMM epilogue can run the
// rank-R product as one more MFMA K-step.  linear_epilogue applies bias / LoRA / activation to an
// already computed y for the paths that do not fuse them (GEMV, f32 activations, ranks above 16
// and every result MLX's dtype promotion makes f32 from a bf16 product).
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
// A workgroup owns `rows` rows of x (NB blocks of 16 rows on the MFMA; rows past its share repeat
// its last row and are not stored) and 16 columns of xa; its 8 waves split K (32 per MFMA step,
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
// Rows per workgroup: 16, except from 4097 to 8192 rows, where ceil(M / 256) (17-32 rows, two
// MFMA blocks) spreads the x stream evenly over at most 256 workgroups, one per CU.  With 16-row
// workgroups M = 4608 made 288 of them, and the 32 CUs that ran two read twice the bytes: same-
// process A/B through mlxq_lora_residual (K = 3072, rank 16), 16-row against balanced workgroups:
// M = 4608 24.0 -> 20.9 us, 5120 23.8 -> 21.3, 6144 26.0 -> 24.3, 8192 29.9 / 30.1 (even);
// 512 balanced workgroups of up to 16 rows (two per CU) gained about half as much, and 32-row
// workgroups past 8192 rows lost (M = 12288 51.5 -> 53.1).
template <bool A16, int NB>
__global__ __launch_bounds__(kXaWaves * 64) void lora_xa_kernel(const uint16_t* __restrict__ x, int M,
                                                                int K, const uint16_t* __restrict__ A,
                                                                int rank, int R, uint16_t* __restrict__ xa,
                                                                int xa_blocks, int rows,
                                                                const uint16_t* __restrict__ B,
                                                                int64_t N, uint16_t* __restrict__ lbt) {
  __shared__ float red[NB][kXaWaves][16 * 16];
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
  const int m0 = blockIdx.x * rows, r0 = blockIdx.y * 16;
  const int m_end = m0 + rows < M ? m0 + rows : M;  // this workgroup's rows [m0, m_end)
  const int r = r0 + c16;
  const bool rvalid = r < rank;
  const int KS = K / 32, per = (KS + kXaWaves - 1) / kXaWaves;
  const int ks0 = __builtin_amdgcn_readfirstlane(wave * per);
  const int ks1 = __builtin_amdgcn_readfirstlane(ks0 + per < KS ? ks0 + per : KS);
  const uint16_t* xp[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int row = m0 + 16 * b + c16;
    xp[b] = x + (int64_t)(row < m_end ? row : m_end - 1) * K + 8 * q;
  }
  const uint16_t* ap = A + (int64_t)(8 * q) * rank + (rvalid ? r : 0);
  struct Chunk {
    bf16x8 a[NB][kXaChunk];
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
#pragma unroll
      for (int b = 0; b < NB; ++b) c.a[b][u] = *reinterpret_cast<const bf16x8*>(xp[b] + k * 32);
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
  f32x4 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
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
#pragma unroll
      for (int b = 0; b < NB; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c.a[b][u], __builtin_bit_cast(bf16x8, bw), acc[b], 0, 0, 0);
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
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[b][wave][(4 * q + e) * 16 + c16] = acc[b][e];
  __syncthreads();
  if (tid < 256 * NB) {
    const int b = tid >> 8, m = (tid >> 4) & 15, n = tid & 15;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kXaWaves; ++w) v += red[b][w][m * 16 + n];
    const int row = m0 + 16 * b + m;
    if (row < m_end) xa[(int64_t)row * R + r0 + n] = f32_to_bf16_bits(v);
  }
}

// DR = f32 (an f32 or fp16 activation, or f32 factors): xa[M,R] = x . A and lbt[N,R] = B^T in f32,
// x and the factors widened exactly (MLX promotes the 16-bit operands of a mixed matmul to f32).
template <typename XT, typename FT>
__global__ void lora_prep_f32_kernel(const XT* __restrict__ x, int64_t M, int64_t K,
                                     const FT* __restrict__ A, const FT* __restrict__ B, int64_t N,
                                     int rank, int R, float* __restrict__ xa, float* __restrict__ lbt) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nxa = M * R;
  if (t < nxa) {
    const int64_t m = t / R;
    const int r = (int)(t % R);
    float acc = 0.0f;
    if (r < rank) {
      for (int64_t k = 0; k < K; ++k) acc = fmaf(Act<XT>::ld(x, m * K + k), Act<FT>::ld(A, k * rank + r), acc);
    }
    xa[t] = acc;
  } else if (t < nxa + N * R) {
    const int64_t u = t - nxa;
    const int64_t n = u / R;
    const int r = (int)(u % R);
    lbt[u] = r < rank ? Act<FT>::ld(B, (int64_t)r * N + n) : 0.0f;
  }
}

int run_lora_prep(const void* x, int x_dtype, int64_t M, int64_t K, const void* A, const void* B,
                  int lora_dtype, int64_t N, int rank, int R, void* xa, void* lbt, hipStream_t st) {
  const int64_t total = M * R + N * R;
  if (total == 0) return MLXQ_OK;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return set_error(MLXQ_EINVAL, "lora: problem too large");
  if (x_dtype != MLXQ_BFLOAT16 || lora_dtype != MLXQ_BFLOAT16) {
    const dim3 g((unsigned)blocks), b(256);
    if (x_dtype == MLXQ_FLOAT16) {
      if (lora_dtype == MLXQ_BFLOAT16)
        hipLaunchKernelGGL((lora_prep_f32_kernel<_Float16, uint16_t>), g, b, 0, st, (const _Float16*)x, M, K,
                           (const uint16_t*)A, (const uint16_t*)B, N, rank, R, (float*)xa, (float*)lbt);
      else
        hipLaunchKernelGGL((lora_prep_f32_kernel<_Float16, float>), g, b, 0, st, (const _Float16*)x, M, K,
                           (const float*)A, (const float*)B, N, rank, R, (float*)xa, (float*)lbt);
    } else if (x_dtype == MLXQ_BFLOAT16)
      hipLaunchKernelGGL((lora_prep_f32_kernel<uint16_t, float>), g, b, 0, st, (const uint16_t*)x, M, K,
                         (const float*)A, (const float*)B, N, rank, R, (float*)xa, (float*)lbt);
    else if (lora_dtype == MLXQ_BFLOAT16)
      hipLaunchKernelGGL((lora_prep_f32_kernel<float, uint16_t>), g, b, 0, st, (const float*)x, M, K,
                         (const uint16_t*)A, (const uint16_t*)B, N, rank, R, (float*)xa, (float*)lbt);
    else
      hipLaunchKernelGGL((lora_prep_f32_kernel<float, float>), g, b, 0, st, (const float*)x, M, K,
                         (const float*)A, (const float*)B, N, rank, R, (float*)xa, (float*)lbt);
    return check_launch("lora_prep");
  }
  const int64_t bt_blocks = (N * R + kXaWaves * 64 - 1) / (kXaWaves * 64);
  if (K % 32 == 0 && M < (1LL << 31) / 16 && K < (1LL << 31) && bt_blocks < (1LL << 30)) {
    // x.A workgroups (`rows` rows x 16 columns each), then the B^T workgroups.
    const int rows = M > 16 * 256 && M <= 32 * 256 ? (int)((M + 255) / 256) : 16;
    const int xa_blocks = (int)((M + rows - 1) / rows);
    const dim3 grid((unsigned)(xa_blocks + bt_blocks), (unsigned)(R / 16));
    if (rows <= 16) {
      if (rank == 16 && R == 16)
        hipLaunchKernelGGL((lora_xa_kernel<true, 1>), grid, dim3(kXaWaves * 64), 0, st, (const uint16_t*)x,
                           (int)M, (int)K, (const uint16_t*)A, rank, R, (uint16_t*)xa, xa_blocks, rows,
                           (const uint16_t*)B, N, (uint16_t*)lbt);
      else
        hipLaunchKernelGGL((lora_xa_kernel<false, 1>), grid, dim3(kXaWaves * 64), 0, st, (const uint16_t*)x,
                           (int)M, (int)K, (const uint16_t*)A, rank, R, (uint16_t*)xa, xa_blocks, rows,
                           (const uint16_t*)B, N, (uint16_t*)lbt);
    } else {
      if (rank == 16 && R == 16)
        hipLaunchKernelGGL((lora_xa_kernel<true, 2>), grid, dim3(kXaWaves * 64), 0, st, (const uint16_t*)x,
                           (int)M, (int)K, (const uint16_t*)A, rank, R, (uint16_t*)xa, xa_blocks, rows,
                           (const uint16_t*)B, N, (uint16_t*)lbt);
      else
        hipLaunchKernelGGL((lora_xa_kernel<false, 2>), grid, dim3(kXaWaves * 64), 0, st, (const uint16_t*)x,
                           (int)M, (int)K, (const uint16_t*)A, rank, R, (uint16_t*)xa, xa_blocks, rows,
                           (const uint16_t*)B, N, (uint16_t*)lbt);
    }
  } else {
    hipLaunchKernelGGL(lora_prep_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint16_t*)x, M, K, (const uint16_t*)A, (const uint16_t*)B, N, rank, R,
                       (uint16_t*)xa, (uint16_t*)lbt);
  }
  return check_launch("lora_prep");
}

__device__ __forceinline__ float ld_any(const void* p, bool bf16, int64_t i) {
  return bf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}
__device__ __forceinline__ float rnd_if(bool bf16, float v) { return bf16 ? round_bf16(v) : v; }

// out = act(y1 + r), y1 = y_in + bias: every stage rounded to its promoted dtype (flags), the
// sequence of LinearBase::forward's bias add and AdaptableLinear::forward's residual sum
// (reference src/adapters.rs:318-320,543-549, Adapter::residual :260-270).  A bf16 activation is
// the bf16 table's entry of its input; in f32 it is evaluated (GELU and the exact GELU as the
// f32 erf form, the tanh GELU op by op).
template <typename YI, typename YO>
__global__ void linear_epilogue_kernel(LinearEpilogueArgs a) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.M * a.N) return;
  const int64_t m = t / a.N, n = t % a.N;
  float o = Act<YI>::ld(static_cast<const YI*>(a.y_in), t);
  if (a.bias) o = rnd_if(a.d1_bf16, o + ld_any(a.bias, a.bias_bf16, n));
  if (a.R > 0) {
    float r = 0.0f;
    for (int k = 0; k < a.R; ++k)
      r = fmaf(ld_any(a.xa, a.dr_bf16, m * a.R + k), ld_any(a.lbt, a.dr_bf16, n * a.R + k), r);
    o = rnd_if(a.d2_bf16, o + rnd_if(a.dr_bf16, rnd_if(a.dr_bf16, r) * a.lora_scale));
  } else if (a.res) {
    o = rnd_if(a.d2_bf16, o + rnd_if(a.dr_bf16, rnd_if(a.dr_bf16, a.res[t]) * a.lora_scale));
  }
  const bool act_bf16 = a.d2_bf16;  // the activation's input dtype
  if (a.act == MLXQ_ACT_GELU) {
    o = gelu_erf(o);
  } else if (a.act == MLXQ_ACT_GELU_TANH || a.act == MLXQ_ACT_GELU_EXACT) {
    if (act_bf16) o = bf16_bits_to_f32(a.act_table[f32_to_bf16_bits(o)]);
    else o = a.act == MLXQ_ACT_GELU_TANH ? gelu_tanh<false>(o) : gelu_erf(o);
  }
  Act<YO>::st(static_cast<YO*>(a.y_out), t, o);
}

int run_linear_epilogue(const LinearEpilogueArgs& a, hipStream_t st) {
  const int64_t total = a.M * a.N;
  if (total == 0) return MLXQ_OK;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return set_error(MLXQ_EINVAL, "linear epilogue: problem too large");
  const bool table_act = a.act == MLXQ_ACT_GELU_TANH || a.act == MLXQ_ACT_GELU_EXACT;
  if (table_act && a.d2_bf16 && a.act_table == nullptr)
    return set_error(MLXQ_EINVAL, "linear epilogue: activation table missing");
  const dim3 g((unsigned)blocks), b(256);
  if (a.y_in_bf16 && a.y_out_bf16) hipLaunchKernelGGL((linear_epilogue_kernel<uint16_t, uint16_t>), g, b, 0, st, a);
  else if (a.y_in_bf16) hipLaunchKernelGGL((linear_epilogue_kernel<uint16_t, float>), g, b, 0, st, a);
  else if (a.y_out_bf16) hipLaunchKernelGGL((linear_epilogue_kernel<float, uint16_t>), g, b, 0, st, a);
  else hipLaunchKernelGGL((linear_epilogue_kernel<float, float>), g, b, 0, st, a);
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
