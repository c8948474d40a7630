// qmm.hip — large-M quantized GEMM y[M,N] = x[M,K] . W^T on gfx950 matrix cores.
//
// Semantics: every weight is dequantized to bf16 as round_bf16(fma(code, scale, bias)) (the
// value MLX's dequantize produces for bf16 scales), multiplied with bf16 activations on
// v_mfma_f32_32x32x16_bf16, accumulated in f32 and rounded once to bf16.
//
// Structure (one 256-thread workgroup = 4 waves in a 2x2 grid, one workgroup per CU):
//   * block tile BM x BN, K advanced 64 at a time (BK = 64);
//   * A (activations) streams global -> registers -> LDS unchanged;
//   * B (packed weights) streams global -> registers, is dequantized in registers (byte-wise
//     int->f32 conversion, FMA with the group's scale/bias, RNE pack to bf16) and written to LDS
//     as a bf16 tile, so each weight is dequantized once per workgroup and shared by the two
//     waves that use it;
//   * LDS rows are 64 bf16 (128 B) with the 16-byte chunk index XOR-swizzled by (row & 7), so the
//     MFMA fragment reads (32 rows x one chunk) and the tile writes are bank-conflict free;
//   * double-buffered LDS: the global loads for step k+1 are in flight while step k's MFMAs run.
// Fragment mapping for 32x32x16: lane l supplies row (l & 31) and 8 consecutive k at chunk
// 2*kk + (l >> 5) for both A and B, so both operands share one k-permutation; the f32x16 result
// holds column (l & 31) and rows 8*(v>>2) + 4*(l>>5) + (v&3).
#include "mlxq_common.h"

namespace mlxq {

constexpr int BK = 64;
// Grids of at least this many 128 x 128 tiles (and under 128 tiles of 256 x 128) take the wide
// kernel's 128 x 128 form instead of the K-split kernel.
constexpr int64_t kQmmMidMinTiles = 136;

__device__ __forceinline__ int swz(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

// EPI = 0: plain y = bf16(acc).  EPI = 1: bias / rank-16 LoRA epilogue; EPI = 2, 3: the same
// followed by the exact-erf or the tanh GELU (EPI - 1 is the mlxq_activation).
template <typename SB, int BITS, int GS, int BM, int BN, int EPI>
__global__ __launch_bounds__(256, 1) void qmm_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                     int64_t K, const uint32_t* __restrict__ wq,
                                                     const SB* __restrict__ scales,
                                                     const SB* __restrict__ biases, int64_t N,
                                                     uint16_t* __restrict__ y, QmmEpilogue epi) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_LD = BM * 8 / 256;                  // 16-B activation chunks per thread
  constexpr int B_CPR = BITS == 4 ? 2 : 4;            // 16-B code chunks per row per K step
  constexpr int B_LD = BN * B_CPR / 256;              // code chunks per thread
  static_assert(A_LD >= 1 && B_LD >= 1, "tile too small for 256 threads");
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;

  __shared__ __attribute__((aligned(16))) unsigned char smem[2][A_BYTES + B_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order: consecutive workgroups walk down M inside one N column of tiles.
  const int64_t tiles_m = (M + BM - 1) / BM;
  const int64_t bm0 = (blockIdx.x % tiles_m) * BM;
  const int64_t bn0 = (blockIdx.x / tiles_m) * BN;

  const int64_t kwords = K * BITS / 32;
  const int64_t groups = K / GS;
  const int ksteps = (int)((K + BK - 1) / BK);

  u32x4 a_reg[A_LD];
  u32x4 b_reg[B_LD];
  float s_reg[B_LD], z_reg[B_LD];

  auto load_global = [&](int kt) {
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + 256 * i;
      const int row = id >> 3, c = id & 7;
      const int64_t m = bm0 + row, k = k0 + c * 8;
      if (m < M && k < K) {
        a_reg[i] = *reinterpret_cast<const u32x4*>(x + m * K + k);
      } else {
        a_reg[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int id = tid + 256 * i;
      const int row = id / B_CPR, j = id % B_CPR;
      const int64_t n = bn0 + row;
      const int64_t kc = k0 + j * (BITS == 4 ? 32 : 16);  // first k of this chunk
      if (n < N && kc < K) {
        b_reg[i] = *reinterpret_cast<const u32x4*>(wq + n * kwords + kc * BITS / 32);
        const int64_t g = n * groups + kc / GS;
        s_reg[i] = SBLoad<SB>::ld(scales, g);
        z_reg[i] = SBLoad<SB>::ld(biases, g);
      } else {
        b_reg[i] = u32x4{0u, 0u, 0u, 0u};
        s_reg[i] = 0.0f;
        z_reg[i] = 0.0f;
      }
    }
  };

  auto store_lds = [&](int buf) {
    unsigned char* As = smem[buf];
    unsigned char* Bs = smem[buf] + A_BYTES;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + 256 * i;
      const int row = id >> 3, c = id & 7;
      *reinterpret_cast<u32x4*>(As + swz(row, c)) = a_reg[i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int id = tid + 256 * i;
      const int row = id / B_CPR, j = id % B_CPR;
      const float s = s_reg[i], z = z_reg[i];
      if constexpr (BITS == 4) {
        // 4 words x 8 nibbles = k [32j, 32j+32): word q -> LDS chunk 4j+q.
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t w = b_reg[i][q];
          const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
          u32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float c0 = (float)((lo >> (8 * e)) & 0xffu);
            const float c1 = (float)((hi >> (8 * e)) & 0xffu);
            o[e] = pack_bf16x2(fmaf(c0, s, z), fmaf(c1, s, z));
          }
          *reinterpret_cast<u32x4*>(Bs + swz(row, 4 * j + q)) = o;
        }
      } else {
        // 4 words x 4 bytes = k [16j, 16j+16): words 2p,2p+1 -> LDS chunk 2j+p.
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          u32x4 o;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t w = b_reg[i][2 * p + h];
            const float c0 = (float)(w & 0xffu), c1 = (float)((w >> 8) & 0xffu);
            const float c2 = (float)((w >> 16) & 0xffu), c3 = (float)(w >> 24);
            o[2 * h] = pack_bf16x2(fmaf(c0, s, z), fmaf(c1, s, z));
            o[2 * h + 1] = pack_bf16x2(fmaf(c2, s, z), fmaf(c3, s, z));
          }
          *reinterpret_cast<u32x4*>(Bs + swz(row, 2 * j + p)) = o;
        }
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  load_global(0);
  store_lds(0);
  __syncthreads();

  const int r32 = lane & 31, half = lane >> 5;
  for (int kt = 0; kt < ksteps; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ksteps) load_global(kt + 1);
    const unsigned char* As = smem[buf];
    const unsigned char* Bs = smem[buf] + A_BYTES;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = kk * 2 + half;
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const bf16x8*>(As + swz(wm * WM + i * 32 + r32, c));
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + swz(wn * WN + j * 32 + r32, c));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ksteps) store_lds(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: y1 = bf16(acc); optional bias, LoRA residual, activation, each rounded to bf16.
  if constexpr (EPI == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t n = bn0 + wn * WN + j * 32 + r32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t m = bm0 + wm * WM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
          if (n < N && m < M) y[m * N + n] = f32_to_bf16_bits(acc[i][j][v]);
        }
      }
  } else {
    // The rank-16 LoRA product (x.A).B runs as one extra 32x32x16 MFMA per output tile; its
    // operands are loaded once per wave (A rows per i, B^T rows per j).
    const bool lora = epi.rank16 > 0;
    bf16x8 xa[TM], lb[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t mrow = bm0 + wm * WM + i * 32 + r32;
      xa[i] = bf16x8{};
      if (lora) xa[i] = *reinterpret_cast<const bf16x8*>(epi.xa + (mrow < M ? mrow : M - 1) * 16 + half * 8);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = bn0 + wn * WN + j * 32 + r32;
      lb[j] = bf16x8{};
      if (lora) lb[j] = *reinterpret_cast<const bf16x8*>(epi.lbt + (n < N ? n : N - 1) * 16 + half * 8);
    }
    // Bias of this lane's columns, loaded together up front (clamped: columns past N are never
    // stored) so the loads are not waited for one at a time.
    float bcol[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) bcol[j] = 0.0f;
    if (epi.bias) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t n = bn0 + wn * WN + j * 32 + r32;
        bcol[j] = bf16_bits_to_f32(epi.bias[n < N ? n : N - 1]);
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t n = bn0 + wn * WN + j * 32 + r32;
        const bool n_ok = n < N;
        f32x16 r = {};
        if (lora) r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[i], lb[j], r, 0, 0, 0);
        const float bn = bcol[j];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t m = bm0 + wm * WM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
          float o = round_bf16(acc[i][j][v]);
          if (epi.bias) o = round_bf16(o + bn);
          if (lora) o = round_bf16(o + round_bf16(round_bf16(r[v]) * epi.lora_scale));
          // o is bf16 here: the activation is the bf16 table's entry for it.
          if constexpr (EPI >= 2) o = bf16_bits_to_f32(epi.act_table[f32_to_bf16_bits(o)]);
          if (n_ok && m < M) y[m * N + n] = f32_to_bf16_bits(o);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

template <typename SB, int BITS, int GS, int BM, int BN>
static int launch_qmm(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                      const void* b, int64_t N, void* y, const QmmEpilogue& epi, hipStream_t st) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles == 0) return MLXQ_OK;
  if (tiles > 0x7fffffff) return set_error(MLXQ_EINVAL, "qmm: problem too large");
  if (epi.rank16 != 0 && epi.rank16 != 16)
    return set_error(MLXQ_EINVAL, "qmm: the fused epilogue takes LoRA rank <= 16");
  const bool fused = epi.bias || epi.rank16 || epi.act != kFusedActNone;
  const int kind = fused ? 1 + epi.act : 0;
  if (kind >= 2 && epi.act_table == nullptr) return set_error(MLXQ_EINVAL, "qmm: activation table missing");
#define MLXQ_QL(E)                                                                                \
  hipLaunchKernelGGL((qmm_kernel<SB, BITS, GS, BM, BN, E>), dim3((unsigned)tiles), dim3(256), 0, st, \
                     (const uint16_t*)x, M, K, wq, (const SB*)s, (const SB*)b, N, (uint16_t*)y, epi)
  switch (kind) {
    case 0: MLXQ_QL(0); break;
    case 1: MLXQ_QL(1); break;
    case 2: MLXQ_QL(2); break;
    case 3: MLXQ_QL(3); break;
    default: return set_error(MLXQ_EINVAL, "qmm: unknown activation %d", epi.act);
  }
#undef MLXQ_QL
  return check_launch("qmm");
}

// 128 x 128 tiles for every shape: the 256 x 256 form held part of its tile in scratch (8-32
// bytes per lane) and measured no faster where it applied (same box, K % 64 == 32 with group size
// 32: M = N = 4096, K = 4064 Q4 262 vs 270 us, with GELU 287 vs 286; M = 2048, N = 8192 Q8 289 vs
// 270; M = 8192, N = 4096, K = 1056 Q4 with GELU 201 vs 170, 256 x 256 first).
template <typename SB, int BITS, int GS>
static int qmm_tile(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                    const void* b, int64_t N, void* y, const QmmEpilogue& epi, hipStream_t st) {
  return launch_qmm<SB, BITS, GS, 128, 128>(x, M, K, wq, s, b, N, y, epi, st);
}

int run_qmm(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s, const void* b,
            int sb_dtype, int64_t N, int gs, int bits, void* y, const QmmEpilogue& epi,
            hipStream_t st) {
  // The wide kernel needs K % 64 == 0 and enough tiles to occupy the CUs: 256x256 tiles, or
  // below 128 of those 256x128 tiles with 4 waves (which beat the K-split kernel from 128 such
  // tiles on: M = 512, N = 12288, K = 3072 52 vs 84 us; M = 2048, N = 3072, K = 8192 120 vs
  // 204 us; below it lost: M = 1024, N = 3072 46 vs 43 us at 96 tiles), and below that
  // 128x128 tiles with 4 waves from kQmmMidMinTiles such tiles on (M = 1024, N = K = 3072, 192
  // tiles: 32 vs 44 us; M = 768, 144 tiles: 31 vs 42 us; even at 128 tiles, M = 512,
  // N = K = 4096: 38 vs 37 us; at 48 tiles 29 vs 15 us).  Small or ragged-K problems take the
  // K-split or the 128/256-tile kernel below.
  const int64_t wide_tiles = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t narrow_tiles = ((M + 255) / 256) * ((N + 127) / 128);
  const int64_t mid_tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (K % 64 == 0 && (wide_tiles >= 128 || narrow_tiles >= 128 || mid_tiles >= kQmmMidMinTiles) &&
      qmm_wide_fits(M, K, N, gs, bits, sb_dtype == MLXQ_BFLOAT16 ? 2 : 4))
    return run_qmm_wide(x, M, K, wq, s, b, sb_dtype, N, gs, bits, y, epi, st);
  // Small grids with a long K: the K-split kernel (64x64 tiles, 8 waves each taking a slice of
  // K).  Measured against the tile kernel on N = K = 3072 (Q4 g64): 13 vs 59 us at M = 256,
  // 42 vs 72 us at M = 1024 (768 small tiles), 65 vs 73 us at M = 1536 (1152), 77 vs 75 us at
  // M = 2048 (1536); M = 512, N = 9216 with bias and GELU (1152) 86 vs 87 us.
  const int64_t small_tiles = ((M + 63) / 64) * ((N + 63) / 64);
  if (K >= 512 && small_tiles <= 1152 && qmm_small_fits(M, K, N, gs, bits, sb_dtype == MLXQ_BFLOAT16 ? 2 : 4))
    return run_qmm_small(x, M, K, wq, s, b, sb_dtype, N, gs, bits, y, epi, st);
#define MLXQ_M(SB, B, G) \
  if (bits == B && gs == G) return qmm_tile<SB, B, G>(x, M, K, wq, s, b, N, y, epi, st);
  if (sb_dtype == MLXQ_BFLOAT16) {
    MLXQ_M(uint16_t, 4, 32) MLXQ_M(uint16_t, 4, 64) MLXQ_M(uint16_t, 4, 128)
    MLXQ_M(uint16_t, 8, 32) MLXQ_M(uint16_t, 8, 64) MLXQ_M(uint16_t, 8, 128)
  } else {
    MLXQ_M(float, 4, 32) MLXQ_M(float, 4, 64) MLXQ_M(float, 4, 128)
    MLXQ_M(float, 8, 32) MLXQ_M(float, 8, 64) MLXQ_M(float, 8, 128)
  }
#undef MLXQ_M
  return set_error(MLXQ_EINVAL, "qmm: unsupported bits=%d group_size=%d", bits, gs);
}

}  // namespace mlxq
