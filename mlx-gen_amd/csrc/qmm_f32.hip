// qmm_f32.hip — large-M quantized GEMM in f32 (y[M,N] = x[M,K] . W^T, M > 8) on gfx950 matrix
// cores, for the operand mixes MLX computes in f32: f32 activations (FLUX.1's f32 residual stream,
// reference mlx-gen-flux/src/model.rs:407-410 into src/adapters.rs:301-317), fp16 activations
// against bf16 scales (SDXL's fp16 U-Net and CLIP encoders over bf16-packed weights,
// mlx-gen-sdxl/src/model.rs:216,283-296: promote(fp16, bf16) is f32) and/or f32 scales.
//
// Semantics: MLX's quantized_matmul casts x, scales and biases to their result type (f32 here),
// dequantizes every weight in f32 and accumulates in f32.  gfx950 has no f32 matrix rate worth
// using (157 TFLOP/s dense), so each f32 operand is carried as two bf16 values whose sum holds it
// to 16 significant bits:
//     v_hi = bf16(v),  v_lo = bf16(v - v_hi)      (both round to nearest even)
// and each product as three bf16 MFMAs accumulated in f32:
//     x.w ~= x_hi.w_hi + x_hi.w_lo + x_lo.w_hi
// The dropped x_lo.w_lo term and the two representation errors are each below 2^-16 of |x.w|, so
// the result is within ~1e-5 relative (Frobenius) of the f32 product, against ~1e-3 for a plain
// bf16 product.  With bf16 activations (f32 scales) x_lo is zero and the third pass is skipped;
// fp16 activations split exactly (x_hi + x_lo == x), so against exact bf16 code operands (the
// factored kernel) their products are exact.
// Weights are dequantized exactly as fma(code, scale, bias) in f32 (scale and bias widened
// exactly from bf16), then split.  That three-pass kernel serves group size 32 and the LoKr dense
// product; group sizes 64 and 128 take the factored kernel further down (qmm_f32c_kernel: the
// codes themselves as exact bf16 operands, two passes for f32 x).
//
// Structure: a workgroup of 8 waves (2 x 4, 64 x 64 each) per 128 x 256 output tile (the LoKr
// dense product: 4 waves, 2 x 2, per 128 x 128 tile), K advanced BK = 32 at a time through a
// double-buffered LDS holding the four bf16 tiles x_hi, x_lo, w_hi, w_lo of a step (48 KB per
// buffer, one workgroup per CU; 32 KB and two for the dense product).  Activations are split and weights
// dequantized and split once per workgroup as they are written to LDS; every wave reads its
// sub-tile's fragments from there.  Global loads run two steps ahead of their use (two register
// slots), so a step's MFMAs and the next step's split/dequant never wait on memory.  Rows of BK bf16 with the 16-byte chunks XOR-swizzled.
// Fragment mapping for v_mfma_f32_32x32x16_bf16: lane l supplies row (l & 31) and 8 consecutive k
// at chunk 2 kk + (l >> 5) for both operands; with the weights as the A operand the f32x16 result
// holds activation row (l & 31) and weight rows 8 (v >> 2) + 4 (l >> 5) + (v & 3).
// Tile order: groups of 8 M-tiles by all N-tiles (M fastest), so the workgroups in flight share
// weight panels and a few activation panels; consecutive workgroup ids are spread over the 8 XCDs,
// so the order is remapped to give each XCD a contiguous slice of it.
#include <type_traits>

#include "mlxq_common.h"

namespace mlxq {

namespace {

constexpr int kF32BM = 128;
constexpr int kF32GroupM = 8;

// The f32 epilogue of LinearBase::forward and the caller's activation (reference
// src/adapters.rs:318-320, mlx-gen-flux/src/transformer.rs:975) on one output: y + bias in f32 (a
// -0 bias when there is none, the identity for every value), then the activation ACT in f32 —
// the elementwise epilogue kernel's arithmetic.
template <bool EPI, int ACT>
__device__ __forceinline__ float f32_finish(float o, float bv) {
  if constexpr (EPI) {
    o += bv;
    if constexpr (ACT == MLXQ_ACT_GELU || ACT == MLXQ_ACT_GELU_EXACT) o = gelu_erf(o);
    else if constexpr (ACT == MLXQ_ACT_GELU_TANH) o = gelu_tanh<false>(o);
  }
  return o;
}

// Runs the tile's store loop once, instantiated for the launch's activation, so the activation
// is chosen once per tile rather than tested per output (a branch per output before).
template <bool EPI, typename Store>
__device__ __forceinline__ void f32_store_dispatch(int act, Store&& store) {
  if constexpr (EPI) {
    if (act == MLXQ_ACT_GELU || act == MLXQ_ACT_GELU_EXACT) store(std::integral_constant<int, MLXQ_ACT_GELU_EXACT>{});
    else if (act == MLXQ_ACT_GELU_TANH) store(std::integral_constant<int, MLXQ_ACT_GELU_TANH>{});
    else store(std::integral_constant<int, MLXQ_ACT_NONE>{});
  } else {
    store(std::integral_constant<int, MLXQ_ACT_NONE>{});
  }
}

// Byte offset of 16-byte chunk `chunk` of tile row `row` for rows of BK bf16: 128-byte rows XOR
// the chunk with row & 7, 64-byte rows with (row >> 1) & 3, so the fragment reads (one chunk of 8
// or more consecutive rows) fall on distinct banks.
template <int BK>
__device__ __forceinline__ int swz32(int row, int chunk) {
  if constexpr (BK == 64) return row * 128 + ((chunk ^ (row & 7)) << 4);
  else return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

// (v0, v1) -> {hi, lo}: the packed bf16 pairs of the two-term split of two values.
__device__ __forceinline__ u32x2 split2(float v0, float v1) {
  const uint32_t hi = pack_bf16x2(v0, v1);
  return u32x2{hi, pack_bf16x2(v0 - __uint_as_float(hi << 16), v1 - __uint_as_float(hi & 0xffff0000u))};
}

// Activation storage: f32 and fp16 values do not fit bf16 and carry a low part in the two-term
// split (for fp16 the split is exact: 11 significant bits are hi's 8 plus a remainder of at most
// 4); an 8-value chunk is W 16-byte loads (2 for f32, 1 for bf16 and fp16).
template <typename XT>
struct XStore {
  static constexpr bool LO = !std::is_same<XT, uint16_t>::value;
  static constexpr int W = std::is_same<XT, float>::value ? 2 : 1;
  // Values 2e and 2e + 1 of a chunk, as f32.
  static __device__ __forceinline__ void pair(const u32x4 (&a)[W], int e, float& v0, float& v1) {
    if constexpr (std::is_same<XT, float>::value) {
      v0 = __uint_as_float(a[e >> 1][2 * (e & 1)]);
      v1 = __uint_as_float(a[e >> 1][2 * (e & 1) + 1]);
    } else if constexpr (std::is_same<XT, _Float16>::value) {
      v0 = f16_lo(a[0][e]);
      v1 = f16_hi(a[0][e]);
    } else {
      v0 = __uint_as_float(a[0][e] << 16);
      v1 = __uint_as_float(a[0][e] & 0xffff0000u);
    }
  }
};

__device__ __forceinline__ void f32_tile_coords(int64_t bid, int64_t tiles_m, int64_t tiles_n,
                                                int64_t& tm, int64_t& tn) {
  const int64_t T = tiles_m * tiles_n;
  const int64_t per = T / 8;
  int64_t L = bid;
  if (bid < per * 8) L = (bid % 8) * per + bid / 8;
  const int64_t span = kF32GroupM * tiles_n;
  const int64_t g = L / span;
  const int64_t gm0 = g * kF32GroupM;
  const int64_t gsz = tiles_m - gm0 < kF32GroupM ? tiles_m - gm0 : kF32GroupM;
  const int64_t idx = L - g * span;
  tm = gm0 + idx % gsz;
  tn = idx / gsz;
}

}  // namespace

// XT: activation storage (float, _Float16, or uint16_t bf16 bits); SB: scale/bias storage.  y is
// f32.
// WAVES: 4 (2 x 2 waves of 64 x 64) or 8 (2 x 4 waves of 64 x 32, two per SIMD).  EPI: the f32
// epilogue (dense bias in its own dtype, then the f32 activation) is applied before the store.
// WT: uint32_t for packed codes (wq, scales, biases); uint16_t (bf16) or float for a dense [N, K]
// weight matrix passed in wq's place (scales, biases, BITS and GS unused), the LoKr residual's
// x . delta^T.  A dense f32 matrix against bf16 activations is rounded to bf16 first (MLX casts
// the delta to the activation dtype).
template <typename XT, typename SB, int BITS, int GS, int WAVES, int BN, int BK, bool EPI,
          typename WT = uint32_t>
__global__ __launch_bounds__(WAVES * 64) void qmm_f32_kernel(const XT* __restrict__ x, int64_t M,
                                                         int64_t K, const uint32_t* __restrict__ wq,
                                                         const SB* __restrict__ scales,
                                                         const SB* __restrict__ biases, int64_t N,
                                                         float* __restrict__ y, F32Epilogue epi) {
  constexpr bool XLO = XStore<XT>::LO;  // activations carry a low part
  constexpr bool DENSE = !std::is_same<WT, uint32_t>::value;
  // Weights carry a low part unless they are bf16 values: dequantized codes are f32, and a dense
  // f32 matrix keeps its low part against f32 activations.
  constexpr bool WLO = !DENSE || (std::is_same<WT, float>::value && XLO);
  constexpr int BM = kF32BM, NT = WAVES * 64;
  constexpr int WGN = WAVES / 2;             // waves along N
  constexpr int WM = BM / 2, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  constexpr int CPR = BK / 8;                // 16-byte bf16 chunks per tile row
  constexpr int A_LD = BM * CPR / NT;        // 8-element activation chunks per thread per step
  constexpr int CPT = BN * BK / NT;          // codes per thread per step
  constexpr int WPT = CPT * BITS / 32;       // their packed words
  constexpr int PPR = BK / CPT;              // threads per weight row
  constexpr int TA = BM * BK * 2, TB = BN * BK * 2;  // bytes of one activation / weight tile
  constexpr int DV = DENSE ? CPT * (int)sizeof(WT) / 16 : 1;  // 16-byte loads of dense weights
  static_assert(A_LD >= 1 && TM >= 1 && TN >= 1 && CPT >= 8 && CPT <= 32 && PPR >= 1, "tile shape");
  // Per buffer: x_hi, x_lo, w_hi, w_lo.
  __shared__ __attribute__((aligned(16))) unsigned char smem[2][2 * TA + 2 * TB];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int64_t tm, tn;
  f32_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t bm0 = tm * BM, bn0 = tn * BN;
  const int64_t kwords = K * BITS / 32;
  const int64_t groups = K / GS;
  const int ksteps = (int)((K + BK - 1) / BK);

  // Staging registers, two slots (steps of even / odd parity): activation chunks (8 values each:
  // two 16-byte f32 loads or one bf16 load) and packed code chunks with their group's scale and
  // bias.  The loads are unconditional (rows past M / N are clamped; their products only reach
  // outputs that are never stored, and every step's k range lies inside K), so the loop is
  // straight-line code and each wait covers exactly the loads it needs.
  u32x4 a_reg[2][A_LD][XStore<XT>::W];
  uint32_t b_reg[2][WPT];
  float s_reg[2], z_reg[2];
  [[maybe_unused]] u32x4 d_reg[2][DV];

  auto load_global = [&](int kt, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + NT * i;
      const int row = id / CPR, c = id % CPR;
      const int64_t m = bm0 + row < M ? bm0 + row : M - 1;
      const int64_t k = k0 + c * 8;  // K % 32 == 0: a chunk never straddles K
#pragma unroll
      for (int h = 0; h < XStore<XT>::W; ++h) a_reg[sl][i][h] = reinterpret_cast<const u32x4*>(x + m * K + k)[h];
    }
    const int row = tid / PPR, part = tid % PPR;
    const int64_t n = bn0 + row < N ? bn0 + row : N - 1;
    const int64_t kc = k0 + part * CPT;
    if constexpr (DENSE) {  // CPT consecutive values of one weight row
      const u32x4* src = reinterpret_cast<const u32x4*>(reinterpret_cast<const WT*>(wq) + n * K + kc);
#pragma unroll
      for (int q = 0; q < DV; ++q) d_reg[sl][q] = src[q];
    } else {  // CPT consecutive codes of one weight row (one group: CPT <= 32 <= group size)
      const uint32_t* src = wq + n * kwords + kc * BITS / 32;
      if constexpr (WPT == 1) {
        b_reg[sl][0] = src[0];
      } else {
#pragma unroll
        for (int q = 0; q < WPT; q += 2) {
          const u32x2 v = *reinterpret_cast<const u32x2*>(src + q);
          b_reg[sl][q] = v[0];
          b_reg[sl][q + 1] = v[1];
        }
      }
      const int64_t g = n * groups + kc / GS;
      s_reg[sl] = SBLoad<SB>::ld(scales, g);
      z_reg[sl] = SBLoad<SB>::ld(biases, g);
    }
  };

  auto store_lds = [&](int buf, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    unsigned char* Ah = smem[buf];
    unsigned char* Al = smem[buf] + TA;
    unsigned char* Bh = smem[buf] + 2 * TA;
    unsigned char* Bl = smem[buf] + 2 * TA + TB;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + NT * i;
      const int row = id / CPR, c = id % CPR;
      if constexpr (XLO) {
        u32x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v0, v1;
          XStore<XT>::pair(a_reg[sl][i], e, v0, v1);
          const u32x2 p = split2(v0, v1);
          hi[e] = p[0];
          lo[e] = p[1];
        }
        *reinterpret_cast<u32x4*>(Ah + swz32<BK>(row, c)) = hi;
        *reinterpret_cast<u32x4*>(Al + swz32<BK>(row, c)) = lo;
      } else {
        *reinterpret_cast<u32x4*>(Ah + swz32<BK>(row, c)) = a_reg[sl][i][0];
      }
    }
    if constexpr (DENSE) {
      const int row = tid / PPR, part = tid % PPR;
      const int c0 = part * CPT / 8;
#pragma unroll
      for (int p = 0; p < CPT / 8; ++p) {
        if constexpr (std::is_same<WT, uint16_t>::value) {
          *reinterpret_cast<u32x4*>(Bh + swz32<BK>(row, c0 + p)) = d_reg[sl][p];
        } else {
          u32x4 hi, lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const u32x4& src = d_reg[sl][2 * p + (e >> 1)];
            const float v0 = __uint_as_float(src[2 * (e & 1)]), v1 = __uint_as_float(src[2 * (e & 1) + 1]);
            if constexpr (WLO) {
              const u32x2 q = split2(v0, v1);
              hi[e] = q[0];
              lo[e] = q[1];
            } else {
              hi[e] = pack_bf16x2(v0, v1);
            }
          }
          *reinterpret_cast<u32x4*>(Bh + swz32<BK>(row, c0 + p)) = hi;
          if constexpr (WLO) *reinterpret_cast<u32x4*>(Bl + swz32<BK>(row, c0 + p)) = lo;
        }
      }
    } else {
      const int row = tid / PPR, part = tid % PPR;
      const float s = s_reg[sl], z = z_reg[sl];
      // LDS chunk c holds k [8c, 8c + 8) of the step; this thread's codes start at chunk part*CPT/8.
      const int c0 = part * CPT / 8;
      if constexpr (BITS == 4) {
        // word q: codes 8q..8q+7 in natural order (low nibble first) -> chunk c0 + q
#pragma unroll
        for (int q = 0; q < WPT; ++q) {
          const uint32_t w = b_reg[sl][q];
          u32x4 hi, lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float c0f = (float)((w >> (8 * e)) & 0xfu);
            const float c1f = (float)((w >> (8 * e + 4)) & 0xfu);
            const u32x2 p = split2(fmaf(c0f, s, z), fmaf(c1f, s, z));
            hi[e] = p[0];
            lo[e] = p[1];
          }
          *reinterpret_cast<u32x4*>(Bh + swz32<BK>(row, c0 + q)) = hi;
          *reinterpret_cast<u32x4*>(Bl + swz32<BK>(row, c0 + q)) = lo;
        }
      } else {
        // words 2p, 2p+1: codes 8p..8p+7 -> chunk c0 + p
        static_assert(WPT % 2 == 0, "Q8 words come in pairs");
#pragma unroll
        for (int p = 0; p < WPT / 2; ++p) {
          u32x4 hi, lo;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t w = b_reg[sl][2 * p + h];
            const u32x2 p0 = split2(fmaf((float)(w & 0xffu), s, z), fmaf((float)((w >> 8) & 0xffu), s, z));
            const u32x2 p1 = split2(fmaf((float)((w >> 16) & 0xffu), s, z), fmaf((float)(w >> 24), s, z));
            hi[2 * h] = p0[0];
            lo[2 * h] = p0[1];
            hi[2 * h + 1] = p1[0];
            lo[2 * h + 1] = p1[1];
          }
          *reinterpret_cast<u32x4*>(Bh + swz32<BK>(row, c0 + p)) = hi;
          *reinterpret_cast<u32x4*>(Bl + swz32<BK>(row, c0 + p)) = lo;
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

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  const int r32 = lane & 31, half = lane >> 5;
  // Step kt's products from LDS buffer kt & 1.
  auto mfma_step = [&](int buf) {
    const unsigned char* Ah = smem[buf];
    const unsigned char* Al = smem[buf] + TA;
    const unsigned char* Bh = smem[buf] + 2 * TA;
    const unsigned char* Bl = smem[buf] + 2 * TA + TB;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c = kk * 2 + half;
      bf16x8 ah[TM], al[TM], bh[TN], bl[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        ah[i] = *reinterpret_cast<const bf16x8*>(Ah + swz32<BK>(wm * WM + i * 32 + r32, c));
        if constexpr (XLO) al[i] = *reinterpret_cast<const bf16x8*>(Al + swz32<BK>(wm * WM + i * 32 + r32, c));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        bh[j] = *reinterpret_cast<const bf16x8*>(Bh + swz32<BK>(wn * WN + j * 32 + r32, c));
        if constexpr (WLO) bl[j] = *reinterpret_cast<const bf16x8*>(Bl + swz32<BK>(wn * WN + j * 32 + r32, c));
      }
      // Three passes over the independent accumulators, so no MFMA waits on its predecessor.
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[j], ah[i], acc[i][j], 0, 0, 0);
      if constexpr (WLO) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bl[j], ah[i], acc[i][j], 0, 0, 0);
      }
      if constexpr (XLO) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[j], al[i], acc[i][j], 0, 0, 0);
      }
    }
  };
  // Software pipeline, global loads two steps ahead of their use: iteration kt issues step kt+2's
  // loads into the register slot step kt has vacated, then runs step kt's MFMAs from one LDS buffer
  // while step kt+1's operands (loaded during iteration kt-1) are split, dequantized and written
  // into the other, so the split/dequant VALU work overlaps the MFMAs instead of following them.
  // Past the last step the loads repeat the last step (in bounds, never used) and the writes fill
  // the idle buffer, which keeps the body free of branches.
  auto body = [&](int kt, auto SLOT, auto NSLOT) {
    load_global(kt + 2 < ksteps ? kt + 2 : ksteps - 1, SLOT);
    mfma_step(kt & 1);
    store_lds((kt + 1) & 1, NSLOT);
    __syncthreads();
  };
  load_global(0, S0{});
  load_global(ksteps > 1 ? 1 : 0, S1{});
  store_lds(0, S0{});
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < ksteps; kt += 2) {
    body(kt, S0{}, S1{});
    body(kt + 1, S1{}, S0{});
  }
  if (kt < ksteps) body(kt, S0{}, S1{});

  // acc[i][j] element v: column m = row of A's fragment (lane & 31), rows n = 8 (v >> 2) +
  // 4 half + (v & 3) of B's fragment: the weight operand is MFMA's A side, so each lane holds four
  // runs of 4 consecutive n for one m and stores them as 16-byte rows.
  const bool vec_ok = (N % 4) == 0;
  // The f32 epilogue (f32_finish): y + bias in f32, then the activation in f32.
  [[maybe_unused]] float bcol[TN][16];
  if constexpr (EPI) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t n = bn0 + wn * WN + j * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        const int64_t nc = n < N ? n : N - 1;  // columns past N are never stored
        bcol[j][v] = epi.bias == nullptr ? -0.0f
                     : epi.bias_bf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(epi.bias)[nc])
                                     : static_cast<const float*>(epi.bias)[nc];
      }
  }
  auto store = [&](auto A) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = bm0 + wm * WM + i * 32 + r32;
      if (m >= M) continue;
      float* yrow = y + m * N;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int64_t n = bn0 + wn * WN + j * 32 + 8 * a + 4 * half;
          f32x4 v;
#pragma unroll
          for (int b = 0; b < 4; ++b) v[b] = f32_finish<EPI, decltype(A)::value>(acc[i][j][4 * a + b], EPI ? bcol[j][4 * a + b] : 0.0f);
          if (vec_ok && n + 3 < N) {
            *reinterpret_cast<f32x4*>(yrow + n) = v;
          } else {
#pragma unroll
            for (int b = 0; b < 4; ++b)
              if (n + b < N) yrow[n + b] = v[b];
          }
        }
      }
    }
  };
  f32_store_dispatch<EPI>(epi.act, store);
}

// The factored form for group sizes 64 and 128: since
//     x . w = sum_g ( s_g * sum_{k in g} x_k c_k  +  b_g * X_g ),   X_g = sum_{k in g} x_k,
// the codes c (small integers, exact in bf16) are the weight operand and only the activations are
// split: x_hi.c + x_lo.c is two MFMA passes for f32 x (one for bf16 x) instead of three, with no
// dequantization or weight split.  Each group's product accumulates in `acc` (the first MFMA of a
// group starts from zero) and is folded into the running f32 sum y by two FMAs per output with the
// group's scale and bias (one per weight row) and activation sum (one per activation row), which
// the staging threads leave in two small LDS tables next to the step's tiles (with bf16 scales and
// K / GS a multiple of 16, one FMA: the bias term runs on the matrix cores, see BMF).  The loop is
// unrolled by the group's GS/32 steps, so group starts and ends are compile-time positions.
// Tiles, waves, buffers and the load pipeline are those of qmm_f32_kernel (128 x 256, 8 waves of
// 64 x 64, 32-deep K steps, loads two steps ahead).
template <typename XT, typename SB, int BITS, int GS, bool EPI, bool BMF, int WAVES, int BN>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void qmm_f32c_kernel(const XT* __restrict__ x, int64_t M, int64_t K,
                                                   const uint32_t* __restrict__ wq,
                                                   const SB* __restrict__ scales,
                                                   const SB* __restrict__ biases, int64_t N,
                                                   float* __restrict__ y, F32Epilogue epi) {
  constexpr bool XLO = XStore<XT>::LO;  // activations carry a low part
  constexpr int BK = 32;
  constexpr int BM = kF32BM, NT = WAVES * 64;
  constexpr int WGN = WAVES / 2;
  constexpr int WM = BM / 2, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  constexpr int CPR = BK / 8;                // 16-byte bf16 chunks per tile row
  constexpr int A_LD = BM * CPR / NT;        // activation chunks per thread per step (1 or 2)
  constexpr int CPT = BN * BK / NT;          // codes per thread per step (16)
  constexpr int WPT = CPT * BITS / 32;       // their packed words
  constexpr int PPR = BK / CPT;              // threads per weight row (2)
  constexpr int GSTEP = GS / BK;             // steps per group (2 or 4)
  constexpr int TA = BM * BK * 2, TB = BN * BK * 2;
  constexpr int OFF_SB = 2 * TA + TB, OFF_X = OFF_SB + BN * 8, BUF = OFF_X + BM * 4;
  static_assert(A_LD * NT == BM * CPR && CPT == 16 && GSTEP >= 2 && GSTEP % 2 == 0 && WPT >= 1, "tile shape");
  // Per buffer: x_hi, x_lo, codes, then the (s, b) pairs of the tile's weight rows and the
  // activation sums of its rows for the group the buffer's step closes.
  __shared__ __attribute__((aligned(16))) unsigned char smem[2][BUF];
  // BMF (bf16 scales, K / GS a multiple of 16): the bias term b.X goes to the matrix cores, 16
  // groups at a time: each group's bf16 biases per weight row and hi/lo split activation sums per
  // activation row wait in 16-group tables (rows of 32 bytes), and every 16th group adds
  // b[n, g..g+15] . X[g..g+15, m] into y with one MFMA pair per block.  The per-group fold is then
  // one FMA per output, y += s * acc.
  constexpr int BT = BN * 32, XT_ = BM * 32;
  static_assert(!BMF || std::is_same<SB, uint16_t>::value, "bias MFMA needs bf16 biases (exact bf16 operands)");
  __shared__ __attribute__((aligned(16))) unsigned char btab[BMF ? BT + 2 * XT_ : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int64_t tm, tn;
  f32_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t bm0 = tm * BM, bn0 = tn * BN;
  const int64_t kwords = K * BITS / 32;
  const int64_t groups = K / GS;
  const int ksteps = (int)(K / BK);  // a multiple of GSTEP (K % GS == 0)

  // Staging registers, two slots (see qmm_f32_kernel): thread tid stages activation chunks
  // id = tid + NT i (row id / 4, chunk id % 4), and codes CPT of weight row tid / 2 with that row's
  // scale and bias.
  u32x4 a_reg[2][A_LD][XStore<XT>::W];
  uint32_t b_reg[2][WPT];
  float s_reg[2], z_reg[2];
  float xrun[A_LD];  // each staged row's activation sum over the current group's steps so far

  auto load_global = [&](int kt, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + NT * i;
      const int row = id / CPR, c = id % CPR;
      const int64_t m = bm0 + row < M ? bm0 + row : M - 1;
#pragma unroll
      for (int h = 0; h < XStore<XT>::W; ++h)
        a_reg[sl][i][h] = reinterpret_cast<const u32x4*>(x + m * K + k0 + c * 8)[h];
    }
    const int row = tid / PPR, part = tid % PPR;
    const int64_t n = bn0 + row < N ? bn0 + row : N - 1;
    const int64_t kc = k0 + part * CPT;
    const uint32_t* src = wq + n * kwords + kc * BITS / 32;
    if constexpr (WPT == 1) {
      b_reg[sl][0] = src[0];
    } else {
#pragma unroll
      for (int q = 0; q < WPT; q += 2) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(src + q);
        b_reg[sl][q] = v[0];
        b_reg[sl][q + 1] = v[1];
      }
    }
    const int64_t g = n * groups + kc / GS;
    s_reg[sl] = SBLoad<SB>::ld(scales, g);
    z_reg[sl] = SBLoad<SB>::ld(biases, g);
  };

  // Step `POS` (its position in its group `grp`) from register slot SLOT into LDS buffer buf.
  auto store_lds = [&](int buf, auto SLOT, auto POS, int grp) {
    constexpr int sl = decltype(SLOT)::value;
    constexpr int pos = decltype(POS)::value;
    unsigned char* Ah = smem[buf];
    unsigned char* Al = smem[buf] + TA;
    unsigned char* Bc = smem[buf] + 2 * TA;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = tid + NT * i;
      const int row = id / CPR, c = id % CPR;
      float t = 0.0f;
      if constexpr (XLO) {
        u32x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v0, v1;
          XStore<XT>::pair(a_reg[sl][i], e, v0, v1);
          t += v0 + v1;
          const u32x2 p = split2(v0, v1);
          hi[e] = p[0];
          lo[e] = p[1];
        }
        *reinterpret_cast<u32x4*>(Ah + swz32<BK>(row, c)) = hi;
        *reinterpret_cast<u32x4*>(Al + swz32<BK>(row, c)) = lo;
      } else {
        const u32x4 v = a_reg[sl][i][0];
#pragma unroll
        for (int e = 0; e < 4; ++e) t += __uint_as_float(v[e] << 16) + __uint_as_float(v[e] & 0xffff0000u);
        *reinterpret_cast<u32x4*>(Ah + swz32<BK>(row, c)) = v;
      }
      // the row's sum over this step: its 4 chunks sit in 4 consecutive lanes
      t += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0xb1, 0xf, 0xf, true));
      t += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x4e, 0xf, 0xf, true));
      xrun[i] = pos == 0 ? t : xrun[i] + t;
      if constexpr (pos == GSTEP - 1) {
        if (c == 0) {
          reinterpret_cast<float*>(smem[buf] + OFF_X)[row] = xrun[i];
          if constexpr (BMF) {
            const uint16_t hb = f32_to_bf16_bits(xrun[i]);
            const uint16_t lb = f32_to_bf16_bits(xrun[i] - bf16_bits_to_f32(hb));
            reinterpret_cast<uint16_t*>(btab + BT)[row * 16 + (grp & 15)] = hb;
            reinterpret_cast<uint16_t*>(btab + BT + XT_)[row * 16 + (grp & 15)] = lb;
          }
        }
      }
    }
    const int row = tid / PPR, part = tid % PPR;
    const int c0 = part * CPT / 8;  // LDS chunk c holds k [8c, 8c + 8) of the step
    if constexpr (BITS == 4) {
      // word q: codes 8q..8q+7 in natural order (low nibble first) -> chunk c0 + q, as bf16(c).
      // The nibbles are split into bytes and interleaved back into code order (bytes c0..c3 and
      // c4..c7); a byte c <= 15 read as OCP fp8 E4M3 is exactly c * 2^-9, so one scaled convert
      // turns two code bytes into two exact bf16 values: 9 VALU ops per word instead of 20.
#pragma unroll
      for (int q = 0; q < WPT; ++q) {
        const uint32_t w = b_reg[sl][q];
        const uint32_t ev = w & 0x0f0f0f0fu, od = (w >> 4) & 0x0f0f0f0fu;  // c0 c2 c4 c6 / c1 c3 c5 c7
        const uint32_t n0 = __builtin_amdgcn_perm(od, ev, 0x05010400u);     // c0 c1 c2 c3
        const uint32_t n1 = __builtin_amdgcn_perm(od, ev, 0x07030602u);     // c4 c5 c6 c7
        u32x4 cv;
        cv[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n0, 512.0f, false));
        cv[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n0, 512.0f, true));
        cv[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n1, 512.0f, false));
        cv[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n1, 512.0f, true));
        *reinterpret_cast<u32x4*>(Bc + swz32<BK>(row, c0 + q)) = cv;
      }
    } else {
#pragma unroll
      for (int p = 0; p < WPT / 2; ++p) {
        u32x4 cv;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t w = b_reg[sl][2 * p + h];
          cv[2 * h] = pack_bf16x2((float)(w & 0xffu), (float)((w >> 8) & 0xffu));
          cv[2 * h + 1] = pack_bf16x2((float)((w >> 16) & 0xffu), (float)(w >> 24));
        }
        *reinterpret_cast<u32x4*>(Bc + swz32<BK>(row, c0 + p)) = cv;
      }
    }
    if constexpr (pos == GSTEP - 1) {
      if (part == 0) {
        *reinterpret_cast<f32x2*>(smem[buf] + OFF_SB + row * 8) = f32x2{s_reg[sl], z_reg[sl]};
        if constexpr (BMF)
          reinterpret_cast<uint16_t*>(btab)[row * 16 + (grp & 15)] = (uint16_t)(__float_as_uint(z_reg[sl]) >> 16);
      }
    }
  };

  f32x16 acc[TM][TN], yv[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) yv[i][j][v] = 0.0f;

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  const int r32 = lane & 31, half = lane >> 5;
  // Step products from LDS buffer buf; the first MFMA of a group's first step starts from zero.
  auto mfma_step = [&](int buf, auto FIRST) {
    constexpr bool first = decltype(FIRST)::value;
    const unsigned char* Ah = smem[buf];
    const unsigned char* Al = smem[buf] + TA;
    const unsigned char* Bc = smem[buf] + 2 * TA;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c = kk * 2 + half;
      bf16x8 ah[TM], al[TM], bc[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        ah[i] = *reinterpret_cast<const bf16x8*>(Ah + swz32<BK>(wm * WM + i * 32 + r32, c));
        if constexpr (XLO) al[i] = *reinterpret_cast<const bf16x8*>(Al + swz32<BK>(wm * WM + i * 32 + r32, c));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) bc[j] = *reinterpret_cast<const bf16x8*>(Bc + swz32<BK>(wn * WN + j * 32 + r32, c));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (first && kk == 0) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bc[j], ah[i], f32x16{}, 0, 0, 0);
          else acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bc[j], ah[i], acc[i][j], 0, 0, 0);
        }
      if constexpr (XLO) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bc[j], al[i], acc[i][j], 0, 0, 0);
      }
    }
  };
  // y += s * acc + b * X for the group closed by buffer buf's step.  Element v of acc[i][j]:
  // activation row wm WM + 32 i + r32, weight row wn WN + 32 j + 8 (v >> 2) + 4 half + (v & 3).
  auto fold = [&](int buf, int grp) {
    const float* sb = reinterpret_cast<const float*>(smem[buf] + OFF_SB);
    const float* xs = reinterpret_cast<const float*>(smem[buf] + OFF_X);
    float xg[TM];
    if constexpr (!BMF) {
#pragma unroll
      for (int i = 0; i < TM; ++i) xg[i] = xs[wm * WM + i * 32 + r32];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int n0 = wn * WN + j * 32 + 8 * t + 4 * half;
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(sb + 2 * n0);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(sb + 2 * n0 + 4);
        const float sv[4] = {p0[0], p0[2], p1[0], p1[2]}, zv[4] = {p0[1], p0[3], p1[1], p1[3]};
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if constexpr (BMF) yv[i][j][4 * t + u] = fmaf(sv[u], acc[i][j][4 * t + u], yv[i][j][4 * t + u]);
            else yv[i][j][4 * t + u] = fmaf(sv[u], acc[i][j][4 * t + u], fmaf(zv[u], xg[i], yv[i][j][4 * t + u]));
          }
      }
    if constexpr (BMF) {
      if ((grp & 15) == 15) {  // the 16-group batch is complete: y += b . X on the matrix cores
        const unsigned char* bt = btab;
        const unsigned char* xh = btab + BT;
        const unsigned char* xl = btab + BT + XT_;
        bf16x8 bf[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(bt + (wn * WN + j * 32 + r32) * 32 + half * 16);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int rr = (wm * WM + i * 32 + r32) * 32 + half * 16;
          const bf16x8 ah = *reinterpret_cast<const bf16x8*>(xh + rr);
          const bf16x8 al = *reinterpret_cast<const bf16x8*>(xl + rr);
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            yv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], ah, yv[i][j], 0, 0, 0);
            yv[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], al, yv[i][j], 0, 0, 0);
          }
        }
      }
    }
  };
  // One group: GSTEP steps, loads two steps ahead (clamped to the last step past the end).
  auto body = [&](int kt, auto SLOT, auto NSLOT, auto POS) {
    constexpr int pos = decltype(POS)::value;
    load_global(kt + 2 < ksteps ? kt + 2 : ksteps - 1, SLOT);
    mfma_step(kt & 1, std::integral_constant<bool, pos == 0>{});
    if constexpr (pos == GSTEP - 1) fold(kt & 1, kt / GSTEP);
    store_lds((kt + 1) & 1, NSLOT, std::integral_constant<int, (pos + 1) % GSTEP>{}, (kt + 1) / GSTEP);
    __syncthreads();
  };
  load_global(0, S0{});
  load_global(ksteps > 1 ? 1 : 0, S1{});
  store_lds(0, S0{}, std::integral_constant<int, 0>{}, 0);
  __syncthreads();
  for (int kt = 0; kt < ksteps; kt += GSTEP) {
    body(kt, S0{}, S1{}, std::integral_constant<int, 0>{});
    body(kt + 1, S1{}, S0{}, std::integral_constant<int, 1>{});
    if constexpr (GSTEP == 4) {
      body(kt + 2, S0{}, S1{}, std::integral_constant<int, 2>{});
      body(kt + 3, S1{}, S0{}, std::integral_constant<int, 3>{});
    }
  }

  // Epilogue as in qmm_f32_kernel: y + bias in f32, then the activation in f32.
  const bool vec_ok = (N % 4) == 0;
  [[maybe_unused]] float bcol[TN][16];
  if constexpr (EPI) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t n = bn0 + wn * WN + j * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        const int64_t nc = n < N ? n : N - 1;  // columns past N are never stored
        bcol[j][v] = epi.bias == nullptr ? -0.0f
                     : epi.bias_bf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(epi.bias)[nc])
                                     : static_cast<const float*>(epi.bias)[nc];
      }
  }
  auto store = [&](auto A) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = bm0 + wm * WM + i * 32 + r32;
      if (m >= M) continue;
      float* yrow = y + m * N;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int64_t n = bn0 + wn * WN + j * 32 + 8 * a + 4 * half;
          f32x4 v;
#pragma unroll
          for (int b = 0; b < 4; ++b) v[b] = f32_finish<EPI, decltype(A)::value>(yv[i][j][4 * a + b], EPI ? bcol[j][4 * a + b] : 0.0f);
          if (vec_ok && n + 3 < N) {
            *reinterpret_cast<f32x4*>(yrow + n) = v;
          } else {
#pragma unroll
            for (int b = 0; b < 4; ++b)
              if (n + b < N) yrow[n + b] = v[b];
          }
        }
      }
    }
  };
  f32_store_dispatch<EPI>(epi.act, store);
}

template <typename XT, typename SB, int BITS, int GS>
static int launch_qmm_f32(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                          const void* b, int64_t N, void* y, const F32Epilogue& epi, hipStream_t st) {
  // 8 waves (2 x 4 of 64 x 64) on 128 x 256 tiles with 32-deep K steps (96 KB of LDS, one
  // workgroup per CU).  With loads two steps ahead, same-box A/B on the FLUX shapes (f32 x, Q4
  // g64, up / down in ms): this form 1.103 / 1.346; 4 waves on 128 x 128 (two workgroups per CU)
  // 1.199 / 1.348; 8 waves on 128 x 128 1.200 / 1.362; 4 waves on 128 x 256 1.433 / 1.729.
  // (Before the prefetch rework the 128 x 128 four-wave form had led: 1225 us on the up shape
  // against 1279 with 8 waves, 1336 with 128 x 256 tiles, 1614 with 64-deep steps.)
  constexpr int WAVES = 8, BN = 256, BK = 32;
  const int64_t tiles = ((M + kF32BM - 1) / kF32BM) * ((N + BN - 1) / BN);
  if (tiles == 0) return MLXQ_OK;
  if (tiles > 0x7fffffff) return set_error(MLXQ_EINVAL, "qmm_f32: problem too large");
  if constexpr (GS >= 64) {  // the factored form (codes as the weight operand)
    const bool epi_on = epi.bias || epi.act != MLXQ_ACT_NONE;
    const bool bmf = std::is_same<SB, uint16_t>::value && (K / GS) % 16 == 0;
    // 8 waves on 128 x 256 tiles, as the three-pass kernel.  4 waves on 128 x 128 (two workgroups
    // per CU, so the two waves of a SIMD fold at different times) measured slower on the FLUX
    // shapes (same box: up 0.850 -> 0.926 ms, down 0.948 -> 1.020 ms).
    constexpr int CW = 8, CBN = 256;
    const int64_t ctiles = ((M + kF32BM - 1) / kF32BM) * ((N + CBN - 1) / CBN);
#define MLXQ_F32C(E, B)                                                                                 \
  hipLaunchKernelGGL((qmm_f32c_kernel<XT, SB, BITS, GS, E, B, CW, CBN>), dim3((unsigned)ctiles), dim3(CW * 64), 0, st, \
                     (const XT*)x, M, K, wq, (const SB*)s, (const SB*)b, N, (float*)y, epi)
    if constexpr (std::is_same<SB, uint16_t>::value) {
      if (bmf) {
        if (epi_on) MLXQ_F32C(true, true);
        else MLXQ_F32C(false, true);
        return check_launch("qmm_f32");
      }
    }
    if (epi_on) MLXQ_F32C(true, false);
    else MLXQ_F32C(false, false);
#undef MLXQ_F32C
    return check_launch("qmm_f32");
  }
  if (epi.bias || epi.act != MLXQ_ACT_NONE)
    hipLaunchKernelGGL((qmm_f32_kernel<XT, SB, BITS, GS, WAVES, BN, BK, true>), dim3((unsigned)tiles),
                       dim3(WAVES * 64), 0, st, (const XT*)x, M, K, wq, (const SB*)s, (const SB*)b, N,
                       (float*)y, epi);
  else
    hipLaunchKernelGGL((qmm_f32_kernel<XT, SB, BITS, GS, WAVES, BN, BK, false>), dim3((unsigned)tiles),
                       dim3(WAVES * 64), 0, st, (const XT*)x, M, K, wq, (const SB*)s, (const SB*)b, N,
                       (float*)y, epi);
  return check_launch("qmm_f32");
}

template <typename XT, typename SB>
static int qmm_f32_bits_gs(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                           const void* b, int64_t N, int gs, int bits, void* y, const F32Epilogue& epi,
                           hipStream_t st) {
#define MLXQ_F(B, G) \
  if (bits == B && gs == G) return launch_qmm_f32<XT, SB, B, G>(x, M, K, wq, s, b, N, y, epi, st);
  MLXQ_F(4, 32) MLXQ_F(4, 64) MLXQ_F(4, 128) MLXQ_F(8, 32) MLXQ_F(8, 64) MLXQ_F(8, 128)
#undef MLXQ_F
  return set_error(MLXQ_EINVAL, "qmm_f32: unsupported bits=%d group_size=%d", bits, gs);
}

int run_qmm_f32(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y, hipStream_t st,
                const F32Epilogue& epi) {
  if (x_dtype == MLXQ_BFLOAT16 && sb_dtype == MLXQ_BFLOAT16)
    return set_error(MLXQ_EINVAL, "qmm_f32: bf16 operands take the bf16 GEMM");
  if (x_dtype == MLXQ_FLOAT32) {
    if (sb_dtype == MLXQ_BFLOAT16)
      return qmm_f32_bits_gs<float, uint16_t>(x, M, K, wq, s, b, N, gs, bits, y, epi, st);
    return qmm_f32_bits_gs<float, float>(x, M, K, wq, s, b, N, gs, bits, y, epi, st);
  }
  if (x_dtype == MLXQ_FLOAT16) {
    if (sb_dtype == MLXQ_BFLOAT16)
      return qmm_f32_bits_gs<_Float16, uint16_t>(x, M, K, wq, s, b, N, gs, bits, y, epi, st);
    return qmm_f32_bits_gs<_Float16, float>(x, M, K, wq, s, b, N, gs, bits, y, epi, st);
  }
  return qmm_f32_bits_gs<uint16_t, float>(x, M, K, wq, s, b, N, gs, bits, y, epi, st);
}

// y[M, N] (f32) = x . d^T for a dense [N, K] matrix d (bf16 or f32; cast to bf16 against bf16
// x), on the same tiles: one bf16 pass for bf16 x with a bf16 (or bf16-cast) d, two for f32 x
// with bf16 d (d is exact in bf16), three for f32 x with f32 d.  K % 32 == 0.
int run_dense_f32(const void* x, int x_dtype, int64_t M, int64_t K, const void* d, int d_dtype,
                  int64_t N, float* y, hipStream_t st) {
  constexpr int WAVES = 4, BN = 128, BK = 32;
  if (K % BK != 0) return set_error(MLXQ_EINVAL, "dense product: K=%lld is not a multiple of 32", (long long)K);
  const int64_t tiles = ((M + kF32BM - 1) / kF32BM) * ((N + BN - 1) / BN);
  if (tiles == 0) return MLXQ_OK;
  if (tiles > 0x7fffffff) return set_error(MLXQ_EINVAL, "dense product: problem too large");
  const F32Epilogue none{};
#define MLXQ_D(XT, WT)                                                                                    \
  hipLaunchKernelGGL((qmm_f32_kernel<XT, float, 4, 32, WAVES, BN, BK, false, WT>), dim3((unsigned)tiles), \
                     dim3(WAVES * 64), 0, st, (const XT*)x, M, K, (const uint32_t*)d, nullptr, nullptr, N, y, none)
  if (x_dtype == MLXQ_BFLOAT16) {
    if (d_dtype == MLXQ_BFLOAT16) MLXQ_D(uint16_t, uint16_t);
    else MLXQ_D(uint16_t, float);
  } else {
    if (d_dtype == MLXQ_BFLOAT16) MLXQ_D(float, uint16_t);
    else MLXQ_D(float, float);
  }
#undef MLXQ_D
  return check_launch("dense_f32");
}

}  // namespace mlxq
