// qmm_wide.hip — the main large-M quantized GEMM for gfx950 (K % 64 == 0).
//
// y[M,N] = x[M,K] . W^T with W dequantized to bf16 (round_bf16(fma(code, scale, bias))) and
// v_mfma_f32_32x32x16_bf16 accumulating in f32.
//
// Workgroup: WAVES waves (8 by default: two per SIMD, so one wave's VALU/LDS work overlaps the
// other's MFMAs), block tile 256 (M) x 256 (N), K advanced 64 per step.  The waves split the tile
// along N only: wave w owns columns [w*256/WAVES, (w+1)*256/WAVES) of all 256 rows.
//   * weights: every lane loads its own packed words straight into registers (one 16-byte
//     buffer load per 32-column sub-tile per K step for Q4, two for Q8) and dequantizes them into
//     the MFMA operand registers — no LDS round trip, and each weight is dequantized exactly once
//     per workgroup because no two waves share columns;
//   * activations: the 256x64 bf16 tile is staged global -> registers -> LDS through a 3-deep
//     ring (one barrier per K step) and every wave reads all of it.  16-byte chunks are
//     XOR-swizzled by f(row) = (row & 7) ^ ((row >> 3) & 1), which keeps both the 16-lane
//     fragment reads (16 rows, one chunk) and the row-wise tile writes on distinct banks;
//   * the MFMA takes the weight fragment as its A operand (rows = n) and the activation fragment
//     as B (columns = m), so each lane's f32x16 result holds 4 runs of 4 consecutive n for one m
//     and the epilogue writes 8-byte (4 x bf16) row segments directly.
// Within a K step, lane half h (lane >> 5) covers k in [8(4h+kk), 8(4h+kk)+8) for MFMA kk = 0..3,
// i.e. packed words 4h..4h+3 of the row's 8-word (Q4) K step — one contiguous load.
// Q4 dequant: lo = w & 0x0f0f0f0f holds the even codes in its bytes, w & 0xf0f0f0f0 the odd codes
// times 16, so each code is one v_cvt_f32_ubyteN and one FMA (with scale/16 for the odd codes —
// an exact power-of-two rescale, so fma(16c, s/16, b) == fma(c, s, b) bit for bit).
//
// Tile order is XCD-aware: workgroups are dispatched round-robin over the 8 XCDs, so consecutive
// ids are remapped to give each XCD a contiguous slice of a grouped (4 M-tiles x all N-tiles)
// tile order, keeping the activation and weight tiles a slice shares resident in that XCD's L2.
#include <type_traits>

#include "mlxq_common.h"

namespace mlxq {

namespace {

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kGroupM = 4;
constexpr int kBufferFlags = 0x00020000;  // raw buffer resource word 3 for gfx9-family loads

__device__ __forceinline__ void tile_coords(int64_t bid, int64_t tiles_m, int64_t tiles_n,
                                            int64_t& tm, int64_t& tn) {
  const int64_t T = tiles_m * tiles_n;
  const int64_t per = T / 8;
  int64_t L = bid;
  if (bid < per * 8) L = (bid % 8) * per + bid / 8;
  const int64_t span = kGroupM * tiles_n;
  const int64_t g = L / span;
  const int64_t gm0 = g * kGroupM;
  const int64_t gsz = tiles_m - gm0 < kGroupM ? tiles_m - gm0 : kGroupM;
  const int64_t idx = L - g * span;
  tm = gm0 + idx % gsz;
  tn = idx / gsz;
}

__device__ __forceinline__ int swz_f(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <int B>
__device__ __forceinline__ float ubyte(uint32_t v) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// Dequantize the 8 codes of k-run [8(4h+kk), +8) into a bf16x8 MFMA operand.
// s16 = s/16 (exact) pairs with the odd Q4 codes, which are extracted still shifted left by 4.
template <int BITS>
__device__ __forceinline__ bf16x8 dequant8(const uint32_t* w, int kk, float s, float s16, float z) {
  u32x4 o;
  if constexpr (BITS == 4) {
    const uint32_t v = w[kk];
    const uint32_t lo = v & 0x0f0f0f0fu, hi = v & 0xf0f0f0f0u;
    o[0] = pack_bf16x2(fmaf(ubyte<0>(lo), s, z), fmaf(ubyte<0>(hi), s16, z));
    o[1] = pack_bf16x2(fmaf(ubyte<1>(lo), s, z), fmaf(ubyte<1>(hi), s16, z));
    o[2] = pack_bf16x2(fmaf(ubyte<2>(lo), s, z), fmaf(ubyte<2>(hi), s16, z));
    o[3] = pack_bf16x2(fmaf(ubyte<3>(lo), s, z), fmaf(ubyte<3>(hi), s16, z));
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t v = w[2 * kk + h];
      o[2 * h] = pack_bf16x2(fmaf(ubyte<0>(v), s, z), fmaf(ubyte<1>(v), s, z));
      o[2 * h + 1] = pack_bf16x2(fmaf(ubyte<2>(v), s, z), fmaf(ubyte<3>(v), s, z));
    }
  }
  return __builtin_bit_cast(bf16x8, o);
}

// Scale/bias element as raw bits.  The conversion to f32 happens one K step later (sb_to_f32 in
// take_b): converting right after the load would make the loop wait for it at the end of the
// step it was issued in.
template <typename SB>
__device__ __forceinline__ uint32_t load_sb_bits(__amdgpu_buffer_rsrc_t r, uint32_t idx) {
  if constexpr (sizeof(SB) == 2)
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, idx * 2u, 0, 0);
  else
    return __builtin_amdgcn_raw_buffer_load_b32(r, idx * 4u, 0, 0);
}
template <typename SB>
__device__ __forceinline__ float sb_to_f32(uint32_t bits) {
  if constexpr (sizeof(SB) == 2) return bf16_bits_to_f32(bits & 0xffffu);
  else return __uint_as_float(bits);
}

}  // namespace

// EPI selects the epilogue at compile time: 0 plain y = bf16(acc); 1 bias / rank-16 LoRA; 2 and 3
// the same followed by the exact-erf or the tanh GELU (EPI - 1 is the mlxq_activation).  One
// epilogue per instantiation keeps it small enough that the accumulator tile stays in registers.
template <typename SB, int BITS, int GS, int WAVES, int EPI>
__global__ __launch_bounds__(WAVES * 64, 1) void qmm_wide_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, const uint32_t* __restrict__ wq,
    const SB* __restrict__ scales, const SB* __restrict__ biases, int64_t N,
    uint16_t* __restrict__ y, QmmEpilogue epi, QmmBatch bat) {
  constexpr bool FUSED = EPI != 0;
  constexpr int ACT = FUSED ? EPI - 1 : MLXQ_ACT_NONE;
  constexpr int NT = WAVES * 64;
  constexpr int TMW = kBM / 32;          // m sub-tiles per wave (all 256 rows)
  constexpr int TNW = kBN / WAVES / 32;  // n sub-tiles per wave
  constexpr int WPL = BITS;              // packed words per lane per n sub-tile per K step (4 or 8)
  constexpr int A_PER = kBM * 8 / NT;    // 16-byte activation chunks per thread per K step
  constexpr int A_ROWS = NT / 8;         // row stride between a thread's chunks
  static_assert(TNW >= 1 && A_PER >= 1 && A_ROWS % 16 == 0, "tile/wave shape");
  __shared__ __attribute__((aligned(16))) unsigned char smem[3][kBM * 128];

  // Stacked launch: grid.y selects the matrix (expert); one matrix has all strides zero.
  if (gridDim.y > 1) {
    const int64_t e = blockIdx.y;
    x += e * bat.x;
    wq += e * bat.w;
    scales += e * bat.sb;
    biases += e * bat.sb;
    y += e * bat.y;
    if (epi.bias) epi.bias += e * bat.bias;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, r32 = lane & 31, half = lane >> 5;
  const int64_t tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int64_t tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t bm0 = tm * kBM, bn0 = tn * kBN;
  const int64_t kwords = K * BITS / 32;
  const int64_t groups = K / GS;
  const int KT = (int)(K / 64);
  const int64_t wn0 = bn0 + (int64_t)wave * (kBN / WAVES);
  // Dense bias of the tile's kBN columns: one value per thread, loaded now and parked in LDS for
  // the epilogue, so the epilogue issues no global loads (each would wait on the tile's pending
  // output stores too, since vmcnt counts stores).
  __shared__ float bias_lds[kBN];
  float bias_t = 0.0f;
  if constexpr (FUSED) {
    if (epi.bias && tid < kBN && bn0 + tid < N) bias_t = bf16_bits_to_f32(epi.bias[bn0 + tid]);
  }

  // Buffer resources: 32-bit offsets (the host checks every operand fits in 4 GiB).  Rows past
  // M / N are clamped so every offset stays inside its operand.
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (int)(uint32_t)(M * K * 2), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(wq), (short)0, (int)(uint32_t)(N * kwords * 4), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<SB*>(scales), (short)0, (int)(uint32_t)(N * groups * sizeof(SB)), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<SB*>(biases), (short)0, (int)(uint32_t)(N * groups * sizeof(SB)), kBufferFlags);

  // ---- activation staging: thread owns chunk (tid & 7) of rows (tid >> 3) + A_ROWS * i.
  const int a_row0 = tid >> 3, a_c = tid & 7;
  uint32_t a_goff[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int64_t r = bm0 + a_row0 + A_ROWS * i < M ? bm0 + a_row0 + A_ROWS * i : M - 1;
    a_goff[i] = (uint32_t)((r * K + a_c * 8) * 2);
  }
  const int a_lds = a_row0 * 128 + ((a_c ^ swz_f(a_row0)) << 4);
  u32x4 areg[A_PER];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      areg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, a_goff[i] + (uint32_t)kt * 128u, 0, 0));
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      *reinterpret_cast<u32x4*>(smem[buf] + a_lds + i * A_ROWS * 128) = areg[i];
  };

  // ---- weight rows of this lane: n = wn0 + 32 j + r32 (clamped to N-1 like A rows)
  uint32_t w_goff[TNW], g_base[TNW];
  bool n_ok[TNW];
#pragma unroll
  for (int j = 0; j < TNW; ++j) {
    const int64_t n = wn0 + j * 32 + r32;
    n_ok[j] = n < N;
    const int64_t nn = n_ok[j] ? n : N - 1;
    w_goff[j] = (uint32_t)((nn * kwords + half * WPL) * 4);
    g_base[j] = (uint32_t)(nn * groups);
  }
  uint32_t braw[TNW][WPL];
  uint32_t bs[TNW], bz[TNW];  // raw scale/bias bits
  auto load_b = [&](int kt) {
    const uint32_t g = (uint32_t)((kt * 64 + half * 32) / GS);
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
#pragma unroll
      for (int q = 0; q < WPL / 4; ++q) {
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, w_goff[j] + (uint32_t)kt * (8u * WPL) + 16u * q, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) braw[j][4 * q + e] = v[e];
      }
      bs[j] = load_sb_bits<SB>(rs, g_base[j] + g);
      bz[j] = load_sb_bits<SB>(rz, g_base[j] + g);
    }
  };

  // ---- fragment read offsets (LDS): row i*32 + r32, chunk 4h + kk
  int a_off[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a_off[kk] = r32 * 128 + (((4 * half + kk) ^ swz_f(r32)) << 4);

  f32x16 acc[TMW][TNW];
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // ---- software pipeline.  A tiles rotate through 3 LDS buffers: step kt reads buffer kt%3
  // while A(kt+1) is written to (kt+1)%3 at the top of the step and A(kt+2) is in flight in
  // registers.  One barrier per step, between the tile write and the first read of it (the
  // prefetch of step kt+1's first fragments during MFMA group kk=3).  Within a step, the next
  // group's activation fragments (LDS) and weight fragments (dequantized in registers) are
  // prepared while the current group's MFMAs run.
  uint32_t bcur[TNW][WPL];
  float scur[TNW], s16cur[TNW], zcur[TNW];
  auto take_b = [&]() {
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
#pragma unroll
      for (int e = 0; e < WPL; ++e) bcur[j][e] = braw[j][e];
      scur[j] = sb_to_f32<SB>(bs[j]);
      s16cur[j] = scur[j] * 0.0625f;
      zcur[j] = sb_to_f32<SB>(bz[j]);
    }
  };
  bf16x8 af[2][TMW], bfr[2][TNW];
  auto read_a = [&](int slot, const unsigned char* As, int kk) {
#pragma unroll
    for (int i = 0; i < TMW; ++i) af[slot][i] = *reinterpret_cast<const bf16x8*>(As + i * 4096 + a_off[kk]);
  };
  auto deq_b = [&](int slot, int kk) {
#pragma unroll
    for (int j = 0; j < TNW; ++j) bfr[slot][j] = dequant8<BITS>(bcur[j], kk, scur[j], s16cur[j], zcur[j]);
  };
  auto mfma_group = [&](int slot) {
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
      for (int j = 0; j < TNW; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[slot][j], af[slot][i], acc[i][j], 0, 0, 0);
  };
  constexpr int MF = TMW * TNW;  // MFMAs per group

  load_a(0);
  load_b(0);
  store_a(0);
  if (KT > 1) load_a(1);
  take_b();
  if (KT > 1) load_b(1);
  __syncthreads();
  read_a(0, smem[0], 0);
  deq_b(0, 0);

  // One K step.  NEXT: a step kt+1 exists; NEXT2: a step kt+2 exists.  Compile-time so the body
  // is branch-free and the two scheduling regions (split by the barrier) can be interleaved:
  // each MFMA is followed by a share of the next group's LDS reads, dequant VALU and loads.
  auto step = [&](int kt, auto NEXT, auto NEXT2) {
    constexpr bool next = decltype(NEXT)::value, next2 = decltype(NEXT2)::value;
    const unsigned char* As = smem[kt % 3];
    const unsigned char* An = smem[(kt + 1) % 3];
    if constexpr (next) {
      store_a((kt + 1) % 3);
      if constexpr (next2) load_a(kt + 2);
    }
    read_a(1, As, 1);
    deq_b(1, 1);
    mfma_group(0);
    read_a(0, As, 2);
    deq_b(0, 2);
    mfma_group(1);
    if constexpr (next) __builtin_amdgcn_sched_group_barrier(0x200, A_PER, 0);  // tile writes first
#pragma unroll
    for (int q = 0; q < 2 * MF; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                          // MFMA
      if (q % MF < TMW) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);       // LDS read
      if (next2 && q < A_PER) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // global load
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);                          // VALU
    }
    __syncthreads();
    read_a(1, As, 3);
    deq_b(1, 3);
    mfma_group(0);
    if constexpr (next) {
      take_b();
      if constexpr (next2) load_b(kt + 2);
      read_a(0, An, 0);
      deq_b(0, 0);
    }
    mfma_group(1);
#pragma unroll
    for (int q = 0; q < 2 * MF; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (q < MF || next) {
        if (q % MF < TMW) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if (next2 && q >= MF && q < MF + 2 + TNW * WPL / 4) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  int kt = 0;
  for (; kt + 2 < KT; ++kt) step(kt, T_{}, T_{});
  if (kt + 1 < KT) {
    step(kt, T_{}, F_{});
    ++kt;
  }
  step(kt, F_{}, F_{});

  // ---- epilogue: lane holds m = bm0 + 32 i + r32 and n = wn0 + 32 j + 8 a + 4 h + b.
  if constexpr (FUSED) {
    if (epi.bias) {
      if (tid < kBN) bias_lds[tid] = bias_t;
      __syncthreads();
    }
  }
  const bool vec_ok = (N % 4) == 0;
  bf16x8 xa[TMW], lb[TNW];
  const bool lora = FUSED && epi.rank16 > 0;
  if constexpr (FUSED) {
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
      const int64_t m = bm0 + i * 32 + r32;
      xa[i] = bf16x8{};
      if (lora && m < M) xa[i] = *reinterpret_cast<const bf16x8*>(epi.xa + m * 16 + half * 8);
    }
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
      lb[j] = bf16x8{};
      if (lora && n_ok[j])
        lb[j] = *reinterpret_cast<const bf16x8*>(epi.lbt + (wn0 + j * 32 + r32) * 16 + half * 8);
    }
  }
  // One 32-column sub-tile per call; J is a compile-time index so acc stays in registers.
  auto epilogue_cols = [&](auto J) {
    constexpr int j = decltype(J)::value;
    const int64_t nb = wn0 + j * 32 + 4 * half;
    float bias_v[16];
    if constexpr (FUSED) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          bias_v[4 * a + b] = epi.bias ? bias_lds[nb - bn0 + 8 * a + b] : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
      const int64_t m = bm0 + i * 32 + r32;
      f32x16 v = acc[i][j];
      if constexpr (FUSED) {
        f32x16 r = {};
        if (lora) r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lb[j], xa[i], r, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float o = round_bf16(v[e]);
          if (epi.bias) o = round_bf16(o + bias_v[e]);
          if (lora) o = round_bf16(o + round_bf16(round_bf16(r[e]) * epi.lora_scale));
          if constexpr (ACT == MLXQ_ACT_GELU) o = gelu_erf(o);
          else if constexpr (ACT == MLXQ_ACT_GELU_TANH) o = gelu_tanh<true>(o);
          v[e] = o;
        }
      }
      if (m < M) {
        uint16_t* yrow = y + m * N;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int64_t n = nb + 8 * a;
          if (vec_ok && n + 3 < N) {
            u32x2 p = {pack_bf16x2(v[4 * a], v[4 * a + 1]), pack_bf16x2(v[4 * a + 2], v[4 * a + 3])};
            *reinterpret_cast<u32x2*>(yrow + n) = p;
          } else {
#pragma unroll
            for (int b = 0; b < 4; ++b)
              if (n + b < N) yrow[n + b] = f32_to_bf16_bits(v[4 * a + b]);
          }
        }
      }
    }
  };
  epilogue_cols(std::integral_constant<int, 0>{});
  if constexpr (TNW > 1) epilogue_cols(std::integral_constant<int, 1>{});
}

template <typename SB, int BITS, int GS, int WAVES>
static int launch_wide_w(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                         const void* b, int64_t N, void* y, const QmmEpilogue& epi, hipStream_t st,
                         int64_t tiles, const QmmBatch& bat) {
  const bool fused = epi.bias || epi.rank16 || epi.act != MLXQ_ACT_NONE;
  const int kind = fused ? 1 + epi.act : 0;
  const dim3 grid((unsigned)tiles, (unsigned)bat.count);
#define MLXQ_WL(E)                                                                                    \
  hipLaunchKernelGGL((qmm_wide_kernel<SB, BITS, GS, WAVES, E>), grid, dim3(WAVES * 64), 0, st,        \
                     (const uint16_t*)x, M, K, wq, (const SB*)s, (const SB*)b, N, (uint16_t*)y, epi, bat)
  switch (kind) {
    case 0: MLXQ_WL(0); break;
    case 1: MLXQ_WL(1); break;
    case 2: MLXQ_WL(2); break;
    case 3: MLXQ_WL(3); break;
    default: return set_error(MLXQ_EINVAL, "qmm: unknown activation %d", epi.act);
  }
#undef MLXQ_WL
  return check_launch("qmm_wide");
}

template <typename SB, int BITS, int GS>
static int launch_wide(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                       const void* b, int64_t N, void* y, const QmmEpilogue& epi, hipStream_t st,
                       const QmmBatch& bat) {
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  if (tiles == 0 || bat.count == 0) return MLXQ_OK;
  if (tiles > 0x7fffffff || bat.count > 65535) return set_error(MLXQ_EINVAL, "qmm: problem too large");
  // 8 waves (two per SIMD) measured faster than 4 waves with twice the columns per wave.
  return launch_wide_w<SB, BITS, GS, 8>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
}

bool qmm_wide_fits(int64_t M, int64_t K, int64_t N, int gs, int bits, int sb_bytes) {
  const int64_t lim = (int64_t)1 << 32;
  return M * K * 2 < lim && N * (K * bits / 32) * 4 < lim && N * (K / gs) * sb_bytes < lim;
}

int run_qmm_wide(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s, const void* b,
                 int sb_dtype, int64_t N, int gs, int bits, void* y, const QmmEpilogue& epi,
                 hipStream_t st, const QmmBatch& batch) {
#define MLXQ_W(SB, B, G) \
  if (bits == B && gs == G) return launch_wide<SB, B, G>(x, M, K, wq, s, b, N, y, epi, st, batch);
  if (sb_dtype == MLXQ_BFLOAT16) {
    MLXQ_W(uint16_t, 4, 32) MLXQ_W(uint16_t, 4, 64) MLXQ_W(uint16_t, 4, 128)
    MLXQ_W(uint16_t, 8, 32) MLXQ_W(uint16_t, 8, 64) MLXQ_W(uint16_t, 8, 128)
  } else {
    MLXQ_W(float, 4, 32) MLXQ_W(float, 4, 64) MLXQ_W(float, 4, 128)
    MLXQ_W(float, 8, 32) MLXQ_W(float, 8, 64) MLXQ_W(float, 8, 128)
  }
#undef MLXQ_W
  return set_error(MLXQ_EINVAL, "qmm: unsupported bits=%d group_size=%d", bits, gs);
}

}  // namespace mlxq
