// qmm_small.hip — quantized GEMM for small grids (text-encoder prefill: M up to a few hundred).
//
// y[M,N] = x[M,K] . W^T with the semantics of the other GEMM kernels: every weight dequantized
// to bf16 as round_bf16(fma(code, scale, bias)), v_mfma_f32_32x32x16_bf16 accumulating in f32,
// the epilogue's ops rounded to bf16 where the reference's separate ops round.
//
// When M x N gives few tiles, a tile kernel leaves most CUs idle and each workgroup walks all of
// K one latency-bound step after another.  Here a workgroup of 8 waves owns a 64x64 output tile
// and the waves split K: wave w takes K steps [w*KT/8, (w+1)*KT/8), so a tile has eight
// independent load chains of KT/8 steps instead of one of KT.  Each wave moves its activation
// rows global -> LDS with direct-to-LDS loads one step ahead (a private 2-stage ring, 8 rows x
// 128 bytes per load, i.e. whole cache lines) and reads MFMA fragments back with ds_read_b128;
// its weight fragments go straight into registers two steps ahead.  The eight partial tiles meet
// in LDS (over the rings) and are added in wave order (deterministic); waves 0-3 then finish one
// 32x32 sub-tile each.
// MFMA roles (as in qmm_wide.hip): weights are the A operand (rows n), activations the B operand
// (columns m); lane (h = lane >> 5, r = lane & 31) holds m = r and n = 8a + 4h + b in element
// 4a + b of its f32x16, and covers k in [8(4h+kk), +8) of a 64-wide K step for MFMA kk.
//
// bf16 scales and biases with K / GS a multiple of 8 (SZS) are staged per wave in LDS, in blocks
// of 8 groups for the tile's 64 weight rows: lane L loads row L's 8 scales and 8 biases with two
// 16-byte loads one block ahead, writes them to the wave's 2 KB region at the block boundary, and
// every K step reads its row's pair from there.  Per-step 2-byte loads would touch 32 cache
// lines per load instruction for 64 useful bytes; the block load touches one line per row per 8
// groups.
#include "mlxq_common.h"

namespace mlxq {

namespace {

constexpr int kTile = 64;   // output tile rows and columns
constexpr int kWaves = 8;   // waves per workgroup, splitting K
constexpr int kBufferFlags = 0x00020000;

template <typename SB, int BITS>
struct SmallOps {           // one K step of one lane's register operands
  uint32_t w[2][BITS];      // packed words: column sub-tile j
  uint32_t s[2], z[2];      // raw scale / bias bits of sub-tile j
};

template <typename SB, int BITS, int GS, int EPI, bool SZS>
__global__ __launch_bounds__(kWaves * 64, 1) void qmm_small_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, const uint32_t* __restrict__ wq,
    const SB* __restrict__ scales, const SB* __restrict__ biases, int64_t N,
    uint16_t* __restrict__ y, QmmEpilogue epi) {
  constexpr bool FUSED = EPI != 0;
  constexpr int ACT = FUSED ? EPI - 1 : kFusedActNone;
  constexpr int WPL = BITS;  // packed words per lane per sub-tile per K step
  // One LDS object (a second one makes the compiler wait for every direct-to-LDS load before
  // any LDS read): per wave 16 KB — its 2-stage activation ring [stage][64 rows][128 B] during
  // the loop, its partial tile [sub-tile][quad][lane] x 4 floats after it — then, with SZS, the
  // staged scale/bias blocks [wave][scales, biases][64 rows][8 groups] bf16.
  constexpr int kWaveBytes = 16384;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kWaves * kWaveBytes + (SZS ? kWaves * 2048 : 0)];
  auto part = reinterpret_cast<f32x4 (*)[4][4][64]>(lds);
  uint16_t* const sz_lds = reinterpret_cast<uint16_t*>(lds + kWaves * kWaveBytes);
  static_assert(!SZS || sizeof(SB) == 2, "staged scales are bf16");

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, r32 = lane & 31, half = lane >> 5;
  const int64_t tiles_m = (M + kTile - 1) / kTile;
  const int64_t bm0 = (blockIdx.x % tiles_m) * kTile, bn0 = (blockIdx.x / tiles_m) * kTile;
  const int64_t kwords = K * BITS / 32, groups = K / GS;
  const int KT = (int)(K / 64);
  // Scalar (wave-uniform) K range: the step branches below stay scalar branches, never EXEC
  // predication (which MFMA does not honour).
  const int k_begin = __builtin_amdgcn_readfirstlane(wave * KT / kWaves);
  const int nst = __builtin_amdgcn_readfirstlane((wave + 1) * KT / kWaves) - k_begin;

  // Buffer resources (32-bit offsets: the host checks the operands fit in 4 GiB); rows past M
  // and N are clamped to the last row, so every offset stays inside its operand.
  [[maybe_unused]] const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (int)(uint32_t)(M * K * 2), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(wq), (short)0, (int)(uint32_t)(N * kwords * 4), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<SB*>(scales), (short)0, (int)(uint32_t)(N * groups * sizeof(SB)), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<SB*>(biases), (short)0, (int)(uint32_t)(N * groups * sizeof(SB)), kBufferFlags);
  uint32_t w_off[2], g_base[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = bn0 + 32 * j + r32 < N ? bn0 + 32 * j + r32 : N - 1;
    w_off[j] = (uint32_t)((n * kwords + half * WPL) * 4);
    g_base[j] = (uint32_t)(n * groups);
  }
  // Activation ring: load u of a step fills rows 8u .. 8u+7 of the stage, lane L the chunk at
  // position L & 7 of row 8u + (L >> 3), i.e. global chunk (L & 7) ^ swz_f(row) (rows past M
  // repeat row M-1).  Fragment (i, kk) of lane (h, r) is chunk 4h + kk of row 32i + r.
  unsigned char* const ring = lds + wave * kWaveBytes;
  uint32_t a_goff[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int rl = 8 * u + (lane >> 3);
    const int64_t m = bm0 + rl < M ? bm0 + rl : M - 1;
    a_goff[u] = (uint32_t)((m * K + ((lane & 7) ^ swz_f(rl)) * 8) * 2);
  }
  int a_rd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a_rd[kk] = r32 * 128 + (((4 * half + kk) ^ swz_f(r32)) << 4);
  auto dma_a = [&](int kt, int stage) {
#if defined(__HIP_DEVICE_COMPILE__)
    unsigned char* base = ring + stage * 8192;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (__attribute__((address_space(3))) void*)(base + u * 1024), 16, a_goff[u] + (uint32_t)kt * 128u, 0, 0, 0);
#else
    (void)kt; (void)stage;
#endif
  };

  auto load = [&](int kt, SmallOps<SB, BITS>& d) {
    const uint32_t g = (uint32_t)((kt * 64 + half * 32) / GS);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int q = 0; q < WPL / 4; ++q) {
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, w_off[j] + (uint32_t)kt * (8u * WPL) + 16u * q, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) d.w[j][4 * q + e] = v[e];
      }
      if constexpr (!SZS) {
        d.s[j] = load_sb_bits<SB>(rs, g_base[j] + g);
        d.z[j] = load_sb_bits<SB>(rz, g_base[j] + g);
      }
    }
    (void)g;
  };
  // Scale/bias block staging (SZS): pending block in registers, lane L = tile row L.
  constexpr int SPB = 8 * GS / 64;  // K steps per block of 8 groups
  u32x4 ps = {}, pz = {};
  const int64_t srow = bn0 + lane < N ? bn0 + lane : N - 1;
  const uint32_t sz_row = (uint32_t)(srow * groups * 2);
  const int last_blk = (int)(groups / 8) - 1;
  uint16_t* const sz_w = sz_lds + (SZS ? wave * 1024 : 0);
  auto load_blk = [&](int b) {
    if constexpr (SZS) {
      const uint32_t off = sz_row + (uint32_t)(b < last_blk ? b : last_blk) * 16u;
      ps = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      pz = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rz, off, 0, 0));
    }
    (void)b;
  };
  auto write_blk = [&]() {
    if constexpr (SZS) {
      *reinterpret_cast<u32x4*>(sz_w + lane * 8) = ps;
      *reinterpret_cast<u32x4*>(sz_w + 512 + lane * 8) = pz;
    }
  };
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  auto compute = [&](const SmallOps<SB, BITS>& c, int kt, int stage) {
    const unsigned char* As = ring + stage * 8192;
    u32x4 af[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) af[i][kk] = *reinterpret_cast<const u32x4*>(As + i * 4096 + a_rd[kk]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float s, z;
      if constexpr (SZS) {
        const int gi = ((kt * 64 + half * 32) / GS) & 7;
        s = bf16_bits_to_f32(sz_w[(32 * j + r32) * 8 + gi]);
        z = bf16_bits_to_f32(sz_w[512 + (32 * j + r32) * 8 + gi]);
      } else {
        s = sb_to_f32<SB>(c.s[j]);
        z = sb_to_f32<SB>(c.z[j]);
      }
      (void)kt;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8 b = dequant8<BITS>(c.w[j], kk, s, z);
#pragma unroll
        for (int i = 0; i < 2; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              b, __builtin_bit_cast(bf16x8, af[i][kk]), acc[i][j], 0, 0, 0);
      }
    }
  };

  // Two register slots, loads two steps ahead.  Loads past the wave's last step repeat that
  // step (never computed), so every iteration issues the same loads and the compiler's waits
  // count exactly; the scheduling fences keep each slot's refill after its last read.
  // Scale blocks: the block of the wave's first step is written before the loop and the next
  // one loaded; a step that starts a block writes the pending block (loaded a block earlier) and
  // loads the one after it.
  // Per step t: [scale block edge], A(t+1) into stage (t+1)&1, wait for A(t), compute, W(t+2).
  // A(t) was followed by W(t+1) (NW ops), possibly a block load (2) and A(t+1) (8): waiting for
  // at most NW + 8 outstanding completes it (a block load only makes the wait longer).  Loads past
  // the wave's last step repeat that step (never computed), so every step issues the same ops.
  constexpr int NW = 2 * (WPL / 4) + (SZS ? 0 : 4);
  if (nst > 0) {
    auto kt_of = [&](int t) { return k_begin + (t < nst ? t : nst - 1); };
    auto block_edge = [&](int kt) {
      if constexpr (SZS) {
        if (kt != k_begin && kt % SPB == 0) {
          write_blk();
          load_blk(kt / SPB + 1);
        }
      }
    };
    SmallOps<SB, BITS> o0, o1;
    load_blk(k_begin / SPB);
    dma_a(k_begin, 0);
    load(kt_of(0), o0);
    load(kt_of(1), o1);
    write_blk();
    load_blk(k_begin / SPB + 1);
    for (int t = 0; t < nst; t += 2) {
      block_edge(k_begin + t);
      dma_a(kt_of(t + 1), 1);
      mlxq_vmcnt<NW + 8>();
      __builtin_amdgcn_sched_barrier(0);
      compute(o0, k_begin + t, 0);
      __builtin_amdgcn_sched_barrier(0);
      load(kt_of(t + 2), o0);
      if (t + 1 < nst) {
        block_edge(k_begin + t + 1);
        dma_a(kt_of(t + 2), 0);
        mlxq_vmcnt<NW + 8>();
        __builtin_amdgcn_sched_barrier(0);
        compute(o1, k_begin + t + 1, 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      load(kt_of(t + 3), o1);
    }
  }
  // Every direct-to-LDS load has landed before the ring is overwritten by the partial tile.
  mlxq_vmcnt<0>();
  __builtin_amdgcn_sched_barrier(0);

  // ---- reduction over the eight K slices, in wave order.
#pragma unroll
  for (int sub = 0; sub < 4; ++sub)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x16& a = acc[sub >> 1][sub & 1];
      part[wave][sub][q][lane] = f32x4{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
    }
  __syncthreads();
  if (wave >= 4) return;
  const int i = wave >> 1, j = wave & 1;  // this wave's sub-tile
  f32x16 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 t = part[0][wave][q][lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) t += part[w][wave][q][lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * q + e] = t[e];
  }

  // ---- epilogue (lane: m = bm0 + 32 i + r32, n = bn0 + 32 j + 8 a + 4 h + b).
  const int64_t m = bm0 + 32 * i + r32;
  const int64_t nb = bn0 + 32 * j + 4 * half;
  if constexpr (FUSED) {
    const bool lora = epi.rank16 > 0;
    f32x16 r = {};
    // Rows past M and columns past N read clamped operands (never stored): per-lane conditional
    // loads made the compiler wait for each one in turn.
    if (lora) {
      const int64_t nr = bn0 + 32 * j + r32 < N ? bn0 + 32 * j + r32 : N - 1;
      const int64_t mr = m < M ? m : M - 1;
      const bf16x8 xa = *reinterpret_cast<const bf16x8*>(epi.xa + mr * 16 + half * 8);
      const bf16x8 lb = *reinterpret_cast<const bf16x8*>(epi.lbt + nr * 16 + half * 8);
      r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lb, xa, r, 0, 0, 0);
    }
    float bv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) bv[e] = 0.0f;
    if (epi.bias) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t n = nb + 8 * (e >> 2) + (e & 3);
        bv[e] = bf16_bits_to_f32(epi.bias[n < N ? n : N - 1]);
      }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; b += 2) {
        const int e = 4 * a + b;
        const float b0 = bv[e], b1 = bv[e + 1];
        float o0 = v[e], o1 = v[e + 1];
        epilogue_terms2<kTermRuntime, kTermRuntime, kTermRuntime>(o0, o1, epi.bias != nullptr, b0, b1, lora,
                                                                 r[e], r[e + 1], epi.lora_scale);
        v[e] = o0;
        v[e + 1] = o1;
        if constexpr (ACT != kFusedActNone) {  // bf16 values: the table's entries for them
          v[e] = bf16_bits_to_f32(epi.act_table[f32_to_bf16_bits(v[e])]);
          v[e + 1] = bf16_bits_to_f32(epi.act_table[f32_to_bf16_bits(v[e + 1])]);
        }
      }
  }
  if (m < M) {
    uint16_t* yrow = y + m * N;
    const bool vec_ok = (N % 4) == 0;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int64_t n = nb + 8 * a;
      if (vec_ok && n + 3 < N) {
        *reinterpret_cast<u32x2*>(yrow + n) =
            u32x2{pack_bf16x2(v[4 * a], v[4 * a + 1]), pack_bf16x2(v[4 * a + 2], v[4 * a + 3])};
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          if (n + b < N) yrow[n + b] = f32_to_bf16_bits(v[4 * a + b]);
      }
    }
  }
}

template <typename SB, int BITS, int GS>
static int launch_small(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                        const void* b, int64_t N, void* y, const QmmEpilogue& epi, hipStream_t st) {
  const int64_t tiles = ((M + kTile - 1) / kTile) * ((N + kTile - 1) / kTile);
  const bool fused = epi.bias || epi.rank16 || epi.act != kFusedActNone;
  const int kind = fused ? 1 + epi.act : 0;
  if (kind > 3) return set_error(MLXQ_EINVAL, "qmm: unknown activation %d", epi.act);
  if (kind >= 2 && epi.act_table == nullptr) return set_error(MLXQ_EINVAL, "qmm: activation table missing");
  // bf16 scales with whole blocks of 8 groups are staged in LDS (16-byte aligned row blocks).
  const bool szs = std::is_same<SB, uint16_t>::value && (K / GS) % 8 == 0;
#define MLXQ_SL(E, Z)                                                                                 \
  hipLaunchKernelGGL((qmm_small_kernel<SB, BITS, GS, E, Z>), dim3((unsigned)tiles), dim3(kWaves * 64), \
                     0, st, (const uint16_t*)x, M, K, wq, (const SB*)s, (const SB*)b, N,               \
                     (uint16_t*)y, epi)
  if constexpr (std::is_same<SB, uint16_t>::value) {
    if (szs) {
      switch (kind) {
        case 0: MLXQ_SL(0, true); break;
        case 1: MLXQ_SL(1, true); break;
        case 2: MLXQ_SL(2, true); break;
        default: MLXQ_SL(3, true); break;
      }
      return check_launch("qmm_small");
    }
  }
  switch (kind) {
    case 0: MLXQ_SL(0, false); break;
    case 1: MLXQ_SL(1, false); break;
    case 2: MLXQ_SL(2, false); break;
    default: MLXQ_SL(3, false); break;
  }
#undef MLXQ_SL
  return check_launch("qmm_small");
}

}  // namespace

bool qmm_small_fits(int64_t M, int64_t K, int64_t N, int gs, int bits, int sb_bytes) {
  const int64_t lim = (int64_t)1 << 32;
  return K % 64 == 0 && M * K * 2 < lim && N * (K * bits / 32) * 4 < lim &&
         N * (K / gs) * sb_bytes < lim && (M + kTile - 1) / kTile * ((N + kTile - 1) / kTile) < 0x7fffffff;
}

int run_qmm_small(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                  const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y,
                  const QmmEpilogue& epi, hipStream_t st) {
  if (M == 0 || N == 0) return MLXQ_OK;
#define MLXQ_SM(SB, B, G) \
  if (bits == B && gs == G) return launch_small<SB, B, G>(x, M, K, wq, s, b, N, y, epi, st);
  if (sb_dtype == MLXQ_BFLOAT16) {
    MLXQ_SM(uint16_t, 4, 32) MLXQ_SM(uint16_t, 4, 64) MLXQ_SM(uint16_t, 4, 128)
    MLXQ_SM(uint16_t, 8, 32) MLXQ_SM(uint16_t, 8, 64) MLXQ_SM(uint16_t, 8, 128)
  } else {
    MLXQ_SM(float, 4, 32) MLXQ_SM(float, 4, 64) MLXQ_SM(float, 4, 128)
    MLXQ_SM(float, 8, 32) MLXQ_SM(float, 8, 64) MLXQ_SM(float, 8, 128)
  }
#undef MLXQ_SM
  return set_error(MLXQ_EINVAL, "qmm: unsupported bits=%d group_size=%d", bits, gs);
}

}  // namespace mlxq
