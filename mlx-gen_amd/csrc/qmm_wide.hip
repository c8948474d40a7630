// qmm_wide.hip — the main large-M quantized GEMM for gfx950 (K % 64 == 0).
//
// y[M,N] = x[M,K] . W^T with W dequantized to bf16 (round_bf16(fma(code, scale, bias))) and
// v_mfma_f32_32x32x16_bf16 accumulating in f32.
//
// Workgroup: WAVES waves (8 by default: two per SIMD, so one wave's VALU/LDS work overlaps the
// other's MFMAs), block tile BM (M, 256 or 224) x 256 (N), K advanced 64 per step.  The waves split
// the tile along N only: wave w owns columns [w*256/WAVES, (w+1)*256/WAVES) of all BM rows.  The
// host picks BM per problem so that the tile count fills the CUs in as few, full rounds as
// possible (1 workgroup per CU): e.g. M = 4608, N = 3072 gives 216 tiles of 256 rows (one round
// with 40 CUs idle) but 252 tiles of 224 rows (one round of 12.5% shorter tiles).
//   * weights: every lane loads its own packed words straight into registers (one 16-byte
//     buffer load per 32-column sub-tile per K step for Q4, two for Q8) and dequantizes them into
//     the MFMA operand registers — no LDS round trip, and each weight is dequantized exactly once
//     per workgroup because no two waves share columns;
//   * activations: the 256x64 bf16 tile goes global -> LDS by direct-to-LDS buffer loads into a
//     4-stage ring, issued two K steps ahead (one barrier per K step), and every wave reads all of
//     it.  16-byte chunks are XOR-swizzled by f(row) = (row & 7) ^ ((row >> 3) & 1) on the source
//     side, which keeps the 16-lane fragment reads (16 rows, one chunk) on distinct banks;
//   * the MFMA takes the weight fragment as its A operand (rows = n) and the activation fragment
//     as B (columns = m), so each lane's f32x16 result holds 4 runs of 4 consecutive n for one m
//     and the epilogue writes 8-byte (4 x bf16) row segments directly.
// Within a K step, lane half h (lane >> 5) covers k in [8(4h+kk), 8(4h+kk)+8) for MFMA kk = 0..3,
// i.e. packed words 4h..4h+3 of the row's 8-word (Q4) K step — one contiguous load.
// Q4 dequant: w & 0x0f0f0f0f holds the even codes in its bytes, (w >> 4) & 0x0f0f0f0f the odd
// ones; each pair of codes becomes two exact f32 values in one fp8 convert (a byte 0..15 read as
// E4M3 is c * 2^-9, rescaled by 2^9), then one FMA per code and one bf16 pack per pair.
//
// Tile order is XCD-aware: workgroups are dispatched round-robin over the 8 XCDs, so consecutive
// ids are remapped to give each XCD a contiguous slice of a grouped (4 M-tiles x all N-tiles)
// tile order, keeping the activation and weight tiles a slice shares resident in that XCD's L2.
#include <atomic>
#include <type_traits>

#include "mlxq_common.h"

namespace mlxq {

namespace {

constexpr int kBM = 256;  // rows of the large tiles' LDS activation ring (224-row tiles use 256)
constexpr int kBN = 256;
constexpr int kGroupM = 4;
constexpr int kStages = 4;  // activation LDS ring depth (power of two)
constexpr int kBufferFlags = 0x00020000;  // raw buffer resource word 3 for gfx9-family loads

// GELU tables: entry h is the bf16 result of the dtype-preserving exact GELU ([0], reference
// src/nn.rs:344-355) and tanh GELU ([1], src/nn.rs:321-329) for the bf16 input with bits h,
// each evaluated as the reference's separate bf16 ops: every op computed in f32 and its result
// rounded to bf16, the constants cast to bf16 first.  The f32 value of each op is taken as the
// correctly rounded one: the op is evaluated in double (erf and tanh to within an ulp of double)
// and rounded to float, which for + - * / of two floats is the correctly rounded float result.
// This is the uncompiled op sequence: the reference runs gelu_exact under compile(f, true), and
// its comments (src/nn.rs:339-343) say the fused kernel rounds 16-bit types differently from the
// separate ops, so bf16 parity with it is unpinned.
// Filled once per device by act_table_kernel.
__device__ uint16_t g_act_table[2][65536];

__device__ __forceinline__ float bf16_op(double v) { return round_bf16((float)v); }

__global__ __launch_bounds__(256) void act_table_kernel() {
  const int h = blockIdx.x * 256 + threadIdx.x;
  const float x = bf16_bits_to_f32((uint32_t)h);
  const double xd = (double)x;
  {  // gelu_exact: inner = erf(x / sqrt2); gate = 1 + inner; (x * gate) / 2
    const float sqrt2 = round_bf16(1.41421356237309515f);
    const float t1 = bf16_op(xd / (double)sqrt2);
    const float t2 = bf16_op(erf((double)t1));
    const float t3 = bf16_op(1.0 + (double)t2);
    const float t4 = bf16_op(xd * (double)t3);
    g_act_table[0][h] = f32_to_bf16_bits(bf16_op((double)t4 / 2.0));
  }
  {  // gelu_tanh: x3 = x^3; inner = (x + x3 * k) * c; gate = tanh(inner) + 1; (x * 0.5) * gate
    const float c = round_bf16(0.7978845608028654f);
    const float k = round_bf16(0.044715f);
    const float x3 = bf16_op(xd * xd * xd);  // exact in double: 3 x 8 significant bits
    const float t1 = bf16_op((double)x3 * (double)k);
    const float t2 = bf16_op(xd + (double)t1);
    const float inner = bf16_op((double)t2 * (double)c);
    const float th = bf16_op(tanh((double)inner));
    const float gate = bf16_op((double)th + 1.0);
    const float xh = bf16_op(xd * 0.5);
    g_act_table[1][h] = f32_to_bf16_bits(bf16_op((double)xh * (double)gate));
  }
}

}  // namespace


namespace {

// Tile L of the grouped order: kGroupM M-tiles x all N-tiles per group, M fastest in a group.
__device__ __forceinline__ void grouped_coords(int64_t L, int64_t tiles_m, int64_t tiles_n,
                                               int64_t& tm, int64_t& tn) {
  const int64_t span = kGroupM * tiles_n;
  const int64_t g = L / span;
  const int64_t gm0 = g * kGroupM;
  const int64_t gsz = tiles_m - gm0 < kGroupM ? tiles_m - gm0 : kGroupM;
  const int64_t idx = L - g * span;
  tm = gm0 + idx % gsz;
  tn = idx / gsz;
}

// Tile of workgroup bid.  Workgroups are dispatched round-robin over the 8
// XCDs, so consecutive ids are remapped to give each XCD a contiguous slice of the grouped order.
__device__ __forceinline__ void tile_coords(int64_t bid, int64_t tiles_m, int64_t tiles_n,
                                            int64_t& tm, int64_t& tn) {
  const int64_t T = tiles_m * tiles_n;
  const int64_t per = T / 8;
  int64_t L = bid;
  if (bid < per * 8) L = (bid % 8) * per + bid / 8;
  grouped_coords(L, tiles_m, tiles_n, tm, tn);
}



// Workgroup barrier for the pipelined loop: this wave's LDS reads done (lgkmcnt(0)), then
// s_barrier.  Unlike __syncthreads() it has no release fence, which on this target would also
// wait for every outstanding direct-to-LDS load; the loop waits for exactly the loads it needs
// with mlxq_vmcnt before calling this.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
  __builtin_amdgcn_s_barrier();
}

// 16-byte-per-lane buffer load straight into LDS (lane L's data lands at lds_addr + 16 L), as
// inline asm: the compiler then adds no conservative wait for it before later LDS reads (it
// cannot tell they touch other buffers); callers prove completion from their own vmcnt waits.
// rsrc is a raw buffer resource in SGPRs.  M0 (the LDS base of the load) is saved and restored
// inside the statement, since the compiler keeps its own values in it; gfx9 needs one wait state
// between an SALU write of M0 and an LDS DMA reading it, after the load's setup and after the
// restore (the compiler's next LDS DMA may follow directly).
__device__ __forceinline__ void lds_dma16(u32x4 rsrc, uint32_t lds_addr, uint32_t voffset) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voffset), "s"(rsrc)
      : "memory");
}

// Register copy the compiler cannot elide: the weight ring's take must not be coalesced with
// the ring slot, or the slot's next (in-flight) load would need a copy of its own — and a wait
// for that load — at the loop back-edge.
__device__ __forceinline__ uint32_t opaque_copy(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

}  // namespace

// EPI selects the epilogue at compile time: 0 plain y = bf16(acc); 1 bias / rank-16 LoRA; 2 and 3
// the same followed by the bf16 exact or tanh GELU (EPI - 1 is the FusedAct).  One
// epilogue per instantiation keeps it small enough that the accumulator tile stays in registers.
// SZL: bf16 scales/biases staged through LDS in 8-group blocks (needs K / GS % 8 == 0 and both
// arrays within 4 GiB of each other); otherwise every K step loads them into registers.
template <typename SB, int BITS, int GS, int WAVES, int EPI, int BM, bool SZL, int BN>
__global__ __launch_bounds__(WAVES * 64, 1) void qmm_wide_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, const uint32_t* __restrict__ wq,
    const SB* __restrict__ scales, const SB* __restrict__ biases, int64_t N,
    uint16_t* __restrict__ y, QmmEpilogue epi, QmmBatch bat) {
  constexpr bool FUSED = EPI != 0;
  constexpr int ACT = FUSED ? EPI - 1 : kFusedActNone;
  constexpr int NT = WAVES * 64;
  constexpr int TMW = BM / 32;           // m sub-tiles per wave (all BM rows)
  constexpr int TNW = BN / WAVES / 32;  // n sub-tiles per wave
  constexpr int WPL = BITS;              // packed words per lane per n sub-tile per K step (4 or 8)
  // LDS activation ring rows: the tile's rows, or 256 for 224-row tiles (whose 8 waves fill rows
  // in blocks of 64: the last 32 ring rows repeat the tile's last row and are never read).
  constexpr int RB = BM == 224 ? kBM : BM;
  constexpr int A_PER = RB * 8 / NT;     // 16-byte activation chunks per thread per K step
  constexpr int A_ROWS = NT / 8;         // row stride between a thread's chunks
  static_assert(TNW >= 1 && A_PER >= 1 && A_PER * NT == RB * 8 && A_ROWS % 16 == 0 && BM % 32 == 0 &&
                    BM <= RB, "tile/wave shape");
  // bf16 scales/biases are staged through LDS in blocks of 8 groups (SPB K steps): per wave and
  // 32-column sub-tile, two 1 KB buffers of [32 rows x 8 scales][32 rows x 8 biases], plus one
  // 1 KB sink per wave for the placeholder loads (see load_b).
  constexpr bool SZ_LDS = SZL;
  static_assert(!SZL || sizeof(SB) == 2, "LDS-staged scales are bf16");
  constexpr int SPB = 8 * GS / 64;
  constexpr int kSzBytes = SZ_LDS ? WAVES * TNW * 2048 + WAVES * 1024 : 0;
  // The epilogue reuses the ring (and scale region) for the output tile, BM rows of BN bf16 at
  // a 528-byte pitch; the dense bias sits after both.
  constexpr int kRing = kStages * RB * 128 + kSzBytes;
  constexpr int kOut = BM * (BN * 2 + 16);
  // A GELU epilogue copies its 128 KB bf16 table to the start of this region.
  constexpr int kTab = (FUSED && ACT != kFusedActNone) ? 65536 * 2 : 0;
  constexpr int kMain0 = kRing > kOut ? kRing : kOut;
  constexpr int kMain = kMain0 > kTab ? kMain0 : kTab;
  __shared__ __attribute__((aligned(16))) unsigned char lds_all[kMain + BN * 4];
  auto smem = reinterpret_cast<unsigned char (*)[RB * 128]>(lds_all);
  unsigned char* const sz_lds = lds_all + kStages * RB * 128;

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
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int64_t kwords = K * BITS / 32;
  const int64_t groups = K / GS;
  int64_t tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int KT = (int)(K / 64);
  const int64_t bm0 = tm * BM, bn0 = tn * BN;
  const int64_t wn0 = bn0 + (int64_t)wave * (BN / WAVES);
  // Dense bias of the tile's BN columns: one value per thread, loaded now and written to its LDS
  // slot (after the ring and scale blocks, in the kernel's single LDS object) in the epilogue,
  // so the epilogue issues no global loads (each would wait on the tile's pending output stores
  // too, since vmcnt counts stores).  The load is unconditional on a clamped column (columns past
  // N are never stored) and kept as raw bits until the epilogue: a per-lane conditional load, or
  // converting the value right away, made the compiler wait for it before the first operand loads.
  uint32_t bias_bits = 0;
  if constexpr (FUSED) {
    if (epi.bias) {
      const int64_t nn = bn0 + (tid < BN ? tid : 0);
      bias_bits = epi.bias[nn < N ? nn : N - 1];
    }
  }
  // Buffer resources: 32-bit offsets (the host checks every operand fits in 4 GiB).  Rows past
  // M / N are clamped so every offset stays inside its operand.
  [[maybe_unused]] const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (int)(uint32_t)(M * K * 2), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(wq), (short)0, (int)(uint32_t)(N * kwords * 4), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<SB*>(scales), (short)0, (int)(uint32_t)(N * groups * sizeof(SB)), kBufferFlags);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<SB*>(biases), (short)0, (int)(uint32_t)(N * groups * sizeof(SB)), kBufferFlags);

  // ---- activation staging: global -> LDS directly (buffer_load ... lds), 4-stage ring.  One such
  // load moves 1 KB per wave: lane L's 16 bytes land at block + 16 L.  Wave wv's round i fills
  // the block of rows A_ROWS i + 8 wv .. +7, so lane L loads the chunk of row
  // A_ROWS i + 8 wv + (L >> 3) that belongs at position L & 7 under the swizzle, i.e. global
  // chunk (L & 7) ^ f(row).  All RB LDS rows are filled (uniform code); rows at or past BM
  // repeat the tile's last row and are never read.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  uint32_t a_goff[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int rl = A_ROWS * i + 8 * wv + (lane >> 3);
    const int c = (lane & 7) ^ swz_f(rl);
    const int rt = rl < BM ? rl : BM - 1;
    const int64_t r = bm0 + rt < M ? bm0 + rt : M - 1;
    a_goff[i] = (uint32_t)((r * K + c * 8) * 2);
  }
  auto dma_a = [&](int kt) {
    unsigned char* base = smem[kt & (kStages - 1)];
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (__attribute__((address_space(3))) void*)(base + (A_ROWS * i + 8 * wv) * 128), 16,
          a_goff[i] + (uint32_t)kt * 128u, 0, 0, 0);
#else
    (void)base;
#endif
  };

  // ---- weight rows of this lane: n = wn0 + 32 j + r32 (clamped to N-1 like A rows).  Packed
  // words and raw scale/bias bits go through a 2-slot register ring (slot = step parity).
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
  uint32_t braw[2][TNW][WPL];
  uint32_t bs[2][TNW], bz[2][TNW];  // raw scale/bias bits (f32 scales: loaded with the words)
  // bf16 scales and biases: one resource over both arrays (the host checks that they lie within
  // 4 GiB of each other), so that one load can fetch scales in half 0 and biases in half 1.
  // Lane (h, r32) of a block load fetches 8 groups of row r32 of its sub-tile; lane L lands at
  // buffer + 16 L, i.e. [32 rows x 16 B scales][32 rows x 16 B biases].
  const uint16_t* sb_lo = (const uint16_t*)scales < (const uint16_t*)biases ? (const uint16_t*)scales
                                                                          : (const uint16_t*)biases;
  const uint32_t s_rel = (uint32_t)((const uint16_t*)scales - sb_lo) * 2u;
  const uint32_t z_rel = (uint32_t)((const uint16_t*)biases - sb_lo) * 2u;
  const uint64_t sb_addr = (uint64_t)(uintptr_t)sb_lo;
  const u32x4 rsz = {(uint32_t)sb_addr, (uint32_t)(sb_addr >> 32) & 0xffffu,
                     (uint32_t)((s_rel > z_rel ? s_rel : z_rel) + (uint64_t)N * groups * 2),
                     (uint32_t)kBufferFlags};
  const uint32_t sz_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)sz_lds;
  const uint32_t sz_sink = sz_base + WAVES * TNW * 2048 + wv * 1024;
  // The scale/bias load that goes with load_b(kt), issued as if by step kt-3: it fetches block
  // b+1 when step kt-3's take starts reading block b (kt-2 = b*SPB) and block b+1 exists;
  // otherwise all lanes read the first 16 bytes of the scales into this wave's sink.  Issuing
  // one op with every load_b keeps the loop body free of branches (a branch here made the
  // compiler's own waits conservative) and the vmcnt counts fixed.
  auto dma_sz = [&](int kt) {
    const int ks = kt - 2;  // first step of the block the issuing take starts
    const bool fetch = (ks & (SPB - 1)) == 0 && ks + SPB < KT;
    const int blk = ks / SPB + 1;
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
      const uint32_t dst = fetch ? sz_base + (uint32_t)((wv * TNW + j) * 2048 + (blk & 1) * 1024) : sz_sink;
      const uint32_t off = fetch ? (half ? z_rel : s_rel) + (g_base[j] + (uint32_t)blk * 8u) * 2u : s_rel;
      lds_dma16(rsz, dst, off);
    }
  };
  auto load_b = [&](int kt, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    const uint32_t g = (uint32_t)((kt * 64 + half * 32) / GS);
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
#pragma unroll
      for (int q = 0; q < WPL / 4; ++q) {
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, w_goff[j] + (uint32_t)kt * (8u * WPL) + 16u * q, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) braw[sl][j][4 * q + e] = v[e];
      }
      if constexpr (!SZ_LDS) {
        bs[sl][j] = load_sb_bits<SB>(rs, g_base[j] + g);
        bz[sl][j] = load_sb_bits<SB>(rz, g_base[j] + g);
      }
    }
    if constexpr (SZ_LDS) dma_sz(kt);
    (void)g;
  };
  constexpr int B_OPS = TNW * (WPL / 4 + (SZ_LDS ? 1 : 2));  // vector memory ops of one load_b
  // Ops of one load_b issued after the last op the take needs (the bf16 path's scale/bias load
  // goes to LDS and is waited for separately).
  constexpr int B_TAIL = SZ_LDS ? TNW : 0;


  // ---- fragment read offsets (LDS): row i*32 + r32, chunk 4h + kk
  int a_off[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a_off[kk] = r32 * 128 + (((4 * half + kk) ^ swz_f(r32)) << 4);

  // LoRA operands of the epilogue (x.A rows per m sub-tile, B^T rows per n sub-tile), loaded in
  // the last K step so their latency hides behind its MFMAs (rows past M / N are clamped: never
  // stored).
  [[maybe_unused]] const bool lora_on = FUSED && epi.rank16 > 0;
  [[maybe_unused]] bf16x8 xa_pf[TMW], lb_pf[TNW];
  auto prefetch_lora = [&]() {
    if constexpr (FUSED) {
#pragma unroll
      for (int i = 0; i < TMW; ++i) xa_pf[i] = bf16x8{};
#pragma unroll
      for (int j = 0; j < TNW; ++j) lb_pf[j] = bf16x8{};
      if (lora_on) {
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
          const int64_t m = bm0 + i * 32 + r32 < M ? bm0 + i * 32 + r32 : M - 1;
          xa_pf[i] = *reinterpret_cast<const bf16x8*>(epi.xa + m * 16 + half * 8);
        }
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
          const int64_t n = wn0 + j * 32 + r32 < N ? wn0 + j * 32 + r32 : N - 1;
          lb_pf[j] = *reinterpret_cast<const bf16x8*>(epi.lbt + n * 16 + half * 8);
        }
      }
    }
  };
  f32x16 acc[TMW][TNW];
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // ---- software pipeline.  Step kt reads LDS stage kt%4; the activation tiles of steps kt+1
  // (landed), kt+2 and kt+3 (in flight) occupy the other stages, and the weights of steps kt+1
  // and kt+2 sit in the register ring, so every global load is issued two steps before its
  // use.  One barrier per step, mid-step: before it each wave waits for its own loads of
  // A(kt+1), after it the tile is complete for all waves and stage (kt+3)%4 — last read in step
  // kt-1 — is refilled.  The waits are explicit vmcnt counts over the fixed issue order
  // A(0) W(0) A(1) W(1) ...; a scheduling fence keeps the weight take (VALU on loaded
  // registers) from being hoisted across the barrier, where it would force an early wait.
  uint32_t bcur[TNW][WPL];
  float scur[TNW], zcur[TNW];
  auto take_b = [&](auto SLOT, int ktn) {  // ktn: the step these weights belong to
    constexpr int sl = decltype(SLOT)::value;
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
#pragma unroll
      for (int e = 0; e < WPL; ++e) bcur[j][e] = opaque_copy(braw[sl][j][e]);
      if constexpr (SZ_LDS) {
        const int g = (ktn * 64 + half * 32) / GS;
        const unsigned char* p =
            sz_lds + (wave * TNW + j) * 2048 + ((g >> 3) & 1) * 1024 + r32 * 16 + (g & 7) * 2;
        scur[j] = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p));
        zcur[j] = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p + 512));
      } else {
        scur[j] = sb_to_f32<SB>(bs[sl][j]);
        zcur[j] = sb_to_f32<SB>(bz[sl][j]);
      }
    }
  };
  bf16x8 af[2][TMW], bfr[2][TNW];
  auto read_a = [&](int slot, const unsigned char* As, int kk) {
#pragma unroll
    for (int i = 0; i < TMW; ++i) af[slot][i] = *reinterpret_cast<const bf16x8*>(As + i * 4096 + a_off[kk]);
  };
  auto deq_b = [&](int slot, int kk) {
#pragma unroll
    for (int j = 0; j < TNW; ++j) bfr[slot][j] = dequant8<BITS>(bcur[j], kk, scur[j], zcur[j]);
  };
  auto mfma_group = [&](int slot) {
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
      for (int j = 0; j < TNW; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[slot][j], af[slot][i], acc[i][j], 0, 0, 0);
  };
  constexpr int MF = TMW * TNW;  // MFMAs per group
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  // Prologue: issue A(0) W(0) A(1) W(1) A(2) W(2), wait for A(0) and W(0).  W(j) goes to ring
  // slot (KT - j) & 1, counted from the end so that the last three steps always use the same
  // slots whatever KT is.
  auto prologue = [&](auto SA, auto SB_) __attribute__((always_inline)) {  // SA = slot of W(0)
    if constexpr (SZ_LDS) {  // block 0, before A(0): complete once A(0) is
#pragma unroll
      for (int j = 0; j < TNW; ++j)
        lds_dma16(rsz, sz_base + (uint32_t)((wv * TNW + j) * 2048), (half ? z_rel : s_rel) + g_base[j] * 2u);
    }
    dma_a(0);
    load_b(0, SA);
    if (KT > 1) {
      dma_a(1);
      load_b(1, SB_);
    }
    if (KT > 2) {
      dma_a(2);
      mlxq_vmcnt<B_TAIL + A_PER + B_OPS + A_PER>();
    } else if (KT > 1) {
      mlxq_vmcnt<B_TAIL + A_PER + B_OPS>();
    } else {
      mlxq_vmcnt<B_TAIL>();
    }
    __builtin_amdgcn_sched_barrier(0);
    take_b(SA, 0);
    if (KT > 2) load_b(2, SA);
  };
  // bf16 scales: KT is a whole number of scale blocks (SPB >= 4 steps), so even.
  if (!SZ_LDS && (KT & 1)) prologue(S1{}, S0{});
  else prologue(S0{}, S1{});
  lds_barrier();
  read_a(0, smem[0], 0);
  deq_b(0, 0);

  // One K step.  N1/N2/N3: steps kt+1/kt+2/kt+3 exist; SLOT = (KT-kt-1)&1 holds W(kt+1) and
  // then receives W(kt+3).  All compile-time so the body is branch-free and the two scheduling regions
  // (split by the barrier) interleave each MFMA with a share of LDS reads, dequant VALU and loads.
  auto step = [&](int kt, auto SLOT, auto N1_, auto N2_, auto N3_) __attribute__((always_inline)) {
    constexpr bool N1 = decltype(N1_)::value, N2 = decltype(N2_)::value, N3 = decltype(N3_)::value;
    const unsigned char* As = smem[kt & (kStages - 1)];
    const unsigned char* An = smem[(kt + 1) & (kStages - 1)];
    read_a(1, As, 1);
    deq_b(1, 1);
    mfma_group(0);
    read_a(0, As, 2);
    deq_b(0, 2);
    mfma_group(1);
#pragma unroll
    for (int q = 0; q < 2 * MF; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                     // MFMA
      if (q % MF < TMW) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);                     // VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    // A(kt+1) issued before W(kt+1) [, A(kt+2), W(kt+2)].
    if constexpr (N1) mlxq_vmcnt<B_OPS + (N2 ? A_PER + B_OPS : 0)>();
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!N1) prefetch_lora();  // last step: no explicit waits follow
    if constexpr (N3) dma_a(kt + 3);
    read_a(1, As, 3);
    deq_b(1, 3);
    mfma_group(0);
    if constexpr (N1) {
      // W(kt+1) issued before [A(kt+2), W(kt+2),] [A(kt+3)].
      mlxq_vmcnt<B_TAIL + (N2 ? A_PER + B_OPS : 0) + (N3 ? A_PER : 0)>();
      take_b(SLOT, kt + 1);
      if constexpr (N3) load_b(kt + 3, SLOT);
      read_a(0, An, 0);
      deq_b(0, 0);
    }
    mfma_group(1);
#pragma unroll
    for (int q = 0; q < 2 * MF; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (q < MF || N1) {
        if (q % MF < TMW) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if (N3 && q < A_PER) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (N3 && q >= MF && q < MF + B_OPS) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  // Scale/bias block b+1 is fetched with load_b(kt+3) by the step kt = b*SPB - 1 whose take starts
  // reading block b, into the buffer block b-1 used.  Completion: the load is issued before
  // A(kt+4), and step kt+3 waits for A(kt+4) before its barrier; block b+1 is first read by the
  // take of step kt+SPB, SPB >= 4.
  // Steps 0 .. KT-4 in pairs (one peeled when their count is odd), then the last three steps.
  if (KT >= 4) {
    int kt = 0;
    if (SZ_LDS || ((KT - 3) & 1)) {
      step(0, S1{}, T_{}, T_{}, T_{});
      kt = 1;
    }
    for (; kt < KT - 3; kt += 2) {
      step(kt, S0{}, T_{}, T_{}, T_{});
      step(kt + 1, S1{}, T_{}, T_{}, T_{});
    }
  }
  if (KT >= 3) step(KT - 3, S0{}, T_{}, T_{}, F_{});
  if (KT >= 2) step(KT - 2, S1{}, T_{}, F_{}, F_{});
  step(KT - 1, S0{}, F_{}, F_{}, F_{});

  // ---- epilogue: lane holds m = bm0 + 32 i + r32 and n = wn0 + 32 j + 8 a + 4 h + b.
  // With an activation, the input of the GELU is a bf16 value (the rounded sum of the product,
  // bias and LoRA terms), so the activation is a lookup in a 65536-entry bf16 table of the same
  // device function (g_act_table, bit-identical to evaluating it): the table is copied into the
  // now idle activation ring while the first pass rounds and adds into the accumulators, and a
  // second pass looks up and stores.  Evaluating the exact-erf GELU cost ~20 VALU ops per output
  // with the MFMA idle (~15 k cycles per 224x256 tile).
  constexpr bool TABLE = ACT != kFusedActNone;
  // Output rows go out through LDS when N % 8 == 0: the tile is written to LDS row-major (pitch
  // 528 bytes, so the 32 rows of a lane group fall on different banks) and stored with 16 bytes
  // per lane, two whole 512-byte rows per instruction, instead of 8-byte pieces of 32 rows —
  // ~900 instead of ~7000 cache-line writes per 224x256 tile.
  constexpr int PITCH = BN * 2 + 16;
  const bool via_lds = (N % 8) == 0;
  float* bias_lds = reinterpret_cast<float*>(lds_all + kMain);
  if constexpr (FUSED) {
    if (epi.bias && tid < BN) {
      asm volatile("" : "+v"(bias_bits));  // first use here, so the load is waited for here
      bias_lds[tid] = bf16_bits_to_f32(bias_bits);
    }
  }
  __syncthreads();  // bias visible; every wave past its last ring read
  if constexpr (TABLE) {
    const uint64_t ta = (uint64_t)(uintptr_t)&g_act_table[ACT - 1][0];
    const u32x4 rt = {(uint32_t)ta, (uint32_t)(ta >> 32) & 0xffffu, 65536u * 2u, (uint32_t)kBufferFlags};
    const uint32_t lbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds_all;
    constexpr int kPer = 65536 * 2 / 1024 / WAVES;  // 1 KB loads per wave
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const uint32_t blk = (uint32_t)(wv * kPer + r) * 1024u;
      lds_dma16(rt, lbase + blk, blk + (uint32_t)lane * 16u);
    }
  }
  const bool vec_ok = (N % 4) == 0;
  bf16x8 xa[TMW], lb[TNW];
  const bool lora = FUSED && epi.rank16 > 0;
  if constexpr (FUSED) {
#pragma unroll
    for (int i = 0; i < TMW; ++i) xa[i] = xa_pf[i];
#pragma unroll
    for (int j = 0; j < TNW; ++j) lb[j] = lb_pf[j];
  }
  // 16 outputs of accumulator (i, j) as bf16 bits, two per word: to the LDS tile, or straight
  // to y (N % 8 != 0).
  auto put_tile = [&](int i, int j, const uint32_t (&pk)[8]) {
    const int cl = wave * (BN / WAVES) + j * 32 + 4 * half;  // tile column of element 0
    if (via_lds) {
      unsigned char* row = lds_all + (i * 32 + r32) * PITCH + cl * 2;
#pragma unroll
      for (int a = 0; a < 4; ++a) *reinterpret_cast<u32x2*>(row + 16 * a) = u32x2{pk[2 * a], pk[2 * a + 1]};
      return;
    }
    const int64_t m = bm0 + i * 32 + r32;
    if (m < M) {
      uint16_t* yrow = y + m * N;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int64_t n = bn0 + cl + 8 * a;
        if (vec_ok && n + 3 < N) {
          *reinterpret_cast<u32x2*>(yrow + n) = u32x2{pk[2 * a], pk[2 * a + 1]};
        } else {
#pragma unroll
          for (int b = 0; b < 4; ++b)
            if (n + b < N) yrow[n + b] = (uint16_t)(pk[2 * a + b / 2] >> (16 * (b & 1)));
        }
      }
    }
  };
  // First pass, one 32-column sub-tile per call (J compile-time so acc stays in registers):
  // bias, LoRA and their roundings in place; without an activation, pack and put.  Each term
  // (HB bias, HL LoRA, HS LoRA scale != 1) is a kTerm* value chosen once per tile below.
  auto epilogue_cols = [&](auto J, auto HB, auto HL, auto HS) {
    constexpr int j = decltype(J)::value;
    constexpr int kB = decltype(HB)::value, kL = decltype(HL)::value, kS = decltype(HS)::value;
    const int cb = wave * (BN / WAVES) + j * 32 + 4 * half;
    // Without a bias the GELU pass adds -0, the identity for every value (-0 and NaN included),
    // instead of branching on the bias.
    float bias_v[16] = {};
    if constexpr (kB != kTermOff) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) bias_v[4 * a + b] = epi.bias ? bias_lds[cb + 8 * a + b] : -0.0f;
    }
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
      f32x16& v = acc[i][j];
      if constexpr (FUSED) {
        f32x16 r = {};
        if (kL == kTermOn || (kL == kTermRuntime && lora))
          r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lb[j], xa[i], r, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          float o0 = v[e], o1 = v[e + 1];
          epilogue_terms2<kB, kL, kS>(o0, o1, epi.bias != nullptr, bias_v[e], bias_v[e + 1], lora, r[e],
                                      r[e + 1], epi.lora_scale);
          v[e] = o0;
          v[e + 1] = o1;
        }
      }
      if constexpr (!TABLE) {
        uint32_t pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) pk[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
        put_tile(i, j, pk);
      }
    }
  };
  auto first_pass = [&](auto HB, auto HL, auto HS) {
    epilogue_cols(std::integral_constant<int, 0>{}, HB, HL, HS);
    if constexpr (TNW > 1) epilogue_cols(std::integral_constant<int, 1>{}, HB, HL, HS);
  };
  using Off = std::integral_constant<int, kTermOff>;
  using On = std::integral_constant<int, kTermOn>;
  using Rt = std::integral_constant<int, kTermRuntime>;
  if constexpr (!FUSED) {
    first_pass(Off{}, Off{}, Off{});
  } else if constexpr (TABLE) {
    // With neither term the lookup pass rounds the products itself (FLUX up with GELU 337.9 ->
    // 328.7 us against the pass with runtime conditions, outputs identical).  Otherwise one pass
    // adds the bias unconditionally (-0 without one: 350.8 -> 348.8 us with a bias) and keeps
    // LoRA a runtime condition: a second copy of the pass (one per combination, or a bias-only one
    // beside the general one) pushes the GELU kernels past 256 VGPRs into scratch.
    if (epi.bias || lora) first_pass(On{}, Rt{}, Rt{});
  } else {
    // Bias and LoRA without an activation (the host sends no launch with neither term):
    // measured on M = 4608, K = 3072 with rank-16 LoRA and bias, 98.7 -> 97.2 us (N = 3072) and
    // 265.6 -> 260.9 us (N = 9216) against runtime conditions, outputs identical.
    const bool hs = epi.lora_scale != 1.0f;
    if (epi.bias && lora) {
      if (hs) first_pass(On{}, On{}, On{});
      else first_pass(On{}, On{}, Off{});
    } else if (lora) {
      if (hs) first_pass(Off{}, On{}, On{});
      else first_pass(Off{}, On{}, Off{});
    } else {
      first_pass(On{}, Off{}, Off{});
    }
  }
  if constexpr (TABLE) {
    mlxq_vmcnt<0>();  // this wave's table loads
    __syncthreads();  // and every other wave's
    const uint16_t* tab = reinterpret_cast<const uint16_t*>(lds_all);
    // Look up every output first (the packed codes replace the accumulators), since the LDS
    // tile overwrites the table.
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
      for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          // The bf16 codes of the GELU inputs: the products rounded here (RNE, as the first
          // pass rounds; values it already rounded pass unchanged).
          const uint32_t code = pack_bf16x2(acc[i][j][2 * q], acc[i][j][2 * q + 1]);
          const uint32_t lo = tab[code & 0xffffu];
          const uint32_t hi = tab[code >> 16];
          acc[i][j][q] = __uint_as_float(lo | (hi << 16));
        }
    if (via_lds) __syncthreads();  // table reads done before the tile overwrites it
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
      for (int i = 0; i < TMW; ++i) {
        uint32_t pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) pk[q] = __float_as_uint(acc[i][j][q]);
        put_tile(i, j, pk);
      }
  }
  if (via_lds) {
    __syncthreads();
    // Row-major copy out: LPR lanes per BN * 2-byte row, NT / LPR rows per pass of the workgroup.
    constexpr int LPR = BN * 2 / 16;
    const int c16 = tid % LPR;
    const int64_t n = bn0 + c16 * 8;
#pragma unroll 4
    for (int r = tid / LPR; r < BM; r += NT / LPR) {
      const int64_t m = bm0 + r;
      const u32x4 v = *reinterpret_cast<const u32x4*>(lds_all + r * PITCH + c16 * 16);
      if (m < M && n < N) *reinterpret_cast<u32x4*>(y + m * N + n) = v;
    }
  }
}

static int ensure_act_table(hipStream_t st);

template <typename SB, int BITS, int GS, int WAVES, int BM, bool SZL, int BN>
static int launch_wide_w(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                         const void* b, int64_t N, void* y, const QmmEpilogue& epi, hipStream_t st,
                         int64_t tiles, const QmmBatch& bat) {
  const bool fused = epi.bias || epi.rank16 || epi.act != kFusedActNone;
  const int kind = fused ? 1 + epi.act : 0;
  if (kind >= 2) {
    const int rc = ensure_act_table(st);
    if (rc != MLXQ_OK) return rc;
  }
  const dim3 grid((unsigned)tiles, (unsigned)bat.count);
#define MLXQ_WL(E)                                                                                    \
  hipLaunchKernelGGL((qmm_wide_kernel<SB, BITS, GS, WAVES, E, BM, SZL, BN>), grid, dim3(WAVES * 64), 0, st, \
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

// The GELU tables are filled on a device's first GELU launch and the host waits for that fill
// once, so later launches on any stream find them complete.  Under graph capture (no waiting
// possible) the fill is captured ahead of the GEMM instead and the device stays unmarked.  Two
// threads making a device's first GELU call at once may both fill the tables; both write the
// same values, so either order leaves them correct.
static std::atomic<int> g_act_table_ready[64];
static std::atomic<uintptr_t> g_act_table_addr[64];

static int ensure_act_table(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(MLXQ_EDEVICE, "qmm: no current device");
  const bool slot = dev >= 0 && dev < 64;
  if (slot && g_act_table_ready[dev].load(std::memory_order_acquire)) return MLXQ_OK;
  hipLaunchKernelGGL(act_table_kernel, dim3(256), dim3(256), 0, st);
  int rc = check_launch("act_table");
  if (rc != MLXQ_OK) return rc;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (slot && hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
    if (hipStreamSynchronize(st) != hipSuccess) return set_error(MLXQ_EDEVICE, "qmm: act table fill failed");
    g_act_table_ready[dev].store(1, std::memory_order_release);
  }
  return MLXQ_OK;
}

const uint16_t* act_table_ptr(int fused_act, hipStream_t st) {
  if (fused_act != kFusedActGeluExact && fused_act != kFusedActGeluTanh) {
    set_error(MLXQ_EINVAL, "act table: activation %d has no bf16 table", fused_act);
    return nullptr;
  }
  if (ensure_act_table(st) != MLXQ_OK) return nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error(MLXQ_EDEVICE, "act table: no usable current device");
    return nullptr;
  }
  uintptr_t a = g_act_table_addr[dev].load(std::memory_order_acquire);
  if (a == 0) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_act_table)) != hipSuccess || p == nullptr) {
      set_error(MLXQ_EDEVICE, "act table: hipGetSymbolAddress failed");
      return nullptr;
    }
    a = (uintptr_t)p;
    g_act_table_addr[dev].store(a, std::memory_order_release);
  }
  return reinterpret_cast<const uint16_t*>(a) + (fused_act == kFusedActGeluExact ? 0 : 65536);
}

int64_t device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// Workgroups that run at once: one per CU (the kernel's LDS and registers allow no second).
static int64_t resident_workgroups() { return device_cu_count(); }

// Tile height for a problem.  A launch takes ceil(tiles / CUs) rounds (one workgroup per CU).
// Fewer rounds win.  At equal round counts, 224-row tiles win when there are several rounds
// (each round does 12.5% less MFMA work: measured 329 vs 343 us on M=4608, N=12288, K=3072),
// but a single round is as long as its slowest tile, and a 224-row tile is no faster than a
// 256-row one when more CUs share the memory system (304 vs 299 us on M=4608, N=3072,
// K=12288), so one round keeps 256 rows.
static int qmm_wide_tile_rows(int64_t M, int64_t N, int64_t count) {
  const int64_t cus = resident_workgroups();
  const int64_t tn = (N + kBN - 1) / kBN;
  const int64_t r256 = ((M + 255) / 256 * tn * count + cus - 1) / cus;
  const int64_t r224 = ((M + 223) / 224 * tn * count + cus - 1) / cus;
  if (r224 < r256 || (r224 == r256 && r256 > 1)) return 224;
  return 256;
}

template <typename SB, int BITS, int GS>
static int launch_wide(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                       const void* b, int64_t N, void* y, const QmmEpilogue& epi, hipStream_t st,
                       const QmmBatch& bat) {
  if (M == 0 || N == 0 || bat.count == 0) return MLXQ_OK;
  if (bat.count > 65535) return set_error(MLXQ_EINVAL, "qmm: problem too large");
  // 8 waves (two per SIMD) measured faster than 4 waves with twice the columns per wave.
  // bf16 scales (the reference's layout) with LDS-staged scale blocks also get the 224-row
  // tile; other layouts keep 256 rows.
  constexpr bool kBf16 = std::is_same<SB, uint16_t>::value;
  const bool szl = kBf16 && (K / GS) % 8 == 0 && qmm_wide_sb_reach(s, b, N * (K / GS) * 2, 2);
  // Grids under 128 tiles of 256 x 256 take 256 x 128 tiles with 4 waves (the same 256 x 32
  // strip per wave, twice the tiles), and grids under 128 of those 128 x 128 tiles with 4 waves
  // of 128 x 32 and a ring of 128 rows (mid-size prefill).
  const bool narrow = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN) * bat.count < 128;
  const bool mid = narrow && ((M + kBM - 1) / kBM) * ((N + 127) / 128) * bat.count < 128;
  if (mid) {
    const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
    if (tiles > 0x7fffffff) return set_error(MLXQ_EINVAL, "qmm: problem too large");
    if constexpr (kBf16) {
      if (szl) return launch_wide_w<SB, BITS, GS, 4, 128, true, 128>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
    }
    return launch_wide_w<SB, BITS, GS, 4, 128, false, 128>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
  }
  if (narrow) {
    const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + 127) / 128);
    if (tiles > 0x7fffffff) return set_error(MLXQ_EINVAL, "qmm: problem too large");
    if constexpr (kBf16) {
      if (szl) return launch_wide_w<SB, BITS, GS, 4, kBM, true, 128>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
    }
    return launch_wide_w<SB, BITS, GS, 4, kBM, false, 128>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
  }
  const int bm = szl ? qmm_wide_tile_rows(M, N, bat.count) : kBM;
  const int64_t tiles = ((M + bm - 1) / bm) * ((N + kBN - 1) / kBN);
  if (tiles > 0x7fffffff) return set_error(MLXQ_EINVAL, "qmm: problem too large");
  if constexpr (kBf16) {
    if (szl && bm == 224) return launch_wide_w<SB, BITS, GS, 8, 224, true, kBN>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
    if (szl) return launch_wide_w<SB, BITS, GS, 8, kBM, true, kBN>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
  }
  return launch_wide_w<SB, BITS, GS, 8, kBM, false, kBN>(x, M, K, wq, s, b, N, y, epi, st, tiles, bat);
}

bool qmm_wide_sb_reach(const void* scales, const void* biases, int64_t bytes, int sb_bytes) {
  if (sb_bytes != 2) return true;
  const uint64_t s = (uint64_t)(uintptr_t)scales, b = (uint64_t)(uintptr_t)biases;
  const uint64_t lo = s < b ? s : b, hi = s < b ? b : s;
  return hi - lo + (uint64_t)bytes < ((uint64_t)1 << 32);
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
