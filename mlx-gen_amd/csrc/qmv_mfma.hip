// qmv_mfma.hip — decode GEMV y[M,N] = x[M,K] . W^T for M <= 8 on gfx950 matrix cores.
//
// Two kernels: the 16-row tile kernel described here (M = 2..8, Q8, and K not a multiple of
// 1024), and, further down, the one-row kernel that serves M = 1 with Q4 codes (one weight row per
// wave, no split-K reduction).  Both compute the same exact-f32 factored form.
//
// The path is HBM-bound and small (a few MB per call), so the kernel is built around the load
// shape the memory system streams best and around latency: every 16-byte weight load a wave
// needs is issued up front, each load covers 16 rows x 64 contiguous bytes (4 lanes per row), the
// packed codes go straight into MFMA operand registers, and each load step is folded as soon as
// its data arrives (the step code is branch-free, so the compiler waits for one load per step).
//
// Semantics are the exact-f32 factored form (no bf16 rounding of dequantized weights):
//   y[m,n] = sum_g ( s[n,g] * sum_{k in g} x[m,k]*c[n,k]  +  b[n,g] * X[m,g] ),  X = sum_{k in g} x.
// Q4 codes enter the MFMA as exact bf16 values c, two per fp8 scaled convert (unpack_q4), and
// Q8 codes as bf16(c) (exact for c < 256); both fold per group as y += s*acc + b*X.
// X comes from the same activation fragments multiplied by an all-ones operand on the MFMA.
//
// v_mfma_f32_16x16x32_bf16 with A = activations (rows m = lane&15; rows >= M read row 0 and are
// never stored) and B = weights (columns n = lane&15).  Lane quarter q = lane>>4 holds the 16
// bytes [16q, 16q+16) of the row's 64-byte load step: 32 Q4 codes (4 words) or 16 Q8 codes.
// Each MFMA takes one 8-code run per lane, and all four runs of one MFMA must lie in one group:
//   * Q8 (64 codes per step): MFMA j takes words 2j, 2j+1 of every lane — one 64-code block.
//   * Q4, group 128 (128 codes per step, one group): MFMA i takes word i of every lane.
//   * Q4, group 64: lanes q = 0,1 hold group 2t and lanes q = 2,3 group 2t+1.  Two
//     v_permlane32_swap ops exchange words 2,3 of the low lane half with words 0,1 of the high
//     half, after which words 0,1 of every lane belong to group 2t and words 2,3 to group 2t+1.
//   * Q8, group 32: lanes q = 0,1 hold group 2t and q = 2,3 group 2t+1; the same two swaps as
//     for Q4 group 64 make words 0,1 (MFMA 0) group 2t and words 2,3 (MFMA 1) group 2t+1.
//   * Q4, group 32: lane quarter q holds group 4t+q whole.  The same two swaps followed by two
//     v_permlane16_swap ops (odd 16-lane rows against even rows) transpose the 4 x 4 block of
//     (quarter, word), after which word i of every lane belongs to group 4t+i.
// Each lane reads the activation run matching its code run from LDS (per-lane offsets below).
// The 16x16 result holds column n = lane&15 for rows m = 4q + e.
// A workgroup owns up to 16 weight rows (one MFMA tile); its waves split K and reduce through LDS
// at the end.
// Q4 k-order inside an 8-run is [0,2,4,6,1,3,5,7] (low nibbles first, see unpack_q4); the
// activation rows are permuted to match with v_perm_b32 as they are copied into LDS.
#include <atomic>
#include <type_traits>
#include <utility>

#include "mlxq_common.h"

namespace mlxq {

namespace {

constexpr int kBufferFlags = 0x00020000;
constexpr int kMaxWaves = 16;  // waves per workgroup (they split K)
constexpr int kCopySlots = 8;  // 16-byte activation chunks a lane stages (registers), all rows
constexpr int kMaxLds = 160 * 1024;
constexpr uint32_t kOob = 0x7ffffff0u;  // buffer offset past every resource: loads return zero

// Q4 word (codes c0..c7, c_i at bits 4i) -> bf16 pairs (c0, c2), (c4, c6), (c1, c3), (c5, c7).
// The low and high nibbles are split into bytes once; a byte c <= 15 read as OCP fp8 E4M3 is
// exactly c * 2^-9, so v_cvt_scalef32_pk_bf16_fp8 with scale 2^9 turns two code bytes into two
// exact bf16 values.
__device__ __forceinline__ bf16x8 unpack_q4(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu;          // bytes c0, c2, c4, c6
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;   // bytes c1, c3, c5, c7
  u32x4 o;
  o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, false));
  o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, true));
  o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, false));
  o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, true));
  return __builtin_bit_cast(bf16x8, o);
}

// Activation run x0..x7 (raw bf16 pairs r0..r3) -> order [0,2,4,6,1,3,5,7], matching unpack_q4.
__device__ __forceinline__ u32x4 perm_q4(u32x4 r) {
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(r[1], r[0], 0x05040100u);
  o[1] = __builtin_amdgcn_perm(r[3], r[2], 0x05040100u);
  o[2] = __builtin_amdgcn_perm(r[1], r[0], 0x07060302u);
  o[3] = __builtin_amdgcn_perm(r[3], r[2], 0x07060302u);
  return o;
}

// Two Q8 words (codes c0..c7 in natural order) -> bf16(c).
__device__ __forceinline__ bf16x8 cvt_q8(uint32_t w0, uint32_t w1) {
  u32x4 o;
  o[0] = pack_bf16x2((float)(w0 & 0xffu), (float)((w0 >> 8) & 0xffu));
  o[1] = pack_bf16x2((float)((w0 >> 16) & 0xffu), (float)(w0 >> 24));
  o[2] = pack_bf16x2((float)(w1 & 0xffu), (float)((w1 >> 8) & 0xffu));
  o[3] = pack_bf16x2((float)((w1 >> 16) & 0xffu), (float)(w1 >> 24));
  return __builtin_bit_cast(bf16x8, o);
}

__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Raw buffer resource over `bytes` bytes at p: loads at offsets past the end return zero.
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const T* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(p), (short)0, bytes, kBufferFlags);
}

// v_permlane32_swap_b32: lanes 32..63 of `lo_keep` trade places with lanes 0..31 of `hi_keep`.
// Afterwards lanes 0..31 still hold their own `lo_keep` and lanes 32..63 their own `hi_keep`.
__device__ __forceinline__ void swap_lane_halves(uint32_t& lo_keep, uint32_t& hi_keep) {
  const auto r = __builtin_amdgcn_permlane32_swap(lo_keep, hi_keep, false, false);
  lo_keep = r[0];
  hi_keep = r[1];
}

// v_permlane16_swap_b32: the odd 16-lane rows (1, 3) of `even_keep` trade places with the even
// rows (0, 2) of `odd_keep`; row 2k keeps its own `even_keep`, row 2k + 1 its own `odd_keep`.
__device__ __forceinline__ void swap_lane_rows(uint32_t& even_keep, uint32_t& odd_keep) {
  const auto r = __builtin_amdgcn_permlane16_swap(even_keep, odd_keep, false, false);
  even_keep = r[0];
  odd_keep = r[1];
}

// Row pitch in floats of the per-row (s, zc) pair table in LDS: at least 2G, a multiple of 4 (the
// fold reads 16 bytes) and an odd multiple of 4, so the 16 rows read in one step (one per lane)
// land on 16 distinct 16-byte bank quads.  A pitch of exactly 2G puts every row on the same banks
// whenever 2G is a multiple of 64 (K = 8192, group 64: a 16-way conflict on every fold).
__host__ __device__ constexpr int sz_pitch(int G) {
  const int p = (2 * G + 3) & ~3;
  return (p & 4) ? p : p + 4;
}

// Whether a tile of `steps` load steps per wave and MR activation rows stays within the 128
// registers per lane of a 1024-thread workgroup (the counts the compiler reports for these
// kernels): 8 steps only with one row, and for Q4 with group 64 (two groups per step) 6 steps
// with at most two rows.  Larger combinations spilled (and spills doubled a launch's time).
constexpr bool qmv_steps_fit(int bits, int gs, int steps, int mr) {
  return !(steps == 8 && mr > 1) && !(bits == 4 && gs == 64 && steps == 6 && mr > 2) &&
         !(gs == 32 && steps > 4);
}

}  // namespace

// Scale/bias group slots one wave keeps: the groups its load steps touch (a group 128 of Q8 spans
// two steps and may straddle two waves, hence the spare slot).
__host__ __device__ constexpr int qmv_wave_groups(int bits, int gs, int steps) {
  return bits == 8 ? (gs == 128 ? (steps + 2) / 2 : steps * (64 / gs)) : steps * (128 / gs);
}

// Bytes of LDS one wave owns: its activation rows (M rows of steps * 64 bytes of codes' worth of
// activations, padded so rows start on different banks) and its (s, zc) table.
__host__ __device__ constexpr int qmv_wave_lds(int bits, int gs, int steps, int M) {
  return M * (steps * (512 / bits) * 2 + 16) + 16 * sz_pitch(qmv_wave_groups(bits, gs, steps)) * 4;
}

// One 16-row GEMV tile as seen by one wave: the wave's K range of T load steps, the operand
// registers between the issue of its loads and their use, and its private LDS region.  The
// weights pass through a ring of STEPS load registers: the first STEPS steps are issued up front
// and each register is reloaded with step d + STEPS as soon as step d's MFMAs have read it (T = 2
// STEPS reaches twice the K of one register round at the same register count).  The last wave's
// range may run past K: its activations there load as zero (so those steps' products and group
// sums are zero, whatever codes the weight loads find past the row's end) and so do the scales
// and biases of groups past the row's end.
// Contract of every kernel built from it (checked on the host by qmv_plan):
// 1 <= M <= MR, K % (512/BITS) == 0, K % group == 0, bf16 scales and biases, the row's
// K*BITS/512 load steps covered by the waves of one matrix (T each, the last wave's range may end
// past K), dynamic LDS of at least max(waves * qmv_wave_lds, waves * 16 * 17 * 4) bytes, every
// buffer < 2 GiB.
template <int BITS, int GS, int STEPS, int MR, int T>
struct GemvTile {
  static_assert(T >= STEPS, "ring shorter than the wave's steps");
  static constexpr int CPL = 512 / BITS;          // codes per row in one 64-byte load step
  static constexpr bool G64 = GS == 64, G32 = GS == 32;
  static constexpr bool Q4G32 = BITS == 4 && G32;  // four groups per step, one per lane quarter
  // two groups per step, one per lane half (Q4 group 64, Q8 group 32)
  static constexpr bool PAIR = (BITS == 4 && G64) || (BITS == 8 && G32);
  static constexpr int NACC = Q4G32 ? 4 : 2;      // group accumulators per load step
  static constexpr int NM = BITS == 4 ? 4 : 2;    // MFMAs per load step
  static constexpr int E = MR < 4 ? MR : 4;       // result registers per lane that can hold a row < M
  static constexpr int XCH = T * CPL / 8;         // 16-byte activation chunks per row in the wave's range
  static constexpr int XSL = (XCH + 63) / 64;     // ... per lane
  static constexpr int NGW = qmv_wave_groups(BITS, GS, T);
  static constexpr int PW = sz_pitch(NGW);        // (s, zc) table row pitch, floats
  static constexpr int SBL = (16 * NGW + 63) / 64;  // scale entries per lane
  static constexpr int XW = T * CPL * 2 + 16;       // LDS pitch of the wave's activation rows

  int lane, c16, q, n0, nr, M, K, N, G, ls0, kb, g0;
  unsigned char* wl;  // this wave's LDS region: activation rows, then the (s, zc) table
  float* szw;
  u32x4 cx[MR][XSL];
  uint32_t cs[SBL], cz[SBL];
  u32x4 wv[STEPS];
  __amdgpu_buffer_rsrc_t rw;
  uint32_t w_base;

  // wave_all: the wave's index in the workgroup (selects its LDS region); wave: its index among
  // the waves of its matrix (selects its K range); rows [n0, n0 + nr) of an [N, K] matrix, nr <= 16
  // (MFMA columns past nr load nothing and are never stored).
  __device__ __forceinline__ GemvTile(int lane_, int wave_all, int wave, int n0_, int nr_, int M_, int K_,
                                      int N_, unsigned char* lds) {
    lane = lane_;
    c16 = lane & 15;
    q = lane >> 4;
    n0 = n0_;
    nr = nr_;
    M = M_;
    K = K_;
    N = N_;
    G = K / GS;
    ls0 = wave * T;
    kb = ls0 * CPL;
    g0 = kb / GS;
    wl = lds + wave_all * (M * XW + 16 * PW * 4);
    szw = reinterpret_cast<float*>(wl + M * XW);
  }

  // The wave's activation range as 16-byte chunks (out-of-range chunks read as zero).
  __device__ __forceinline__ void issue_x(__amdgpu_buffer_rsrc_t rx) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
#pragma unroll
        for (int j = 0; j < XSL; ++j) {
          const int c = lane + 64 * j;
          cx[m][j] = load16(rx, c < XCH && kb + c * 8 < K ? (uint32_t)((m * K + kb + c * 8) * 2) : kOob);
        }
      }
    }
  }

  // The scale and bias of each (row, group) slot the wave folds.
  __device__ __forceinline__ void issue_sb(__amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rz) {
#pragma unroll
    for (int j = 0; j < SBL; ++j) {
      const int e = lane + 64 * j;
      const int r = e / NGW, gl = e - r * NGW;  // constant divisor
      const bool ok = e < 16 * NGW && r < nr && g0 + gl < G;
      const uint32_t off = ok ? ((uint32_t)(n0 + r) * (uint32_t)G + (uint32_t)(g0 + gl)) * 2u : kOob;
      cs[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
      cz[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rz, off, 0, 0);
    }
  }

  // The wave's first STEPS weight loads: 16 rows x 64 contiguous bytes per load; the lanes of
  // rows past the workgroup's nr read past every buffer (zero, no memory traffic).
  __device__ __forceinline__ void issue_w(__amdgpu_buffer_rsrc_t rw_) {
    rw = rw_;
    w_base = c16 < nr ? (uint32_t)(n0 + c16) * (uint32_t)(K * BITS / 8) + (uint32_t)(ls0 * 64 + q * 16) : kOob;
#pragma unroll
    for (int d = 0; d < STEPS; ++d) wv[d] = load16(rw, w_base + (uint32_t)d * 64u);
  }

  // Operands into the wave's LDS region.  Q4 activation runs are stored permuted to
  // [0,2,4,6,1,3,5,7] so they pair with the unpacked code layout; scales and biases become
  // f32 pairs (s, b), ready for the fold.  Only this wave
  // reads them back, so a wave-level ordering point replaces a workgroup barrier.
  __device__ __forceinline__ void stage() {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
#pragma unroll
        for (int j = 0; j < XSL; ++j) {
          const int c = lane + 64 * j;
          if (c < XCH)
            *reinterpret_cast<u32x4*>(wl + m * XW + c * 16) = BITS == 4 ? perm_q4(cx[m][j]) : cx[m][j];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < SBL; ++j) {
      const int e = lane + 64 * j;
      if (e < 16 * NGW) {
        const int r = e / NGW, gl = e - r * NGW;
        const float sv = __uint_as_float(cs[j] << 16), zv = __uint_as_float(cz[j] << 16);
        *reinterpret_cast<f32x2*>(szw + r * PW + 2 * gl) = f32x2{sv, zv};
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // Per load step: NM MFMAs x . codes and NM MFMAs x . ones (group sums), then the fold of
  // each group, y += s*acc + zc*X.  yacc[e] is result row 4q + e of column c16.
  __device__ __forceinline__ void fold(float (&yacc)[E]) {
    const unsigned char* xa[NM];  // this lane's activation run for MFMA i at the wave's first step
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      int k;
      if constexpr (BITS == 8 && G32) k = (q < 2 ? 16 * q : 16 * (q - 2) + 8) + 32 * i;
      else if constexpr (BITS == 8) k = 16 * q + 8 * i;
      else if constexpr (G32) k = 32 * i + 8 * q;  // after the word transpose: MFMA i = group i
      else if constexpr (!G64) k = 32 * q + 8 * i;
      else if (i < 2) k = (q < 2 ? 32 * q : 32 * (q - 2) + 16) + 8 * i;
      else k = (q < 2 ? 64 + 32 * q : 32 * q + 16) + 8 * (i - 2);
      xa[i] = wl + (c16 < M ? c16 : 0) * XW + k * 2;
    }
    const float* sz = szw + c16 * PW;
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (__bf16)1.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) yacc[e] = 0.0f;

    auto fold1 = [&](const f32x4& acc, const f32x4& xsum, float s, float zc) {
#pragma unroll
      for (int e = 0; e < E; ++e) yacc[e] = fmaf(s, acc[e], fmaf(zc, xsum[e], yacc[e]));
    };

    // Activation runs: every lane reads, lanes of A rows c16 >= M the run of row 0 (an A row
    // m >= M only feeds result row m, which is never stored).  The 16 lanes of a quarter then read
    // at most M distinct addresses (broadcast); a read restricted to the lanes of rows < M cost
    // the compiler ten 64-bit register copies per step to keep the other lanes' operands.
    using SZ = typename std::conditional<PAIR, f32x4, f32x2>::type;
    bf16x8 a[T][NM];
    SZ p[T];
    f32x4 p32[T][2];  // group 32: the (s, zc) pairs of the step's four groups
    f32x4 acc[T][NACC], xsum[T][NACC];

    // A step's LDS operands: its activation runs and its (s, zc) pairs.
    auto read_step = [&](int d) {
#pragma unroll
      for (int i = 0; i < NM; ++i) a[d][i] = *reinterpret_cast<const bf16x8*>(xa[i] + d * (CPL * 2));
      if constexpr (Q4G32) {
        p32[d][0] = *reinterpret_cast<const f32x4*>(sz + 8 * d);  // groups 4ls, 4ls+1
        p32[d][1] = *reinterpret_cast<const f32x4*>(sz + 8 * d + 4);  // groups 4ls+2, 4ls+3
      } else if constexpr (PAIR) {
        p[d] = *reinterpret_cast<const f32x4*>(sz + 4 * d);  // groups 2ls, 2ls+1
      } else {
        // Q4/128 and Q8/64: one group per step; Q8/128: a group every two steps
        const int gl = (BITS == 4 || G64) ? d : ((ls0 + d) >> 1) - g0;
        p[d] = *reinterpret_cast<const f32x2*>(sz + 2 * gl);
      }
    };
    // A step's products: NM MFMAs x . codes and NM MFMAs x . ones (the group sums); then the ring
    // register is reloaded with step d + STEPS.
    auto mfma_step = [&](int d) {
      const int slot = d % STEPS;
      uint32_t w[4] = {wv[slot][0], wv[slot][1], wv[slot][2], wv[slot][3]};
      if constexpr (PAIR) {  // Q8 group 32: words 0,1 and 2,3 are its two MFMAs' pairs
        swap_lane_halves(w[0], w[2]);
        swap_lane_halves(w[1], w[3]);
      } else if constexpr (Q4G32) {
        // Quarter q's 16 bytes are group q of the step (words = 8-code runs).  Transpose the
        // 4 x 4 (quarter, word) block: afterwards word i of quarter q is run q of group i, so
        // MFMA i covers group i alone.
        swap_lane_halves(w[0], w[2]);
        swap_lane_halves(w[1], w[3]);
        swap_lane_rows(w[0], w[1]);
        swap_lane_rows(w[2], w[3]);
      }
#pragma unroll
      for (int h = 0; h < NACC; ++h) {
        acc[d][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        xsum[d][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        const int h = (Q4G32 || (BITS == 8 && G32)) ? i : ((BITS == 4 && G64) ? i >> 1 : 0);
        const bf16x8 b = BITS == 4 ? unpack_q4(w[i]) : cvt_q8(w[2 * i], w[2 * i + 1]);
        acc[d][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d][i], b, acc[d][h], 0, 0, 0);
        xsum[d][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d][i], ones, xsum[d][h], 0, 0, 0);
      }
      if (d + STEPS < T) wv[slot] = load16(rw, w_base + (uint32_t)(d + STEPS) * 64u);
    };
    // A step's fold into the result.  The result is pinned after each fold: otherwise the
    // compiler sinks every fold below the last step and keeps all steps' products live at once.
    auto fold_step = [&](int d) {
      if constexpr (Q4G32) {
        fold1(acc[d][0], xsum[d][0], p32[d][0][0], p32[d][0][1]);
        fold1(acc[d][1], xsum[d][1], p32[d][0][2], p32[d][0][3]);
        fold1(acc[d][2], xsum[d][2], p32[d][1][0], p32[d][1][1]);
        fold1(acc[d][3], xsum[d][3], p32[d][1][2], p32[d][1][3]);
      } else if constexpr (PAIR) {
        fold1(acc[d][0], xsum[d][0], p[d][0], p[d][1]);
        fold1(acc[d][1], xsum[d][1], p[d][2], p[d][3]);
      } else {
        fold1(acc[d][0], xsum[d][0], p[d][0], p[d][1]);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) asm volatile("" : "+v"(yacc[e]));
    };

    // Software pipeline over the steps: iteration d reads step d+1's LDS operands, runs step d's
    // MFMAs (waiting for its weight load only) and folds step d-1, whose products have completed
    // meanwhile, so the LDS-read and MFMA latencies of consecutive steps overlap.  Scheduling
    // fences between iterations keep at most two steps' operands live.
    read_step(0);
#pragma unroll
    for (int d = 0; d < T; ++d) {
      __builtin_amdgcn_sched_barrier(0);
      if (d + 1 < T) read_step(d + 1 < T ? d + 1 : d);
      mfma_step(d);
      if (d > 0) fold_step(d - 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    fold_step(T - 1);
  }
};

// Split-K reduction of a tile's partial sums through LDS (reusing the operand area):
// [wave][m 0..15][n 0..15], waves [0, W) of matrix 0 and [W, 2W) of matrix 1.  Only rows
// 4q + e with e < E can be < M; the rest are never written or read.  NMAT = 2 stores
// round(silu(round(g)) * round(u)) with silu(g) = round(g * round(sigmoid(g)))
// (qwen3.rs:178-181, src/nn.rs:301-303), else round(y), into y [M, N].
template <int NMAT, int E>
__device__ __forceinline__ void gemv_reduce_store(unsigned char* lds, const float (&yacc)[E],
                                                  int wave_all, int W, int lane, int tid, int NT,
                                                  int M, int n0, int nr, int N, uint16_t* __restrict__ y) {
  const int c16 = lane & 15, q = lane >> 4;
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int e = 0; e < E; ++e) red[(wave_all * 16 + 4 * q + e) * 17 + c16] = yacc[e];
  __syncthreads();
  for (int idx = tid; idx < 16 * M; idx += NT) {  // a one-wave workgroup has 64 < 16*M threads
    const int m = idx >> 4, nl = idx & 15;
    float v = 0.0f;
    for (int w = 0; w < W; ++w) v += red[(w * 16 + m) * 17 + nl];
    if constexpr (NMAT == 2) {
      float u = 0.0f;
      for (int w = 0; w < W; ++w) u += red[((W + w) * 16 + m) * 17 + nl];
      // each op rounded to bf16 as the reference's separate ops are (qwen3.rs:178-181)
      v = silu_bf16(round_bf16(v)) * round_bf16(u);
    }
    if (nl < nr) y[m * N + n0 + nl] = f32_to_bf16_bits(v);
  }
}

// The GEMV launch: a workgroup owns `rows` <= 16 weight rows and its waves split K.  NMAT = 2 is the
// SwiGLU decode form: the second wave half streams the same 16 rows of a second matrix (up).
// Each wave stages only its own operands (its K range of the activations, the scales and biases
// of its groups) into its own LDS region, so it starts on its weights as soon as its own operands
// land; the only workgroup barrier is the final split-K reduction.
template <int BITS, int GS, int STEPS, int MR, int NMAT, int RING>
__global__ __launch_bounds__(kMaxWaves * 64) void qmv_mfma_kernel(
    const uint16_t* __restrict__ x, int M, int K, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint32_t* __restrict__ wq2, const uint16_t* __restrict__ scales2,
    const uint16_t* __restrict__ biases2, int N, int rows, uint16_t* __restrict__ y) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int NT = blockDim.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = (NT >> 6) / NMAT;  // waves per matrix
  const int mat = NMAT == 1 ? 0 : __builtin_amdgcn_readfirstlane(wave_all / W);
  const int n0 = blockIdx.x * rows;
  const int nr = N - n0 < rows ? N - n0 : rows;
  using Tile = GemvTile<BITS, GS, STEPS, MR, STEPS * RING>;
  Tile t(lane, wave_all, wave_all - mat * W, n0, nr, M, K, N, lds);
  const int sb_total = (int)(((uint32_t)N * (uint32_t)t.G * 2u + 3u) & ~3u);  // whole dwords
  t.issue_x(make_rsrc(x, M * K * 2));
  t.issue_sb(make_rsrc(mat ? scales2 : scales, sb_total), make_rsrc(mat ? biases2 : biases, sb_total));
  // The weight streams are issued once every wave of the workgroup has issued its operand
  // loads: a CU's vector memory requests are served in order, and a wave whose small operand
  // loads queue behind its neighbours' weight streams waits microseconds for them.  (A bare
  // s_barrier: nothing here waits for the loads themselves.)  The SwiGLU launch skips it: two of
  // its workgroups share a CU, and waiting for the workgroup's last-launched wave cost more there
  // (8.27 -> 8.02 us without it; the one-matrix launches are unchanged either way).
  if constexpr (NMAT == 1) __builtin_amdgcn_s_barrier();
  t.issue_w(make_rsrc(mat ? wq2 : wq, (int)((uint32_t)N * (uint32_t)(K * BITS / 8))));
  t.stage();
  float yacc[Tile::E];
  t.fold(yacc);
  gemv_reduce_store<NMAT>(lds, yacc, wave_all, W, lane, tid, NT, M, n0, nr, N, y);
}

// ---------------------------------------------------------------------------------------------
// M = 1, Q4: one weight row per wave.
//
// A wave streams its whole row (its gate and up rows in the SwiGLU form) in contiguous 512-byte
// loads, 8 bytes per lane, all issued up front, and computes the row's dot product alone: no
// split-K partials, no reduction through LDS, and no workgroup barrier after the one that
// publishes the staged activations.  (Streaming rows whole measured 3.66-3.70 us for the down
// codes against 4.08 us for the 16-row x 64-byte loads of the tile kernel above.)
//
// A 512-byte load holds 16 columns of 64 codes.  Lane L reads bytes [32n + 8q, +8) with
// n = L & 15, q = L >> 4: codes [16q, 16q + 16) of column n, i.e. its two words feed two MFMAs
// (v_mfma_f32_16x16x32_bf16) whose B column n is column n's 64 codes.  The A operand's row m is
// the activation run of column m (16 different K slices of the one activation row), so the
// product's diagonal C[n][n] is column n's dot product sum x*c, and the off-diagonal
// entries are discarded.  A row of K codes takes LS = ceil(K / 1024) loads; when K is not a
// multiple of 1024 the last load's upper columns reach into the next row (or past the buffer end,
// where the loads return zero), and those columns fold exactly zero: their staged activations,
// activation sums and (s, b) table entries are all zero.  C[n][n] sits in lane n + 16 (n >> 2), register n & 3: 16 lanes of the
// wave fold one column each per load,
//   y += s*C[n][n] + b*X[column],
// with X the column's activation sum (computed once per workgroup while staging).  The wave's
// 16 partial sums are added at the end with row shifts and lane reads.
constexpr int kRowColPitch = 144;  // LDS bytes per 64-element activation column (128 + pad)

// Loads per row (K <= 1024 times this): 32 for one matrix, 16 for the SwiGLU pair, whose wave
// holds two rows' codes in registers.
constexpr int kRowMaxLoads[2] = {32, 16};

// Whether the one-row kernel takes a problem (bf16 x and scales are checked by the caller): the
// group count per row must be even (scales and biases are read as group pairs, 4-byte aligned).
__host__ __device__ constexpr bool qmv_row_fits(int64_t M, int64_t K, int gs, int bits, int nmat) {
  return M == 1 && bits == 4 && (gs == 64 || gs == 128) && K % (2 * gs) == 0 && K >= 1024 &&
         K <= 1024 * kRowMaxLoads[nmat - 1];
}

// LDS bytes of a one-row workgroup: the activation columns, their sums and each wave's (s, zc)
// table per matrix.
__host__ __device__ constexpr int qmv_row_lds(int LS, bool g64, int nmat, int wpb) {
  return LS * 16 * kRowColPitch + LS * 16 * 4 + wpb * nmat * (g64 ? LS * 16 : LS * 8) * 8;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Contract (checked on the host by qmv_row_fits): M = 1, 1024 (LS - 1) < K <= 1024 LS, an even
// number of groups per row, bf16 x/scales/biases, Q4 codes, group 64 or 128, 8..16 waves per
// workgroup, dynamic LDS of qmv_row_lds bytes, every buffer < 2 GiB.  NMAT = 2: wave f streams
// gate row f and up row f and writes round(silu(round(g)) * round(u)) with
// silu(g) = round(g * round(sigmoid(g))) (qwen3.rs:178-181, src/nn.rs:301-303); else round(y).
// VALU: the same loads, unpack, staging and fold with the matrix cores left out — each lane forms
// the dot product of its 16 codes with their activations by v_dot2_f32_bf16, two products per
// instruction with f32 accumulation (y += s * dot, plus b * X once per column), and all 64 lanes' partial sums are added at the end.  It exists for the kernel-choice
// A/B (mlxq_qmv_valu), not for quantized_matmul.
template <bool G64, int LS, int NMAT, bool VALU = false>
__global__ __launch_bounds__(1024) void qmv_row_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint32_t* __restrict__ wq2,
    const uint16_t* __restrict__ scales2, const uint16_t* __restrict__ biases2, int K, int N,
    uint16_t* __restrict__ y) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  constexpr int C = 16 * LS;                  // 64-code columns per row, padded to whole loads
  constexpr int G = G64 ? C : C / 2;          // groups per padded row (table entries)
  constexpr int XCH = 128 * LS;               // 16-byte activation chunks of the padded row
  constexpr int XPT = (XCH + 511) / 512;      // ... per thread (at least 8 waves)
  constexpr int SBPL = (G + 127) / 128;       // scale/bias word pairs per lane
  const int Gr = K / (G64 ? 64 : 128);        // groups per row
  const uint32_t RB = (uint32_t)K / 2u;       // bytes per packed row
  const int NT = blockDim.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = blockIdx.x * (NT >> 6) + wave;
  const int r = row < N ? row : N - 1;  // waves past N take part in the staging, store nothing
  unsigned char* xs = lds;
  float* xsum = reinterpret_cast<float*>(lds + C * kRowColPitch);
  float* tab = xsum + C + wave * NMAT * G * 2;

  // Operand loads first (they queue ahead of the weight streams), then every weight load.  The
  // activation chunks past K read as zeros (past the resource's end).
  const auto rx = make_rsrc(x, K * 2);
  u32x4 cx[XPT];
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int ch = tid + j * NT;
    cx[j] = load16(rx, ch < XCH ? (uint32_t)ch * 16u : kOob);
  }
  const int sb_bytes = (int)((uint32_t)N * (uint32_t)Gr * 2u);
  uint32_t cs[NMAT][SBPL], cb[NMAT][SBPL];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const auto rs = make_rsrc(mat ? scales2 : scales, sb_bytes);
    const auto rz = make_rsrc(mat ? biases2 : biases, sb_bytes);
#pragma unroll
    for (int i = 0; i < SBPL; ++i) {
      const int g0 = 2 * lane + 128 * i;
      const uint32_t off = g0 < Gr ? ((uint32_t)r * (uint32_t)Gr + (uint32_t)g0) * 2u : kOob;
      cs[mat][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
      cb[mat][i] = __builtin_amdgcn_raw_buffer_load_b32(rz, off, 0, 0);
    }
  }
  // Every wave's activation loads go ahead of all weight streams in the CU's in-order memory
  // queue: the staging below needs the whole workgroup's (a bare s_barrier, no memory wait).
  __builtin_amdgcn_s_barrier();
  // Weight loads in fold order (step d of every matrix before step d + 1), so a step's operands
  // arrive together.
  u32x2 wv[NMAT][LS];
  const uint32_t lo = 32u * (uint32_t)(lane & 15) + 8u * (uint32_t)(lane >> 4);
  const int w_bytes = (int)((uint32_t)N * RB);
  const __amdgpu_buffer_rsrc_t rw[2] = {make_rsrc(wq, w_bytes), make_rsrc(NMAT == 2 ? wq2 : wq, w_bytes)};
#pragma unroll
  for (int d = 0; d < LS; ++d) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
      wv[mat][d] = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw[mat], (uint32_t)r * RB + (uint32_t)d * 512u + lo, 0, 0));
  }

  // Activation columns (runs permuted to the unpacked code order) and their sums: the 8 chunks
  // of a column sit in 8 consecutive lanes of one wave (NT is a multiple of 64).
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int ch = tid + j * NT;
    const u32x4 v = cx[j];
    float t = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) t += __uint_as_float(v[e] << 16) + __uint_as_float(v[e] & 0xffff0000u);
    t += dpp_f32<0xb1>(t);   // quad_perm [1,0,3,2]
    t += dpp_f32<0x4e>(t);   // quad_perm [2,3,0,1]: every lane holds its quad's sum
    t += dpp_f32<0x104>(t);  // row_shl:4: lane 8k adds lane 8k+4's quad
    // (only lanes 8k, the column's first chunk, store the sum)
    if (ch < XCH) {
      *reinterpret_cast<u32x4*>(xs + (ch >> 3) * kRowColPitch + (ch & 7) * 16) = perm_q4(v);
      if ((ch & 7) == 0) xsum[ch >> 3] = t;
    }
  }
  // Publish the activations with LDS-only fences: a __syncthreads() release fence would also
  // wait for every outstanding weight load.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  // The wave's (s, b) pairs per group, f32, after the barrier: only this wave reads them,
  // so the workgroup waits for the activations alone, not for every wave's scale loads.  Groups
  // past the row's end get (0, 0) (their loads returned zero).
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
#pragma unroll
    for (int i = 0; i < SBPL; ++i) {
      const int g0 = 2 * lane + 128 * i;
      if (g0 < G) {
        const float s0 = __uint_as_float(cs[mat][i] << 16), s1 = __uint_as_float(cs[mat][i] & 0xffff0000u);
        const float b0 = __uint_as_float(cb[mat][i] << 16), b1 = __uint_as_float(cb[mat][i] & 0xffff0000u);
        *reinterpret_cast<f32x4*>(tab + (mat * G + g0) * 2) = f32x4{s0, b0, s1, b1};
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");

  // Load d covers columns 16d .. 16d+15.  Lane (m, q) = (L & 15, L >> 4) reads A runs 2q, 2q+1 of
  // column 16d + m, and folds column 16d + n (n = m) from register e = L & 3 of the product.
  const int m = lane & 15, q = lane >> 4, e = lane & 3;
  const unsigned char* xa = xs + m * kRowColPitch + q * 32;
  bf16x8 a[LS][2];
  f32x2 p[LS][NMAT];
  float xg[LS];
  f32x4 acc[LS][NMAT];
  float ya[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) ya[mat] = 0.0f;
  auto read_step = [&](int d) {
    a[d][0] = *reinterpret_cast<const bf16x8*>(xa + d * 16 * kRowColPitch);
    a[d][1] = *reinterpret_cast<const bf16x8*>(xa + d * 16 * kRowColPitch + 16);
    const int col = 16 * d + m;
    const int g = G64 ? col : col >> 1;
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) p[d][mat] = *reinterpret_cast<const f32x2*>(tab + (mat * G + g) * 2);
    xg[d] = xsum[col];
  };
  auto mfma_step = [&](int d) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      if constexpr (VALU) {
        // unpack_q4's pairs line up with the activation run's bf16 pairs (the MFMA operands'
        // element order), so each v_dot2 adds two code-activation products.
        float part[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const u32x4 wb = __builtin_bit_cast(u32x4, unpack_q4(wv[mat][d][h]));
          const u32x4 xr = __builtin_bit_cast(u32x4, a[d][h]);
          float t = 0.0f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            // Elements copied out first: __builtin_bit_cast of a vector subscript (xr[j]) reads
            // element 0 for every j with this compiler.
            const uint32_t xj = xr[j], wj = wb[j];
            t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, xj), __builtin_bit_cast(bf16x2, wj), t, false);
          }
          part[h] = t;
        }
        const float dot = part[0] + part[1];
        acc[d][mat][0] = dot;
      } else {
        const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d][0], unpack_q4(wv[mat][d][0]),
                                                                f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        acc[d][mat] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d][1], unpack_q4(wv[mat][d][1]), c, 0, 0, 0);
      }
    }
  };
  auto fold_step = [&](int d) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      if constexpr (VALU) {
        // lane (m, q): s times its 16 codes' dot product; b times the column's activation sum
        // once per column (q == 0)
        ya[mat] = fmaf(p[d][mat][0], acc[d][mat][0], fmaf(q == 0 ? p[d][mat][1] : 0.0f, xg[d], ya[mat]));
      } else {
        const f32x4 c = acc[d][mat];
        float v = e == 1 ? c[1] : c[0];
        v = e == 2 ? c[2] : v;
        v = e == 3 ? c[3] : v;
        ya[mat] = fmaf(p[d][mat][0], v, fmaf(p[d][mat][1], xg[d], ya[mat]));
      }
      asm volatile("" : "+v"(ya[mat]));
    }
  };
  read_step(0);
#pragma unroll
  for (int d = 0; d < LS; ++d) {
    __builtin_amdgcn_sched_barrier(0);
    if (d + 1 < LS) read_step(d + 1 < LS ? d + 1 : d);
    mfma_step(d);
    if (d > 0) fold_step(d - 1);
  }
  __builtin_amdgcn_sched_barrier(0);
  fold_step(LS - 1);

  // The 16 diagonal lanes (n + 16 (n >> 2)) hold the partial sums (every lane in the VALU form):
  // a row-shift scan leaves each 16-lane row's sum in its lane 15.
  const bool diag = VALU || q == (m >> 2);
  float tot[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    float v = diag ? ya[mat] : 0.0f;
    v += dpp_f32<0x111>(v);
    v += dpp_f32<0x112>(v);
    v += dpp_f32<0x114>(v);
    v += dpp_f32<0x118>(v);
    tot[mat] = (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15)) +
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31))) +
               (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47)) +
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)));
  }
  if (lane == 0 && row < N) {
    float v = tot[0];
    if constexpr (NMAT == 2) {
      // each op rounded to bf16 as the reference's separate ops are (qwen3.rs:178-181)
      v = silu_bf16(round_bf16(v)) * round_bf16(tot[1]);
    }
    y[row] = f32_to_bf16_bits(v);
  }
}

namespace {

struct QmvPlan {
  int waves, steps, ring, mr, lds;  // waves: all waves of the workgroup (per matrix x matrices)
  int rows;                         // activation rows per launch: M, or 4 or 2 when M is split
};

constexpr int kStepChoices[] = {1, 2, 3, 4, 6, 8};

// Whether a kernel with a ring of `ring` rounds exists: two rounds only with 4..8 load registers
// and at most four activation rows (two with group 32, whose four-row ring spilled; more rows
// split into launches of four or two).
constexpr bool qmv_ring_built(int bits, int gs, int steps, int mr, int ring) {
  return ring == 1 || (ring == 2 && (bits == 4 || bits == 8) && steps >= 4 && mr <= (gs == 32 ? 2 : 4));
}

// Picks the load steps per wave: among the counts that divide the row's load steps, fit a
// workgroup of at most kMaxWaves waves, its LDS and its registers (qmv_steps_fit), the one whose
// workgroup comes closest to 12 waves (fewer steps on a tie).  Measured on the decode shapes
// (M = 1..8, K = 3072 and 8192, per-wave operand staging, pipelined fold), 8-12 waves of 3-8 steps
// finish first: a wave starts folding as soon as its own operands arrive, and more, shorter waves
// spread the fold's VALU work (which bounds the last waves' tail) over the SIMDs, while a 16-wave
// workgroup fills a CU on its own (128 registers per wave).  12 against 8: the down GEMV
// (K = 8192) 6.10 -> 5.84 us, gate (K = 3072) 5.40 -> 5.28 us, SwiGLU unchanged; 16 was no better.
//
// When no count divides the row's load steps within those limits (K = 11008: 86 steps of Q4),
// the waves take ceil(steps / waves) each and the last one's range ends past K (cost as above,
// then the fewest padded steps); failing that, each wave takes two rounds of its load registers
// (ring 2: twice the K at the same registers).  A launch holds its activation rows whole in LDS
// (M x K x 2 bytes), so rows that fit no plan go out as launches of four, else two rows (M = 8,
// K = 18944: four launches of two rows 46 us against 85 us on the VALU GEMV; single rows would
// stream the weights M times and lose to it).
static bool qmv_plan_rows(int64_t M, int64_t K, int gs, int bits, int nmat, QmvPlan& p) {
  const int64_t cpl = 512 / bits;
  const int64_t LS = K / cpl;
  const int mr = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
  for (int pass = 0; pass < 3; ++pass) {  // exact; ragged; ragged with two rounds
    const int ring = pass == 2 ? 2 : 1;
    bool found = false;
    int64_t best_cost = 0, best_pad = 0;
    for (int steps : kStepChoices) {
      if (!qmv_steps_fit(bits, gs, steps, mr) || !qmv_ring_built(bits, gs, steps, mr, ring)) continue;
      const int64_t t = (int64_t)steps * ring;  // load steps per wave
      if (pass == 0 && LS % t != 0) continue;
      const int64_t wpm = (LS + t - 1) / t;
      const int64_t waves = nmat * wpm;
      if (waves > kMaxWaves) continue;
      // activation chunks a lane stages (registers): at most kCopySlots across the rows
      if (mr * ((t * cpl / 8 + 63) / 64) > kCopySlots) continue;
      const int64_t operands = waves * (int64_t)qmv_wave_lds(bits, gs, (int)t, (int)M);
      const int64_t red = waves * 16 * 17 * 4;
      const int64_t lds = operands > red ? operands : red;
      if (lds > kMaxLds) continue;
      const int64_t cost = waves > 12 ? waves - 12 : 12 - waves;
      const int64_t pad = wpm * t - LS;
      if (found && (cost > best_cost || (cost == best_cost && pad >= best_pad))) continue;
      found = true;
      best_cost = cost;
      best_pad = pad;
      p = {(int)waves, steps, ring, mr, (int)lds, (int)M};
    }
    if (found) return true;
  }
  return false;
}

bool qmv_plan(int64_t M, int64_t K, int gs, int bits, int nmat, QmvPlan& p) {
  if (M < 1 || M > 8 || (bits != 4 && bits != 8)) return false;
  if (gs != 32 && gs != 64 && gs != 128) return false;
  const int64_t cpl = 512 / bits;
  if (K <= 0 || K % cpl != 0 || K % gs != 0) return false;
  if (qmv_plan_rows(M, K, gs, bits, nmat, p)) return true;
  for (int rows : {4, 2})  // launches of fewer rows
    if (M > rows && qmv_plan_rows(rows, K, gs, bits, nmat, p)) return true;
  return false;
}

// Device operands of one launch (the second matrix is used by the SwiGLU form only).
struct QmvArgs {
  const void* x;
  int64_t M, K, N;
  const uint32_t* wq;
  const void *s, *b;
  const uint32_t* wq2;
  const void *s2, *b2;
  void* y;
};

}  // namespace

static int qmv_row_wpb(int64_t N, int nmat);

// Rows per tile workgroup: 16 for SwiGLU; for one matrix, of 16, 12 and 8 the count whose
// busiest CU streams the fewest rows, the rule of the one-row kernel (the MFMA columns past the
// count load nothing).  The down projection of a decode MLP (N = 3072) takes 12 rows: 256
// workgroups, every CU, where 16-row tiles left 64 CUs idle.
template <int BITS, int GS, int STEPS, int MR, int NMAT, int RING>
static int launch_qmv_mfma(const QmvArgs& a, const QmvPlan& p, hipStream_t st) {
  // The dynamic-LDS limit is raised once per device (any thread may get here first; setting it
  // twice is harmless).
  static std::atomic<bool> attr_set[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(MLXQ_EDEVICE, "qmv: no current device");
  if (dev < 0 || dev >= 64 || !attr_set[dev].load(std::memory_order_acquire)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&qmv_mfma_kernel<BITS, GS, STEPS, MR, NMAT, RING>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds) != hipSuccess)
      return set_error(MLXQ_EDEVICE, "qmv: hipFuncSetAttribute failed");
    if (dev >= 0 && dev < 64) attr_set[dev].store(true, std::memory_order_release);
  }
  const int rows = NMAT == 1 ? qmv_row_wpb(a.N, 1) : 16;
  hipLaunchKernelGGL((qmv_mfma_kernel<BITS, GS, STEPS, MR, NMAT, RING>), dim3((unsigned)((a.N + rows - 1) / rows)),
                     dim3(p.waves * 64), p.lds, st, (const uint16_t*)a.x, (int)a.M, (int)a.K, a.wq,
                     (const uint16_t*)a.s, (const uint16_t*)a.b, a.wq2, (const uint16_t*)a.s2,
                     (const uint16_t*)a.b2, (int)a.N, rows, (uint16_t*)a.y);
  return check_launch(NMAT == 2 ? "swiglu_qmv" : "qmv_mfma");
}

template <int BITS, int GS, int STEPS, int MR, int NMAT>
static int qmv_mr(const QmvArgs& a, const QmvPlan& p, hipStream_t st) {
  if constexpr (qmv_steps_fit(BITS, GS, STEPS, MR)) {
    if (p.ring == 1) return launch_qmv_mfma<BITS, GS, STEPS, MR, NMAT, 1>(a, p, st);
    if constexpr (qmv_ring_built(BITS, GS, STEPS, MR, 2))
      if (p.ring == 2) return launch_qmv_mfma<BITS, GS, STEPS, MR, NMAT, 2>(a, p, st);
    return set_error(MLXQ_EINVAL, "qmv: no kernel with %d load rounds for this plan", p.ring);
  } else {
    return set_error(MLXQ_EINVAL, "qmv: %d load steps per wave with %d rows exceed the registers", STEPS, MR);
  }
}

template <int BITS, int GS, int STEPS, int NMAT>
static int qmv_rows(const QmvArgs& a, const QmvPlan& p, hipStream_t st) {
  switch (p.mr) {
    case 1: return qmv_mr<BITS, GS, STEPS, 1, NMAT>(a, p, st);
    case 2: return qmv_mr<BITS, GS, STEPS, 2, NMAT>(a, p, st);
    case 4: return qmv_mr<BITS, GS, STEPS, 4, NMAT>(a, p, st);
    default: return qmv_mr<BITS, GS, STEPS, 8, NMAT>(a, p, st);
  }
}

template <int BITS, int GS, int NMAT>
static int qmv_steps(const QmvArgs& a, const QmvPlan& p, hipStream_t st) {
  switch (p.steps) {
    case 1: return qmv_rows<BITS, GS, 1, NMAT>(a, p, st);
    case 2: return qmv_rows<BITS, GS, 2, NMAT>(a, p, st);
    case 3: return qmv_rows<BITS, GS, 3, NMAT>(a, p, st);
    case 4: return qmv_rows<BITS, GS, 4, NMAT>(a, p, st);
    case 6: return qmv_rows<BITS, GS, 6, NMAT>(a, p, st);
    default: return qmv_rows<BITS, GS, 8, NMAT>(a, p, st);
  }
}

template <int NMAT>
static int qmv_kind(const QmvArgs& a, int gs, int bits, const QmvPlan& p, hipStream_t st) {
  if (bits == 8) {
    if (gs == 32) return qmv_steps<8, 32, NMAT>(a, p, st);
    if (gs == 64) return qmv_steps<8, 64, NMAT>(a, p, st);
    return qmv_steps<8, 128, NMAT>(a, p, st);
  }
  if (gs == 32) return qmv_steps<4, 32, NMAT>(a, p, st);
  if (gs == 64) return qmv_steps<4, 64, NMAT>(a, p, st);
  return qmv_steps<4, 128, NMAT>(a, p, st);
}

// CUs of the current device.
static int64_t gemv_cus() { return device_cu_count(); }

// Waves (rows) per one-row workgroup.  SwiGLU (two rows per wave): 8, i.e. the staging barrier
// among fewer waves (K = 3072, F = 8192: 7.7 -> 7.1 us against 16 waves; 4 measured slower).
// One matrix: of 16, 12 and 8 the one whose busiest CU streams the fewest rows,
// ceil(ceil(N / w) / CUs) * w, the larger on a tie.  Measured over 14 shapes (K = 2048..28672,
// N = 1536..8192) the launch time follows that count: N = 3072 takes 12 (4.74 us against 4.94 at 8
// and 5.37 at 16), N = 5120 takes 12 (K = 13824: 13.6 us against 15.1 at 16), N = 1536 takes 8
// (3.99 against 5.29 at 16), N = 3584 and 8192 take 16.
static int qmv_row_wpb(int64_t N, int nmat) {
  if (nmat == 2) return 8;
  const int64_t cus = gemv_cus();
  int best = 16;
  int64_t best_rows = 0;
  for (int w : {16, 12, 8}) {
    const int64_t rows = ((N + w - 1) / w + cus - 1) / cus * w;
    if (best_rows == 0 || rows < best_rows) {
      best = w;
      best_rows = rows;
    }
  }
  return best;
}

template <bool G64, int LS, int NMAT, bool VALU = false>
static int launch_qmv_row(const QmvArgs& a, hipStream_t st) {
  static_assert(qmv_row_lds(LS, G64, NMAT, 16) <= kMaxLds, "one-row workgroup exceeds the LDS");
  static std::atomic<bool> attr_set[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(MLXQ_EDEVICE, "qmv: no current device");
  if (dev < 0 || dev >= 64 || !attr_set[dev].load(std::memory_order_acquire)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&qmv_row_kernel<G64, LS, NMAT, VALU>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds) != hipSuccess)
      return set_error(MLXQ_EDEVICE, "qmv: hipFuncSetAttribute failed");
    if (dev >= 0 && dev < 64) attr_set[dev].store(true, std::memory_order_release);
  }
  const int wpb = qmv_row_wpb(a.N, NMAT);
  const int lds = qmv_row_lds(LS, G64, NMAT, wpb);
  hipLaunchKernelGGL((qmv_row_kernel<G64, LS, NMAT, VALU>), dim3((unsigned)((a.N + wpb - 1) / wpb)),
                     dim3(wpb * 64), lds, st, (const uint16_t*)a.x, a.wq, (const uint16_t*)a.s,
                     (const uint16_t*)a.b, a.wq2, (const uint16_t*)a.s2, (const uint16_t*)a.b2, (int)a.K,
                     (int)a.N, (uint16_t*)a.y);
  return check_launch(NMAT == 2 ? "swiglu_qmv_row" : VALU ? "qmv_row_valu" : "qmv_row");
}

// Launchers by loads per row (1 .. kRowMaxLoads).
template <bool G64, int NMAT, bool VALU = false, int... L>
static int qmv_row_ls(const QmvArgs& a, hipStream_t st, std::integer_sequence<int, L...>) {
  using Launch = int (*)(const QmvArgs&, hipStream_t);
  static constexpr Launch launch[] = {&launch_qmv_row<G64, L + 1, NMAT, VALU>...};
  return launch[(a.K + 1023) / 1024 - 1](a, st);
}

template <int NMAT>
static int qmv_row(const QmvArgs& a, int gs, hipStream_t st) {
  constexpr auto ls = std::make_integer_sequence<int, kRowMaxLoads[NMAT - 1]>{};
  return gs == 64 ? qmv_row_ls<true, NMAT>(a, st, ls) : qmv_row_ls<false, NMAT>(a, st, ls);
}

static bool buffers_fit(int64_t M, int64_t K, int64_t N) {
  const int64_t lim = (int64_t)1 << 31;  // every buffer (Q8 weights: N*K bytes) under 2 GiB
  return N * K < lim && M * K * 2 < lim;
}

bool qmv_mfma_applicable(int x_dtype, int sb_dtype, int64_t M, int64_t K, int64_t N, int gs, int bits) {
  if (x_dtype != MLXQ_BFLOAT16 || sb_dtype != MLXQ_BFLOAT16 || !buffers_fit(M, K, N)) return false;
  QmvPlan p;
  return qmv_row_fits(M, K, gs, bits, 1) || qmv_plan(M, K, gs, bits, 1, p);
}

int run_qmv_mfma(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s, const void* b,
                 int64_t N, int gs, int bits, void* y, hipStream_t st) {
  const QmvArgs a = {x, M, K, N, wq, s, b, nullptr, nullptr, nullptr, y};
  if (qmv_row_fits(M, K, gs, bits, 1)) return qmv_row<1>(a, gs, st);
  QmvPlan p;
  if (!qmv_plan(M, K, gs, bits, 1, p))
    return set_error(MLXQ_EINVAL, "qmv: no GEMV plan for M=%lld K=%lld", (long long)M, (long long)K);
  if (p.rows == M) return qmv_kind<1>(a, gs, bits, p, st);
  for (int64_t m0 = 0; m0 < M; m0 += p.rows) {  // launches of p.rows activation rows
    const int64_t rows = M - m0 < p.rows ? M - m0 : p.rows;
    const int rc = run_qmv_mfma(static_cast<const uint16_t*>(x) + m0 * K, rows, K, wq, s, b, N, gs, bits,
                                static_cast<uint16_t*>(y) + m0 * N, st);
    if (rc != MLXQ_OK) return rc;
  }
  return MLXQ_OK;
}

// The VALU form of the one-row kernel (the kernel-choice A/B behind mlxq_qmv_valu): bf16 x and
// scales, M = 1, Q4 group 64/128, K up to kRowValuMaxLoads * 1024 (the decode shapes).
constexpr int kRowValuMaxLoads = 8;

bool qmv_row_valu_applicable(int x_dtype, int sb_dtype, int64_t M, int64_t K, int64_t N, int gs, int bits) {
  return x_dtype == MLXQ_BFLOAT16 && sb_dtype == MLXQ_BFLOAT16 && buffers_fit(M, K, N) &&
         qmv_row_fits(M, K, gs, bits, 1) && K <= 1024 * kRowValuMaxLoads;
}

int run_qmv_row_valu(const void* x, int64_t K, const uint32_t* wq, const void* s, const void* b, int64_t N,
                     int gs, void* y, hipStream_t st) {
  const QmvArgs a = {x, 1, K, N, wq, s, b, nullptr, nullptr, nullptr, y};
  constexpr auto ls = std::make_integer_sequence<int, kRowValuMaxLoads>{};
  return gs == 64 ? qmv_row_ls<true, 1, true>(a, st, ls) : qmv_row_ls<false, 1, true>(a, st, ls);
}

bool swiglu_qmv_applicable(int x_dtype, int sb_dtype, int64_t M, int64_t K, int64_t F, int gs, int bits) {
  if (x_dtype != MLXQ_BFLOAT16 || sb_dtype != MLXQ_BFLOAT16 || !buffers_fit(M, K, F)) return false;
  QmvPlan p;
  return qmv_row_fits(M, K, gs, bits, 2) || qmv_plan(M, K, gs, bits, 2, p);
}

int run_swiglu_qmv(const void* x, int64_t M, int64_t K, const uint32_t* wq_g, const void* s_g,
                   const void* b_g, const uint32_t* wq_u, const void* s_u, const void* b_u, int64_t F,
                   int gs, int bits, void* h, hipStream_t st) {
  const QmvArgs a = {x, M, K, F, wq_g, s_g, b_g, wq_u, s_u, b_u, h};
  if (qmv_row_fits(M, K, gs, bits, 2)) return qmv_row<2>(a, gs, st);
  QmvPlan p;
  if (!qmv_plan(M, K, gs, bits, 2, p))
    return set_error(MLXQ_EUNSUPPORTED, "swiglu: no fused GEMV plan for M=%lld K=%lld", (long long)M,
                     (long long)K);
  if (p.rows == M) return qmv_kind<2>(a, gs, bits, p, st);
  for (int64_t m0 = 0; m0 < M; m0 += p.rows) {  // launches of p.rows activation rows
    const int64_t rows = M - m0 < p.rows ? M - m0 : p.rows;
    const int rc = run_swiglu_qmv(static_cast<const uint16_t*>(x) + m0 * K, rows, K, wq_g, s_g, b_g, wq_u, s_u,
                                  b_u, F, gs, bits, static_cast<uint16_t*>(h) + m0 * F, st);
    if (rc != MLXQ_OK) return rc;
  }
  return MLXQ_OK;
}

}  // namespace mlxq
