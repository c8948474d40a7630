// qmv_mfma.hip — decode GEMV y[M,N] = x[M,K] . W^T for M <= 8 on gfx950 matrix cores.
//
// The path is HBM-bound and small (a few MB per call), so what matters is latency: every load a
// wave needs is issued up front, the packed weights go straight into MFMA operand registers, and
// each K step is folded as soon as its weights arrive (the step code is branch-free, so the
// compiler waits for exactly one load per step instead of the whole stream).
//
// Semantics are the exact-f32 factored form (no bf16 rounding of dequantized weights):
//   y[m,n] = sum_g ( s[n,g] * sum_{k in g} x[m,k]*c[n,k]  +  b[n,g] * X[m,g] ),  X = sum_{k in g} x.
// Q4 codes enter the MFMA as the exact bf16 value 128+c (bf16 bits 0x4300|c, built with one
// and-or per code pair), so acc = sum x*(128+c) and the fold per 64-wide K step is
//   y += s*acc + (b - 128*s)*X.
// Q8 codes enter as bf16(c) (exact for c < 256) and fold as y += s*acc + b*X.
// X comes from the same activation fragments multiplied by an all-ones operand on the MFMA.
//
// v_mfma_f32_16x16x32_bf16 with A = activations (rows m = lane&15; rows >= M read row 0 and are
// never stored) and B = weights (columns n = lane&15).  Lane quarter q = lane>>4 supplies the
// 16 codes [16q, 16q+16) of the row's 64-wide K step (one 8-byte load for Q4, 16 bytes for Q8);
// MFMA j takes codes [16q+8j, 16q+8j+8), so every MFMA stays inside one group (group_size 64 or
// 128).  The 16x16 result holds column n = lane&15 for rows m = 4q + e.
// A workgroup owns 16 weight rows; its SPLIT waves split K and reduce through LDS at the end.
// Q4 k-order inside an 8-run is [0,4,1,5,2,6,3,7] (how the and-or pairs nibbles i and i+4); the
// activation rows are permuted to match with v_perm_b32 as they are copied into LDS.
#include "mlxq_common.h"

namespace mlxq {

namespace {

constexpr int kBufferFlags = 0x00020000;
constexpr int kMaxSteps = 8;   // K steps per wave (all loads issued at once)
constexpr int kMaxRows = 8;    // activation rows
constexpr int kMaxLds = 160 * 1024;
constexpr uint32_t kOob = 0x7ffffff0u;  // buffer offset past every resource: loads return zero

// LDS: activations [M][K] (rows padded by 16 bytes so rows start on different banks), then the
// workgroup's 16 scale rows and 16 bias rows [16][G] in the scales dtype.
struct QmvLds {
  int x_stride, sb_off, sb_bytes, total;
};
__host__ __device__ inline QmvLds qmv_lds_layout(int M, int64_t K, int gs, int sb_size) {
  QmvLds L;
  L.x_stride = (int)(K * 2 + 16);
  L.sb_off = M * L.x_stride;
  L.sb_bytes = 16 * (int)(K / gs) * sb_size;
  L.total = L.sb_off + 2 * L.sb_bytes;
  return L;
}

// Q4 word -> bf16 pairs (128+c_i, 128+c_{i+4}), i = 0..3.
__device__ __forceinline__ bf16x8 magic_q4(uint32_t w) {
  u32x4 o;
  o[0] = (w & 0x000f000fu) | 0x43004300u;
  o[1] = ((w >> 4) & 0x000f000fu) | 0x43004300u;
  o[2] = ((w >> 8) & 0x000f000fu) | 0x43004300u;
  o[3] = ((w >> 12) & 0x000f000fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8, o);
}

// Activation run x0..x7 (raw bf16 pairs r0..r3) -> order [0,4,1,5,2,6,3,7].
__device__ __forceinline__ u32x4 perm_q4(u32x4 r) {
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(r[2], r[0], 0x05040100u);
  o[1] = __builtin_amdgcn_perm(r[2], r[0], 0x07060302u);
  o[2] = __builtin_amdgcn_perm(r[3], r[1], 0x05040100u);
  o[3] = __builtin_amdgcn_perm(r[3], r[1], 0x07060302u);
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

}  // namespace

// Launch contract (checked on the host by qmv_mfma_applicable): 1 <= M <= 8, K % 64 == 0,
// K/8 <= SPLIT*64 (one activation chunk per thread and row), G*sizeof(SB) <= SPLIT*64 (one scale
// chunk and one bias chunk per thread), ceil(K/64 / SPLIT) == STEPS, every buffer < 2 GiB.
template <typename SB, int BITS, int SPLIT, int STEPS>
__global__ __launch_bounds__(SPLIT * 64) void qmv_mfma_kernel(
    const uint16_t* __restrict__ x, int M, int K, const uint32_t* __restrict__ wq,
    const SB* __restrict__ scales, const SB* __restrict__ biases, int N, int gs,
    uint16_t* __restrict__ y) {
  constexpr int WW = BITS == 4 ? 2 : 4;  // packed words per lane per K step
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = n0 + c16;
  const int nn = n < N ? n : N - 1;
  const int kwords = K * BITS / 32;
  const int gshift = gs == 128 ? 1 : 0;  // 64-wide K steps per group: 1 or 2
  const int G = (K >> 6) >> gshift;
  const int KT = K / 64;
  const int kt0 = wave * STEPS;  // this wave's K steps: [kt0, min(kt0 + STEPS, KT))
  QmvLds L;  // qmv_lds_layout without the division
  L.x_stride = K * 2 + 16;
  L.sb_off = M * L.x_stride;
  L.sb_bytes = 16 * G * (int)sizeof(SB);

  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, M * K * 2, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(wq), (short)0, (int)((uint32_t)N * (uint32_t)kwords * 4u), kBufferFlags);
  // Rounded up to whole dwords: buffer range checks are per dword, and the last bf16 scale may
  // share its dword with 2 bytes past the end (same aligned dword, so never another page; the
  // extra value lands in the LDS slot of a row >= N, which is never stored).
  const int sb_total = (int)(((uint32_t)N * (uint32_t)G * sizeof(SB) + 3u) & ~3u);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<SB*>(scales), (short)0, sb_total, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rz =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<SB*>(biases), (short)0, sb_total, kBufferFlags);

  // 1. Workgroup operands first (small; they return before the weight stream): one 16-byte chunk
  //    per thread of each activation row, and of the contiguous scale and bias rows of this
  //    workgroup's 16 weight rows.  Threads past the end read at an out-of-range offset (zero).
  const int x_chunks = K / 8;
  const int sb_chunks = L.sb_bytes / 16;
  const uint32_t x_off = tid < x_chunks ? (uint32_t)tid * 16u : kOob;
  const uint32_t sb_off = tid < sb_chunks ? (uint32_t)n0 * (uint32_t)G * sizeof(SB) + (uint32_t)tid * 16u : kOob;
  u32x4 cx[kMaxRows];
#pragma unroll
  for (int m = 0; m < kMaxRows; ++m)
    if (m < M) cx[m] = load16(rx, x_off + (uint32_t)(m * K * 2));
  const u32x4 cs = load16(rs, sb_off);
  const u32x4 cz = load16(rz, sb_off);

  // 2. The wave's whole weight stream (branch-free: steps past KT, only possible in the last
  //    wave, re-read step KT-1 and are folded with weight zero).
  const uint32_t w_base = ((uint32_t)nn * (uint32_t)kwords + (uint32_t)(q * WW)) * 4u;
  uint32_t wv[STEPS][WW];
#pragma unroll
  for (int d = 0; d < STEPS; ++d) {
    const int kt = kt0 + d < KT ? kt0 + d : KT - 1;
    if constexpr (BITS == 4) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(rw, w_base + (uint32_t)kt * 32u, 0, 0);
      wv[d][0] = v[0];
      wv[d][1] = v[1];
    } else {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rw, w_base + (uint32_t)kt * 64u, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) wv[d][e] = v[e];
    }
  }

  // 3. Operands into LDS.  Q4 activation runs are stored permuted to [0,4,1,5,2,6,3,7] so they
  //    pair with the and-or code layout without per-wave work.
  if (tid < x_chunks) {
#pragma unroll
    for (int m = 0; m < kMaxRows; ++m)
      if (m < M)
        *reinterpret_cast<u32x4*>(lds + m * L.x_stride + tid * 16) = BITS == 4 ? perm_q4(cx[m]) : cx[m];
  }
  if (tid < sb_chunks) {
    *reinterpret_cast<u32x4*>(lds + L.sb_off + tid * 16) = cs;
    *reinterpret_cast<u32x4*>(lds + L.sb_off + L.sb_bytes + tid * 16) = cz;
  }
  __syncthreads();

  // 4. Per K step: 2 MFMAs x . codes and 2 MFMAs x . ones (group sums), then the fold.  Steps
  //    past KT recompute step KT-1 with scale and bias zero.
  const unsigned char* xrow = lds + (c16 < M ? c16 : 0) * L.x_stride + q * 32;
  const SB* s_lds = reinterpret_cast<const SB*>(lds + L.sb_off) + c16 * G;
  const SB* z_lds = reinterpret_cast<const SB*>(lds + L.sb_off + L.sb_bytes) + c16 * G;
  bf16x8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (__bf16)1.0f;
  f32x4 yacc = {0.0f, 0.0f, 0.0f, 0.0f};  // rows m = 4q + e, column n
#pragma unroll
  for (int d = 0; d < STEPS; ++d) {
    const bool valid = kt0 + d < KT;
    const int kt = valid ? kt0 + d : KT - 1;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, xsum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(xrow + kt * 128 + j * 16);
      const bf16x8 b = BITS == 4 ? magic_q4(wv[d][j]) : cvt_q8(wv[d][2 * j], wv[d][2 * j + 1]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
      xsum = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, xsum, 0, 0, 0);
    }
    const int g = kt >> gshift;
    const float s_raw = SBLoad<SB>::ld(s_lds, g), z_raw = SBLoad<SB>::ld(z_lds, g);
    const float s = valid ? s_raw : 0.0f;
    const float z = valid ? z_raw : 0.0f;
    const float zc = BITS == 4 ? fmaf(-128.0f, s, z) : z;
#pragma unroll
    for (int e = 0; e < 4; ++e) yacc[e] = fmaf(s, acc[e], fmaf(zc, xsum[e], yacc[e]));
  }

  // 5. Split-K reduction through LDS (reuses the operand area): [wave][m 0..15][n 0..15].
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int e = 0; e < 4; ++e) red[(wave * 16 + 4 * q + e) * 17 + c16] = yacc[e];
  __syncthreads();
  if (tid < 128) {
    const int m = tid >> 4, nl = tid & 15;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < SPLIT; ++w) v += red[(w * 16 + m) * 17 + nl];
    if (m < M && n0 + nl < N) y[(int64_t)m * N + n0 + nl] = f32_to_bf16_bits(v);
  }
}

template <typename SB, int BITS, int SPLIT, int STEPS>
static int launch_qmv_mfma(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                           const void* b, int64_t N, int gs, void* y, hipStream_t st) {
  const int64_t blocks = (N + 15) / 16;
  const QmvLds L = qmv_lds_layout((int)M, K, gs, sizeof(SB));
  const int red = SPLIT * 16 * 17 * 4;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&qmv_mfma_kernel<SB, BITS, SPLIT, STEPS>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds) != hipSuccess)
      return set_error(MLXQ_EDEVICE, "qmv: hipFuncSetAttribute failed");
    attr_set = true;
  }
  hipLaunchKernelGGL((qmv_mfma_kernel<SB, BITS, SPLIT, STEPS>), dim3((unsigned)blocks),
                     dim3(SPLIT * 64), L.total > red ? L.total : red, st, (const uint16_t*)x, (int)M,
                     (int)K, wq, (const SB*)s, (const SB*)b, (int)N, gs, (uint16_t*)y);
  return check_launch("qmv_mfma");
}

// 16 waves split K (fewer when K is short); each wave gets STEPS = ceil(KT/16) <= 8 steps.
static void qmv_shape(int64_t K, int& split, int& steps) {
  const int64_t KT = K / 64;
  split = KT >= 16 ? 16 : (KT >= 8 ? 8 : (KT >= 4 ? 4 : (KT >= 2 ? 2 : 1)));
  steps = (int)((KT + split - 1) / split);
}

template <typename SB, int BITS>
static int qmv_mfma_dispatch(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                             const void* b, int64_t N, int gs, void* y, hipStream_t st) {
  int split, steps;
  qmv_shape(K, split, steps);
#define MLXQ_S(SP, ST) \
  if (split == SP && steps == ST) return launch_qmv_mfma<SB, BITS, SP, ST>(x, M, K, wq, s, b, N, gs, y, st);
  MLXQ_S(16, 1) MLXQ_S(16, 2) MLXQ_S(16, 3) MLXQ_S(16, 4) MLXQ_S(16, 5) MLXQ_S(16, 6) MLXQ_S(16, 7)
  MLXQ_S(16, 8) MLXQ_S(8, 1) MLXQ_S(8, 2) MLXQ_S(4, 1) MLXQ_S(4, 2) MLXQ_S(2, 1) MLXQ_S(2, 2)
  MLXQ_S(1, 1)
#undef MLXQ_S
  return set_error(MLXQ_EINVAL, "qmv: no GEMV shape for K=%lld", (long long)K);
}

bool qmv_mfma_applicable(int x_dtype, int64_t M, int64_t K, int64_t N, int gs) {
  const int64_t lim = (int64_t)1 << 31;
  if (x_dtype != MLXQ_BFLOAT16 || M < 1 || M > kMaxRows || (gs != 64 && gs != 128) || K % 64 != 0)
    return false;
  // every buffer (Q8 weights are the largest, N*K bytes; f32 scales N*G*4) under 2 GiB
  if (N * K >= lim || M * K * 2 >= lim || N * (K / gs) * 4 >= lim) return false;
  int split, steps;
  qmv_shape(K, split, steps);
  const int64_t threads = (int64_t)split * 64;
  if (steps > kMaxSteps || K / 8 > threads || (K / gs) * 4 > threads) return false;
  return qmv_lds_layout((int)M, K, gs, 4).total <= kMaxLds;
}

int run_qmv_mfma(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s, const void* b,
                 int sb_dtype, int64_t N, int gs, int bits, void* y, hipStream_t st) {
  if (sb_dtype == MLXQ_BFLOAT16) {
    if (bits == 4) return qmv_mfma_dispatch<uint16_t, 4>(x, M, K, wq, s, b, N, gs, y, st);
    return qmv_mfma_dispatch<uint16_t, 8>(x, M, K, wq, s, b, N, gs, y, st);
  }
  if (bits == 4) return qmv_mfma_dispatch<float, 4>(x, M, K, wq, s, b, N, gs, y, st);
  return qmv_mfma_dispatch<float, 8>(x, M, K, wq, s, b, N, gs, y, st);
}

}  // namespace mlxq
