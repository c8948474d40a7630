// quantize.hip — affine group quantize / dequantize for gfx950.
//
// Both kernels are HBM-bound streaming passes over a flat 1-D grid.  quantize: one thread owns 32
// consecutive elements of a row (four 16-byte bf16 loads; four or eight packed words out), a
// group of gs elements is gs/32 adjacent lanes, and the group's min/max is a DPP exchange over
// those lanes.  dequantize: one thread owns 8 elements (one or two packed words in, one 16-byte bf16
// store out).
#include "mlxq_common.h"

namespace mlxq {

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]);

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float (&v)[8]) {
  u32x4 r = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(r[i] << 16);
    v[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&v)[8]) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = a[i];
    v[4 + i] = b[i];
  }
}

// Codes: clamp(round((w - bias) / s), 0, nb) with round half away from zero and an IEEE
// quotient, as MLX computes them.  The fast form evaluates y = (w - bias) * rcp(s) + 0.5 + 2^-12
// in one FMA; for t >= 0, round half away is floor(t + 0.5), so the code is floor(y) clamped to
// [0, nb] (a truncating convert of med3(y, 0, nb)).  The product differs from the exact quotient
// by at most ~3 ulp of t <= 255 (under 2^-14 with y's own rounding), so floor(y) is right unless
// t lies within 2^-12 of a half-integer, i.e. unless fract(y) < 2^-11.  Those codes (about one
// element in 2000) are recomputed with the exact division and roundf in a rarely taken second
// pass.  w - bias is formed before the product on purpose: folding it into
// fma(w, 1/s, -bias/s) would add an error proportional to |bias / s|, unbounded for a narrow
// group far from zero.
__device__ __forceinline__ uint32_t code_exact(float a, float s, float nb) {
  return (uint32_t)fminf(fmaxf(roundf(a / s), 0.0f), nb);
}

// max / min over the LANES (1, 2 or 4) adjacent lanes of a group: DPP quad permutes (xor 1,
// xor 2), no LDS traffic.
template <int LANES>
__device__ __forceinline__ void group_minmax(float& mx, float& mn) {
  if constexpr (LANES >= 2) {
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0xB1, 0xF, 0xF, false)));
    mn = fminf(mn, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mn), 0xB1, 0xF, 0xF, false)));
  }
  if constexpr (LANES >= 4) {
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x4E, 0xF, 0xF, false)));
    mn = fminf(mn, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mn), 0x4E, 0xF, 0xF, false)));
  }
  static_assert(LANES == 1 || LANES == 2 || LANES == 4, "group lanes");
}

// w [N,K] (bf16 bits or f32) -> wq [N, K*BITS/32], scales/biases [N, K/GS] in T.
// Group parameters follow MLX's edge-exact affine scheme: the larger-magnitude end of the group
// range is reproduced exactly (it becomes the bias) and the scale carries the sign.
// A thread owns EPT = 32 consecutive elements (four 16-byte bf16 loads), so a group is GS/32
// lanes (1, 2 or 4): the per-group work (three IEEE divisions, the lane exchange) is shared by
// 32 elements, and each element costs about seven VALU operations.  Thread `chunk` of the
// weight's flat grid does chunk `chunk`.
template <typename T, int BITS, int GS>
__device__ __forceinline__ void quantize_chunk(const T* __restrict__ w, int64_t n_chunks,
                                               uint32_t* __restrict__ wq, T* __restrict__ scales,
                                               T* __restrict__ biases, int64_t chunk) {
  constexpr int EPT = 32;
  constexpr int LANES = GS / EPT;  // lanes per group
  constexpr int WPT = EPT * BITS / 32;  // packed words per thread: 4 (Q4) or 8 (Q8)
  constexpr float nb = (float)((1 << BITS) - 1);
  constexpr float kTieWin = 0x1p-12f;
  // n_chunks is a multiple of LANES, so whole groups are either fully in or fully out.  Threads
  // past the end read chunk 0 (in bounds; n_chunks > 0) and return before storing anything.
  const bool live = chunk < n_chunks;
  const int64_t src = live ? chunk : 0;
  float v[EPT];
#pragma unroll
  for (int q = 0; q < EPT / 8; ++q)
    load8<T>(w + src * EPT + 8 * q, *reinterpret_cast<float(*)[8]>(&v[8 * q]));
  float mx = v[0], mn = v[0];
#pragma unroll
  for (int i = 1; i < EPT; ++i) {
    mx = fmaxf(mx, v[i]);
    mn = fminf(mn, v[i]);
  }
  group_minmax<LANES>(mx, mn);
  if (!live) return;
  float s = fmaxf((mx - mn) / nb, 1e-7f);
  const bool side = fabsf(mn) > fabsf(mx);
  s = side ? s : -s;
  const float edge = side ? mn : mx;
  const float q0 = roundf(edge / s);
  const bool at_zero = q0 == 0.0f;
  s = at_zero ? s : edge / q0;
  const float bias = at_zero ? 0.0f : edge;
  const float rs = __builtin_amdgcn_rcpf(s);  // error covered by the near-tie window

  if ((threadIdx.x & (LANES - 1)) == 0) {
    const int64_t g = chunk / LANES;  // row-major group index == row*(K/GS) + group
    SBLoad<T>::st(scales, g, s);
    SBLoad<T>::st(biases, g, bias);
  }
  uint32_t words[WPT];
  bool near[EPT];
  bool any_near = false;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const float y = fmaf(v[i] - bias, rs, 0.5f + kTieWin);
    near[i] = __builtin_amdgcn_fractf(y) < 2.0f * kTieWin;
    any_near |= near[i];
    const uint32_t c = (uint32_t)__builtin_amdgcn_fmed3f(y, 0.0f, nb);
    constexpr int per = 32 / BITS;
    if (i % per == 0) words[i / per] = c;
    else words[i / per] |= c << ((i % per) * BITS);
  }
  if (__builtin_expect(any_near, 0)) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      if (near[i]) {
        const uint32_t sh = (i * BITS) % 32, m = ((1u << BITS) - 1u) << sh;
        words[i * BITS / 32] = (words[i * BITS / 32] & ~m) | (code_exact(v[i] - bias, s, nb) << sh);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < WPT / 4; ++q)
    *reinterpret_cast<u32x4*>(wq + chunk * WPT + 4 * q) =
        u32x4{words[4 * q], words[4 * q + 1], words[4 * q + 2], words[4 * q + 3]};
}

template <typename T, int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_kernel(const T* __restrict__ w, int64_t n_chunks,
                                                       uint32_t* __restrict__ wq,
                                                       T* __restrict__ scales, T* __restrict__ biases) {
  quantize_chunk<T, BITS, GS>(w, n_chunks, wq, scales, biases, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// Several weights of one shape in one launch: blockIdx.y picks the weight.  One launch pays the
// ramp at its start and the partly filled last round of workgroups once for all of them (the
// bench's stream kernel over four config-3 weights: 56.5 us in one launch against 65.1 us in four).
constexpr int kQuantizeBatch = 16;  // weights per launch
template <typename T>
struct QuantizeBatch {
  const T* w[kQuantizeBatch];
  uint32_t* wq[kQuantizeBatch];
  T* s[kQuantizeBatch];
  T* b[kQuantizeBatch];
};

template <typename T, int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_batch_kernel(QuantizeBatch<T> batch, int64_t n_chunks) {
  const int e = blockIdx.y;
  quantize_chunk<T, BITS, GS>(batch.w[e], n_chunks, batch.wq[e], batch.s[e], batch.b[e],
                              (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// wq/scales/biases -> out [N,K] in the scales dtype: out = round(fma(code, scale, bias)).
template <typename T, int BITS, int GS>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint32_t* __restrict__ wq,
                                                         const T* __restrict__ scales,
                                                         const T* __restrict__ biases,
                                                         int64_t n_chunks, T* __restrict__ out) {
  const int64_t chunk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (chunk >= n_chunks) return;
  const int64_t g = (chunk * 8) / GS;
  const float s = SBLoad<T>::ld(scales, g);
  const float b = SBLoad<T>::ld(biases, g);
  float o[8];
  if constexpr (BITS == 4) {
    const uint32_t word = wq[chunk];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = fmaf((float)((word >> (4 * i)) & 0xfu), s, b);
  } else {
    const u32x2 words = *reinterpret_cast<const u32x2*>(wq + chunk * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = fmaf((float)((words[0] >> (8 * i)) & 0xffu), s, b);
      o[4 + i] = fmaf((float)((words[1] >> (8 * i)) & 0xffu), s, b);
    }
  }
  if constexpr (sizeof(T) == 2) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(o[2 * i], o[2 * i + 1]);
    *reinterpret_cast<u32x4*>(out + chunk * 8) = r;
  } else {
    f32x4 a = {o[0], o[1], o[2], o[3]};
    f32x4 c = {o[4], o[5], o[6], o[7]};
    *reinterpret_cast<f32x4*>(out + chunk * 8) = a;
    *reinterpret_cast<f32x4*>(out + chunk * 8 + 4) = c;
  }
}

template <typename T, int BITS, int GS>
static int launch_quantize(const void* w, int64_t N, int64_t K, uint32_t* wq, void* s, void* b,
                           hipStream_t st) {
  const int64_t n_chunks = N * K / 32;  // K % GS == 0 and GS >= 32, so K % 32 == 0
  if (n_chunks == 0) return MLXQ_OK;
  const int64_t blocks = (n_chunks + 255) / 256;
  hipLaunchKernelGGL((quantize_kernel<T, BITS, GS>), dim3((unsigned)blocks), dim3(256), 0, st,
                     (const T*)w, n_chunks, wq, (T*)s, (T*)b);
  return check_launch("quantize");
}

// count weights (1 <= count) in launches of up to kQuantizeBatch.
template <typename T, int BITS, int GS>
static int launch_quantize_batched(const void* const* w, int count, int64_t N, int64_t K, uint32_t* const* wq,
                                   void* const* s, void* const* b, hipStream_t st) {
  const int64_t n_chunks = N * K / 32;
  if (n_chunks == 0) return MLXQ_OK;
  const int64_t blocks = (n_chunks + 255) / 256;
  for (int e0 = 0; e0 < count; e0 += kQuantizeBatch) {
    const int n = count - e0 < kQuantizeBatch ? count - e0 : kQuantizeBatch;
    QuantizeBatch<T> batch = {};
    for (int e = 0; e < n; ++e) {
      batch.w[e] = static_cast<const T*>(w[e0 + e]);
      batch.wq[e] = wq[e0 + e];
      batch.s[e] = static_cast<T*>(s[e0 + e]);
      batch.b[e] = static_cast<T*>(b[e0 + e]);
    }
    hipLaunchKernelGGL((quantize_batch_kernel<T, BITS, GS>), dim3((unsigned)blocks, (unsigned)n), dim3(256), 0, st,
                       batch, n_chunks);
    const int rc = check_launch("quantize_batched");
    if (rc != MLXQ_OK) return rc;
  }
  return MLXQ_OK;
}

template <typename T, int BITS, int GS>
static int launch_dequantize(const uint32_t* wq, const void* s, const void* b, int64_t N, int64_t K,
                             void* out, hipStream_t st) {
  const int64_t n_chunks = N * K / 8;
  if (n_chunks == 0) return MLXQ_OK;
  const int64_t blocks = (n_chunks + 255) / 256;
  hipLaunchKernelGGL((dequantize_kernel<T, BITS, GS>), dim3((unsigned)blocks), dim3(256), 0, st, wq,
                     (const T*)s, (const T*)b, n_chunks, (T*)out);
  return check_launch("dequantize");
}

// Dispatch over (dtype, bits, group_size); arguments were validated by the ABI layer.
int run_quantize(const void* w, int dtype, int64_t N, int64_t K, int gs, int bits, uint32_t* wq,
                 void* s, void* b, hipStream_t st) {
#define MLXQ_Q(T, B, G) \
  if (bits == B && gs == G) return launch_quantize<T, B, G>(w, N, K, wq, s, b, st);
  if (dtype == MLXQ_BFLOAT16) {
    MLXQ_Q(uint16_t, 4, 32) MLXQ_Q(uint16_t, 4, 64) MLXQ_Q(uint16_t, 4, 128)
    MLXQ_Q(uint16_t, 8, 32) MLXQ_Q(uint16_t, 8, 64) MLXQ_Q(uint16_t, 8, 128)
  } else {
    MLXQ_Q(float, 4, 32) MLXQ_Q(float, 4, 64) MLXQ_Q(float, 4, 128)
    MLXQ_Q(float, 8, 32) MLXQ_Q(float, 8, 64) MLXQ_Q(float, 8, 128)
  }
#undef MLXQ_Q
  return set_error(MLXQ_EINVAL, "quantize: unsupported bits=%d group_size=%d", bits, gs);
}

int run_quantize_batched(const void* const* w, int count, int dtype, int64_t N, int64_t K, int gs, int bits,
                         uint32_t* const* wq, void* const* s, void* const* b, hipStream_t st) {
#define MLXQ_Q(T, B, G) \
  if (bits == B && gs == G) return launch_quantize_batched<T, B, G>(w, count, N, K, wq, s, b, st);
  if (dtype == MLXQ_BFLOAT16) {
    MLXQ_Q(uint16_t, 4, 32) MLXQ_Q(uint16_t, 4, 64) MLXQ_Q(uint16_t, 4, 128)
    MLXQ_Q(uint16_t, 8, 32) MLXQ_Q(uint16_t, 8, 64) MLXQ_Q(uint16_t, 8, 128)
  } else {
    MLXQ_Q(float, 4, 32) MLXQ_Q(float, 4, 64) MLXQ_Q(float, 4, 128)
    MLXQ_Q(float, 8, 32) MLXQ_Q(float, 8, 64) MLXQ_Q(float, 8, 128)
  }
#undef MLXQ_Q
  return set_error(MLXQ_EINVAL, "quantize_batched: unsupported bits=%d group_size=%d", bits, gs);
}

int run_dequantize(const uint32_t* wq, const void* s, const void* b, int dtype, int64_t N, int64_t K,
                   int gs, int bits, void* out, hipStream_t st) {
#define MLXQ_D(T, B, G) \
  if (bits == B && gs == G) return launch_dequantize<T, B, G>(wq, s, b, N, K, out, st);
  if (dtype == MLXQ_BFLOAT16) {
    MLXQ_D(uint16_t, 4, 32) MLXQ_D(uint16_t, 4, 64) MLXQ_D(uint16_t, 4, 128)
    MLXQ_D(uint16_t, 8, 32) MLXQ_D(uint16_t, 8, 64) MLXQ_D(uint16_t, 8, 128)
  } else {
    MLXQ_D(float, 4, 32) MLXQ_D(float, 4, 64) MLXQ_D(float, 4, 128)
    MLXQ_D(float, 8, 32) MLXQ_D(float, 8, 64) MLXQ_D(float, 8, 128)
  }
#undef MLXQ_D
  return set_error(MLXQ_EINVAL, "dequantize: unsupported bits=%d group_size=%d", bits, gs);
}

}  // namespace mlxq
