// mlxq_common.h — shared device helpers for the gfx950 quantized-linear kernels.
//
// Storage conventions (identical to MLX's affine packing, which the reference consumes through
// mlx_rs::ops::{quantize, dequantize, quantized_matmul}):
//   * W [N, K] is packed row-major into uint32 words, 32/bits codes per word, element i of a word
//     at bit offset i*bits (low bits first); a row holds K*bits/32 words.
//   * scales / biases are [N, K/group_size] in the weight dtype (bf16 or f32).
//   * bf16 travels as raw uint16 bits; conversions below are round-to-nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mlxq.h"
#include "mlxq_internal.h"

namespace mlxq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Two f32 -> packed bf16 pair (lo in bits 0..15), RNE; lowers to v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return (uint16_t)(pack_bf16x2(f, 0.0f) & 0xffffu);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Rounds a and b to bf16 (RNE) in place with one conversion for both.
__device__ __forceinline__ void round_bf16x2(float& a, float& b) {
  const uint32_t w = pack_bf16x2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

// The fused bias / LoRA epilogue on two outputs, rounded to bf16 after each op as the
// reference's separate ops round: o = rnd(rnd(rnd(acc) + bias) + rnd(rnd(r) * scale)); with
// scale == 1 the product's rounding is the identity and is skipped.  Each term (HB bias, HL LoRA,
// HS LoRA scale != 1) is either fixed at compile time (kTermOff / kTermOn) or read from its
// runtime flag (kTermRuntime): epilogues that choose the combination once per tile avoid the
// three uniform branches per output pair that runtime flags cost.
enum : int { kTermOff = 0, kTermOn = 1, kTermRuntime = 2 };
template <int HB, int HL, int HS>
__device__ __forceinline__ void epilogue_terms2(float& o0, float& o1, bool has_bias, float b0, float b1,
                                                bool lora, float r0, float r1, float scale) {
  round_bf16x2(o0, o1);
  if (HB == kTermOn || (HB == kTermRuntime && has_bias)) {
    o0 += b0;
    o1 += b1;
    round_bf16x2(o0, o1);
  }
  if (HL == kTermOn || (HL == kTermRuntime && lora)) {
    round_bf16x2(r0, r1);
    if (HS == kTermOn || (HS == kTermRuntime && scale != 1.0f)) {
      r0 *= scale;
      r1 *= scale;
      round_bf16x2(r0, r1);
    }
    o0 += r0;
    o1 += r1;
    round_bf16x2(o0, o1);
  }
}

// LDS row swizzle of 16-byte chunks for 128-byte activation rows: chunk c of row r is stored at
// position c ^ swz_f(r), which keeps the MFMA fragment reads (32 rows, one chunk each) spread
// over all banks.
__device__ __forceinline__ int swz_f(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Wait until at most N vector memory operations of this wave are outstanding, leaving the LDS and
// export counters open (gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void mlxq_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Scale/bias element loaders for the two supported storage dtypes.
template <typename SB>
struct SBLoad;
template <>
struct SBLoad<uint16_t> {
  static __device__ __forceinline__ float ld(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ void st(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
  static __device__ __forceinline__ float rnd(float v) { return round_bf16(v); }
};
template <>
struct SBLoad<float> {
  static __device__ __forceinline__ float ld(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void st(float* p, int64_t i, float v) { p[i] = v; }
  static __device__ __forceinline__ float rnd(float v) { return v; }
};

// Activation element access: bf16 (uint16 bits) or f32.
template <typename T>
struct Act;
template <>
struct Act<uint16_t> {
  static __device__ __forceinline__ float ld(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ void st(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
  static __device__ __forceinline__ float rnd(float v) { return round_bf16(v); }
};
template <>
struct Act<float> {
  static __device__ __forceinline__ float ld(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void st(float* p, int64_t i, float v) { p[i] = v; }
  static __device__ __forceinline__ float rnd(float v) { return v; }
};
// fp16 activations (MLXQ_FLOAT16): widened exactly to f32.  MLX promotes fp16 against bf16 or f32
// operands to f32, so every product with fp16 x is an f32 product.
template <>
struct Act<_Float16> {
  static __device__ __forceinline__ float ld(const _Float16* p, int64_t i) { return (float)p[i]; }
  static __device__ __forceinline__ void st(_Float16* p, int64_t i, float v) { p[i] = (_Float16)v; }
  static __device__ __forceinline__ float rnd(float v) { return (float)(_Float16)v; }
};

// The two fp16 values of a 32-bit word (element 0 in the low half), widened exactly to f32.
__device__ __forceinline__ float f16_lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

// Exact-erf GELU, 0.5*v*(1+erf(v/sqrt(2))), branch-free so it can run on values held in the
// MFMA accumulators without forcing them out of registers.  With z = |v|/sqrt(2):
//   v >= 0:  0.5*v*(2 - erfc(z)),   v < 0:  0.5*v*erfc(z),
// where erfc(z) = t*exp(-z^2 + P(t)), t = 1/(1 + z/2), P the degree-9 Chebyshev-fitted
// polynomial of Press et al., Numerical Recipes 2nd ed. sec. 6.2 ("erfcc"; fractional error
// below 1.2e-7 for all z >= 0).  Evaluated with the hardware reciprocal and exp2.
__device__ __forceinline__ float gelu_erf(float v) {
  const float z = fabsf(v) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(p, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  p = fmaf(p, t, -1.26551223f);
  const float e = fmaf(-z, z, p);
  const float erfc_z = t * __builtin_amdgcn_exp2f(e * 1.44269504088896341f);
  const float g = v >= 0.0f ? 2.0f - erfc_z : erfc_z;
  return 0.5f * v * g;
}

// tanh from the hardware exp2 and reciprocal: tanh|z| = 1 - 2 / (exp(2|z|) + 1), sign restored.
// Absolute error a few 1e-7 (the GELU below adds it to 1, so relative accuracy near 0 is not
// needed); exp2 overflows to +inf for |z| > 44 and the reciprocal then gives exactly 1.  Kept
// small on purpose: the fused GEMM epilogue inlines it, and the library tanhf made that epilogue
// large enough to push the accumulator tile out of registers.
__device__ __forceinline__ float tanh_hw(float z) {
  const float e = __builtin_amdgcn_exp2f(fabsf(z) * 2.88539008177792681f);  // 2 / ln 2
  const float t = fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
  return copysignf(t, z);
}

// Tanh-approximate GELU, 0.5 x (1 + tanh(c (x + 0.044715 x^3))) with c = sqrt(2/pi), evaluated
// as the separate ops of reference src/nn.rs:321-329: every op rounded to the activation dtype
// (bf16 when BF16, else f32) and the constants cast to it first.  x^3 of a bf16 value is exact in
// f32 (24 significant bits), so rounding the f32 cube once is the rounded power.
template <bool BF16>
__device__ __forceinline__ float gelu_tanh(float x) {
  auto rnd = [](float v) { return BF16 ? round_bf16(v) : v; };
  const float c = rnd(0.7978845608028654f);
  const float k = rnd(0.044715f);
  const float x3 = rnd(x * x * x);
  const float inner = rnd(rnd(x + rnd(x3 * k)) * c);
  const float gate = rnd(rnd(tanh_hw(inner)) + 1.0f);
  return rnd(rnd(x * 0.5f) * gate);
}

// bf16 SiLU as the reference's two ops, multiply(x, sigmoid(x)) (src/nn.rs:301-303): the sigmoid
// rounded to bf16, then the product (exact in f32: two 8-bit significands) rounded to bf16.  g is
// a bf16 value.  The f32 sigmoid is the correctly rounded one: 1 / (1 + expf(-g)) is within ~2 ulp
// of it, so only where that lands within 8 ulp of a bf16 rounding midpoint (low 16 bits near
// 0x8000), or below the f32 normal range (expf overflows for g < -88.7), is it recomputed in
// double.  Every bf16 input then rounds as the correctly rounded f32 sigmoid does.
__device__ __forceinline__ float silu_bf16(float g) {
  float s = 1.0f / (1.0f + expf(-g));
  const uint32_t lo = __float_as_uint(s) & 0xffffu;
  if (lo - 0x7ff8u < 0x10u || s < 1.17549435e-38f) s = (float)(1.0 / (1.0 + exp(-(double)g)));
  return round_bf16(g * round_bf16(s));
}

// ---- MFMA GEMM weight dequantization (shared by the GEMM kernels)
// v_cvt_f32_ubyteN: byte N of v as an exact f32.
template <int B>
__device__ __forceinline__ float ubyte(uint32_t v) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  if constexpr (B == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// Dequantize 8 codes into a bf16x8 MFMA operand: word kk of w (Q4, codes 0..7) or words 2kk,
// 2kk+1 (Q8), each value bf16(fma(code, s, z)).
// Q4: the even codes are the bytes of w & 0x0f0f0f0f, the odd ones the bytes of
// (w >> 4) & 0x0f0f0f0f.  A byte c in 0..15 read as an OCP fp8 E4M3 value is exactly c * 2^-9
// (mantissa c * 2^-9 below 8, exponent field 1 from 8 on), so v_cvt_scalef32_pk_f32_fp8 with
// scale 2^9 turns two codes into exact f32 values in one instruction: 19 VALU ops per 8 codes
// (3 extract, 4 convert, 8 FMA, 4 pack) where one v_cvt_f32_ubyteN per code took 22.
template <int BITS>
__device__ __forceinline__ bf16x8 dequant8(const uint32_t* w, int kk, float s, float z) {
  u32x4 o;
  if constexpr (BITS == 4) {
    const uint32_t v = w[kk];
    const uint32_t ev = v & 0x0f0f0f0fu, od = (v >> 4) & 0x0f0f0f0fu;
    const f32x2 e01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ev, 512.0f, false);  // codes 0, 2
    const f32x2 e23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ev, 512.0f, true);   // codes 4, 6
    const f32x2 o01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(od, 512.0f, false);  // codes 1, 3
    const f32x2 o23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(od, 512.0f, true);   // codes 5, 7
    o[0] = pack_bf16x2(fmaf(e01[0], s, z), fmaf(o01[0], s, z));
    o[1] = pack_bf16x2(fmaf(e01[1], s, z), fmaf(o01[1], s, z));
    o[2] = pack_bf16x2(fmaf(e23[0], s, z), fmaf(o23[0], s, z));
    o[3] = pack_bf16x2(fmaf(e23[1], s, z), fmaf(o23[1], s, z));
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

// Scale/bias element as raw bits, converted with sb_to_f32 when used: a conversion right after
// the load would make the caller wait for it there.
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

}  // namespace mlxq
