// embedding.hip — quantized token-embedding lookup for gfx950.
//
// TokenEmbedding::forward's quantized arm (reference src/nn.rs:42-58) gathers the packed rows of
// the token ids, dequantizes them (MLX dequantize: fma(code, scale, bias) in f32, rounded once to
// the scales dtype) and casts the result to f32.  Here that is one pass: each thread produces 8
// consecutive outputs of one token row from one packed word (Q4) or two (Q8) and writes them as
// 16- or 32-byte stores; the gathered packed rows never exist as a separate tensor.
// Ids outside [0, vocab) produce a row of NaN (the reference's gather leaves that case undefined).
#include "mlxq_common.h"

namespace mlxq {

template <typename SB, typename OT, int BITS, int GS>
__global__ __launch_bounds__(256) void embedding_kernel(const int32_t* __restrict__ ids, int64_t T,
                                                        const uint32_t* __restrict__ wq,
                                                        const SB* __restrict__ scales,
                                                        const SB* __restrict__ biases,
                                                        int64_t vocab, int64_t hidden,
                                                        OT* __restrict__ out) {
  const int64_t cpr = hidden / 8;  // 8-value chunks per row
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= T * cpr) return;
  const int64_t t = idx / cpr, c = idx - t * cpr;
  const int64_t row = ids[t];
  float o[8];
  if (row < 0 || row >= vocab) {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = __builtin_nanf("");
  } else {
    const int64_t groups = hidden / GS;
    const int64_t g = row * groups + (c * 8) / GS;
    const float s = SBLoad<SB>::ld(scales, g);
    const float b = SBLoad<SB>::ld(biases, g);
    const uint32_t* w = wq + row * (hidden * BITS / 32);
    if constexpr (BITS == 4) {
      const uint32_t word = w[c];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = SBLoad<SB>::rnd(fmaf((float)((word >> (4 * i)) & 0xfu), s, b));
    } else {
      const u32x2 words = *reinterpret_cast<const u32x2*>(w + c * 2);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = SBLoad<SB>::rnd(fmaf((float)((words[0] >> (8 * i)) & 0xffu), s, b));
        o[4 + i] = SBLoad<SB>::rnd(fmaf((float)((words[1] >> (8 * i)) & 0xffu), s, b));
      }
    }
  }
  OT* dst = out + t * hidden + c * 8;
  if constexpr (sizeof(OT) == 2) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(o[2 * i], o[2 * i + 1]);
    *reinterpret_cast<u32x4*>(dst) = r;
  } else {
    *reinterpret_cast<f32x4*>(dst) = f32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
  }
}

template <typename SB, typename OT, int BITS, int GS>
static int launch_embedding(const int32_t* ids, int64_t T, const uint32_t* wq, const void* s,
                            const void* b, int64_t vocab, int64_t hidden, void* out, hipStream_t st) {
  const int64_t n = T * (hidden / 8);
  if (n == 0) return MLXQ_OK;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return set_error(MLXQ_EINVAL, "embedding: problem too large");
  hipLaunchKernelGGL((embedding_kernel<SB, OT, BITS, GS>), dim3((unsigned)blocks), dim3(256), 0, st,
                     ids, T, wq, (const SB*)s, (const SB*)b, vocab, hidden, (OT*)out);
  return check_launch("embedding");
}

template <typename SB, typename OT>
static int embedding_bits_gs(const int32_t* ids, int64_t T, const uint32_t* wq, const void* s,
                             const void* b, int64_t vocab, int64_t hidden, int gs, int bits,
                             void* out, hipStream_t st) {
#define MLXQ_E(B, G) \
  if (bits == B && gs == G) return launch_embedding<SB, OT, B, G>(ids, T, wq, s, b, vocab, hidden, out, st);
  MLXQ_E(4, 32) MLXQ_E(4, 64) MLXQ_E(4, 128) MLXQ_E(8, 32) MLXQ_E(8, 64) MLXQ_E(8, 128)
#undef MLXQ_E
  return set_error(MLXQ_EINVAL, "embedding: unsupported bits=%d group_size=%d", bits, gs);
}

int run_embedding(const int32_t* ids, int64_t T, const uint32_t* wq, const void* s, const void* b,
                  int sb_dtype, int64_t vocab, int64_t hidden, int gs, int bits, void* out,
                  int out_dtype, hipStream_t st) {
  if (sb_dtype == MLXQ_BFLOAT16) {
    if (out_dtype == MLXQ_BFLOAT16)
      return embedding_bits_gs<uint16_t, uint16_t>(ids, T, wq, s, b, vocab, hidden, gs, bits, out, st);
    return embedding_bits_gs<uint16_t, float>(ids, T, wq, s, b, vocab, hidden, gs, bits, out, st);
  }
  if (out_dtype == MLXQ_BFLOAT16)
    return embedding_bits_gs<float, uint16_t>(ids, T, wq, s, b, vocab, hidden, gs, bits, out, st);
  return embedding_bits_gs<float, float>(ids, T, wq, s, b, vocab, hidden, gs, bits, out, st);
}

}  // namespace mlxq
