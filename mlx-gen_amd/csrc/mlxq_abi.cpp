// mlxq_abi.cpp — the extern "C" boundary of libmlxq_hip.so: argument validation, kernel
// dispatch and the thread-local error string.  No entry point aborts; every failure returns an
// mlxq_status and leaves a message for mlxq_last_error().
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "mlxq_common.h"

namespace mlxq {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MLXQ_EDEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MLXQ_OK;
}

static int check_pack(const char* op, int64_t N, int64_t K, int gs, int bits) {
  if (bits != 4 && bits != 8)
    return set_error(MLXQ_EINVAL, "%s: bits must be 4 or 8 (got %d)", op, bits);
  if (gs != 32 && gs != 64 && gs != 128)
    return set_error(MLXQ_EINVAL, "%s: group_size must be 32, 64 or 128 (got %d)", op, gs);
  if (N < 0 || K <= 0)
    return set_error(MLXQ_EINVAL, "%s: bad shape N=%lld K=%lld", op, (long long)N, (long long)K);
  if (K % gs != 0)
    return set_error(MLXQ_EINVAL, "%s: K=%lld is not a multiple of group_size=%d", op, (long long)K, gs);
  return MLXQ_OK;
}

static int check_dtype(const char* op, const char* what, int dt) {
  if (dt != MLXQ_FLOAT32 && dt != MLXQ_BFLOAT16)
    return set_error(MLXQ_EINVAL, "%s: %s dtype %d is not float32 or bfloat16", op, what, dt);
  return MLXQ_OK;
}

static int check_aligned(const char* op, const char* what, const void* p, uintptr_t align = 16) {
  if (p == nullptr) return set_error(MLXQ_EINVAL, "%s: %s is null", op, what);
  if (reinterpret_cast<uintptr_t>(p) % align != 0)
    return set_error(MLXQ_EINVAL, "%s: %s must be %d-byte aligned", op, what, (int)align);
  return MLXQ_OK;
}

static int check_mm(const char* op, const void* x, int x_dtype, int64_t M, int64_t K,
                    const uint32_t* wq, const void* s, const void* b, int sb_dtype, int64_t N,
                    int gs, int bits, const void* y) {
  int rc;
  if ((rc = check_pack(op, N, K, gs, bits))) return rc;
  if (M < 0) return set_error(MLXQ_EINVAL, "%s: M=%lld < 0", op, (long long)M);
  if ((rc = check_dtype(op, "x", x_dtype)) || (rc = check_dtype(op, "scales", sb_dtype))) return rc;
  if (M == 0 || N == 0) return MLXQ_OK;
  if ((rc = check_aligned(op, "x", x)) || (rc = check_aligned(op, "wq", wq)) ||
      (rc = check_aligned(op, "y", y)))
    return rc;
  // scales/biases are read as whole dwords (16-byte chunks in the GEMV)
  if ((rc = check_aligned(op, "scales", s, 4)) || (rc = check_aligned(op, "biases", b, 4))) return rc;
  return MLXQ_OK;
}

static const QmmEpilogue kNoEpilogue = {nullptr, nullptr, nullptr, 0, 1.0f, MLXQ_ACT_NONE};

static inline int64_t round16(int64_t r) { return (r + 15) / 16 * 16; }

}  // namespace mlxq

using namespace mlxq;

extern "C" {

const char* mlxq_last_error(void) { return g_err; }

const char* mlxq_version(void) { return "mlxq-hip 0.1 (gfx950)"; }

int mlxq_packed_bits(int64_t wq_cols, int64_t scales_cols, int group_size) {
  g_err[0] = 0;
  if (group_size <= 0 || scales_cols <= 0 || wq_cols <= 0) {
    set_error(MLXQ_EINVAL, "packed_bits: malformed triple (wq cols %lld, scales cols %lld, gs %d)",
              (long long)wq_cols, (long long)scales_cols, group_size);
    return -1;
  }
  const int64_t in_dim = scales_cols * group_size;
  if ((wq_cols * 32) % in_dim != 0) {
    set_error(MLXQ_EINVAL, "packed_bits: wq cols %lld do not pack %lld inputs", (long long)wq_cols,
              (long long)in_dim);
    return -1;
  }
  const int64_t bits = wq_cols * 32 / in_dim;
  if (bits != 4 && bits != 8) {
    set_error(MLXQ_EINVAL, "packed_bits: inferred bits=%lld is not 4 or 8", (long long)bits);
    return -1;
  }
  return (int)bits;
}

int mlxq_quantize(const void* w, int w_dtype, int64_t N, int64_t K, int group_size, int bits,
                  uint32_t* wq, void* scales, void* biases, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_pack("quantize", N, K, group_size, bits))) return rc;
  if ((rc = check_dtype("quantize", "w", w_dtype))) return rc;
  if (N == 0) return MLXQ_OK;
  if ((rc = check_aligned("quantize", "w", w)) || (rc = check_aligned("quantize", "wq", wq))) return rc;
  if (!scales || !biases) return set_error(MLXQ_EINVAL, "quantize: scales/biases are null");
  return run_quantize(w, w_dtype, N, K, group_size, bits, wq, scales, biases, (hipStream_t)stream);
}

int mlxq_dequantize(const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                    int64_t N, int64_t K, int group_size, int bits, void* out, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_pack("dequantize", N, K, group_size, bits))) return rc;
  if ((rc = check_dtype("dequantize", "scales", sb_dtype))) return rc;
  if (N == 0) return MLXQ_OK;
  if ((rc = check_aligned("dequantize", "wq", wq)) || (rc = check_aligned("dequantize", "out", out)))
    return rc;
  if (!scales || !biases) return set_error(MLXQ_EINVAL, "dequantize: scales/biases are null");
  return run_dequantize(wq, scales, biases, sb_dtype, N, K, group_size, bits, out, (hipStream_t)stream);
}

int mlxq_embedding(const int32_t* ids, int64_t T, const uint32_t* wq, const void* scales,
                   const void* biases, int sb_dtype, int64_t vocab, int64_t hidden, int group_size,
                   int bits, void* out, int out_dtype, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_pack("embedding", vocab, hidden, group_size, bits))) return rc;
  if ((rc = check_dtype("embedding", "scales", sb_dtype)) || (rc = check_dtype("embedding", "out", out_dtype)))
    return rc;
  if (T < 0) return set_error(MLXQ_EINVAL, "embedding: T=%lld < 0", (long long)T);
  if (T == 0 || hidden == 0) return MLXQ_OK;
  if (vocab == 0) return set_error(MLXQ_EINVAL, "embedding: empty table");
  if ((rc = check_aligned("embedding", "ids", ids, 4)) || (rc = check_aligned("embedding", "wq", wq)) ||
      (rc = check_aligned("embedding", "scales", scales, 4)) ||
      (rc = check_aligned("embedding", "biases", biases, 4)) || (rc = check_aligned("embedding", "out", out)))
    return rc;
  return run_embedding(ids, T, wq, scales, biases, sb_dtype, vocab, hidden, group_size, bits, out,
                       out_dtype, (hipStream_t)stream);
}

int mlxq_qmm(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
             const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
             int bits, void* y, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_mm("qmm", x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y)))
    return rc;
  if (x_dtype != MLXQ_BFLOAT16) return set_error(MLXQ_EINVAL, "qmm: the MFMA GEMM takes bfloat16 x");
  if (M == 0 || N == 0) return MLXQ_OK;
  return run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, kNoEpilogue,
                 (hipStream_t)stream);
}

int mlxq_qmv(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
             const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
             int bits, void* y, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_mm("qmv", x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y)))
    return rc;
  if (M > 8) return set_error(MLXQ_EINVAL, "qmv: M=%lld exceeds the GEMV limit of 8", (long long)M);
  if (M == 0 || N == 0) return MLXQ_OK;
  return run_qmv(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y,
                 (hipStream_t)stream);
}

int mlxq_quantized_matmul(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
                          const void* scales, const void* biases, int sb_dtype, int64_t N,
                          int transpose, int group_size, int bits, void* y, void* stream) {
  g_err[0] = 0;
  int rc;
  if (!transpose)
    return set_error(MLXQ_EUNSUPPORTED, "quantized_matmul: transpose=false is not implemented");
  if ((rc = check_mm("quantized_matmul", x, x_dtype, M, K, wq, scales, biases, sb_dtype, N,
                     group_size, bits, y)))
    return rc;
  if (M == 0 || N == 0) return MLXQ_OK;
  if (x_dtype == MLXQ_BFLOAT16 && M > 8)
    return run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, kNoEpilogue,
                   (hipStream_t)stream);
  return run_qmv(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y,
                 (hipStream_t)stream);
}

size_t mlxq_linear_workspace_size(int64_t M, int64_t N, int64_t lora_rank) {
  if (lora_rank <= 0 || M <= 0 || N <= 0) return 0;
  const int64_t R = round16(lora_rank);
  // xa [M,R] and lbt [N,R], 4 bytes per element (enough for f32 activations), 256-B aligned.
  const int64_t xa = (M * R * 4 + 255) / 256 * 256;
  return (size_t)(xa + N * R * 4);
}

int mlxq_swiglu(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq_gate,
                const void* scales_gate, const void* biases_gate, const uint32_t* wq_up,
                const void* scales_up, const void* biases_up, int sb_dtype, int64_t F,
                int group_size, int bits, void* h, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_mm("swiglu", x, x_dtype, M, K, wq_gate, scales_gate, biases_gate, sb_dtype, F,
                     group_size, bits, h)))
    return rc;
  if (M == 0 || F == 0) return MLXQ_OK;
  if ((rc = check_aligned("swiglu", "wq_up", wq_up)) || (rc = check_aligned("swiglu", "scales_up", scales_up, 4)) ||
      (rc = check_aligned("swiglu", "biases_up", biases_up, 4)))
    return rc;
  if (!swiglu_qmv_applicable(x_dtype, sb_dtype, M, K, F, group_size, bits))
    return set_error(MLXQ_EUNSUPPORTED,
                     "swiglu: the fused decode form takes bf16 x and scales, 1 <= M <= 8, group_size "
                     "64 or 128 and K a multiple of %d (got M=%lld K=%lld)", 512 / bits, (long long)M,
                     (long long)K);
  return run_swiglu_qmv(x, M, K, wq_gate, scales_gate, biases_gate, wq_up, scales_up, biases_up, F,
                        group_size, bits, h, (hipStream_t)stream);
}

int mlxq_lora_residual(const void* x, int x_dtype, int64_t M, int64_t K, const void* lora_a,
                       const void* lora_b, int64_t N, int64_t rank, float lora_scale, void* y,
                       void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_dtype("lora_residual", "x", x_dtype))) return rc;
  if (M < 0 || K <= 0 || N < 0) return set_error(MLXQ_EINVAL, "lora_residual: bad shape M=%lld K=%lld N=%lld",
                                                  (long long)M, (long long)K, (long long)N);
  if (rank < 1 || rank > 256)
    return set_error(MLXQ_EINVAL, "lora_residual: rank %lld outside [1, 256]", (long long)rank);
  if (M == 0 || N == 0) return MLXQ_OK;
  if (!x || !lora_a || !lora_b || !y) return set_error(MLXQ_EINVAL, "lora_residual: null operand");
  const size_t need = mlxq_linear_workspace_size(M, N, rank);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(MLXQ_EINVAL, "lora_residual: workspace of %zu bytes is smaller than the %zu required",
                     workspace_bytes, need);
  if ((rc = check_aligned("lora_residual", "workspace", workspace))) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int R = (int)round16(rank);
  void* xa = workspace;
  void* lbt = (char*)workspace + (M * R * 4 + 255) / 256 * 256;
  if ((rc = run_lora_prep(x, x_dtype, M, K, lora_a, lora_b, N, (int)rank, R, xa, lbt, st))) return rc;
  float scale = lora_scale;
  if (x_dtype == MLXQ_BFLOAT16) {
    uint32_t u;
    memcpy(&u, &scale, 4);
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    memcpy(&scale, &u, 4);
  }
  return run_linear_epilogue(y, x_dtype, M, N, nullptr, xa, lbt, R, scale, MLXQ_ACT_NONE, st);
}

int mlxq_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_dtype("cast", "src", src_dtype)) || (rc = check_dtype("cast", "dst", dst_dtype))) return rc;
  if (n < 0) return set_error(MLXQ_EINVAL, "cast: n=%lld < 0", (long long)n);
  if (n == 0) return MLXQ_OK;
  if ((rc = check_aligned("cast", "src", src, 4)) || (rc = check_aligned("cast", "dst", dst, 4))) return rc;
  return run_cast(src, src_dtype, dst, dst_dtype, n, (hipStream_t)stream);
}

int mlxq_qmm_experts(const void* x, int x_dtype, int x_per_expert, int64_t E, int64_t M, int64_t K,
                     const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                     const void* bias, int64_t N, int group_size, int bits, void* y, void* stream) {
  g_err[0] = 0;
  int rc;
  if (E < 0) return set_error(MLXQ_EINVAL, "qmm_experts: E=%lld < 0", (long long)E);
  if ((rc = check_mm("qmm_experts", x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size,
                     bits, y)))
    return rc;
  if (E == 0 || M == 0 || N == 0) return MLXQ_OK;
  const int xb = x_dtype == MLXQ_BFLOAT16 ? 2 : 4;
  const int sbb = sb_dtype == MLXQ_BFLOAT16 ? 2 : 4;
  if (bias && (rc = check_aligned("qmm_experts", "bias", bias, xb))) return rc;
  QmmBatch bat;
  bat.count = E;
  bat.x = x_per_expert ? M * K : 0;
  bat.w = N * (K * bits / 32);
  bat.sb = N * (K / group_size);
  bat.y = M * N;
  bat.bias = N;
  hipStream_t st = (hipStream_t)stream;
  // All experts in one launch of the wide GEMM (grid.y = expert) when it applies: per-expert
  // problems of an encoder batch are a few dozen tiles each, too few to fill 256 CUs alone.
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  if (x_dtype == MLXQ_BFLOAT16 && M > 8 && K % 64 == 0 && E * tiles >= 128 && E <= 65535 &&
      qmm_wide_fits(M, K, N, group_size, bits, sbb)) {
    const QmmEpilogue qe = {(const uint16_t*)bias, nullptr, nullptr, 0, 1.0f, MLXQ_ACT_NONE};
    return run_qmm_wide(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, qe, st, bat);
  }
  // Otherwise expert by expert through the single-matrix paths (same rounding points).
  for (int64_t e = 0; e < E; ++e) {
    const mlxq_epilogue ep = {bias ? (const char*)bias + e * bat.bias * xb : nullptr, nullptr, nullptr,
                              0, 1.0f, MLXQ_ACT_NONE};
    if ((rc = mlxq_linear((const char*)x + e * bat.x * xb, x_dtype, M, K, wq + e * bat.w,
                          (const char*)scales + e * bat.sb * sbb, (const char*)biases + e * bat.sb * sbb,
                          sb_dtype, N, group_size, bits, &ep, (char*)y + e * bat.y * xb, nullptr, 0,
                          stream)))
      return rc;
  }
  return MLXQ_OK;
}

int mlxq_linear(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
                const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
                int bits, const mlxq_epilogue* ep, void* y, void* workspace, size_t workspace_bytes,
                void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_mm("linear", x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y)))
    return rc;
  if (M == 0 || N == 0) return MLXQ_OK;
  hipStream_t st = (hipStream_t)stream;
  mlxq_epilogue none = {nullptr, nullptr, nullptr, 0, 1.0f, MLXQ_ACT_NONE};
  const mlxq_epilogue& e = ep ? *ep : none;
  if (e.activation != MLXQ_ACT_NONE && e.activation != MLXQ_ACT_GELU &&
      e.activation != MLXQ_ACT_GELU_TANH)
    return set_error(MLXQ_EINVAL, "linear: unknown activation %d", e.activation);
  if (e.lora_rank < 0 || e.lora_rank > 256)
    return set_error(MLXQ_EINVAL, "linear: lora_rank %lld outside [0, 256]", (long long)e.lora_rank);
  const bool lora = e.lora_rank > 0;
  const int R = lora ? (int)round16(e.lora_rank) : 0;
  void* xa = nullptr;
  void* lbt = nullptr;
  if (lora) {
    if (!e.lora_a || !e.lora_b) return set_error(MLXQ_EINVAL, "linear: lora_rank > 0 but A/B are null");
    const size_t need = mlxq_linear_workspace_size(M, N, e.lora_rank);
    if (workspace == nullptr || workspace_bytes < need)
      return set_error(MLXQ_EINVAL, "linear: workspace of %zu bytes is smaller than the %zu required",
                       workspace_bytes, need);
    if ((rc = check_aligned("linear", "workspace", workspace))) return rc;
    xa = workspace;
    lbt = (char*)workspace + (M * R * 4 + 255) / 256 * 256;
    if ((rc = run_lora_prep(x, x_dtype, M, K, e.lora_a, e.lora_b, N, (int)e.lora_rank, R, xa, lbt, st)))
      return rc;
  }
  // The lora scale is applied as a scalar of the activation dtype (src/adapters.rs:268-269).
  float scale = e.lora_scale;
  if (x_dtype == MLXQ_BFLOAT16) {
    uint32_t u;
    memcpy(&u, &scale, 4);
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    memcpy(&scale, &u, 4);
  }
  if (x_dtype == MLXQ_BFLOAT16 && M > 8) {
    // The GEMM fuses the whole epilogue for LoRA rank <= 16; a wider adapter runs the plain
    // GEMM followed by the elementwise epilogue (same rounding points).
    if (R <= 16) {
      QmmEpilogue qe = {(const uint16_t*)e.bias, (const uint16_t*)xa, (const uint16_t*)lbt, R,
                        scale, e.activation};
      return run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, qe, st);
    }
    if ((rc = run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, kNoEpilogue, st)))
      return rc;
    return run_linear_epilogue(y, x_dtype, M, N, e.bias, xa, lbt, R, scale, e.activation, st);
  }
  if ((rc = run_qmv(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, st)))
    return rc;
  if (!e.bias && !lora && e.activation == MLXQ_ACT_NONE) return MLXQ_OK;
  return run_linear_epilogue(y, x_dtype, M, N, e.bias, xa, lbt, R, scale, e.activation, st);
}

}  // extern "C"
