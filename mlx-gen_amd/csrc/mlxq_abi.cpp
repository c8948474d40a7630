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

// Storage dtypes: f32 and bf16 for every operand; fp16 only as the activations x of the entry
// points that take it (check_x_dtype), MLXQ_EUNSUPPORTED elsewhere.
static int check_dtype(const char* op, const char* what, int dt) {
  if (dt == MLXQ_FLOAT16)
    return set_error(MLXQ_EUNSUPPORTED, "%s: %s dtype float16 is not supported (float16 is taken as "
                                        "activations only)", op, what);
  if (dt != MLXQ_FLOAT32 && dt != MLXQ_BFLOAT16)
    return set_error(MLXQ_EINVAL, "%s: %s dtype %d is not float32, bfloat16 or float16", op, what, dt);
  return MLXQ_OK;
}

static int check_x_dtype(const char* op, int dt) {
  return dt == MLXQ_FLOAT16 ? MLXQ_OK : check_dtype(op, "x", dt);
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
  if ((rc = check_x_dtype(op, x_dtype)) || (rc = check_dtype(op, "scales", sb_dtype))) return rc;
  if (M == 0 || N == 0) return MLXQ_OK;
  if ((rc = check_aligned(op, "x", x)) || (rc = check_aligned(op, "wq", wq)) ||
      (rc = check_aligned(op, "y", y)))
    return rc;
  // scales/biases are read as whole dwords (16-byte chunks in the GEMV)
  if ((rc = check_aligned(op, "scales", s, 4)) || (rc = check_aligned(op, "biases", b, 4))) return rc;
  return MLXQ_OK;
}

static const QmmEpilogue kNoEpilogue = {nullptr, nullptr, nullptr, 0, 1.0f, kFusedActNone, nullptr};

static inline int64_t round16(int64_t r) { return (r + 15) / 16 * 16; }
static inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// A scalar cast to bf16 (round to nearest even), as scalar(v).as_dtype(Bfloat16) does.
static float bf16_scalar(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  memcpy(&v, &u, 4);
  return v;
}

// The dtype of every stage of mlxq_linear under MLX's promotion (bf16 iff every operand that
// meets there is bf16), from the reference op sequence of src/adapters.rs:243-252,300-322,543-549.
struct LinearPlan {
  bool d0_bf16 = true;   // qmm(x): promote(x, scales)
  bool bias = false, d1_bf16 = true;  // + bias: promote(D0, bias)
  bool lora = false, dr_bf16 = true;  // residual: promote(x, factors)
  bool d2_bf16 = true;   // + residual: promote(D1, DR)
  int act = MLXQ_ACT_NONE;
  bool out_bf16 = true;  // GELU (mlx_rs::nn::gelu) returns f32
  int R = 0;             // padded LoRA rank
  // Workspace layout (byte offsets), total bytes.
  size_t xa = 0, lbt = 0, y0 = 0, total = 0;
  bool promoted() const { return d0_bf16 && !out_bf16; }  // bf16 product, f32 result
};

static int plan_linear(const char* op, int x_dtype, int sb_dtype, const mlxq_epilogue* ep,
                       int64_t M, int64_t N, LinearPlan& p) {
  int rc;
  if ((rc = check_x_dtype(op, x_dtype)) || (rc = check_dtype(op, "scales", sb_dtype))) return rc;
  p = LinearPlan{};
  p.d0_bf16 = x_dtype == MLXQ_BFLOAT16 && sb_dtype == MLXQ_BFLOAT16;
  if (ep) {
    if (ep->activation < MLXQ_ACT_NONE || ep->activation > MLXQ_ACT_GELU_EXACT)
      return set_error(MLXQ_EINVAL, "%s: unknown activation %d", op, ep->activation);
    if (ep->lora_rank < 0 || ep->lora_rank > 256)
      return set_error(MLXQ_EINVAL, "%s: lora_rank %lld outside [0, 256]", op, (long long)ep->lora_rank);
    p.bias = ep->bias != nullptr;
    if (p.bias && (rc = check_dtype(op, "bias", ep->bias_dtype))) return rc;
    p.lora = ep->lora_rank > 0;
    if (p.lora && (rc = check_dtype(op, "LoRA factors", ep->lora_dtype))) return rc;
    p.act = ep->activation;
  }
  p.d1_bf16 = p.d0_bf16 && (!p.bias || ep->bias_dtype == MLXQ_BFLOAT16);
  p.dr_bf16 = x_dtype == MLXQ_BFLOAT16 && (!p.lora || ep->lora_dtype == MLXQ_BFLOAT16);
  p.d2_bf16 = p.d1_bf16 && (!p.lora || p.dr_bf16);
  p.out_bf16 = p.d2_bf16 && p.act != MLXQ_ACT_GELU;
  p.R = p.lora ? (int)round16(ep->lora_rank) : 0;
  size_t off = 0;
  if (p.lora && M > 0 && N > 0) {
    p.xa = off;
    off += align256((size_t)(M * p.R * 4));
    p.lbt = off;
    off += align256((size_t)(N * p.R * 4));
  }
  if (p.promoted() && M > 0 && N > 0) {
    p.y0 = off;
    off += align256((size_t)(M * N * 2));
  }
  p.total = off;
  return MLXQ_OK;
}

static LinearEpilogueArgs epilogue_args(const LinearPlan& p, const void* y_in, bool y_in_bf16,
                                        void* y_out, int64_t M, int64_t N, const mlxq_epilogue* ep,
                                        const void* xa, const void* lbt, float scale_dr) {
  LinearEpilogueArgs a;
  a.y_in = y_in;
  a.y_in_bf16 = y_in_bf16;
  a.y_out = y_out;
  a.y_out_bf16 = p.out_bf16;
  a.M = M;
  a.N = N;
  a.bias = p.bias ? ep->bias : nullptr;
  a.bias_bf16 = p.bias && ep->bias_dtype == MLXQ_BFLOAT16;
  a.d1_bf16 = p.d1_bf16;
  a.xa = xa;
  a.lbt = lbt;
  a.R = p.lora ? p.R : 0;
  a.dr_bf16 = p.dr_bf16;
  a.lora_scale = scale_dr;
  a.d2_bf16 = p.d2_bf16;
  a.act = p.act;
  return a;
}

static int fused_act_of(int act) {
  return act == MLXQ_ACT_GELU_EXACT ? kFusedActGeluExact
         : act == MLXQ_ACT_GELU_TANH ? kFusedActGeluTanh : kFusedActNone;
}

// The bf16 table an elementwise epilogue reads for a bf16 activation (null when none is read).
static int epilogue_table(LinearEpilogueArgs& a, hipStream_t st) {
  if ((a.act == MLXQ_ACT_GELU_TANH || a.act == MLXQ_ACT_GELU_EXACT) && a.d2_bf16) {
    a.act_table = act_table_ptr(fused_act_of(a.act), st);
    if (!a.act_table) return MLXQ_EDEVICE;
  }
  return MLXQ_OK;
}

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

int mlxq_quantize_batched(const void* const* w, int count, int w_dtype, int64_t N, int64_t K, int group_size,
                          int bits, uint32_t* const* wq, void* const* scales, void* const* biases, void* stream) {
  g_err[0] = 0;
  int rc;
  if (count < 0) return set_error(MLXQ_EINVAL, "quantize_batched: count %d < 0", count);
  if ((rc = check_pack("quantize_batched", N, K, group_size, bits))) return rc;
  if ((rc = check_dtype("quantize_batched", "w", w_dtype))) return rc;
  if (count == 0 || N == 0) return MLXQ_OK;
  if (!w || !wq || !scales || !biases) return set_error(MLXQ_EINVAL, "quantize_batched: a pointer array is null");
  for (int e = 0; e < count; ++e) {
    if ((rc = check_aligned("quantize_batched", "w", w[e])) || (rc = check_aligned("quantize_batched", "wq", wq[e])))
      return rc;
    if (!scales[e] || !biases[e]) return set_error(MLXQ_EINVAL, "quantize_batched: scales/biases %d are null", e);
  }
  return run_quantize_batched(w, count, w_dtype, N, K, group_size, bits, wq, scales, biases, (hipStream_t)stream);
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

int mlxq_qmv_valu(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
                  const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
                  int bits, void* y, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_mm("qmv_valu", x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y)))
    return rc;
  if (M > 8) return set_error(MLXQ_EINVAL, "qmv_valu: M=%lld exceeds the GEMV limit of 8", (long long)M);
  if (M == 0 || N == 0) return MLXQ_OK;
  return run_qmv_valu(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y,
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
  // MLX casts x, scales and biases to their result type: bf16 tiles only when all are bf16.
  if (x_dtype == MLXQ_BFLOAT16 && sb_dtype == MLXQ_BFLOAT16 && M > 8)
    return run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, kNoEpilogue,
                   (hipStream_t)stream);
  return run_qmv(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y,
                 (hipStream_t)stream);
}

int mlxq_linear_out_dtype(int x_dtype, int sb_dtype, const mlxq_epilogue* epilogue) {
  g_err[0] = 0;
  LinearPlan p;
  if (plan_linear("linear_out_dtype", x_dtype, sb_dtype, epilogue, 0, 0, p)) return -1;
  return p.out_bf16 ? MLXQ_BFLOAT16 : MLXQ_FLOAT32;
}

size_t mlxq_linear_workspace_size(int x_dtype, int sb_dtype, int64_t M, int64_t N,
                                  const mlxq_epilogue* epilogue) {
  if (M <= 0 || N <= 0) return 0;
  LinearPlan p;
  char saved[sizeof(g_err)];
  memcpy(saved, g_err, sizeof(g_err));  // a size query leaves the error string alone
  const int rc = plan_linear("linear_workspace_size", x_dtype, sb_dtype, epilogue, M, N, p);
  memcpy(g_err, saved, sizeof(g_err));
  return rc ? 0 : p.total;
}

size_t mlxq_lora_residual_workspace_size(int x_dtype, int lora_dtype, int64_t M, int64_t N,
                                         int64_t rank) {
  if (M <= 0 || N <= 0 || rank <= 0 || rank > 256) return 0;
  (void)x_dtype;
  (void)lora_dtype;
  const int64_t R = round16(rank);
  // xa [M,R] and lbt [N,R], 4 bytes per element (enough for f32), 256-byte aligned.
  return align256((size_t)(M * R * 4)) + align256((size_t)(N * R * 4));
}

size_t mlxq_lokr_residual_workspace_size(int x_dtype, int64_t M, int64_t N) {
  (void)x_dtype;
  if (M <= 0 || N <= 0) return 0;
  return align256((size_t)(M * N * 4));  // the f32 product x . delta^T
}

int mlxq_lokr_residual(const void* x, int x_dtype, int64_t M, int64_t K, const void* delta,
                       int delta_dtype, int64_t N, float scale, const void* y_in, int y_dtype,
                       void* y_out, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_dtype("lokr_residual", "x", x_dtype)) ||
      (rc = check_dtype("lokr_residual", "delta", delta_dtype)) ||
      (rc = check_dtype("lokr_residual", "y", y_dtype)))
    return rc;
  if (M < 0 || K <= 0 || N < 0)
    return set_error(MLXQ_EINVAL, "lokr_residual: bad shape M=%lld K=%lld N=%lld", (long long)M,
                     (long long)K, (long long)N);
  if (K % 32 != 0)
    return set_error(MLXQ_EUNSUPPORTED, "lokr_residual: K=%lld is not a multiple of 32 (a quantized "
                                        "base's K is a multiple of its group size)", (long long)K);
  if (M == 0 || N == 0) return MLXQ_OK;
  if (!x || !delta || !y_in || !y_out) return set_error(MLXQ_EINVAL, "lokr_residual: null operand");
  if ((rc = check_aligned("lokr_residual", "x", x)) || (rc = check_aligned("lokr_residual", "delta", delta)))
    return rc;
  // The residual runs in the activation dtype (delta cast to it); the sum promotes with y.
  const bool dr_bf16 = x_dtype == MLXQ_BFLOAT16;
  const bool out_bf16 = y_dtype == MLXQ_BFLOAT16 && dr_bf16;
  if (y_in == y_out && out_bf16 != (y_dtype == MLXQ_BFLOAT16))
    return set_error(MLXQ_EINVAL, "lokr_residual: the sum promotes to float32 and cannot overwrite the "
                                  "bfloat16 y_in in place");
  const size_t need = mlxq_lokr_residual_workspace_size(x_dtype, M, N);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(MLXQ_EINVAL, "lokr_residual: workspace of %zu bytes is smaller than the %zu required",
                     workspace_bytes, need);
  if ((rc = check_aligned("lokr_residual", "workspace", workspace))) return rc;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = run_dense_f32(x, x_dtype, M, K, delta, delta_dtype, N, (float*)workspace, st))) return rc;
  LinearEpilogueArgs a;
  a.y_in = y_in;
  a.y_in_bf16 = y_dtype == MLXQ_BFLOAT16;
  a.y_out = y_out;
  a.y_out_bf16 = out_bf16;
  a.M = M;
  a.N = N;
  a.d1_bf16 = a.y_in_bf16;
  a.res = (const float*)workspace;
  a.dr_bf16 = dr_bf16;
  a.lora_scale = dr_bf16 ? bf16_scalar(scale) : scale;
  a.d2_bf16 = out_bf16;
  return run_linear_epilogue(a, st);
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
                     "32, 64 or 128 and K a multiple of %d whose activation rows and load steps fit "
                     "one workgroup (got M=%lld K=%lld)", 512 / bits, (long long)M,
                     (long long)K);
  return run_swiglu_qmv(x, M, K, wq_gate, scales_gate, biases_gate, wq_up, scales_up, biases_up, F,
                        group_size, bits, h, (hipStream_t)stream);
}

int mlxq_lora_residual(const void* x, int x_dtype, int64_t M, int64_t K, const void* lora_a,
                       const void* lora_b, int lora_dtype, int64_t N, int64_t rank,
                       float lora_scale, const void* y_in, int y_dtype, void* y_out,
                       void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_x_dtype("lora_residual", x_dtype)) ||
      (rc = check_dtype("lora_residual", "LoRA factors", lora_dtype)) ||
      (rc = check_dtype("lora_residual", "y", y_dtype)))
    return rc;
  if (M < 0 || K <= 0 || N < 0) return set_error(MLXQ_EINVAL, "lora_residual: bad shape M=%lld K=%lld N=%lld",
                                                  (long long)M, (long long)K, (long long)N);
  if (rank < 1 || rank > 256)
    return set_error(MLXQ_EINVAL, "lora_residual: rank %lld outside [1, 256]", (long long)rank);
  if (M == 0 || N == 0) return MLXQ_OK;
  if (!x || !lora_a || !lora_b || !y_in || !y_out) return set_error(MLXQ_EINVAL, "lora_residual: null operand");
  const bool dr_bf16 = x_dtype == MLXQ_BFLOAT16 && lora_dtype == MLXQ_BFLOAT16;
  const bool out_bf16 = y_dtype == MLXQ_BFLOAT16 && dr_bf16;
  if (y_in == y_out && out_bf16 != (y_dtype == MLXQ_BFLOAT16))
    return set_error(MLXQ_EINVAL, "lora_residual: the sum promotes to float32 and cannot overwrite the "
                                  "bfloat16 y_in in place");
  const size_t need = mlxq_lora_residual_workspace_size(x_dtype, lora_dtype, M, N, rank);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(MLXQ_EINVAL, "lora_residual: workspace of %zu bytes is smaller than the %zu required",
                     workspace_bytes, need);
  if ((rc = check_aligned("lora_residual", "workspace", workspace))) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int R = (int)round16(rank);
  void* xa = workspace;
  void* lbt = (char*)workspace + align256((size_t)(M * R * 4));
  if ((rc = run_lora_prep(x, x_dtype, M, K, lora_a, lora_b, lora_dtype, N, (int)rank, R, xa, lbt, st)))
    return rc;
  LinearEpilogueArgs a;
  a.y_in = y_in;
  a.y_in_bf16 = y_dtype == MLXQ_BFLOAT16;
  a.y_out = y_out;
  a.y_out_bf16 = out_bf16;
  a.M = M;
  a.N = N;
  a.d1_bf16 = a.y_in_bf16;
  a.xa = xa;
  a.lbt = lbt;
  a.R = R;
  a.dr_bf16 = dr_bf16;
  a.lora_scale = dr_bf16 ? bf16_scalar(lora_scale) : lora_scale;
  a.d2_bf16 = out_bf16;
  return run_linear_epilogue(a, st);
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
                     const void* bias, int bias_dtype, int64_t N, int group_size, int bits, void* y,
                     void* stream) {
  g_err[0] = 0;
  int rc;
  if (E < 0) return set_error(MLXQ_EINVAL, "qmm_experts: E=%lld < 0", (long long)E);
  if ((rc = check_mm("qmm_experts", x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size,
                     bits, y)))
    return rc;
  const bool d0_bf16 = x_dtype == MLXQ_BFLOAT16 && sb_dtype == MLXQ_BFLOAT16;
  if (bias) {
    if ((rc = check_dtype("qmm_experts", "bias", bias_dtype))) return rc;
    if (d0_bf16 && bias_dtype != MLXQ_BFLOAT16)
      return set_error(MLXQ_EUNSUPPORTED, "qmm_experts: a float32 bias over a bfloat16 product (the "
                                          "stacked packs carry bfloat16 biases)");
  }
  if (E == 0 || M == 0 || N == 0) return MLXQ_OK;
  const int xb = x_dtype == MLXQ_FLOAT32 ? 4 : 2;
  const int yb = d0_bf16 ? 2 : 4;
  const int sbb = sb_dtype == MLXQ_BFLOAT16 ? 2 : 4;
  const int bb = bias_dtype == MLXQ_BFLOAT16 ? 2 : 4;
  if (bias && (rc = check_aligned("qmm_experts", "bias", bias, bb))) return rc;
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
  if (d0_bf16 && M > 8 && K % 64 == 0 && E * tiles >= 128 && E <= 65535 &&
      qmm_wide_fits(M, K, N, group_size, bits, sbb)) {
    const QmmEpilogue qe = {(const uint16_t*)bias, nullptr, nullptr, 0, 1.0f, kFusedActNone, nullptr};
    return run_qmm_wide(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, qe, st, bat);
  }
  // Otherwise expert by expert through the single-matrix paths (same rounding points; no
  // workspace: without LoRA nothing is staged and the result never promotes past D0).  Each
  // expert's slices must meet mlxq_linear's alignment: y 16 bytes, scales and biases 4 bytes.
  if (E > 1 && ((M * N * yb) % 16 != 0 || (bat.sb * sbb) % 4 != 0))
    return set_error(MLXQ_EUNSUPPORTED,
                     "qmm_experts: expert by expert, each expert's y slice (M*N = %lld elements of %d "
                     "bytes) must be a multiple of 16 bytes and its scales/biases slice (N*K/group_size "
                     "= %lld of %d bytes) a multiple of 4 bytes; run such packs one expert at a time "
                     "on aligned copies", (long long)(M * N), yb, (long long)bat.sb, sbb);
  for (int64_t e = 0; e < E; ++e) {
    mlxq_epilogue ep = {};
    ep.bias = bias ? (const char*)bias + e * bat.bias * bb : nullptr;
    ep.lora_scale = 1.0f;
    ep.activation = MLXQ_ACT_NONE;
    ep.bias_dtype = bias_dtype;
    ep.lora_dtype = x_dtype;
    if ((rc = mlxq_linear((const char*)x + e * bat.x * xb, x_dtype, M, K, wq + e * bat.w,
                          (const char*)scales + e * bat.sb * sbb, (const char*)biases + e * bat.sb * sbb,
                          sb_dtype, N, group_size, bits, &ep, (char*)y + e * bat.y * yb, nullptr, 0,
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
  LinearPlan p;
  if ((rc = plan_linear("linear", x_dtype, sb_dtype, ep, M, N, p))) return rc;
  if (M == 0 || N == 0) return MLXQ_OK;
  if (p.lora && (!ep->lora_a || !ep->lora_b))
    return set_error(MLXQ_EINVAL, "linear: lora_rank > 0 but A/B are null");
  if (p.bias && (rc = check_aligned("linear", "bias", ep->bias, ep->bias_dtype == MLXQ_BFLOAT16 ? 2 : 4)))
    return rc;
  if (p.total > 0) {
    if (workspace == nullptr || workspace_bytes < p.total)
      return set_error(MLXQ_EINVAL, "linear: workspace of %zu bytes is smaller than the %zu required",
                       workspace_bytes, p.total);
    if ((rc = check_aligned("linear", "workspace", workspace))) return rc;
  }
  hipStream_t st = (hipStream_t)stream;
  void* xa = p.lora ? (char*)workspace + p.xa : nullptr;
  void* lbt = p.lora ? (char*)workspace + p.lbt : nullptr;
  if (p.lora && (rc = run_lora_prep(x, x_dtype, M, K, ep->lora_a, ep->lora_b, ep->lora_dtype, N,
                                    (int)ep->lora_rank, p.R, xa, lbt, st)))
    return rc;
  // The LoRA scale is a scalar cast to the residual's dtype (src/adapters.rs:268-269).
  const float scale = p.lora ? (p.dr_bf16 ? bf16_scalar(ep->lora_scale) : ep->lora_scale) : 1.0f;
  const bool epilogue = p.bias || p.lora || p.act != MLXQ_ACT_NONE;
  if (p.d0_bf16 && M > 8 && p.out_bf16) {
    // Everything in bf16: the GEMM fuses the whole epilogue for LoRA rank <= 16; a wider adapter
    // runs the plain GEMM followed by the elementwise epilogue (same rounding points).
    if (p.R <= 16) {
      QmmEpilogue qe = {p.bias ? (const uint16_t*)ep->bias : nullptr, (const uint16_t*)xa,
                        (const uint16_t*)lbt, p.R, scale, fused_act_of(p.act), nullptr};
      if (qe.act != kFusedActNone && !(qe.act_table = act_table_ptr(qe.act, st))) return MLXQ_EDEVICE;
      return run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, qe, st);
    }
    if ((rc = run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, kNoEpilogue, st)))
      return rc;
    LinearEpilogueArgs a = epilogue_args(p, y, true, y, M, N, ep, xa, lbt, scale);
    if ((rc = epilogue_table(a, st))) return rc;
    return run_linear_epilogue(a, st);
  }
  // An f32 product at GEMM size fuses the bias and the activation (all in f32) unless a LoRA
  // adapter needs the elementwise epilogue.
  if (!p.d0_bf16 && M > 8 && !p.lora) {
    F32Epilogue fe;
    fe.bias = p.bias ? ep->bias : nullptr;
    fe.bias_bf16 = p.bias && ep->bias_dtype == MLXQ_BFLOAT16;
    fe.act = p.act;
    return run_qmm_f32(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y, st, fe);
  }
  // The product in D0, straight into y when y has that dtype; a bf16 product whose result
  // promotes to f32 goes through the workspace (the elementwise epilogue widens it into y).
  void* y0 = p.promoted() ? (char*)workspace + p.y0 : y;
  if (p.d0_bf16 && M > 8) rc = run_qmm(x, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y0,
                                       kNoEpilogue, st);
  else rc = run_qmv(x, x_dtype, M, K, wq, scales, biases, sb_dtype, N, group_size, bits, y0, st);
  if (rc) return rc;
  if (!epilogue && !p.promoted()) return MLXQ_OK;
  LinearEpilogueArgs a = epilogue_args(p, y0, p.d0_bf16, y, M, N, ep, xa, lbt, scale);
  if ((rc = epilogue_table(a, st))) return rc;
  return run_linear_epilogue(a, st);
}

}  // extern "C"
