// mlxq_internal.h — declarations shared between the ABI layer and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlxq {

// Activation fused into a bf16 GEMM epilogue (QmmEpilogue::act).  Both are functions of the
// bf16 pre-activation, evaluated as a lookup in a per-device table of the bf16 result.
enum FusedAct : int {
  kFusedActNone = 0,
  kFusedActGeluExact = 1,  // MLXQ_ACT_GELU_EXACT in bf16 (table 0)
  kFusedActGeluTanh = 2,   // MLXQ_ACT_GELU_TANH in bf16 (table 1)
};

// Fused GEMM epilogue operands (all bf16, device pointers, nullable).
struct QmmEpilogue {
  const uint16_t* bias;  // [N]
  const uint16_t* xa;    // [M, rank16] = round_bf16(x . A), zero padded
  const uint16_t* lbt;   // [N, rank16] = B^T, zero padded
  int rank16;            // padded LoRA rank (multiple of 16), 0 = no LoRA
  float lora_scale;      // already rounded to the activation dtype
  int act;               // FusedAct
  const uint16_t* act_table;  // [65536] bf16 table of act (act_table_ptr), null when act is none
};

// The elementwise epilogue of a linear on an already computed product y_in [M, N]: bias, LoRA
// residual and activation with each stage rounded to its promoted dtype (the *_bf16 flags), the
// result written to y_out (may alias y_in when both have the same dtype).
struct LinearEpilogueArgs {
  const void* y_in = nullptr;
  bool y_in_bf16 = true;
  void* y_out = nullptr;
  bool y_out_bf16 = true;
  int64_t M = 0, N = 0;
  const void* bias = nullptr;  // [N]
  bool bias_bf16 = true;
  bool d1_bf16 = true;         // y + bias rounds to bf16
  const void* xa = nullptr;    // [M, R] x . A, already rounded to DR
  const void* lbt = nullptr;   // [N, R] B^T
  int R = 0;                   // padded rank, 0 = no LoRA
  bool dr_bf16 = true;         // xa / lbt stored as bf16, r rounded to bf16
  float lora_scale = 1.0f;     // already cast to DR
  bool d2_bf16 = true;         // y + r rounds to bf16
  int act = 0;                 // mlxq_activation
  const uint16_t* act_table = nullptr;  // bf16 table of act when the activation runs in bf16
  const float* res = nullptr;  // [M, N] f32 product of a dense residual (LoKr), R must be 0: r is
                               // this value rounded to DR, then scaled like the LoRA residual
};

// A stacked launch over `count` matrices of the same shape (the experts of an [E, out, ...] pack):
// matrix e uses each operand's base pointer advanced by e times its stride (in elements of that
// operand; a zero stride shares the operand, e.g. one activation matrix for every expert).
struct QmmBatch {
  int64_t count = 1;
  int64_t x = 0, w = 0, sb = 0, y = 0, bias = 0;
};

int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

int run_quantize(const void* w, int dtype, int64_t N, int64_t K, int gs, int bits, uint32_t* wq,
                 void* s, void* b, hipStream_t st);
int run_quantize_batched(const void* const* w, int count, int dtype, int64_t N, int64_t K, int gs, int bits,
                         uint32_t* const* wq, void* const* s, void* const* b, hipStream_t st);
int run_dequantize(const uint32_t* wq, const void* s, const void* b, int dtype, int64_t N, int64_t K,
                   int gs, int bits, void* out, hipStream_t st);
// The f32-dequant product; y in promote(x_dtype, sb_dtype): the GEMV for M <= 8 (exact f32), the
// split-bf16 GEMM for larger M (f32 operands, within ~1e-5 relative of the f32 product).
int run_qmv(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq, const void* s,
            const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y, hipStream_t st);
int run_qmm(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s, const void* b,
            int sb_dtype, int64_t N, int gs, int bits, void* y, const QmmEpilogue& epi,
            hipStream_t st);
bool qmm_wide_fits(int64_t M, int64_t K, int64_t N, int gs, int bits, int sb_bytes);
// Whether bf16 scales and biases (bytes each) lie within 4 GiB of the lower of the two, so the
// wide GEMM can read both through one 32-bit-offset buffer resource.  Always true for f32.
bool qmm_wide_sb_reach(const void* scales, const void* biases, int64_t bytes, int sb_bytes);
bool qmm_small_fits(int64_t M, int64_t K, int64_t N, int gs, int bits, int sb_bytes);
int run_qmm_small(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                  const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y,
                  const QmmEpilogue& epi, hipStream_t st);
int run_qmm_wide(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s, const void* b,
                 int sb_dtype, int64_t N, int gs, int bits, void* y, const QmmEpilogue& epi,
                 hipStream_t st, const QmmBatch& batch = QmmBatch{});
bool qmv_mfma_applicable(int x_dtype, int sb_dtype, int64_t M, int64_t K, int64_t N, int gs, int bits);
int run_qmv_mfma(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* s, const void* b,
                 int64_t N, int gs, int bits, void* y, hipStream_t st);
bool swiglu_qmv_applicable(int x_dtype, int sb_dtype, int64_t M, int64_t K, int64_t F, int gs, int bits);
int run_swiglu_qmv(const void* x, int64_t M, int64_t K, const uint32_t* wq_g, const void* s_g,
                   const void* b_g, const uint32_t* wq_u, const void* s_u, const void* b_u, int64_t F,
                   int gs, int bits, void* h, hipStream_t st);
// The one-row GEMV (M = 1) with its MFMA dot products replaced by VALU v_dot2_f32_bf16, same
// loads, unpack and fold:
// the VALU side of the kernel-choice A/B for bf16 operands at M = 1, Q4 group 64/128, K <= 8192.
bool qmv_row_valu_applicable(int x_dtype, int sb_dtype, int64_t M, int64_t K, int64_t N, int gs, int bits);
int run_qmv_row_valu(const void* x, int64_t K, const uint32_t* wq, const void* s, const void* b, int64_t N,
                     int gs, void* y, hipStream_t st);
// The VALU GEMV with exact f32 dequant, whatever the operand dtypes (the forced-kernel entry
// point for measuring it against the matrix-core GEMV).
int run_qmv_valu(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                 const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y, hipStream_t st);
// Compute units of the current device (cached per device; 256 if the query fails).
int64_t device_cu_count();
// The f32 epilogue the f32 GEMM can fuse: y + bias (bias in its own dtype, the sum in f32), then
// an activation evaluated in f32 (mlxq_activation; the sequence of linear_epilogue_kernel in f32).
struct F32Epilogue {
  const void* bias = nullptr;  // [N]
  bool bias_bf16 = false;
  int act = 0;                 // mlxq_activation
};
// Large-M GEMM for operands MLX computes in f32 (f32 x and/or f32 scales), f32 y, as three bf16
// MFMA passes over two-term bf16 splits of x and of the f32-dequantized weights.
int run_qmm_f32(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq, const void* s,
                const void* b, int sb_dtype, int64_t N, int gs, int bits, void* y, hipStream_t st,
                const F32Epilogue& epi = F32Epilogue{});
// y[M, N] f32 = x[M, K] . d^T for a dense d [N, K] in d_dtype, cast to bf16 against bf16 x, on
// the matrix cores (bf16 passes over two-term splits of the f32 operands).  K % 32 == 0.
int run_dense_f32(const void* x, int x_dtype, int64_t M, int64_t K, const void* d, int d_dtype,
                  int64_t N, float* y, hipStream_t st);
int run_embedding(const int32_t* ids, int64_t T, const uint32_t* wq, const void* s, const void* b,
                  int sb_dtype, int64_t vocab, int64_t hidden, int gs, int bits, void* out,
                  int out_dtype, hipStream_t st);
// x.A and B^T for a LoRA residual in DR = promote(x_dtype, lora_dtype): bf16 arrays when both
// are bf16, else f32 arrays (x and the factors widened exactly).
int run_lora_prep(const void* x, int x_dtype, int64_t M, int64_t K, const void* A, const void* B,
                  int lora_dtype, int64_t N, int rank, int R, void* xa, void* lbt, hipStream_t st);
int run_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, hipStream_t st);
int run_linear_epilogue(const LinearEpilogueArgs& a, hipStream_t st);
// Device address of the bf16 table of a FusedAct (filled on the device's first request), or
// null with the error set.
const uint16_t* act_table_ptr(int fused_act, hipStream_t st);

}  // namespace mlxq
