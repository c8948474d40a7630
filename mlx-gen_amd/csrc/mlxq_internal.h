// mlxq_internal.h — declarations shared between the ABI layer and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlxq {

// Fused GEMM epilogue operands (all bf16, device pointers, nullable).
struct QmmEpilogue {
  const uint16_t* bias;  // [N]
  const uint16_t* xa;    // [M, rank16] = round_bf16(x . A), zero padded
  const uint16_t* lbt;   // [N, rank16] = B^T, zero padded
  int rank16;            // padded LoRA rank (multiple of 16), 0 = no LoRA
  float lora_scale;      // already rounded to the activation dtype
  int act;               // mlxq_activation
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
int run_dequantize(const uint32_t* wq, const void* s, const void* b, int dtype, int64_t N, int64_t K,
                   int gs, int bits, void* out, hipStream_t st);
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
int run_embedding(const int32_t* ids, int64_t T, const uint32_t* wq, const void* s, const void* b,
                  int sb_dtype, int64_t vocab, int64_t hidden, int gs, int bits, void* out,
                  int out_dtype, hipStream_t st);
int run_lora_prep(const void* x, int x_dtype, int64_t M, int64_t K, const void* A, const void* B,
                  int64_t N, int rank, int R, void* xa, void* lbt, hipStream_t st);
int run_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, hipStream_t st);
int run_linear_epilogue(void* y, int x_dtype, int64_t M, int64_t N, const void* bias, const void* xa,
                        const void* lbt, int R, float lora_scale, int act, hipStream_t st);

}  // namespace mlxq
