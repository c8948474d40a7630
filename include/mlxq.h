/*
 * mlxq.h — C ABI of libmlxq_hip.so, the MI355X (gfx950) implementation of mlx-gen's group-wise
 * affine Q4/Q8 quantized-linear path.
 *
 * The reference reaches this arithmetic through three MLX ops and one MLX layer, all external to
 * the reference (pmetal-mlx-rs 0.25.8 -> MLX 0.31.2, reference Cargo.toml:38,43):
 *   mlx_rs::ops::quantize            called at src/quant.rs:140, src/nn.rs:91-93, and via
 *                                    nn::QuantizedLinear::try_from_linear at src/adapters.rs:533-537
 *   mlx_rs::ops::dequantize          called at src/nn.rs:55, mlx-gen-flux/src/text_encoder.rs:78
 *   mlx_rs::ops::quantized_matmul    called at src/adapters.rs:309-317 (LinearBase::forward)
 * Each entry point below replaces one of them; a Rust -sys crate binds these symbols one-to-one.
 *
 * Conventions
 *   - All tensor pointers are DEVICE pointers owned by the caller; the library allocates nothing
 *     on these paths except where a workspace size query says so.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the default stream).
 *   - Row-major, contiguous.  Packing: 32/bits codes per uint32, element i of a word at bit offset
 *     i*bits (low bits first); wq [N, K*bits/32]; scales/biases [N, K/group_size].
 *   - group_size in {32, 64, 128}, bits in {4, 8}, K % group_size == 0.
 *   - Alignment: activations, packed weights, outputs and workspaces 16 bytes; scales and biases
 *     4 bytes.  Misaligned pointers are rejected with MLXQ_EINVAL.
 *   - Every call returns an mlxq_status; on failure mlxq_last_error() (thread-local) describes
 *     it.  Arguments that contradict each other here (dtype codes, group_size/bits, K % gs,
 *     alignment, null pointers) are rejected with MLXQ_EINVAL.  This layer sees pointers, not
 *     tensor shapes: the C++ and Python hosts check every operand's shape and dtype against x
 *     before they call in (the reference's packed_bits panics on malformed triples,
 *     src/quant.rs:38-41).
 *   - Dtypes follow MLX's promotion: an op on a bf16 and an f32 operand computes and returns f32
 *     (quantized_matmul returns promote(x, scales); a bias add and a LoRA residual promote the
 *     output the same way).  mlxq_linear_out_dtype gives the dtype y must have.
 *   - Re-entrant per stream.  Process-wide state, all of it per device and written once: the two
 *     GELU tables (device memory in the code object, filled by the first GELU GEMM on a device),
 *     the cached CU count, the decode GEMV's raised dynamic-LDS limit (atomic flags), the device
 *     address of mlxq_linear_noalloc's static scratch (guarded by a mutex), plus the thread-local
 *     error string.
 */
#ifndef MLXQ_H
#define MLXQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MLXQ_FLOAT32 = 0,
  MLXQ_BFLOAT16 = 1,
  /* fp16 is taken as the activation x of quantized_matmul, qmv, qmv_valu, linear, linear_noalloc,
   * lora_residual and qmm_experts: the dtype SDXL's U-Net, CLIP encoders and ControlNets run in
   * (mlx-gen-sdxl/src/model.rs:216) over bf16-packed weights (src/adapters.rs:508-537).  MLX
   * promotes fp16 against bf16 or f32 to f32, so those products and their results are f32.
   * Elsewhere (weights, scales, biases, LoRA factors, outputs) fp16 returns MLXQ_EUNSUPPORTED. */
  MLXQ_FLOAT16 = 2,
} mlxq_dtype;

typedef enum {
  MLXQ_OK = 0,
  MLXQ_EINVAL = 1,       /* bad shape / dtype / group_size / bits / null pointer */
  MLXQ_EUNSUPPORTED = 2, /* valid for MLX but not implemented here (e.g. transpose=false) */
  MLXQ_EDEVICE = 3,      /* HIP launch or runtime error */
} mlxq_status;

typedef enum {
  MLXQ_ACT_NONE = 0,
  /* mlx_rs::nn::gelu, the exact-erf GELU of FLUX's FeedForward (mlx-gen-flux/src/transformer.rs:975;
   * also mlx-gen-qwen-image/src/text_encoder/vision/merger.rs:49, mlx-gen-ltx/src/connector.rs:252):
   * its constants are f32 arrays, so a bf16 input promotes and the result is f32 (src/nn.rs:335-338) */
  MLXQ_ACT_GELU = 1,
  /* tanh-approximate GELU as separate ops in the input dtype, src/nn.rs:321-329 (FLUX
   * single-stream FFN and GeluApprox, mlx-gen-flux/src/transformer.rs:506,708,979) */
  MLXQ_ACT_GELU_TANH = 2,
  /* dtype-preserving exact GELU, src/nn.rs:344-355 gelu_exact (x * (1 + erf(x / sqrt2))) / 2; the
   * GELU of most crates' FFNs (bernini, boogu, pid, svd, ...).  In bf16 each op of the sequence is
   * rounded to bf16 (the uncompiled op sequence).  The reference runs it under compile(f, true),
   * whose fused kernel its own comments say rounds 16-bit types differently from the separate ops
   * (src/nn.rs:339-343): bf16 parity with the reference is unpinned.  f32 is unaffected. */
  MLXQ_ACT_GELU_EXACT = 3,
} mlxq_activation;

/* Thread-local description of the last failure on this thread ("" if none). */
const char* mlxq_last_error(void);
/* Library version string. */
const char* mlxq_version(void);

/*
 * quantize — replaces mlx_rs::ops::quantize(w, group_size, bits) (src/quant.rs:140;
 * src/adapters.rs:533-537 through QuantizedLinear::try_from_linear).
 * w [N,K] in w_dtype; writes wq [N, K*bits/32] and scales/biases [N, K/group_size] in w_dtype.
 */
int mlxq_quantize(const void* w, int w_dtype, int64_t N, int64_t K, int group_size, int bits,
                  uint32_t* wq, void* scales, void* biases, void* stream);

/*
 * quantize over `count` weights of one shape [N,K] and dtype: the same outputs as `count`
 * mlxq_quantize calls (w[i] -> wq[i], scales[i], biases[i]), in launches of up to 16 weights,
 * which pay a launch's ramp and its partly filled last round once for all of them.  No single
 * counterpart in the reference, which quantizes weight by weight (quantize_map, src/quant.rs:125-149,
 * calling a-1 per target); for converters that pack many same-shaped weights.  The pointer arrays
 * are host memory; count == 0 does nothing.
 */
int mlxq_quantize_batched(const void* const* w, int count, int w_dtype, int64_t N, int64_t K, int group_size,
                          int bits, uint32_t* const* wq, void* const* scales, void* const* biases, void* stream);

/*
 * dequantize — replaces mlx_rs::ops::dequantize(wq, scales, biases, group_size, bits)
 * (src/nn.rs:55).  out [N,K] in sb_dtype (the scales dtype, as MLX returns).
 */
int mlxq_dequantize(const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                    int64_t N, int64_t K, int group_size, int bits, void* out, void* stream);

/*
 * quantized_matmul — replaces mlx_rs::ops::quantized_matmul(x, wq, scales, biases, transpose,
 * group_size, bits) (src/adapters.rs:309-317).  x [M,K] in x_dtype (batch dims flattened into
 * M); y [M,N] in promote(x_dtype, sb_dtype) (bf16 only when both are bf16, as MLX casts x, scales
 * and biases to their result type); fp32 accumulation.  Only transpose=1 (y = x . W^T, the only
 * form the reference uses) is implemented; transpose=0 returns MLXQ_EUNSUPPORTED.
 * Dispatch: bf16 x and scales with M > 8 run the MFMA GEMM (weights dequantized to bf16 tiles);
 * bf16 with M <= 8 runs the bandwidth-bound GEMV (weights dequantized in f32, factored per
 * group); an f32 operand, or fp16 x (which MLX promotes to f32 against bf16 or f32 scales), runs
 * the f32 kernels (exact f32 dequant, f32 result).
 */
int mlxq_quantized_matmul(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
                          const void* scales, const void* biases, int sb_dtype, int64_t N,
                          int transpose, int group_size, int bits, void* y, void* stream);

/*
 * Quantized token-embedding lookup — replaces TokenEmbedding::forward's quantized arm
 * (src/nn.rs:42-58: take_axis of wq/scales/biases by ids, dequantize, cast to f32) in one pass.
 * ids [T] int32 device array; table wq [vocab, hidden*bits/32] with scales/biases
 * [vocab, hidden/group_size] in sb_dtype; out [T, hidden] in out_dtype (MLXQ_FLOAT32 reproduces
 * the reference's cast).  Each value is dequantize()'s, i.e. rounded to sb_dtype first.  Ids
 * outside [0, vocab) produce a row of NaN.
 */
int mlxq_embedding(const int32_t* ids, int64_t T, const uint32_t* wq, const void* scales,
                   const void* biases, int sb_dtype, int64_t vocab, int64_t hidden, int group_size,
                   int bits, void* out, int out_dtype, void* stream);

/* Forced-kernel variants of quantized_matmul (same arguments, transpose implied = 1). */
/* MFMA bf16-tile GEMM; x must be bf16; any M >= 1; y is bf16 whatever sb_dtype is (the kernel's
 * native output: with f32 scales this is not quantized_matmul's promoted f32 result). */
int mlxq_qmm(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
             const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
             int bits, void* y, void* stream);
/* GEMV; bf16, f32 or fp16 x; 1 <= M <= 8; y in promote(x_dtype, sb_dtype). */
int mlxq_qmv(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
             const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
             int bits, void* y, void* stream);

/* A GEMV on the VALU only (no matrix cores); any x / scales dtype; 1 <= M <= 8; y in
 * promote(x_dtype, sb_dtype).  The VALU GEMV with exact f32 dequant (the kernel quantized_matmul
 * uses for f32 operands and group size 32), except at M = 1 with bf16 x and scales, Q4, group
 * 64/128 and K <= 8192, where it is the M = 1 matrix-core kernel's loads and fold with VALU dot
 * products.  Forced here so it can be measured against the matrix-core GEMV on bf16 decode
 * shapes. */
int mlxq_qmv_valu(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
                  const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
                  int bits, void* y, void* stream);

/*
 * Fused AdaptableLinear forward over a quantized base — replaces the op sequence of
 * LinearBase::forward's quantized arm plus AdaptableLinear::forward (src/adapters.rs:300-322,
 * 543-549) for one LoRA adapter (Adapter::residual, src/adapters.rs:260-270), optionally followed
 * by the caller's activation (FeedForward::forward, mlx-gen-flux/src/transformer.rs:970-977):
 *   y0 = qmm(x)                 in D0 = promote(x_dtype, sb_dtype)          (:309-317)
 *   y1 = y0 + bias              in D1 = promote(D0, bias_dtype)             (:318-320)
 *   r  = ((x.A).B) * scale      in DR = promote(x_dtype, lora_dtype), each op rounded to DR and
 *                               scale cast to DR first (the factors keep their file dtype, :243-252)
 *   y2 = y1 + r                 in D2 = promote(D1, DR), not cast back     (:546)
 *   y  = act(y2)                GELU_TANH / GELU_EXACT per op in D2; GELU in f32
 * Each round() happens exactly where the reference's separate MLX ops round, and y has dtype
 * mlxq_linear_out_dtype().  bias [N] (bias_dtype), lora_a [K,rank] and lora_b [rank,N]
 * (lora_dtype) are nullable (rank 0 = no LoRA); rank <= 256.  workspace must hold
 * mlxq_linear_workspace_size() bytes (NULL when that is 0).
 */
typedef struct {
  const void* bias;
  const void* lora_a;
  const void* lora_b;
  int64_t lora_rank;
  float lora_scale;
  int activation; /* mlxq_activation */
  int bias_dtype; /* mlxq_dtype of bias (ignored when bias is NULL) */
  int lora_dtype; /* mlxq_dtype of lora_a and lora_b (ignored when lora_rank is 0) */
} mlxq_epilogue;

/* The dtype y of mlxq_linear has for these operands (an mlxq_dtype), or -1 (with
 * mlxq_last_error set) when a dtype code or the activation is invalid.  epilogue may be NULL. */
int mlxq_linear_out_dtype(int x_dtype, int sb_dtype, const mlxq_epilogue* epilogue);

/* Bytes of device workspace mlxq_linear needs (0: pass NULL): the LoRA staging (x.A and B^T
 * padded to rank 16, 4 bytes per element) and, when a bf16 product promotes to an f32 result,
 * the bf16 product itself [M, N].  0 as well for invalid arguments (mlxq_linear reports them). */
size_t mlxq_linear_workspace_size(int x_dtype, int sb_dtype, int64_t M, int64_t N,
                                  const mlxq_epilogue* epilogue);

int mlxq_linear(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
                const void* scales, const void* biases, int sb_dtype, int64_t N, int group_size,
                int bits, const mlxq_epilogue* epilogue, void* y, void* workspace,
                size_t workspace_bytes, void* stream);

/*
 * mlxq_linear without a workspace argument: the workspace mlxq_linear_workspace_size reports
 * (LoRA staging, and the bf16 product of a promoted result) lives in a static device array of
 * MLXQ_NOALLOC_SCRATCH_BYTES that each GPU holds from the first call on it until the process ends.
 * No counterpart in the reference: this entry point exists for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It calls no allocator.  A problem that needs more scratch than the array holds is
 * rejected with MLXQ_EINVAL before any device work.  The first call on each device resolves the
 * array's device address (hipGetSymbolAddress), so make it outside graph capture.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (several streams or threads)
 * race and must be serialised by the caller.  Same arguments, results and errors as mlxq_linear
 * otherwise.
 */
#define MLXQ_NOALLOC_SCRATCH_BYTES (8u << 20)

int mlxq_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq,
                        const void* scales, const void* biases, int sb_dtype, int64_t N,
                        int group_size, int bits, const mlxq_epilogue* epilogue, void* y,
                        void* stream);

/*
 * Stacked-expert projection — Proj::forward of the quantized MoE experts
 * (mlx-gen-lens/src/text_encoder/gpt_oss.rs:412-425, quantized_matmul(x, wq, s, b, true) + bias)
 * run for every expert of a stacked pack split along axis 0 (mlx-gen-lens/src/quant.rs:93-137):
 *   for e in [0, E):  y[e] = round(round(x[e] . dequant(wq[e])^T) + bias[e])
 * rounded to D0 = promote(x_dtype, sb_dtype) and then promote(D0, bias_dtype), as mlxq_linear.
 * wq [E, N, K*bits/32], scales/biases [E, N, K/group_size] (sb_dtype), bias [E, N] in bias_dtype
 * or NULL, y [E, M, N].  The reference's stacked packs carry a bf16 bias (gpt_oss.rs:478-487); an
 * f32 bias over a bf16 product would need a promoted second pass and returns MLXQ_EUNSUPPORTED.
 * x is [M, K] shared by every expert when x_per_expert == 0 (the gate_up projection of
 * gpt_oss.rs:702), else [E, M, K] (the down projection of :714).  Each expert's result equals the
 * single-matrix mlxq_linear with that bias.  bf16 x and scales with M > 8, K a multiple of 64 and at
 * least 128 GEMM tiles over all experts run every expert in one launch; otherwise the experts run
 * one after another through mlxq_linear, which needs each expert's slices aligned: M*N elements of
 * y a multiple of 16 bytes and N*K/group_size scales (biases) a multiple of 4 bytes, else
 * MLXQ_EUNSUPPORTED (the Python and C++ hosts then run those experts on aligned copies).
 */
int mlxq_qmm_experts(const void* x, int x_dtype, int x_per_expert, int64_t E, int64_t M, int64_t K,
                     const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                     const void* bias, int bias_dtype, int64_t N, int group_size, int bits, void* y,
                     void* stream);

/*
 * Fused SwiGLU gate/up for decode — the first two ops of Mlp::forward
 * (mlx-gen-sensenova/src/qwen3.rs:178-181): h = multiply(silu(gate.forward(x)), up.forward(x))
 * with gate/up quantized linears [F,K] sharing x [M,K]; one launch streams both weight matrices
 * (launches of four or two activation rows when the M rows do not fit one workgroup):
 *   h = round(round(silu(round(x.Wg^T))) * round(x.Wu^T))      (round() to bf16)
 * Decode form only: bf16 x and scales, 1 <= M <= 8, group_size 32, 64 or 128, K a multiple of
 * 512/bits within the fused kernels' reach (Q4: K <= 16384 at M = 1, 12288 at M = 2..8, 8192
 * with group 32; Q8: 8192 at M = 1, 6144 at M = 2..8, 4096 with group 32); anything else
 * returns MLXQ_EUNSUPPORTED (callers then run the two linears).
 * This entry point has no single counterpart in the reference; it replaces a three-op sequence.
 */
int mlxq_swiglu(const void* x, int x_dtype, int64_t M, int64_t K, const uint32_t* wq_gate,
                const void* scales_gate, const void* biases_gate, const uint32_t* wq_up,
                const void* scales_up, const void* biases_up, int sb_dtype, int64_t F,
                int group_size, int bits, void* h, void* stream);

/*
 * One more LoRA adapter on an already computed output — the `out + adapter.residual(x)` step of
 * AdaptableLinear::forward (src/adapters.rs:543-549, Adapter::residual :260-270) for adapter
 * stacks beyond the one mlxq_linear fuses:
 *   y_out = y_in + r,  r = ((x.A).B) * scale in DR = promote(x_dtype, lora_dtype) (each op rounded
 *   to DR, scale cast to DR), the sum in promote(y_dtype, DR) — the dtype y_out must have.
 * A [K,rank], B [rank,N] in lora_dtype, 1 <= rank <= 256.  y_out may be y_in when the sum keeps
 * y_dtype; otherwise the two must not overlap.  workspace: mlxq_lora_residual_workspace_size().
 */
size_t mlxq_lora_residual_workspace_size(int x_dtype, int lora_dtype, int64_t M, int64_t N,
                                         int64_t rank);
int mlxq_lora_residual(const void* x, int x_dtype, int64_t M, int64_t K, const void* lora_a,
                       const void* lora_b, int lora_dtype, int64_t N, int64_t rank,
                       float lora_scale, const void* y_in, int y_dtype, void* y_out,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * One LoKr adapter on an already computed output — the Adapter::Lokr arm of Adapter::residual
 * (src/adapters.rs:263-266) in AdaptableLinear::forward's residual sum (:543-549):
 *   d = delta cast to x_dtype;  r = x . d^T in x_dtype (f32 accumulation, rounded once);
 *   r = r * scale (scale cast to x_dtype first);  y_out = y_in + r in promote(y_dtype, x_dtype).
 * delta [N, K] in delta_dtype is the reconstructed kron delta (reconstruct_lokr_delta,
 * src/adapters.rs:26-128; the reference stores it bf16).  K must be a multiple of 32.  y_out may be
 * y_in when the sum keeps y_dtype; otherwise the two must not overlap.  workspace:
 * mlxq_lokr_residual_workspace_size() bytes (the f32 product, M*N*4).
 */
size_t mlxq_lokr_residual_workspace_size(int x_dtype, int64_t M, int64_t N);
int mlxq_lokr_residual(const void* x, int x_dtype, int64_t M, int64_t K, const void* delta,
                       int delta_dtype, int64_t N, float scale, const void* y_in, int y_dtype,
                       void* y_out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Element-wise dtype conversion f32 <-> bf16 (round to nearest even) — the `as_dtype(Bfloat16)`
 * casts that precede packing in AdaptableLinear::quantize (src/adapters.rs:508-521) and
 * quant::quantize_map (src/quant.rs:140).  src/dst 4-byte aligned.
 */
int mlxq_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream);

/*
 * Host-side shape helper — replaces quant::packed_bits (src/quant.rs:38-41): from the packed
 * shapes infer bits = wq_cols*32 / (scales_cols*group_size).  Returns 4 or 8, or -1 (with
 * mlxq_last_error set) for a malformed triple instead of panicking.
 */
int mlxq_packed_bits(int64_t wq_cols, int64_t scales_cols, int group_size);

#ifdef __cplusplus
}
#endif

#endif /* MLXQ_H */
