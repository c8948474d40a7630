/*
 * mlxq_oracle.c — CPU restatement of mlx-gen's group-wise affine Q4/Q8 quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP path is compared against; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The product
 * library (libmlxq_hip.so) never links or calls it, and there is no CPU fallback.
 *
 * The arithmetic being restated lives in MLX 0.31.2 (C++/Metal), reached through the git-pinned
 * crate pmetal-mlx-rs 0.25.8 (rev 38e1cc1730a11b1e40c2c8ecda01606763a12d51, reference
 * Cargo.toml:38,43, Cargo.lock:1120-1147).  That source is not present, so each function restates
 * MLX's published affine-quantization algorithm and cites the reference call site it serves.
 *
 * Pinning (what fixes each function besides its own text):
 *   oracle_quantize    pinned: reference tests/fixtures/quant_q4q8.safetensors (q4/q8 .wq, .scales,
 *                      .biases, bit-exact, f32 input); closed forms for all-zero and constant
 *                      groups; row-split commutation (mlx-gen-sdxl/src/quant.rs:89-110).
 *                      Parity unpinned for: the bf16-input scale rounding point, the tie rule of
 *                      round() (fixture holds no exact .5 ties), eps for near-constant groups.
 *   oracle_dequantize  pinned: fixture q4/q8 .deq (single-rounded fma, 0 mismatches).
 *   oracle_qmm         pinned: fixture q4/q8 .qmm (f32 activations, exact dequant); textbook
 *                      matmul over the dequantized matrix for the bf16-tile variant.
 *   oracle_linear      pinned by composition: qmm + the reference op sequence of
 *                      src/adapters.rs:300-322,543-549 (bias add, then LoRA residual) under MLX's
 *                      bf16/f32 promotion (src/adapters.rs:243-252); its rounding points follow
 *                      MLX's per-op rounding (not pinned by a golden: parity unpinned for the
 *                      bf16 rounding points).
 *   oracle_lokr_residual  pinned: the reference's LoKr tests (src/adapters.rs:695-764, 1089-1119:
 *                      the 2x2 kron delta, a bf16 residual within 5e-2 of the f32 one, scale 0 is
 *                      a bit-exact no-op, LoRA + LoKr stacks sum their residuals) and the
 *                      closed form x . delta^T of a rank-1 (kron of vectors) delta; the bf16
 *                      rounding points are parity unpinned (MLX per-op rounding, as elsewhere).
 *   oracle_gelu_erf    textbook closed form (special values tested).
 *   oracle_silu        the op sequence of src/nn.rs:301-303 (sigmoid, then multiply, each rounded
 *                      to the activation dtype); in f32 pinned by the closed form x / (1 + e^-x)
 *                      and its special values; in bf16 parity unpinned (MLX's internal sigmoid
 *                      precision is not fixed by any golden; the correctly rounded f32 sigmoid is
 *                      taken).
 *   oracle_gelu_exact  the op sequence of src/nn.rs:344-355 in the input dtype; in f32 pinned by
 *                      its distance to the closed form, in bf16 parity unpinned (rounding points).
 *   oracle_gelu_tanh   pinned in f32 by the closed form (the reference test points of
 *                      src/nn.rs:722-738 among them) and by its distance to the exact GELU; the
 *                      per-op bf16 rounding points follow src/nn.rs:321-329 and are not pinned
 *                      by a golden (parity unpinned for bf16).
 *
 * Data convention: every float tensor crosses this interface as f32.  A bf16 tensor is passed as
 * the f32 values it represents (exact), and the `*_bf16` flags say where results are rounded to
 * bf16 (round-to-nearest-even), as the reference does when its arrays have dtype bf16.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_OK 0
#define ORACLE_EINVAL 1

/*
 * Round-to-nearest-even f32 -> IEEE binary16 (fp16), returned widened back to f32: the value an
 * fp16 activation holds (SDXL runs fp16, reference mlx-gen-sdxl/src/model.rs:216).  Magnitudes
 * from 65520 up round to infinity; subnormals (steps of 2^-24) are kept; NaN stays NaN.  fp16
 * activations then enter every function below as these f32 values with the bf16 flags off: MLX
 * promotes fp16 against bf16 or f32 scales to f32, so the product is the f32 one.
 */
float oracle_fp16_round(float x) {
    if (isnan(x) || isinf(x)) return x;
    const double ax = fabs((double)x);
    if (ax >= 65520.0) return x > 0 ? INFINITY : -INFINITY;
    if (ax == 0.0) return x;
    int e2;
    frexp(ax, &e2);                    /* ax = m * 2^e2, m in [0.5, 1): leading bit at 2^(e2-1) */
    int e = e2 - 1;
    if (e < -14) e = -14;              /* subnormal range: fixed step 2^-24 */
    const double ulp = ldexp(1.0, e - 10);
    return (float)(nearbyint((double)x / ulp) * ulp);
}

void oracle_fp16_round_array(float* a, int64_t n) {
    for (int64_t i = 0; i < n; ++i) a[i] = oracle_fp16_round(a[i]);
}

/* Round-to-nearest-even f32 -> bf16, returned widened back to f32 (NaN kept quiet). */
float oracle_bf16_round(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        u |= 0x00400000u;
        u &= 0xffff0000u;
    } else {
        uint32_t lsb = (u >> 16) & 1u;
        u += 0x7fffu + lsb;
        u &= 0xffff0000u;
    }
    float r;
    memcpy(&r, &u, 4);
    return r;
}

static inline float rnd(float x, int to_bf16) { return to_bf16 ? oracle_bf16_round(x) : x; }

static int valid_shape(int64_t N, int64_t K, int gs, int bits) {
    if (N < 0 || K <= 0) return 0;
    if (bits != 4 && bits != 8) return 0;
    if (gs != 32 && gs != 64 && gs != 128) return 0;
    if (K % gs) return 0;
    return 1;
}

/*
 * Affine group quantization, MLX `quantize(w, group_size, bits)` (affine mode), as called at
 * reference src/quant.rs:140, src/adapters.rs:533-537 (QuantizedLinear::try_from_linear) and
 * src/nn.rs:91-93, with the fixture produced by tools/dump_quant.py:25 and checked by
 * tests/quant_parity.rs:34-51.
 *
 * Per row n and per group g of `gs` consecutive elements along K:
 *   mx, mn   = max, min of the group
 *   s        = max((mx - mn) / (2^bits - 1), eps)            eps = 1e-7
 *   side     = |mn| > |mx|;  s = side ? s : -s;  edge = side ? mn : mx
 *   q0       = round(edge / s)
 *   s        = q0 != 0 ? edge / q0 : s;   bias = q0 != 0 ? edge : 0
 *   code[k]  = clamp(round((w[k] - bias) / s), 0, 2^bits - 1)
 * so one end of the group range (the larger-magnitude one) is reproduced exactly and the scale
 * may be negative.  Codes are computed from the f32 scale; the stored scale/bias are rounded to
 * the weight dtype (bf16 when sb_bf16).  Packing: 32/bits codes per uint32 word, element i of the
 * word at bit offset i*bits (low bits first); words row-major, K/(32/bits) words per row.
 * round() is half-away-from-zero (the Metal stdlib rule).
 */
int oracle_quantize(const float* w, int64_t N, int64_t K, int gs, int bits, int sb_bf16,
                    uint32_t* wq, float* scales, float* biases) {
    if (!valid_shape(N, K, gs, bits)) return ORACLE_EINVAL;
    const float eps = 1e-7f;
    const float nb = (float)((1 << bits) - 1);
    const int per = 32 / bits;
    const int64_t G = K / gs;
    const int64_t W = K / per;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t g = 0; g < G; ++g) {
            const float* src = w + n * K + g * gs;
            float mx = src[0], mn = src[0];
            for (int i = 1; i < gs; ++i) {
                mx = fmaxf(mx, src[i]);
                mn = fminf(mn, src[i]);
            }
            float s = fmaxf((mx - mn) / nb, eps);
            int side = fabsf(mn) > fabsf(mx);
            s = side ? s : -s;
            float edge = side ? mn : mx;
            float q0 = roundf(edge / s);
            int at_zero = (q0 == 0.0f);
            s = at_zero ? s : edge / q0;
            float bias = at_zero ? 0.0f : edge;
            scales[n * G + g] = rnd(s, sb_bf16);
            biases[n * G + g] = rnd(bias, sb_bf16);
            for (int i = 0; i < gs; i += per) {
                uint32_t word = 0;
                for (int j = 0; j < per; ++j) {
                    float v = roundf((src[i + j] - bias) / s);
                    v = fminf(fmaxf(v, 0.0f), nb);
                    word |= ((uint32_t)v) << (j * bits);
                }
                wq[n * W + (g * gs + i) / per] = word;
            }
        }
    }
    return ORACLE_OK;
}

static inline uint32_t code_at(const uint32_t* row, int64_t k, int bits) {
    const int per = 32 / bits;
    return (row[k / per] >> ((k % per) * bits)) & ((1u << bits) - 1u);
}

/*
 * MLX `dequantize(wq, scales, biases, group_size, bits)` (reference src/nn.rs:55,
 * mlx-gen-flux/src/text_encoder.rs:78): w = fma(code, scale, bias) in f32, rounded once, then to
 * the scales dtype (bf16 when out_bf16).  The single-rounding form is pinned by the fixture's
 * q*.deq (tests/quant_parity.rs:53-57).
 */
int oracle_dequantize(const uint32_t* wq, const float* scales, const float* biases, int64_t N,
                      int64_t K, int gs, int bits, int out_bf16, float* out) {
    if (!valid_shape(N, K, gs, bits)) return ORACLE_EINVAL;
    const int per = 32 / bits;
    const int64_t G = K / gs, W = K / per;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        const uint32_t* row = wq + n * W;
        for (int64_t k = 0; k < K; ++k) {
            float s = scales[n * G + k / gs], b = biases[n * G + k / gs];
            out[n * K + k] = rnd(fmaf((float)code_at(row, k, bits), s, b), out_bf16);
        }
    }
    return ORACLE_OK;
}

/*
 * MLX `quantized_matmul(x, wq, scales, biases, transpose=true, group_size, bits)` as called from
 * LinearBase::forward (reference src/adapters.rs:309-317): y[M,N] = x[M,K] . What[N,K]^T with
 * What = dequantize(...).  w_bf16 selects the dequantized-weight precision (1: each weight rounded
 * to bf16 as in a bf16-tile GEMM; 0: exact f32 fma as in the factored small-M form).  Products
 * are accumulated in double; out_bf16 rounds y to bf16 (activation dtype bf16), else y is rounded
 * to f32.
 */
int oracle_qmm(const float* x, int64_t M, int64_t K, const uint32_t* wq, const float* scales,
               const float* biases, int64_t N, int gs, int bits, int w_bf16, int out_bf16,
               float* y) {
    if (!valid_shape(N, K, gs, bits) || M < 0) return ORACLE_EINVAL;
    const int per = 32 / bits;
    const int64_t G = K / gs, W = K / per;
#pragma omp parallel
    {
        double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            const uint32_t* row = wq + n * W;
            for (int64_t k = 0; k < K; ++k) {
                float s = scales[n * G + k / gs], b = biases[n * G + k / gs];
                wrow[k] = (double)rnd(fmaf((float)code_at(row, k, bits), s, b), w_bf16);
            }
            for (int64_t m = 0; m < M; ++m) {
                const float* xr = x + m * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * wrow[k];
                y[m * N + n] = rnd((float)acc, out_bf16);
            }
        }
        free(wrow);
    }
    return ORACLE_OK;
}

/* Dense y[M,N] = x[M,K] . B[K,N] (row-major B), double accumulate, rounded per out_bf16. */
static void dense_mm(const float* x, int64_t M, int64_t K, const float* B, int64_t N, int out_bf16,
                     float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += (double)x[m * K + k] * (double)B[k * N + n];
            y[m * N + n] = rnd((float)acc, out_bf16);
        }
    }
}

/*
 * Exact-erf GELU, MLX `gelu` as applied in FLUX's FeedForward (reference
 * mlx-gen-flux/src/transformer.rs:975): 0.5 * v * (1 + erf(v / sqrt(2))), evaluated in double and
 * rounded to the activation dtype.
 */
float oracle_gelu_erf(float v, int out_bf16) {
    double d = (double)v;
    return rnd((float)(0.5 * d * (1.0 + erf(d / sqrt(2.0)))), out_bf16);
}

/*
 * Dtype-preserving exact GELU of reference src/nn.rs:344-355 (gelu_exact): the ops
 *   inner = erf(x / s2); gate = 1 + inner; y = (x * gate) / 2
 * with s2 = (float)sqrt(2) cast to the input dtype, every op's result rounded to it (bf16 when
 * out_bf16): each op is computed in f32 (correctly rounded: evaluated in double, then rounded to
 * float) and then rounded, as MLX's bf16 elementwise ops compute through float.
 */
float oracle_gelu_exact(float v, int out_bf16) {
    const float s2 = rnd((float)sqrt(2.0), out_bf16);
    const float t1 = rnd((float)((double)v / (double)s2), out_bf16);
    const float t2 = rnd((float)erf((double)t1), out_bf16);
    const float t3 = rnd((float)(1.0 + (double)t2), out_bf16);
    const float t4 = rnd((float)((double)v * (double)t3), out_bf16);
    return rnd((float)((double)t4 / 2.0), out_bf16);
}

/*
 * Tanh-approximate GELU of reference src/nn.rs:321-329 (FLUX single-stream FFN,
 * mlx-gen-flux/src/transformer.rs:506,708,979): the eager op sequence
 *   x3 = x^3; inner = (x + x3 * 0.044715) * c; gate = tanh(inner) + 1; y = (x * 0.5) * gate
 * with c = (float)sqrt(2/pi) taken in double, every constant cast to the activation dtype and every
 * op's result rounded to it.  The cube and tanh are evaluated in double, then rounded.
 */
float oracle_gelu_tanh(float v, int out_bf16) {
    const float c = rnd((float)sqrt(2.0 / 3.14159265358979323846), out_bf16);
    const float k = rnd(0.044715f, out_bf16);
    const double d = (double)v;
    const float x3 = rnd((float)(d * d * d), out_bf16);
    const float inner = rnd(rnd(v + rnd(x3 * k, out_bf16), out_bf16) * c, out_bf16);
    const float gate = rnd(rnd((float)tanh((double)inner), out_bf16) + 1.0f, out_bf16);
    return rnd(rnd(v * 0.5f, out_bf16) * gate, out_bf16);
}

/*
 * SiLU as the reference's two ops, multiply(v, sigmoid(v)) (src/nn.rs:301-303, used by the SwiGLU
 * of mlx-gen-sensenova/src/qwen3.rs:179): the sigmoid is computed in double, rounded to f32 (the
 * correctly rounded f32 sigmoid) and then to the activation dtype; the product of the two is
 * rounded to the activation dtype.
 */
float oracle_silu(float v, int out_bf16) {
    const double d = (double)v;
    const float sig = rnd((float)(1.0 / (1.0 + exp(-d))), out_bf16);
    return rnd(v * sig, out_bf16);
}

/*
 * AdaptableLinear::forward over a quantized base (reference src/adapters.rs:543-549 and the
 * quantized arm of LinearBase::forward, :300-322) under MLX's dtype promotion: each op computes
 * in the result type of its operands (bf16 only when all are bf16) and rounds to it.
 *   y0 = qmm(x)                    D0 = promote(x, scales)          (src/adapters.rs:309-317)
 *   y1 = y0 + bias   if bias       D1 = promote(D0, bias)           (:318-320)
 *   xa = x . A                     DR = promote(x, factors)         (Adapter::residual, :260-270;
 *   r  = xa . B                                                      A = lora_down^T, B = lora_up^T
 *   r2 = r * scale   scale cast to DR                                with alpha/rank folded in,
 *                                                                    src/adapters/loader.rs:568-599)
 *   y2 = y1 + r2     if lora       D2 = promote(D1, DR), not cast back (:243-252, :546)
 *   y  = act(y2)     act: 0 none; 1 mlx_rs::nn::gelu (exact erf in f32: its f32 constants
 *                    promote a bf16 input, mlx-gen-flux/src/transformer.rs:975, src/nn.rs:335-338);
 *                    2 tanh GELU per op in D2 (src/nn.rs:321-329); 3 exact GELU per op in D2
 *                    (src/nn.rs:344-355)
 * The activation is the caller's next op (FeedForward::forward, transformer.rs:970-977), listed
 * here so a fused epilogue has a checker.  w_bf16 as in oracle_qmm.  *out_bf16 receives whether
 * y's dtype is bf16.
 */
int oracle_linear(const float* x, int64_t M, int64_t K, const uint32_t* wq, const float* scales,
                  const float* biases, int64_t N, int gs, int bits, int w_bf16, int x_bf16,
                  int sb_bf16, const float* bias, int bias_bf16, const float* lora_a,
                  const float* lora_b, int64_t rank, int lora_bf16, float lora_scale, int act,
                  float* y, int* out_bf16) {
    const int lora = lora_a && lora_b && rank > 0;
    const int d0 = x_bf16 && sb_bf16;
    const int d1 = d0 && (!bias || bias_bf16);
    const int dr = x_bf16 && (!lora || lora_bf16);
    const int d2 = d1 && (!lora || dr);
    if (act < 0 || act > 3) return ORACLE_EINVAL;
    int rc = oracle_qmm(x, M, K, wq, scales, biases, N, gs, bits, w_bf16, d0, y);
    if (rc) return rc;
    if (bias) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < M * N; ++i) y[i] = rnd(y[i] + bias[i % N], d1);
    }
    if (lora) {
        float* xa = (float*)malloc(sizeof(float) * (size_t)(M * rank));
        float* r = (float*)malloc(sizeof(float) * (size_t)(M * N));
        if (!xa || !r) {
            free(xa);
            free(r);
            return ORACLE_EINVAL;
        }
        dense_mm(x, M, K, lora_a, rank, dr, xa);
        dense_mm(xa, M, rank, lora_b, N, dr, r);
        float sc = rnd(lora_scale, dr);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < M * N; ++i) y[i] = rnd(y[i] + rnd(r[i] * sc, dr), d2);
        free(xa);
        free(r);
    }
    if (act == 1) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < M * N; ++i) y[i] = oracle_gelu_erf(y[i], 0);
    } else if (act == 2) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < M * N; ++i) y[i] = oracle_gelu_tanh(y[i], d2);
    } else if (act == 3) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < M * N; ++i) y[i] = oracle_gelu_exact(y[i], d2);
    }
    if (out_bf16) *out_bf16 = d2 && act != 1;
    return ORACLE_OK;
}

/*
 * SwiGLU decode MLP of reference mlx-gen-sensenova/src/qwen3.rs:178-181:
 *   h = silu(gate(x)) * up(x)   (each op rounded to the activation dtype),  y = down(h).
 * gate/up are [F,K] packs; down is an [Nd,F] pack.  h [M,F] and y [M,Nd] are outputs.
 */
int oracle_swiglu_mlp(const float* x, int64_t M, int64_t K, const uint32_t* wq_g,
                      const float* s_g, const float* b_g, const uint32_t* wq_u, const float* s_u,
                      const float* b_u, int64_t F, const uint32_t* wq_d, const float* s_d,
                      const float* b_d, int64_t Nd, int gs, int bits, int w_bf16, int act_bf16,
                      float* h, float* y) {
    float* g = (float*)malloc(sizeof(float) * (size_t)(M * F));
    float* u = (float*)malloc(sizeof(float) * (size_t)(M * F));
    if (!g || !u) {
        free(g);
        free(u);
        return ORACLE_EINVAL;
    }
    int rc = oracle_qmm(x, M, K, wq_g, s_g, b_g, F, gs, bits, w_bf16, act_bf16, g);
    if (!rc) rc = oracle_qmm(x, M, K, wq_u, s_u, b_u, F, gs, bits, w_bf16, act_bf16, u);
    if (!rc) {
        for (int64_t i = 0; i < M * F; ++i)
            h[i] = rnd(oracle_silu(g[i], act_bf16) * u[i], act_bf16);
        rc = oracle_qmm(h, M, F, wq_d, s_d, b_d, Nd, gs, bits, w_bf16, act_bf16, y);
    }
    free(g);
    free(u);
    return rc;
}

/*
 * One LoKr adapter of AdaptableLinear::forward's residual sum (reference src/adapters.rs:543-549)
 * through Adapter::residual's Lokr arm (:263-266):
 *   d  = delta.as_dtype(x)          DX = x's dtype (bf16 when x_bf16)
 *   r  = x . d^T                    in DX (double accumulate, rounded once)
 *   r2 = r * scale                  scale cast to DX first (the dtype-matched scalar, :268-269)
 *   y  = y_in + r2                  in promote(y_in, DX)
 * delta [N,K] row-major (the reconstructed kron delta, :26-128).  *out_bf16 receives whether y's
 * dtype is bf16.
 */
int oracle_lokr_residual(const float* x, int64_t M, int64_t K, const float* delta, int64_t N,
                         float scale, int x_bf16, const float* y_in, int y_bf16, float* y,
                         int* out_bf16) {
    const int dout = y_bf16 && x_bf16;
    const float sc = rnd(scale, x_bf16);
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k)
                acc += (double)x[m * K + k] * (double)rnd(delta[n * K + k], x_bf16);
            const float r = rnd((float)acc, x_bf16);
            y[m * N + n] = rnd(y_in[m * N + n] + rnd(r * sc, x_bf16), dout);
        }
    }
    if (out_bf16) *out_bf16 = dout;
    return ORACLE_OK;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
