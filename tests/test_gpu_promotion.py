"""GPU parity of MLX's dtype promotion at the fused seams and of the bf16 GELU tables.

The reference keeps a LoRA adapter's factors and a dense bias in their file dtype, so a bf16
product meeting an f32 bias or f32 factors promotes to f32 (src/adapters.rs:243-252,318-320,546),
and FLUX's mlx_rs::nn::gelu returns f32 for a bf16 input (mlx-gen-flux/src/transformer.rs:975,
src/nn.rs:335-338).  Every case checks the result dtype against the oracle's promotion and the
values against the oracle (relFro <= 2e-3 and |delta| <= 1e-2 max|y|; f32 paths far inside).

The GELU tables: the fused bf16 epilogues look the activation up in a 65536-entry table of the
reference's per-op bf16 GELU.  A GEMM whose weight picks column 0 of x (code 1 at k = 0, scale 1,
bias 0: the product is x[:, 0] exactly, -0 becoming +0) feeds every bf16 bit pattern through each
GEMM kernel's epilogue, and every output is compared bit for bit with the oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, banner, bf16_normal, errors, to_gpu, to_np, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


# ---------------------------------------------------------------- GELU tables, every bf16 input

def _selector_pack(N, K, gs):
    """Packed Q4 weights whose dequantized rows are e_0 (code 1 at k = 0, scale 1, bias 0)."""
    wq = np.zeros((N, K // 8), np.uint32)
    wq[:, 0] = 1
    s = np.ones((N, K // gs), np.float32)
    b = np.zeros((N, K // gs), np.float32)
    return wq, s, b


def _expected(fn, vals):
    return np.array([fn(float(v)) for v in vals], dtype=np.float32)


def _plus_zero(vals):
    with np.errstate(invalid="ignore"):
        return vals + np.float32(0.0)


def _same_bits(got, want):
    both_nan = np.isnan(got) & np.isnan(want)
    return (got.view(np.uint32) == want.view(np.uint32)) | both_nan


@pytest.mark.parametrize("act", [3, 2])
@pytest.mark.parametrize("kernel,K,gs,chunk", [
    ("wide", 64, 64, 65536),    # 256 tiles of 256 x 256: the wide kernel's LDS table copy
    ("tile", 32, 32, 65536),    # K % 64 != 0: the tile kernel, table read from global memory
    ("small", 512, 64, 8192),   # 64 x 64 K-split kernel (8 launches of 8192 rows)
])
def test_bf16_gelu_table_every_input(mlxq, act, kernel, K, gs, chunk):
    banner("gelu table", act, kernel)
    N = 64 if kernel != "wide" else 256
    bits = np.arange(65536, dtype=np.uint32)
    vals = (bits << 16).view(np.float32)
    fn = oracle.gelu_exact if act == 3 else oracle.gelu_tanh
    # The pre-activation is the sum x*1 + 0*0 + ...: x itself, except that -0 + 0 is +0.
    want = _expected(fn, _plus_zero(vals))
    wq, s, b = _selector_pack(N, K, gs)
    gw, gs_, gb = wq_to_gpu(wq), to_gpu(s), to_gpu(b)
    mism = 0
    for m0 in range(0, 65536, chunk):
        x = np.zeros((chunk, K), np.float32)
        x[:, 0] = vals[m0:m0 + chunk]
        xb = torch.from_numpy(x).to("cuda").to(torch.bfloat16)  # exact: every value is bf16
        y = mlxq.linear(xb, gw, gs_, gb, gs, 4, activation=act)
        torch.cuda.synchronize()
        got = y.float().cpu().numpy()
        assert got.dtype == np.float32 and y.dtype == torch.bfloat16
        for n in (0, N - 1):
            mism += int((~_same_bits(got[:, n], want[m0:m0 + chunk])).sum())
    print(f"    {kernel} act={act}: {mism} mismatches over 65536 inputs x 2 columns")
    assert mism == 0


def test_bf16_gelu_table_through_the_elementwise_epilogue(mlxq):
    """M <= 8 (GEMV + elementwise epilogue): every finite bf16 input with |x| < 2^60, as 8 rows
    times an identity weight with group size 32, which the VALU GEMV evaluates as
    s * sum(x c) + b * sum(x) with s = 1, b = 0: exactly x (the group sums stay finite)."""
    banner("gelu table, elementwise epilogue")
    bits = np.arange(65536, dtype=np.uint32)
    vals = (bits << 16).view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) < 2.0 ** 60)]
    K = 8192
    rows = int(np.ceil(vals.size / K))
    x = np.zeros((rows * K,), np.float32)
    x[:vals.size] = vals
    x = x.reshape(rows, K)
    # W = identity [K, K]: row n has code 1 at k = n (scale 1, bias 0)
    wq = np.zeros((K, K // 8), np.uint32)
    idx = np.arange(K)
    wq[idx, idx // 8] = np.left_shift(np.uint32(1), (4 * (idx % 8)).astype(np.uint32))
    s = np.ones((K, K // 32), np.float32)
    b = np.zeros((K, K // 32), np.float32)
    gw, gs_, gb = wq_to_gpu(wq), to_gpu(s), to_gpu(b)
    for act, fn in ((3, oracle.gelu_exact), (2, oracle.gelu_tanh)):
        got = np.empty_like(x)
        for r0 in range(0, rows, 8):
            xb = torch.from_numpy(x[r0:r0 + 8]).to("cuda").to(torch.bfloat16)
            y = mlxq.linear(xb, gw, gs_, gb, 32, 4, activation=act)
            got[r0:r0 + 8] = y.float().cpu().numpy()
        got = got.reshape(-1)[:vals.size]
        want = _expected(fn, _plus_zero(vals))  # -0 + 0 = +0 in the sum
        mism = int((~_same_bits(got, want)).sum())
        print(f"    elementwise act={act}: {mism} mismatches over {vals.size} inputs")
        assert mism == 0


# ---------------------------------------------------------------- promotion at the seams

def _pack(rng, N, K, gs=64, bits=4):
    w = bf16_normal(rng, (N, K), 0.02)
    wq, s, b = oracle.quantize(w, gs, bits, sb_bf16=True)
    return (wq, s, b), (wq_to_gpu(wq), to_gpu(s), to_gpu(b))


@pytest.mark.parametrize("M", [4, 300, 2100])
@pytest.mark.parametrize("bias_dt,lora_dt,act,rank", [
    ("f32", None, 0, 16),        # f32 bias: y0 bf16 + bias f32 -> f32
    (None, "f32", 0, 16),        # f32 factors (the reference's golden LoRA files)
    ("bf16", "bf16", 1, 16),     # mlx_rs::nn::gelu on a bf16 pre-activation -> f32
    ("f32", "bf16", 2, 16),      # bf16 residual into an f32 sum, tanh GELU in f32
    ("bf16", "f32", 3, 24),      # f32 factors at rank 24, exact GELU in f32
    ("bf16", "bf16", 0, 16),     # all bf16: no promotion, the fused path
])
def test_linear_promotion(mlxq, M, bias_dt, lora_dt, act, rank):
    banner("linear promotion", M, bias_dt, lora_dt, act, rank)
    rng = np.random.default_rng(M + rank + act + (bias_dt == "f32") * 7)
    K, N = 512, 4200 if M == 2100 else 520
    x = bf16_normal(rng, (M, K))
    (rwq, rs, rb), g = _pack(rng, N, K)
    kw, okw = {}, {}
    if bias_dt:
        bias = rng.standard_normal(N).astype(np.float32) * 0.5
        if bias_dt == "bf16":
            bias = oracle.bf16_round(bias)
        kw["bias"] = to_gpu(bias, torch.bfloat16 if bias_dt == "bf16" else torch.float32)
        okw.update(bias=bias, bias_bf16=bias_dt == "bf16")
    if lora_dt:
        A = (rng.standard_normal((K, rank)) * 0.05).astype(np.float32)
        B = (rng.standard_normal((rank, N)) * 0.05).astype(np.float32)
        if lora_dt == "bf16":
            A, B = oracle.bf16_round(A), oracle.bf16_round(B)
        tdt = torch.bfloat16 if lora_dt == "bf16" else torch.float32
        kw.update(lora_a=to_gpu(A, tdt), lora_b=to_gpu(B, tdt), lora_scale=0.75)
        okw.update(lora_a=A, lora_b=B, lora_scale=0.75, lora_bf16=lora_dt == "bf16")
    y = mlxq.linear(to_gpu(x), *g, 64, 4, activation=act, **kw)
    ref, out_bf16 = oracle.linear(x, rwq, rs, rb, 64, 4, w_bf16=M > 8, act_bf16=True, act=act,
                                  return_dtype=True, **okw)
    assert y.dtype == (torch.bfloat16 if out_bf16 else torch.float32), (y.dtype, out_bf16)
    assert y.dtype == mlxq.ops.linear_out_dtype(torch.bfloat16, torch.bfloat16,
                                                None if not bias_dt else (torch.bfloat16 if bias_dt == "bf16" else torch.float32),
                                                None if not lora_dt else (torch.bfloat16 if lora_dt == "bf16" else torch.float32),
                                                act)
    assert_close(to_np(y), ref, f"promotion M={M} bias={bias_dt} lora={lora_dt} act={act}")


@pytest.mark.parametrize("M", [3, 40, 700])
def test_quantized_matmul_f32_scales_promote(mlxq, M):
    """bf16 x with f32 scales: MLX casts x to f32 and returns f32 with the exact f32 dequant."""
    banner("qmm f32 scales promote", M)
    rng = np.random.default_rng(M)
    K, N = 384, 264
    x = bf16_normal(rng, (M, K))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    rwq, rs, rb = oracle.quantize(w, 64, 8)
    y = mlxq.quantized_matmul(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs, torch.float32),
                              to_gpu(rb, torch.float32), True, 64, 8)
    assert y.dtype == torch.float32
    ref = oracle.quantized_matmul(x, rwq, rs, rb, 64, 8, w_bf16=False, out_bf16=False)
    assert errors(to_np(y), ref)[0] < 1e-5


def test_lora_residual_promotes_out_of_place(mlxq):
    banner("lora_residual promotion")
    rng = np.random.default_rng(5)
    M, K, N, r = 70, 256, 300, 8
    x = bf16_normal(rng, (M, K))
    y = bf16_normal(rng, (M, N))
    A = (rng.standard_normal((K, r)) * 0.05).astype(np.float32)
    B = (rng.standard_normal((r, N)) * 0.05).astype(np.float32)
    gy = to_gpu(y)
    out = mlxq.ops.lora_residual(to_gpu(x), gy, to_gpu(A, torch.float32), to_gpu(B, torch.float32), 1.5)
    assert out.dtype == torch.float32 and out.data_ptr() != gy.data_ptr()
    ref = (y.astype(np.float64) + ((x.astype(np.float64) @ A.astype(np.float64)).astype(np.float32)
                                   .astype(np.float64) @ B.astype(np.float64)) * 1.5)
    assert errors(to_np(out), ref)[0] < 1e-5
    assert torch.equal(gy, to_gpu(y)), "y_in changed"
    # bf16 factors on bf16 y: in place
    Ab, Bb = oracle.bf16_round(A), oracle.bf16_round(B)
    out2 = mlxq.ops.lora_residual(to_gpu(x), gy, to_gpu(Ab), to_gpu(Bb), 1.5)
    assert out2.dtype == torch.bfloat16 and out2.data_ptr() == gy.data_ptr()
    rr = oracle.bf16_round((oracle.bf16_round((x.astype(np.float64) @ Ab).astype(np.float32))
                            .astype(np.float64) @ Bb).astype(np.float32))
    want = oracle.bf16_round(y + oracle.bf16_round(rr * np.float32(1.5)))
    assert_close(to_np(out2), want, "lora_residual bf16 in place")


def test_adaptable_linear_mixed_adapter_stack(mlxq):
    """Python AdaptableLinear over a quantized base with an f32 bias (as a converted snapshot keeps
    it), a bf16 adapter and an f32 adapter: every adapter in the library, sums promoted."""
    banner("AdaptableLinear mixed stack")
    rng = np.random.default_rng(8)
    M, K, N = 260, 512, 384
    x = bf16_normal(rng, (M, K))
    (rwq, rs, rb), g = _pack(rng, N, K)
    bias = (rng.standard_normal(N) * 0.3).astype(np.float32)
    A1, B1 = bf16_normal(rng, (K, 16), 0.05), bf16_normal(rng, (16, N), 0.05)
    A2 = (rng.standard_normal((K, 8)) * 0.05).astype(np.float32)
    B2 = (rng.standard_normal((8, N)) * 0.05).astype(np.float32)
    layer = mlxq.AdaptableLinear.from_quantized_parts(g[0], g[1], g[2], to_gpu(bias, torch.float32), 64, 4)
    layer.push(mlxq.Adapter(to_gpu(A1), to_gpu(B1), 0.5))
    layer.push(mlxq.Adapter(to_gpu(A2, torch.float32), to_gpu(B2, torch.float32), 2.0))
    y = layer.forward(to_gpu(x))
    assert y.dtype == torch.float32
    ref = oracle.linear(x, rwq, rs, rb, 64, 4, w_bf16=True, act_bf16=True, bias=bias, bias_bf16=False,
                        lora_a=A1, lora_b=B1, lora_scale=0.5)
    xa2 = (x.astype(np.float64) @ A2).astype(np.float32)
    ref = ref + ((xa2.astype(np.float64) @ B2).astype(np.float32) * np.float32(2.0))
    assert_close(to_np(y), ref, "mixed adapter stack")


def test_experts_bias_promotion_rules(mlxq):
    banner("experts bias promotion")
    rng = np.random.default_rng(3)
    E, M, K, N = 2, 20, 256, 96
    packs = [oracle.quantize(bf16_normal(rng, (N, K), 0.02), 64, 4, sb_bf16=True) for _ in range(E)]
    wq = torch.stack([wq_to_gpu(p[0]) for p in packs])
    s = torch.stack([to_gpu(p[1]) for p in packs])
    b = torch.stack([to_gpu(p[2]) for p in packs])
    x = bf16_normal(rng, (M, K))
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.qmm_experts(to_gpu(x), wq, s, b, 64, 4, bias=torch.zeros((E, N), device="cuda"))
    assert e.value.status == 2
    # f32 activations: D0 is f32 already and a bf16 bias adds into it.
    bias = bf16_normal(rng, (E, N), 0.5)
    xf = rng.standard_normal((M, K)).astype(np.float32)
    y = mlxq.qmm_experts(to_gpu(xf, torch.float32), wq, s, b, 64, 4, bias=to_gpu(bias))
    assert y.dtype == torch.float32
    for ex in range(E):
        ref = oracle.linear(xf, *packs[ex], 64, 4, w_bf16=False, act_bf16=False, bias=bias[ex])
        assert errors(to_np(y[ex]), ref)[0] < 1e-5


def test_noalloc_promoted_result(mlxq):
    """mlxq_linear_noalloc stages a promoted product in its static scratch when it fits, and
    rejects one that does not."""
    from mlxq import _lib
    banner("noalloc promoted")
    lib = _lib.load()
    rng = np.random.default_rng(2)
    M, K, N = 300, 512, 1000
    x = bf16_normal(rng, (M, K))
    (rwq, rs, rb), g = _pack(rng, N, K)
    bias = (rng.standard_normal(N) * 0.3).astype(np.float32)
    gb = to_gpu(bias, torch.float32)
    want = mlxq.linear(to_gpu(x), *g, 64, 4, bias=gb)
    assert want.dtype == torch.float32
    y = torch.empty_like(want)
    ep = _lib.Epilogue(gb.data_ptr(), None, None, 0, 1.0, 0, _lib.MLXQ_FLOAT32, _lib.MLXQ_BFLOAT16)
    gx = to_gpu(x)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.mlxq_linear_noalloc(gx.data_ptr(), 1, M, K, g[0].data_ptr(), g[1].data_ptr(),
                                       g[2].data_ptr(), 1, N, 64, 4, ctypes.byref(ep), y.data_ptr(), st))
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    big_m = (_lib.MLXQ_NOALLOC_SCRATCH_BYTES // (2 * N)) + 64
    st2 = lib.mlxq_linear_noalloc(gx.data_ptr(), 1, big_m, K, g[0].data_ptr(), g[1].data_ptr(),
                                  g[2].data_ptr(), 1, N, 64, 4, ctypes.byref(ep), y.data_ptr(), st)
    assert st2 == _lib.MLXQ_EINVAL and b"static buffer" in lib.mlxq_last_error()
