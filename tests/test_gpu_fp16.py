"""fp16 activations over bf16-packed weights: SDXL's quantized path.

SDXL runs its U-Net, both CLIP text encoders and its ControlNets in fp16
(mlx-gen-sdxl/src/model.rs:216,226,250-251,260-263) and quantizes them with
AdaptableLinear::quantize (:283-296), which casts each weight and bias to bf16 before packing
(src/adapters.rs:508-537).  LinearBase::forward hands the activations to quantized_matmul as they
are (src/adapters.rs:300-317), so an fp16 x meets bf16 scales and MLX computes the product in
promote(fp16, bf16) = f32: x widened exactly, weights dequantized in f32, f32 result, and every
later op of the linear (bias, LoRA residual, activation) in f32 too.

Checks, through the C ABI: the product at SDXL U-Net and CLIP shapes (M > 8 on the f32 matrix-core
GEMM, M <= 8 on the f32 GEMV) against the exact f32 oracle, held ten times closer than the same
product with x rounded to bf16; the fused linear (bf16 bias, exact-erf GELU, a bf16 LoRA adapter)
against the oracle's op sequence in f32; stacked experts; and the entry points that do not take
fp16 reporting MLXQ_EUNSUPPORTED or MLXQ_EINVAL without running anything.
"""
import numpy as np
import pytest
import torch

from gpu_util import banner, errors, to_gpu, to_np, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _fp16_normal(rng, shape, std=1.0):
    return oracle.fp16_round((rng.standard_normal(shape) * std).astype(np.float32))


def _packed(rng, N, K, gs, bits):
    w = oracle.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    return oracle.quantize(w, gs, bits, sb_bf16=True)


def _gpu(t):
    rwq, rs, rb = t
    return wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb)


# (M, K, N, gs, bits): SDXL at 1024^2 — CLIP-L (hidden 768, MLP 3072) and CLIP-G (1280 / 5120)
# over 77 tokens; U-Net transformer blocks at 32x32 (1024 tokens, 1280 channels, GEGLU 10240) and
# 64x64 latents (4096 tokens, 640 channels); a ragged shape; then decode-size M <= 8.
SDXL_CASES = [
    (77, 768, 3072, 64, 4),
    (77, 1280, 5120, 64, 8),
    (77, 5120, 1280, 128, 4),
    (1024, 1280, 1280, 64, 4),
    (1024, 1280, 10240, 64, 8),
    (4096, 640, 640, 32, 4),
    (300, 640, 2500, 128, 8),
    (1, 1280, 1280, 64, 4),
    (2, 768, 3072, 64, 8),
    (5, 640, 300, 128, 4),
    (8, 2048, 640, 32, 4),
]


@pytest.mark.parametrize("M,K,N,gs,bits", SDXL_CASES)
def test_fp16_x_quantized_matmul_vs_exact_f32(mlxq, M, K, N, gs, bits):
    banner("fp16 qmm", M, K, N, gs, bits)
    rng = np.random.default_rng(M + 3 * K + N + gs + bits)
    x = _fp16_normal(rng, (M, K))
    pk = _packed(rng, N, K, gs, bits)
    y = mlxq.quantized_matmul(to_gpu(x, torch.float16), *_gpu(pk), True, gs, bits)
    assert y.dtype == torch.float32  # promote(fp16, bf16)
    ref = oracle.quantized_matmul(x, *pk, gs, bits, w_bf16=False, out_bf16=False)
    rel, peak = errors(to_np(y), ref)
    bf16_x = oracle.quantized_matmul(oracle.bf16_round(x), *pk, gs, bits, w_bf16=False, out_bf16=False)
    rel16, _ = errors(bf16_x, ref)
    print(f"    relFro={rel:.3e} peak={peak:.3e} (x rounded to bf16: {rel16:.3e})", flush=True)
    assert rel < 2e-5 and peak < 2e-4
    assert rel < rel16 / 10


@pytest.mark.parametrize("M,K,N,act", [(77, 768, 3072, 3), (1024, 640, 1000, 1), (4, 1280, 640, 3)])
def test_fp16_x_linear_bias_gelu(mlxq, M, K, N, act):
    """bias (bf16, as AdaptableLinear::quantize leaves it) and the GELU all in f32."""
    banner("fp16 linear", M, K, N, act)
    rng = np.random.default_rng(M + K + N + act)
    x = _fp16_normal(rng, (M, K))
    pk = _packed(rng, N, K, 64, 4)
    bias = oracle.bf16_round((rng.standard_normal(N) * 0.5).astype(np.float32))
    y = mlxq.linear(to_gpu(x, torch.float16), *_gpu(pk), 64, 4, bias=to_gpu(bias), activation=act)
    assert y.dtype == torch.float32
    ref, ref_bf16 = oracle.linear(x, *pk, 64, 4, w_bf16=False, x_bf16=False, sb_bf16=True, bias=bias,
                                  bias_bf16=True, act=act, return_dtype=True)
    assert not ref_bf16
    rel, peak = errors(to_np(y), ref)
    print(f"    relFro={rel:.3e} peak={peak:.3e}", flush=True)
    assert rel < 2e-5 and peak < 2e-4


@pytest.mark.parametrize("M", [3, 600])
def test_fp16_x_linear_lora(mlxq, M):
    """A bf16 rank-16 LoRA adapter on an fp16 stream: the residual in promote(fp16, bf16) = f32."""
    banner("fp16 linear lora", M)
    K, N, r = 640, 520, 16
    rng = np.random.default_rng(M + 17)
    x = _fp16_normal(rng, (M, K))
    pk = _packed(rng, N, K, 64, 4)
    A = oracle.bf16_round((rng.standard_normal((K, r)) * 0.05).astype(np.float32))
    B = oracle.bf16_round((rng.standard_normal((r, N)) * 0.05).astype(np.float32))
    y = mlxq.linear(to_gpu(x, torch.float16), *_gpu(pk), 64, 4, lora_a=to_gpu(A), lora_b=to_gpu(B),
                    lora_scale=0.75)
    assert y.dtype == torch.float32
    ref = oracle.linear(x, *pk, 64, 4, w_bf16=False, x_bf16=False, sb_bf16=True, lora_a=A, lora_b=B,
                        lora_bf16=True, lora_scale=0.75)
    rel, peak = errors(to_np(y), ref)
    print(f"    relFro={rel:.3e} peak={peak:.3e}", flush=True)
    assert rel < 2e-5 and peak < 2e-4


def test_fp16_x_stacked_experts(mlxq):
    banner("fp16 experts")
    rng = np.random.default_rng(23)
    E, M, K, N = 3, 40, 256, 192
    x = _fp16_normal(rng, (M, K))
    packs = [_packed(rng, N, K, 64, 4) for _ in range(E)]
    wq = torch.stack([wq_to_gpu(p[0]) for p in packs])
    s = torch.stack([to_gpu(p[1]) for p in packs])
    b = torch.stack([to_gpu(p[2]) for p in packs])
    y = mlxq.qmm_experts(to_gpu(x, torch.float16), wq, s, b, 64, 4)
    assert y.dtype == torch.float32 and tuple(y.shape) == (E, M, N)
    for e, p in enumerate(packs):
        ref = oracle.quantized_matmul(x, *p, 64, 4, w_bf16=False, out_bf16=False)
        rel, peak = errors(to_np(y[e]), ref)
        assert rel < 2e-5 and peak < 2e-4, (e, rel, peak)


def test_fp16_outside_the_activation_role_is_refused(mlxq):
    """fp16 where the library does not take it: status, nothing launched."""
    banner("fp16 refused")
    rng = np.random.default_rng(29)
    x16 = to_gpu(_fp16_normal(rng, (4, 256)), torch.float16)
    pk = _gpu(_packed(rng, 128, 256, 64, 4))
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.quantize(torch.zeros((64, 256), dtype=torch.float16, device="cuda"), 64, 4)
    assert e.value.status == mlxq._lib.MLXQ_EUNSUPPORTED
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.swiglu(x16, pk, pk, 64, 4)
    assert e.value.status == mlxq._lib.MLXQ_EUNSUPPORTED
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.qmm(x16, *pk, 64, 4)
    assert e.value.status == mlxq._lib.MLXQ_EINVAL
    y = torch.zeros((4, 128), dtype=torch.float32, device="cuda")
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.lokr_residual(x16, y, torch.zeros((128, 256), dtype=torch.bfloat16, device="cuda"))
    assert e.value.status == mlxq._lib.MLXQ_EUNSUPPORTED
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.quantized_matmul(x16, pk[0], pk[1].half(), pk[2].half(), True, 64, 4)
    assert e.value.status == mlxq._lib.MLXQ_EUNSUPPORTED
