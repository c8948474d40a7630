"""Stacked-expert projection (the quantized MoE experts of mlx-gen-lens): mlxq_qmm_experts against
the oracle's per-expert linear (quantized_matmul + dense bias, mlx-gen-lens/src/text_encoder/
gpt_oss.rs:412-425), on the one-launch GEMM path and on the per-expert paths, and the stack/split
commutation of the packing that the stacked on-disk layout relies on (mlx-gen-lens/src/quant.rs:85-92).

Bars: bit-exact for packing; relFro <= 2e-3 and |delta| <= 1e-2*max|y| for the products.
"""
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


def _stack(rng, E, N, K, gs, bits):
    packs = [oracle.quantize(bf16_normal(rng, (N, K), 0.02), gs, bits, sb_bf16=True) for _ in range(E)]
    wq = np.stack([p[0] for p in packs])
    s = np.stack([p[1] for p in packs])
    b = np.stack([p[2] for p in packs])
    return packs, wq, s, b


def _check(mlxq, y, x, packs, bias, gs, bits, per_expert, w_bf16, rows=None, what=""):
    for e, p in enumerate(packs):
        xe = x[e] if per_expert else x
        sel = rows if rows is not None else np.arange(xe.shape[0])
        ref = oracle.linear(xe[sel], *p, gs, bits, w_bf16=w_bf16, act_bf16=True,
                            bias=None if bias is None else bias[e])
        assert_close(y[e][sel], ref, f"{what} expert {e}")


@pytest.mark.parametrize("per_expert,K", [(False, 512), (True, 512), (True, 2880)])
def test_experts_one_launch(mlxq, per_expert, K):
    """E = 8 experts of [2048, K] Q4 g64 at M = 512: 128 GEMM tiles, one launch over grid.y.
    K = 512 stages the scales in LDS blocks of 8 groups; K = 2880 (45 groups, the gpt-oss
    expert width) loads them per K step."""
    banner("experts one launch", per_expert, K)
    rng = np.random.default_rng(5 + per_expert + K)
    E, M, N, gs, bits = 8, 512, 2048, 64, 4
    packs, wq, s, b = _stack(rng, E, N, K, gs, bits)
    bias = bf16_normal(rng, (E, N), 0.5)
    x = bf16_normal(rng, (E, M, K) if per_expert else (M, K))
    y = to_np(mlxq.qmm_experts(to_gpu(x), wq_to_gpu(wq), to_gpu(s), to_gpu(b), gs, bits,
                               bias=to_gpu(bias), per_expert=per_expert))
    assert y.shape == (E, M, N)
    rows = np.concatenate([np.arange(8), rng.choice(M, 40, replace=False), [M - 1]])
    _check(mlxq, y, x, packs, bias, gs, bits, per_expert, w_bf16=True, rows=rows, what="one launch")


@pytest.mark.parametrize("M", [1, 4, 40])
def test_experts_per_expert_paths(mlxq, M):
    """Few, small experts: the GEMV (M <= 8) and the small GEMM, expert by expert, with bias."""
    banner("experts per-expert path", M)
    rng = np.random.default_rng(50 + M)
    E, N, K, gs, bits = 3, 72, 256, 128, 8
    packs, wq, s, b = _stack(rng, E, N, K, gs, bits)
    bias = bf16_normal(rng, (E, N), 0.5)
    x = bf16_normal(rng, (E, M, K))
    y = to_np(mlxq.qmm_experts(to_gpu(x), wq_to_gpu(wq), to_gpu(s), to_gpu(b), gs, bits,
                               bias=to_gpu(bias), per_expert=True))
    _check(mlxq, y, x, packs, bias, gs, bits, True, w_bf16=(M > 8), what=f"M={M}")


def test_experts_f32_activations(mlxq):
    """f32 activations and f32 bias: every op in f32, against the oracle's exact-f32 sequence."""
    banner("experts f32")
    rng = np.random.default_rng(61)
    E, M, N, K, gs, bits = 2, 6, 40, 128, 64, 4
    ws = [(rng.standard_normal((N, K)) * 0.02).astype(np.float32) for _ in range(E)]
    packs = [oracle.quantize(w, gs, bits) for w in ws]
    wq = np.stack([p[0] for p in packs])
    s = np.stack([p[1] for p in packs])
    b = np.stack([p[2] for p in packs])
    bias = rng.standard_normal((E, N)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = to_np(mlxq.qmm_experts(to_gpu(x, torch.float32), wq_to_gpu(wq), to_gpu(s, torch.float32),
                               to_gpu(b, torch.float32), gs, bits, bias=to_gpu(bias, torch.float32)))
    for e in range(E):
        ref = oracle.linear(x, *packs[e], gs, bits, w_bf16=False, act_bf16=False, bias=bias[e])
        assert errors(y[e], ref)[0] < 1e-5


def test_stacked_pack_split_matches_per_expert(mlxq):
    """Packing the stack [E*out, in] on the GPU is byte-identical to packing each expert (affine
    quantization is per row), so the stacked triple splits back into the per-expert packs
    (mlx-gen-lens/src/quant.rs:85-92); StackedExperts.forward equals the split layers' forwards."""
    banner("stacked pack split")
    rng = np.random.default_rng(70)
    E, N, K, gs, bits = 4, 96, 512, 64, 4
    w = bf16_normal(rng, (E, N, K), 0.02)
    wq_s, s_s, b_s = mlxq.quantize(to_gpu(w.reshape(E * N, K)), gs, bits)
    for e in range(E):
        wq_e, s_e, b_e = mlxq.quantize(to_gpu(w[e]), gs, bits)
        assert torch.equal(wq_s[e * N:(e + 1) * N], wq_e)
        assert torch.equal(s_s[e * N:(e + 1) * N], s_e) and torch.equal(b_s[e * N:(e + 1) * N], b_e)
    bias = to_gpu(bf16_normal(rng, (E, N), 0.5))
    st = mlxq.StackedExperts(wq_s.reshape(E, N, -1), s_s.reshape(E, N, -1), b_s.reshape(E, N, -1),
                             bias, gs, bits)
    x = to_gpu(bf16_normal(rng, (2, 5, K)))
    y = st.forward(x)
    assert y.shape == (E, 2, 5, N)
    for e, layer in enumerate(st.split()):
        assert_close(to_np(y[e]), to_np(layer.forward(x)), f"split expert {e}")


def test_experts_empty_and_mismatch(mlxq):
    rng = np.random.default_rng(80)
    packs, wq, s, b = _stack(rng, 2, 16, 128, 64, 4)
    x = to_gpu(bf16_normal(rng, (0, 128)))
    assert mlxq.qmm_experts(x, wq_to_gpu(wq), to_gpu(s), to_gpu(b), 64, 4).shape == (2, 0, 16)
    with pytest.raises(mlxq.MlxqError, match="lead with E"):
        mlxq.qmm_experts(to_gpu(bf16_normal(rng, (3, 4, 128))), wq_to_gpu(wq), to_gpu(s), to_gpu(b),
                         64, 4, per_expert=True)
