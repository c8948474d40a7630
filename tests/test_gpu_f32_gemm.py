"""GPU parity of the f32 large-M GEMM (qmm_f32.hip): operands MLX computes in f32 at M > 8.

FLUX.1's residual stream is f32 (mlx-gen-flux/src/model.rs:407-410) and quantized_matmul takes the
activations as they come (src/adapters.rs:301-317), so an f32 x against bf16 (or f32) scales is
an f32 product: x, scales and biases cast to f32, weights dequantized in f32, f32 accumulation.
The kernel carries both operands as two-term bf16 splits and adds three bf16 MFMA products.  The
checks hold it to the exact f32 oracle (fp64 over the f32-dequantized weights) at relFro < 1e-4,
and to at least ten times closer than the same product with x rounded to bf16 — what a single
bf16 pass would give — so a missing correction pass fails them.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, banner, errors, to_gpu, to_np, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _tdt(name):
    return torch.float32 if name == "f32" else torch.bfloat16


# (M, N, K, gs, bits, x dtype, scales dtype): ragged M and N (N % 4 != 0), every group size,
# Q4 and Q8, f32 or bf16 scales, bf16 x against f32 scales, the M = 9 boundary.  Group sizes 64
# and 128 run the factored kernel; with bf16 scales and K / gs a multiple of 16 its bias term goes
# through the batched MFMA (the last four cases: one, three, two and one 16-group batches, the
# last at the M = 9 boundary).
CASES = [
    (200, 198, 512, 64, 4, "f32", "bf16"),
    (130, 264, 1024, 32, 8, "f32", "f32"),
    (300, 128, 768, 128, 4, "bf16", "f32"),
    (9, 64, 256, 64, 4, "f32", "bf16"),
    (513, 1000, 384, 128, 8, "f32", "bf16"),
    (256, 256, 96, 32, 4, "f32", "bf16"),
    (200, 262, 1024, 64, 4, "f32", "bf16"),
    (137, 300, 3072, 64, 8, "f32", "bf16"),
    (260, 520, 4096, 128, 4, "f32", "bf16"),
    (9, 100, 1024, 64, 4, "f32", "bf16"),
]


@pytest.mark.parametrize("M,N,K,gs,bits,xdt,sdt", CASES)
def test_f32_gemm_vs_exact_oracle(mlxq, M, N, K, gs, bits, xdt, sdt):
    banner("f32 gemm", M, N, K, gs, bits, xdt, sdt)
    rng = np.random.default_rng(M * 3 + N + K + bits + gs)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if xdt == "bf16":
        x = oracle.bf16_round(x)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if sdt == "bf16":
        w = oracle.bf16_round(w)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=(sdt == "bf16"))
    y = mlxq.quantized_matmul(to_gpu(x, _tdt(xdt)), wq_to_gpu(rwq), to_gpu(rs, _tdt(sdt)),
                              to_gpu(rb, _tdt(sdt)), True, gs, bits)
    assert y.dtype == torch.float32
    ref = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=False, out_bf16=False)
    rel, peak = errors(to_np(y), ref)
    print(f"    relFro={rel:.3e} peak={peak:.3e}", flush=True)
    assert rel < 1e-4 and peak < 1e-3
    if xdt == "f32":
        one_pass = oracle.quantized_matmul(oracle.bf16_round(x), rwq, rs, rb, gs, bits, w_bf16=True,
                                           out_bf16=False)
        assert rel * 10 < errors(one_pass, ref)[0]


@pytest.mark.parametrize("act", [0, 1, 3])
def test_f32_flux_mlp_up_every_tile_band(mlxq, act):
    """The FLUX.1 f32 stream at config-2 size: x [4608, 3072] f32 through a Q4-g64 [12288, 3072]
    linear with an f32 bias and mlx_rs::nn::gelu (act 1) or the exact GELU in f32 (act 3), checked
    on two rows of every 128-row tile band (all 12288 columns) against the oracle's f32 linear."""
    banner("f32 flux up", act)
    rng = np.random.default_rng(4608 + act)
    M, K, N = 4608, 3072, 12288
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = oracle.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    y = mlxq.linear(to_gpu(x, torch.float32), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), 64, 4,
                    bias=to_gpu(bias, torch.float32), activation=act)
    assert y.dtype == torch.float32
    rows = np.concatenate([np.arange(0, M, 128), np.arange(127, M, 128)])
    rows.sort()
    got = y[torch.from_numpy(rows).to(y.device)].cpu().numpy()
    ref = oracle.linear(x[rows], rwq, rs, rb, 64, 4, w_bf16=False, act_bf16=False, bias=bias, act=act,
                        sb_bf16=True)
    rel, peak = assert_close(got, ref, f"f32 flux up act={act}")
    assert rel < 1e-4


@pytest.mark.parametrize("act", [0, 1, 2, 3])
@pytest.mark.parametrize("bias_dt", ["f32", "bf16", None])
def test_f32_fused_epilogue_matches_elementwise(mlxq, act, bias_dt):
    """The f32 GEMM applies the bias and the activation before its store; a LoRA adapter sends the
    same linear through the product followed by the elementwise epilogue kernel instead.  With a
    zero B factor the residual adds exactly 0.0 in f32, so both routes must agree bit for bit
    (bias in either dtype, every activation), and both must match the oracle's f32 linear."""
    banner("f32 fused epilogue", act, bias_dt)
    rng = np.random.default_rng(77 + act)
    M, K, N = 200, 512, 262
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = oracle.bf16_round((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    bias = None
    if bias_dt is not None:
        bias = (rng.standard_normal(N) * 0.5).astype(np.float32)
        if bias_dt == "bf16":
            bias = oracle.bf16_round(bias)
    gb = None if bias is None else to_gpu(bias, _tdt(bias_dt))
    args = (to_gpu(x, torch.float32), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), 64, 4)
    fused = mlxq.linear(*args, bias=gb, activation=act)
    la = to_gpu((rng.standard_normal((K, 4)) * 0.1).astype(np.float32), torch.float32)
    lb = torch.zeros((4, N), dtype=torch.float32, device=la.device)
    split = mlxq.linear(*args, bias=gb, lora_a=la, lora_b=lb, lora_scale=1.0, activation=act)
    assert fused.dtype == torch.float32 and split.dtype == torch.float32
    assert torch.equal(fused, split), "fused f32 epilogue differs from the elementwise epilogue"
    ref = oracle.linear(x, rwq, rs, rb, 64, 4, w_bf16=False, act_bf16=False, bias=bias, act=act,
                        sb_bf16=True, bias_bf16=(bias_dt == "bf16"))
    rel, peak = assert_close(to_np(fused), ref, f"f32 fused epilogue act={act} bias={bias_dt}")
    assert rel < 1e-4
