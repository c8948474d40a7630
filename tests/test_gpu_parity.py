"""GPU parity: libmlxq_hip.so (through its C ABI) against the CPU oracle and the reference's golden.

Mirrors the reference's tests/quant_parity.rs (byte-level packing parity, dequant and
quantized_matmul within tolerance) and extends it to bf16 inputs, all six (bits, group_size)
pairs, both kernels (MFMA GEMM, GEMV), ragged shapes and the fused linear epilogue.
Bars: bit-exact for quantize / dequantize; relFro <= 2e-3 and |delta| <= 1e-2*max|y| for matmuls.
"""
import os

import numpy as np
import pytest
import torch
from safetensors.numpy import load_file

from gpu_util import (assert_close, banner, bf16_normal, errors, to_gpu, to_np, wq_to_gpu)
from oracle import oracle

pytestmark = pytest.mark.gpu

GOLD = load_file(os.path.join(os.path.dirname(__file__), "golden", "quant_q4q8.safetensors"))


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


# ---------------------------------------------------------------- golden (tests/quant_parity.rs)

@pytest.mark.parametrize("bits", [8, 4])
def test_golden_quantize_dequantize_qmm(mlxq, bits):
    banner("golden f32 fixture", f"bits={bits}")
    w = to_gpu(GOLD["w"], torch.float32)
    wq, s, b = mlxq.quantize(w, 64, bits)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(wq), GOLD[f"q{bits}.wq"])
    assert np.array_equal(to_np(s), GOLD[f"q{bits}.scales"])
    assert np.array_equal(to_np(b), GOLD[f"q{bits}.biases"])
    deq = mlxq.dequantize(wq, s, b, 64, bits)
    assert np.array_equal(to_np(deq), GOLD[f"q{bits}.deq"])
    x = to_gpu(GOLD["x"], torch.float32)
    y = to_np(mlxq.quantized_matmul(x, wq, s, b, True, 64, bits))
    ref = GOLD[f"q{bits}.qmm"]
    # tests/quant_parity.rs:59-64 (rtol=atol=1e-2); the f32 kernel is far inside it.
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- quantize / dequantize

QUANT_CASES = [
    # (N, K, gs, bits)
    (96, 256, 32, 4), (96, 256, 64, 4), (96, 256, 128, 4),
    (96, 256, 32, 8), (96, 256, 64, 8), (96, 256, 128, 8),
    (1, 64, 64, 4), (3, 128, 128, 8), (257, 96, 32, 4),
]


@pytest.mark.parametrize("N,K,gs,bits", QUANT_CASES)
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_quantize_bit_exact(mlxq, N, K, gs, bits, dtype):
    banner("quantize", dtype, N, K, gs, bits)
    rng = np.random.default_rng(N * 7 + K + gs + bits)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if dtype == "bf16":
        w = oracle.bf16_round(w)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    wq, s, b = mlxq.quantize(to_gpu(w, tdt), gs, bits)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=(dtype == "bf16"))
    assert np.array_equal(to_np(wq), rwq)
    assert np.array_equal(to_np(s), rs)
    assert np.array_equal(to_np(b), rb)
    deq = to_np(mlxq.dequantize(wq, s, b, gs, bits))
    assert np.array_equal(deq, oracle.dequantize(rwq, rs, rb, gs, bits, out_bf16=(dtype == "bf16")))


# mlxq_quantize_batched: several weights of one shape per launch (up to 16; 17 takes two launches),
# bit for bit what one quantize per weight gives, and the oracle's packing for the first weight.
@pytest.mark.parametrize("count,N,K,gs,bits,dtype", [(1, 40, 256, 64, 4, "bf16"), (4, 640, 5120, 64, 8, "bf16"),
                                                     (17, 33, 384, 128, 4, "bf16"), (3, 257, 96, 32, 8, "f32"),
                                                     (5, 1, 64, 64, 4, "f32"), (16, 96, 1024, 32, 4, "bf16")])
def test_quantize_batched_matches_per_weight(mlxq, count, N, K, gs, bits, dtype):
    banner("quantize batched", count, N, K, gs, bits, dtype)
    rng = np.random.default_rng(count * 31 + N + K + gs + bits)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    ws = [(rng.standard_normal((N, K)) * 0.02 * (i + 1)).astype(np.float32) for i in range(count)]
    if dtype == "bf16":
        ws = [oracle.bf16_round(w) for w in ws]
    gws = [to_gpu(w, tdt) for w in ws]
    got = mlxq.quantize_batched(gws, gs, bits)
    assert len(got) == count
    for gw, (wq, s, b) in zip(gws, got):
        rwq, rs, rb = mlxq.quantize(gw, gs, bits)
        assert torch.equal(wq, rwq) and torch.equal(s, rs) and torch.equal(b, rb)
    owq, os_, ob = oracle.quantize(ws[0], gs, bits, sb_bf16=(dtype == "bf16"))
    assert np.array_equal(to_np(got[0][0]), owq)
    assert np.array_equal(to_np(got[0][1]), os_) and np.array_equal(to_np(got[0][2]), ob)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_special_groups(mlxq, bits):
    """Zero, constant, all-negative, tiny-range and huge-range groups."""
    banner("quantize special groups", bits)
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((6, 512)) * 0.02).astype(np.float32)
    w[0, :64] = 0.0
    w[1, 64:128] = 0.375
    w[2, :] = -np.abs(w[2, :]) - 0.01
    w[3, 128:192] = 1e-9 * rng.standard_normal(64)
    w[4, 192:256] *= 1e4
    w[5, ::2] = 0.0
    w = oracle.bf16_round(w)
    wq, s, b = mlxq.quantize(to_gpu(w), 64, bits)
    rwq, rs, rb = oracle.quantize(w, 64, bits, sb_bf16=True)
    assert np.array_equal(to_np(wq), rwq)
    assert np.array_equal(to_np(s), rs)
    assert np.array_equal(to_np(b), rb)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_quantize_narrow_groups_far_from_zero(mlxq, bits, dtype):
    """Groups whose range is tiny next to their magnitude (|bias / scale| up to ~1e7): the code
    of w is (w - bias) / scale, and any evaluation that loses w - bias to cancellation in large
    terms would misround codes here."""
    banner("quantize narrow far groups", bits, dtype)
    rng = np.random.default_rng(12 + bits)
    rows = []
    for centre in (100.0, -3.0e3, 0.5, 7.25e4, -1.0):
        for width in (1e-2, 3e-4, 1e-5):
            rows.append(centre + width * rng.random(512))
    w = np.stack(rows).astype(np.float32)
    if dtype == "bf16":
        w = oracle.bf16_round(w)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    wq, s, b = mlxq.quantize(to_gpu(w, tdt), 64, bits)
    rwq, rs, rb = oracle.quantize(w, 64, bits, sb_bf16=(dtype == "bf16"))
    assert np.array_equal(to_np(wq), rwq)
    assert np.array_equal(to_np(s), rs)
    assert np.array_equal(to_np(b), rb)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_quantize_half_integer_ties(mlxq, bits, dtype):
    """Groups whose quotients (w - bias)/s land exactly on half-integers, and one ulp either side.

    With min 0 and max nb*d (d a power of two) the scale is -d and the bias nb*d exactly, so
    w = (k + 0.5) d gives the quotient nb - k - 0.5: a tie, which MLX's round() sends away from
    zero.  These are the codes the kernel recomputes with an exact division."""
    banner("quantize ties", bits, dtype)
    nb = (1 << bits) - 1
    gs = 64
    rows = []
    for e in (-6, -3, 0, 2):
        d = np.float32(2.0 ** e)
        k = np.arange(gs - 2) % nb
        ties = ((k + 0.5) * d).astype(np.float32)
        for nudge in (0, 1, -1):  # exact ties, then one ulp above and below
            w = ties.copy()
            if nudge:
                w = np.nextafter(w, np.float32(np.inf) if nudge > 0 else np.float32(-np.inf)).astype(np.float32)
            rows.append(np.concatenate([[0.0, nb * d], w]).astype(np.float32))
    w = np.stack(rows)
    if dtype == "bf16":
        w = oracle.bf16_round(w)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    wq, s, b = mlxq.quantize(to_gpu(w, tdt), gs, bits)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=(dtype == "bf16"))
    assert np.array_equal(to_np(wq), rwq)
    assert np.array_equal(to_np(s), rs)
    assert np.array_equal(to_np(b), rb)


def test_quantize_config1_full_size(mlxq):
    """Config 1: W [3072,3072] bf16 ~ N(0,0.02), seed 0, Q4 g64 — bit-exact against the oracle."""
    banner("quantize config1 [3072,3072] q4 g64")
    rng = np.random.default_rng(0)
    w = bf16_normal(rng, (3072, 3072), 0.02)
    wq, s, b = mlxq.quantize(to_gpu(w), 64, 4)
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    assert np.array_equal(to_np(wq), rwq)
    assert np.array_equal(to_np(s), rs) and np.array_equal(to_np(b), rb)
    deq = to_np(mlxq.dequantize(wq, s, b, 64, 4))
    assert np.array_equal(deq, oracle.dequantize(rwq, rs, rb, 64, 4, out_bf16=True))


# ---------------------------------------------------------------- GEMM (MFMA, bf16 tiles)

GEMM_CASES = [
    # (M, K, N, gs, bits).  With K >= 512 and at most 1152 64x64 tiles the K-split kernel
    # (qmm_small) runs unless the wide kernel has 128 tiles of 256x256 or 256x128; shorter K
    # takes the tile kernel.  qmm_small stages bf16 scales in LDS blocks of 8 groups when
    # K / gs % 8 == 0 (waves whose K range starts mid-block, 4/8/16 steps per block) and loads
    # them per step otherwise (K / gs = 45 and 12 below).
    (256, 3072, 3072, 64, 4),   # config 1 shape
    (64, 256, 128, 64, 4),
    (200, 320, 136, 32, 4),     # ragged M, N; K % 64 == 0
    (77, 96, 40, 32, 8),        # K % 64 == 32, tiny N
    (300, 512, 520, 128, 8),
    (129, 384, 264, 64, 8),
    (9, 256, 256, 32, 4),       # smallest GEMM M
    (600, 1024, 1280, 64, 4),
    (16, 3072, 3072, 64, 4),
    (512, 2048, 1000, 32, 8),   # ragged N
    (130, 4096, 2056, 128, 4),  # ragged M and N
    (96, 1024, 704, 32, 4),     # 4 steps per block, 2 steps per wave
    (64, 6144, 1024, 128, 8),   # 16 steps per block, 12 per wave
    (100, 2880, 1088, 64, 4),   # K / gs = 45: per-step scale loads
    (40, 1536, 520, 128, 4),    # K / gs = 12: per-step scale loads
    (1000, 1024, 2000, 64, 8),  # 512 small tiles
    (2048, 1024, 3072, 64, 4),  # 1536 small tiles: wide kernel, 256x128 tiles
]


@pytest.mark.parametrize("M,K,N,gs,bits", GEMM_CASES)
def test_qmm_gemm_vs_oracle(mlxq, M, K, N, gs, bits):
    banner("qmm gemm", M, K, N, gs, bits)
    rng = np.random.default_rng(M + K + N)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=True)
    y = to_np(mlxq.qmm(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), gs, bits))
    ref = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=True, out_bf16=True)
    assert_close(y, ref, f"gemm M={M} K={K} N={N} gs={gs} b={bits}")


WIDE_CASES = [
    # Shapes with >= 128 256x256 tiles take the wide kernel.  With K / group_size a multiple of
    # 8, bf16 scales/biases are staged in LDS in blocks of 8 groups: cases cover 1..3 scale
    # blocks, ragged M and N, and both tile heights (on 256 CUs the one-round cases run 256-row
    # tiles, the two-round cases marked 224 run 224-row tiles).  Otherwise (marked "regs") each
    # K step loads its scales into registers, 256-row tiles, odd and even step counts.
    (2304, 512, 4096, 64, 4),    # one block
    (2000, 256, 4136, 32, 8),    # ragged M and N, one block of 4 steps
    (2048, 2048, 4096, 128, 4),  # two blocks of 16 steps
    (2304, 512, 8192, 64, 8),    # 224
    (2000, 768, 8400, 32, 4),    # 224, ragged, three blocks of 4 steps
    (512, 1024, 32768, 64, 4),
    (500, 512, 32768, 32, 8),
    (2304, 256, 4096, 64, 4),    # regs, K / gs = 4, 4 steps
    (512, 2880, 8192, 64, 4),    # regs, K / gs = 45 (the gpt-oss expert width), 45 steps
    (1000, 192, 8200, 32, 8),    # regs, ragged, K / gs = 6, 3 steps
    # Under 128 256x256 tiles but at least 128 of 256x128 (4 waves, "narrow"):
    (1536, 3072, 3072, 64, 4),   # narrow, 144 tiles
    (600, 1024, 6000, 32, 8),    # narrow, ragged M and N
    (1030, 512, 4100, 64, 4),    # narrow, N % 8 != 0: direct stores
    (1030, 576, 4097, 64, 4),    # narrow, N % 4 != 0: element stores, K / gs = 9: regs
    # Under 128 of those but at least 136 tiles of 128x128 (4 waves, 128-row ring, "mid"):
    (1024, 3072, 3072, 64, 4),   # mid, 192 tiles
    (768, 1024, 3072, 32, 8),    # mid, 144 tiles
    (1000, 512, 3000, 128, 4),   # mid, ragged M and N
    (1030, 576, 2049, 64, 4),    # mid, N % 4 != 0: element stores, K / gs = 9: regs
]
@pytest.mark.parametrize("M,K,N,gs,bits", WIDE_CASES)
def test_qmm_wide_vs_oracle(mlxq, M, K, N, gs, bits):
    banner("qmm wide", M, K, N, gs, bits)
    rng = np.random.default_rng(M + K + N + bits)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=True)
    y = to_np(mlxq.qmm(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), gs, bits))
    ref = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=True, out_bf16=True)
    assert_close(y, ref, f"wide M={M} K={K} N={N} gs={gs} b={bits}")


@pytest.mark.parametrize("M,K,N,gs,bits", [(2048, 192, 4096, 64, 4), (2048, 64, 4096, 32, 4),
                                           (2100, 320, 4352, 64, 8), (2048, 512, 4096, 128, 8),
                                           (1024, 256, 4096, 64, 4), (1024, 256, 3072, 64, 4),
                                           (1000, 320, 3000, 64, 8), (128, 1024, 512, 64, 4),
                                           (200, 768, 300, 32, 8)])
def test_qmm_wide_f32_scales(mlxq, M, K, N, gs, bits):
    """bf16 activations with f32 scales/biases: the wide kernel's register-loaded scale path,
    any K % 64 == 0 (K/64 = 3, 1, 5 and 8 steps cover both prologue parities), its 256x128
    form (M = 1024, N = 4096), its 128x128 form (N = 3072 and the ragged 1000 x 3000) and the
    K-split kernel's per-step scale loads (M = 128, 200)."""
    banner("qmm wide f32 scales", M, K, N, gs, bits)
    rng = np.random.default_rng(M + K + N + 7 * bits)
    x = bf16_normal(rng, (M, K))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    rwq, rs, rb = oracle.quantize(w, gs, bits)
    assert rs.dtype == np.float32
    y = to_np(mlxq.qmm(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs, torch.float32), to_gpu(rb, torch.float32),
                       gs, bits))
    ref = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=True, out_bf16=True)
    assert_close(y, ref, f"wide f32 scales M={M} K={K} N={N} gs={gs} b={bits}")


# Grids that fill their last round of CUs poorly, with every epilogue: checked on sampled rows
# (each output row depends only on its input row; the samples include every 256-row tile
# boundary) and bit-identical on a rerun.
ODD_GRID_CASES = [
    # M, K, N, gs, bits, act, bias
    (2304, 4096, 4096, 64, 4, 0, False),   # 144 tiles: one round at 56 %
    (2304, 1024, 4096, 64, 8, 3, True),    # bias + exact GELU
    (1000, 2048, 6000, 32, 4, 2, True),    # ragged M and N (256x128 tiles), tanh GELU
    (4608, 3072, 4352, 64, 4, 0, False),   # 357 224-row tiles: two rounds at 70 %
]


@pytest.mark.parametrize("M,K,N,gs,bits,act,bias", ODD_GRID_CASES)
def test_qmm_odd_grids(mlxq, M, K, N, gs, bits, act, bias):
    banner("odd grid", M, K, N, gs, bits, act, bias)
    rng = np.random.default_rng(M + K + N + act)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    bv = bf16_normal(rng, (N,), 0.5) if bias else None
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=True)
    args = (to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), gs, bits)
    kw = dict(bias=to_gpu(bv) if bias else None, activation=act)
    y1 = mlxq.linear(*args, **kw)
    y2 = mlxq.linear(*args, **kw)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "result differs between runs"
    edges = [r for t in range(0, M, 256) for r in (t, t + 255) if r < M]
    rows = np.unique(np.concatenate([edges, rng.choice(M, 24, replace=False), [M - 1]]))
    ref = oracle.linear(x[rows], rwq, rs, rb, gs, bits, w_bf16=True, act_bf16=True, bias=bv, act=act)
    assert_close(to_np(y1)[rows], ref, f"odd grid M={M} K={K} N={N}")


@pytest.mark.parametrize("M,N", [(2100, 4200), (1100, 4200), (2100, 4100), (1024, 3000)])
@pytest.mark.parametrize("act,scale", [(0, 1.0), (3, 1.0), (2, 1.0), (0, 0.75), (3, 1.5)])
def test_linear_wide_bias_lora_act(mlxq, act, scale, M, N):
    """Fused bias + LoRA + activation epilogue on 256x256 tiles (M = 2100), on 256x128 tiles
    with 4 waves (M = 1100: 85 wide tiles, 165 narrow ones), on 128x128 tiles (M = 1024,
    N = 3000: 96 narrow tiles, 192 of 128x128) and with ragged N (4100), with LoRA
    scales other than 1 (their product rounding runs only then)."""
    banner("linear wide epilogue", act, scale, M, N)
    rng = np.random.default_rng(77 + act + M + N)
    K, r = 512, 16
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    bias = bf16_normal(rng, (N,), 0.5)
    A = bf16_normal(rng, (K, r), 0.01)
    B = bf16_normal(rng, (r, N), 0.01)
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    y = to_np(mlxq.linear(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), 64, 4,
                          bias=to_gpu(bias), lora_a=to_gpu(A), lora_b=to_gpu(B), lora_scale=scale,
                          activation=act))
    ref = oracle.linear(x, rwq, rs, rb, 64, 4, w_bf16=True, act_bf16=True, bias=bias,
                        lora_a=A, lora_b=B, lora_scale=scale, act=act)
    assert_close(y, ref, f"linear wide act={act} scale={scale}")


# Every bias / LoRA / LoRA-scale / activation combination of the wide kernel's epilogue: without
# an activation each combination has its own compile-time pass, with a GELU the terms are runtime
# conditions and a launch with neither term skips the first pass (the lookup rounds the products).
@pytest.mark.parametrize("bias,lora,scale,act", [
    (True, False, 1.0, 0), (False, True, 1.0, 0), (False, True, 0.5, 0), (True, True, 1.0, 0),
    (True, True, 0.5, 0), (False, False, 1.0, 3), (True, False, 1.0, 3), (False, True, 0.5, 3),
    (True, True, 1.5, 2)])
@pytest.mark.parametrize("M,N", [(2048, 4096), (1024, 3000)])
def test_linear_wide_epilogue_combinations(mlxq, bias, lora, scale, act, M, N):
    """256x256 tiles of 8 waves (M = 2048, N = 4096: 128 tiles) and 128x128 tiles of 4 waves
    (M = 1024, N = 3000, ragged N), sampled rows in every tile band against the oracle."""
    banner("linear wide epilogue combination", bias, lora, scale, act, M, N)
    rng = np.random.default_rng(M + N + 7 * act + (3 if bias else 0) + (5 if lora else 0) + int(4 * scale))
    K, r = 512, 16
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    bv = bf16_normal(rng, (N,), 0.5) if bias else None
    A = bf16_normal(rng, (K, r), 0.01) if lora else None
    B = bf16_normal(rng, (r, N), 0.01) if lora else None
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    kw = {}
    if bias:
        kw["bias"] = to_gpu(bv)
    if lora:
        kw.update(lora_a=to_gpu(A), lora_b=to_gpu(B), lora_scale=scale)
    y = to_np(mlxq.linear(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), 64, 4, activation=act, **kw))
    rows = _band_rows(rng, M, heights=(128, 256))
    okw = {"bias": bv} if bias else {}
    if lora:
        okw.update(lora_a=A, lora_b=B, lora_scale=scale)
    ref = oracle.linear(x[rows], rwq, rs, rb, 64, 4, w_bf16=True, act_bf16=True, act=act, **okw)
    assert_close(y[rows], ref, f"wide epilogue bias={bias} lora={lora} scale={scale} act={act}")


def _band_rows(rng, M, heights=(224, 256)):
    """At least one row in every M-tile band of each tile height (a random row per band, plus the
    band edges of the first and last bands)."""
    rows = {0, M - 1}
    for h in heights:
        for t in range(0, M, h):
            hi = min(t + h, M)
            rows.add(int(rng.integers(t, hi)))
        rows.update({min(h, M - 1), min(h - 1, M - 1)})
    return np.array(sorted(rows))


def test_flux_mlp_full_size_all_rows(mlxq):
    """Config 2 at full size, every output element against the OpenMP oracle: the up projection
    with the dtype-preserving exact GELU fused (a bf16 stream), then the down projection."""
    banner("config2 full size: up+gelu, down, all rows")
    M, K, F = 4608, 3072, 12288
    rng = np.random.default_rng(0)
    x = bf16_normal(rng, (M, K))
    wu = bf16_normal(rng, (F, K), 0.02)
    wd = bf16_normal(rng, (K, F), 0.02)
    qu = oracle.quantize(wu, 64, 4, sb_bf16=True)
    qd = oracle.quantize(wd, 64, 4, sb_bf16=True)
    gu = [wq_to_gpu(qu[0]), to_gpu(qu[1]), to_gpu(qu[2])]
    gd = [wq_to_gpu(qd[0]), to_gpu(qd[1]), to_gpu(qd[2])]
    h = mlxq.linear(to_gpu(x), *gu, 64, 4, activation=mlxq.MLXQ_ACT_GELU_EXACT)
    y = mlxq.quantized_matmul(h, *gd, True, 64, 4)
    torch.cuda.synchronize()
    assert h.dtype == torch.bfloat16 and y.dtype == torch.bfloat16
    h_np = to_np(h)
    assert np.isfinite(h_np).all()
    ref_h = oracle.linear(x, *qu, 64, 4, w_bf16=True, act_bf16=True, act=3)
    assert_close(h_np, ref_h, "config2 up+gelu, all rows")
    del ref_h
    ref_y = oracle.quantized_matmul(h_np, *qd, 64, 4, w_bf16=True, out_bf16=True)
    assert_close(to_np(y), ref_y, "config2 down, all rows")


def test_qmm_dispatch_matches_forced_kernels(mlxq):
    banner("dispatch")
    rng = np.random.default_rng(5)
    w = bf16_normal(rng, (256, 512), 0.02)
    wq, s, b = mlxq.quantize(to_gpu(w), 64, 4)
    for M, forced in ((8, mlxq.qmv), (9, mlxq.qmm), (64, mlxq.qmm), (1, mlxq.qmv)):
        x = to_gpu(bf16_normal(rng, (M, 512)))
        a = mlxq.quantized_matmul(x, wq, s, b, True, 64, 4)
        c = forced(x, wq, s, b, 64, 4)
        assert torch.equal(a, c), M


# ---------------------------------------------------------------- GEMV (exact f32 dequant)

@pytest.mark.parametrize("M", [1, 2, 4, 8, 3])
@pytest.mark.parametrize("K,N,gs,bits", [(3072, 512, 64, 4), (256, 96, 32, 8), (384, 40, 128, 4)])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_qmv_vs_oracle(mlxq, M, K, N, gs, bits, dtype):
    banner("qmv", dtype, M, K, N, gs, bits)
    rng = np.random.default_rng(M * 1000 + K + N)
    x = bf16_normal(rng, (M, K))
    if dtype == "f32":
        x = rng.standard_normal((M, K)).astype(np.float32)
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=True)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    y = to_np(mlxq.qmv(to_gpu(x, tdt), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), gs, bits))
    ref = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=False, out_bf16=(dtype == "bf16"))
    rel, peak = assert_close(y, ref, f"gemv {dtype} M={M}")
    if dtype == "f32":
        assert rel < 1e-5


@pytest.mark.parametrize("M", [1, 2, 4, 8])
@pytest.mark.parametrize("K,N,gs,bits", [(3072, 8192, 64, 4), (8192, 3072, 64, 4), (512, 2064, 64, 8),
                                         (1024, 520, 128, 8), (192, 17, 64, 4), (320, 33, 64, 8),
                                         (640, 45, 128, 4), (512, 40, 64, 4), (256, 24, 128, 8)])
def test_qmv_config4_shapes(mlxq, M, K, N, gs, bits):
    """Config 4 decode shapes (gate/up [8192,3072], down [3072,8192]) plus Q8 and ragged N.

    (192,17), (320,33), (640,45) have an odd number of bf16 scales in total, so the final scale
    sits in a half-filled dword at the end of its buffer; (512,40) and (256,24) run on a one-wave
    workgroup, where 64 threads store the 16*M outputs."""
    banner("qmv config4", M, K, N, gs, bits)
    rng = np.random.default_rng(M * 31 + K + N + bits)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=True)
    y = to_np(mlxq.quantized_matmul(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), True, gs, bits))
    ref = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=False, out_bf16=True)
    assert_close(y, ref, f"qmv M={M} K={K} N={N} gs={gs} b={bits}")


def _close_to_exact(y, ref, what):
    """Every output within one bf16 ulp of the exact result plus 1e-4 of the largest output: the
    f32 accumulation of the factored form stays orders of magnitude inside that, while a dropped
    column, a misplaced scale or a wrong group index moves outputs by percent."""
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    bound = ulp + 1e-4 * np.abs(ref).max()
    worst = float((np.abs(y.astype(np.float64) - ref) / bound).max())
    print(f"    {what} worst |delta| / (ulp + 1e-4 max) = {worst:.3f}", flush=True)
    assert worst <= 1.0, what


# Q4, K a multiple of 1024: at M = 1 the one-row-per-wave kernel (K from 1 to 16 loads per row,
# N not a multiple of the 8/12/16 rows of a workgroup, N below one workgroup); M = 2..4 run the
# 16-row tile kernel on the same shapes, held to the same bound.
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N,gs", [(1024, 77, 64), (3072, 8192, 128), (5120, 1000, 64), (8192, 3072, 128),
                                    (16384, 40, 64), (16384, 24, 128), (2048, 5, 64), (7168, 2051, 64)])
def test_qmv_one_row_kernel_vs_exact(mlxq, M, K, N, gs):
    banner("qmv one row", M, K, N, gs)
    rng = np.random.default_rng(K + 3 * N + gs + 101 * M)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, 4, sb_bf16=True)
    y = to_np(mlxq.quantized_matmul(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), True, gs, 4))
    exact = oracle.quantized_matmul(x, rwq, rs, rb, gs, 4, w_bf16=False, out_bf16=False)
    _close_to_exact(y, exact, f"one-row M={M} K={K} N={N} gs={gs}")
    assert_close(y, oracle.bf16_round(exact), f"one-row M={M} K={K} N={N} gs={gs}")


# Biases far below their scales: every code 0, scales +-1, biases 2^-40 .. 2^-20, so each output is
# sum_g b_g * X_g alone.  The GEMVs fold s * sum(x * c) + b * X with the codes as exact bf16 values,
# so the bias term keeps its own precision; a fold through an offset code (128 + c, with
# b - 128 s) would round the bias away entirely.  One-row kernel (M = 1, Q4 g64/g128), tile
# kernel (M = 2, 8, Q4 g32 and Q8), held to the one-ulp bound of the exact product.
@pytest.mark.parametrize("M", [1, 2, 8])
@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 128), (4, 32), (8, 64)])
def test_qmv_bias_far_below_scale(mlxq, M, bits, gs):
    banner("qmv small bias", M, bits, gs)
    K, N = 3072, 520
    rng = np.random.default_rng(7 * M + bits + gs)
    x = bf16_normal(rng, (M, K))
    rwq = np.zeros((N, K * bits // 32), dtype=np.uint32)
    rs = oracle.bf16_round(rng.choice([-1.0, 1.0], size=(N, K // gs)).astype(np.float32))
    rb = oracle.bf16_round((np.exp2(rng.uniform(-40, -20, size=(N, K // gs)))
                            * rng.choice([-1.0, 1.0], size=(N, K // gs))).astype(np.float32))
    y = to_np(mlxq.quantized_matmul(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), True, gs, bits))
    exact = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=False, out_bf16=False)
    assert np.abs(exact).max() < 1e-3  # the outputs are the bias terms alone
    _close_to_exact(y, exact, f"small bias M={M} Q{bits} gs={gs}")


@pytest.mark.parametrize("K,N,gs", [(1152, 33, 64), (11008, 300, 64), (8960, 257, 128), (13824, 130, 64),
                                    (18944, 100, 64), (29568, 48, 64), (32768, 40, 128), (2560, 4097, 128)])
def test_qmv_one_row_kernel_ragged_k(mlxq, K, N, gs):
    """M = 1, Q4, K not a multiple of 1024 (an even group count per row), up to 32 loads per row:
    the last load of a row is partial, its upper columns reach into the next row's codes (past the
    buffer's end for the last row) and must fold exactly zero.  The activation row sits in a longer
    buffer whose tail past K is NaN, so a read past K shows in every output."""
    banner("qmv one row ragged K", K, N, gs)
    rng = np.random.default_rng(K + 5 * N + gs)
    x = bf16_normal(rng, (1, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, 4, sb_bf16=True)
    xbig = torch.full((1, K + 2048), float("nan"), dtype=torch.bfloat16, device="cuda")
    xbig[:, :K] = to_gpu(x)
    y = to_np(mlxq.quantized_matmul(xbig[:, :K], wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), True, gs, 4))
    exact = oracle.quantized_matmul(x, rwq, rs, rb, gs, 4, w_bf16=False, out_bf16=False)
    _close_to_exact(y, exact, f"one-row ragged K={K} N={N} gs={gs}")
    assert_close(y, oracle.bf16_round(exact), f"one-row ragged K={K} N={N} gs={gs}")


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("K,N,gs,bits", [(11008, 300, 64, 4), (14336, 257, 64, 4), (8960, 130, 128, 4),
                                         (16384, 64, 128, 4), (24576, 40, 64, 4), (1088, 70, 64, 8),
                                         (18944, 33, 64, 4), (11008, 200, 64, 8), (4224, 90, 128, 8)])
def test_qmv_tile_kernel_long_and_ragged_k(mlxq, M, K, N, gs, bits):
    """M = 2..8 (and Q8 at M = 1) where K's load steps have no even split over the tile kernel's
    waves or exceed one register round: the last wave's range runs past K (K = 11008, 8960 and the
    Q8 K = 1088, 4224), waves take two rounds of their load registers (M = 3..8 at K = 11008 /
    14336 / 16384, M = 2 at 18944 and 24576, Q8 K = 11008), and rows that fit no plan go out as
    launches of four rows (M = 5, 8 at K = 11008 / 14336) or two rows (M = 3..8 at K = 18944 and
    24576).  Q4 at M = 1 runs the one-row kernel on the same shapes.  The activations sit in a
    longer buffer whose tail is NaN, so a read past M x K shows, and a read past K within a row
    takes the next row's values and moves the result."""
    banner("qmv tile long / ragged K", M, K, N, gs, bits)
    rng = np.random.default_rng(M * 13 + K + 7 * N + gs + bits)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=True)
    xbig = torch.full((M * K + 4096,), float("nan"), dtype=torch.bfloat16, device="cuda")
    xbig[:M * K] = to_gpu(x).reshape(-1)
    xg = xbig[:M * K].view(M, K)
    y = to_np(mlxq.quantized_matmul(xg, wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), True, gs, bits))
    exact = oracle.quantized_matmul(x, rwq, rs, rb, gs, bits, w_bf16=False, out_bf16=False)
    _close_to_exact(y, exact, f"tile long K M={M} K={K} N={N} gs={gs} b={bits}")
    assert_close(y, oracle.bf16_round(exact), f"tile long K M={M} K={K} N={N} gs={gs} b={bits}")


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("K,N,bits", [(3072, 300, 4), (8192, 130, 4), (11008, 70, 4), (14336, 40, 4),
                                      (512, 33, 4), (16384, 24, 4), (3072, 200, 8), (8192, 64, 8),
                                      (4160, 90, 8)])
def test_qmv_group32_on_matrix_cores(mlxq, M, K, N, bits):
    """Group 32 on the tile kernel (it ran the VALU GEMV before).  Q4: each lane quarter's 16
    bytes are one whole group, and a 4 x 4 transpose of (quarter, word) by permlane swaps puts
    each MFMA on one group; exact splits (K = 3072, 8192, 512), the ragged last wave (11008), two
    register rounds (11008, 14336, 16384) and launches of two rows (M >= 3 at K >= 11008).  Q8:
    each lane half holds one group and two half swaps regroup the word pairs (K = 4160 ragged)."""
    banner("qmv group 32", M, K, N, bits)
    rng = np.random.default_rng(M * 5 + K + N + 32 + bits)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, 32, bits, sb_bf16=True)
    y = to_np(mlxq.quantized_matmul(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), True, 32, bits))
    exact = oracle.quantized_matmul(x, rwq, rs, rb, 32, bits, w_bf16=False, out_bf16=False)
    _close_to_exact(y, exact, f"group 32 M={M} K={K} N={N} b={bits}")
    assert_close(y, oracle.bf16_round(exact), f"group 32 M={M} K={K} N={N} b={bits}")


@pytest.mark.parametrize("M", [1, 2, 4, 8])
@pytest.mark.parametrize("K,F,bits", [(3072, 200, 4), (8192, 64, 4), (5120, 100, 4), (3072, 96, 8)])
def test_swiglu_group32(mlxq, M, K, F, bits):
    """The fused SwiGLU launch with group 32 (two-row launches at M >= 3 for Q4 K = 8192)."""
    banner("swiglu group 32", M, K, F, bits)
    rng = np.random.default_rng(M + K + F + 32 + bits)
    x = bf16_normal(rng, (M, K))
    tg, tu = [oracle.quantize(bf16_normal(rng, (F, K), 0.02), 32, bits, sb_bf16=True) for _ in range(2)]
    h = to_np(mlxq.swiglu(to_gpu(x), [wq_to_gpu(tg[0]), to_gpu(tg[1]), to_gpu(tg[2])],
                          [wq_to_gpu(tu[0]), to_gpu(tu[1]), to_gpu(tu[2])], 32, bits))
    gr = oracle.quantized_matmul(x, *tg, 32, bits, w_bf16=False, out_bf16=True)
    ur = oracle.quantized_matmul(x, *tu, 32, bits, w_bf16=False, out_bf16=True)
    ref = oracle.bf16_round(oracle.bf16_round(np.vectorize(oracle.silu)(gr).astype(np.float32)) * ur)
    assert_close(h, ref, f"swiglu group 32 M={M} K={K} F={F}")
    print(f"    bit-identical outputs: {np.mean(h == ref) * 100:.2f} %", flush=True)
    assert np.mean(h == ref) > 0.99


@pytest.mark.parametrize("M", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("K,F,gs,bits", [(5120, 300, 64, 4), (7168, 130, 64, 4), (12288, 40, 128, 4),
                                         (20480, 24, 64, 4), (6144, 48, 128, 8)])
def test_swiglu_tile_kernel_long_and_ragged_k(mlxq, M, K, F, gs, bits):
    """The SwiGLU launch at M = 2..8 past the exact wave splits: the last wave's range past K
    (K = 5120 at M = 2), two register rounds per wave (K = 7168, K = 5120 at M >= 3, K = 12288 at
    M = 2), launches of four rows (M = 5, 8 at K = 5120 / 7168) and of two rows (M = 3..8 at
    K = 12288), Q8 at K = 6144 (two rounds); K = 20480 fits no fused plan at M >= 2 and must be
    refused (MLXQ_EUNSUPPORTED), not run."""
    banner("swiglu tile long K", M, K, F, gs, bits)
    rng = np.random.default_rng(M + K + F + gs)
    x = bf16_normal(rng, (M, K))
    tg, tu = [oracle.quantize(bf16_normal(rng, (F, K), 0.02), gs, bits, sb_bf16=True) for _ in range(2)]
    args = (to_gpu(x), [wq_to_gpu(tg[0]), to_gpu(tg[1]), to_gpu(tg[2])],
            [wq_to_gpu(tu[0]), to_gpu(tu[1]), to_gpu(tu[2])], gs, bits)
    if K == 20480:
        with pytest.raises(mlxq.MlxqError) as ei:
            mlxq.swiglu(*args)
        assert ei.value.status == mlxq._lib.MLXQ_EUNSUPPORTED
        return
    h = to_np(mlxq.swiglu(*args))
    gr = oracle.quantized_matmul(x, *tg, gs, bits, w_bf16=False, out_bf16=True)
    ur = oracle.quantized_matmul(x, *tu, gs, bits, w_bf16=False, out_bf16=True)
    ref = oracle.bf16_round(oracle.bf16_round(np.vectorize(oracle.silu)(gr).astype(np.float32)) * ur)
    assert_close(h, ref, f"swiglu tile long K M={M} K={K} F={F} b={bits}")
    print(f"    bit-identical outputs: {np.mean(h == ref) * 100:.2f} %", flush=True)
    assert np.mean(h == ref) > 0.99


@pytest.mark.parametrize("K,F,gs", [(3584, 300, 64), (2560, 129, 128), (15488, 24, 64)])
def test_swiglu_one_row_kernel_ragged_k(mlxq, K, F, gs):
    """The SwiGLU pair at M = 1 with K not a multiple of 1024 (up to 16 loads per row)."""
    banner("swiglu one row ragged K", K, F, gs)
    rng = np.random.default_rng(K + F + gs + 3)
    x = bf16_normal(rng, (1, K))
    tg, tu = [oracle.quantize(bf16_normal(rng, (F, K), 0.02), gs, 4, sb_bf16=True) for _ in range(2)]
    h = to_np(mlxq.swiglu(to_gpu(x), [wq_to_gpu(tg[0]), to_gpu(tg[1]), to_gpu(tg[2])],
                          [wq_to_gpu(tu[0]), to_gpu(tu[1]), to_gpu(tu[2])], gs, 4))
    gr = oracle.quantized_matmul(x, *tg, gs, 4, w_bf16=False, out_bf16=True)
    ur = oracle.quantized_matmul(x, *tu, gs, 4, w_bf16=False, out_bf16=True)
    ref = oracle.bf16_round(oracle.bf16_round(np.vectorize(oracle.silu)(gr).astype(np.float32)) * ur)
    assert_close(h, ref, f"swiglu one row ragged K={K} F={F}")
    print(f"    bit-identical outputs: {np.mean(h == ref) * 100:.2f} %", flush=True)
    assert np.mean(h == ref) > 0.99


@pytest.mark.parametrize("K,N,gs", [(3072, 8192, 64), (8192, 3072, 64), (4096, 520, 128)])
def test_qmv_one_row_kernel_matches_tile_kernel(mlxq, K, N, gs):
    """The one-row kernel (M = 1) and the 16-row tile kernel (M = 2..4 and 8, different wave plans)
    compute the same exact-f32 product: the first M rows of an M = 8 launch bound the M-row
    launches of the same rows."""
    banner("qmv one row vs tile", K, N, gs)
    rng = np.random.default_rng(K + N)
    x = bf16_normal(rng, (8, K))
    w = bf16_normal(rng, (N, K), 0.02)
    wq, s, b = [to_gpu(a) if i else wq_to_gpu(a) for i, a in enumerate(oracle.quantize(w, gs, 4, sb_bf16=True))]
    y8 = to_np(mlxq.quantized_matmul(to_gpu(x), wq, s, b, True, gs, 4))
    for M in (1, 2, 3, 4):
        yM = to_np(mlxq.quantized_matmul(to_gpu(x[:M]), wq, s, b, True, gs, 4))
        _close_to_exact(yM, y8[:M].astype(np.float64), f"rows vs tile M={M} K={K} N={N}")
        print(f"    M={M} bit-identical outputs: {np.mean(yM == y8[:M]) * 100:.2f} %", flush=True)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,F,gs", [(3072, 8192, 64), (4096, 77, 128), (1024, 1000, 64)])
def test_swiglu_one_row_kernel_vs_exact(mlxq, M, K, F, gs):
    """SwiGLU at M = 1 on the one-row kernel (gate row f and up row f in one wave), M = 2..4 on the
    tile kernel: h against the op-by-op rounding of the exact gate and up products."""
    banner("swiglu one row", M, K, F, gs)
    rng = np.random.default_rng(K + F + gs + 1 + 7 * M)
    x = bf16_normal(rng, (M, K))
    tg, tu = [oracle.quantize(bf16_normal(rng, (F, K), 0.02), gs, 4, sb_bf16=True) for _ in range(2)]
    h = to_np(mlxq.swiglu(to_gpu(x), [wq_to_gpu(tg[0]), to_gpu(tg[1]), to_gpu(tg[2])],
                          [wq_to_gpu(tu[0]), to_gpu(tu[1]), to_gpu(tu[2])], gs, 4))
    gr = oracle.quantized_matmul(x, *tg, gs, 4, w_bf16=False, out_bf16=True)
    ur = oracle.quantized_matmul(x, *tu, gs, 4, w_bf16=False, out_bf16=True)
    ref = oracle.bf16_round(oracle.bf16_round(np.vectorize(oracle.silu)(gr).astype(np.float32)) * ur)
    assert_close(h, ref, f"swiglu one row M={M} K={K} F={F}")
    print(f"    bit-identical outputs: {np.mean(h == ref) * 100:.2f} %", flush=True)
    assert np.mean(h == ref) > 0.99


@pytest.mark.parametrize("M", [1, 2, 4, 8])
@pytest.mark.parametrize("K,F,Nd,gs,bits", [(3072, 8192, 3072, 64, 4), (1024, 640, 256, 128, 8),
                                            (512, 192, 64, 64, 4)])
def test_swiglu_decode_mlp_vs_oracle(mlxq, M, K, F, Nd, gs, bits):
    """Decode MLP of qwen3.rs:178-181 as two launches: the fused gate/up SwiGLU GEMV, then the
    down GEMV; h and y against the oracle's op-by-op MLP (exact-f32 dequant, bf16 rounding per op)."""
    banner("swiglu mlp", M, K, F, Nd, gs, bits)
    rng = np.random.default_rng(M * 7 + K + F + bits)
    x = bf16_normal(rng, (M, K))
    trip = [oracle.quantize(bf16_normal(rng, shape, 0.02), gs, bits, sb_bf16=True)
            for shape in ((F, K), (F, K), (Nd, F))]
    g, u, d = [(wq_to_gpu(t[0]), to_gpu(t[1]), to_gpu(t[2])) for t in trip]
    h = mlxq.swiglu(to_gpu(x), g, u, gs, bits)
    y = mlxq.quantized_matmul(h, *d, True, gs, bits)
    ref_h, ref_y = oracle.swiglu_mlp(x, trip[0], trip[1], trip[2], gs, bits, w_bf16=False, act_bf16=True)
    assert_close(to_np(h), ref_h, f"swiglu h M={M}")
    assert_close(to_np(y), oracle.quantized_matmul(to_np(h), *trip[2], gs, bits, w_bf16=False,
                                                   out_bf16=True), f"swiglu y M={M}")
    assert_close(to_np(y), ref_y, f"swiglu y vs oracle mlp M={M}")


@pytest.mark.parametrize("M", [1, 3, 8])
def test_swiglu_ragged_rows(mlxq, M):
    """F = 40 rows (not a multiple of the 16-row workgroup): h against silu(g) * u op by op."""
    banner("swiglu ragged", M)
    rng = np.random.default_rng(40 + M)
    x = bf16_normal(rng, (M, 512))
    tg, tu = [oracle.quantize(bf16_normal(rng, (40, 512), 0.02), 64, 4, sb_bf16=True) for _ in range(2)]
    h = mlxq.swiglu(to_gpu(x), [wq_to_gpu(tg[0]), to_gpu(tg[1]), to_gpu(tg[2])],
                    [wq_to_gpu(tu[0]), to_gpu(tu[1]), to_gpu(tu[2])], 64, 4)
    gr = oracle.quantized_matmul(x, *tg, 64, 4, w_bf16=False, out_bf16=True)
    ur = oracle.quantized_matmul(x, *tu, 64, 4, w_bf16=False, out_bf16=True)
    ref = oracle.bf16_round(np.vectorize(oracle.silu)(gr).astype(np.float32) * ur)
    assert_close(to_np(h), ref, f"swiglu ragged M={M}")


def test_swiglu_outside_the_decode_form_is_unsupported(mlxq):
    banner("swiglu unsupported")
    rng = np.random.default_rng(9)
    t = oracle.quantize(bf16_normal(rng, (64, 256), 0.02), 64, 4, sb_bf16=True)
    g = (wq_to_gpu(t[0]), to_gpu(t[1]), to_gpu(t[2]))
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.swiglu(to_gpu(bf16_normal(rng, (9, 256))), g, g, 64, 4)
    assert e.value.status == 2
    with pytest.raises(mlxq.MlxqError) as e:
        mlxq.swiglu(to_gpu(bf16_normal(rng, (2, 256)), torch.float32), g, g, 64, 4)
    assert e.value.status == 2


def test_f32_activations_large_m(mlxq):
    """f32 activations at GEMM-sized M keep exact-f32 semantics (the FLUX.1 f32 stream)."""
    banner("f32 large M")
    rng = np.random.default_rng(9)
    x = rng.standard_normal((40, 256)).astype(np.float32)
    w = (rng.standard_normal((72, 256)) * 0.02).astype(np.float32)
    wq, s, b = mlxq.quantize(to_gpu(w, torch.float32), 64, 8)
    y = to_np(mlxq.quantized_matmul(to_gpu(x, torch.float32), wq, s, b, True, 64, 8))
    rwq, rs, rb = oracle.quantize(w, 64, 8)
    ref = oracle.quantized_matmul(x, rwq, rs, rb, 64, 8, w_bf16=False, out_bf16=False)
    assert errors(y, ref)[0] < 1e-5


# ---------------------------------------------------------------- fused linear epilogue

@pytest.mark.parametrize("act", [1, 2, 3])
def test_linear_f32_activations_act(mlxq, act):
    """f32 activations (the FLUX.1 f32 stream): bias and activation evaluated in f32, no bf16
    rounding anywhere, against the oracle's f32 op sequence."""
    banner("linear f32 act", act)
    rng = np.random.default_rng(31 + act)
    M, K, N = 24, 256, 72
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    wq, s, b = mlxq.quantize(to_gpu(w, torch.float32), 64, 8)
    y = to_np(mlxq.linear(to_gpu(x, torch.float32), wq, s, b, 64, 8, bias=to_gpu(bias, torch.float32),
                          activation=act))
    rwq, rs, rb = oracle.quantize(w, 64, 8)
    ref = oracle.linear(x, rwq, rs, rb, 64, 8, w_bf16=False, act_bf16=False, bias=bias, act=act)
    assert errors(y, ref)[0] < 1e-5

@pytest.mark.parametrize("M", [4, 300])
@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_linear_bias_lora_act(mlxq, M, act):
    banner("linear epilogue", M, act)
    rng = np.random.default_rng(21 + M + act)
    K, N, r = 512, 264, 16
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    bias = bf16_normal(rng, (N,), 0.5)
    A = bf16_normal(rng, (K, r), 0.01)
    B = bf16_normal(rng, (r, N), 0.01)
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    yt = mlxq.linear(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), 64, 4,
                     bias=to_gpu(bias), lora_a=to_gpu(A), lora_b=to_gpu(B), lora_scale=0.75,
                     activation=act)
    ref, out_bf16 = oracle.linear(x, rwq, rs, rb, 64, 4, w_bf16=(M > 8), act_bf16=True, bias=bias,
                                  lora_a=A, lora_b=B, lora_scale=0.75, act=act, return_dtype=True)
    assert yt.dtype == (torch.bfloat16 if out_bf16 else torch.float32)  # GELU (act 1) promotes
    assert_close(to_np(yt), ref, f"linear M={M} act={act}")


@pytest.mark.parametrize("K", [64, 256, 320])
@pytest.mark.parametrize("rank,scale", [(8, 1.0), (16, 0.75), (24, 1.5)])
def test_linear_lora_short_k_ranks(mlxq, K, rank, scale):
    """LoRA with K < 512 (the 128/256-tile GEMM, whose epilogue fuses rank <= 16) and rank 24
    (plain GEMM + elementwise epilogue): the x.A preparation with one or two K steps per wave
    and padding columns (rank 8 and 24 pad to 16 and 32)."""
    banner("linear lora short K", K, rank, scale)
    rng = np.random.default_rng(K + rank)
    M, N = 37, 192
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    bias = bf16_normal(rng, (N,), 0.1)
    A = bf16_normal(rng, (K, rank), 0.05)
    B = bf16_normal(rng, (rank, N), 0.05)
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    y = to_np(mlxq.linear(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), 64, 4,
                          bias=to_gpu(bias), lora_a=to_gpu(A), lora_b=to_gpu(B), lora_scale=scale))
    ref = oracle.linear(x, rwq, rs, rb, 64, 4, w_bf16=True, act_bf16=True, bias=bias,
                        lora_a=A, lora_b=B, lora_scale=scale)
    assert_close(y, ref, f"lora K={K} rank={rank}")


# The x.A preparation from 4097 to 8192 rows spreads the rows over at most 256 workgroups of 17-32
# (two MFMA blocks; rows past a workgroup's share repeat its last row and are never stored):
# M just past 4096 (17 rows each), the config-5 M = 4608 (18), 8192 (32) and beyond (16-row
# workgroups again), ranks 16 (the 4 KB A-chunk form) and 24 (the general form, two column
# blocks).  y = 0, so the outputs are the LoRA term alone: each row's x.A is checked, not hidden
# under a base product.
@pytest.mark.parametrize("M", [4097, 4608, 8192, 8229])
@pytest.mark.parametrize("rank", [16, 24])
def test_lora_xa_rows_per_workgroup(mlxq, M, rank):
    banner("lora x.A rows", M, rank)
    rng = np.random.default_rng(M + rank)
    K, N = 256, 64
    x = bf16_normal(rng, (M, K))
    A = bf16_normal(rng, (K, rank), 0.05)
    B = bf16_normal(rng, (rank, N), 0.05)
    y = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    out = to_np(mlxq.ops.lora_residual(to_gpu(x), y, to_gpu(A), to_gpu(B), 1.0))
    xa = oracle.bf16_round((x.astype(np.float64) @ A.astype(np.float64)).astype(np.float32))
    want = oracle.bf16_round((xa.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
    assert_close(out, want, f"lora x.A M={M} rank={rank}")
    # every row carries its own term: a row computed from a neighbour's x would be off by O(1)
    rowerr = np.abs(out - want).max(axis=1) / (np.abs(want).max(axis=1) + 1e-30)
    assert rowerr.max() < 0.05, int(rowerr.argmax())


# ---------------------------------------------------------------- errors never crash

def test_invalid_arguments_return_errors(mlxq):
    banner("invalid arguments")
    w = torch.zeros((4, 100), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mlxq.MlxqError, match="multiple of group_size"):
        mlxq.quantize(w, 64, 4)
    w = torch.zeros((4, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mlxq.MlxqError, match="bits"):
        mlxq.quantize(w, 64, 3)
    wq, s, b = mlxq.quantize(w, 64, 4)
    x = torch.zeros((2, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mlxq.MlxqError, match="transpose"):
        mlxq.quantized_matmul(x, wq, s, b, False, 64, 4)
    with pytest.raises(mlxq.MlxqError, match="GEMV limit"):
        mlxq.qmv(torch.zeros((9, 128), dtype=torch.bfloat16, device="cuda"), wq, s, b, 64, 4)


# ---------------------------------------------------------------- configs 3 and 5 at full size

def test_config3_wan_projection_full_size_sampled_rows(mlxq):
    """Config 3: x[32760,5120] bf16 . Q8-g64 W[5120,5120]^T at full size (sampled rows), with the
    full-size quantize bit-exact against the oracle."""
    banner("config3 full size")
    rng = np.random.default_rng(33)
    M, D = 32760, 5120
    x = bf16_normal(rng, (M, D))
    w = bf16_normal(rng, (D, D), 0.02)
    wq, s, b = mlxq.quantize(to_gpu(w), 64, 8)
    y = mlxq.quantized_matmul(to_gpu(x), wq, s, b, True, 64, 8)
    torch.cuda.synchronize()
    rwq, rs, rb = oracle.quantize(w, 64, 8, sb_bf16=True)
    assert np.array_equal(to_np(wq), rwq)
    assert np.array_equal(to_np(s), rs) and np.array_equal(to_np(b), rb)
    rows = _band_rows(rng, M)  # a row in every 224- and 256-row M-tile band
    ref = oracle.quantized_matmul(x[rows], rwq, rs, rb, 64, 8, w_bf16=True, out_bf16=True)
    assert_close(to_np(y)[rows], ref, f"config3 {rows.size} rows (every M-tile band)")


CONFIG5_SHAPES = [(9216, 3072), (3072, 3072), (12288, 3072), (3072, 12288), (18432, 3072)]
_CONFIG5_X = {}


def _config5_x(K):
    """Activations x[4608, K] shared by the cells with the same K (host copy and device copy)."""
    if K not in _CONFIG5_X:
        x = bf16_normal(np.random.default_rng(K), (4608, K))
        _CONFIG5_X.clear()
        _CONFIG5_X[K] = (x, to_gpu(x))
    return _CONFIG5_X[K]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("N,K", sorted(CONFIG5_SHAPES, key=lambda nk: nk[1]))
def test_config5_block_sweep_with_lora_sampled_rows(mlxq, bits, gs, N, K):
    """Config 5 cell at full size: M=4608, rank-16 bf16 LoRA (A, B ~ N(0,0.01)) fused into the
    epilogue, checked on sampled rows against the oracle's op-by-op linear.  The packed codes the
    GPU produced are checked bit-exact on a slice and then fed to the oracle."""
    banner("config5", bits, gs, N, K)
    rng = np.random.default_rng(bits * 1000 + gs + N + K)
    M = 4608
    x, gx = _config5_x(K)
    w = bf16_normal(rng, (N, K), 0.02)
    a = bf16_normal(rng, (K, 16), 0.01)
    bb = bf16_normal(rng, (16, N), 0.01)
    wq, s, b = mlxq.quantize(to_gpu(w), gs, bits)
    y = mlxq.linear(gx, wq, s, b, gs, bits, lora_a=to_gpu(a), lora_b=to_gpu(bb))
    torch.cuda.synchronize()
    gwq, gs_, gb = to_np(wq), to_np(s), to_np(b)
    rwq, rs, rb = oracle.quantize(w[:64], gs, bits, sb_bf16=True)
    assert np.array_equal(gwq[:64], rwq) and np.array_equal(gs_[:64], rs) and np.array_equal(gb[:64], rb)
    rows = _band_rows(rng, M)  # a row in every 224- and 256-row M-tile band
    scale = 0.75 if (bits, gs, N, K) == (4, 64, 3072, 3072) else 1.0
    if scale != 1.0:
        y = mlxq.linear(gx, wq, s, b, gs, bits, lora_a=to_gpu(a), lora_b=to_gpu(bb), lora_scale=scale)
    ref = oracle.linear(x[rows], gwq, gs_, gb, gs, bits, w_bf16=True, act_bf16=True, lora_a=a,
                        lora_b=bb, lora_scale=scale)
    assert_close(to_np(y)[rows], ref, f"config5 Q{bits} g{gs} {N}x{K} ({rows.size} rows)")
