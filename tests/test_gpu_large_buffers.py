"""Operands past the 2 GiB and 4 GiB marks (maximum sizes).

The fast kernels address their operands through buffer resources with 32-bit offsets: the wide
and K-split GEMMs take operands under 4 GiB, the matrix-core GEMVs under 2 GiB, and the host
routes anything larger to kernels that index with 64-bit pointers (the 128 x 128 tile GEMM, the
VALU GEMV).  Each test builds one operand just past such a mark and checks the outputs whose
inputs lie on both sides of it against the oracle: rows (or weight rows) at the start, just below
and just above the boundary, and at the end.  About 4.3 GB of device memory per test.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, banner, to_np
from oracle import oracle

pytestmark = pytest.mark.gpu

GIB2, GIB4 = 1 << 31, 1 << 32


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _bf16_rows(gen, rows, cols, std):
    return (torch.randn((rows, cols), generator=gen, device="cuda", dtype=torch.float32) * std).to(torch.bfloat16)


def _boundary_rows(n_rows, row_bytes, mark):
    """Rows at the start, on either side of the byte offset `mark`, and at the end."""
    b = mark // row_bytes
    rows = sorted({0, 1, b - 2, b - 1, b, b + 1, n_rows - 2, n_rows - 1})
    return [r for r in rows if 0 <= r < n_rows]


def test_gemm_activations_past_4gib(mlxq):
    """x [2^20 + 40, 2048] bf16 (4 GiB + 160 KB) through quantized_matmul (Q4 g64, N = 96): the
    wide kernel's 4 GiB condition sends it to the 64-bit tile GEMM; rows on both sides of the
    4 GiB offset match the bf16-tile GEMM oracle."""
    M, K, N = (1 << 20) + 40, 2048, 96
    banner("large gemm x", M, K, N)
    gen = torch.Generator(device="cuda").manual_seed(11)
    x = _bf16_rows(gen, M, K, 1.0)
    assert x.numel() * 2 > GIB4
    w = _bf16_rows(gen, N, K, 0.02)
    wq, s, b = mlxq.quantize(w, 64, 4)
    y = mlxq.quantized_matmul(x, wq, s, b, True, 64, 4)
    torch.cuda.synchronize()
    rows = _boundary_rows(M, K * 2, GIB4)
    xr = x[rows].float().cpu().numpy()
    ref = oracle.quantized_matmul(xr, to_np(wq), to_np(s), to_np(b), 64, 4, w_bf16=True, out_bf16=True)
    assert_close(to_np(y[rows]), ref, "gemm x past 4 GiB")


def test_f32_gemm_activations_past_4gib(mlxq):
    """x [2^19 + 40, 2048] f32 (4 GiB + 320 KB) on the factored f32 GEMM (64-bit indexing):
    rows on both sides of the 4 GiB offset within 1e-4 relFro of the exact f32 oracle."""
    M, K, N = (1 << 19) + 40, 2048, 256
    banner("large f32 gemm x", M, K, N)
    gen = torch.Generator(device="cuda").manual_seed(12)
    x = torch.randn((M, K), generator=gen, device="cuda", dtype=torch.float32)
    assert x.numel() * 4 > GIB4
    w = _bf16_rows(gen, N, K, 0.02)
    wq, s, b = mlxq.quantize(w, 64, 4)
    y = mlxq.quantized_matmul(x, wq, s, b, True, 64, 4)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    rows = _boundary_rows(M, K * 4, GIB4)
    ref = oracle.quantized_matmul(x[rows].cpu().numpy(), to_np(wq), to_np(s), to_np(b), 64, 4,
                                  w_bf16=False, out_bf16=False)
    rel, _ = assert_close(to_np(y[rows]), ref, "f32 gemm x past 4 GiB")
    assert rel < 1e-4


def test_gemv_and_embedding_weights_past_2gib(mlxq):
    """A Q8 g64 pack of [2^20 + 8, 2048] (codes 2 GiB + 16 KB): the decode GEMV at M = 1 and 4
    (past the matrix-core GEMVs' 2 GiB condition: the VALU GEMV) against the exact-f32 GEMV
    oracle on weight rows either side of the 2 GiB offset, and the quantized embedding gather of
    those rows bit for bit."""
    N, K = (1 << 20) + 8, 2048
    banner("large gemv / embedding weights", N, K)
    gen = torch.Generator(device="cuda").manual_seed(13)
    w = _bf16_rows(gen, N, K, 0.02)
    wq, s, b = mlxq.quantize(w, 64, 8)
    del w
    assert wq.numel() * 4 > GIB2
    rows = _boundary_rows(N, K, GIB2)
    wq_r, s_r, b_r = to_np(wq[rows]), to_np(s[rows]), to_np(b[rows])
    for M in (1, 4):
        x = _bf16_rows(gen, M, K, 1.0)
        y = mlxq.quantized_matmul(x, wq, s, b, True, 64, 8)
        torch.cuda.synchronize()
        ref = oracle.quantized_matmul(x.float().cpu().numpy(), wq_r, s_r, b_r, 64, 8, w_bf16=False,
                                      out_bf16=True)
        assert_close(to_np(y[:, rows]), ref, f"gemv past 2 GiB M={M}")
    ids = torch.tensor(rows, dtype=torch.int32, device="cuda")
    e = mlxq.embedding(ids, wq, s, b, 64, 8)
    table = oracle.dequantize(wq_r, s_r, b_r, 64, 8, out_bf16=True)
    assert np.array_equal(to_np(e), table)


def test_quantize_weight_past_4gib(mlxq):
    """quantize of a bf16 [2^20 + 8, 2048] weight (4 GiB + 32 KB), Q4 g64: codes, scales and
    biases of the rows either side of the 4 GiB offset bit-exact against the oracle; dequantize
    of the same pack bit-exact on those rows."""
    N, K = (1 << 20) + 8, 2048
    banner("large quantize", N, K)
    gen = torch.Generator(device="cuda").manual_seed(14)
    w = _bf16_rows(gen, N, K, 0.02)
    assert w.numel() * 2 > GIB4
    wq, s, b = mlxq.quantize(w, 64, 4)
    torch.cuda.synchronize()
    rows = _boundary_rows(N, K * 2, GIB4)
    rwq, rs, rb = oracle.quantize(w[rows].float().cpu().numpy(), 64, 4, sb_bf16=True)
    assert np.array_equal(to_np(wq[rows]), rwq)
    assert np.array_equal(to_np(s[rows]), rs) and np.array_equal(to_np(b[rows]), rb)
    del w
    d = mlxq.dequantize(wq, s, b, 64, 4)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(d[rows]), oracle.dequantize(rwq, rs, rb, 64, 4, out_bf16=True))


def test_stacked_experts_pack_past_4gib(mlxq):
    """A stacked Q4 g64 pack of 80 experts [14336, 8192] (codes 4.7 GB) in one qmm_experts launch
    (grid.y = expert, each expert's operands addressed from its own base): the first expert and the
    last one, whose codes start past 4 GiB, against the bf16-tile GEMM oracle on two rows."""
    E, M, N, K = 80, 256, 14336, 8192
    banner("large stacked experts", E, M, N, K)
    gen = torch.Generator(device="cuda").manual_seed(15)
    wq = torch.empty((E, N, K // 8), dtype=torch.int32, device="cuda")
    s = torch.empty((E, N, K // 64), dtype=torch.bfloat16, device="cuda")
    b = torch.empty_like(s)
    for e in range(E):
        pe = mlxq.quantize(_bf16_rows(gen, N, K, 0.02), 64, 4)
        wq[e].copy_(pe[0])
        s[e].copy_(pe[1])
        b[e].copy_(pe[2])
    assert wq.numel() * 4 > GIB4
    x = _bf16_rows(gen, M, K, 1.0)
    y = mlxq.qmm_experts(x, wq, s, b, 64, 4)
    torch.cuda.synchronize()
    assert y.shape == (E, M, N)
    rows = [0, M - 1]
    xr = x[rows].float().cpu().numpy()
    for e in (0, E - 1):
        ref = oracle.quantized_matmul(xr, to_np(wq[e]), to_np(s[e]), to_np(b[e]), 64, 4, w_bf16=True,
                                      out_bf16=True)
        assert_close(to_np(y[e, rows]), ref, f"stacked experts past 4 GiB, expert {e}")
