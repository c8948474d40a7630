"""Empty inputs through every operation: MLX takes zero-size arrays (no tokens, an empty id batch,
a weight with no rows) and returns zero-size results of the right shape and dtype; so must the
library, without launching anything and without an error."""
import pytest
import torch

from gpu_util import banner

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _pack(mlxq, N, K, bits=4, gs=64):
    w = (torch.randn((N, K), device="cuda") * 0.02).to(torch.bfloat16)
    return mlxq.quantize(w, gs, bits)


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32, torch.float16])
def test_products_with_no_rows(mlxq, xdt):
    banner("empty products", xdt)
    K, N = 256, 96
    wq, s, b = _pack(mlxq, N, K)
    x = torch.empty((0, K), dtype=xdt, device="cuda")
    ydt = torch.bfloat16 if xdt == torch.bfloat16 else torch.float32
    y = mlxq.quantized_matmul(x, wq, s, b, True, 64, 4)
    assert y.shape == (0, N) and y.dtype == ydt
    x3 = torch.empty((2, 0, K), dtype=xdt, device="cuda")
    assert mlxq.quantized_matmul(x3, wq, s, b, True, 64, 4).shape == (2, 0, N)
    bias = torch.randn(N, device="cuda").to(torch.bfloat16)
    la = (torch.randn((K, 16), device="cuda") * 0.01).to(torch.bfloat16)
    lb = (torch.randn((16, N), device="cuda") * 0.01).to(torch.bfloat16)
    for act in (0, 1, 3):
        y = mlxq.linear(x, wq, s, b, 64, 4, bias=bias, lora_a=la, lora_b=lb, lora_scale=0.5, activation=act)
        assert y.shape == (0, N)
    y0 = torch.empty((0, N), dtype=ydt, device="cuda")
    assert mlxq.lora_residual(x, y0, la, lb, 1.0).shape == (0, N)
    if xdt != torch.float16:  # the LoKr product takes bf16 or f32 activations
        delta = (torch.randn((N, K), device="cuda") * 0.01).to(torch.bfloat16)
        assert mlxq.lokr_residual(x, y0, delta, 1.0).shape == (0, N)


def test_decode_forms_with_no_rows(mlxq):
    banner("empty decode forms")
    K, F = 1024, 256
    g, u = _pack(mlxq, F, K), _pack(mlxq, F, K)
    x = torch.empty((0, K), dtype=torch.bfloat16, device="cuda")
    assert mlxq.qmv(x, *g, 64, 4).shape == (0, F)
    assert mlxq.qmv_valu(x, *g, 64, 4).shape == (0, F)
    h = mlxq.swiglu(x, g, u, 64, 4)
    assert h.shape == (0, F) and h.dtype == torch.bfloat16


def test_weights_with_no_rows(mlxq):
    banner("empty weights")
    K = 256
    w = torch.empty((0, K), dtype=torch.bfloat16, device="cuda")
    wq, s, b = mlxq.quantize(w, 64, 4)
    assert wq.shape == (0, K // 8) and s.shape == (0, K // 64) and b.shape == (0, K // 64)
    assert mlxq.dequantize(wq, s, b, 64, 4).shape == (0, K)
    x = torch.randn((5, K), device="cuda").to(torch.bfloat16)
    y = mlxq.quantized_matmul(x, wq, s, b, True, 64, 4)
    assert y.shape == (5, 0)
    x300 = torch.randn((300, K), device="cuda").to(torch.bfloat16)
    assert mlxq.quantized_matmul(x300, wq, s, b, True, 64, 4).shape == (300, 0)


def test_embedding_with_no_ids(mlxq):
    banner("empty embedding")
    wq, s, b = _pack(mlxq, 50, 128)
    for shape in ((0,), (2, 0)):
        ids = torch.empty(shape, dtype=torch.int32, device="cuda")
        e = mlxq.embedding(ids, wq, s, b, 64, 4)
        assert e.shape == shape + (128,) and e.dtype == torch.float32
