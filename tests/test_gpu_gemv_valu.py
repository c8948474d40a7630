"""GPU parity of the forced VALU GEMV (mlxq_qmv_valu) on bf16 decode shapes.

The VALU kernel serves f32 activations, f32 scales and group size 32; forced on bf16 operands it
is the VALU side of the kernel-choice A/B against the matrix-core GEMV in bench.py's gemv leg (at
M = 1 on the one-row kernel's own loads with VALU dot products).  Both have the f32 semantics of
MLX's qmv, checked against the oracle and against each other.
"""
import numpy as np
import pytest

from gpu_util import assert_close, banner, bf16_normal, to_gpu, to_np, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


# M = 1 bf16 Q4 with group 64/128 and K <= 8192 runs the one-row kernel's loads with VALU dot
# products (ragged last load at K = 3584, ragged N, group 128); K = 16384 and the other rows the
# VALU GEMV proper.
@pytest.mark.parametrize("M,K,N,gs,bits", [(1, 3072, 8192, 64, 4), (8, 8192, 3072, 64, 4),
                                          (3, 1024, 200, 128, 8), (2, 512, 96, 32, 4),
                                          (1, 8192, 3072, 64, 4), (1, 3584, 300, 64, 4),
                                          (1, 2048, 520, 128, 4), (1, 16384, 64, 64, 4)])
def test_qmv_valu_bf16_vs_oracle(mlxq, M, K, N, gs, bits):
    """The VALU GEMV forced on bf16 operands (the kernel the matrix-core GEMV replaced there):
    exact-f32 semantics like qmv, against the oracle and against the matrix-core GEMV."""
    banner("qmv_valu", M, K, N, gs, bits)
    rng = np.random.default_rng(M + K + N + bits)
    x = bf16_normal(rng, (M, K))
    t = oracle.quantize(bf16_normal(rng, (N, K), 0.02), gs, bits, sb_bf16=True)
    dev = (wq_to_gpu(t[0]), to_gpu(t[1]), to_gpu(t[2]))
    y = to_np(mlxq.qmv_valu(to_gpu(x), *dev, gs, bits))
    ref = oracle.quantized_matmul(x, *t, gs, bits, w_bf16=False, out_bf16=True)
    assert_close(y, ref, f"qmv_valu M={M}")
    assert_close(y, to_np(mlxq.qmv(to_gpu(x), *dev, gs, bits)).astype(np.float64), "valu vs mfma")
