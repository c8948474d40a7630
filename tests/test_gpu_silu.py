"""SwiGLU epilogue of the decode MLP (reference mlx-gen-sensenova/src/qwen3.rs:178-181) on every
normal bf16 gate value, bit for bit against the oracle.

h = round(silu(round(g)) * round(u)) with silu(g) = round(g * round(sigmoid(g))), the reference's
silu as two ops (src/nn.rs:301-303).  The products are made exact so that only the epilogue is
under test: x = c * e_0 (one non-zero element, c a power of two), every code 0, scales 0 and the
biases of row f equal to the f-th bf16 value, so gate row f is exactly c * b_f (or its overflow to
+-inf, the same in every implementation) and up row f is c * u_f for a chosen bf16 value u_f.
(With every code 0 the scale does not enter the product.)  Every normal
bf16 value and both zeros appear as b_f; subnormal values are left out (the rounding of the exact
product's subnormal tail is not what this test is about).
"""
import numpy as np
import pytest
import torch

from gpu_util import banner, to_gpu, to_np, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _normal_bf16():
    h = np.arange(65536, dtype=np.uint32)
    e = (h >> 7) & 0xFF
    h = h[((e != 0) & (e != 0xFF)) | ((h & 0x7FFF) == 0)]
    return (h << 16).view(np.float32)


@pytest.mark.parametrize("M", [1, 2, 8])
def test_swiglu_every_normal_bf16_gate(mlxq, M):
    banner("swiglu every bf16 gate", M)
    K, gs, bits = 1024, 64, 4
    g_vals = _normal_bf16()
    F = g_vals.size
    rng = np.random.default_rng(11)
    u_vals = oracle.bf16_round(rng.uniform(0.5, 2.0, F).astype(np.float32))
    coef = np.array([1.0, -1.0, 2.0, -2.0, 4.0, -4.0, 8.0, -8.0], np.float32)[:M]
    x = np.zeros((M, K), np.float32)
    x[:, 0] = coef
    wq = np.zeros((F, K * bits // 32), np.uint32)
    zeros = np.zeros((F, K // gs), np.float32)
    gate = (wq_to_gpu(wq), to_gpu(zeros), to_gpu(np.repeat(g_vals[:, None], K // gs, 1)))
    up = (wq_to_gpu(wq), to_gpu(zeros), to_gpu(np.repeat(u_vals[:, None], K // gs, 1)))
    h = to_np(mlxq.swiglu(to_gpu(x), gate, up, gs, bits))
    with np.errstate(over="ignore"):
        g = oracle.bf16_round((coef[:, None] * g_vals[None, :]).astype(np.float32))
        u = coef[:, None] * u_vals[None, :]  # exact: a power of two times a bf16 value below 2
        silu = np.array([oracle.silu(float(v)) for v in g.ravel()], np.float32).reshape(g.shape)
        ref = oracle.bf16_round((silu * u).astype(np.float32))
    same = (h == ref) | (np.isnan(h) & np.isnan(ref))
    bad = np.argwhere(~same)
    print(f"    {F} gate values x {M} rows: {bad.shape[0]} mismatches", flush=True)
    for m, f in bad[:8]:
        print(f"      row {m} g={g[m, f]!r} u={u[m, f]!r}: got {h[m, f]!r} want {ref[m, f]!r}")
    assert bad.shape[0] == 0
