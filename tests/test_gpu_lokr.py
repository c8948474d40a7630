"""GPU parity of the LoKr adapter arm (mlxq_lokr_residual and the host layers' LoKr adapters).

Adapter::Lokr (reference src/adapters.rs:234-235, residual :263-266) adds scale * x . delta^T to a
linear's output, delta being the reconstructed kron delta (stored bf16) cast to the activation
dtype, the residual in the activation dtype and the sum promoted with the output
(AdaptableLinear::forward, :543-549).  The product runs on the matrix cores (one bf16 pass for bf16
x; for f32 x the activation's two-term bf16 split against the exact bf16 delta, plus a third pass for
an f32 delta); the checks hold it to the oracle's fp64 restatement at the north-star tolerance
(bf16 results) or relFro < 1e-4 (f32 results), bit-exact for scale 0 and for the reference's own
2x2 fixture, and through the Python layers for mixed LoRA + LoKr stacks.
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


def _data(rng, M, N, K, x_dt, y_dt, d_dt):
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = rng.standard_normal((M, N)).astype(np.float32)
    delta = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if x_dt == "bf16":
        x = oracle.bf16_round(x)
    if y_dt == "bf16":
        y = oracle.bf16_round(y)
    if d_dt == "bf16":
        delta = oracle.bf16_round(delta)
    return x, y, delta


# (M, N, K, x dtype, y dtype, delta dtype): ragged M and N, decode M = 1, a FLUX-size projection,
# the f32 stream, every promotion (bf16 y + f32 residual, f32 y + bf16 residual), an f32 delta
# cast to bf16 against bf16 x and kept f32 against f32 x.
CASES = [
    (200, 262, 512, "bf16", "bf16", "bf16"),
    (1, 3072, 3072, "bf16", "bf16", "bf16"),
    (4608, 3072, 3072, "bf16", "bf16", "bf16"),
    (130, 264, 1024, "f32", "f32", "bf16"),
    (300, 128, 768, "bf16", "f32", "bf16"),
    (64, 200, 256, "f32", "bf16", "bf16"),
    (96, 96, 256, "bf16", "bf16", "f32"),
    (77, 160, 512, "f32", "f32", "f32"),
]


@pytest.mark.parametrize("M,N,K,x_dt,y_dt,d_dt", CASES)
def test_lokr_residual_vs_oracle(mlxq, M, N, K, x_dt, y_dt, d_dt):
    banner("lokr residual", M, N, K, x_dt, y_dt, d_dt)
    rng = np.random.default_rng(M + N + K + len(x_dt + y_dt + d_dt))
    x, y, delta = _data(rng, M, N, K, x_dt, y_dt, d_dt)
    gy = to_gpu(y, _tdt(y_dt))
    out = mlxq.lokr_residual(to_gpu(x, _tdt(x_dt)), gy, to_gpu(delta, _tdt(d_dt)), 0.75)
    ref, ref_bf16 = oracle.lokr_residual(x, y, delta, 0.75, x_bf16=x_dt == "bf16", y_bf16=y_dt == "bf16",
                                         return_dtype=True)
    assert out.dtype == (torch.bfloat16 if ref_bf16 else torch.float32)
    if ref_bf16:
        assert_close(to_np(out), ref, f"lokr {x_dt}/{y_dt}/{d_dt}")
    else:
        rel, peak = errors(to_np(out), ref)
        print(f"    relFro={rel:.3e} peak={peak:.3e}", flush=True)
        assert rel < 1e-4 and peak < 1e-3
        # the residual itself (not only y + r) against the oracle's: x_lo and d_lo passes present
        r = to_np(out) - y.astype(np.float64)
        r_ref = ref.astype(np.float64) - y.astype(np.float64)
        assert errors(r, r_ref)[0] < 1e-4


@pytest.mark.parametrize("x_dt,y_dt", [("bf16", "bf16"), ("f32", "f32")])
def test_lokr_scale_zero_is_bit_exact_noop(mlxq, x_dt, y_dt):
    """src/adapters.rs:717-728: a LoKr adapter with scale 0 leaves the output bit for bit."""
    banner("lokr scale 0", x_dt, y_dt)
    rng = np.random.default_rng(5)
    x, y, delta = _data(rng, 150, 200, 256, x_dt, y_dt, "bf16")
    gy = to_gpu(y, _tdt(y_dt))
    before = gy.clone()
    out = mlxq.lokr_residual(to_gpu(x, _tdt(x_dt)), gy, to_gpu(delta), 0.0)
    assert torch.equal(out, before)


def test_lokr_reference_2x2_fixture(mlxq):
    """The reference's lokr_2x2 delta and x32 (src/adapters.rs:695-764), zero-padded along K to the
    kernel's multiple of 32 (zeros add nothing): every product and sum is exact, so the residual is
    bit-identical to the oracle's, and bf16."""
    banner("lokr 2x2 fixture")
    w1 = np.array([[0.5], [0.6]], np.float32)
    w2 = np.array([[0.7, 0.8]], np.float32)
    delta = oracle.bf16_round(np.kron(w1, w2).astype(np.float32) * np.float32(2.0))
    x = np.array([[1.0, -2.0], [0.5, 0.25], [-1.0, 2.0]], np.float32)
    xp = np.zeros((3, 32), np.float32)
    xp[:, :2] = x
    dp = np.zeros((2, 32), np.float32)
    dp[:, :2] = delta
    zero = torch.zeros((3, 2), dtype=torch.bfloat16, device="cuda")
    out = mlxq.lokr_residual(to_gpu(xp), zero, to_gpu(dp), 0.5)
    assert out.dtype == torch.bfloat16
    ref = oracle.lokr_residual(x, np.zeros((3, 2), np.float32), delta, 0.5)
    np.testing.assert_array_equal(to_np(out), ref)
    np.testing.assert_array_equal(to_np(out)[0], np.array([-0.451171875, -0.5390625], np.float32))


@pytest.mark.parametrize("order", ["lora_lokr", "lokr_lora", "lokr_f32_stream"])
def test_adaptable_linear_with_lokr(mlxq, order):
    """AdaptableLinear over a quantized base with mixed adapter stacks (src/adapters.rs:1089-1119):
    each adapter's residual summed in turn, against the oracle's linear + residual steps."""
    banner("adaptable linear lokr", order)
    from mlxq import nn
    rng = np.random.default_rng(len(order))
    M, K, N, R = 120, 512, 384, 16
    w = oracle.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    bias = oracle.bf16_round((rng.standard_normal(N) * 0.1).astype(np.float32))
    A = oracle.bf16_round((rng.standard_normal((K, R)) * 0.02).astype(np.float32))
    B = oracle.bf16_round((rng.standard_normal((R, N)) * 0.02).astype(np.float32))
    delta = oracle.bf16_round((rng.standard_normal((N, K)) * 0.01).astype(np.float32))
    f32_stream = order == "lokr_f32_stream"
    x = rng.standard_normal((M, K)).astype(np.float32)
    if not f32_stream:
        x = oracle.bf16_round(x)
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    layer = nn.AdaptableLinear.from_quantized_parts(wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), to_gpu(bias),
                                                    64, 4)
    lora = nn.Adapter(to_gpu(A), to_gpu(B), 0.5)
    lokr = nn.LokrAdapter(to_gpu(delta), 0.7)
    xb = x.astype(np.float32)
    if order == "lora_lokr":
        layer.set_adapters([lora, lokr])
        ref = oracle.linear(xb, rwq, rs, rb, 64, 4, bias=bias, lora_a=A, lora_b=B, lora_scale=0.5)
        ref = oracle.lokr_residual(xb, ref, delta, 0.7)
    elif order == "lokr_lora":
        layer.set_adapters([lokr, lora])
        ref = oracle.lokr_residual(xb, oracle.linear(xb, rwq, rs, rb, 64, 4, bias=bias), delta, 0.7)
        # then the LoRA residual in bf16, each op rounded (src/adapters.rs:260-270)
        xa = oracle.bf16_round((xb.astype(np.float64) @ A.astype(np.float64)).astype(np.float32))
        r = oracle.bf16_round((xa.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
        ref = oracle.bf16_round(ref + oracle.bf16_round(r * np.float32(0.5)))
    else:
        layer.set_adapters([lokr])
        ref = oracle.linear(xb, rwq, rs, rb, 64, 4, w_bf16=False, act_bf16=False, bias=bias, x_bf16=False,
                            sb_bf16=True, bias_bf16=True)
        ref = oracle.lokr_residual(xb, ref, delta, 0.7, x_bf16=False, y_bf16=False)
    out = layer.forward(to_gpu(x, torch.float32 if f32_stream else torch.bfloat16))
    assert out.dtype == (torch.float32 if f32_stream else torch.bfloat16)
    if f32_stream:
        rel, peak = errors(to_np(out), ref)
        print(f"    relFro={rel:.3e} peak={peak:.3e}", flush=True)
        assert rel < 1e-4
    else:
        assert_close(to_np(out), ref, f"adaptable linear {order}")
