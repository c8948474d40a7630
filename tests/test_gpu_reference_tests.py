"""The reference's own weight-free tests of this path, run on the GPU through the library.

Each test restates one reference test with the same inputs, operations and bars, with the
reference's layer (`AdaptableLinear`) and ops replaced by this build's (`mlxq.nn`, `mlxq.ops`):

* tests/quant_parity.rs:68-96   adaptable_linear_quantize_matches_reference
* tests/quant_parity.rs:98-127  quantized_forward_approximates_dense
* mlx-gen-sdxl/src/quant.rs:89-110  packed_row_slice_commutes_with_split
* mlx-gen-qwen-image/tests/q8_smoke.rs:15-60  q8_forward_close_to_dense

The reference draws its q8_smoke inputs from MLX's RNG (key 0), which cannot be reproduced
without MLX; the same shapes and distributions come from numpy seed 0 here.
"""
import os

import numpy as np
import pytest
import torch
from safetensors.numpy import load_file

from gpu_util import banner

pytestmark = pytest.mark.gpu

GOLD = load_file(os.path.join(os.path.dirname(__file__), "golden", "quant_q4q8.safetensors"))
GROUP_SIZE = 64


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def all_close(a, b, rtol, atol):
    """MLX's all_close (numpy semantics): |a - b| <= atol + rtol * |b| everywhere."""
    a = a.double()
    b = b.double()
    return bool(((a - b).abs() <= atol + rtol * b.abs()).all())


@pytest.mark.parametrize("bits", [8, 4])
def test_adaptable_linear_quantize_matches_reference(mlxq, bits):
    """tests/quant_parity.rs:68-96: AdaptableLinear::quantize packs the bf16 cast of the weight,
    so its forward equals quantize(bf16(w)) then quantized_matmul (rtol 1e-3, atol 1e-4); the
    packed triple itself is checked byte for byte as well."""
    banner("reference adaptable_linear_quantize", bits)
    from mlxq import nn, ops
    w = torch.from_numpy(GOLD["w"]).cuda()
    x = torch.from_numpy(GOLD["x"]).cuda()
    lin = nn.AdaptableLinear.dense(w.clone(), None)
    assert not lin.is_quantized()
    lin.quantize(bits, None)
    assert lin.is_quantized()
    out = lin.forward(x)
    wq, scales, biases = ops.quantize(w.to(torch.bfloat16), GROUP_SIZE, bits)
    reference = ops.quantized_matmul(x, wq, scales, biases, True, GROUP_SIZE, bits)
    q = lin.quantized
    assert torch.equal(q.weight, wq) and torch.equal(q.scales, scales) and torch.equal(q.biases, biases)
    assert out.dtype == reference.dtype == torch.float32
    assert all_close(out, reference, 1e-3, 1e-4), \
        f"q{bits}: AdaptableLinear quantized forward diverged from the bf16 reference"


def test_quantized_forward_approximates_dense(mlxq):
    """tests/quant_parity.rs:98-127: peak-relative error of the quantized forward against the
    dense one, Q8 < 2 %, Q4 < 12 % (the reference measured ~0.4 % and ~6.5 %)."""
    banner("reference quantized_forward_approximates_dense")
    from mlxq import nn
    w = torch.from_numpy(GOLD["w"]).cuda()
    x = torch.from_numpy(GOLD["x"]).cuda()
    dense = nn.AdaptableLinear.dense(w.clone(), None).forward(x)
    peak = dense.abs().max().item()
    for bits, max_rel in [(8, 0.02), (4, 0.12)]:
        q = nn.AdaptableLinear.dense(w.clone(), None)
        q.quantize(bits, None)
        out = q.forward(x)
        rel = (out.double() - dense.double()).abs().max().item() / peak
        print(f"    q{bits}: peak-relative error {rel:.4f}", flush=True)
        assert rel < max_rel, f"q{bits}: peak-relative error {rel:.4f} exceeds {max_rel}"


def test_packed_row_slice_commutes_with_split(mlxq):
    """mlx-gen-sdxl/src/quant.rs:89-110: packing a [4, 128] bf16 weight (cos(i)) whole and taking
    rows [0:2] of the codes equals packing rows [0:2] alone, byte for byte (Q4, group 64); the
    scales and biases are compared the same way here."""
    banner("reference packed_row_slice_commutes_with_split")
    from mlxq import ops
    full = torch.cos(torch.arange(4 * 128, dtype=torch.float32)).reshape(4, 128).to(torch.bfloat16).cuda()
    wq, sc, bi = ops.quantize(full, GROUP_SIZE, 4)
    ewq, esc, ebi = ops.quantize(full[0:2].contiguous(), GROUP_SIZE, 4)
    assert torch.equal(wq[0:2], ewq), "packed row-slice must equal packing the sliced rows"
    assert torch.equal(sc[0:2], esc) and torch.equal(bi[0:2], ebi)


def _mean_rel(a, b):
    """q8_smoke.rs:5-13: sum |a - b| / sum |b| over all elements, in f32 values."""
    a = a.float().double()
    b = b.float().double()
    return ((a - b).abs().sum() / b.abs().sum()).item()


def test_q8_forward_close_to_dense(mlxq):
    """mlx-gen-qwen-image/tests/q8_smoke.rs:15-60: for (out, in) shapes spanning a transformer's
    linears, a bf16 weight with a 0.1 bf16 bias, x [1, 4, in] in f32 and its bf16 cast: the Q8
    forward of either activation dtype stays within 5 % mean-abs-relative error of the dense f32
    forward (the activations reach quantized_matmul as they are)."""
    banner("reference q8_forward_close_to_dense")
    from mlxq import nn
    rng = np.random.default_rng(0)
    worst = 0.0
    for out_f, in_f in [(3072, 64), (3072, 128), (3072, 3072), (3072, 3584), (64, 3072)]:
        w = torch.from_numpy(rng.standard_normal((out_f, in_f)).astype(np.float32)).to(torch.bfloat16).cuda()
        b = torch.full((out_f,), 0.1, dtype=torch.float32).to(torch.bfloat16).cuda()
        x32 = torch.from_numpy(rng.standard_normal((1, 4, in_f)).astype(np.float32)).cuda()
        x16 = x32.to(torch.bfloat16)
        lin = nn.AdaptableLinear.dense(w, b)
        d32 = lin.forward(x32)
        lin.quantize(8, None)
        q32 = lin.forward(x32)
        q16 = lin.forward(x16)
        assert d32.dtype == q32.dtype == torch.float32 and q16.dtype == torch.bfloat16
        assert q32.shape == q16.shape == d32.shape == (1, 4, out_f)
        r32, r16, r1632 = _mean_rel(q32, d32), _mean_rel(q16, d32), _mean_rel(q16, q32)
        print(f"    [out={out_f}, in={in_f}] q8(f32)={r32:.4f}  q8(bf16)={r16:.4f}  q16-vs-q32={r1632:.4f}",
              flush=True)
        worst = max(worst, r32, r16)
    assert worst < 0.05, f"some Q8 shape/dtype diverged: worst {worst:.4f}"
