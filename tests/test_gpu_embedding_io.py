"""GPU parity of the quantized token-embedding lookup and the packed-snapshot round trip.

TokenEmbedding::forward (reference src/nn.rs:42-58) is take_axis on the packed triple, then
dequantize, then a cast to f32; the oracle is the CPU dequantize of the whole table indexed by
the same ids.  Bit-exact: the lookup is integer gathering plus dequantize's single-rounded fma.
The snapshot round trip follows mlx-gen-flux/src/convert.rs:65-78 (load -> quantize_map -> save,
config.json gains a "quantization" block) and src/quant.rs:49-90 (lin / embedding loaders).
"""
import json
import os

import numpy as np
import pytest
import torch

from gpu_util import banner, bf16_normal, to_gpu, to_np, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sb_bf16", [True, False])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_embedding_bit_exact(mlxq, bits, gs, sb_bf16, out_dtype):
    banner("embedding", bits, gs, sb_bf16, out_dtype)
    rng = np.random.default_rng(bits * 100 + gs + int(sb_bf16))
    vocab, hidden = 300, 256
    w = bf16_normal(rng, (vocab, hidden), 0.02)
    wq, s, b = oracle.quantize(w, gs, bits, sb_bf16=sb_bf16)
    ids = rng.integers(0, vocab, size=(3, 17)).astype(np.int32)
    ids[0, :4] = [0, vocab - 1, 5, 5]  # ends of the table and a repeat
    sdt = torch.bfloat16 if sb_bf16 else torch.float32
    y = mlxq.embedding(torch.from_numpy(ids).cuda(), wq_to_gpu(wq), to_gpu(s, sdt), to_gpu(b, sdt),
                       gs, bits, out_dtype)
    assert y.shape == (3, 17, hidden) and y.dtype == out_dtype
    table = oracle.dequantize(wq, s, b, gs, bits, out_bf16=sb_bf16)
    ref = table[ids]
    if out_dtype == torch.bfloat16:
        ref = oracle.bf16_round(ref)
    assert np.array_equal(to_np(y), ref)


def test_embedding_out_of_range_ids_are_nan(mlxq):
    banner("embedding out of range")
    rng = np.random.default_rng(1)
    w = bf16_normal(rng, (64, 128), 0.02)
    wq, s, b = oracle.quantize(w, 64, 4, sb_bf16=True)
    ids = torch.tensor([3, -1, 64, 63], dtype=torch.int32, device="cuda")
    y = to_np(mlxq.embedding(ids, wq_to_gpu(wq), to_gpu(s), to_gpu(b), 64, 4))
    table = oracle.dequantize(wq, s, b, 64, 4, out_bf16=True)
    assert np.array_equal(y[0], table[3]) and np.array_equal(y[3], table[63])
    assert np.isnan(y[1]).all() and np.isnan(y[2]).all()


def test_token_embedding_quantize_then_forward(mlxq):
    """src/nn.rs:83-101: quantize(bits, cast_to_bf16) packs with group size 64; forward is f32."""
    banner("TokenEmbedding")
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((500, 192)) * 0.02).astype(np.float32)
    emb = mlxq.TokenEmbedding.dense(torch.from_numpy(w).cuda())
    ids = torch.from_numpy(rng.integers(0, 500, size=(2, 9))).cuda()
    dense = to_np(emb.forward(ids))
    assert np.array_equal(dense, w[ids.cpu().numpy()])
    emb.quantize(8, cast_to_bf16=True)
    assert emb.is_quantized() and emb.group_size == 64 and emb.bits == 8
    y = emb.forward(ids)
    assert y.dtype == torch.float32
    wq, s, b = oracle.quantize(oracle.bf16_round(w), 64, 8, sb_bf16=True)
    assert np.array_equal(to_np(emb.wq), wq)
    assert np.array_equal(to_np(y), oracle.dequantize(wq, s, b, 64, 8, out_bf16=True)[ids.cpu().numpy()])


def test_quantize_component_roundtrip(mlxq, tmp_path):
    """convert.rs:65-78 then the loaders of src/quant.rs:49-90 on the written snapshot."""
    banner("snapshot roundtrip")
    from safetensors.torch import save_file
    from mlxq import io, nn
    rng = np.random.default_rng(3)
    src, dst = tmp_path / "src", tmp_path / "dst"
    src.mkdir()
    wq_ = torch.from_numpy(bf16_normal(rng, (96, 128), 0.02)).to(torch.bfloat16)
    wo_ = torch.from_numpy(bf16_normal(rng, (128, 96), 0.02)).to(torch.bfloat16)
    tensors = {"blk.to_q.weight": wq_, "blk.to_q.bias": torch.zeros(96, dtype=torch.bfloat16),
               "blk.norm.weight": torch.ones(128, dtype=torch.bfloat16),
               "blk.proj.weight": wo_, "embed.weight": wq_.clone()}
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(src / "model-00001.safetensors"))
    (src / "config.json").write_text(json.dumps({"hidden_size": 128}))
    io.quantize_component(str(src), str(dst), 4, 32, lambda base: base in ("blk.to_q", "embed"))
    cfg = json.loads((dst / "config.json").read_text())
    assert cfg == {"hidden_size": 128, "quantization": {"bits": 4, "group_size": 32}}
    from safetensors import safe_open
    with safe_open(str(dst / "model.safetensors"), "pt") as f:
        assert f.get_slice("blk.to_q.weight").get_dtype() == "U32"
    m = io.load_dir_map(str(dst), device="cuda")
    assert set(m) == {"blk.to_q.weight", "blk.to_q.scales", "blk.to_q.biases", "blk.to_q.bias",
                      "blk.norm.weight", "blk.proj.weight", "embed.weight", "embed.scales",
                      "embed.biases"}
    q = nn.lin(m, "blk.to_q", True, 32)
    assert q.is_quantized() and q.quantized.bits == 4 and q.quantized.bias is not None
    ref = oracle.quantize(wq_.float().numpy(), 32, 4, sb_bf16=True)
    assert np.array_equal(to_np(q.quantized.weight), ref[0])
    assert np.array_equal(to_np(q.quantized.scales), ref[1])
    d = nn.lin(m, "blk.proj", False, 32)
    assert not d.is_quantized()
    e = nn.embedding(m, "embed", 32)
    assert e.is_quantized() and e.bits == 4
    ids = torch.tensor([[0, 95, 7]], device="cuda")
    table = oracle.dequantize(*ref, 32, 4, out_bf16=True)
    assert np.array_equal(to_np(e.forward(ids))[0], table[[0, 95, 7]])


def test_cpp_host_api_gpu_cases():
    """The C++ host API end to end (tests/host_cpp/host_test.cpp, `gpu`): golden fixture bit-exact,
    AdaptableLinear with bias and two LoRA adapters vs the oracle, TokenEmbedding, and the
    quantize_map -> save_map -> load_dir_map -> lin snapshot round trip."""
    import subprocess
    exe = os.path.join(os.path.dirname(__file__), "host_cpp", "host_test")
    assert os.path.exists(exe), "build() compiles tests/host_cpp/host_test"
    banner("C++ host API gpu cases")
    r = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0 and "ALL PASS" in r.stdout, r.stdout + r.stderr
