"""Host-side logic on the CPU: the packed/dense loaders (src/quant.rs:49-90), the packed-snapshot
I/O (src/quant.rs:92-116, mlx-gen-flux/src/convert.rs:46-63) and the reference's golden fixture
read back through it.  No GPU work: only host code and the library's shape helper run."""
import json
import os
import shutil

import numpy as np
import pytest
import torch


def test_lin_and_embedding_choose_packed_or_dense():
    from mlxq import nn
    packed = {"a.weight": torch.zeros((6, 16), dtype=torch.int32),   # 6 rows, K=128 at Q4
              "a.scales": torch.zeros((6, 2), dtype=torch.bfloat16),
              "a.biases": torch.zeros((6, 2), dtype=torch.bfloat16),
              "a.bias": torch.zeros(6),
              "q8.weight": torch.zeros((4, 32), dtype=torch.int32),  # K=128 at Q8
              "q8.scales": torch.zeros((4, 2)), "q8.biases": torch.zeros((4, 2)),
              "d.weight": torch.zeros((3, 5))}
    a = nn.lin(packed, "a", True, 64)
    assert a.is_quantized() and a.quantized.bits == 4 and a.base_shape() == [6, 128]
    assert a.quantized.bias is not None
    assert nn.lin(packed, "q8", False, 64).quantized.bits == 8
    d = nn.lin(packed, "d", False, 64)
    assert not d.is_quantized() and d.base_shape() == [3, 5]
    e = nn.embedding(packed, "a", 64)
    assert e.is_quantized() and e.bits == 4
    assert not nn.embedding(packed, "d", 64).is_quantized()
    with pytest.raises(KeyError):
        nn.lin(packed, "d", True, 64)  # bias requested but absent: Weights::require fails
    bad = dict(packed, **{"a.weight": torch.zeros((6, 24), dtype=torch.int32)})
    from mlxq import MlxqError
    with pytest.raises(MlxqError):
        nn.lin(bad, "a", False, 64)  # 24 words cannot pack 128 inputs at 4 or 8 bits


def test_load_packed_experts_host_logic():
    """mlx-gen-lens/src/quant.rs:80-137: the stacked expert triple is detected by its scales key,
    bits come from the packed shapes, and the axis-0 split yields per-expert packs with bias."""
    from mlxq import nn
    E, N, K = 3, 8, 128
    w = {"m.experts.gate_up_proj.weight": torch.zeros((E, N, K // 8), dtype=torch.int32),
         "m.experts.gate_up_proj.scales": torch.zeros((E, N, K // 64), dtype=torch.bfloat16),
         "m.experts.gate_up_proj.biases": torch.zeros((E, N, K // 64), dtype=torch.bfloat16),
         "m.experts.gate_up_proj_bias": torch.arange(E * N, dtype=torch.float32).reshape(E, N)}
    assert nn.has_packed_experts(w, "m", "gate_up") and not nn.has_packed_experts(w, "m", "down")
    st = nn.load_packed_experts(w, "m", "gate_up")
    assert st.bits == 4 and st.group_size == 64 and st.num_experts == E
    parts = st.split()
    assert len(parts) == E and parts[1].weight.shape == (N, K // 8) and parts[1].in_features() == K
    assert torch.equal(parts[2].bias, w["m.experts.gate_up_proj_bias"][2])
    with pytest.raises(KeyError):
        nn.load_packed_experts(w, "m", "down")


def test_snapshot_io_keeps_u32_and_config(tmp_path):
    from mlxq import io
    from safetensors import safe_open
    m = {"x.weight": torch.tensor([[1, -2]], dtype=torch.int32),
         "x.scales": torch.ones((1, 1), dtype=torch.bfloat16),
         "x.biases": torch.zeros((1, 1), dtype=torch.bfloat16),
         "n.weight": torch.tensor([7], dtype=torch.int32)}   # not packed: stays I32
    io.save_map(str(tmp_path / "out" / "model.safetensors"), m)
    with safe_open(str(tmp_path / "out" / "model.safetensors"), "pt") as f:
        assert f.get_slice("x.weight").get_dtype() == "U32"
        assert f.get_slice("n.weight").get_dtype() == "I32"
    back = io.load_dir_map(str(tmp_path / "out"))
    assert back["x.weight"].dtype == torch.int32 and torch.equal(back["x.weight"], m["x.weight"])
    assert torch.equal(back["n.weight"], m["n.weight"])
    io.write_quantized_config(str(tmp_path / "missing"), str(tmp_path / "cfg"), 8, 64)
    assert json.loads((tmp_path / "cfg" / "config.json").read_text()) == {
        "quantization": {"bits": 8, "group_size": 64}}


def test_golden_fixture_through_load_dir_map(tmp_path):
    """The reference's own fixture (U32 codes) reads back bit-identically through the loader."""
    from mlxq import io
    from safetensors.numpy import load_file
    src = os.path.join(os.path.dirname(__file__), "golden", "quant_q4q8.safetensors")
    shutil.copy(src, tmp_path / "quant_q4q8.safetensors")
    m = io.load_dir_map(str(tmp_path))
    gold = load_file(src)
    for bits in (4, 8):
        assert np.array_equal(m[f"q{bits}.wq"].numpy().view(np.uint32), gold[f"q{bits}.wq"])
        assert np.array_equal(m[f"q{bits}.scales"].numpy(), gold[f"q{bits}.scales"])


HOST_TEST = os.path.join(os.path.dirname(__file__), "host_cpp", "host_test")


def test_cpp_host_api_cpu_cases():
    """The C++ host API's file formats and host logic (tests/host_cpp/host_test.cpp, `cpu`)."""
    import subprocess
    assert os.path.exists(HOST_TEST), "build() compiles tests/host_cpp/host_test"
    r = subprocess.run([HOST_TEST, "cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ALL PASS" in r.stdout, r.stdout + r.stderr
