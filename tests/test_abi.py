"""CPU-side checks of the C ABI and the host logic (no GPU compute is launched here).

* libmlxq_hip.so loads and exports every function include/mlxq.h declares;
* host-only entry points (packed_bits, argument validation that fails before any device work)
  behave like the reference's host code, returning errors instead of panicking;
* the layer mirror's host logic (quantize_map target selection) matches src/quant.rs:125-149.
"""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mlxq.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlxq_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from mlxq import _lib
    return _lib.load()


def test_header_and_binding_agree():
    from mlxq import _lib
    assert sorted(_lib.EXPORTS) == _declared()


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib._name], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (mlxq_\w+)", out))
    missing = [s for s in _declared() if s not in exported]
    assert not missing, missing
    for s in _declared():
        assert hasattr(lib, s)


def test_packed_bits(lib):
    # quant::packed_bits (src/quant.rs:38-41): in = scales.cols*gs; bits = wq.cols*32/in.
    assert lib.mlxq_packed_bits(384, 48, 64) == 4      # [3072,3072] Q4 g64
    assert lib.mlxq_packed_bits(1280, 80, 64) == 8     # Wan [5120,5120] Q8 g64
    assert lib.mlxq_packed_bits(96, 24, 32) == 4
    # Malformed triples are errors, not panics.
    assert lib.mlxq_packed_bits(384, 0, 64) == -1
    assert b"malformed" in lib.mlxq_last_error()
    assert lib.mlxq_packed_bits(100, 48, 64) == -1
    assert lib.mlxq_packed_bits(192, 48, 64) == -1    # would be 2-bit


def test_validation_rejects_before_device_work(lib):
    from mlxq import _lib
    null = ctypes.c_void_p(0)
    st = lib.mlxq_quantize(null, 1, 4, 100, 64, 4, null, null, null, null)
    assert st == _lib.MLXQ_EINVAL and b"multiple of group_size" in lib.mlxq_last_error()
    st = lib.mlxq_quantize(null, 1, 4, 128, 64, 3, null, null, null, null)
    assert st == _lib.MLXQ_EINVAL and b"bits" in lib.mlxq_last_error()
    st = lib.mlxq_quantize(null, 1, 4, 128, 48, 4, null, null, null, null)
    assert st == _lib.MLXQ_EINVAL and b"group_size" in lib.mlxq_last_error()
    st = lib.mlxq_quantize(null, 7, 4, 128, 64, 4, null, null, null, null)
    assert st == _lib.MLXQ_EINVAL and b"dtype" in lib.mlxq_last_error()
    st = lib.mlxq_quantize(null, 1, 4, 128, 64, 4, null, null, null, null)
    assert st == _lib.MLXQ_EINVAL and b"null" in lib.mlxq_last_error()
    st = lib.mlxq_quantized_matmul(null, 1, 4, 128, null, null, null, 1, 8, 0, 64, 4, null, null)
    assert st == _lib.MLXQ_EUNSUPPORTED and b"transpose" in lib.mlxq_last_error()
    st = lib.mlxq_qmv(ctypes.c_void_p(16), 1, 9, 128, ctypes.c_void_p(16), ctypes.c_void_p(16),
                      ctypes.c_void_p(16), 1, 8, 64, 4, ctypes.c_void_p(16), null)
    assert st == _lib.MLXQ_EINVAL and b"GEMV limit" in lib.mlxq_last_error()
    st = lib.mlxq_qmm(ctypes.c_void_p(16), 0, 16, 128, ctypes.c_void_p(16), ctypes.c_void_p(16),
                      ctypes.c_void_p(16), 1, 8, 64, 4, ctypes.c_void_p(16), null)
    assert st == _lib.MLXQ_EINVAL and b"bfloat16" in lib.mlxq_last_error()
    st = lib.mlxq_qmm(ctypes.c_void_p(8), 1, 16, 128, ctypes.c_void_p(16), ctypes.c_void_p(16),
                      ctypes.c_void_p(16), 1, 8, 64, 4, ctypes.c_void_p(16), null)
    assert st == _lib.MLXQ_EINVAL and b"aligned" in lib.mlxq_last_error()
    st = lib.mlxq_qmv(ctypes.c_void_p(16), 1, 4, 128, ctypes.c_void_p(16), ctypes.c_void_p(18),
                      ctypes.c_void_p(16), 1, 8, 64, 4, ctypes.c_void_p(16), null)
    assert st == _lib.MLXQ_EINVAL and b"scales must be 4-byte aligned" in lib.mlxq_last_error()
    # Empty problems are successful no-ops.
    assert lib.mlxq_quantize(null, 1, 0, 128, 64, 4, null, null, null, null) == _lib.MLXQ_OK


def test_linear_workspace_size(lib):
    assert lib.mlxq_linear_workspace_size(100, 200, 0) == 0
    # xa [M,16] and lbt [N,16] at 4 B/element, xa padded to 256 B.
    assert lib.mlxq_linear_workspace_size(4608, 3072, 16) == 4608 * 16 * 4 + 3072 * 16 * 4
    assert lib.mlxq_linear_workspace_size(3, 5, 8) == 256 + 5 * 16 * 4


def test_quantize_map_host_logic(monkeypatch):
    """src/quant.rs:125-149 target/shape guard, with the packing op stubbed out on the CPU."""
    import torch
    from mlxq import nn, ops

    calls = []

    def fake_quantize(w, gs, bits):
        calls.append((tuple(w.shape), w.dtype, gs, bits))
        return (torch.zeros(1), torch.zeros(1), torch.zeros(1))

    monkeypatch.setattr(ops, "quantize", fake_quantize)
    m = {
        "a.weight": torch.zeros(8, 128),
        "a.bias": torch.zeros(8),
        "b.weight": torch.zeros(8, 100),     # K not divisible by gs -> dense
        "c.weight": torch.zeros(8, 32),      # K < gs -> dense
        "norm.weight": torch.zeros(128),     # 1-D -> dense
        "skip.weight": torch.zeros(8, 128),  # not a target -> dense
    }
    out = nn.quantize_map(m, 4, 64, lambda base: base != "skip")
    assert set(out) == {"a.weight", "a.scales", "a.biases", "a.bias", "b.weight", "c.weight",
                        "norm.weight", "skip.weight"}
    assert calls == [((8, 128), torch.bfloat16, 64, 4)]
