"""ctypes binding of libmlxq_hip.so (the C ABI declared in include/mlxq.h).

The shared library is built in-tree (``mlx-gen_amd/mlxq/libmlxq_hip.so``) by
``mlx-gen_amd/csrc/Makefile``.  Loading fails loudly when it is missing: there is no CPU or
PyTorch fallback behind these entry points.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmlxq_hip.so")

MLXQ_FLOAT32 = 0
MLXQ_BFLOAT16 = 1
MLXQ_FLOAT16 = 2  # activations only (SDXL's fp16 stream); promotes to f32 against bf16 / f32

MLXQ_OK = 0
MLXQ_EINVAL = 1
MLXQ_EUNSUPPORTED = 2
MLXQ_EDEVICE = 3

MLXQ_ACT_NONE = 0
MLXQ_ACT_GELU = 1
MLXQ_ACT_GELU_TANH = 2
MLXQ_ACT_GELU_EXACT = 3

# Size of the static per-device scratch array behind mlxq_linear_noalloc.
MLXQ_NOALLOC_SCRATCH_BYTES = 8 << 20

# Every symbol include/mlxq.h declares; tests check the library exports all of them.
EXPORTS = (
    "mlxq_last_error",
    "mlxq_version",
    "mlxq_quantize",
    "mlxq_quantize_batched",
    "mlxq_dequantize",
    "mlxq_quantized_matmul",
    "mlxq_qmm",
    "mlxq_qmv",
    "mlxq_qmv_valu",
    "mlxq_linear_workspace_size",
    "mlxq_linear_out_dtype",
    "mlxq_linear",
    "mlxq_linear_noalloc",
    "mlxq_packed_bits",
    "mlxq_embedding",
    "mlxq_lora_residual",
    "mlxq_lora_residual_workspace_size",
    "mlxq_lokr_residual",
    "mlxq_lokr_residual_workspace_size",
    "mlxq_cast",
    "mlxq_swiglu",
    "mlxq_qmm_experts",
)


class MlxqError(RuntimeError):
    """A non-zero mlxq_status, with the library's thread-local message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[mlxq status {status}] {message}")
        self.status = status


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("bias", ctypes.c_void_p),
        ("lora_a", ctypes.c_void_p),
        ("lora_b", ctypes.c_void_p),
        ("lora_rank", ctypes.c_int64),
        ("lora_scale", ctypes.c_float),
        ("activation", ctypes.c_int),
        ("bias_dtype", ctypes.c_int),
        ("lora_dtype", ctypes.c_int),
    ]


_lib = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


def load():
    """Load libmlxq_hip.so and declare the prototypes (raises if the library is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C mlx-gen_amd/csrc` "
            "(or __graft_entry__.build()); there is no fallback implementation")
    lib = ctypes.CDLL(LIB_PATH)
    lib.mlxq_last_error.restype = ctypes.c_char_p
    lib.mlxq_version.restype = ctypes.c_char_p
    lib.mlxq_quantize.argtypes = [_vp, _int, _i64, _i64, _int, _int, _vp, _vp, _vp, _vp]
    _pp = ctypes.POINTER(ctypes.c_void_p)
    lib.mlxq_quantize_batched.argtypes = [_pp, _int, _int, _i64, _i64, _int, _int, _pp, _pp, _pp, _vp]
    lib.mlxq_dequantize.argtypes = [_vp, _vp, _vp, _int, _i64, _i64, _int, _int, _vp, _vp]
    lib.mlxq_quantized_matmul.argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _vp, _int, _i64, _int,
                                          _int, _int, _vp, _vp]
    for name in ("mlxq_qmm", "mlxq_qmv", "mlxq_qmv_valu"):
        getattr(lib, name).argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _vp, _int, _i64, _int, _int,
                                       _vp, _vp]
    lib.mlxq_linear_workspace_size.argtypes = [_int, _int, _i64, _i64, ctypes.POINTER(Epilogue)]
    lib.mlxq_linear_workspace_size.restype = ctypes.c_size_t
    lib.mlxq_linear_out_dtype.argtypes = [_int, _int, ctypes.POINTER(Epilogue)]
    lib.mlxq_linear_out_dtype.restype = _int
    lib.mlxq_lora_residual_workspace_size.argtypes = [_int, _int, _i64, _i64, _i64]
    lib.mlxq_lora_residual_workspace_size.restype = ctypes.c_size_t
    lib.mlxq_linear.argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _vp, _int, _i64, _int, _int,
                                ctypes.POINTER(Epilogue), _vp, _vp, ctypes.c_size_t, _vp]
    lib.mlxq_linear_noalloc.argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _vp, _int, _i64, _int,
                                        _int, ctypes.POINTER(Epilogue), _vp, _vp]
    lib.mlxq_packed_bits.argtypes = [_i64, _i64, _int]
    lib.mlxq_lora_residual.argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _int, _i64, _i64,
                                       ctypes.c_float, _vp, _int, _vp, _vp, ctypes.c_size_t, _vp]
    lib.mlxq_lokr_residual_workspace_size.argtypes = [_int, _i64, _i64]
    lib.mlxq_lokr_residual_workspace_size.restype = ctypes.c_size_t
    lib.mlxq_lokr_residual.argtypes = [_vp, _int, _i64, _i64, _vp, _int, _i64, ctypes.c_float, _vp,
                                       _int, _vp, _vp, ctypes.c_size_t, _vp]
    lib.mlxq_cast.argtypes = [_vp, _int, _vp, _int, _i64, _vp]
    lib.mlxq_qmm_experts.argtypes = [_vp, _int, _int, _i64, _i64, _i64, _vp, _vp, _vp, _int, _vp,
                                     _int, _i64, _int, _int, _vp, _vp]
    lib.mlxq_swiglu.argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _int, _i64, _int,
                                _int, _vp, _vp]
    lib.mlxq_embedding.argtypes = [_vp, _i64, _vp, _vp, _vp, _int, _i64, _i64, _int, _int, _vp, _int,
                                   _vp]
    for name in ("mlxq_quantize", "mlxq_quantize_batched", "mlxq_dequantize", "mlxq_quantized_matmul", "mlxq_qmm",
                 "mlxq_qmv", "mlxq_qmv_valu", "mlxq_linear", "mlxq_linear_noalloc", "mlxq_packed_bits", "mlxq_embedding",
                 "mlxq_lora_residual", "mlxq_lokr_residual", "mlxq_cast", "mlxq_swiglu",
                 "mlxq_qmm_experts"):
        getattr(lib, name).restype = _int
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != MLXQ_OK:
        raise MlxqError(status, load().mlxq_last_error().decode())
