"""mlxq — MI355X (gfx950) group-wise affine Q4/Q8 quantized linear.

Drop-in for mlx-gen's quantized-linear path: the op triple ``quantize`` / ``dequantize`` /
``quantized_matmul`` (mlx_rs::ops as called from the reference's src/quant.rs and
src/adapters.rs) and the ``QuantizedLinear`` / ``AdaptableLinear`` layer surface built on it.
All compute runs in libmlxq_hip.so (hand-written HIP for gfx950) through its C ABI.
"""
from ._lib import (MLXQ_ACT_GELU, MLXQ_ACT_GELU_EXACT, MLXQ_ACT_GELU_TANH, MLXQ_ACT_NONE,
                   MLXQ_BFLOAT16, MLXQ_FLOAT16, MLXQ_FLOAT32, MlxqError, LIB_PATH, load)
from .ops import (DEFAULT_GROUP_SIZE, dequantize, embedding, linear, linear_out_dtype,
                  linear_workspace_size, lokr_residual, lora_residual, packed_bits, promote, qmm, qmm_experts, qmv,
                  qmv_valu, quantize, quantize_batched, quantized_matmul, swiglu)
from .nn import (Adapter, AdaptableLinear, LokrAdapter, QuantizedLinear, StackedExperts, TokenEmbedding,
                 has_packed_experts, lin, load_packed_experts, quantize_map)
from . import io

__all__ = [
    "MLXQ_ACT_GELU", "MLXQ_ACT_GELU_EXACT", "MLXQ_ACT_GELU_TANH", "MLXQ_ACT_NONE", "MLXQ_BFLOAT16",
    "MLXQ_FLOAT16", "MLXQ_FLOAT32", "MlxqError", "LIB_PATH", "load", "DEFAULT_GROUP_SIZE", "dequantize", "embedding",
    "linear", "linear_out_dtype", "linear_workspace_size", "lokr_residual", "lora_residual", "packed_bits", "promote",
    "qmm", "qmm_experts", "qmv", "qmv_valu", "quantize", "quantize_batched",
    "quantized_matmul", "swiglu", "Adapter", "AdaptableLinear", "LokrAdapter", "QuantizedLinear", "StackedExperts",
    "TokenEmbedding", "has_packed_experts", "lin", "load_packed_experts", "quantize_map", "io",
]
