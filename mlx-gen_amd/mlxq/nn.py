"""Layer surface over the mlxq ops, mirroring the reference's quantized-linear seam.

  QuantizedLinear   ~ mlx_rs::nn::QuantizedLinear (try_from_linear used at src/adapters.rs:533-537)
  Adapter           ~ src/adapters.rs:231-270, LoRA arm (residual = scale * (x.A).B)
  LokrAdapter       ~ src/adapters.rs:231-270, LoKr arm (residual = scale * x.delta^T)
  AdaptableLinear   ~ src/adapters.rs:330-549 (dense / quantized base + adapter stack)
  quantize_map      ~ src/quant.rs:125-149 (offline converter primitive)
  TokenEmbedding    ~ src/nn.rs:20-101 (dense or packed table; forward gathers + dequantizes)
  lin / embedding   ~ src/quant.rs:49-90 (packed when `{base}.scales` is present, else dense)

Only the quantized base runs on libmlxq_hip.so.  The dense base (before ``quantize``) is the
reference's plain ``addmm``/``matmul`` and is evaluated with torch; it is not part of the
quantized path.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional

import torch

from . import ops
from ._lib import MLXQ_ACT_NONE, MLXQ_EUNSUPPORTED, MlxqError


@dataclass
class QuantizedLinear:
    """Packed triple + optional dense bias (MLX nn.QuantizedLinear)."""
    weight: torch.Tensor          # int32 storage of the uint32 packed codes [out, in*bits/32]
    scales: torch.Tensor          # [out, in/group_size]
    biases: torch.Tensor          # [out, in/group_size]
    bias: Optional[torch.Tensor]  # dense bias [out] or None
    group_size: int = ops.DEFAULT_GROUP_SIZE
    bits: int = 4

    @classmethod
    def try_from_linear(cls, weight: torch.Tensor, bias: Optional[torch.Tensor],
                        group_size: int = ops.DEFAULT_GROUP_SIZE, bits: int = 4):
        wq, s, b = ops.quantize(weight, group_size, bits)
        return cls(wq, s, b, bias, group_size, bits)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # src/adapters.rs:309-320: quantized_matmul, then the dense bias as a separate add in its
        # own dtype (an f32 bias promotes a bf16 product to f32, as MLX's add does).
        if self.bias is None:
            return ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                        self.group_size, self.bits)
        return ops.linear(x, self.weight, self.scales, self.biases, self.group_size, self.bits,
                          bias=self.bias)

    def in_features(self) -> int:
        # AdaptableLinear::base_shape (src/adapters.rs:491-502): in = scales.cols * group_size.
        return self.scales.shape[1] * self.group_size


@dataclass
class Adapter:
    """LoRA adapter: residual = scale * (x.A).B, A [in, r], B [r, out] (alpha/rank folded in B),
    the factors kept in their file dtype (src/adapters.rs:243-252)."""
    a: torch.Tensor
    b: torch.Tensor
    scale: float = 1.0

    def residual(self, x: torch.Tensor) -> torch.Tensor:
        """The dense-base arm's residual (src/adapters.rs:260-270): each op in
        promote(x, factors), the scale cast to that dtype.  Over a quantized base the library
        applies adapters instead (ops.linear, ops.lora_residual)."""
        dt = ops.promote(x.dtype, self.a.dtype)
        r = (x.to(dt) @ self.a.to(dt)) @ self.b.to(dt)
        return r * torch.tensor(self.scale, dtype=dt, device=r.device)


@dataclass
class LokrAdapter:
    """LoKr adapter (Adapter::Lokr, src/adapters.rs:234-235): residual = scale * x . delta^T with
    delta [out, in] the reconstructed kron delta (reconstruct_lokr_delta, :26-128; stored bf16),
    cast to the activation dtype (:263-266)."""
    delta: torch.Tensor
    scale: float = 1.0

    def residual(self, x: torch.Tensor) -> torch.Tensor:
        """The dense-base arm's residual, in x's dtype with the scale cast to it.  Over a quantized
        base the library applies it instead (ops.lokr_residual)."""
        # the transposed operand made contiguous: batched bf16 products on a transposed view are
        # avoided on this platform
        r = x @ self.delta.to(x.dtype).t().contiguous()
        return r * torch.tensor(self.scale, dtype=x.dtype, device=r.device)


@dataclass
class AdaptableLinear:
    """A linear base (dense or quantized) plus a stack of adapters: base(x) + sum residual(x)."""
    dense_weight: Optional[torch.Tensor] = None
    dense_bias: Optional[torch.Tensor] = None
    quantized: Optional[QuantizedLinear] = None
    adapters: List[object] = field(default_factory=list)  # Adapter (LoRA) or LokrAdapter

    @classmethod
    def dense(cls, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
        return cls(dense_weight=weight, dense_bias=bias)

    @classmethod
    def from_quantized_parts(cls, weight, scales, biases, bias, group_size: int, bits: int):
        return cls(quantized=QuantizedLinear(weight, scales, biases, bias, group_size, bits))

    def push(self, adapter) -> None:
        self.adapters.append(adapter)

    def set_adapters(self, adapters: List[object]) -> None:
        self.adapters = list(adapters)

    def is_quantized(self) -> bool:
        return self.quantized is not None

    def base_shape(self):
        if self.quantized is not None:
            q = self.quantized
            return [q.scales.shape[0], q.in_features()]
        return list(self.dense_weight.shape)

    def quantize(self, bits: int, group_size: Optional[int] = None) -> None:
        """src/adapters.rs:508-541: cast weight and bias to bf16, then pack (no-op if packed)."""
        if self.quantized is not None:
            return
        w = self.dense_weight.to(torch.bfloat16)
        b = None if self.dense_bias is None else self.dense_bias.to(torch.bfloat16)
        gs = ops.DEFAULT_GROUP_SIZE if group_size is None else group_size
        self.quantized = QuantizedLinear.try_from_linear(w, b, gs, bits)
        self.dense_weight = None
        self.dense_bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.quantized is not None:
            # src/adapters.rs:543-549 over the quantized base, all in the library: a leading LoRA
            # adapter rides in mlxq_linear's epilogue, each further adapter is one
            # mlxq_lora_residual / mlxq_lokr_residual (out = out + residual, promoted as MLX
            # promotes).  Factors and deltas keep their dtype.
            q = self.quantized
            for ad in self.adapters:
                if isinstance(ad, Adapter) and ad.a.shape[1] > 256:
                    raise MlxqError(MLXQ_EUNSUPPORTED, "AdaptableLinear: LoRA rank above 256")
            if not self.adapters:
                return q.forward(x)
            first = self.adapters[0] if isinstance(self.adapters[0], Adapter) else None
            out = ops.linear(x, q.weight, q.scales, q.biases, q.group_size, q.bits, bias=q.bias,
                             lora_a=None if first is None else first.a,
                             lora_b=None if first is None else first.b,
                             lora_scale=1.0 if first is None else first.scale,
                             activation=MLXQ_ACT_NONE)
            for ad in self.adapters[1:] if first is not None else self.adapters:
                if isinstance(ad, LokrAdapter):
                    out = ops.lokr_residual(x, out, ad.delta, ad.scale)
                else:
                    out = ops.lora_residual(x, out, ad.a, ad.b, ad.scale)
            return out
        else:
            w = self.dense_weight
            if self.dense_bias is not None:
                out = torch.addmm(self.dense_bias.to(x.dtype), x.reshape(-1, x.shape[-1]),
                                  w.to(x.dtype).t().contiguous()).reshape(*x.shape[:-1], w.shape[0])
            else:
                out = x @ w.to(x.dtype).t().contiguous()
        for ad in self.adapters:
            out = out + ad.residual(x)
        return out


def quantize_map(tensors: Dict[str, torch.Tensor], bits: int, group_size: int,
                 is_target: Callable[[str], bool]) -> Dict[str, torch.Tensor]:
    """src/quant.rs:125-149: pack every targeted, group-divisible 2-D `{base}.weight` (cast to
    bf16 first) into `{base}.weight/.scales/.biases`; pass everything else through.  Targets of
    one shape and device are packed together (ops.quantize_batched: the same triples as one
    quantize per weight, fewer launches); the output keeps the input's key order."""
    bases = {}
    groups: Dict[tuple, list] = {}
    for k, v in tensors.items():
        base = k[: -len(".weight")] if k.endswith(".weight") else None
        if (base is not None and is_target(base) and v.dim() == 2
                and v.shape[1] % group_size == 0 and v.shape[1] >= group_size):
            bases[k] = base
            groups.setdefault((tuple(v.shape), v.device), []).append(k)
    packed = {}
    for keys in groups.values():
        for k, triple in zip(keys, ops.quantize_batched([tensors[k].to(torch.bfloat16) for k in keys],
                                                        group_size, bits)):
            packed[k] = triple
    out: Dict[str, torch.Tensor] = {}
    for k, v in tensors.items():
        if k in packed:
            base = bases[k]
            out[f"{base}.weight"], out[f"{base}.scales"], out[f"{base}.biases"] = packed[k]
        else:
            out[k] = v
    return out


@dataclass
class TokenEmbedding:
    """Dense `[vocab, hidden]` table or a packed triple (src/nn.rs:20-101)."""
    weight: Optional[torch.Tensor] = None   # dense table
    wq: Optional[torch.Tensor] = None       # packed codes (int32 storage of uint32)
    scales: Optional[torch.Tensor] = None
    biases: Optional[torch.Tensor] = None
    group_size: int = ops.DEFAULT_GROUP_SIZE
    bits: int = 4

    @classmethod
    def dense(cls, weight: torch.Tensor):
        return cls(weight=weight)

    @classmethod
    def from_quantized_parts(cls, wq, scales, biases, group_size: int, bits: int):
        """src/nn.rs:60-81: adopt an already-packed table as is (no re-quantization)."""
        return cls(wq=wq, scales=scales, biases=biases, group_size=group_size, bits=bits)

    def is_quantized(self) -> bool:
        return self.wq is not None

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """src/nn.rs:42-58: rows of ids ([b, s] -> [b, s, hidden]), cast to f32."""
        if self.wq is not None:
            return ops.embedding(ids, self.wq, self.scales, self.biases, self.group_size, self.bits,
                                 torch.float32)
        return self.weight[ids.long()].to(torch.float32)

    def quantize(self, bits: int, cast_to_bf16: bool) -> None:
        """src/nn.rs:83-101: pack with group size 64 (bf16 first when cast_to_bf16); no-op if
        already packed."""
        if self.wq is not None:
            return
        w = self.weight.to(torch.bfloat16) if cast_to_bf16 else self.weight
        self.wq, self.scales, self.biases = ops.quantize(w, 64, bits)
        self.group_size, self.bits = 64, bits
        self.weight = None


@dataclass
class StackedExperts:
    """One MoE expert projection across all E experts as the stacked packed triple plus dense bias
    (mlx-gen-lens/src/text_encoder/gpt_oss.rs:478-487, StackedExpertPack): weight [E, out,
    in*bits/32], scales/biases [E, out, in/group_size], bias [E, out]."""
    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    bias: torch.Tensor
    group_size: int = ops.DEFAULT_GROUP_SIZE
    bits: int = 4

    @property
    def num_experts(self) -> int:
        return self.weight.shape[0]

    def split(self) -> List[QuantizedLinear]:
        """Per-expert packs, the axis-0 split of mlx-gen-lens/src/quant.rs:111-137 (views, no copy;
        the ops copy a view whose start the library cannot take, such as a scales slice that
        starts mid-word)."""
        return [QuantizedLinear(self.weight[e], self.scales[e], self.biases[e], self.bias[e],
                                self.group_size, self.bits) for e in range(self.num_experts)]

    def forward(self, x: torch.Tensor, per_expert: bool = False) -> torch.Tensor:
        """Proj::forward of every expert (gpt_oss.rs:412-425) in one call: x [..., in] shared by all
        experts, or [E, ..., in] with per_expert=True; returns [E, ..., out]."""
        return ops.qmm_experts(x, self.weight, self.scales, self.biases, self.group_size, self.bits,
                               bias=self.bias, per_expert=per_expert)


def has_packed_experts(w: Dict[str, torch.Tensor], prefix: str, name: str) -> bool:
    """mlx-gen-lens/src/quant.rs:80-83: a pre-quantized snapshot stores `{prefix}.experts.{name}_proj.scales`."""
    return f"{prefix}.experts.{name}_proj.scales" in w


def load_packed_experts(w: Dict[str, torch.Tensor], prefix: str, name: str) -> StackedExperts:
    """mlx-gen-lens/src/quant.rs:93-137: the stacked triple `{prefix}.experts.{name}_proj.{weight,
    scales,biases}` [E, out, ...] plus the dense bias `{prefix}.experts.{name}_proj_bias` [E, out];
    bits inferred from the packed shapes, group size 64.  `.split()` gives the per-expert packs."""
    base = f"{prefix}.experts.{name}_proj"
    wq = _require(w, f"{base}.weight")
    scales = _require(w, f"{base}.scales")
    biases = _require(w, f"{base}.biases")
    bias = _require(w, f"{prefix}.experts.{name}_proj_bias")
    bits = ops.packed_bits(wq[0], scales[0], ops.DEFAULT_GROUP_SIZE)
    return StackedExperts(wq, scales, biases, bias, ops.DEFAULT_GROUP_SIZE, bits)


def _require(w: Dict[str, torch.Tensor], key: str) -> torch.Tensor:
    if key not in w:
        raise KeyError(f"missing tensor {key!r}")  # Weights::require (reference src/weights.rs)
    return w[key]


def lin(w: Dict[str, torch.Tensor], base: str, bias: bool, group_size: int) -> AdaptableLinear:
    """src/quant.rs:49-68: `{base}` as a packed AdaptableLinear when `{base}.scales` exists (bits
    inferred by packed_bits), else dense; `bias` also loads the dense `{base}.bias`."""
    b = _require(w, f"{base}.bias") if bias else None
    scales = w.get(f"{base}.scales")
    if scales is not None:
        wq = _require(w, f"{base}.weight")
        bits = ops.packed_bits(wq, scales, group_size)
        return AdaptableLinear.from_quantized_parts(wq, scales, _require(w, f"{base}.biases"), b,
                                                    group_size, bits)
    return AdaptableLinear.dense(_require(w, f"{base}.weight"), b)


def embedding(w: Dict[str, torch.Tensor], base: str, group_size: int) -> TokenEmbedding:
    """src/quant.rs:70-90: the embedding analogue of lin."""
    scales = w.get(f"{base}.scales")
    if scales is not None:
        wq = _require(w, f"{base}.weight")
        bits = ops.packed_bits(wq, scales, group_size)
        return TokenEmbedding.from_quantized_parts(wq, scales, _require(w, f"{base}.biases"),
                                                   group_size, bits)
    return TokenEmbedding.dense(_require(w, f"{base}.weight"))
