"""Packed-snapshot I/O: the read/write side of the reference's offline pre-quantization.

  load_dir_map            ~ src/quant.rs:92-99   (every tensor of a dir's *.safetensors)
  save_map                ~ src/quant.rs:101-116 (one safetensors file)
  write_quantized_config  ~ mlx-gen-flux/src/convert.rs:46-63 ("quantization": {bits, group_size})
  quantize_component      ~ mlx-gen-flux/src/convert.rs:65-78 (load -> quantize_map -> save)

Packed codes live in int32 tensors in memory (same bits as MLX's uint32); on disk they are
written as U32, which is how MLX stores them, so snapshots interchange with the reference.
"""
from __future__ import annotations

import glob
import json
import os
from typing import Callable, Dict

import torch
from safetensors.torch import load_file, save_file

from .nn import quantize_map


def _packed_keys(m: Dict[str, torch.Tensor]):
    return {k for k in m if k.endswith(".weight") and k[: -len(".weight")] + ".scales" in m}


def load_dir_map(path: str, device="cpu") -> Dict[str, torch.Tensor]:
    """All tensors of `path`'s *.safetensors (sharded or single).  U32 packed codes come back as
    int32 views of the same bits."""
    files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors under {path}")
    out: Dict[str, torch.Tensor] = {}
    for f in files:
        for k, v in load_file(f, device=str(device)).items():
            out[k] = v.view(torch.int32) if v.dtype == torch.uint32 else v
    return out


def save_map(path: str, m: Dict[str, torch.Tensor]) -> None:
    """Write `m` to one safetensors file; packed `{base}.weight` codes are stored as U32."""
    packed = _packed_keys(m)
    d = {}
    for k, v in m.items():
        v = v.detach().contiguous().cpu()
        d[k] = v.view(torch.uint32) if (k in packed and v.dtype == torch.int32) else v
    parent = os.path.dirname(path)
    if parent:
        os.makedirs(parent, exist_ok=True)
    save_file(d, path)


def write_quantized_config(src: str, dst: str, bits: int, group_size: int) -> None:
    """Copy src/config.json to dst/config.json with a "quantization": {bits, group_size} block
    (an absent source config starts from {})."""
    cfg_path = os.path.join(src, "config.json")
    cfg = {}
    if os.path.exists(cfg_path):
        with open(cfg_path) as f:
            cfg = json.load(f)
    cfg["quantization"] = {"bits": bits, "group_size": group_size}
    os.makedirs(dst, exist_ok=True)
    with open(os.path.join(dst, "config.json"), "w") as f:
        json.dump(cfg, f, indent=2)


def quantize_component(src: str, dst: str, bits: int, group_size: int,
                       is_target: Callable[[str], bool], device="cuda") -> None:
    """Pre-quantize one component dir into dst/model.safetensors + annotated config.json."""
    m = {k: v.to(device) for k, v in load_dir_map(src).items()}
    save_map(os.path.join(dst, "model.safetensors"), quantize_map(m, bits, group_size, is_target))
    write_quantized_config(src, dst, bits, group_size)
