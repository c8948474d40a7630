"""Op-level API over libmlxq_hip.so, mirroring the three MLX ops the reference calls.

Reference call sites (mlx_rs::ops, MLX 0.31.2 via pmetal-mlx-rs 0.25.8):
  quantize(w, group_size, bits)                          src/quant.rs:140, src/nn.rs:91-93
  dequantize(wq, scales, biases, group_size, bits)       src/nn.rs:55
  quantized_matmul(x, wq, scales, biases, transpose,
                   group_size, bits)                     src/adapters.rs:309-317

Tensors are torch tensors on the GPU (torch only supplies device memory and the current
stream).  bf16 and f32 are supported; outputs follow MLX's dtype rules (scales/biases in the
weight dtype, matmul output in the activation dtype).  Errors raise ``MlxqError`` carrying the
library's status and message.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import MLXQ_BFLOAT16, MLXQ_FLOAT32, Epilogue, check

DEFAULT_GROUP_SIZE = 64  # src/quant.rs:32


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return MLXQ_BFLOAT16
    if t.dtype == torch.float32:
        return MLXQ_FLOAT32
    raise TypeError(f"mlxq supports bfloat16 and float32 tensors, got {t.dtype}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("mlxq operates on GPU tensors only")


def _contig(t):
    return None if t is None else t.contiguous()


def quantize(w: torch.Tensor, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4):
    """Affine group quantization of w [N, K] -> (wq u32-as-int32 [N, K*bits/32], scales, biases)."""
    _need_gpu(w)
    if w.dim() != 2:
        raise ValueError(f"quantize expects a 2-D weight, got shape {tuple(w.shape)}")
    w = w.contiguous()
    N, K = w.shape
    # Packed words are stored in an int32 tensor (same bits as MLX's uint32 array).
    wq = torch.empty((N, max(K * bits // 32, 0)), dtype=torch.int32, device=w.device)
    gcols = K // group_size if group_size > 0 else 0
    s = torch.empty((N, gcols), dtype=w.dtype, device=w.device)
    b = torch.empty((N, gcols), dtype=w.dtype, device=w.device)
    check(_lib.load().mlxq_quantize(_ptr(w), _dt(w), N, K, group_size, bits, _ptr(wq), _ptr(s),
                                    _ptr(b), _stream(w.device)))
    return wq, s, b


def _k_of(wq: torch.Tensor, bits: int) -> int:
    return wq.shape[-1] * 32 // bits


def dequantize(wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4):
    _need_gpu(wq, scales, biases)
    wq, scales, biases = wq.contiguous(), scales.contiguous(), biases.contiguous()
    N = wq.shape[0]
    K = _k_of(wq, bits)
    out = torch.empty((N, K), dtype=scales.dtype, device=wq.device)
    check(_lib.load().mlxq_dequantize(_ptr(wq), _ptr(scales), _ptr(biases), _dt(scales), N, K,
                                      group_size, bits, _ptr(out), _stream(wq.device)))
    return out


def _mm(entry, x, wq, scales, biases, group_size, bits, *extra, out=None):
    _need_gpu(x, wq, scales, biases)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K).contiguous()
    wq, scales, biases = wq.contiguous(), scales.contiguous(), biases.contiguous()
    M, N = x2.shape[0], wq.shape[0]
    if out is None:
        y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    else:
        if out.dtype != x.dtype or out.device != x.device or out.numel() != M * N or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous {x.dtype} tensor of {M * N} elements on {x.device}")
        y = out
    args = [_ptr(x2), _dt(x2), M, K, _ptr(wq), _ptr(scales), _ptr(biases), _dt(scales), N]
    if entry == "mlxq_quantized_matmul":
        args.append(int(extra[0]))
    args += [group_size, bits, _ptr(y), _stream(x.device)]
    check(getattr(_lib.load(), entry)(*args))
    return y.reshape(*lead, N)


def quantized_matmul(x, wq, scales, biases, transpose: bool = True,
                     group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """y = x . dequantize(W)^T (transpose=True, the only form the reference uses)."""
    return _mm("mlxq_quantized_matmul", x, wq, scales, biases, group_size, bits, transpose, out=out)


def qmm(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """Force the MFMA GEMM kernel (bf16 activations)."""
    return _mm("mlxq_qmm", x, wq, scales, biases, group_size, bits, out=out)


def qmv(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """Force the GEMV kernel (M <= 8)."""
    return _mm("mlxq_qmv", x, wq, scales, biases, group_size, bits, out=out)


def embedding(ids, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4,
              out_dtype=torch.float32):
    """TokenEmbedding::forward's quantized arm (src/nn.rs:42-58): gather the packed rows of ids
    (any shape, int32/int64), dequantize, cast to out_dtype (f32 like the reference).  Ids outside
    [0, vocab) give NaN rows."""
    _need_gpu(ids, wq, scales, biases)
    wq, scales, biases = wq.contiguous(), scales.contiguous(), biases.contiguous()
    flat = ids.reshape(-1).to(torch.int32).contiguous()
    vocab = wq.shape[0]
    hidden = _k_of(wq, bits)
    out = torch.empty((flat.numel(), hidden), dtype=out_dtype, device=wq.device)
    odt = MLXQ_BFLOAT16 if out_dtype == torch.bfloat16 else MLXQ_FLOAT32
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"embedding: out_dtype must be bfloat16 or float32, got {out_dtype}")
    check(_lib.load().mlxq_embedding(_ptr(flat), flat.numel(), _ptr(wq), _ptr(scales), _ptr(biases),
                                     _dt(scales), vocab, hidden, group_size, bits, _ptr(out), odt,
                                     _stream(wq.device)))
    return out.reshape(*ids.shape, hidden)


def swiglu(x, gate, up, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """Fused decode SwiGLU h = silu(gate(x)) * up(x) (mlx-gen-sensenova/src/qwen3.rs:178-181), gate
    and up given as packed (wq, scales, biases) triples of shape [F, K].  Decode form only (bf16,
    M <= 8); other shapes raise MlxqError with status MLXQ_EUNSUPPORTED."""
    _need_gpu(x, *gate, *up)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K).contiguous()
    g = [t.contiguous() for t in gate]
    u = [t.contiguous() for t in up]
    M, F = x2.shape[0], g[0].shape[0]
    h = out if out is not None else torch.empty((M, F), dtype=x.dtype, device=x.device)
    check(_lib.load().mlxq_swiglu(_ptr(x2), _dt(x2), M, K, _ptr(g[0]), _ptr(g[1]), _ptr(g[2]), _ptr(u[0]),
                                  _ptr(u[1]), _ptr(u[2]), _dt(g[1]), F, group_size, bits, _ptr(h),
                                  _stream(x.device)))
    return h.reshape(*lead, F)


def qmm_experts(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, bias=None,
                per_expert: bool = False, out=None):
    """Every expert of a stacked packed projection: y[e] = quantized_matmul(x[e], wq[e], scales[e],
    biases[e], transpose=True) + bias[e] — Proj::forward of the quantized MoE experts
    (mlx-gen-lens/src/text_encoder/gpt_oss.rs:412-425) over the axis-0 split of the stacked pack
    (mlx-gen-lens/src/quant.rs:111-137).  wq [E, N, K*bits/32], scales/biases [E, N, K/gs], bias
    [E, N] in the activation dtype or None.  x [..., K] is shared by every expert, or with
    per_expert=True it is [E, ..., K] (one input per expert).  Returns [E, ..., N]."""
    _need_gpu(x, wq, scales, biases, bias)
    E, N = wq.shape[0], wq.shape[1]
    K = x.shape[-1]
    if per_expert:
        if x.shape[0] != E:
            raise ValueError(f"qmm_experts: x has {x.shape[0]} experts, the pack {E}")
        lead = x.shape[1:-1]
    else:
        lead = x.shape[:-1]
    M = 1
    for d in lead:
        M *= d
    x2 = x.contiguous()
    wq, scales, biases = wq.contiguous(), scales.contiguous(), biases.contiguous()
    b = bias.to(x.dtype).contiguous() if bias is not None else None
    y = out if out is not None else torch.empty((E, M, N), dtype=x.dtype, device=x.device)
    check(_lib.load().mlxq_qmm_experts(_ptr(x2), _dt(x2), int(per_expert), E, M, K, _ptr(wq),
                                       _ptr(scales), _ptr(biases), _dt(scales), _ptr(b), N,
                                       group_size, bits, _ptr(y), _stream(x.device)))
    return y.reshape(E, *lead, N)


def linear_workspace_size(M: int, N: int, rank: int) -> int:
    return int(_lib.load().mlxq_linear_workspace_size(M, N, rank))


def linear(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, bias=None,
           lora_a=None, lora_b=None, lora_scale: float = 1.0, activation: int = 0, workspace=None):
    """Quantized AdaptableLinear forward with optional bias, one LoRA adapter and an activation,
    rounded at the same points as the reference's separate ops."""
    _need_gpu(x, wq, scales, biases, bias, lora_a, lora_b)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K).contiguous()
    wq, scales, biases = wq.contiguous(), scales.contiguous(), biases.contiguous()
    bias, lora_a, lora_b = _contig(bias), _contig(lora_a), _contig(lora_b)
    M, N = x2.shape[0], wq.shape[0]
    rank = 0 if lora_a is None else int(lora_a.shape[1])
    ep = Epilogue(bias=None if bias is None else bias.data_ptr(),
                  lora_a=None if lora_a is None else lora_a.data_ptr(),
                  lora_b=None if lora_b is None else lora_b.data_ptr(),
                  lora_rank=rank, lora_scale=float(lora_scale), activation=int(activation))
    need = linear_workspace_size(M, N, rank)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    check(_lib.load().mlxq_linear(_ptr(x2), _dt(x2), M, K, _ptr(wq), _ptr(scales), _ptr(biases),
                                  _dt(scales), N, group_size, bits, ctypes.byref(ep), _ptr(y),
                                  _ptr(workspace), 0 if workspace is None else need,
                                  _stream(x.device)))
    return y.reshape(*lead, N)


def packed_bits(wq, scales, group_size: int) -> int:
    """quant::packed_bits (src/quant.rs:38-41), returning an error instead of panicking."""
    if wq.dim() != 2 or scales.dim() != 2:
        raise _lib.MlxqError(_lib.MLXQ_EINVAL, "packed_bits: wq and scales must be 2-D")
    bits = _lib.load().mlxq_packed_bits(wq.shape[1], scales.shape[1], group_size)
    if bits < 0:
        raise _lib.MlxqError(_lib.MLXQ_EINVAL, _lib.load().mlxq_last_error().decode())
    return bits
