"""Op-level API over libmlxq_hip.so, mirroring the three MLX ops the reference calls.

Reference call sites (mlx_rs::ops, MLX 0.31.2 via pmetal-mlx-rs 0.25.8):
  quantize(w, group_size, bits)                          src/quant.rs:140, src/nn.rs:91-93
  dequantize(wq, scales, biases, group_size, bits)       src/nn.rs:55
  quantized_matmul(x, wq, scales, biases, transpose,
                   group_size, bits)                     src/adapters.rs:309-317

Tensors are torch tensors on the GPU (torch only supplies device memory and the current
stream).  bf16 and f32 are supported everywhere, fp16 as activations (SDXL's dtype, reference
mlx-gen-sdxl/src/model.rs:216), and dtypes follow MLX's promotion: scales/biases in the weight
dtype; a matmul returns promote(x, scales) (bf16 only when both are bf16; fp16 against bf16 or f32
is f32); a bias add or a LoRA residual in f32 promotes the result to f32.  Every operand's shape and dtype is checked
against x before anything is launched, as MLX's quantized_matmul checks them; failures raise
``MlxqError`` with status MLXQ_EINVAL, and library errors carry the library's status and message.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import MLXQ_BFLOAT16, MLXQ_EINVAL, MLXQ_FLOAT16, MLXQ_FLOAT32, Epilogue, MlxqError, check

DEFAULT_GROUP_SIZE = 64  # src/quant.rs:32


_CODES = {torch.float32: MLXQ_FLOAT32, torch.bfloat16: MLXQ_BFLOAT16, torch.float16: MLXQ_FLOAT16}


def _dt(t: torch.Tensor) -> int:
    return _dt_of(t.dtype)


def _dt_of(dtype) -> int:
    if dtype not in _CODES:
        raise TypeError(f"mlxq supports bfloat16, float32 and float16 tensors, got {dtype}")
    return _CODES[dtype]


def _torch_dtype(dt: int):
    return {MLXQ_BFLOAT16: torch.bfloat16, MLXQ_FLOAT16: torch.float16}.get(dt, torch.float32)


def promote(*dtypes) -> torch.dtype:
    """MLX's result type over f32 / bf16 / fp16 operands: a 16-bit type only when every operand
    has it; any f32 operand, or bf16 meeting fp16, gives f32."""
    first = dtypes[0]
    if first in (torch.bfloat16, torch.float16) and all(d == first for d in dtypes):
        return first
    return torch.float32


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


def _aligned(t, align: int):
    """t when its data pointer is `align`-byte aligned, else an aligned copy: views such as one
    expert's slice of a stacked pack can start mid-word, and the library requires 16-byte aligned
    activations and packed codes and 4-byte aligned scales and biases."""
    return t if t is None or t.data_ptr() % align == 0 else t.clone()


def _pack3(wq, scales, biases):
    """A (wq, scales, biases) pack made contiguous and aligned for the library."""
    return (_aligned(wq.contiguous(), 16), _aligned(scales.contiguous(), 4),
            _aligned(biases.contiguous(), 4))


def _bad(op: str, msg: str):
    raise MlxqError(MLXQ_EINVAL, f"{op}: {msg}")


def _float_dtype(op: str, what: str, t: torch.Tensor):
    """A float dtype MLX has.  fp16 is passed through: the library takes it as activations and
    reports MLXQ_EUNSUPPORTED for any other operand."""
    if t.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        _bad(op, f"{what} must be bfloat16, float32 or float16, got {t.dtype}")


def _check_pack(op: str, wq, scales, biases, K: int, group_size: int, bits: int, lead=()):
    """The packed triple against the activation width K (MLX's extract_quantized_matmul_dims):
    wq [*lead, N, K*bits/32] of 32-bit words, scales/biases [*lead, N, K/group_size] alike."""
    if bits not in (4, 8):
        _bad(op, f"bits must be 4 or 8 (got {bits})")
    if group_size not in (32, 64, 128):
        _bad(op, f"group_size must be 32, 64 or 128 (got {group_size})")
    nd = len(lead) + 2
    if wq.dim() != nd or scales.dim() != nd or biases.dim() != nd:
        _bad(op, f"wq, scales and biases must be {nd}-D")
    if wq.dtype not in (torch.int32, torch.uint32):
        _bad(op, f"packed weights must be 32-bit words, got {wq.dtype}")
    if tuple(wq.shape[:-2]) != tuple(lead) or tuple(scales.shape[:-2]) != tuple(lead):
        _bad(op, f"stacked operands must lead with {tuple(lead)}")
    N = wq.shape[-2]
    if K % group_size:
        _bad(op, f"K={K} is not a multiple of group_size={group_size}")
    if wq.shape[-1] * 32 != K * bits:
        _bad(op, f"wq has {wq.shape[-1]} words per row, which packs {wq.shape[-1] * 32 // bits} "
                 f"{bits}-bit codes, not x's K={K}")
    want = tuple(lead) + (N, K // group_size)
    if tuple(scales.shape) != want or tuple(biases.shape) != want:
        _bad(op, f"scales/biases must be {want} (got {tuple(scales.shape)} / {tuple(biases.shape)})")
    _float_dtype(op, "scales", scales)
    if biases.dtype != scales.dtype:
        _bad(op, f"biases dtype {biases.dtype} differs from scales dtype {scales.dtype}")
    return N


def _check_out(op: str, out, dtype, numel: int, device):
    if out.dtype != dtype or out.device != device or out.numel() != numel or not out.is_contiguous():
        _bad(op, f"out must be a contiguous {dtype} tensor of {numel} elements on {device}")


def _scales_biases(N: int, gcols: int, dtype, device):
    """Empty scales and biases [N, gcols] as two views of one allocation, the biases starting 256
    bytes past the scales' end rounded up: the large-M GEMM stages bf16 scales and biases through
    one buffer resource, which needs both arrays within 4 GiB of each other (two separate
    allocations of a large process can lie further apart, which costs that GEMM its fast path)."""
    n = N * gcols
    esz = torch.empty((), dtype=dtype).element_size()
    off = (n * esz + 511) // 256 * 256 // esz
    buf = torch.empty((off + n,), dtype=dtype, device=device)
    return buf[:n].view(N, gcols), buf[off:off + n].view(N, gcols)


def quantize(w: torch.Tensor, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4):
    """Affine group quantization of w [N, K] -> (wq u32-as-int32 [N, K*bits/32], scales, biases).
    scales and biases are views of one allocation (_scales_biases)."""
    _need_gpu(w)
    if w.dim() != 2:
        raise ValueError(f"quantize expects a 2-D weight, got shape {tuple(w.shape)}")
    w = w.contiguous()
    N, K = w.shape
    # Packed words are stored in an int32 tensor (same bits as MLX's uint32 array).
    wq = torch.empty((N, max(K * bits // 32, 0)), dtype=torch.int32, device=w.device)
    gcols = K // group_size if group_size > 0 else 0
    s, b = _scales_biases(N, gcols, w.dtype, w.device)
    check(_lib.load().mlxq_quantize(_ptr(w), _dt(w), N, K, group_size, bits, _ptr(wq), _ptr(s),
                                    _ptr(b), _stream(w.device)))
    return wq, s, b


def quantize_batched(ws, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4):
    """quantize() over a list of weights of one shape and dtype, in launches of up to 16 weights
    (mlxq_quantize_batched): the same (wq, scales, biases) triples as one quantize() per weight."""
    ws = [w.contiguous() for w in ws]
    if not ws:
        return []
    _need_gpu(*ws)
    w0 = ws[0]
    if w0.dim() != 2:
        raise ValueError(f"quantize_batched expects 2-D weights, got shape {tuple(w0.shape)}")
    for w in ws[1:]:
        if w.shape != w0.shape or w.dtype != w0.dtype or w.device != w0.device:
            _bad("quantize_batched", "every weight must have the first one's shape, dtype and device")
    N, K = w0.shape
    gcols = K // group_size if group_size > 0 else 0
    outs = [(torch.empty((N, max(K * bits // 32, 0)), dtype=torch.int32, device=w0.device),
             *_scales_biases(N, gcols, w0.dtype, w0.device)) for _ in ws]
    arr = ctypes.c_void_p * len(ws)
    check(_lib.load().mlxq_quantize_batched(
        arr(*[_ptr(w) for w in ws]), len(ws), _dt(w0), N, K, group_size, bits,
        arr(*[_ptr(o[0]) for o in outs]), arr(*[_ptr(o[1]) for o in outs]), arr(*[_ptr(o[2]) for o in outs]),
        _stream(w0.device)))
    return outs


def _k_of(wq: torch.Tensor, bits: int) -> int:
    return wq.shape[-1] * 32 // bits


def dequantize(wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4):
    if bits not in (4, 8):
        _bad("dequantize", f"bits must be 4 or 8 (got {bits})")
    wq, scales, biases = _pack3(wq, scales, biases)
    K = _k_of(wq, bits)
    N = _check_pack("dequantize", wq, scales, biases, K, group_size, bits)
    _need_gpu(wq, scales, biases)
    out = torch.empty((N, K), dtype=scales.dtype, device=wq.device)
    check(_lib.load().mlxq_dequantize(_ptr(wq), _ptr(scales), _ptr(biases), _dt(scales), N, K,
                                      group_size, bits, _ptr(out), _stream(wq.device)))
    return out


def _mm(entry, x, wq, scales, biases, group_size, bits, *extra, out=None):
    if x.dim() < 1:
        _bad(entry, "x must have a last dimension")
    _float_dtype(entry, "x", x)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = _aligned(x.reshape(-1, K).contiguous(), 16)
    wq, scales, biases = _pack3(wq, scales, biases)
    N = _check_pack(entry, wq, scales, biases, K, group_size, bits)
    M = x2.shape[0]
    # The forced bf16-tile GEMM returns bf16; the others MLX's promote(x, scales).
    ydt = torch.bfloat16 if entry == "mlxq_qmm" else promote(x.dtype, scales.dtype)
    if out is None:
        y = torch.empty((M, N), dtype=ydt, device=x.device)
    else:
        _check_out(entry, out, ydt, M * N, x.device)
        y = out
    _need_gpu(x, wq, scales, biases)
    args = [_ptr(x2), _dt(x2), M, K, _ptr(wq), _ptr(scales), _ptr(biases), _dt(scales), N]
    if entry == "mlxq_quantized_matmul":
        args.append(int(extra[0]))
    args += [group_size, bits, _ptr(y), _stream(x.device)]
    check(getattr(_lib.load(), entry)(*args))
    return y.reshape(*lead, N)


def quantized_matmul(x, wq, scales, biases, transpose: bool = True,
                     group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """y = x . dequantize(W)^T (transpose=True, the only form the reference uses), in
    promote(x, scales)."""
    return _mm("mlxq_quantized_matmul", x, wq, scales, biases, group_size, bits, transpose, out=out)


def qmm(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """Force the MFMA bf16-tile GEMM kernel (bf16 activations, bf16 result)."""
    return _mm("mlxq_qmm", x, wq, scales, biases, group_size, bits, out=out)


def qmv(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """Force the GEMV kernel (M <= 8)."""
    return _mm("mlxq_qmv", x, wq, scales, biases, group_size, bits, out=out)


def qmv_valu(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """Force the VALU GEMV (no matrix cores; M <= 8), the kernel quantized_matmul runs for f32
    operands and group size 32, on any operand dtypes."""
    return _mm("mlxq_qmv_valu", x, wq, scales, biases, group_size, bits, out=out)


def embedding(ids, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4,
              out_dtype=torch.float32):
    """TokenEmbedding::forward's quantized arm (src/nn.rs:42-58): gather the packed rows of ids
    (any shape, int32/int64), dequantize, cast to out_dtype (f32 like the reference).  Ids outside
    [0, vocab) give NaN rows."""
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"embedding: out_dtype must be bfloat16 or float32, got {out_dtype}")
    if bits not in (4, 8):
        _bad("embedding", f"bits must be 4 or 8 (got {bits})")
    wq, scales, biases = _pack3(wq, scales, biases)
    hidden = _k_of(wq, bits)
    vocab = _check_pack("embedding", wq, scales, biases, hidden, group_size, bits)
    _need_gpu(ids, wq, scales, biases)
    flat = ids.reshape(-1).to(torch.int32).contiguous()
    out = torch.empty((flat.numel(), hidden), dtype=out_dtype, device=wq.device)
    odt = MLXQ_BFLOAT16 if out_dtype == torch.bfloat16 else MLXQ_FLOAT32
    check(_lib.load().mlxq_embedding(_ptr(flat), flat.numel(), _ptr(wq), _ptr(scales), _ptr(biases),
                                     _dt(scales), vocab, hidden, group_size, bits, _ptr(out), odt,
                                     _stream(wq.device)))
    return out.reshape(*ids.shape, hidden)


def swiglu(x, gate, up, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, out=None):
    """Fused decode SwiGLU h = silu(gate(x)) * up(x) (mlx-gen-sensenova/src/qwen3.rs:178-181), gate
    and up given as packed (wq, scales, biases) triples of shape [F, K].  Decode form only (bf16,
    M <= 8); other shapes raise MlxqError with status MLXQ_EUNSUPPORTED."""
    _float_dtype("swiglu", "x", x)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = _aligned(x.reshape(-1, K).contiguous(), 16)
    g = list(_pack3(*gate))
    u = list(_pack3(*up))
    F = _check_pack("swiglu", *g, K, group_size, bits)
    if _check_pack("swiglu", *u, K, group_size, bits) != F or u[1].dtype != g[1].dtype:
        _bad("swiglu", "gate and up must be packed alike")
    M = x2.shape[0]
    hdt = promote(x.dtype, g[1].dtype)
    if out is not None:
        _check_out("swiglu", out, hdt, M * F, x.device)
    _need_gpu(x, *gate, *up)
    h = out if out is not None else torch.empty((M, F), dtype=hdt, device=x.device)
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
    [E, N] (bf16 in the reference's packs) or None.  x [..., K] is shared by every expert, or with
    per_expert=True it is [E, ..., K] (one input per expert).  Returns [E, ..., N] in
    promote(x, scales, bias)."""
    _float_dtype("qmm_experts", "x", x)
    if wq.dim() != 3:
        _bad("qmm_experts", "wq must be a stacked [E, N, K*bits/32] pack")
    E = wq.shape[0]
    K = x.shape[-1]
    wq, scales, biases = _pack3(wq, scales, biases)
    N = _check_pack("qmm_experts", wq, scales, biases, K, group_size, bits, lead=(E,))
    if per_expert:
        if x.dim() < 2 or x.shape[0] != E:
            _bad("qmm_experts", f"per-expert x must lead with E={E}, got shape {tuple(x.shape)}")
        lead = x.shape[1:-1]
    else:
        lead = x.shape[:-1]
    M = 1
    for d in lead:
        M *= d
    x2 = x.contiguous()
    b = _contig(bias)
    if b is not None:
        _float_dtype("qmm_experts", "bias", b)
        if tuple(b.shape) != (E, N):
            _bad("qmm_experts", f"bias must be ({E}, {N}), got {tuple(b.shape)}")
    ydt = promote(x.dtype, scales.dtype, *(() if b is None else (b.dtype,)))
    if out is not None:
        _check_out("qmm_experts", out, ydt, E * M * N, x.device)
    _need_gpu(x, wq, scales, biases, bias)
    y = out if out is not None else torch.empty((E, M, N), dtype=ydt, device=x.device)
    rc = _lib.load().mlxq_qmm_experts(_ptr(x2), _dt(x2), int(per_expert), E, M, K, _ptr(wq),
                                      _ptr(scales), _ptr(biases), _dt(scales), _ptr(b),
                                      MLXQ_BFLOAT16 if b is None else _dt(b), N, group_size, bits,
                                      _ptr(y), _stream(x.device))
    misaligned = E > 1 and ((M * N * y.element_size()) % 16 or (N * (K // group_size) * scales.element_size()) % 4)
    if rc == _lib.MLXQ_EUNSUPPORTED and misaligned:
        # The library runs these experts one at a time and each expert's slice of y or of the
        # scales/biases is unaligned for it: run them here (linear aligns its operands, and each
        # expert's result goes through an aligned output).
        y3 = y.view(E, M, N)
        xs = x2.reshape(E, M, K) if per_expert else x2.reshape(M, K)
        for e in range(E):
            ye = linear(xs[e] if per_expert else xs, wq[e], scales[e], biases[e], group_size, bits,
                        bias=None if b is None else b[e])
            y3[e].copy_(ye)
    else:
        check(rc)
    return y.reshape(E, *lead, N)


def _epilogue(bias, lora_a, lora_b, lora_scale, activation, x_dtype):
    rank = 0 if lora_a is None else int(lora_a.shape[1])
    return Epilogue(bias=None if bias is None else bias.data_ptr(),
                    lora_a=None if lora_a is None else lora_a.data_ptr(),
                    lora_b=None if lora_b is None else lora_b.data_ptr(),
                    lora_rank=rank, lora_scale=float(lora_scale), activation=int(activation),
                    bias_dtype=_dt(bias) if bias is not None else _dt_of(x_dtype),
                    lora_dtype=_dt(lora_a) if lora_a is not None else _dt_of(x_dtype))


def linear_out_dtype(x_dtype, scales_dtype, bias_dtype=None, lora_dtype=None, activation: int = 0):
    """The dtype mlxq_linear returns for these operand dtypes (MLX's promotion, the library's rule)."""
    ep = Epilogue(bias=1 if bias_dtype is not None else None, lora_a=None, lora_b=None,
                  lora_rank=16 if lora_dtype is not None else 0, lora_scale=1.0,
                  activation=int(activation),
                  bias_dtype=_dt_of(bias_dtype if bias_dtype is not None else x_dtype),
                  lora_dtype=_dt_of(lora_dtype if lora_dtype is not None else x_dtype))
    dt = _lib.load().mlxq_linear_out_dtype(_dt_of(x_dtype), _dt_of(scales_dtype), ctypes.byref(ep))
    if dt < 0:
        raise MlxqError(MLXQ_EINVAL, _lib.load().mlxq_last_error().decode())
    return _torch_dtype(dt)


def linear_workspace_size(x_dtype, scales_dtype, M: int, N: int, bias=None, lora_a=None,
                          activation: int = 0) -> int:
    ep = _epilogue(bias, lora_a, lora_a, 1.0, activation, x_dtype)
    return int(_lib.load().mlxq_linear_workspace_size(_dt_of(x_dtype), _dt_of(scales_dtype), M, N,
                                                      ctypes.byref(ep)))


def linear(x, wq, scales, biases, group_size: int = DEFAULT_GROUP_SIZE, bits: int = 4, bias=None,
           lora_a=None, lora_b=None, lora_scale: float = 1.0, activation: int = 0, workspace=None):
    """Quantized AdaptableLinear forward with optional bias, one LoRA adapter and an activation,
    rounded at the same points as the reference's separate ops.  bias and the LoRA factors keep
    their own dtypes; the result is in MLX's promoted dtype (linear_out_dtype)."""
    _float_dtype("linear", "x", x)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = _aligned(x.reshape(-1, K).contiguous(), 16)
    wq, scales, biases = _pack3(wq, scales, biases)
    bias, lora_a, lora_b = _contig(bias), _contig(lora_a), _contig(lora_b)
    N = _check_pack("linear", wq, scales, biases, K, group_size, bits)
    M = x2.shape[0]
    if bias is not None:
        _float_dtype("linear", "bias", bias)
        if tuple(bias.shape) != (N,):
            _bad("linear", f"bias must have shape ({N},), got {tuple(bias.shape)}")
    if (lora_a is None) != (lora_b is None):
        _bad("linear", "LoRA needs both factors")
    if lora_a is not None:
        _float_dtype("linear", "LoRA A", lora_a)
        if lora_a.dim() != 2 or lora_b.dim() != 2 or lora_a.shape[0] != K or lora_b.shape[1] != N \
                or lora_a.shape[1] != lora_b.shape[0]:
            _bad("linear", f"LoRA factors must be A [{K}, r] and B [r, {N}], got "
                           f"{tuple(lora_a.shape)} and {tuple(lora_b.shape)}")
        if lora_b.dtype != lora_a.dtype:
            _bad("linear", "LoRA A and B must share a dtype")
    _need_gpu(x, wq, scales, biases, bias, lora_a, lora_b)
    ep = _epilogue(bias, lora_a, lora_b, lora_scale, activation, x.dtype)
    lib = _lib.load()
    odt = lib.mlxq_linear_out_dtype(_dt(x2), _dt(scales), ctypes.byref(ep))
    if odt < 0:
        raise MlxqError(MLXQ_EINVAL, lib.mlxq_last_error().decode())
    need = int(lib.mlxq_linear_workspace_size(_dt(x2), _dt(scales), M, N, ctypes.byref(ep)))
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    y = torch.empty((M, N), dtype=_torch_dtype(odt), device=x.device)
    check(lib.mlxq_linear(_ptr(x2), _dt(x2), M, K, _ptr(wq), _ptr(scales), _ptr(biases),
                          _dt(scales), N, group_size, bits, ctypes.byref(ep), _ptr(y),
                          _ptr(workspace) if need else None, need, _stream(x.device)))
    return y.reshape(*lead, N)


def lora_residual(x, y, lora_a, lora_b, lora_scale: float = 1.0, workspace=None):
    """out = y + scale * (x.A).B — one more adapter of AdaptableLinear::forward's stack
    (src/adapters.rs:543-549, Adapter::residual :260-270) on an already computed y.  The residual
    runs in promote(x, A); the sum in promote(y, residual) (in place when that is y's dtype)."""
    _float_dtype("lora_residual", "x", x)
    _float_dtype("lora_residual", "y", y)
    K = x.shape[-1]
    x2 = _aligned(x.reshape(-1, K).contiguous(), 16)
    M = x2.shape[0]
    N = y.shape[-1]
    if y.numel() != M * N:
        _bad("lora_residual", f"y has {y.numel()} elements, x implies {M} rows of {N}")
    lora_a, lora_b = lora_a.contiguous(), lora_b.contiguous()
    _float_dtype("lora_residual", "LoRA A", lora_a)
    if lora_a.dim() != 2 or lora_b.dim() != 2 or lora_a.shape[0] != K or lora_b.shape[1] != N \
            or lora_a.shape[1] != lora_b.shape[0] or lora_b.dtype != lora_a.dtype:
        _bad("lora_residual", f"LoRA factors must be A [{K}, r] and B [r, {N}] of one dtype")
    _need_gpu(x, y, lora_a, lora_b)
    rank = int(lora_a.shape[1])
    y_in = y.contiguous()
    odt = promote(y.dtype, x.dtype, lora_a.dtype)
    out = y_in if odt == y.dtype else torch.empty(y.shape, dtype=odt, device=y.device)
    lib = _lib.load()
    need = int(lib.mlxq_lora_residual_workspace_size(_dt(x2), _dt(lora_a), M, N, rank))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    check(lib.mlxq_lora_residual(_ptr(x2), _dt(x2), M, K, _ptr(lora_a), _ptr(lora_b), _dt(lora_a), N,
                                 rank, float(lora_scale), _ptr(y_in), _dt(y_in), _ptr(out),
                                 _ptr(workspace), need, _stream(x.device)))
    return out


def lokr_residual(x, y, delta, scale: float = 1.0, workspace=None):
    """out = y + scale * x . delta^T — one LoKr adapter of AdaptableLinear::forward's stack
    (src/adapters.rs:543-549, Adapter::residual's Lokr arm :263-266) on an already computed y.
    delta [out, in] (the reconstructed kron delta, stored bf16 by the reference) is cast to x's
    dtype and the residual runs in x's dtype; the sum in promote(y, x) (in place when that is y's
    dtype)."""
    _float_dtype("lokr_residual", "x", x)
    _float_dtype("lokr_residual", "y", y)
    _float_dtype("lokr_residual", "delta", delta)
    K = x.shape[-1]
    x2 = _aligned(x.reshape(-1, K).contiguous(), 16)
    M = x2.shape[0]
    N = y.shape[-1]
    if y.numel() != M * N:
        _bad("lokr_residual", f"y has {y.numel()} elements, x implies {M} rows of {N}")
    if delta.dim() != 2 or tuple(delta.shape) != (N, K):
        _bad("lokr_residual", f"delta must be [{N}, {K}], got {tuple(delta.shape)}")
    delta = delta.contiguous()
    _need_gpu(x, y, delta)
    y_in = y.contiguous()
    odt = promote(y.dtype, x.dtype)
    out = y_in if odt == y.dtype else torch.empty(y.shape, dtype=odt, device=y.device)
    lib = _lib.load()
    need = int(lib.mlxq_lokr_residual_workspace_size(_dt(x2), M, N))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    check(lib.mlxq_lokr_residual(_ptr(x2), _dt(x2), M, K, _ptr(delta), _dt(delta), N, float(scale),
                                 _ptr(y_in), _dt(y_in), _ptr(out), _ptr(workspace), need,
                                 _stream(x.device)))
    return out


def packed_bits(wq, scales, group_size: int) -> int:
    """quant::packed_bits (src/quant.rs:38-41), returning an error instead of panicking."""
    if wq.dim() != 2 or scales.dim() != 2:
        raise _lib.MlxqError(_lib.MLXQ_EINVAL, "packed_bits: wq and scales must be 2-D")
    bits = _lib.load().mlxq_packed_bits(wq.shape[1], scales.shape[1], group_size)
    if bits < 0:
        raise _lib.MlxqError(_lib.MLXQ_EINVAL, _lib.load().mlxq_last_error().decode())
    return bits
