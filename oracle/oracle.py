"""ctypes front-end to the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, where it is the checker the HIP path is compared against.  The product
library never imports it.

All tensors are numpy arrays.  bf16 tensors travel as float32 arrays holding bf16-representable
values; the ``*_bf16`` flags choose where the oracle rounds to bf16 (see ``mlxq_oracle.c``).  fp16
activations travel as float32 arrays of fp16-representable values (``fp16_round``) with the bf16
flags off: MLX promotes fp16 against bf16 or f32 to f32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build() -> str:
    """Compile liboracle.so from mlxq_oracle.c (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        l.oracle_bf16_round.argtypes = [ctypes.c_float]
        l.oracle_bf16_round.restype = ctypes.c_float
        l.oracle_fp16_round.argtypes = [ctypes.c_float]
        l.oracle_fp16_round.restype = ctypes.c_float
        l.oracle_fp16_round_array.argtypes = [_f32p, _i64]
        l.oracle_quantize.argtypes = [_f32p, _i64, _i64, _int, _int, _int, _u32p, _f32p, _f32p]
        l.oracle_dequantize.argtypes = [_u32p, _f32p, _f32p, _i64, _i64, _int, _int, _int, _f32p]
        l.oracle_qmm.argtypes = [_f32p, _i64, _i64, _u32p, _f32p, _f32p, _i64, _int, _int, _int,
                                 _int, _f32p]
        l.oracle_linear.argtypes = [_f32p, _i64, _i64, _u32p, _f32p, _f32p, _i64, _int, _int, _int,
                                    _int, _int, _f32p, _int, _f32p, _f32p, _i64, _int,
                                    ctypes.c_float, _int, _f32p, ctypes.POINTER(_int)]
        l.oracle_swiglu_mlp.argtypes = [_f32p, _i64, _i64, _u32p, _f32p, _f32p, _u32p, _f32p, _f32p,
                                        _i64, _u32p, _f32p, _f32p, _i64, _int, _int, _int, _int,
                                        _f32p, _f32p]
        l.oracle_lokr_residual.argtypes = [_f32p, _i64, _i64, _f32p, _i64, ctypes.c_float, _int, _f32p,
                                           _int, _f32p, ctypes.POINTER(_int)]
        l.oracle_gelu_erf.argtypes = [ctypes.c_float, _int]
        l.oracle_gelu_erf.restype = ctypes.c_float
        l.oracle_gelu_tanh.argtypes = [ctypes.c_float, _int]
        l.oracle_gelu_tanh.restype = ctypes.c_float
        l.oracle_gelu_exact.argtypes = [ctypes.c_float, _int]
        l.oracle_gelu_exact.restype = ctypes.c_float
        l.oracle_silu.argtypes = [ctypes.c_float, _int]
        l.oracle_silu.restype = ctypes.c_float
        l.oracle_num_threads.restype = _int
        for name in ("oracle_quantize", "oracle_dequantize", "oracle_qmm", "oracle_linear",
                     "oracle_swiglu_mlp"):
            getattr(l, name).restype = _int
        _lib = l
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_f32p)


def _u32(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(_u32p)


def _opt_f32(a):
    if a is None:
        return None, None
    return _f32(a)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"{what}: invalid arguments (oracle status {rc})")


def bf16_round(a) -> np.ndarray:
    """Round float32 values to the nearest-even bf16, returned as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(nan, (u.astype(np.uint32) | 0x00400000) & 0xFFFF0000, r).astype(np.uint32)
    return r.view(np.float32).reshape(a.shape)


def fp16_round(a) -> np.ndarray:
    """Round float32 values to the nearest-even fp16, returned as float32 (oracle_fp16_round)."""
    a = np.array(a, dtype=np.float32, copy=True, order="C")
    lib().oracle_fp16_round_array(a.ctypes.data_as(_f32p), a.size)
    return a


def quantize(w, group_size=64, bits=4, sb_bf16=False):
    """(wq uint32 [N, K*bits/32], scales f32 [N, K/gs], biases f32 [N, K/gs])."""
    w, wp = _f32(w)
    N, K = w.shape
    if K % group_size:
        raise ValueError("K must be divisible by group_size")
    wq = np.empty((N, K * bits // 32), np.uint32)
    s = np.empty((N, K // group_size), np.float32)
    b = np.empty((N, K // group_size), np.float32)
    _check(lib().oracle_quantize(wp, N, K, group_size, bits, int(sb_bf16), _u32(wq)[1],
                                 _f32(s)[1], _f32(b)[1]), "quantize")
    return wq, s, b


def dequantize(wq, scales, biases, group_size=64, bits=4, out_bf16=False):
    wq, wqp = _u32(wq)
    scales, sp = _f32(scales)
    biases, bp = _f32(biases)
    N = wq.shape[0]
    K = wq.shape[1] * 32 // bits
    out = np.empty((N, K), np.float32)
    _check(lib().oracle_dequantize(wqp, sp, bp, N, K, group_size, bits, int(out_bf16),
                                   out.ctypes.data_as(_f32p)), "dequantize")
    return out


def quantized_matmul(x, wq, scales, biases, group_size=64, bits=4, w_bf16=True, out_bf16=True):
    """y = x . dequant(W)^T, double accumulation; see oracle_qmm."""
    x, xp = _f32(x)
    wq, wqp = _u32(wq)
    scales, sp = _f32(scales)
    biases, bp = _f32(biases)
    M, K = x.shape
    N = wq.shape[0]
    if wq.shape[1] * 32 // bits != K:
        raise ValueError("x / wq inner dims disagree")
    y = np.empty((M, N), np.float32)
    _check(lib().oracle_qmm(xp, M, K, wqp, sp, bp, N, group_size, bits, int(w_bf16),
                            int(out_bf16), y.ctypes.data_as(_f32p)), "quantized_matmul")
    return y


def linear(x, wq, scales, biases, group_size=64, bits=4, w_bf16=True, act_bf16=True, bias=None,
           lora_a=None, lora_b=None, lora_scale=1.0, act=0, x_bf16=None, sb_bf16=None,
           bias_bf16=None, lora_bf16=None, return_dtype=False):
    """AdaptableLinear forward over a quantized base with optional bias, LoRA and activation,
    under MLX's promotion.  Each *_bf16 flag says whether that operand is bf16 (values are passed
    as the f32 numbers they hold); unset flags default to act_bf16.  act: 0 none, 1 GELU
    (f32 result), 2 tanh GELU, 3 exact GELU.  With return_dtype, returns (y, out_is_bf16)."""
    x, xp = _f32(x)
    wq, wqp = _u32(wq)
    scales, sp = _f32(scales)
    biases, bp = _f32(biases)
    M, K = x.shape
    N = wq.shape[0]
    bias, biasp = _opt_f32(bias)
    lora_a, ap = _opt_f32(lora_a)
    lora_b, bbp = _opt_f32(lora_b)
    rank = 0 if lora_a is None else lora_a.shape[1]
    flag = lambda f: int(act_bf16 if f is None else f)
    y = np.empty((M, N), np.float32)
    ob = _int(0)
    _check(lib().oracle_linear(xp, M, K, wqp, sp, bp, N, group_size, bits, int(w_bf16),
                               flag(x_bf16), flag(sb_bf16), biasp, flag(bias_bf16), ap, bbp, rank,
                               flag(lora_bf16), float(lora_scale), int(act),
                               y.ctypes.data_as(_f32p), ctypes.byref(ob)), "linear")
    return (y, bool(ob.value)) if return_dtype else y


def swiglu_mlp(x, gate, up, down, group_size=64, bits=4, w_bf16=False, act_bf16=True):
    """gate/up/down are (wq, scales, biases) triples; returns (h, y)."""
    x, xp = _f32(x)
    M, K = x.shape
    g = [_u32(gate[0]), _f32(gate[1]), _f32(gate[2])]
    u = [_u32(up[0]), _f32(up[1]), _f32(up[2])]
    d = [_u32(down[0]), _f32(down[1]), _f32(down[2])]
    F = g[0][0].shape[0]
    Nd = d[0][0].shape[0]
    h = np.empty((M, F), np.float32)
    y = np.empty((M, Nd), np.float32)
    _check(lib().oracle_swiglu_mlp(xp, M, K, g[0][1], g[1][1], g[2][1], u[0][1], u[1][1], u[2][1],
                                   F, d[0][1], d[1][1], d[2][1], Nd, group_size, bits, int(w_bf16),
                                   int(act_bf16), h.ctypes.data_as(_f32p),
                                   y.ctypes.data_as(_f32p)), "swiglu_mlp")
    return h, y


def lokr_residual(x, y_in, delta, scale=1.0, x_bf16=True, y_bf16=True, return_dtype=False):
    """y_in + scale * x . delta^T, one LoKr adapter step of AdaptableLinear::forward (the residual
    in x's dtype, the sum in promote(y, x)).  Values are passed as the f32 numbers they hold."""
    x, xp = _f32(x)
    y_in, yp = _f32(y_in)
    delta, dp = _f32(delta)
    M, K = x.shape
    N = delta.shape[0]
    assert delta.shape == (N, K) and y_in.shape == (M, N)
    y = np.empty((M, N), np.float32)
    ob = _int(0)
    _check(lib().oracle_lokr_residual(xp, M, K, dp, N, float(scale), int(x_bf16), yp, int(y_bf16),
                                      y.ctypes.data_as(_f32p), ctypes.byref(ob)), "lokr_residual")
    return (y, bool(ob.value)) if return_dtype else y


def gelu_erf(v, out_bf16=True):
    return lib().oracle_gelu_erf(float(v), int(out_bf16))


def gelu_tanh(v, out_bf16=True):
    return lib().oracle_gelu_tanh(float(v), int(out_bf16))


def gelu_exact(v, out_bf16=True):
    return lib().oracle_gelu_exact(float(v), int(out_bf16))


def silu(v, out_bf16=True):
    return lib().oracle_silu(float(v), int(out_bf16))


def num_threads() -> int:
    return lib().oracle_num_threads()
