"""mlxq_linear_noalloc (static device scratch, no workspace argument) against mlxq_linear with a
caller workspace, through the C ABI.

Both entry points run the same kernels, so outputs must be bit-identical.  Two calls in a row on
the scratch array, the second with a smaller problem (stale contents of the first call must not
leak into it), on the fused GEMM epilogue (M > 8, rank <= 16), the GEMV paths (the 16-row tile
kernel at M = 5, the one-row kernel at M = 1) and a wide adapter (rank 24: plain GEMM +
elementwise epilogue).  A problem needing more scratch than the
array holds is rejected before any device work.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import banner, bf16_normal, to_gpu, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _case(rng, M, K, N, rank):
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    bias = bf16_normal(rng, (N,), 0.5)
    A = bf16_normal(rng, (K, rank), 0.05)
    B = bf16_normal(rng, (rank, N), 0.05)
    rwq, rs, rb = oracle.quantize(w, 64, 4, sb_bf16=True)
    return dict(x=to_gpu(x), wq=wq_to_gpu(rwq), s=to_gpu(rs), b=to_gpu(rb), bias=to_gpu(bias),
                A=to_gpu(A), B=to_gpu(B), M=M, K=K, N=N, rank=rank)


def _run(mlxq, c, noalloc, scale, act):
    from mlxq import _lib
    lib = _lib.load()
    y = torch.empty((c["M"], c["N"]), dtype=torch.bfloat16, device="cuda")
    ep = _lib.Epilogue(c["bias"].data_ptr(), c["A"].data_ptr(), c["B"].data_ptr(), c["rank"],
                       float(scale), int(act), _lib.MLXQ_BFLOAT16, _lib.MLXQ_BFLOAT16)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [c["x"].data_ptr(), _lib.MLXQ_BFLOAT16, c["M"], c["K"], c["wq"].data_ptr(),
            c["s"].data_ptr(), c["b"].data_ptr(), _lib.MLXQ_BFLOAT16, c["N"], 64, 4,
            ctypes.byref(ep), y.data_ptr()]
    if noalloc:
        _lib.check(lib.mlxq_linear_noalloc(*args, st))
    else:
        need = int(lib.mlxq_linear_workspace_size(_lib.MLXQ_BFLOAT16, _lib.MLXQ_BFLOAT16, c["M"], c["N"],
                                                  ctypes.byref(ep)))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        _lib.check(lib.mlxq_linear(*args, ws.data_ptr(), need, st))
        torch.cuda.synchronize()
        del ws
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("first,second", [
    ((600, 1024, 2304, 16), (300, 512, 520, 16)),   # fused GEMM epilogue twice
    ((256, 512, 1040, 24), (40, 256, 136, 8)),      # rank 24 elementwise, then rank 8 fused
    ((300, 512, 1000, 16), (5, 512, 264, 16)),      # GEMM, then the GEMV path
    ((1, 2048, 520, 16), (1, 1024, 264, 16)),       # the one-row GEMV path (M = 1) twice
])
def test_noalloc_matches_workspace_entry_point(mlxq, first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    for i, (M, K, N, rank) in enumerate((first, second)):
        banner("noalloc", i, M, K, N, rank)
        c = _case(rng, M, K, N, rank)
        scale, act = (0.75, 3) if i == 0 else (1.5, 0)
        want = _run(mlxq, c, False, scale, act)
        got = _run(mlxq, c, True, scale, act)
        assert torch.equal(got, want), f"call {i}: noalloc output differs (M={M} N={N} r={rank})"


def test_noalloc_rejects_oversized_scratch(mlxq):
    from mlxq import _lib
    lib = _lib.load()
    banner("noalloc oversized")
    M, N, rank = 1 << 16, 1 << 14, 64
    # Fail-safe call: real (small) device buffers, and K = 96 is not a multiple of the group size,
    # which mlxq_linear itself rejects before any launch.  The scratch-size check runs first, so
    # the error must name the static buffer; were it to move behind argument validation, the call
    # would still end in an error (naming K), never in a kernel on undersized buffers.
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    p = ctypes.c_void_p(buf.data_ptr())
    ep = _lib.Epilogue(None, buf.data_ptr(), buf.data_ptr(), rank, 1.0, 0, _lib.MLXQ_BFLOAT16,
                       _lib.MLXQ_BFLOAT16)
    need = int(lib.mlxq_linear_workspace_size(_lib.MLXQ_BFLOAT16, _lib.MLXQ_BFLOAT16, M, N,
                                              ctypes.byref(ep)))
    assert need > _lib.MLXQ_NOALLOC_SCRATCH_BYTES
    st = lib.mlxq_linear_noalloc(p, _lib.MLXQ_BFLOAT16, M, 96, p, p, p, _lib.MLXQ_BFLOAT16, N, 64, 4,
                                 ctypes.byref(ep), p, None)
    assert st == _lib.MLXQ_EINVAL
    assert b"static buffer" in lib.mlxq_last_error()


def test_noalloc_without_lora_needs_no_scratch(mlxq):
    """No adapter: no scratch is touched, and the result equals mlxq_linear's."""
    banner("noalloc no lora")
    rng = np.random.default_rng(3)
    c = _case(rng, 64, 256, 192, 8)
    c["rank"] = 0
    c["A"] = c["B"] = torch.zeros(1, device="cuda")
    want = _run(mlxq, c, False, 1.0, 2)
    got = _run(mlxq, c, True, 1.0, 2)
    assert torch.equal(got, want)
