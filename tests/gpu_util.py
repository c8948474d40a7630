"""Shared helpers for the GPU parity tests (seeded inputs, tolerance checks, case banners)."""
import sys

import numpy as np
import torch

from oracle import oracle

# The north-star tolerance for quantized_matmul: relative Frobenius error <= 2e-3 and
# per-element |delta| <= 1e-2 * max|y|.
REL_FRO_TOL = 2e-3
PEAK_TOL = 1e-2


def banner(*parts):
    """Name the case before a GPU step so a fault report says which case was running."""
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def bf16_normal(rng, shape, std=1.0):
    return oracle.bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def to_gpu(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def to_np(t):
    if t.dtype == torch.int32:
        return t.cpu().numpy().view(np.uint32)
    return t.float().cpu().numpy()


def wq_to_gpu(wq):
    return torch.from_numpy(np.ascontiguousarray(wq).view(np.int32)).to("cuda")


def errors(y, ref):
    y = y.astype(np.float64)
    ref = ref.astype(np.float64)
    d = y - ref
    rel_fro = np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30)
    peak = np.abs(d).max() / max(np.abs(ref).max(), 1e-30)
    return rel_fro, peak


def assert_close(y, ref, what=""):
    rel_fro, peak = errors(y, ref)
    print(f"    {what} relFro={rel_fro:.3e} peak={peak:.3e}", flush=True)
    assert rel_fro <= REL_FRO_TOL, f"{what}: relFro {rel_fro:.3e} > {REL_FRO_TOL}"
    assert peak <= PEAK_TOL, f"{what}: peak-relative |delta| {peak:.3e} > {PEAK_TOL}"
    return rel_fro, peak
