"""The hot-path entry points captured in a HIP graph (as a serving loop or the bench runs them):
every replay must reproduce the eager outputs bit for bit; and run from two streams at once, each
stream's outputs must equal what it computes alone (no shared mutable device state).

Captured: the M = 1 decode MLP (SwiGLU launch + down GEMV, the one-row kernel), a wide-GEMM
linear with bias and the exact GELU, the f32 GEMM with its matrix-core bias term, and a quantize.
Between replays the outputs are overwritten from the host side (NaN / all-ones patterns) and the
device synchronized, so a replay that skipped or half-ran a launch cannot pass on stale values.
The GELU table is filled by an eager call first (its one-time fill synchronizes the stream, which
a capture does not allow).
"""
import numpy as np
import pytest
import torch

from gpu_util import banner, bf16_normal, to_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _inputs(mlxq):
    rng = np.random.default_rng(2024)
    K, F, Nd = 3072, 4096, 3072
    d = {}
    d["x1"] = to_gpu(bf16_normal(rng, (1, K)))
    d["g"] = mlxq.quantize(to_gpu(bf16_normal(rng, (F, K), 0.02)), 64, 4)
    d["u"] = mlxq.quantize(to_gpu(bf16_normal(rng, (F, K), 0.02)), 64, 4)
    d["d"] = mlxq.quantize(to_gpu(bf16_normal(rng, (Nd, F), 0.02)), 64, 4)
    d["xw"] = to_gpu(bf16_normal(rng, (1024, K)))
    d["w"] = mlxq.quantize(to_gpu(bf16_normal(rng, (8192, K), 0.02)), 64, 4)
    d["bias"] = to_gpu(bf16_normal(rng, (8192,), 0.1))
    d["xf"] = to_gpu(rng.standard_normal((256, K)).astype(np.float32), torch.float32)
    d["wf"] = mlxq.quantize(to_gpu(bf16_normal(rng, (3072, K), 0.02)), 64, 4)
    d["wq_src"] = to_gpu(bf16_normal(rng, (2048, 2048), 0.02))
    torch.cuda.synchronize()
    return d


def _run(mlxq, d):
    h = mlxq.swiglu(d["x1"], d["g"], d["u"], 64, 4)
    y1 = mlxq.quantized_matmul(h, *d["d"], True, 64, 4)
    yw = mlxq.linear(d["xw"], *d["w"], 64, 4, bias=d["bias"], activation=mlxq.MLXQ_ACT_GELU_EXACT)
    yf = mlxq.quantized_matmul(d["xf"], *d["wf"], True, 64, 4)
    q = mlxq.quantize(d["wq_src"], 64, 4)
    return [h, y1, yw, yf, *q]


def _scrub(t):
    if t.dtype in (torch.float32, torch.bfloat16):
        t.fill_(float("nan"))
    else:
        t.fill_(-1)


def test_graph_replays_match_eager(mlxq):
    banner("graph replay: decode MLP, wide GELU linear, f32 GEMM, quantize")
    d = _inputs(mlxq)
    eager = [t.clone() for t in _run(mlxq, d)]  # also fills the GELU table
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _run(mlxq, d)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _run(mlxq, d)
    names = ["swiglu h", "down y", "wide GELU linear", "f32 GEMM", "quantize wq", "scales", "biases"]
    for rep in range(3):
        for t in outs:
            _scrub(t)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, o, e in zip(names, outs, eager):
            assert torch.equal(o, e), f"replay {rep}: {name} differs from the eager result"
        print(f"    replay {rep}: all {len(outs)} outputs bit-identical", flush=True)
    del graph


def test_two_streams_at_once_match_sequential(mlxq):
    """Re-entrancy per stream: two streams running different decode MLPs, wide GELU linears and f32
    GEMMs at the same time (each stream on its own weights, its launches interleaved with the
    other's) produce what each produces alone."""
    banner("two streams at once")
    a, b = _inputs(mlxq), _inputs(mlxq)
    rng = np.random.default_rng(7)
    b["x1"] = to_gpu(bf16_normal(rng, (1, 3072)))
    b["xw"] = to_gpu(bf16_normal(rng, (1024, 3072)))
    b["xf"] = to_gpu(rng.standard_normal((256, 3072)).astype(np.float32), torch.float32)
    ref_a = [t.clone() for t in _run(mlxq, a)]
    ref_b = [t.clone() for t in _run(mlxq, b)]
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    sa.wait_stream(torch.cuda.current_stream())
    sb.wait_stream(torch.cuda.current_stream())
    outs_a, outs_b = [], []
    for _ in range(3):
        with torch.cuda.stream(sa):
            outs_a.append(_run(mlxq, a))
        with torch.cuda.stream(sb):
            outs_b.append(_run(mlxq, b))
    torch.cuda.synchronize()
    for rep in range(3):
        for o, e in zip(outs_a[rep], ref_a):
            assert torch.equal(o, e), f"stream a, round {rep}"
        for o, e in zip(outs_b[rep], ref_b):
            assert torch.equal(o, e), f"stream b, round {rep}"
    print("    both streams bit-identical to their sequential results", flush=True)
