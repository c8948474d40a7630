"""Seeded random shapes through every dispatch path of the quantized linear, against the oracle.

The other GPU tests pin each kernel at chosen shapes and edges; this one draws (M, N, K, group
size, bits, bias, LoRA, activation) at random from fixed seeds, so shapes nobody picked by hand
reach the GEMV (M <= 8), the small-grid, generic and wide GEMMs (bf16 x) and the f32 GEMM (f32 x),
each checked with the quantized_matmul tolerance (relFro <= 2e-3, per-element |delta| <= 1e-2 of
max|y|) against the oracle on a sample of rows, and the f32 products at the exact-f32 bar.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, banner, bf16_normal, errors, to_gpu, to_np, wq_to_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu

# M buckets: GEMV, small grids, mid-size prefill, wide grids.
M_BUCKETS = [(1, 8), (9, 96), (97, 700), (701, 2400)]


@pytest.fixture(scope="module")
def mlxq():
    import mlxq as m
    m.load()
    return m


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    lo, hi = M_BUCKETS[seed % len(M_BUCKETS)]
    M = int(rng.integers(lo, hi + 1))
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    K = gs * int(rng.integers(2, max(3, 4096 // gs) + 1))
    N = int(rng.integers(1, 3000)) if rng.random() < 0.5 else 8 * int(rng.integers(1, 400))
    bias = bool(rng.random() < 0.5)
    lora = bool(rng.random() < 0.4)
    scale = float(rng.choice([1.0, 0.5, 1.25]))
    act = int(rng.choice([0, 0, 2, 3]))
    return rng, M, N, K, gs, bits, bias, lora, scale, act


def _rows(rng, M):
    if M <= 64:
        return np.arange(M)
    return np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 46)]))


@pytest.mark.parametrize("seed", range(96))
def test_random_bf16_linear_vs_oracle(mlxq, seed):
    rng, M, N, K, gs, bits, bias, lora, scale, act = _draw(seed)
    banner("random bf16 linear", seed, M, N, K, gs, bits, bias, lora, scale, act)
    x = bf16_normal(rng, (M, K))
    w = bf16_normal(rng, (N, K), 0.02)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=True)
    kw, okw = {}, {}
    if bias:
        bv = bf16_normal(rng, (N,), 0.5)
        kw["bias"] = to_gpu(bv)
        okw["bias"] = bv
    if lora:
        A = bf16_normal(rng, (K, 16), 0.01)
        B = bf16_normal(rng, (16, N), 0.01)
        kw.update(lora_a=to_gpu(A), lora_b=to_gpu(B), lora_scale=scale)
        okw.update(lora_a=A, lora_b=B, lora_scale=scale)
    y = to_np(mlxq.linear(to_gpu(x), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb), gs, bits, activation=act, **kw))
    rows = _rows(rng, M)
    ref = oracle.linear(x[rows], rwq, rs, rb, gs, bits, w_bf16=M > 8, act_bf16=True, act=act, **okw)
    assert_close(y[rows], ref, f"seed {seed}")


@pytest.mark.parametrize("seed", range(24))
def test_random_f32_quantized_matmul_vs_exact(mlxq, seed):
    rng = np.random.default_rng(5000 + seed)
    M = int(rng.integers(9, 900))
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    K = gs * int(rng.integers(2, max(3, 3072 // gs) + 1))
    N = int(rng.integers(1, 2000))
    sdt = "bf16" if rng.random() < 0.7 else "f32"
    banner("random f32 qmm", seed, M, N, K, gs, bits, sdt)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if sdt == "bf16":
        w = oracle.bf16_round(w)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=sdt == "bf16")
    tdt = torch.bfloat16 if sdt == "bf16" else torch.float32
    y = mlxq.quantized_matmul(to_gpu(x, torch.float32), wq_to_gpu(rwq), to_gpu(rs, tdt), to_gpu(rb, tdt),
                              True, gs, bits)
    assert y.dtype == torch.float32
    rows = _rows(rng, M)
    ref = oracle.quantized_matmul(x[rows], rwq, rs, rb, gs, bits, w_bf16=False, out_bf16=False)
    rel, peak = errors(to_np(y)[rows], ref)
    print(f"    seed {seed} relFro={rel:.3e} peak={peak:.3e}", flush=True)
    assert rel < 1e-4 and peak < 1e-3


@pytest.mark.parametrize("seed", range(24))
def test_random_quantize_dequantize_bit_exact(mlxq, seed):
    """quantize and dequantize at random shapes, bf16 or f32 weights: codes, scales, biases and the
    dequantized matrix bit for bit against the oracle."""
    rng = np.random.default_rng(7000 + seed)
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    K = gs * int(rng.integers(1, max(2, 4096 // gs) + 1))
    N = int(rng.integers(1, 2000))
    bf = bool(rng.random() < 0.6)
    banner("random quantize", seed, N, K, gs, bits, "bf16" if bf else "f32")
    w = (rng.standard_normal((N, K)) * float(rng.choice([0.02, 1.0, 30.0]))).astype(np.float32)
    if bf:
        w = oracle.bf16_round(w)
    dt = torch.bfloat16 if bf else torch.float32
    wq, s, b = mlxq.quantize(to_gpu(w, dt), gs, bits)
    rwq, rs, rb = oracle.quantize(w, gs, bits, sb_bf16=bf)
    assert np.array_equal(to_np(wq), rwq)
    assert np.array_equal(to_np(s), rs) and np.array_equal(to_np(b), rb)
    d = mlxq.dequantize(wq, s, b, gs, bits)
    assert np.array_equal(to_np(d), oracle.dequantize(rwq, rs, rb, gs, bits, out_bf16=bf))


@pytest.mark.parametrize("seed", range(24))
def test_random_swiglu_vs_oracle(mlxq, seed):
    """The fused decode SwiGLU (M <= 8) at random shapes against the oracle's op-by-op h."""
    rng = np.random.default_rng(9000 + seed)
    M = int(rng.integers(1, 9))
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    step = max(gs, 512 // bits)
    K = step * int(rng.integers(1, 4096 // step + 1))
    F = int(rng.integers(1, 3000))
    banner("random swiglu", seed, M, K, F, gs, bits)
    x = bf16_normal(rng, (M, K))
    tg, tu = [oracle.quantize(bf16_normal(rng, (F, K), 0.02), gs, bits, sb_bf16=True) for _ in range(2)]
    g, u = [(wq_to_gpu(t[0]), to_gpu(t[1]), to_gpu(t[2])) for t in (tg, tu)]
    h = to_np(mlxq.swiglu(to_gpu(x), g, u, gs, bits))
    gr = oracle.quantized_matmul(x, *tg, gs, bits, w_bf16=False, out_bf16=True)
    ur = oracle.quantized_matmul(x, *tu, gs, bits, w_bf16=False, out_bf16=True)
    ref_h = oracle.bf16_round(oracle.bf16_round(np.vectorize(oracle.silu)(gr).astype(np.float32)) * ur)
    assert_close(h, ref_h, f"seed {seed}")
    print(f"    bit-identical h: {np.mean(h == ref_h) * 100:.2f} %", flush=True)


@pytest.mark.parametrize("seed", range(16))
def test_random_stacked_experts_vs_oracle(mlxq, seed):
    """Stacked-expert projections (qmm_experts) at random expert counts and shapes, shared or
    per-expert x, with or without a bf16 bias, each expert against the oracle's linear."""
    rng = np.random.default_rng(11000 + seed)
    E = int(rng.integers(1, 9))
    M = int(rng.choice([int(rng.integers(1, 9)), int(rng.integers(9, 700))]))
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    K = gs * int(rng.integers(2, max(3, 3072 // gs) + 1))
    N = int(rng.integers(1, 2400))
    per_expert = bool(rng.random() < 0.5)
    with_bias = bool(rng.random() < 0.6)
    banner("random experts", seed, E, M, N, K, gs, bits, per_expert, with_bias)
    packs = [oracle.quantize(bf16_normal(rng, (N, K), 0.02), gs, bits, sb_bf16=True) for _ in range(E)]
    wq, s, b = (np.stack([p[i] for p in packs]) for i in range(3))
    bias = bf16_normal(rng, (E, N), 0.5) if with_bias else None
    x = bf16_normal(rng, (E, M, K) if per_expert else (M, K))
    y = to_np(mlxq.qmm_experts(to_gpu(x), wq_to_gpu(wq), to_gpu(s), to_gpu(b), gs, bits,
                               bias=None if bias is None else to_gpu(bias), per_expert=per_expert))
    assert y.shape == (E, M, N)
    rows = _rows(rng, M)
    for e, p in enumerate(packs):
        xe = x[e] if per_expert else x
        ref = oracle.linear(xe[rows], *p, gs, bits, w_bf16=M > 8, act_bf16=True,
                            bias=None if bias is None else bias[e])
        assert_close(y[e][rows], ref, f"seed {seed} expert {e}")


@pytest.mark.parametrize("seed", range(24))
def test_random_f32_fp16_linear_vs_oracle(mlxq, seed):
    """linear with f32 or fp16 activations (FLUX.1's f32 stream, SDXL's fp16 stream) at random
    shapes, bf16 scales, with a bias in either dtype, a bf16 LoRA adapter and an activation: the
    f32 result against the oracle's f32 linear."""
    rng = np.random.default_rng(13000 + seed)
    lo, hi = M_BUCKETS[seed % len(M_BUCKETS)]
    M = int(rng.integers(lo, min(hi, 1200) + 1))
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    K = gs * int(rng.integers(2, max(3, 2048 // gs) + 1))
    N = int(rng.integers(1, 2000))
    fp16 = bool(rng.random() < 0.5)
    bias_dt = str(rng.choice(["none", "bf16", "f32"]))
    lora = bool(rng.random() < 0.4)
    act = int(rng.choice([0, 1, 2, 3]))
    banner("random f32/fp16 linear", seed, M, N, K, gs, bits, "fp16" if fp16 else "f32", bias_dt, lora, act)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x = x.astype(np.float16).astype(np.float32) if fp16 else x
    rwq, rs, rb = oracle.quantize(bf16_normal(rng, (N, K), 0.02), gs, bits, sb_bf16=True)
    kw, okw = {}, {}
    if bias_dt != "none":
        bv = (rng.standard_normal(N) * 0.5).astype(np.float32)
        if bias_dt == "bf16":
            bv = oracle.bf16_round(bv)
        kw["bias"] = to_gpu(bv, torch.bfloat16 if bias_dt == "bf16" else torch.float32)
        okw.update(bias=bv, bias_bf16=bias_dt == "bf16")
    if lora:
        A = bf16_normal(rng, (K, 16), 0.05)
        B = bf16_normal(rng, (16, N), 0.05)
        kw.update(lora_a=to_gpu(A), lora_b=to_gpu(B), lora_scale=0.75)
        okw.update(lora_a=A, lora_b=B, lora_bf16=True, lora_scale=0.75)
    y = mlxq.linear(to_gpu(x, torch.float16 if fp16 else torch.float32), wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb),
                    gs, bits, activation=act, **kw)
    assert y.dtype == torch.float32
    rows = _rows(rng, M)
    ref = oracle.linear(x[rows], rwq, rs, rb, gs, bits, w_bf16=False, x_bf16=False, sb_bf16=True, act=act, **okw)
    rel, peak = errors(to_np(y)[rows], ref)
    print(f"    seed {seed} relFro={rel:.3e} peak={peak:.3e}", flush=True)
    assert rel < 1e-4 and peak < 1e-3


@pytest.mark.parametrize("seed", range(16))
def test_random_embedding_bit_exact(mlxq, seed):
    """The quantized TokenEmbedding gather at random table shapes and id batches, bf16 or f32
    scales, bf16 or f32 output: bit for bit the oracle's dequantized rows."""
    rng = np.random.default_rng(15000 + seed)
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    hidden = gs * int(rng.integers(1, max(2, 2048 // gs) + 1))
    vocab = int(rng.integers(1, 5000))
    sb_bf16 = bool(rng.random() < 0.6)
    out_dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    shape = tuple(int(d) for d in rng.integers(1, 40, size=int(rng.integers(1, 3))))
    banner("random embedding", seed, vocab, hidden, gs, bits, sb_bf16, out_dtype, shape)
    w = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float32)
    if sb_bf16:
        w = oracle.bf16_round(w)
    wq, s, b = oracle.quantize(w, gs, bits, sb_bf16=sb_bf16)
    ids = rng.integers(0, vocab, size=shape).astype(np.int32)
    sdt = torch.bfloat16 if sb_bf16 else torch.float32
    y = mlxq.embedding(torch.from_numpy(ids).cuda(), wq_to_gpu(wq), to_gpu(s, sdt), to_gpu(b, sdt), gs, bits,
                       out_dtype)
    assert y.shape == (*shape, hidden) and y.dtype == out_dtype
    ref = oracle.dequantize(wq, s, b, gs, bits, out_bf16=sb_bf16)[ids]
    if out_dtype == torch.bfloat16:
        ref = oracle.bf16_round(ref)
    assert np.array_equal(to_np(y), ref)


@pytest.mark.parametrize("seed", range(16))
def test_random_lora_residual_vs_reference(mlxq, seed):
    """One more LoRA adapter on a computed bf16 y (Adapter::residual, src/adapters.rs:260-270) at
    random M, K, N, rank (1-64) and scale: round(y + round(round(round(x.A).B) * scale)), each op
    rounded to bf16, from fp64 products."""
    rng = np.random.default_rng(17000 + seed)
    M = int(rng.choice([int(rng.integers(1, 9)), int(rng.integers(9, 600)), int(rng.integers(4000, 6000))]))
    K = 8 * int(rng.integers(1, 384))
    N = int(rng.integers(1, 1500))
    rank = int(rng.integers(1, 65))
    scale = float(rng.choice([1.0, 0.5, 1.25, 2.0]))
    banner("random lora residual", seed, M, K, N, rank, scale)
    x = bf16_normal(rng, (M, K))
    y = bf16_normal(rng, (M, N))
    A = bf16_normal(rng, (K, rank), 0.05)
    B = bf16_normal(rng, (rank, N), 0.05)
    out = to_np(mlxq.ops.lora_residual(to_gpu(x), to_gpu(y), to_gpu(A), to_gpu(B), scale))
    xa = oracle.bf16_round((x.astype(np.float64) @ A.astype(np.float64)).astype(np.float32))
    r = oracle.bf16_round((xa.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
    if scale != 1.0:
        r = oracle.bf16_round(r * np.float32(scale))
    want = oracle.bf16_round(y + r)
    assert_close(out, want, f"seed {seed}")


@pytest.mark.parametrize("seed", range(8))
def test_random_quantize_batched_matches_per_weight(mlxq, seed):
    """mlxq_quantize_batched over 1-20 weights of a random shape: bit for bit one quantize per
    weight (launches of up to 16 weights)."""
    rng = np.random.default_rng(19000 + seed)
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    K = gs * int(rng.integers(1, max(2, 2048 // gs) + 1))
    N = int(rng.integers(1, 1500))
    count = int(rng.integers(1, 21))
    dt = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    banner("random quantize batched", seed, count, N, K, gs, bits, dt)
    ws = [to_gpu((rng.standard_normal((N, K)) * 0.02).astype(np.float32), dt) for _ in range(count)]
    got = mlxq.quantize_batched(ws, gs, bits)
    assert len(got) == count
    for w, (wq, s, b) in zip(ws, got):
        rq, rs, rb = mlxq.quantize(w, gs, bits)
        assert torch.equal(wq, rq) and torch.equal(s, rs) and torch.equal(b, rb)


@pytest.mark.parametrize("seed", range(16))
def test_random_forced_kernels_vs_oracle(mlxq, seed):
    """The forced entry points at random shapes: mlxq_qmm (the bf16-tile GEMM at any M, small M
    included) against the GEMM oracle, mlxq_qmv (the matrix-core GEMV) and mlxq_qmv_valu (the
    VALU GEMV) at M <= 8 against the exact-f32 oracle."""
    rng = np.random.default_rng(21000 + seed)
    gs = int(rng.choice([32, 64, 128]))
    bits = int(rng.choice([4, 8]))
    K = gs * int(rng.integers(1, max(2, 3072 // gs) + 1))
    N = int(rng.integers(1, 2500))
    Mg = int(rng.integers(1, 600))
    Mv = int(rng.integers(1, 9))
    banner("random forced kernels", seed, Mg, Mv, N, K, gs, bits)
    rwq, rs, rb = oracle.quantize(bf16_normal(rng, (N, K), 0.02), gs, bits, sb_bf16=True)
    g = (wq_to_gpu(rwq), to_gpu(rs), to_gpu(rb))
    x = bf16_normal(rng, (Mg, K))
    rows = _rows(rng, Mg)
    y = to_np(mlxq.qmm(to_gpu(x), *g, gs, bits))
    assert_close(y[rows], oracle.quantized_matmul(x[rows], rwq, rs, rb, gs, bits, w_bf16=True, out_bf16=True),
                 f"qmm seed {seed}")
    xv = bf16_normal(rng, (Mv, K))
    ref = oracle.quantized_matmul(xv, rwq, rs, rb, gs, bits, w_bf16=False, out_bf16=True)
    assert_close(to_np(mlxq.qmv(to_gpu(xv), *g, gs, bits)), ref, f"qmv seed {seed}")
    assert_close(to_np(mlxq.qmv_valu(to_gpu(xv), *g, gs, bits)), ref, f"qmv_valu seed {seed}")
