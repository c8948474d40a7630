"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric, config 2 — FLUX.1-dev double-stream DiT MLP at 1024^2):
  x [4608,3072] bf16 ~ N(0,1);  W_up [12288,3072], W_down [3072,12288] ~ N(0,0.02), Q4 g64.
  One step = y = qmm(gelu(qmm(x, W_up)), W_down): the up projection with the exact-erf GELU fused
  into its epilogue, then the down projection — 695.8 GFLOP of algorithmic work.
  value = whole-step TFLOP/s over the median of K timed steps (HIP events per step; inputs
  resident in HBM), after an untimed clock pre-run (--prerun-seconds) and W warm-up steps.

Also reported (same JSON line):
  roofline     qmm kernel: algorithmic FLOP per launch / median launch time (HIP events around
               each launch on the launching stream) vs the 2.5166 PFLOP/s dense bf16 MFMA peak;
  gemv         config 4 decode GEMV, M in {1,2,4,8}: HBM GB/s over gate/up/down with the weights
               rotated over 8 copies (> the 256 MB Infinity Cache);
  quantize     config 3 quantize pass (4 x [5120,5120] bf16 -> Q8 g64): GB/s;
  config1/3/5  the other BASELINE configs (quantize/dequantize/qmm, the Q8 projection, the LoRA sweep);
  experts      the stacked-expert MoE projections (one launch vs one linear per expert);
  f32_mlp      config 2 on FLUX.1's f32 stream (f32 x and h, f32 matrix-core GEMM on split bf16);
  dense_bf16_reference  context only: the library dense bf16 GEMM (torch.mm) on the same shapes;
  cpu_baseline the CPU oracle (fp64-accumulating C restatement, OpenMP) on a bounded row sample of
               the same up-projection, scaled to TFLOP/s.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mlx-gen_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "qmatmul TFLOP/s (Q4 g64, FLUX MLP shape) + GEMV HBM GB/s, 1×MI355X"
MFMA_BF16_PEAK_TFLOPS = 2516.6
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-extras", action="store_true", help="headline GEMM only")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--prerun-seconds", type=float, default=1.0,
                   help="untimed clock pre-run of the headline MLP before its warm-up steps")
    p.add_argument("--only", choices=("all", "mlp", "gemv", "quantize", "copy", "configs", "experts", "f32",
                                       "dense", "gemv_long"),
                   default="all",
                   help="run one leg only (for profiling); 'copy' is the plain-copy calibration "
                        "kernel for the HBM byte counters; 'gemv_long' (not part of 'all') times "
                        "the decode GEMV over long and ragged K")
    p.add_argument("--pmc-sets", metavar="A,B", default=None,
                   help="with --summarize-pmc: only these counter-set subdirectories (copy_* always read)")
    p.add_argument("--summarize-trace", metavar="DIR",
                   help="print per-launch-shape duration statistics of the mlxq kernels in the "
                        "rocprofv3 --kernel-trace csv files under DIR and exit")
    p.add_argument("--trace-skip", type=int, default=0, metavar="N",
                   help="with --summarize-trace: leave out each launch shape's first N launches "
                        "(the warm-up steps), so the averages cover the timed launches")
    p.add_argument("--trace-last", type=int, default=0, metavar="N",
                   help="with --summarize-trace: keep only each launch shape's last N launches "
                        "(the timed steps after the clock pre-run and warm-up)")
    p.add_argument("--summarize-pmc", metavar="DIR",
                   help="print the counter summary of the rocprofv3 --pmc runs under DIR (one "
                        "subdirectory per counter set, see summarize_pmc) and exit")
    return p.parse_args()


def gen_bf16(shape, std, seed, device):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)


def bench_flux_mlp(mlxq, torch, steps, warmup, prerun_s):
    dev = torch.device("cuda:0")
    M, K, F = 4608, 3072, 12288
    x = gen_bf16((M, K), 1.0, 0, dev)
    wu = gen_bf16((F, K), 0.02, 1, dev)
    wd = gen_bf16((K, F), 0.02, 2, dev)
    qu = mlxq.quantize(wu, 64, 4)
    qd = mlxq.quantize(wd, 64, 4)
    del wu, wd
    h = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    y = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    from mlxq import _lib
    import ctypes
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    # bf16 stream: the dtype-preserving exact GELU (src/nn.rs:344-355), so h stays bf16.
    ep_gelu = _lib.Epilogue(None, None, None, 0, 1.0, _lib.MLXQ_ACT_GELU_EXACT, _lib.MLXQ_BFLOAT16,
                            _lib.MLXQ_BFLOAT16)

    def up():
        _lib.check(lib.mlxq_linear(x.data_ptr(), 1, M, K, qu[0].data_ptr(), qu[1].data_ptr(),
                                   qu[2].data_ptr(), 1, F, 64, 4, ctypes.byref(ep_gelu), h.data_ptr(),
                                   None, 0, sp))

    def down():
        _lib.check(lib.mlxq_quantized_matmul(h.data_ptr(), 1, M, F, qd[0].data_ptr(), qd[1].data_ptr(),
                                             qd[2].data_ptr(), 1, K, 1, 64, 4, y.data_ptr(), sp))

    # Untimed clock pre-run: the same two launches back to back for `prerun_s` seconds, so the
    # timed steps see the clock the chip settles at under this load rather than its ramp from
    # idle (the first steps of a cold process run several per cent slower).
    n_pre = 0
    t_pre = time.perf_counter()
    while time.perf_counter() - t_pre < prerun_s:
        for _ in range(8):
            up()
            down()
        torch.cuda.synchronize()
        n_pre += 8
    prerun = time.perf_counter() - t_pre
    for _ in range(warmup):
        up()
        down()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(stream)
        up()
        ev[i][1].record(stream)
        down()
        ev[i][2].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ups = [e[0].elapsed_time(e[1]) for e in ev]
    dns = [e[1].elapsed_time(e[2]) for e in ev]
    stp = [e[0].elapsed_time(e[2]) for e in ev]
    t_step = statistics.median(stp)
    flop_launch = 2.0 * M * K * F
    return {
        "ms_per_step": t_step,
        "mean_ms_per_step": sum(stp) / steps,
        "span_ms_per_step": ev[0][0].elapsed_time(ev[-1][2]) / steps,
        "wall_ms_per_step": wall * 1e3 / steps,
        "tflops": 2 * flop_launch / (t_step * 1e-3) / 1e12,
        "up_ms": statistics.median(ups), "down_ms": statistics.median(dns),
        "mean_up_ms": sum(ups) / steps, "mean_down_ms": sum(dns) / steps,
        "step_ms": [round(v, 4) for v in stp],
        "prerun": {"seconds": round(prerun, 3), "steps": n_pre},
        "qmm_launch_ms": (statistics.median(ups) + statistics.median(dns)) / 2,
        "qmm_flop_per_launch": flop_launch,
    }


def bench_gemv(mlxq, torch, reps=20):
    """Config 4: decode MLP GEMVs (Q4 g64) gate/up [8192,3072] and down [3072,8192].

    The weights are rotated over 8 MLP copies (340 MB, more than the 256 MB Infinity Cache), and
    one replay of a captured HIP graph runs 8 MLPs back to back, so the rate is GPU time
    including the gaps between kernels but without host launch overhead.  Two forms: three GEMV
    launches per MLP (gate, up, down, then silu(g)*u left to the caller) and the fused form
    (one SwiGLU launch reading gate and up, then down), which also does the activation."""
    dev = torch.device("cuda:0")
    K, F = 3072, 8192
    copies = []
    for c in range(8):
        g = mlxq.quantize(gen_bf16((F, K), 0.02, 100 + 3 * c, dev), 64, 4)
        u = mlxq.quantize(gen_bf16((F, K), 0.02, 101 + 3 * c, dev), 64, 4)
        d = mlxq.quantize(gen_bf16((K, F), 0.02, 102 + 3 * c, dev), 64, 4)
        copies.append((g, u, d))
    torch.cuda.synchronize()
    out = {}
    wbytes_gu = F * K // 2 + F * (K // 64) * 4  # codes + bf16 scales and biases
    wbytes_d = K * F // 2 + K * (F // 64) * 4
    for M in (1, 2, 4, 8):
        x = gen_bf16((M, K), 1.0, 7, dev)
        hh = gen_bf16((M, F), 1.0, 8, dev)
        yg = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
        yu = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
        h = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
        yd = torch.empty((M, K), dtype=torch.bfloat16, device=dev)

        def mlps():
            for (g, u, d) in copies:
                mlxq.qmv(x, *g, 64, 4, out=yg)
                mlxq.qmv(x, *u, 64, 4, out=yu)
                mlxq.qmv(hh, *d, 64, 4, out=yd)

        def fused():
            for (g, u, d) in copies:
                mlxq.swiglu(x, g, u, 64, 4, out=h)
                mlxq.qmv(h, *d, 64, 4, out=yd)

        def valu():
            for (g, u, d) in copies:
                mlxq.qmv_valu(x, *g, 64, 4, out=yg)
                mlxq.qmv_valu(x, *u, 64, 4, out=yu)
                mlxq.qmv_valu(hh, *d, 64, 4, out=yd)

        us3 = graph_ms(torch, mlps, inner=1, reps=reps) * 1e3 / len(copies)
        us2 = graph_ms(torch, fused, inner=1, reps=reps) * 1e3 / len(copies)
        usv = graph_ms(torch, valu, inner=1, reps=reps) * 1e3 / len(copies)
        nbytes3 = 2 * wbytes_gu + wbytes_d + 2 * (2 * M * K) + 2 * (2 * M * F) + 2 * M * F + 2 * M * K
        nbytes2 = 2 * wbytes_gu + wbytes_d + 2 * M * K + 2 * M * F + 2 * M * F + 2 * M * K
        out[f"M{M}"] = {"us_per_mlp": round(us3, 3), "GBs": round(nbytes3 / (us3 * 1e-6) / 1e9, 1),
                        "bytes_per_mlp": nbytes3,
                        "fused_us_per_mlp": round(us2, 3),
                        "fused_GBs": round(nbytes2 / (us2 * 1e-6) / 1e9, 1),
                        "fused_frac_of_hbm_peak": round(nbytes2 / (us2 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        "valu_us_per_mlp": round(usv, 3),
                        "valu_GBs": round(nbytes3 / (usv * 1e-6) / 1e9, 1)}
    out["note"] = ("per decode MLP, replayed from a HIP graph (rates include inter-kernel gaps): "
                   "3 matrix-core GEMV launches (gate, up, down); the fused form (SwiGLU gate/up "
                   "launch + down launch); and, for the kernel-choice A/B, 3 VALU GEMV launches "
                   "(mlxq_qmv_valu); per-kernel durations are in profiles/")
    return out


GEMV_LONG_SHAPES = ((11008, 4096), (14336, 4096), (13824, 5120), (18944, 3584))


def bench_gemv_long(mlxq, torch, reps=10):
    """Decode GEMVs over the long and ragged K of common decoder down projections (Q4 g64,
    M = 1, 2, 4, 8): the matrix-core path (one-row kernel at M = 1; tile kernel with a ragged last
    wave, two-round load rings or launches of four / two rows at M >= 2) against the VALU GEMV on
    the same weights.  Weight copies rotate past the 256 MB Infinity Cache; one graph replay runs
    every copy once."""
    dev = torch.device("cuda:0")
    out = {}
    for K, N in GEMV_LONG_SHAPES:
        wbytes = N * K // 2 + N * (K // 64) * 4
        ncopy = max(2, -(-320_000_000 // wbytes))
        copies = [mlxq.quantize(gen_bf16((N, K), 0.02, 200 + c, dev), 64, 4) for c in range(ncopy)]
        torch.cuda.synchronize()
        for M in (1, 2, 4, 8):
            x = gen_bf16((M, K), 1.0, 9, dev)
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

            def mfma():
                for w in copies:
                    mlxq.qmv(x, *w, 64, 4, out=y)

            def valu():
                for w in copies:
                    mlxq.qmv_valu(x, *w, 64, 4, out=y)

            us = graph_ms(torch, mfma, inner=1, reps=reps) * 1e3 / ncopy
            usv = graph_ms(torch, valu, inner=1, reps=reps) * 1e3 / ncopy
            nbytes = wbytes + 2 * M * K + 2 * M * N
            out[f"M{M}_K{K}_N{N}"] = {"us": round(us, 2), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
                                      "valu_us": round(usv, 2),
                                      "valu_GBs": round(nbytes / (usv * 1e-6) / 1e9, 1)}
        del copies
        torch.cuda.empty_cache()
    out["note"] = ("per launch (a launch sequence when M is split), replayed from a HIP graph over "
                   "rotated weight copies; valu: mlxq_qmv_valu on the same operands")
    return out


QUANT_SETS = 2  # config-3 weight sets rotated (8 x 52 MB read + 8 x 28 MB written: > 256 MB MALL)


def bench_quantize(mlxq, torch, iters=10):
    """Config 3 quantize pass: 4 x [5120,5120] bf16 -> Q8 g64 (321.1 MB algorithmic), timed over
    QUANT_SETS distinct sets of four weights so the Infinity Cache cannot hold one pass's data."""
    dev = torch.device("cuda:0")
    # Each set's four weights are consecutive row blocks of one tensor, so the batched legs can
    # stream a set as one buffer; the per-weight legs see four ordinary contiguous weights.
    sets = [gen_bf16((4 * 5120, 5120), 0.02, 200 + i, dev) for i in range(QUANT_SETS)]
    ws = [t[5120 * j:5120 * (j + 1)] for t in sets for j in range(4)]
    outs = [(torch.empty((5120, 1280), dtype=torch.int32, device=dev),
             torch.empty((5120, 80), dtype=torch.bfloat16, device=dev),
             torch.empty((5120, 80), dtype=torch.bfloat16, device=dev)) for _ in ws]
    from mlxq import _lib
    import ctypes
    lib = _lib.load()

    def run():
        sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)  # the capturing stream
        for w, (q, s, b) in zip(ws, outs):
            _lib.check(lib.mlxq_quantize(w.data_ptr(), 1, 5120, 5120, 64, 8, q.data_ptr(), s.data_ptr(),
                                         b.data_ptr(), sp))

    arr4 = ctypes.c_void_p * 4

    def run_batched():  # one mlxq_quantize_batched launch per set of four
        sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for i in range(QUANT_SETS):
            sw, so = ws[4 * i:4 * i + 4], outs[4 * i:4 * i + 4]
            _lib.check(lib.mlxq_quantize_batched(
                arr4(*[w.data_ptr() for w in sw]), 4, 1, 5120, 5120, 64, 8, arr4(*[o[0].data_ptr() for o in so]),
                arr4(*[o[1].data_ptr() for o in so]), arr4(*[o[2].data_ptr() for o in so]), sp))
    # Replayed from a HIP graph like the GEMV leg, so the ~17 us launches are not spaced out by
    # the host's per-call overhead (the rate still includes the gaps between the four kernels).
    # Every weight writes its own preallocated outputs: outputs allocated per call inside a graph
    # reuse one freed buffer, whose repeated writes then stay in the caches (~15 % faster, not
    # the traffic of a real conversion).
    ms = graph_ms(torch, run, inner=1, reps=iters) / QUANT_SETS
    nbytes = 4 * (5120 * 5120 * 2 + 5120 * 5120 + 5120 * 80 * 4)
    # Reference point: the same memory pattern and launch shape with trivial arithmetic (the
    # stream kernel of libmlxq_bench.so), reading the same weights and writing the Q8 code bytes
    # into buffers of their own, same timing.
    ref = stream_reference(torch, ws, 8, iters) / QUANT_SETS
    rbytes = 4 * (5120 * 5120 * 2 + 5120 * 5120)
    # The same pass as one launch per set (mlxq_quantize_batched), against the stream kernel over
    # each set's four weights in one launch.
    mb = graph_ms(torch, run_batched, inner=1, reps=iters) / QUANT_SETS
    refb = stream_reference(torch, sets, 8, iters) / QUANT_SETS
    return {"us_per_pass": ms * 1e3, "GBs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes,
            "frac_of_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "stream_reference_us_per_pass": round(ref * 1e3, 2),
            "stream_reference_GBs": round(rbytes / (ref * 1e-3) / 1e9, 1),
            "frac_of_stream_reference_time": round(ref / ms, 4),
            "batched_us_per_pass": round(mb * 1e3, 2),
            "batched_GBs": round(nbytes / (mb * 1e-3) / 1e9, 1),
            "batched_frac_of_hbm_peak": round(nbytes / (mb * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "batched_stream_reference_us_per_pass": round(refb * 1e3, 2),
            "batched_stream_reference_GBs": round(rbytes / (refb * 1e-3) / 1e9, 1),
            "note": "4 launches per pass (the reference's weight-by-weight calls), each weight into its "
                    f"own outputs, passes rotated over {QUANT_SETS} weight sets; stream_reference: "
                    "quantize's load/store pattern and grid with trivial arithmetic on the same weights "
                    "(reads the weights, writes the code bytes; no scales), same timing; batched_*: the "
                    "same pass as one mlxq_quantize_batched launch per set of four, against the stream "
                    "kernel over the four weights in one launch"}


def stream_reference(torch, ws, words, reps):
    """Milliseconds per pass of the bench stream kernel over the weights ws (each 64-byte chunk of
    a weight read, 4 * words bytes written into its own output), with quantize's grid: one
    256-thread workgroup per 256 chunks, one chunk per thread."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "mlx-gen_amd", "mlxq", "libmlxq_bench.so"))
    lib.mlxq_bench_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                      ctypes.c_int64, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    chunks = [w.numel() * w.element_size() // 64 for w in ws]
    outs = [torch.empty(c * 4 * words, dtype=torch.uint8, device=dev) for c in chunks]

    for w, c, o in zip(ws, chunks, outs):  # host-side shape check before any launch
        assert w.is_contiguous() and w.numel() * w.element_size() == c * 64 and o.numel() == c * 4 * words

    def run():
        sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for w, c, o in zip(ws, chunks, outs):
            blocks = (c + 255) // 256
            if lib.mlxq_bench_stream(w.data_ptr(), c, o.data_ptr(), words, blocks, sp) != 0:
                raise RuntimeError("bench stream kernel failed")
    return graph_ms(torch, run, inner=1, reps=reps)


def graph_ms(torch, fn, inner=8, reps=5):
    """Mean milliseconds of fn() on the GPU: `inner` calls captured in one HIP graph, replayed
    `reps` times between events (no host launch overhead in the measurement)."""
    dev = torch.device("cuda:0")
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn()  # warm-up outside capture
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(inner):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) / (reps * inner)


def bench_f32_mlp(mlxq, torch):
    """Config 2's MLP on FLUX.1's f32 residual stream (mlx-gen-flux/src/model.rs:407-410): f32 x
    [4608,3072] through the Q4-g64 up projection with mlx_rs::nn::gelu (f32), then the f32 h through
    the down projection.  Both products are f32 (MLX's promotion) and run on the factored f32 GEMM
    (group size 64): the codes as exact bf16 operands against the two-term split of x, two bf16
    MFMA passes per product, so its MFMA work is 2x the algorithmic flops."""
    dev = torch.device("cuda:0")
    M, K, F = 4608, 3072, 12288
    x = gen_bf16((M, K), 1.0, 900, dev).float()
    qu = mlxq.quantize(gen_bf16((F, K), 0.02, 901, dev), 64, 4)
    qd = mlxq.quantize(gen_bf16((K, F), 0.02, 902, dev), 64, 4)
    h = mlxq.linear(x, *qu, 64, 4, activation=mlxq.MLXQ_ACT_GELU)
    y = torch.empty((M, K), dtype=torch.float32, device=dev)
    up = lambda: mlxq.linear(x, *qu, 64, 4, activation=mlxq.MLXQ_ACT_GELU)
    down = lambda: mlxq.quantized_matmul(h, *qd, True, 64, 4, out=y)
    t_up = graph_ms(torch, up, inner=2, reps=3)
    t_dn = graph_ms(torch, down, inner=2, reps=3)
    flop = 2.0 * M * K * F
    tf = 2 * flop / ((t_up + t_dn) * 1e-3) / 1e12
    return {"up_ms": round(t_up, 4), "down_ms": round(t_dn, 4),
            "up_TFLOPs": round(flop / (t_up * 1e-3) / 1e12, 1),
            "down_TFLOPs": round(flop / (t_dn * 1e-3) / 1e12, 1),
            "TFLOPs": round(tf, 1),
            "roofline": {"bound": "mfma", "unit": "TFLOP/s", "peak": MFMA_BF16_PEAK_TFLOPS,
                         "achieved": round(2 * tf, 1), "frac": round(2 * tf / MFMA_BF16_PEAK_TFLOPS, 4),
                         "note": "bf16 MFMA work: two passes (hi and lo halves of the f32 "
                                 "activations) per algorithmic flop, against the bf16 dense peak"},
            "note": "f32 x and h; GELU fused into the up GEMM epilogue; TFLOPs counts algorithmic "
                    "flops once"}


def bench_dense_reference(torch):
    """Context for the roofline fraction, not part of the path: the library dense bf16 GEMM
    (torch.mm on hipBLASLt) on config 2's two shapes with the bf16 weights themselves (no
    quantization, no dequantization, no GELU).  The right operand is W^T made contiguous [K, N]."""
    dev = torch.device("cuda:0")
    M, K, F = 4608, 3072, 12288
    x = gen_bf16((M, K), 1.0, 0, dev)
    wu_t = gen_bf16((F, K), 0.02, 1, dev).t().contiguous()
    wd_t = gen_bf16((K, F), 0.02, 2, dev).t().contiguous()
    h = gen_bf16((M, F), 1.0, 3, dev)
    yu = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    yd = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    def ev_ms(fn, reps=20):  # plain launches between events (no graph capture of library calls)
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    t_up = ev_ms(lambda: torch.mm(x, wu_t, out=yu))
    t_dn = ev_ms(lambda: torch.mm(h, wd_t, out=yd))
    flop = 2.0 * M * K * F
    tf = 2 * flop / ((t_up + t_dn) * 1e-3) / 1e12
    return {"up_ms": round(t_up, 4), "down_ms": round(t_dn, 4),
            "up_TFLOPs": round(flop / (t_up * 1e-3) / 1e12, 1),
            "down_TFLOPs": round(flop / (t_dn * 1e-3) / 1e12, 1),
            "TFLOPs": round(tf, 1), "frac_of_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "note": "torch.mm (hipBLASLt) on dense bf16 weights of the config-2 shapes: the vendor "
                    "GEMM without dequantization, for context only"}


CONFIG1_COPIES = 16  # distinct config-1 weights rotated (16 x 24 MB > the 256 MB Infinity Cache)


def bench_config1(mlxq, torch):
    """Config 1 round trip: W[3072,3072] bf16 -> Q4 g64, dequantize, x[256,3072] . W^T.  Each op is
    timed over CONFIG1_COPIES distinct weights (each with its own outputs), one launch per weight,
    so a weight's 24 MB are not served from the Infinity Cache by the previous launch."""
    dev = torch.device("cuda:0")
    ws = [gen_bf16((3072, 3072), 0.02, 300 + 7 * i, dev) for i in range(CONFIG1_COPIES)]
    x = gen_bf16((256, 3072), 1.0, 301, dev)
    qs = [mlxq.quantize(w, 64, 4) for w in ws]
    qo = [tuple(torch.empty_like(t) for t in q) for q in qs]
    do = [torch.empty_like(w) for w in ws]
    yo = torch.empty((256, 3072), dtype=torch.bfloat16, device=dev)
    from mlxq import _lib
    import ctypes
    lib = _lib.load()

    def quant():
        sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for w, (wq, sc, bi) in zip(ws, qo):
            _lib.check(lib.mlxq_quantize(w.data_ptr(), 1, 3072, 3072, 64, 4, wq.data_ptr(), sc.data_ptr(),
                                         bi.data_ptr(), sp))

    def deq():
        sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for (wq, sc, bi), d in zip(qs, do):
            _lib.check(lib.mlxq_dequantize(wq.data_ptr(), sc.data_ptr(), bi.data_ptr(), 1, 3072, 3072, 64, 4,
                                           d.data_ptr(), sp))

    def mm():
        for q in qs:
            mlxq.quantized_matmul(x, *q, True, 64, 4, out=yo)
    # The vendor's dense bf16 GEMM on the same shape (torch.mm, hipBLASLt), W^T made contiguous
    # [K, N], rotated over the same number of distinct weights and timed the same way (a HIP
    # graph, since a ~10 us launch from the host would be launch-bound): context for the
    # small-grid kernel, not a measure of it (it reads 18.9 MB of bf16 weights where the Q4 GEMM
    # reads 5.3 MB).  The graph's last output is checked against an eager call.
    wts = [w.t().contiguous() for w in ws]
    yd = torch.empty((256, 3072), dtype=torch.bfloat16, device=dev)

    def dense():
        for wt in wts:
            torch.mm(x, wt, out=yd)
    qbytes = 3072 * 3072 * 2 + 3072 * 3072 // 2 + 3072 * 48 * 4
    n = len(ws)
    t_q = graph_ms(torch, quant, inner=1, reps=10) / n
    t_r = stream_reference(torch, ws, 4, 10) / n
    t_d = graph_ms(torch, deq, inner=1, reps=10) / n
    t_m = graph_ms(torch, mm, inner=1, reps=10) / n
    t_dense = graph_ms(torch, dense, inner=1, reps=10) / n
    torch.cuda.synchronize()
    dense_ok = bool(torch.equal(yd, torch.mm(x, wts[-1])))
    del wts
    flop = 2.0 * 256 * 3072 * 3072
    return {"quantize_us": round(t_q * 1e3, 2), "quantize_GBs": round(qbytes / (t_q * 1e-3) / 1e9, 1),
            "quantize_stream_reference_us": round(t_r * 1e3, 2),
            "dequantize_us": round(t_d * 1e3, 2), "dequantize_GBs": round(qbytes / (t_d * 1e-3) / 1e9, 1),
            "qmm_us": round(t_m * 1e3, 2), "qmm_TFLOPs": round(flop / (t_m * 1e-3) / 1e12, 1),
            "dense_bf16_reference_us": round(t_dense * 1e3, 2),
            "dense_bf16_reference_TFLOPs": round(flop / (t_dense * 1e-3) / 1e12, 1),
            "dense_bf16_reference_graph_matches_eager": dense_ok,
            "note": f"per launch, rotated over {CONFIG1_COPIES} distinct weights (HIP graph, gaps "
                    "included); 24.2 MB per quantize/dequantize: latency-bound at this size"}


def bench_config3(mlxq, torch):
    """Config 3: Wan2.2 self-attention projections, x[32760,5120] bf16 . 4 x Q8-g64 W[5120,5120],
    including the quantize pass over all four weights."""
    dev = torch.device("cuda:0")
    M, D = 32760, 5120
    x = gen_bf16((M, D), 1.0, 400, dev)
    ws = [gen_bf16((D, D), 0.02, 401 + i, dev) for i in range(4)]
    qs = [mlxq.quantize(w, 64, 8) for w in ws]
    ys = [torch.empty((M, D), dtype=torch.bfloat16, device=dev) for _ in range(4)]
    # The quantize pass is timed over QUANT_SETS weight sets (the four weights plus copies) so the
    # Infinity Cache cannot hold a pass's data, each weight into its own outputs.
    wq_all = ws + [gen_bf16((D, D), 0.02, 451 + i, dev) for i in range(4 * (QUANT_SETS - 1))]
    qouts = [tuple(torch.empty_like(t) for t in qs[0]) for _ in wq_all]
    from mlxq import _lib
    import ctypes
    lib = _lib.load()

    def proj():
        for q, y in zip(qs, ys):
            mlxq.quantized_matmul(x, *q, True, 64, 8, out=y)

    def quant():
        sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for w, (wq, sc, bi) in zip(wq_all, qouts):
            _lib.check(lib.mlxq_quantize(w.data_ptr(), 1, D, D, 64, 8, wq.data_ptr(), sc.data_ptr(),
                                         bi.data_ptr(), sp))
    t_p = graph_ms(torch, proj, inner=2, reps=3)
    t_q = graph_ms(torch, quant, inner=1, reps=5) / QUANT_SETS
    flop = 4 * 2.0 * M * D * D
    qbytes = 4 * (D * D * 2 + D * D + D * (D // 64) * 4)
    return {"qmm_ms": round(t_p, 3), "qmm_TFLOPs": round(flop / (t_p * 1e-3) / 1e12, 1),
            "qmm_frac_of_mfma_peak": round(flop / (t_p * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "quantize_ms": round(t_q, 4), "quantize_GBs": round(qbytes / (t_q * 1e-3) / 1e9, 1),
            "quantize_frac_of_hbm_peak": round(qbytes / (t_q * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "total_ms": round(t_p + t_q, 3)}


def bench_config5(mlxq, torch):
    """Config 5: FLUX.1-dev double-stream block linear sweep at 4608 tokens, {Q4,Q8} x group
    {32,64,128}, each with a bf16 rank-16 LoRA residual (A, B ~ N(0, 0.01)) fused in the epilogue."""
    dev = torch.device("cuda:0")
    M = 4608
    shapes = [(9216, 3072), (3072, 3072), (12288, 3072), (3072, 12288), (18432, 3072)]
    xs = {K: gen_bf16((M, K), 1.0, 500 + K, dev) for K in (3072, 12288)}
    cells, total_flop, total_ms = {}, 0.0, 0.0
    for bits in (4, 8):
        for gs in (32, 64, 128):
            for (N, K) in shapes:
                q = mlxq.quantize(gen_bf16((N, K), 0.02, 600 + N + K, dev), gs, bits)
                a = gen_bf16((K, 16), 0.01, 700 + K, dev)
                b = gen_bf16((16, N), 0.01, 701 + N, dev)
                ws = torch.empty(mlxq.linear_workspace_size(torch.bfloat16, torch.bfloat16, M, N, lora_a=a),
                                 dtype=torch.uint8, device=dev)
                ms = graph_ms(torch, lambda: mlxq.linear(xs[K], *q, gs, bits, lora_a=a, lora_b=b,
                                                         workspace=ws), inner=4, reps=3)
                flop = 2.0 * M * K * N + 2.0 * M * 16 * (K + N)
                cells[f"Q{bits}g{gs} {N}x{K}"] = round(flop / (ms * 1e-3) / 1e12, 1)
                total_flop += flop
                total_ms += ms
                del q
    return {"sweep_TFLOPs": round(total_flop / (total_ms * 1e-3) / 1e12, 1),
            "sweep_ms": round(total_ms, 3), "cells_TFLOPs": cells}


def bench_experts(mlxq, torch, n=512):
    """Stacked-expert MoE projections of the Lens gpt-oss text encoder (mlx-gen-lens/src/config.rs:
    hidden 2880, intermediate 2880, 32 experts; Q4 g64 packs with dense bias) at n = 512 tokens:
    gate_up [32, 5760, 2880] on the shared x, down [32, 2880, 2880] on per-expert inputs.  One
    qmm_experts launch per projection against the reference's call pattern, one quantized linear
    (qmm + bias) per expert (mlx-gen-lens/src/text_encoder/gpt_oss.rs:700-720)."""
    dev = torch.device("cuda:0")
    E, H, I = 32, 2880, 2880
    gu = [t.reshape(E, 2 * I, -1) for t in mlxq.quantize(gen_bf16((E * 2 * I, H), 0.02, 800, dev), 64, 4)]
    dn = [t.reshape(E, H, -1) for t in mlxq.quantize(gen_bf16((E * H, I), 0.02, 801, dev), 64, 4)]
    gu_bias = gen_bf16((E, 2 * I), 0.5, 802, dev)
    dn_bias = gen_bf16((E, H), 0.5, 803, dev)
    x = gen_bf16((n, H), 1.0, 804, dev)
    xe = gen_bf16((E, n, I), 1.0, 805, dev)
    y1 = torch.empty((E, n, 2 * I), dtype=torch.bfloat16, device=dev)
    y2 = torch.empty((E, n, H), dtype=torch.bfloat16, device=dev)

    def stacked():
        mlxq.qmm_experts(x, *gu, 64, 4, bias=gu_bias, out=y1)
        mlxq.qmm_experts(xe, *dn, 64, 4, bias=dn_bias, per_expert=True, out=y2)

    def per_expert():
        for e in range(E):
            mlxq.linear(x, gu[0][e], gu[1][e], gu[2][e], 64, 4, bias=gu_bias[e])
            mlxq.linear(xe[e], dn[0][e], dn[1][e], dn[2][e], 64, 4, bias=dn_bias[e])

    flop = 2.0 * n * H * 2 * I * E + 2.0 * n * I * H * E
    ms_one = graph_ms(torch, stacked, inner=2, reps=3)
    ms_loop = graph_ms(torch, per_expert, inner=1, reps=3)
    return {"tokens": n, "experts": E, "gflop": round(flop / 1e9, 1),
            "one_launch_ms": round(ms_one, 3), "one_launch_TFLOPs": round(flop / (ms_one * 1e-3) / 1e12, 1),
            "per_expert_ms": round(ms_loop, 3),
            "per_expert_TFLOPs": round(flop / (ms_loop * 1e-3) / 1e12, 1)}


def cpu_baseline(budget_s):
    """The CPU oracle on a bounded row sample of the config-2 up projection."""
    import numpy as np
    from oracle import oracle
    rng = np.random.default_rng(0)
    K, F = 3072, 12288
    w = oracle.bf16_round((rng.standard_normal((F, K)) * 0.02).astype(np.float32))
    wq, s, b = oracle.quantize(w, 64, 4, sb_bf16=True)
    rows = 8
    while True:
        x = oracle.bf16_round(rng.standard_normal((rows, K)).astype(np.float32))
        t0 = time.perf_counter()
        oracle.quantized_matmul(x, wq, s, b, 64, 4, w_bf16=True, out_bf16=True)
        dt = time.perf_counter() - t0
        if dt >= budget_s / 3 or rows >= 4608:
            break
        rows = min(4608, max(rows * 2, int(rows * budget_s / 3 / max(dt, 1e-3))))
    flop = 2.0 * rows * K * F
    res = {"value": flop / dt / 1e12, "unit": "TFLOP/s", "cores": oracle.num_threads(),
           "kind": "port",
           "sample": f"x[{rows},3072] . Q4-g64 W_up[12288,3072]^T (the config-2 up projection "
                     f"restricted to {rows} of 4608 rows), fp64-accumulating C oracle with OpenMP, "
                     f"{dt:.1f} s"}
    # Beside it, an optimised CPU library path on the same sample: the weights dequantized once
    # (untimed) and the product by torch's CPU f32 GEMM over all host threads.
    import torch
    wd = torch.from_numpy(oracle.dequantize(wq, s, b, 64, 4, out_bf16=True))
    xt = torch.from_numpy(x)
    torch.mm(xt[:8], wd.t())
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s / 6 or reps < 2:
        torch.mm(xt, wd.t())
        reps += 1
    dt_mm = (time.perf_counter() - t0) / reps
    res["cpu_library_gemm"] = {"value": round(flop / dt_mm / 1e12, 4), "unit": "TFLOP/s",
                               "threads": torch.get_num_threads(),
                               "note": "torch CPU f32 GEMM (x . dequant(W)^T, weights dequantized "
                                       "beforehand, untimed) on the same sample: an optimised CPU "
                                       "library figure, not the reference's MLX CPU path"}
    return res


COPY_BYTES = 1 << 30  # plain-copy calibration: 1 GiB read + 1 GiB written per launch
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "qmm_wide_flux_mlp_counters.txt")


def run_copy(torch, reps=5):
    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "reps": reps}))


def _pmc_table(d):
    """{kernel name: {counter: [per-dispatch values]}} from the rocprofv3 --pmc csv files under d."""
    import csv
    import glob
    out = {}
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            k = r["Kernel_Name"].replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
            out.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return out


def _med(v):
    v = sorted(v)
    return v[len(v) // 2]


SIMDS = 256 * 4  # MI355X: 256 CUs x 4 SIMDs; GRBM_GUI_ACTIVE is summed over its 8 XCDs


def summarize_pmc(d, sets=None):
    """Summary of the rocprofv3 --pmc runs under d, one subdirectory per counter set:
    <leg>_mfma (SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_BF16),
    <leg>_dram (TCC_EA0_RDREQ_DRAM_32B_sum TCC_EA0_WRREQ_WRITE_DRAM_32B_sum), <leg>_fetch (FETCH_SIZE),
    <leg>_write (WRITE_SIZE), with leg 'copy' the 1 GiB plain-copy calibration.  Per mlxq kernel:
    MFMA busy = busy cycles / (GUI-active cycles per XCD x SIMDs), bf16 MFMA flop = MOPS x 512,
    memory-side read / write bytes = 32-byte requests x 32 scaled by the copy calibration, and
    FETCH_SIZE / WRITE_SIZE (KiB per dispatch) scaled by the same.  Medians over dispatches."""
    import glob
    subs = {os.path.basename(p): _pmc_table(p) for p in sorted(glob.glob(os.path.join(d, "*"))) if os.path.isdir(p)}
    keep = set(sets.split(",")) if sets else None
    copy_ctr = lambda sub, c: max((_med(v[c]) for k, v in subs.get(sub, {}).items() if "copy" in k.lower() and c in v),
                                  default=None)
    cal = {}
    rd, wr = copy_ctr("copy_dram", "TCC_EA0_RDREQ_DRAM_32B_sum"), copy_ctr("copy_dram", "TCC_EA0_WRREQ_WRITE_DRAM_32B_sum")
    cal["rd"] = COPY_BYTES / (rd * 32) if rd else 1.0
    cal["wr"] = COPY_BYTES / (wr * 32) if wr else 1.0
    fe, wi = copy_ctr("copy_fetch", "FETCH_SIZE"), copy_ctr("copy_write", "WRITE_SIZE")
    cal["fetch"] = (COPY_BYTES / 1024.0) / fe if fe else None
    cal["write"] = (COPY_BYTES / 1024.0) / wi if wi else None
    lines = [f"calibration (1 GiB plain copy): DRAM read requests x32 B x{cal['rd']:.4f}, write x{cal['wr']:.4f}; "
             f"FETCH_SIZE x{cal['fetch'] or 0:.4f}, WRITE_SIZE x{cal['write'] or 0:.4f} (expected / counted)"]
    wide = []
    for sub, tab in subs.items():
        if sub.startswith("copy") or (keep is not None and sub not in keep):
            continue
        for k in sorted(tab):
            if "mlxq" not in k:
                continue
            c = tab[k]
            n = len(next(iter(c.values())))
            parts = []
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c and "GRBM_GUI_ACTIVE" in c:
                busy = _med(c["SQ_VALU_MFMA_BUSY_CYCLES"]) / (_med(c["GRBM_GUI_ACTIVE"]) / 8 * SIMDS)
                parts.append(f"MFMA busy {100 * busy:.1f}%")
            if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in c:
                parts.append(f"bf16 MFMA {_med(c['SQ_INSTS_VALU_MFMA_MOPS_BF16']) * 512 / 1e9:.2f} GFLOP")
            if "TCC_EA0_RDREQ_DRAM_32B_sum" in c:
                r = _med(c["TCC_EA0_RDREQ_DRAM_32B_sum"]) * 32 * cal["rd"]
                w = _med(c.get("TCC_EA0_WRREQ_WRITE_DRAM_32B_sum", [0.0])) * 32 * cal["wr"]
                parts.append(f"memory-side read {r / 1e6:.2f} MB write {w / 1e6:.2f} MB")
            if "FETCH_SIZE" in c and cal["fetch"]:
                f = _med(c["FETCH_SIZE"]) * 1024 * cal["fetch"]
                parts.append(f"FETCH_SIZE {f / 1e6:.2f} MB")
                if "qmm_wide" in k:
                    wide.append(("fetch", k, f))
            if "WRITE_SIZE" in c and cal["write"]:
                w = _med(c["WRITE_SIZE"]) * 1024 * cal["write"]
                parts.append(f"WRITE_SIZE {w / 1e6:.2f} MB")
                if "qmm_wide" in k:
                    wide.append(("write", k, w))
            lines.append(f"[{sub}] {k}: " + "; ".join(parts) + f" ({n} dispatches)")
    kernels = sorted({k for _, k, _ in wide})
    if kernels:
        per = [sum(v for t, k2, v in wide if k2 == k) for k in kernels]
        lines.append(f"traffic_bytes_per_launch: {int(sum(per) / len(per))}")
    print("\n".join(lines))


def summarize_trace(d, skip=0, last=0):
    """Per mlxq kernel and launch shape (grid in workgroups x workgroup size) of the rocprofv3
    --kernel-trace csv files under d: launch count and average / median / minimum duration, over
    the launches after each shape's first `skip` (in start-time order), or its last `last`."""
    import csv
    import glob
    shapes = {}
    for f in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            name = r["Kernel_Name"].replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
            if "mlxq" not in name:
                continue
            wg = int(r["Workgroup_Size_X"]) * int(r.get("Workgroup_Size_Y", 1) or 1)
            grid = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
            gy = int(r.get("Grid_Size_Y", 1) or 1) // max(1, int(r.get("Workgroup_Size_Y", 1) or 1))
            key = (name, grid if gy <= 1 else f"{grid} x {gy}", wg)
            shapes.setdefault(key, []).append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    lines = []
    durs = {}
    for key, ts in shapes.items():
        ts.sort()
        kept = ts[skip:] if len(ts) > skip else ts
        if last > 0:
            kept = kept[-last:]
        durs[key] = [(e - b) / 1e3 for b, e in kept]
    for (name, grid, wg), v in sorted(durs.items(), key=lambda kv: -sum(kv[1]) / len(kv[1])):
        lines.append(f"  {name}  grid {grid} x {wg}: launches {len(v)}  avg {sum(v) / len(v):.2f} us  "
                     f"median {_med(v):.2f} us  min {min(v):.2f}")
    print("\n".join(lines))


def read_traffic():
    """HBM bytes per qmm launch from the committed rocprofv3 --pmc summary, or None."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.trace_skip, args.trace_last)
        return
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc, args.pmc_sets)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the quantized-linear "
              "path is single-device by design, so multi-GPU runs are not supported.", file=sys.stderr)
        sys.exit(2)
    import torch
    import mlxq
    mlxq.load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    if args.only == "copy":
        run_copy(torch)
        return
    if args.only == "gemv":
        print(json.dumps({"gemv": bench_gemv(mlxq, torch)}))
        return
    if args.only == "gemv_long":
        print(json.dumps({"gemv_long": bench_gemv_long(mlxq, torch)}))
        return
    if args.only == "quantize":
        print(json.dumps({"quantize": bench_quantize(mlxq, torch)}))
        return
    if args.only == "experts":
        print(json.dumps({"experts": bench_experts(mlxq, torch)}))
        return
    if args.only == "f32":
        print(json.dumps({"f32_mlp": bench_f32_mlp(mlxq, torch)}))
        return
    if args.only == "dense":
        print(json.dumps({"dense_bf16_reference": bench_dense_reference(torch)}))
        return
    if args.only == "configs":
        print(json.dumps({"config1": bench_config1(mlxq, torch), "config3": bench_config3(mlxq, torch),
                          "config5": bench_config5(mlxq, torch)}))
        return
    g = bench_flux_mlp(mlxq, torch, args.steps, args.warmup, args.prerun_seconds)
    achieved = g["qmm_flop_per_launch"] / (g["qmm_launch_ms"] * 1e-3) / 1e12
    res = {
        "metric": METRIC,
        "value": round(g["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 4),
        "timing": {"statistic": "median of the per-step HIP-event times (value and ms_per_step)",
                   "mean_ms_per_step": round(g["mean_ms_per_step"], 4),
                   "span_ms_per_step": round(g["span_ms_per_step"], 4),
                   "first_ms": g["step_ms"][0], "last_ms": g["step_ms"][-1],
                   "step_ms": g["step_ms"],
                   "prerun": dict(g["prerun"], note="untimed: the same up+down launches back to back "
                                  "before the warm-up steps, so the timed steps run at the settled clock")},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch N(0,1) activations, N(0,0.02) weights quantized on device)",
        "config": {"workload": "config 2: FLUX.1-dev double-stream MLP at 1024^2, x[4608,3072] bf16, "
                               "Q4-g64 W_up[12288,3072] + exact-erf GELU + Q4-g64 W_down[3072,12288]",
                   "M": 4608, "K": 3072, "F": 12288, "bits": 4, "group_size": 64,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": read_traffic(),
                     "traffic_source": "from profiles/qmm_wide_flux_mlp_counters.txt (rocprofv3 --pmc "
                                       "FETCH_SIZE + WRITE_SIZE per launch, copy-calibrated), not "
                                       "measured in this run",
                     "kernel": "qmm_wide_kernel (up: fused GELU epilogue, down: plain)",
                     "launch_ms": {"up": round(g["up_ms"], 4), "down": round(g["down_ms"], 4),
                                   "statistic": "median over the timed steps",
                                   "mean_up": round(g["mean_up_ms"], 4),
                                   "mean_down": round(g["mean_down_ms"], 4)}},
    }
    if not args.no_extras and args.only == "all":
        res["gemv"] = bench_gemv(mlxq, torch)
        res["quantize"] = bench_quantize(mlxq, torch)
        res["config1"] = bench_config1(mlxq, torch)
        res["config3"] = bench_config3(mlxq, torch)
        res["config5"] = bench_config5(mlxq, torch)
        res["experts"] = bench_experts(mlxq, torch)
        res["f32_mlp"] = bench_f32_mlp(mlxq, torch)
        res["dense_bf16_reference"] = bench_dense_reference(torch)
    if not args.no_cpu and args.only == "all":
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
