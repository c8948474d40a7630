"""Pins the CPU oracle (oracle/mlxq_oracle.c) before anything is compared against it.

Each check is chosen so a plausible slip in the oracle (a dropped term, the simplified
``scale=(max-min)/15, bias=min`` scheme, high-bits-first packing, a mul-then-add dequant, a
transposed operand) fails at least one of them:

* the reference's golden fixture (tests/golden/quant_q4q8.safetensors, from the reference's
  tools/dump_quant.py and tests/quant_parity.rs:30-66) — bit-exact packing, scales, biases and
  dequant, and the fixture's quantized_matmul;
* closed forms (all-zero and constant groups, a hand-computed packed word);
* invariants the reference relies on (row-split commutation, mlx-gen-sdxl/src/quant.rs:89-110;
  the quantization-error envelope of tests/quant_parity.rs:99-127);
* library routines for what is textbook (numpy float64 matmul, torch bf16 rounding, math.erf).
"""
import math
import os

import numpy as np
import pytest
import torch
from safetensors.numpy import load_file

from oracle import oracle

GOLD = load_file(os.path.join(os.path.dirname(__file__), "golden", "quant_q4q8.safetensors"))
GS = 64


@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_matches_golden_bit_exact(bits):
    wq, s, b = oracle.quantize(GOLD["w"], GS, bits)
    assert np.array_equal(wq, GOLD[f"q{bits}.wq"]), "packed words diverge from MLX 0.31"
    assert np.array_equal(s, GOLD[f"q{bits}.scales"])
    assert np.array_equal(b, GOLD[f"q{bits}.biases"])
    # The edge-exact scheme yields negative scales for about half of the N(0,1) groups.
    assert 0.3 < (s < 0).mean() < 0.7


@pytest.mark.parametrize("bits", [8, 4])
def test_simplified_scheme_is_rejected_by_golden(bits):
    """The (max-min)/nb, bias=min scheme would fail the same bit-exact check."""
    w = GOLD["w"].reshape(128, -1, GS)
    nb = np.float32(2 ** bits - 1)
    mn, mx = w.min(-1), w.max(-1)
    s = ((mx - mn) / nb).astype(np.float32)
    assert not np.array_equal(s, GOLD[f"q{bits}.scales"])


@pytest.mark.parametrize("bits", [8, 4])
def test_dequantize_matches_golden_bit_exact(bits):
    deq = oracle.dequantize(GOLD[f"q{bits}.wq"], GOLD[f"q{bits}.scales"], GOLD[f"q{bits}.biases"],
                            GS, bits)
    assert np.array_equal(deq, GOLD[f"q{bits}.deq"])
    # A mul-then-add dequant (two roundings) is distinguishable by the same golden.
    codes = _codes(GOLD[f"q{bits}.wq"], bits).reshape(128, -1, GS).astype(np.float32)
    two_round = (codes * GOLD[f"q{bits}.scales"][..., None]).astype(np.float32) + \
        GOLD[f"q{bits}.biases"][..., None]
    assert not np.array_equal(two_round.reshape(128, 256), GOLD[f"q{bits}.deq"])


@pytest.mark.parametrize("bits", [8, 4])
def test_qmm_matches_golden(bits):
    y = oracle.quantized_matmul(GOLD["x"], GOLD[f"q{bits}.wq"], GOLD[f"q{bits}.scales"],
                                GOLD[f"q{bits}.biases"], GS, bits, w_bf16=False, out_bf16=False)
    ref = GOLD[f"q{bits}.qmm"]
    # tests/quant_parity.rs:60-64 allows 1e-2; the f32 restatement is far inside that.
    assert np.abs(y - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    # A transposed weight operand is caught.
    wrong = GOLD["x"] @ GOLD[f"q{bits}.deq"][:, ::-1].T
    assert np.abs(wrong - ref).max() > 1e-1


def _codes(wq, bits):
    per = 32 // bits
    sh = (np.arange(per, dtype=np.uint32) * bits)
    return ((wq[..., None] >> sh) & ((1 << bits) - 1)).reshape(wq.shape[0], -1)


def test_low_bits_first_hand_computed_word():
    # One Q8 group holding 0..63: mx=63 wins the edge (|0| > |63| is false) so the scale is
    # negative and code(k) = round((k-63) / (63/-255)) = round((63-k)*255/63).
    w = np.arange(64, dtype=np.float32)[None, :]
    wq, s, b = oracle.quantize(w, 64, 8)
    assert b[0, 0] == 63.0 and s[0, 0] < 0
    word0 = int(wq[0, 0])
    assert word0 & 0xFF == 255            # element 0 in the lowest byte
    assert (word0 >> 24) & 0xFF == round(60 * 255 / 63)
    # Q4 of 0..15 * 2 (range 30, nb 15 -> scale -2, edge 30): code(k) = 15 - k.
    w4 = np.tile(np.arange(16, dtype=np.float32) * 2, 4)[None, :]
    wq4, s4, b4 = oracle.quantize(w4, 64, 4)
    assert s4[0, 0] == -2.0 and b4[0, 0] == 30.0
    assert int(wq4[0, 0]) == 0x89ABCDEF     # codes 15,14,...,8 from low nibble up


@pytest.mark.parametrize("bits", [4, 8])
def test_zero_and_constant_groups(bits):
    w = np.zeros((3, 128), np.float32)
    w[1, :64] = 0.75          # constant group
    w[2, 64:] = -1.5          # constant negative group
    wq, s, b = oracle.quantize(w, 64, bits)
    assert np.all(wq == 0)
    assert s[0, 0] == np.float32(-1e-7) and b[0, 0] == 0.0
    assert b[1, 0] == 0.75 and b[2, 1] == -1.5
    deq = oracle.dequantize(wq, s, b, 64, bits)
    assert np.array_equal(deq, w)


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (8, 128)])
def test_row_split_commutes(bits, gs):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((48, 256)) * 0.02).astype(np.float32)
    full = oracle.quantize(w, gs, bits)
    top = oracle.quantize(w[:20], gs, bits)
    bot = oracle.quantize(w[20:], gs, bits)
    for f, t, bt in zip(full, top, bot):
        assert np.array_equal(f, np.concatenate([t, bt]))


@pytest.mark.parametrize("bits,max_rel", [(8, 0.02), (4, 0.12)])
def test_quantization_error_envelope(bits, max_rel):
    """tests/quant_parity.rs:99-127: bf16-cast quantize then qmm stays near the dense output."""
    w, x = GOLD["w"], GOLD["x"]
    dense = x.astype(np.float64) @ w.astype(np.float64).T
    wq, s, b = oracle.quantize(oracle.bf16_round(w), GS, bits, sb_bf16=True)
    y = oracle.quantized_matmul(x, wq, s, b, GS, bits, w_bf16=False, out_bf16=False)
    rel = np.abs(y - dense).max() / np.abs(dense).max()
    assert rel < max_rel


@pytest.mark.parametrize("w_bf16", [False, True])
def test_qmm_against_numpy_matmul(w_bf16):
    rng = np.random.default_rng(2)
    x = oracle.bf16_round(rng.standard_normal((5, 192)).astype(np.float32))
    w = oracle.bf16_round((rng.standard_normal((24, 192)) * 0.02).astype(np.float32))
    wq, s, b = oracle.quantize(w, 64, 4, sb_bf16=True)
    deq = oracle.dequantize(wq, s, b, 64, 4, out_bf16=w_bf16)
    ref = oracle.bf16_round((x.astype(np.float64) @ deq.astype(np.float64).T).astype(np.float32))
    y = oracle.quantized_matmul(x, wq, s, b, 64, 4, w_bf16=w_bf16, out_bf16=True)
    assert np.array_equal(y, ref)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-6, 6, 10000),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.0e38, np.inf, -np.inf], np.float32)])
    v = v.astype(np.float32)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(oracle.bf16_round(v), ref)
    assert all(oracle.lib().oracle_bf16_round(float(a)) == r for a, r in zip(v[:200], ref[:200]))


def test_gelu_and_silu_closed_forms():
    for v in (-3.0, -0.5, 0.0, 0.25, 1.0, 4.0):
        want = 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))
        assert oracle.gelu_erf(v, out_bf16=False) == pytest.approx(want, rel=1e-6, abs=1e-12)
        assert oracle.silu(v, out_bf16=False) == pytest.approx(v / (1 + math.exp(-v)), rel=1e-6,
                                                               abs=1e-12)
    assert oracle.gelu_erf(0.0) == 0.0 and oracle.gelu_erf(30.0) == 30.0


def test_gelu_tanh_closed_form_and_exact_gelu():
    """Tanh GELU (reference src/nn.rs:321-329).  In f32 it is the closed form, at the reference's
    own test points (src/nn.rs:722-738) and on a sweep; with bf16 rounding per op it stays within
    bf16 rounding of the closed form and within the approximation's known distance (< 1e-3
    absolute) of the exact-erf GELU; tanh saturation gives x for large x and 0 for large -x."""
    c = math.sqrt(2.0 / math.pi)

    def closed(v):
        return 0.5 * v * (1.0 + math.tanh(c * (v + 0.044715 * v ** 3)))

    pts = [-2.0, -0.5, 0.0, 0.5, 1.0, 3.0] + [float(np.float32(t)) for t in np.linspace(-6, 6, 97)]
    for v in pts:
        assert oracle.gelu_tanh(v, out_bf16=False) == pytest.approx(closed(v), rel=2e-6, abs=1e-7)
    for v in oracle.bf16_round(np.linspace(-6, 6, 241).astype(np.float32)):
        g = oracle.gelu_tanh(float(v))
        assert g == oracle.bf16_round(np.float32(g))
        assert abs(g - closed(float(v))) <= 0.016 * abs(float(v)) + 1e-3
        assert abs(g - oracle.gelu_erf(float(v))) <= 0.016 * abs(float(v)) + 2e-3
    assert oracle.gelu_tanh(0.0) == 0.0
    assert oracle.gelu_tanh(8.0) == 8.0 and oracle.gelu_tanh(-8.0) == 0.0


def _torch_gelu_exact(v):
    """src/nn.rs:344-355 in torch ops (each op in v's dtype, constants cast to it)."""
    import torch
    s2 = torch.tensor(math.sqrt(2.0), dtype=torch.float32).to(v.dtype)
    inner = torch.erf(v / s2)
    gate = torch.tensor(1.0, dtype=v.dtype) + inner
    return (v * gate) / torch.tensor(2.0, dtype=v.dtype)


def _torch_gelu_tanh(v):
    """src/nn.rs:321-329 in torch ops (each op in v's dtype, constants cast to it)."""
    import torch
    c = torch.tensor(math.sqrt(2.0 / math.pi), dtype=torch.float32).to(v.dtype)
    k = torch.tensor(0.044715, dtype=torch.float32).to(v.dtype)
    x3 = (v.float() ** 3).to(v.dtype)  # MLX's power: one float pow, rounded once (torch's bf16
    #                                     pow multiplies and rounds step by step)
    inner = (v + x3 * k) * c
    gate = torch.tanh(inner) + torch.tensor(1.0, dtype=v.dtype)
    return (v * torch.tensor(0.5, dtype=v.dtype)) * gate


def _all_bf16_values():
    bits = np.arange(65536, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    return v[np.isfinite(v)]


@pytest.mark.parametrize("which", ["exact", "tanh"])
def test_bf16_gelu_every_input_against_torch_ops(which):
    """The oracle's per-op bf16 GELUs on every finite bf16 input against the same op sequence run
    as torch bf16 tensor ops (an independent implementation of per-op bf16 rounding and of erf/
    tanh).  A dropped op, a wrong constant or a wrong rounding point moves thousands of entries;
    torch's own f32 erf/tanh are within an ulp, which can move a rare entry by one bf16 ulp."""
    import torch
    v = _all_bf16_values()
    f = oracle.gelu_exact if which == "exact" else oracle.gelu_tanh
    got = np.array([f(float(t)) for t in v], dtype=np.float32)
    tf = _torch_gelu_exact if which == "exact" else _torch_gelu_tanh
    want = tf(torch.from_numpy(v).to(torch.bfloat16)).float().numpy()
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same)
    ulps = np.abs(got[bad].view(np.int32) - want[bad].view(np.int32)) >> 16
    print(f"{which}: {bad.size} of {v.size} inputs differ from torch's ops, max {ulps.max() if bad.size else 0} ulp")
    assert bad.size <= 16 and (bad.size == 0 or ulps.max() <= 1)


def test_gelu_exact_f32_is_the_closed_form():
    # Per op in f32, 1 + erf(v/sqrt2) is computed to within an f32 ulp of 1, so the result is within
    # |v| * 2^-23 (plus the other ops' relative rounding) of the closed form.
    for v in (-5.0, -1.0, -0.25, 0.0, 0.3, 2.0, 7.0):
        want = 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))
        got = oracle.gelu_exact(v, out_bf16=False)
        assert abs(got - want) <= abs(v) * 2.0 ** -23 + abs(want) * 4e-7
    # per-op bf16: 1 + erf rounds to 0 for large negative inputs, so the result is -0
    assert oracle.gelu_exact(-4.0) == 0.0 and oracle.gelu_exact(4.0) == 4.0


@pytest.mark.parametrize("bias_dt,lora_dt,act", [
    ("bf16", "bf16", 0), ("bf16", "bf16", 1), ("bf16", "bf16", 2), ("bf16", "bf16", 3),
    ("f32", "bf16", 0), ("bf16", "f32", 0), ("f32", "f32", 2), ("bf16", "f32", 3), (None, "f32", 1),
])
def test_linear_sequence_matches_torch_promotion(bias_dt, lora_dt, act):
    """oracle.linear against the reference's op sequence (src/adapters.rs:309-320, :260-270,
    :543-549) written as torch tensor ops on operands of the stated dtypes: torch promotes bf16 and
    f32 exactly as MLX does (bf16 only when both operands are bf16) and rounds per op, so this
    checks the oracle's promotion and rounding points by an independent route.  Matmuls are done
    in float64 and rounded to their result dtype on both sides."""
    import torch
    rng = np.random.default_rng(4 + act)
    M, K, N, r = 6, 128, 40, 16
    bf, f32 = torch.bfloat16, torch.float32
    tdt = {"bf16": bf, "f32": f32}
    x = oracle.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    w = oracle.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    bias = rng.standard_normal(N).astype(np.float32)
    A = (rng.standard_normal((K, r)) * 0.05).astype(np.float32)
    B = (rng.standard_normal((r, N)) * 0.05).astype(np.float32)
    if bias_dt == "bf16":
        bias = oracle.bf16_round(bias)
    if lora_dt == "bf16":
        A, B = oracle.bf16_round(A), oracle.bf16_round(B)
    wq, s, b = oracle.quantize(w, 64, 4, sb_bf16=True)
    y, out_bf16 = oracle.linear(x, wq, s, b, 64, 4, bias=None if bias_dt is None else bias,
                                lora_a=A, lora_b=B, lora_scale=0.75, act=act, x_bf16=True,
                                sb_bf16=True, bias_bf16=bias_dt == "bf16", lora_bf16=lora_dt == "bf16",
                                return_dtype=True)
    # torch restatement
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    y0 = t(oracle.quantized_matmul(x, wq, s, b, 64, 4, out_bf16=False), f32).to(bf)
    out = y0 + t(bias, tdt[bias_dt]) if bias_dt else y0
    dr = bf if lora_dt == "bf16" else f32
    xa = t(x.astype(np.float64) @ A.astype(np.float64), f32).to(dr)
    rr = t(xa.double().numpy() @ B.astype(np.float64), f32).to(dr)
    out = out + rr * torch.tensor(0.75, dtype=f32).to(dr)
    if act == 1:
        out = t(0.5 * out.double().numpy() * (1.0 + np.vectorize(math.erf)(out.double().numpy() /
                                                                          math.sqrt(2.0))), f32)
    elif act == 2:
        out = _torch_gelu_tanh(out)
    elif act == 3:
        out = _torch_gelu_exact(out)
    assert out_bf16 == (out.dtype == bf)
    want = out.float().numpy()
    if act in (0, 1):
        tol = 0.0 if act == 0 else 1e-6
        np.testing.assert_allclose(y, want, rtol=tol, atol=0)
    elif out_bf16:  # bf16: every input agrees with torch's ops (test above)
        np.testing.assert_array_equal(y, want)
    else:  # f32: torch's float erf / tanh are within a few ulps of the oracle's double ones
        diff = np.abs(y.view(np.int32) - want.view(np.int32))
        assert (diff <= 8).all()


def test_invalid_shapes_rejected():
    with pytest.raises(ValueError):
        oracle.quantize(np.zeros((2, 100), np.float32), 64, 4)
    with pytest.raises(ValueError):
        oracle.quantize(np.zeros((2, 128), np.float32), 64, 3)


def test_stack_split_commutes_with_packing():
    """Affine quantization is per row, so packing a stacked expert weight [E*out, in] equals
    packing each expert and stacking (the property mlx-gen-lens/src/quant.rs:85-92 relies on to
    split a stacked on-disk pack back into per-expert packs)."""
    rng = np.random.default_rng(12)
    E, N, K = 3, 20, 256
    w = oracle.bf16_round((rng.standard_normal((E, N, K)) * 0.02).astype(np.float32))
    for bits in (4, 8):
        stacked = oracle.quantize(w.reshape(E * N, K), 64, bits, sb_bf16=True)
        for e in range(E):
            per = oracle.quantize(w[e], 64, bits, sb_bf16=True)
            for a, b in zip(stacked, per):
                assert np.array_equal(a[e * N:(e + 1) * N], b)


def _lokr_2x2():
    """The reference's lokr_2x2 fixture (src/adapters.rs:695-708): reconstruct_lokr_delta(alpha 8,
    rank 4, [2, 2], w1 = [[0.5], [0.6]], w2 = [[0.7, 0.8]], bf16) = bf16(2 * kron(w1, w2)), the
    kron and the scale taken in f32 (src/adapters.rs:117-119)."""
    w1 = np.array([[0.5], [0.6]], np.float32)
    w2 = np.array([[0.7, 0.8]], np.float32)
    return oracle.bf16_round((np.kron(w1, w2).astype(np.float32) * np.float32(8.0 / 4.0)).reshape(2, 2))


def test_lokr_delta_fixture_hand_values():
    """2 * [[0.35, 0.4], [0.42, 0.48]] rounded to 8 significant bits: 0.7 = 1.0110011|0011.. x 2^-1
    rounds down to 0.69921875, 0.8 = 1.1001100|1100.. up to 0.80078125, 0.84 = 1.1010111|0000.. down
    to 0.83984375, 0.96 = 1.1110101|1100.. up to 0.9609375."""
    np.testing.assert_array_equal(_lokr_2x2(), np.array([[0.69921875, 0.80078125],
                                                          [0.83984375, 0.9609375]], np.float32))


def test_lokr_residual_reference_known_answers():
    """The reference's LoKr tests on the oracle (src/adapters.rs:711-764): a bf16-input residual of
    the 2x2 delta at scale 0.5 stays bf16 and is within 5e-2 of the f32 one; the products are exact
    here, so the hand-computed values hold bit for bit; scale 0 is a bit-exact no-op."""
    delta = _lokr_2x2()
    x32 = np.array([[1.0, -2.0], [0.5, 0.25], [-1.0, 2.0]], np.float32)
    zero = np.zeros((3, 2), np.float32)
    got, out_bf16 = oracle.lokr_residual(x32, zero, delta, 0.5, x_bf16=True, y_bf16=True,
                                         return_dtype=True)
    assert out_bf16
    want = (x32.astype(np.float64) @ delta.astype(np.float64).T * 0.5).astype(np.float32)
    np.testing.assert_allclose(got, oracle.bf16_round(want), rtol=5e-2, atol=5e-2)
    # row 0: r = (0.69921875 - 1.6015625, 0.83984375 - 1.921875) = (-0.90234375, -1.08203125); the
    # second needs 9 significant bits (1.0001010|1) and ties to even at -1.078125; times 0.5:
    np.testing.assert_array_equal(got[0], np.array([-0.451171875, -0.5390625], np.float32))
    y = oracle.bf16_round(np.array([[0.1, 0.2], [0.3, 0.4], [1.5, -7.0]], np.float32))
    np.testing.assert_array_equal(oracle.lokr_residual(x32, y, delta, 0.0), y)
    np.testing.assert_array_equal(oracle.lokr_residual(x32, y, delta, 0.0, x_bf16=False, y_bf16=False), y)


@pytest.mark.parametrize("x_dt,y_dt,delta_dt", [("bf16", "bf16", "bf16"), ("f32", "f32", "bf16"),
                                                ("bf16", "f32", "bf16"), ("f32", "bf16", "f32"),
                                                ("bf16", "bf16", "f32")])
def test_lokr_residual_matches_torch_promotion(x_dt, y_dt, delta_dt):
    """oracle.lokr_residual against Adapter::residual's Lokr arm and the sum of
    AdaptableLinear::forward (src/adapters.rs:263-269, :545-547) as torch ops on operands of the
    stated dtypes: delta.to(x.dtype), matmul (float64, rounded to x's dtype), times the scale cast to
    x's dtype, then y + r with torch's (= MLX's) promotion.  Bit-exact."""
    import torch
    rng = np.random.default_rng(len(x_dt + y_dt + delta_dt))
    M, K, N = 5, 64, 24
    bf, f32 = torch.bfloat16, torch.float32
    tdt = {"bf16": bf, "f32": f32}
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = rng.standard_normal((M, N)).astype(np.float32)
    delta = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = oracle.bf16_round(x) if x_dt == "bf16" else x
    y = oracle.bf16_round(y) if y_dt == "bf16" else y
    delta = oracle.bf16_round(delta) if delta_dt == "bf16" else delta
    got, out_bf16 = oracle.lokr_residual(x, y, delta, 0.3, x_bf16=x_dt == "bf16", y_bf16=y_dt == "bf16",
                                         return_dtype=True)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    d = t(delta, tdt[delta_dt]).to(tdt[x_dt])
    r = t(x.astype(np.float64) @ d.double().numpy().T, f32).to(tdt[x_dt])
    r = r * torch.tensor(0.3, dtype=f32).to(tdt[x_dt])
    out = t(y, tdt[y_dt]) + r
    assert out_bf16 == (out.dtype == bf)
    np.testing.assert_array_equal(got, out.float().numpy())


def test_bf16_silu_is_sigmoid_then_multiply():
    """The bf16 SiLU of the reference is two ops, multiply(x, sigmoid(x)) (src/nn.rs:301-303): the
    sigmoid is rounded to bf16 before the product.  Checked on every finite bf16 input against
    torch's CPU bf16 ops doing the same two steps (an independent f32 sigmoid); the two may part
    only where torch's f32 sigmoid lands on the other side of a bf16 rounding midpoint.  The
    single-rounded form x / (1 + e^-x) must differ on a visible share of inputs, so a rounding
    point dropped from the oracle would fail here."""
    h = np.arange(65536, dtype=np.uint32)
    h = h[((h >> 7) & 0xFF) != 0xFF]  # finite bf16 bit patterns
    v = (h << 16).view(np.float32)
    got = np.array([oracle.silu(float(a)) for a in v], dtype=np.float32)
    xt = torch.from_numpy(v).to(torch.bfloat16)
    two_op = (xt * torch.sigmoid(xt)).float().numpy()
    with np.errstate(over="ignore"):  # e^-x overflows to inf for large negative x: x / inf = -0
        one_op = torch.from_numpy((v.astype(np.float64) / (1.0 + np.exp(-v.astype(np.float64))))
                                  .astype(np.float32)).to(torch.bfloat16).float().numpy()
    same = (got == two_op) | (np.isnan(got) & np.isnan(two_op))
    assert np.count_nonzero(~same) <= 16, np.count_nonzero(~same)
    assert np.count_nonzero(got != one_op) > 500
    assert oracle.silu(0.0) == 0.0 and oracle.silu(100.0) == 100.0 and oracle.silu(-200.0) == 0.0


def test_fp16_round_matches_numpy():
    """oracle_fp16_round against numpy's float32 -> float16 conversion (round to nearest even):
    random values over the whole fp16 range and beyond, the overflow threshold (65504 stays,
    65520 and up become inf), ties at both the normal and the subnormal step, and specials."""
    rng = np.random.default_rng(5)
    v = (rng.standard_normal(200000) * 10.0 ** rng.uniform(-9, 5.2, 200000)).astype(np.float32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e9, 2.0 ** -24,
                     2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1.0 + 2.0 ** -11,
                     1.0 + 3 * 2.0 ** -11, 2048.0 + 1.0, np.inf, -np.inf, np.nan], np.float32)
    v = np.concatenate([v, edge])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).astype(np.float32)
    got = oracle.fp16_round(v)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all(), v[~same][:10]
    assert np.array_equal(np.signbit(got[v == 0]), np.signbit(v[v == 0]))
