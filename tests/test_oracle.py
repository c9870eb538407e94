"""Pins for the CPU oracle (oracle/q4_oracle.c) - no GPU.

Each function of the oracle is checked against something it did not compute itself:
the reference's committed Q4 fixture (real mx.quantize output), exact rational
arithmetic, closed forms and brute force. See oracle/q4_oracle.h for the map.
"""
from fractions import Fraction
import math

import numpy as np
import pytest

import oracle as O
import st_reader
from hyperion_amd import synthetic as syn


def rne_bf16(value) -> float:
    """Round a finite rational to the nearest bf16 value, ties to even (exact arithmetic)."""
    fr = Fraction(value)
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                      # subnormal spacing below the normal range
    ulp = Fraction(2) ** (e - 7)
    q = round(a / ulp)                    # Fraction.__round__ is half-to-even
    return sign * float(q * ulp)


def bits_of(x: float) -> int:
    return int(np.array([x], np.float32).view(np.uint32)[0] >> 16)


# ---------------------------------------------------------------- bf16 conversion

def test_bf16_rne_matches_exact_rounding():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    f = f[np.isfinite(f) & (np.abs(f) < np.float32(3.3e38))]
    got = O.bf16_from_f32(f)
    for x, g in zip(f[:4000], got[:4000]):
        assert g == bits_of(rne_bf16(float(x))) or (rne_bf16(float(x)) == 0.0 and g in (0, 0x8000))
    # the numpy path used by the benchmark's data generator agrees everywhere
    np.testing.assert_array_equal(got, syn.bf16_bits(f))


def test_bf16_special_values():
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 1.0, -2.5, 3.3895314e38], np.float32)
    got = O.bf16_from_f32(specials)
    assert list(got[:6]) == [0x0000, 0x8000, 0x7F80, 0xFF80, 0x3F80, 0xC020]
    assert got[6] == 0x7F7F                          # largest finite bf16 stays finite
    # exact ties: 1 + 2^-8 sits halfway between 1 and 1 + 2^-7 -> even (1.0)
    tie_lo = np.array([1.0 + 2.0**-8], np.float32)
    tie_hi = np.array([1.0 + 3 * 2.0**-8], np.float32)   # halfway to an even mantissa above
    assert O.bf16_from_f32(tie_lo)[0] == 0x3F80
    assert O.bf16_from_f32(tie_hi)[0] == 0x3F82
    nan = O.bf16_from_f32(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_bf16_matches_torch_if_present():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    f = (rng.standard_normal(50000) * 10.0 ** rng.integers(-30, 30, 50000)).astype(np.float32)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.bf16_from_f32(f), ref)


# ---------------------------------------------------------------- quantize

@pytest.fixture(scope="module")
def fixture_q4(fixture_dir):
    return st_reader.q4_tensors(fixture_dir)


def test_fixture_layout(fixture_q4):
    # 42 Q4 projections, 19,456 groups of 64 (the reference's tiny artifact)
    assert len(fixture_q4) == 42
    assert sum(s.size for _, s, _ in fixture_q4.values()) == 19456
    w, s, b = fixture_q4["language_model.model.layers.0.self_attn.q_proj"]
    assert w.shape == (256, 16) and s.shape == (256, 2) and b.shape == (256, 2)


def test_fixture_zero_point_invariants(fixture_q4):
    """mx.quantize's edge rule: sign(scale) = -sign(bias); code 0 in every group."""
    for name, (w, s, b) in fixture_q4.items():
        sf = syn.bf16_to_f32(s)
        bf = syn.bf16_to_f32(b)
        assert np.all(np.sign(sf) == -np.sign(bf)), name
        codes = syn.unpack_codes(w).reshape(w.shape[0], -1, 64)
        assert np.all((codes == 0).any(-1)), name


@pytest.mark.parametrize("mode", [0, 1])
def test_quantize_reproduces_fixture(fixture_q4, mode):
    """dequantize -> requantize returns MLX's own (codes, scale, bias) bit-exactly on
    every group whose codes reach 15 (16,578 of 19,456 groups)."""
    total = exact = 0
    for name, (w, s, b) in fixture_q4.items():
        wd = O.dequantize(w, s, b, mode=mode)
        w2, s2, b2 = O.quantize(wd)
        codes = syn.unpack_codes(w).reshape(w.shape[0], -1, 64)
        codes2 = syn.unpack_codes(w2).reshape(w.shape[0], -1, 64)
        same = (codes == codes2).all(-1) & (s == s2) & (b == b2)
        has15 = (codes == 15).any(-1)
        total += int(has15.sum())
        exact += int((same & has15).sum())
    assert total == 16578
    assert exact == total


def test_quantize_exact_grid():
    """Values on a 2^-7 grid spanning codes 0..15 with the negative extreme larger."""
    c = np.tile(np.arange(16), 4)
    w = ((c - 8) * 2.0**-7).astype(np.float32)[None, :]
    wq, s, b = O.quantize(syn.bf16_bits(w))
    assert syn.bf16_to_f32(s)[0, 0] == 2.0**-7
    assert syn.bf16_to_f32(b)[0, 0] == -(2.0**-4)
    np.testing.assert_array_equal(syn.unpack_codes(wq)[0], c)


def test_quantize_rounds_half_to_even():
    """(w - b)/s = 2.5 exactly must give code 2 (rint), not 3 (round half away)."""
    c = np.tile(np.arange(16), 4).astype(np.float64)
    c[5] = 2.5
    w = ((c - 8) * 2.0**-7).astype(np.float32)[None, :]
    wq, s, b = O.quantize(syn.bf16_bits(w))
    assert syn.bf16_to_f32(s)[0, 0] == 2.0**-7
    assert syn.unpack_codes(wq)[0, 5] == 2


def test_quantize_positive_extreme_uses_negative_scale():
    """|max| >= |min| puts the edge at the max: scale < 0 and bias = max."""
    vals = np.linspace(-0.05, 0.0625, 64).astype(np.float32)
    vals[-1] = 0.0625
    wq, s, b = O.quantize(syn.bf16_bits(vals[None, :]))
    assert syn.bf16_to_f32(s)[0, 0] < 0
    assert syn.bf16_to_f32(b)[0, 0] == syn.bf16_to_f32(syn.bf16_bits(np.float32(0.0625)))
    assert syn.unpack_codes(wq)[0, -1] == 0          # the edge itself is code 0
    # a tie |min| == |max| also takes the max as the edge
    vals = np.zeros(64, np.float32)
    vals[0], vals[1] = -0.5, 0.5
    _, s2, b2 = O.quantize(syn.bf16_bits(vals[None, :]))
    assert syn.bf16_to_f32(s2)[0, 0] < 0 and syn.bf16_to_f32(b2)[0, 0] == 0.5


def test_quantize_constant_groups():
    zero = np.zeros((1, 64), np.uint16)
    wq, s, b = O.quantize(zero)
    assert np.all(wq == 0) and b[0, 0] == 0
    assert s[0, 0] == syn.bf16_bits(np.float32(-1e-7))   # eps with the sign of the max edge
    const = syn.bf16_bits(np.full((1, 64), 0.01, np.float32))
    wq, s, b = O.quantize(const)
    assert np.all(wq == 0) and b[0, 0] == const[0, 0]     # reconstructs exactly as the bias
    neg = syn.bf16_bits(np.full((1, 64), -0.25, np.float32))
    wq, s, b = O.quantize(neg)
    assert np.all(syn.unpack_codes(wq) == 0) and syn.bf16_to_f32(b)[0, 0] == -0.25


def test_quantize_error_bound_random():
    """Every interior code (1..14) reconstructs within half a step plus the bf16 rounding
    of scale and bias. Codes 0 and 15 are excluded: the edge rule re-derives the scale
    from the larger-magnitude extreme, so the far extreme may clip at 15."""
    w = syn.quantize_input(64, 256, seed=3)
    wq, s, b = O.quantize(w)
    codes = syn.unpack_codes(wq).astype(np.float64).reshape(64, 4, 64)
    sf = syn.bf16_to_f32(s).astype(np.float64)[..., None]
    bf = syn.bf16_to_f32(b).astype(np.float64)[..., None]
    x = syn.bf16_to_f32(w).astype(np.float64).reshape(64, 4, 64)
    err = np.abs(codes * sf + bf - x)
    bound = 0.5 * np.abs(sf) + 16 * np.abs(sf) * 2.0**-8 + np.abs(bf) * 2.0**-8
    interior = (codes > 0) & (codes < 15)
    assert interior.mean() > 0.8
    assert np.all(err[interior] <= np.broadcast_to(bound, err.shape)[interior])


# ---------------------------------------------------------------- dequantize

def test_dequantize_modes_match_exact_arithmetic():
    rng = np.random.default_rng(4)
    n, k = 8, 128
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    s = syn.bf16_bits(rng.standard_normal((n, k // 64)).astype(np.float32) * np.float32(0.01))
    b = syn.bf16_bits(rng.standard_normal((n, k // 64)).astype(np.float32) * np.float32(0.05))
    codes = syn.unpack_codes(w)
    for mode in (0, 1):
        got = O.dequantize(w, s, b, mode=mode)
        for r in range(n):
            for c in range(0, k, 7):
                sv = np.float32(syn.bf16_to_f32(s)[r, c // 64])
                bv = np.float32(syn.bf16_to_f32(b)[r, c // 64])
                q = np.float32(codes[r, c])
                prod = sv * q                              # exact in fp32
                if mode == 0:
                    v = np.float32(rne_bf16(float(prod))) + bv
                else:
                    v = prod + bv
                assert got[r, c] == bits_of(rne_bf16(float(v))), (mode, r, c)


def test_dequantize_row_gather_and_exact_grid():
    c = np.tile(np.arange(16), 4)
    w = syn.pack_codes(np.stack([c, c[::-1]]).astype(np.uint8))
    s = syn.bf16_bits(np.full((2, 1), 2.0**-7, np.float32))
    b = syn.bf16_bits(np.full((2, 1), -(2.0**-4), np.float32))
    out = O.dequantize(w, s, b, rows=np.array([1, 0, 1], np.uint32))
    expect = ((np.stack([c[::-1], c, c[::-1]]) - 8) * 2.0**-7).astype(np.float32)
    np.testing.assert_array_equal(syn.bf16_to_f32(out), expect)


# ---------------------------------------------------------------- qmatmul

def _rand_q4(n, k, seed):
    return syn.q4_weights(n, k, seed)


def test_qmatmul_one_hot_pins_nibble_order():
    n, k = 16, 256
    w, s, b = _rand_q4(n, k, 5)
    codes = syn.unpack_codes(w)
    sf, bf = syn.bf16_to_f32(s), syn.bf16_to_f32(b)
    for j in (0, 1, 7, 8, 63, 64, 130, 255):
        x = np.zeros((1, k), np.float32)
        x[0, j] = 1.0
        xb = syn.bf16_bits(x)
        expect = sf[:, j // 64].astype(np.float64) * codes[:, j] + bf[:, j // 64]
        np.testing.assert_array_equal(O.qmatmul_f64(xb, w, s, b)[0], expect)
        np.testing.assert_array_equal(O.qmatmul_f32_grouped(xb, w, s, b)[0], expect.astype(np.float32))
        # the CPU-loop restatement rounds after every bf16 op, so its one-hot row is the
        # op-composed dequantize (mode 0), not the single-rounded one of MLX's dequantize
        deq = O.dequantize(w, s, b, mode=0)[:, j]
        np.testing.assert_array_equal(O.qmatmul_mlx_cpu(xb, w, s, b)[0], deq)


def test_qmatmul_exact_integer_case():
    """x in {-1,0,1}, scale 2^-7, bias -8*scale: every partial sum is exact in fp32."""
    rng = np.random.default_rng(6)
    m, n, k = 3, 40, 3840
    x = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
    codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
    w = syn.pack_codes(codes)
    s = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
    b = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
    exact = (x.astype(np.int64) @ (codes.astype(np.int64) - 8).T) * 2.0**-7
    xb = syn.bf16_bits(x)
    np.testing.assert_array_equal(O.qmatmul_f64(xb, w, s, b), exact)
    np.testing.assert_array_equal(O.qmatmul_f32_grouped(xb, w, s, b), exact.astype(np.float32))


def test_qmatmul_brute_force_small():
    rng = np.random.default_rng(7)
    m, n, k = 3, 5, 192
    x = syn.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    w, s, b = _rand_q4(n, k, 8)
    codes = syn.unpack_codes(w).astype(np.float64)
    sf = np.repeat(syn.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bf = np.repeat(syn.bf16_to_f32(b).astype(np.float64), 64, axis=1)
    ref = syn.bf16_to_f32(x).astype(np.float64) @ (codes * sf + bf).T
    np.testing.assert_allclose(O.qmatmul_f64(x, w, s, b), ref, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(O.qmatmul_f32_grouped(x, w, s, b), ref, rtol=1e-4, atol=1e-6)


def test_qmatmul_reference_weights_test_on_fixture(fixture_q4):
    """native/hyperion_mlx/tests/weights_test.cc:101-139 on the tiny artifact's q_proj:
    x = 0.1 (M=4) against dequantize(f32)+matmul at allclose(rtol=1e-3, atol=1e-2)."""
    w, s, b = fixture_q4["language_model.model.layers.0.self_attn.q_proj"]
    k = s.shape[1] * 64
    x = syn.bf16_bits(np.full((4, k), 0.1, np.float32))
    wd = O.dequantize(w, s, b, mode=1)
    ref = syn.bf16_to_f32(x) @ syn.bf16_to_f32(wd).T
    got = O.qmatmul_f32_grouped(x, w, s, b)
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-2)


def test_mlx_cpu_restatement_accumulates_in_bf16():
    """The MLX CPU restatement (parity unpinned) keeps a bf16 running sum, which the
    mathematics of bf16 fixes on this input: adding 1.0 to a bf16 sum stalls at 256,
    because 256 + 1 rounds back to 256 (ties to even)."""
    k = 3840
    x = syn.bf16_bits(np.ones((1, k), np.float32))
    w = syn.pack_codes(np.ones((1, k), np.uint8))
    s = syn.bf16_bits(np.ones((1, k // 64), np.float32))
    b = np.zeros((1, k // 64), np.uint16)
    assert syn.bf16_to_f32(O.qmatmul_mlx_cpu(x, w, s, b))[0, 0] == 256.0
    assert O.qmatmul_f64(x, w, s, b)[0, 0] == float(k)
    # on the decode workload its error against the fp64 truth is large (reported
    # beside the GPU result as the reference-side error), fp32 grouped is tiny
    x = syn.activations(1, k, seed=9)
    w, s, b = _rand_q4(64, k, 10)
    truth = O.qmatmul_f64(x, w, s, b)
    mlx = syn.bf16_to_f32(O.qmatmul_mlx_cpu(x, w, s, b))
    assert 1e-3 < syn.sig_rel(mlx, truth) < 0.5
    assert syn.sig_rel(O.qmatmul_f32_grouped(x, w, s, b), truth) < 1e-5


def test_mlx_cpu_restatement_threaded_is_identical():
    """The multi-core CPU baseline deals output rows over threads; each row is still one
    sequential bf16 accumulation, so its output equals the single-thread loop bit for
    bit (ragged last block of rows, m = 1 and 3)."""
    k = 640
    w, s, b = _rand_q4(203, k, 11)
    for m in (1, 3):
        x = syn.activations(m, k, seed=12 + m)
        one = O.qmatmul_mlx_cpu(x, w, s, b)
        for threads in (1, 3, 8):
            np.testing.assert_array_equal(O.qmatmul_mlx_cpu_mt(x, w, s, b, threads), one)


# ---------------------------------------------------------------- gelu / softcap

def test_gelu_chain_constants_and_accuracy():
    assert O.scale(syn.bf16_bits(np.float32(1.0)), 0.044715) == syn.bf16_bits(np.float32(0.044677734375))
    assert O.scale(syn.bf16_bits(np.float32(1.0)), 0.7978845608) == syn.bf16_bits(np.float32(0.796875))
    xs = np.linspace(-6, 6, 2001).astype(np.float32)
    xb = syn.bf16_bits(xs)
    xf = syn.bf16_to_f32(xb).astype(np.float64)
    got = syn.bf16_to_f32(O.gelu_tanh(xb)).astype(np.float64)
    ref = 0.5 * xf * (1 + np.tanh(math.sqrt(2 / math.pi) * (xf + 0.044715 * xf**3)))
    assert np.max(np.abs(got - ref)) < 0.05
    assert O.gelu_tanh(syn.bf16_bits(np.float32(0.0)))[0] == 0
    big = syn.bf16_bits(np.float32(20.0))
    assert O.gelu_tanh(big)[0] == big[0]
    up = syn.bf16_bits(np.full(xs.shape, 2.0, np.float32))
    np.testing.assert_array_equal(O.gelu_tanh_mul(xb, up), O.scale(O.gelu_tanh(xb), 2.0))


def test_softcap_accuracy():
    xs = np.linspace(-200, 200, 4001).astype(np.float32)
    xb = syn.bf16_bits(xs)
    got = syn.bf16_to_f32(O.softcap(xb, 30.0)).astype(np.float64)
    ref = 30.0 * np.tanh(syn.bf16_to_f32(xb).astype(np.float64) / 30.0)
    assert np.max(np.abs(got - ref)) <= 0.25       # a few bf16 ulps at |y| ~ 30
    assert np.all(np.abs(got) <= 30.0)


def test_qmatmul_deq_f64_against_dequantize_and_truth():
    rng = np.random.default_rng(11)
    m, n, k = 2, 7, 256
    x = syn.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    w, s, b = _rand_q4(n, k, 12)
    for mode in (0, 1):
        deq = syn.bf16_to_f32(O.dequantize(w, s, b, mode=mode)).astype(np.float64)
        ref = syn.bf16_to_f32(x).astype(np.float64) @ deq.T
        np.testing.assert_allclose(O.qmatmul_deq_f64(x, w, s, b, mode=mode), ref, rtol=1e-12, atol=1e-14)
    # exact bf16 weights (2^-7 grid): identical to the undequantized truth
    s2 = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
    b2 = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
    np.testing.assert_array_equal(O.qmatmul_deq_f64(x, w, s2, b2, mode=0), O.qmatmul_f64(x, w, s2, b2))


def _greedy_by_definition(row_bits):
    """ForwardPass::sample_greedy's result from its definition, computed with numpy:
    the first index of the largest non-NaN value (0 when none exceeds -inf), that value,
    and whether it leads the largest of the other values by less than 0.5."""
    v = syn.bf16_to_f32(row_bits.reshape(-1)).astype(np.float32)
    v = np.where(np.isnan(v), np.float32(-np.inf), v)
    if v.size == 0 or not (v > -np.inf).any():
        return 0, float("-inf"), False
    tok = int(np.argmax(v))
    top1 = v[tok]
    rest = np.delete(v, tok)
    top2 = rest.max() if rest.size else np.float32(-np.inf)
    return tok, float(top1), bool(np.float32(top1) - np.float32(top2) < np.float32(0.5))


def test_sample_greedy_restatement_matches_definition():
    rng = np.random.default_rng(21)
    for trial in range(40):
        n = int(rng.choice([1, 2, 7, 64, 1000, 4099]))
        v = rng.standard_normal(n).astype(np.float32) * 4
        bits = syn.bf16_bits(v)
        if trial % 4 == 1 and n > 3:          # a tie at the maximum, later index
            j, k2 = sorted(rng.choice(n, 2, replace=False))
            bits[j] = bits[k2] = syn.bf16_bits(np.float32([50.0]))[0]
        if trial % 4 == 2 and n > 3:          # NaN and infinities
            bits[rng.integers(n)] = 0x7FC0
            bits[rng.integers(n)] = 0xFF80
            if trial % 8 == 2:
                bits[rng.integers(n)] = 0x7F80
        if trial % 4 == 3 and n > 1:          # near tie just under / over 0.5
            top = int(np.argmax(syn.bf16_to_f32(bits)))
            other = (top + 1) % n
            bits[top] = syn.bf16_bits(np.float32([20.0]))[0]
            bits[other] = syn.bf16_bits(np.float32([19.5 if trial % 8 == 3 else 19.625]))[0]
        assert O.sample_greedy(bits) == _greedy_by_definition(bits), f"trial {trial}"
    # hand cases
    assert O.sample_greedy(np.zeros(0, np.uint16)) == (0, float("-inf"), False)
    assert O.sample_greedy(np.full(5, 0xFF80, np.uint16)) == (0, float("-inf"), False)
    assert O.sample_greedy(np.full(5, 0x7FC0, np.uint16)) == (0, float("-inf"), False)
    assert O.sample_greedy(syn.bf16_bits(np.float32([1, 3, 3, 2]))) == (1, 3.0, True)
    assert O.sample_greedy(syn.bf16_bits(np.float32([1, 3, 2.5, 2]))) == (1, 3.0, False)
    assert O.sample_greedy(syn.bf16_bits(np.float32([1, 3, 2.75, 2]))) == (1, 3.0, True)




def test_gelu_chain_closed_forms_outside_the_tabulated_band():
    """The dual GEMM's epilogue tabulates the GELU chain for 2^-10 <= |x| < 8 and uses
    closed forms elsewhere: bf16(x / 2) below the band (tanh's argument is under 2^-9, so
    1 + t rounds to 1), x above it (and +inf), -0 below -8 (t = -1, so 1 + t = 0). Checked
    here against the oracle's chain for every other finite bf16 input and +inf."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    a = bits & 0x7FFF
    outside = ((a < 0x3A80) | (a >= 0x4100)) & (a <= 0x7F80) & (bits != 0xFF80)
    xs = bits[outside]
    got = O.gelu_tanh(xs)
    x = syn.bf16_to_f32(xs)
    small = (xs & 0x7FFF) < 0x3A80
    want = np.where(small, O.bf16_from_f32((np.float32(0.5) * x).astype(np.float32)),
                    np.where(x > 0, xs, np.uint16(0x8000)))
    assert xs.size == 65536 - 2 * (0x4100 - 0x3A80) - 2 * 127 - 1
    np.testing.assert_array_equal(got, want.astype(np.uint16))

# ---------------------------------------------------------------- top-k sidecar of the greedy epilogue
def _distinct_top_row(rng, n, k=O.TOP_K):
    """A row whose k + 1 largest values are distinct: normal draws in [-8, 8] plus k + 1
    distinct planted values above them, at random positions."""
    bits = syn.bf16_bits(np.clip(rng.standard_normal(n) * 3, -8, 8).astype(np.float32))
    top = min(n, k + 1)
    planted = syn.bf16_bits((16.0 + 0.125 * rng.permutation(64)[:top]).astype(np.float32))
    bits[rng.choice(n, top, replace=False)] = planted
    return bits


@pytest.mark.parametrize("n", [1, 7, 8, 9, 100, 4099, 262144])
def test_topk_equals_partial_sort_where_values_are_distinct(n):
    """Where the top k + 1 values are distinct, any conforming std::partial_sort gives one
    answer: libstdc++'s, called with the reference's comparator, is the pin."""
    rng = np.random.default_rng(n)
    for trial in range(3):
        bits = _distinct_top_row(rng, n)
        p = syn.bf16_to_f32(bits)
        cnt, ids, vals = O.sample_topk(bits)
        want = O.stl_partial_sort_topk(p)
        assert cnt == min(O.TOP_K, n) == want.size
        np.testing.assert_array_equal(ids[:cnt], want, err_msg=f"n={n} trial {trial}")
        np.testing.assert_array_equal(vals[:cnt].view(np.uint32), p[want].view(np.uint32))
        assert not ids[cnt:].any() and not vals[cnt:].any()


def test_topk_values_equal_partial_sort_with_ties():
    """A vocabulary-sized bf16 row of normal logits nearly always has equal values among
    its top 9 (bf16 keeps 8 significant bits); the values returned are still partial_sort's,
    and the ids name elements of those values; only which tied ids, and their order, is
    defined here rather than left to the library."""
    rng = np.random.default_rng(5)
    ties_seen = 0
    for trial in range(8):
        bits = syn.bf16_bits((rng.standard_normal(262144) * 3).astype(np.float32))
        p = syn.bf16_to_f32(bits)
        cnt, ids, vals = O.sample_topk(bits)
        want = O.stl_partial_sort_topk(p)
        np.testing.assert_array_equal(vals[:cnt], p[want])
        np.testing.assert_array_equal(vals[:cnt], p[ids[:cnt]])
        assert len(set(ids[:cnt].tolist())) == cnt
        top9 = np.sort(p)[::-1][:9]
        ties_seen += len(set(top9.tolist())) < 9
        # the defined order: within a run of equal values the ids ascend, and they are
        # the lowest indices holding that value
        for v in set(vals[:cnt].tolist()):
            sel = ids[:cnt][vals[:cnt] == v]
            assert list(sel) == sorted(sel)
            np.testing.assert_array_equal(sel, np.flatnonzero(p == v)[: sel.size])
    assert ties_seen >= 6


def _topk_by_sorting(bits, k=O.TOP_K):
    """The defined order by a full sort (Python's sorted on a key), for small rows."""
    p = syn.bf16_to_f32(bits.reshape(-1))
    order = sorted(range(p.size), key=lambda i: (bool(np.isnan(p[i])), 0.0 if np.isnan(p[i]) else -float(p[i]), i))
    return order[:k]


def test_topk_defined_order_hand_cases():
    f = lambda xs: syn.bf16_bits(np.float32(xs))
    nan, inf = float("nan"), float("inf")
    assert O.sample_topk(np.zeros(0, np.uint16))[0] == 0
    cnt, ids, vals = O.sample_topk(f([3, 5, 5, 1, 5]), 2)
    assert (cnt, list(ids)) == (2, [1, 2])
    cnt, ids, _ = O.sample_topk(f([7.0] * 20))
    assert list(ids) == list(range(8))
    cnt, ids, vals = O.sample_topk(np.array([0x8000, 0x0000, 0x8000], np.uint16))   # -0, +0, -0
    assert (cnt, list(ids[:3])) == (3, [0, 1, 2])
    assert list(vals[:3].view(np.uint32)) == [0x80000000, 0, 0x80000000]
    cnt, ids, vals = O.sample_topk(f([nan, 1, nan, -inf]))
    assert (cnt, list(ids[:4])) == (4, [1, 3, 0, 2]) and not ids[4:].any()
    cnt, ids, vals = O.sample_topk(f([nan] * 10))
    assert list(ids) == list(range(8)) and np.isnan(vals).all()
    cnt, ids, vals = O.sample_topk(f([-inf, 2, inf, -1, inf, 0]))
    assert list(ids[:6]) == [2, 4, 1, 5, 3, 0]
    rng = np.random.default_rng(77)
    for trial in range(30):
        n = int(rng.integers(1, 300))
        bits = syn.bf16_bits(rng.integers(-4, 5, n).astype(np.float32))   # many ties
        bits[rng.random(n) < 0.05] = 0x7FC0
        bits[rng.random(n) < 0.05] = 0xFF80
        bits[rng.random(n) < 0.05] = 0x8000
        cnt, ids, _ = O.sample_topk(bits)
        assert list(ids[:cnt]) == _topk_by_sorting(bits), f"trial {trial}"


def test_topk_head_agrees_with_greedy():
    """The sidecar's first entry is the greedy token whenever some value exceeds -inf, and
    its second value is the greedy scan's top2 (the largest other non-NaN value)."""
    rng = np.random.default_rng(31)
    for trial in range(40):
        n = int(rng.choice([2, 9, 1000, 4099]))
        bits = syn.bf16_bits((rng.standard_normal(n) * 4).astype(np.float32))
        if trial % 3 == 1:
            bits[rng.choice(n, 2, replace=False)] = syn.bf16_bits(np.float32([50.0]))[0]
        if trial % 3 == 2:
            bits[rng.integers(n)] = 0x7FC0
            bits[rng.integers(n)] = 0x7F80
        tok, logit, tie = O.sample_greedy(bits)
        cnt, ids, vals = O.sample_topk(bits)
        assert ids[0] == tok and vals[0] == logit
        top2 = vals[1] if not np.isnan(vals[1]) else np.float32(-np.inf)
        assert tie == bool(np.float32(logit) - top2 < np.float32(0.5))

# ---------------------------------------------------------------- exhaustive pins of the bf16 op chains
#
# Independent restatements of the reference's op chains (forward.cc:154-160 softcap,
# forward.cc:324-336 gelu_pytorch_tanh, forward.cc:338-343 the gating product), evaluated
# over all 65,536 bf16 inputs. Each MLX op on bf16 arrays computes in fp32 and rounds the
# result to bf16; here every op is evaluated exactly in float64 (a product of two bf16
# values has at most 16 significant bits; a sum of two whose exponents differ by more
# than 29 rounds to the larger operand in fp32 either way), then rounded to fp32 and to
# bf16 with an integer round-half-even of the bit pattern. tanh comes from float64;
# inputs whose float64 tanh lies within 2^-20 (relative) of a bf16 rounding boundary are
# excluded and counted, since fp32 tanhf may round to the other side there.

def _rne_bf16_of_f32(f32):
    """float32 array -> bf16 values (as float64), round half to even on the bit pattern."""
    f = np.atleast_1d(np.asarray(f32, np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    out = (r.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    out[np.isnan(f)] = np.nan
    return out if np.ndim(f32) else out[0]


def _op(v64):
    """One MLX bf16 op: the exact value, to fp32, to bf16."""
    with np.errstate(over="ignore", invalid="ignore"):
        return _rne_bf16_of_f32(np.asarray(v64, np.float64).astype(np.float32))


def _near_bf16_boundary(v64, rel=2.0**-20):
    """True where v64 is within rel of a midpoint between two adjacent bf16 values."""
    v = np.abs(np.asarray(v64, np.float64))
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(v > 0, v, 1.0)))
    ulp = np.exp2(np.maximum(e, -126.0) - 7.0)
    frac = v / ulp - np.floor(v / ulp)
    return (np.abs(frac - 0.5) * ulp <= rel * np.maximum(v, 1e-300)) & (v > 0)


def _all_bf16():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    with np.errstate(invalid="ignore"):
        vals = syn.bf16_to_f32(bits).astype(np.float64)
    return bits, vals


def _cmp_bits(got_bits, want64, keep, what):
    got = syn.bf16_to_f32(got_bits).astype(np.float64)
    both_nan = np.isnan(got) & np.isnan(want64)
    same = (got == want64) & (np.signbit(got) == np.signbit(want64))
    bad = keep & ~(same | both_nan)
    assert not bad.any(), f"{what}: {int(bad.sum())} inputs differ, first at bits {np.nonzero(bad)[0][:5]}"


def test_gelu_chain_bit_exact_over_all_bf16_inputs():
    bits, x = _all_bf16()
    c_coeff = _op(0.044715)        # mx::array(0.044715F, bf16)
    c_inner = _op(0.7978845608028654)
    with np.errstate(over="ignore", invalid="ignore"):
        sq = _op(x * x)                          # square(x)
        x3 = _op(x * sq)                         # multiply(x, square(x))
        inner = _op(c_coeff * x3)
        inner = _op(inner + x)
        inner = _op(c_inner * inner)
        t64 = np.tanh(inner)
        t = _op(t64)
        half_x = _op(0.5 * x)
        one_t = _op(1.0 + t)
        want = _op(half_x * one_t)
    keep = ~_near_bf16_boundary(t64)
    excluded = int((~keep).sum())
    print(f"gelu chain: {excluded} of 65536 inputs excluded (tanh within 2^-20 of a bf16 tie)")
    assert excluded < 200
    _cmp_bits(O.gelu_tanh(bits), want, keep, "gelu chain")
    # the gating product with a second operand, over a sweep of up values
    rng = np.random.default_rng(5)
    up_bits = syn.bf16_bits(rng.standard_normal(65536).astype(np.float32))
    up = syn.bf16_to_f32(up_bits).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        want_mul = _op(want * up)
    _cmp_bits(O.gelu_tanh_mul(bits, up_bits), want_mul, keep, "gelu * up")


def test_softcap_bit_exact_over_all_bf16_inputs():
    bits, x = _all_bf16()
    for cap in (30.0, 50.0):
        c = _op(cap)                                   # mx::array(cap, logits dtype)
        with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
            d = _op(x / c)                             # divide: correctly rounded fp32, then bf16
            t64 = np.tanh(d)
            want = _op(_op(t64) * c)
        keep = ~_near_bf16_boundary(t64)
        excluded = int((~keep).sum())
        print(f"softcap {cap}: {excluded} of 65536 inputs excluded")
        assert excluded < 200
        _cmp_bits(O.softcap(bits, cap), want, keep, f"softcap {cap}")


def test_mlx_cpu_restatement_per_element_step_exact():
    """The MLX CPU loop's per-element step, restated with exact rationals: dq = bf16(
    bf16(scale * q) + bias); sum = bf16(sum + bf16(x * dq)), in k order, each op an fp32
    result rounded to bf16. Small random cases, compared bit for bit."""
    rng = np.random.default_rng(21)

    def rne32(fr):
        """Round a rational to float32, half to even (exact)."""
        return float(np.float32(float(fr))) if fr == Fraction(float(fr)) else _rne_rational_f32(fr)

    def op(fr):
        return Fraction(rne_bf16(Fraction(rne32(fr))))

    for case in range(6):
        m, n, k = 2, 3, 128
        x = syn.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
        codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
        w = syn.pack_codes(codes)
        s = syn.bf16_bits((np.abs(rng.standard_normal((n, k // 64))) * 0.05).astype(np.float32))
        b = syn.bf16_bits((-rng.random((n, k // 64)) * 0.4).astype(np.float32))
        got = O.qmatmul_mlx_cpu(x, w, s, b)
        xf = [[Fraction(float(v)) for v in row] for row in syn.bf16_to_f32(x)]
        sf = syn.bf16_to_f32(s)
        bfv = syn.bf16_to_f32(b)
        for i in range(m):
            for r in range(n):
                acc = Fraction(0)
                for kk in range(k):
                    g = kk // 64
                    dq = op(op(Fraction(float(sf[r, g])) * int(codes[r, kk])) + Fraction(float(bfv[r, g])))
                    acc = op(acc + op(xf[i][kk] * dq))
                assert syn.bf16_bits(np.float32(float(acc))) == got[i, r], (case, i, r)


def _rne_rational_f32(fr):
    """Round a rational to the nearest float32 (half to even), exactly."""
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    return sign * float(round(a / ulp) * ulp)


def test_dequantize_modes_mismatch_rate_on_the_decode_weights():
    """(A) bf16(bf16(s*q) + b) against (B) bf16(fma(s, q, b)) on the decode workload's
    weights [15360, 3840] (bias = -8 * scale). There s*q + b is exact in fp32 (at most 12
    significant bits), so (B) is the correctly rounded value: checked exactly on a sample.
    (A) rounds s*q to 8 bits before the subtraction and differs on a large fraction of
    values (printed). MLX's is (B): tests/test_golden_embed.py decides it on the reference's
    12B embed golden."""
    w, s, b = syn.q4_weights(15360, 3840, seed=105)
    a = O.dequantize(w, s, b, mode=0)
    bb = O.dequantize(w, s, b, mode=1)
    rate = float(np.mean(a != bb))
    print(f"dequantize (A) vs (B): {rate:.4%} of {a.size} values differ")
    codes = syn.unpack_codes(w[:64])
    sf = syn.bf16_to_f32(s[:64]).astype(np.float64)
    bf = syn.bf16_to_f32(b[:64]).astype(np.float64)
    exact = sf.repeat(64, axis=1) * codes + bf.repeat(64, axis=1)     # exact in float64
    np.testing.assert_array_equal(bb[:64], syn.bf16_bits(exact.astype(np.float32)))
    assert 0.2 < rate < 0.6


# ---------------------------------------------------------------- rms norm with weight, rope

def test_rms_norm_oracle_against_closed_form_and_exact_cases():
    rng = np.random.default_rng(31)
    for rows, k in ((3, 3840), (5, 256), (2, 1000), (4, 512)):
        x = syn.bf16_bits((rng.standard_normal((rows, k)) * rng.choice([1e-3, 1.0, 50.0], (rows, 1))).astype(np.float32))
        w = syn.bf16_bits((1.0 + 0.3 * rng.standard_normal(k)).astype(np.float32))
        xf = syn.bf16_to_f32(x).astype(np.float64)
        wf = syn.bf16_to_f32(w).astype(np.float64)
        inv = 1.0 / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-6)
        plain = syn.bf16_to_f32(O.rms_norm(x, None, 1e-6)).astype(np.float64)
        ref = xf * inv
        assert np.all(np.abs(plain - ref) <= np.abs(ref) * 2.0**-8 * 1.01 + 1e-30), (rows, k)
        got = syn.bf16_to_f32(O.rms_norm(x, w, 1e-6)).astype(np.float64)
        refw = wf * ref
        assert np.all(np.abs(got - refw) <= np.abs(refw) * 2.0**-7 * 1.01 + 1e-30), (rows, k)
        # the weighted form is the weightless one times w, rounded once more
        np.testing.assert_array_equal(O.rms_norm(x, w, 1e-6), syn.bf16_bits((syn.bf16_to_f32(O.rms_norm(x, None, 1e-6)) * syn.bf16_to_f32(w)).astype(np.float32)))
        # a weight of ones changes nothing; a power-of-two weight scales exactly
        ones = syn.bf16_bits(np.ones(k, np.float32))
        np.testing.assert_array_equal(O.rms_norm(x, ones, 1e-6), O.rms_norm(x, None, 1e-6))
        four = syn.bf16_bits(np.full(k, 4.0, np.float32))
        np.testing.assert_array_equal(syn.bf16_to_f32(O.rms_norm(x, four, 1e-6)), 4.0 * syn.bf16_to_f32(O.rms_norm(x, None, 1e-6)))
    # a constant row c: inv = 1/sqrt(c^2 + eps); with eps = 0, every output is exactly 1
    x = syn.bf16_bits(np.full((2, 640), 3.0, np.float32))
    assert np.all(syn.bf16_to_f32(O.rms_norm(x, None, 0.0)) == 1.0)


def _rope_truth(x, heads, d, rotated, base, offset):
    rows = x.shape[0]
    xf = syn.bf16_to_f32(x).astype(np.float64).reshape(rows, heads, d)
    half = d // 2
    i = np.arange(half)
    inv = np.where(2 * i < rotated, base ** (-2.0 * i / d), 0.0)
    pos = (offset + np.arange(rows))[:, None]
    th = pos * inv[None, :]
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    x1, x2 = xf[..., :half], xf[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def test_rope_oracle_against_closed_form():
    rng = np.random.default_rng(32)
    for rows, heads, d, rotated, base, offset in ((4, 3, 256, 256, 1e4, 0), (3, 2, 512, 128, 1e6, 17),
                                                  (2, 4, 256, 256, 1e4, 4095), (1, 16, 256, 256, 1e4, 100000)):
        x = syn.bf16_bits(rng.standard_normal((rows, heads * d)).astype(np.float32))
        got = syn.bf16_to_f32(O.rope(x, rows, heads, d, rotated, base, offset)).astype(np.float64)
        truth = _rope_truth(x, heads, d, rotated, base, offset)
        # one bf16 rounding, plus theta's fp32 rounding (|d theta| <= pos * 2^-24)
        mag = np.abs(syn.bf16_to_f32(x).astype(np.float64).reshape(rows, heads, d))
        pair = np.sqrt(mag[..., : d // 2] ** 2 + mag[..., d // 2:] ** 2)
        pair = np.concatenate([pair, pair], axis=-1)
        pos = (offset + np.arange(rows))[:, None, None]
        bound = np.abs(truth) * 2.0**-8 * 1.01 + pair * (2.0**-22 + pos * 2.0**-23)
        assert np.all(np.abs(got - truth) <= bound), (rows, heads, d, rotated, offset)
        if offset == 0:   # position 0 is the identity
            np.testing.assert_array_equal(O.rope(x, rows, heads, d, rotated, base, 0)[0], x.reshape(rows, heads, d)[0])
        if rotated < d:   # pairs past the rotated ones are left as they are
            xr = x.reshape(rows, heads, d)
            gr = O.rope(x, rows, heads, d, rotated, base, offset)
            np.testing.assert_array_equal(gr[..., rotated // 2: d // 2], xr[..., rotated // 2: d // 2])
            np.testing.assert_array_equal(gr[..., d // 2 + rotated // 2:], xr[..., d // 2 + rotated // 2:])


def test_rope_oracle_pairs_and_sign_on_one_hot_inputs():
    """A one in element i of the first half rotates into (cos, sin) at (i, i + D/2); a one
    in element i + D/2 into (-sin, cos): this pins the non-traditional pairing and the sign."""
    d, heads, pos = 256, 1, 7
    for i in (0, 1, 63, 127):
        inv = 1e4 ** (-2.0 * i / d)
        th = np.float32(np.float32(pos) * np.float32(inv))
        for src, want in ((i, (np.cos(th), np.sin(th))), (i + d // 2, (-np.sin(th), np.cos(th)))):
            x = np.zeros((1, d), np.float32)
            x[0, src] = 1.0
            y = syn.bf16_to_f32(O.rope(syn.bf16_bits(x), 1, heads, d, d, 1e4, pos)).reshape(d)
            assert y[i] == syn.bf16_to_f32(syn.bf16_bits(np.float32(want[0]))), (i, src)
            assert y[i + d // 2] == syn.bf16_to_f32(syn.bf16_bits(np.float32(want[1]))), (i, src)
            others = np.delete(y, [i, i + d // 2])
            assert not others.any()


# ---------------------------------------------------------------- attention (scale 1, causal + window, GQA)
def _attention_dense(q, k, v, ck, cv, offset, prefix_len, window):
    """The same attention written densely with numpy: gather the key/value rows by position,
    a [L, T] visibility matrix by broadcasting, scores by einsum, softmax along T."""
    qf = syn.bf16_to_f32(q).astype(np.float64)
    L, H, D = qf.shape
    KVH = k.shape[1]
    cap = ck.shape[0]
    pos = np.arange(offset - prefix_len, offset + L)
    keys = np.concatenate([syn.bf16_to_f32(ck)[(pos[:prefix_len] % cap)], syn.bf16_to_f32(k)], 0).astype(np.float64)
    vals = np.concatenate([syn.bf16_to_f32(cv)[(pos[:prefix_len] % cap)], syn.bf16_to_f32(v)], 0).astype(np.float64)
    qpos = offset + np.arange(L)
    vis = pos[None, :] <= qpos[:, None]
    if window:
        vis &= pos[None, :] > qpos[:, None] - window
    g = H // KVH
    kh = np.repeat(keys, g, axis=1)          # [T, H, D]
    vh = np.repeat(vals, g, axis=1)
    sc = np.einsum("lhd,thd->lht", qf, kh)
    sc = np.where(vis[:, None, :], sc, -np.inf)
    sc = sc - sc.max(-1, keepdims=True)
    p = np.exp(sc)
    p = p / p.sum(-1, keepdims=True)
    return np.einsum("lht,thd->lhd", p, vh)


@pytest.mark.parametrize("L,H,KVH,D,cap,offset,prefix,window", [
    (1, 4, 2, 64, 16, 0, 0, 8), (3, 4, 2, 64, 16, 5, 5, 8), (4, 4, 2, 64, 16, 30, 8, 8),   # ring wrapped
    (1, 8, 1, 128, 64, 40, 40, 0), (6, 8, 1, 128, 64, 10, 10, 0), (20, 4, 2, 64, 16, 0, 0, 8),
    (5, 16, 8, 32, 12, 100, 10, 11)])
def test_attention_oracle_matches_dense_numpy(L, H, KVH, D, cap, offset, prefix, window):
    rng = np.random.default_rng(L * 100 + offset)
    b = lambda *shape: syn.bf16_bits(rng.standard_normal(shape).astype(np.float32))  # noqa: E731
    q, k, v, ck, cv = b(L, H, D), b(L, KVH, D), b(L, KVH, D), b(cap, KVH, D), b(cap, KVH, D)
    got = O.attention_f64(q, k, v, ck, cv, offset, prefix, window)
    np.testing.assert_allclose(got, _attention_dense(q, k, v, ck, cv, offset, prefix, window), rtol=1e-12, atol=1e-12)


def test_attention_oracle_closed_forms():
    rng = np.random.default_rng(9)
    b = lambda *shape: syn.bf16_bits(rng.standard_normal(shape).astype(np.float32))  # noqa: E731
    L, H, KVH, D, cap = 3, 4, 2, 64, 16
    q, k, v, ck, cv = b(L, H, D), b(L, KVH, D), b(L, KVH, D), b(cap, KVH, D), b(cap, KVH, D)
    # window 1: each query sees only itself -> its own value row (per kv head)
    out = O.attention_f64(q, k, v, ck, cv, 7, 7, 1)
    vf = syn.bf16_to_f32(v).astype(np.float64)
    np.testing.assert_allclose(out, np.repeat(vf, H // KVH, axis=1), rtol=0, atol=1e-15)
    # all keys equal -> the mean of the visible values
    kk = np.repeat(k[:1], L, 0)
    ckk = np.broadcast_to(k[:1], (cap, KVH, D)).copy()
    out = O.attention_f64(q, kk, v, ckk, cv, 4, 4, 0)
    allv = np.concatenate([syn.bf16_to_f32(cv)[np.arange(0, 4) % cap], vf], 0)
    for t in range(L):
        mean = allv[: 4 + t + 1].mean(0)
        np.testing.assert_allclose(out[t], np.repeat(mean, H // KVH, axis=0), rtol=1e-12, atol=1e-12)
    # values all one -> ones (the weights sum to one)
    ones = np.full((L, KVH, D), 0x3F80, np.uint16)
    out = O.attention_f64(q, k, ones, ck, np.full((cap, KVH, D), 0x3F80, np.uint16), 9, 9, 5)
    np.testing.assert_allclose(out, 1.0, rtol=1e-12)


# ---- the decoder restatement (DecoderOracle) ---------------------------------------------

def _tiny_dims_model(tmp_path, seed=3, layer_types=None):
    import json
    cfg = {
        "model_type": "gemma4_unified_text", "hidden_size": 128, "intermediate_size": 256,
        "layer_types": layer_types or ["sliding_attention"] * 2 + ["full_attention"], "num_attention_heads": 4,
        "head_dim": 64, "global_head_dim": 128, "num_key_value_heads": 2, "num_global_key_value_heads": 1,
        "attention_k_eq_v": True, "sliding_window": 8,
        "rope_parameters": {"sliding_attention": {"rope_theta": 10000.0},
                            "full_attention": {"rope_theta": 1e6, "partial_rotary_factor": 0.25,
                                               "rope_type": "proportional"}},
        "final_logit_softcapping": 30.0, "rms_norm_eps": 1e-6, "vocab_size": 64, "max_position_embeddings": 64,
    }
    cfg["num_hidden_layers"] = len(cfg["layer_types"])
    T = syn.write_model(str(tmp_path), cfg, seed)
    return dict(T), json.loads(json.dumps(cfg))


def _zero_proj(T, base):
    T[base + ".weight"] = np.zeros_like(T[base + ".weight"])
    T[base + ".scales"] = np.zeros_like(T[base + ".scales"])
    T[base + ".biases"] = np.zeros_like(T[base + ".biases"])


def test_decoder_oracle_residual_wiring_closed_form(tmp_path):
    """With every o_proj and down_proj zero, each branch's rms_norm of a zero row is zero
    (0 * 1/sqrt(eps)), so the residual stream is the embedding times the layer scalars,
    rounded after each product (forward.cc:518-539), and the output its final norm."""
    T, cfg = _tiny_dims_model(tmp_path)
    P = "language_model.model."
    for i in range(cfg["num_hidden_layers"]):
        _zero_proj(T, f"{P}layers.{i}.self_attn.o_proj")
        _zero_proj(T, f"{P}layers.{i}.mlp.down_proj")
    ids = [3, 17, 60, 0, 41]
    got = O.DecoderOracle(T, cfg).forward(ids, 0)
    # closed form, numpy only: dequantized rows (one rounding of s*q + b, as MLX's
    # dequantize), times bf16(sqrt(128)), times each bf16 scalar, then the weighted RMS norm
    # in fp64.
    e = P + "embed_tokens"
    codes = syn.unpack_codes(T[e + ".weight"][ids]).astype(np.float32)
    s = np.repeat(syn.bf16_to_f32(T[e + ".scales"][ids]), 64, axis=1)
    b = np.repeat(syn.bf16_to_f32(T[e + ".biases"][ids]), 64, axis=1)
    x = syn.bf16_to_f32(syn.bf16_bits(s * codes + b))
    x = syn.bf16_to_f32(syn.bf16_bits(x * syn.bf16_to_f32(syn.bf16_bits(np.float32(np.sqrt(np.float32(128)))))))
    for i in range(cfg["num_hidden_layers"]):
        x = syn.bf16_to_f32(syn.bf16_bits(x * syn.bf16_to_f32(T[f"{P}layers.{i}.layer_scalar"])[0]))
    xd = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-6)
    ref = syn.bf16_to_f32(T[P + "norm.weight"]).astype(np.float64) * syn.bf16_to_f32(syn.bf16_bits(
        (xd * inv).astype(np.float32))).astype(np.float64)
    # the norm's fp32 statistics against fp64: within one bf16 rounding of each product
    np.testing.assert_allclose(syn.bf16_to_f32(got), ref, rtol=2 ** -7, atol=0)


def test_decoder_oracle_single_token_attention_is_v(tmp_path):
    """At offset 0 a single token's only visible key is itself, so SDPA returns V: the layer
    must equal the same layer with the attention replaced by V = v_norm(v_proj(x)) on
    sliding layers and v_norm(k_proj(x)) on global (K = V) layers, kv head h // G for query
    head h (forward.cc:403-412, :497-505). q, k, RoPE and the scores drop out."""
    T, cfg = _tiny_dims_model(tmp_path, seed=4)
    P = "language_model.model."
    D = O.DecoderOracle(T, cfg)
    x = D.embed([9])
    for i, kind in enumerate(D.kinds):
        got = D.layer(x.copy(), i, 0)
        pre = f"layers.{i}."
        sliding = kind == "sliding"
        d, kvh = (D.d_local, D.kv_local) if sliding else (D.d_global, D.kv_global)
        h = O.rms_norm(x, T[P + pre + "input_layernorm.weight"])
        src = "self_attn.v_proj" if sliding else "self_attn.k_proj"
        raw = D._proj(h, pre + src).reshape(kvh, d)
        v = O.rms_norm(raw, None)
        att = v[np.arange(D.heads) // (D.heads // kvh)].reshape(1, -1)
        o = D._proj(att, pre + "self_attn.o_proj")
        y = O.add_bf16(x, O.rms_norm(o, T[P + pre + "post_attention_layernorm.weight"]))
        hh = O.rms_norm(y, T[P + pre + "pre_feedforward_layernorm.weight"])
        gu = O.gelu_tanh_mul(D._proj(hh, pre + "mlp.gate_proj"), D._proj(hh, pre + "mlp.up_proj"))
        dn = D._proj(gu, pre + "mlp.down_proj")
        y = O.add_bf16(y, O.rms_norm(dn, T[P + pre + "post_feedforward_layernorm.weight"]))
        y = O.mul_bf16(y, T[P + pre + "layer_scalar"])
        np.testing.assert_array_equal(got, y, err_msg=f"layer {i} ({kind})")
        x = got


def test_decoder_oracle_chunking_invariance(tmp_path):
    """Prefix then continuation equals one shot, bit for bit (the invariant of
    forward_test.cc:412-482, exact here because every op of the oracle is row-wise): the
    caches, positions, prefix lengths and windows are threaded consistently; the window (8)
    is crossed."""
    T, cfg = _tiny_dims_model(tmp_path, seed=5)
    ids = [(7 * i + 3) % 64 for i in range(21)]
    whole = O.DecoderOracle(T, cfg).forward(ids, 0)
    D = O.DecoderOracle(T, cfg)
    parts = [D.forward(ids[:12], 0), D.forward(ids[12:13], 12), D.forward(ids[13:], 13)]
    np.testing.assert_array_equal(np.concatenate(parts), whole)


def test_decoder_oracle_window_hides_old_tokens(tmp_path):
    """On a sliding layer (window 8) a token 8 or more positions before the query is
    invisible to it (build_mask, forward.cc:365-371), while one inside the window is seen."""
    T, cfg = _tiny_dims_model(tmp_path, seed=6, layer_types=["sliding_attention", "full_attention"])
    D = O.DecoderOracle(T, cfg)
    a = [(5 * i + 1) % 64 for i in range(12)]
    b = list(a)
    b[3] = (b[3] + 1) % 64          # position 3 < 11 - 8 + 1: outside the last query's window
    xa, xb = D.embed(a), D.embed(b)
    Da, Db = O.DecoderOracle(T, cfg), O.DecoderOracle(T, cfg)
    ya, yb = Da.layer(xa, 0, 0), Db.layer(xb, 0, 0)
    np.testing.assert_array_equal(ya[11], yb[11])
    assert not np.array_equal(ya[4], yb[4])   # position 4 still sees position 3
