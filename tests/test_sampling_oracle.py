"""The oracle's temperature draw (orc_sample_stochastic_bf16) pinned against the reference's
host sampler and against the mathematics.

ForwardPass::sample_stochastic (forward.cc:191-301) scales the fp32 logits by 1/temperature,
takes a std::exp softmax, masks the tokens outside the top-p nucleus (std::sort of the
probabilities), below min_p times the largest probability and outside the top-k
(std::partial_sort of the scaled logits), then draws u = uniform_real_distribution<float>(0, sz)
from std::mt19937_64(rng_state) and returns the first index whose running sum of the kept
exp(t - max) reaches u. oracle/stl_sample_stochastic.cc restates that host algorithm over
libstdc++ (the library the reference links); the oracle restates the HIP kernels' defined
algorithm (fixed tie order and summation order, which the reference's contract leaves open:
hyperion_mlx.h:125-133). The bars:

  * the RNG: std::mt19937_64's 10000th output from the default seed is the C++ standard's
    check value; the uniform the kernels scale (generate_canonical<float, 24>) is the first
    64-bit output over 2^64 rounded to fp32, and uniform_real_distribution<float>(0, b)
    equals b times it, bit for bit;
  * det_exp within 2 ulp of the correctly rounded exp on (-86, 0], exact at 0, 0 below;
  * kept sets: equal to the first n of (value descending, index ascending) with n from a
    float64 softmax, wherever the float64 running mass is not within 1e-5 of top_p; equal
    to the reference host sampler's mask on rows of distinct values wherever no float32
    running mass of the reference sits within 1e-5 of top_p;
  * tokens: equal to the reference host sampler's draw for the same RNG state, except where
    u lies within 2e-6 (relative) of a running-sum boundary between the two tokens;
  * the frequencies over 20,000 seeds match the filtered softmax (chi-square, p > 1e-4);
  * top_k = 1 and near-zero temperatures give the greedy token; rows with +inf, NaN or no
    finite scaled logit give what the reference's arithmetic gives (last index / index 0);
    u = 0 gives index 0; temperature +inf gives the closed-form uniform draw.
"""
import math

import numpy as np
import pytest

import oracle as O
from hyperion_amd import synthetic as syn


def bf16(x):
    return syn.bf16_bits(np.asarray(x, np.float32))


def f32(bits):
    return syn.bf16_to_f32(bits)


def order_of(bits):
    """Indices in (value descending, index ascending) order; finite values only."""
    v = f32(bits).astype(np.float64)
    idx = np.arange(v.size)
    fin = np.isfinite(v)
    v, idx = v[fin], idx[fin]
    o = np.lexsort((idx, -v))
    return idx[o]


def kept_n_float64(bits, temperature, top_k, top_p, min_p):
    """n of the kept prefix from a float64 softmax, the order, the distance of the nearest
    filter boundary (running mass to top_p, probability to the min-p threshold), and the
    float64 probabilities in that order."""
    order = order_of(bits)
    t = f32(bits)[order].astype(np.float64) / temperature
    w = np.exp(t - t.max())
    p = w / w.sum()
    total = order.size
    n, margin = total, np.inf
    if 0 < top_p <= 1:
        c = np.cumsum(p)
        hit = np.nonzero(c >= top_p)[0]
        if hit.size:
            n = int(hit[0]) + 1
        margin = float(np.min(np.abs(c - top_p)))
    if 0 < min_p < 1:
        n = min(n, int((p >= min_p * p.max()).sum()))
        margin = min(margin, float(np.min(np.abs(p - min_p * p.max())) / p.max()))
    if 0 < top_k < bits.size:
        n = min(n, top_k)
    return n, order, margin, p


def distinct_row(rng, vocab, scale):
    """bf16 logits with no two equal values and no two equal fp32 probabilities (no tie order
    to choose): distinct bit patterns of magnitude 2^-6 .. 4 * scale, either sign, in random
    order (neighbouring values then differ by at least 2^-14, far above fp32 rounding of
    their exp)."""
    mags = np.arange(0x3C80, 0x7F80, dtype=np.uint32)          # 2^-6 and up
    mags = mags[f32(mags.astype(np.uint16)) <= 4.0 * scale]
    pool = np.concatenate([mags, mags | 0x8000]).astype(np.uint16)
    assert pool.size >= vocab
    return rng.permutation(pool)[:vocab].astype(np.uint16)


# ---- the RNG --------------------------------------------------------------------------

def test_mt19937_64_check_value():
    """[rand.predef]: the 10000th invocation of a default-constructed mt19937_64 (seed 5489)."""
    assert O.mt19937_64_nth(5489, 10000) == 9981545732273789042


@pytest.mark.parametrize("state", [0, 1, 5489, 12345, 999, 2 ** 64 - 1, 0x9E3779B97F4A7C15])
def test_canonical_is_the_first_output_over_2_64(state):
    """generate_canonical<float, 24> of a 64-bit engine takes one output x and returns
    fp32(x) / 2^64 (below 1)."""
    x = O.mt19937_64_nth(state, 1)
    want = np.float32(np.float32(x) / np.float32(2.0 ** 64))
    if want >= 1.0:
        want = np.nextafter(np.float32(1.0), np.float32(0.0))
    got = np.float32(O.canonical(state))
    assert got.view(np.uint32) == want.view(np.uint32)
    assert 0.0 <= got < 1.0


def test_uniform_real_is_canonical_scaled():
    """uniform_real_distribution<float>(0, b) = canonical * b (libstdc++), the product the
    draw kernel forms with its kept total, for totals from 1 to the largest vocabularies."""
    state = 12345
    for i in range(300):
        b = np.float32([1.0, 2.5, 7.25, 1000.125, 262143.0, 3.3e6][i % 6] * (1 + i / 1000))
        want = np.float32(np.float32(O.canonical(state)) * b)
        got = np.float32(O.stl_uniform_real(state, float(b)))
        assert got.view(np.uint32) == want.view(np.uint32), (state, b)
        state = O.advance_rng(state)


def test_rng_advance_is_the_decode_loops_lcg():
    """model.cc:944: state * 6364136223846793005 + 1442695040888963407 mod 2^64."""
    s = 7
    for _ in range(5):
        s2 = O.advance_rng(s)
        assert s2 == (s * 6364136223846793005 + 1442695040888963407) % 2 ** 64
        s = s2
    assert O.advance_rng(2 ** 64 - 1) == (-6364136223846793005 + 1442695040888963407) % 2 ** 64


# ---- det_exp --------------------------------------------------------------------------

def test_det_exp_within_two_ulp():
    xs = np.concatenate([np.linspace(-85.999, 0.0, 40001, dtype=np.float32),
                         -np.float32(2.0) ** -np.arange(1, 40, dtype=np.float32)])
    worst = 0.0
    for x in xs:
        got = np.float32(O.det_exp(float(x)))
        ref = math.exp(float(x))
        ulp = float(np.spacing(np.float32(ref)))
        worst = max(worst, abs(float(got) - ref) / ulp)
    print(f"det_exp: worst {worst:.3f} ulp over {xs.size} points")
    assert worst <= 2.0
    assert O.det_exp(0.0) == 1.0 and O.det_exp(-0.0) == 1.0
    assert O.det_exp(-86.0) == 0.0 and O.det_exp(-1000.0) == 0.0 and O.det_exp(float("-inf")) == 0.0
    assert O.det_exp(float("nan")) == 0.0
    assert O.det_exp(-85.99) > 2.0 ** -126     # a normal number


def _exp_variant(x, low=1.42860677e-06):
    """det_exp's operations in numpy float32, with the low part of ln 2 as a parameter."""
    f = np.float32
    kf = f(np.rint(f(x) * f(1.44269502)))
    r = f(f(f(x) - f(kf * f(0.693145751953125))) - f(kf * f(low)))
    p = f(1.98412701e-04)
    for c in (1.38888892e-03, 8.33333377e-03, 4.16666679e-02, 1.66666672e-01, 0.5, 1.0, 1.0):
        p = f(f(p * r) + f(c))
    return float(f(p * f(2.0 ** int(kf))))


def test_det_exp_planted_error_is_caught():
    """The restatement in numpy reproduces det_exp bit for bit; the same with the low part of
    ln 2 dropped (a plausible slip) misses the 2-ulp bar by far at large |x|."""
    for x in (-0.34, -1.0, -10.5, -42.0, -80.0):
        assert _exp_variant(x) == O.det_exp(x)
    x = -80.0
    ref = math.exp(x)
    assert abs(_exp_variant(x, low=0.0) - ref) / float(np.spacing(np.float32(ref))) > 100.0


# ---- kept sets --------------------------------------------------------------------------

CONFIGS = [
    (1.0, 0, 0.0, 0.0), (0.7, 40, 0.0, 0.0), (1.3, 0, 0.9, 0.0), (1.0, 0, 0.0, 0.05),
    (0.8, 50, 0.95, 0.02), (2.0, 0, 0.5, 0.0), (0.5, 3, 0.0, 0.0), (1.0, 0, 1.0, 0.0),
    (1.0, 0, float("nan"), 0.0),
]


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("kind", ["distinct", "ties"])
def test_kept_prefix_matches_float64_softmax(cfg, kind):
    """The kept prefix equals the float64 one where every filter boundary is clear by 1e-5;
    otherwise the two differ only by tokens of total probability below 1e-5 (top_p = 1 is
    always such a case: the fp32 running mass reaches 1 where rounding decides)."""
    T, k, p, m = cfg
    rng = np.random.default_rng(11)
    exact = 0
    for trial in range(12):
        vocab = int(rng.integers(20, 2000))
        if kind == "distinct":
            bits = distinct_row(rng, vocab, 2.0)
        else:
            bits = bf16(rng.integers(-6, 7, vocab) * 0.5)
        n, order, margin, prob = kept_n_float64(bits, T, k, p, m)
        tok, logit, kept = O.sample_stochastic(bits, T, k, p, m, canon=0.37)
        if margin >= 1e-5:
            assert kept == n, (trial, vocab, kept, n)
            exact += 1
        else:
            assert prob[min(kept, n):max(kept, n)].sum() < 1e-5, (trial, kept, n)
        assert tok in set(order[:kept].tolist()), (trial, tok)
        assert logit == float(f32(bits[tok:tok + 1])[0])
    if not p == 1.0:
        assert exact >= 8


def test_tied_boundary_keeps_lowest_indices():
    """Equal values at a top-k cut: the lower indices are kept (the defined tie order)."""
    bits = bf16([1.0, 3.0, 2.0, 3.0, 2.0, 2.0, 3.0, 0.5])
    # order: 3.0 at 1, 3, 6; 2.0 at 2, 4, 5; ... top_k = 4 keeps 1, 3, 6 and 2
    seen = set()
    for i in range(400):
        tok, _, kept = O.sample_stochastic(bits, 1.0, 4, 0.0, 0.0, canon=(i + 0.5) / 400)
        assert kept == 4
        seen.add(tok)
    assert seen == {1, 3, 6, 2}


@pytest.mark.parametrize("cfg", CONFIGS[:8])
def test_matches_reference_host_sampler(cfg):
    """Same RNG state, rows of distinct values: the kept mask and the token of the
    reference's host algorithm (libstdc++). Kept sets may differ only at a top-p boundary,
    by tokens of total probability below 1e-5 (the two fp32 running masses round apart);
    tokens only where u lies within 2e-6 of the kept total from the running sum between
    the two tokens."""
    T, k, p, m = cfg
    rng = np.random.default_rng(5)
    equal_tok = equal_set = trials = 0
    for trial in range(40):
        vocab = int(rng.integers(2, 1500))
        bits = distinct_row(rng, vocab, float(rng.choice([0.5, 2.0, 5.0])))
        state = int(rng.integers(0, 2 ** 63))
        ref_tok, ref_kept, u = O.stl_sample_stochastic(f32(bits), T, k, p, m, state)
        tok, _, n = O.sample_stochastic(bits, T, k, p, m, canon=O.canonical(state))
        _, order, _, prob = kept_n_float64(bits, T, 0, 0.0, 0.0)
        mine = np.zeros(vocab, bool)
        mine[order[:n]] = True
        trials += 1
        if (mine == ref_kept).all():
            equal_set += 1
        else:
            assert 0 < p <= 1, trial
            rank_prob = np.zeros(vocab)
            rank_prob[order] = prob
            assert rank_prob[mine != ref_kept].sum() < 1e-5, (trial, int(ref_kept.sum()), n)
        if tok == ref_tok:
            equal_tok += 1
        else:
            both = mine & ref_kept
            w = np.where(both, np.exp(f32(bits).astype(np.float64) / T - f32(bits).max() / T), 0.0)
            c = np.cumsum(w)
            edge = c[min(tok, ref_tok)]
            assert abs(edge - u) <= 2e-6 * c[-1], (trial, tok, ref_tok, edge, u)
    print(f"{trials} rows: kept sets equal {equal_set}, tokens equal {equal_tok}")
    assert equal_tok >= trials - 2


@pytest.mark.parametrize("scale,T,k,p,m", [(1.5, 0.8, 25, 0.9, 0.01), (0.5, 1.5, 25, 0.0, 0.0),
                                           (0.5, 1.0, 0, 0.8, 0.0)])
def test_frequencies_match_the_filtered_softmax(scale, T, k, p, m):
    """20,000 draws (RNG states 0..19999) over one row: chi-square against the float64
    filtered softmax."""
    from scipy import stats
    rng = np.random.default_rng(3)
    bits = distinct_row(rng, 60, scale)
    n, order, _, _ = kept_n_float64(bits, T, k, p, m)
    t = f32(bits)[order[:n]].astype(np.float64) / T
    prob = np.exp(t - t.max())
    prob /= prob.sum()
    counts = np.zeros(bits.size, np.int64)
    draws = 20000
    for s in range(draws):
        tok, _, kept = O.sample_stochastic(bits, T, k, p, m, canon=O.canonical(s))
        counts[tok] += 1
    assert counts[order[n:]].sum() == 0
    chi2, pval = stats.chisquare(counts[order[:n]], prob * draws)
    print(f"kept {n}: chi2 {chi2:.1f}, p {pval:.3g}")
    assert pval > 1e-4


# ---- special rows and closed forms ------------------------------------------------------

def test_top_k_one_and_tiny_temperature_are_greedy():
    """sampler_test.cc:196-204: top_k = 1 forces the argmax (its first index) whatever the
    seed; a temperature of 1e-3 over values at least 0.125 apart leaves weight only on the
    largest value (one of its indices; the greedy one where it is unique)."""
    rng = np.random.default_rng(8)
    for _ in range(20):
        bits = bf16(rng.integers(-50, 50, 500) * 0.125)
        gtok, gval, _ = O.sample_greedy(bits)
        unique = int((f32(bits) == gval).sum()) == 1
        for s in (0, 1, 999, 12345):
            c = O.canonical(s)
            assert O.sample_stochastic(bits, 1.0, 1, 0.0, 0.0, canon=c)[0] == gtok
            tok = O.sample_stochastic(bits, 1e-3, 0, 0.0, 0.0, canon=c)[0]
            assert f32(bits[tok:tok + 1])[0] == gval
            if unique:
                assert tok == gtok


def test_zero_uniform_draws_index_zero():
    """u = 0: the reference's first running sum already reaches it (index 0, kept or not)."""
    bits = bf16([-5.0, 1.0, 2.0, 3.0])
    assert O.sample_stochastic(bits, 1.0, 1, 0.0, 0.0, canon=0.0)[0] == 0


def test_infinite_temperature_is_uniform_closed_form():
    """temperature = +inf: t = logit * 0 = 0 for every finite logit, each weight exp(0) = 1,
    sz = vocab and the draw is the first i with u <= i + 1: ceil(vocab * U) - 1."""
    rng = np.random.default_rng(4)
    bits = bf16(rng.standard_normal(777) * 3)
    for s in range(50):
        c = O.canonical(s)
        u = np.float32(np.float32(777.0) * np.float32(c))
        want = max(int(math.ceil(float(u))) - 1, 0)
        assert O.sample_stochastic(bits, float("inf"), 0, 0.0, 0.0, canon=c)[0] == want
        ref = O.stl_sample_stochastic(f32(bits), float("inf"), 0, 0.0, 0.0, s)[0]
        assert ref == want


@pytest.mark.parametrize("case", ["all_neg_inf", "nan", "pos_inf", "tiny_temp_neg", "tiny_temp_pos",
                                  "inf_temp_neg_inf", "overflow"])
def test_non_finite_rows_follow_the_reference(case):
    """The reference's arithmetic on these rows (filters off, where its sorts are defined):
    a NaN draw total gives the last index, a zero total index 0. Compared with the restated
    host sampler and the expected index."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(300) * 2).astype(np.float32)
    T = 1.0
    if case == "all_neg_inf":
        x[:] = -np.inf
        want = 0
    elif case == "nan":
        x[17] = np.nan
        want = 299
    elif case == "pos_inf":
        x[40] = np.inf
        want = 299
    elif case == "tiny_temp_neg":       # 1/1e-45 = +inf over negative values: all -inf, total 0
        x = -np.abs(x) - 0.5
        T = 1e-45
        want = 0
    elif case == "tiny_temp_pos":       # +inf - +inf = NaN
        T = 1e-45
        want = 299
    elif case == "inf_temp_neg_inf":    # -inf * 0 = NaN
        x[3] = -np.inf
        T = float("inf")
        want = 299
    else:                               # 3e38 * 2 overflows to +inf
        x[5] = 3.0e38
        T = 0.5
        want = 299
    bits = bf16(x)
    tok, logit, kept = O.sample_stochastic(bits, T, 0, 0.0, 0.0, canon=O.canonical(77))
    ref = O.stl_sample_stochastic(f32(bits), T, 0, 0.0, 0.0, 77)[0]
    assert tok == want == ref, (case, tok, want, ref)
    assert kept == 0
    assert np.float32(logit).view(np.uint32) == f32(bits[tok:tok + 1]).view(np.uint32)[0]


@pytest.mark.parametrize("vocab", [1, 2, 1023, 1024, 1025, 262144])
def test_sizes_and_chunk_edges(vocab):
    """Rows shorter than, equal to and longer than the 1024 chunks; the draw's token is in
    the kept prefix and the full 262144-wide row agrees with the reference host sampler's
    kept set."""
    rng = np.random.default_rng(vocab)
    bits = bf16(rng.standard_normal(vocab) * 4)
    for s in range(3):
        tok, _, n = O.sample_stochastic(bits, 0.9, 64, 0.95, 0.0, canon=O.canonical(s))
        order = order_of(bits)
        assert tok in set(order[:n].tolist())
    if vocab == 262144:
        ref_tok, ref_kept, _ = O.stl_sample_stochastic(f32(bits), 0.9, 64, 0.0, 0.0, 9)
        tok, _, n = O.sample_stochastic(bits, 0.9, 64, 0.0, 0.0, canon=O.canonical(9))
        assert n == int(ref_kept.sum()) == 64
