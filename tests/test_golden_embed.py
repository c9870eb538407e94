"""MLX's dequantize rounding, pinned by the reference's own 12B embed golden.

The golden is `ForwardPass::embed` of ten tokens on the real 12B
(native/hyperion_mlx/src/forward.cc:126-131, weights_loader.cc:52-69), which the reference's
native/hyperion_mlx/tests/forward_12b_test.cc:218 holds its forward to. `embed_fit` recovers,
per 64-element group, which bf16 rounding of the dequantize can produce the golden's values
(see its docstring for the search); these tests decide the rounding from it and then hold the
oracle to the golden bit for bit.
"""
from types import SimpleNamespace

import numpy as np
import pytest

import embed_fit as F
import oracle as O


@pytest.fixture(scope="module")
def golden():
    return F.load()


@pytest.fixture(scope="module")
def fitted(golden):
    return F.fitted_rows(golden[1])


def test_golden_decides_single_rounding(golden):
    """Every one of the 600 groups fits bf16(s*q + b); at least 500 do not fit the op-composed
    bf16(bf16(s*q) + b), and none fits only that one."""
    ids, e = golden
    assert e.shape == (10, 3840) and ids.tolist()[:3] == [818, 3823, 8864]
    c = F.classify(e)
    print(f"groups fitting: {c}")
    assert c["neither"] == 0 and c["double"] == 0
    assert c["single"] + c["both"] == 600
    assert c["single"] >= 500


def test_search_rejects_a_planted_wrong_value(golden):
    """The search is strict: one golden value moved by one bf16 ulp in a group makes that group
    fit neither rounding (checked on the first 20 groups of row 0)."""
    e = golden[1][0].copy()
    for g in range(20):
        obs = e[g * 64:(g + 1) * 64].copy()
        i = int(np.argmax(F.from_bf16(obs) != 0))
        obs[i] += 1
        assert F.fit_group(obs, "single") is None, g


def test_oracle_dequantize_reproduces_the_golden(golden, fitted):
    """The oracle's default dequantize, times bf16(sqrt(3840)), returns the golden's bits from
    the recovered Q4 rows; its op-composed mode does not."""
    _, e = golden
    w, s, b = fitted
    got = O.scale(O.dequantize(w, s, b), float(np.sqrt(np.float32(3840))))
    np.testing.assert_array_equal(got, e)
    other = O.scale(O.dequantize(w, s, b, mode=0), float(np.sqrt(np.float32(3840))))
    bad_groups = int((other != e).reshape(10, 60, 64).any(-1).sum())
    assert bad_groups >= 500, bad_groups


def test_decoder_oracle_embed_reproduces_the_golden(golden, fitted):
    """DecoderOracle.embed (the decoder tests' reference) gathers rows by id and gives the
    golden's bits."""
    ids, e = golden
    w, s, b = fitted
    vocab = int(ids.max()) + 1
    table = {
        ".weight": np.zeros((vocab, w.shape[1]), np.uint32),
        ".scales": np.zeros((vocab, s.shape[1]), np.uint16),
        ".biases": np.zeros((vocab, b.shape[1]), np.uint16),
    }
    for i, t in enumerate(ids):
        table[".weight"][t], table[".scales"][t], table[".biases"][t] = w[i], s[i], b[i]
    ns = SimpleNamespace(hidden=3840, _t=lambda name: table[name[len("embed_tokens"):]])
    np.testing.assert_array_equal(O.DecoderOracle.embed(ns, ids), e)
