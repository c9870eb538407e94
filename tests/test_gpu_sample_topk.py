"""GPU parity of the greedy epilogue's top-k sidecar (hyp_sample_greedy_topk): the
HYP_TOP_K_LOGPROBS = 8 largest post-softcap logits and their ids as the reference fills
them after its std::partial_sort (model.cc:272-288, forward.cc:203-220), with the tie order
defined by the entry point (larger value, then lower index; -0 == +0; NaN last). Bar:
count, ids and value bits equal to the oracle's restatement (oracle/q4_oracle.c
orc_sample_topk_bf16, pinned against libstdc++'s partial_sort on the CPU), and the greedy
fields equal to hyp_sample_greedy's on the same rows.
"""
import sys

import numpy as np
import pytest

import hyperion_amd as hy
import oracle as O
from hyperion_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rows(kind, rows, vocab, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":          # N(0, 36): bf16 ties in the top 9 are the rule at 262144
        return syn.bf16_bits((rng.standard_normal((rows, vocab)) * 6).astype(np.float32))
    if kind == "integers":        # heavy ties everywhere
        return syn.bf16_bits(rng.integers(-3, 4, (rows, vocab)).astype(np.float32))
    if kind == "specials":        # NaN, +-inf, -0 and +0 planted among normals
        x = syn.bf16_bits(rng.standard_normal((rows, vocab)).astype(np.float32))
        for code, frac in ((0x7FC0, 0.02), (0xFFC1, 0.01), (0x7F80, 0.002), (0xFF80, 0.02), (0x8000, 0.05),
                           (0x0000, 0.05)):
            x[rng.random((rows, vocab)) < frac] = code
        return x
    if kind == "constant":
        return np.full((rows, vocab), syn.bf16_bits(np.float32([2.5]))[0], np.uint16)
    if kind == "neg_inf":
        return np.full((rows, vocab), 0xFF80, np.uint16)
    if kind == "nan":
        return np.full((rows, vocab), 0x7FC0, np.uint16)
    if kind == "zeros":           # -0 and +0 alternating: all equal to the comparator
        x = np.zeros((rows, vocab), np.uint16)
        x[:, ::2] = 0x8000
        return x
    raise ValueError(kind)


def _check(stream, x, rows, vocab, row_offset=0, label=""):
    total = x.shape[0]
    xd = hy.DeviceArray.from_host(x, stream)
    out = hy.DeviceArray((max(rows, 1), 20), np.uint32)
    g = hy.DeviceArray((max(rows, 1), 3), np.uint32)
    hy.sample_greedy_topk(xd, rows, vocab, out, stream, row_offset=row_offset)
    hy.sample_greedy(xd, rows, vocab, g, stream, row_offset=row_offset)
    got = hy.topk_samples(out, rows, stream)
    greedy = hy.greedy_samples(g, rows, stream)
    assert total >= row_offset + rows
    for r in range(rows):
        row = x[row_offset + r]
        cnt, ids, vals = O.sample_topk(row)
        s = got[r]
        where = f"{label} row {r}"
        assert s["count"] == cnt, where
        np.testing.assert_array_equal(s["ids"], ids, err_msg=where)
        np.testing.assert_array_equal(s["logprobs"].view(np.uint32), vals.view(np.uint32), err_msg=where)
        tok, logit, tie = O.sample_greedy(row)
        assert (s["token_id"], s["near_tie"]) == (tok, tie) == (greedy[r][0], greedy[r][2]), where
        assert np.float32(s["logit"]).view(np.uint32) == np.float32(greedy[r][1]).view(np.uint32), where
        assert s["logit"] == logit, where
    for a in (xd, out, g):
        a.close()


@pytest.mark.parametrize("vocab", [262144, 262143, 4099, 1000, 9, 8, 7, 1])
@pytest.mark.parametrize("kind", ["normal", "integers", "specials"])
def test_topk_matches_oracle(stream, vocab, kind):
    rows = 2
    say(f"topk vocab={vocab} kind={kind}")
    _check(stream, _rows(kind, rows, vocab, vocab + len(kind)), rows, vocab, label=f"{kind} vocab={vocab}")


@pytest.mark.parametrize("kind", ["constant", "neg_inf", "nan", "zeros"])
@pytest.mark.parametrize("vocab", [262144, 100, 3])
def test_topk_uniform_rows(stream, kind, vocab):
    """Rows with one repeated value (or -0/+0): the lowest indices, in order."""
    say(f"topk uniform vocab={vocab} kind={kind}")
    _check(stream, _rows(kind, 1, vocab, 0), 1, vocab, label=kind)


def test_topk_many_rows_and_offsets(stream):
    """More rows than one pair of launches holds (8), and a row offset that leaves the
    rows 16-byte misaligned (odd vocab: the scalar path; even vocab misaligned too)."""
    for vocab, rows, off in ((262144, 19, 0), (262144, 5, 3), (4098, 11, 1), (262143, 3, 2)):
        say(f"topk rows={rows} vocab={vocab} offset={off}")
        x = _rows("normal", rows + off, vocab, rows * 31 + off)
        _check(stream, x, rows, vocab, row_offset=off, label=f"rows={rows} off={off}")


def test_topk_empty_row(stream):
    out = hy.DeviceArray((1, 20), np.uint32)
    out.upload(np.full((1, 20), 0xAAAAAAAA, np.uint32), stream)
    x = hy.DeviceArray((1, 8), np.uint16)
    hy.sample_greedy_topk(x, 1, 0, out, stream)
    s = hy.topk_samples(out, 1, stream)[0]
    assert (s["token_id"], s["count"], s["near_tie"]) == (0, 0, False)
    assert s["logit"] == float("-inf")
    assert not s["ids"].any() and not s["logprobs"].view(np.uint32).any()
    for a in (out, x):
        a.close()


def test_topk_in_a_graph(stream):
    """Recorded into a graph (no allocation, no memset), replayed with eager work between:
    every replay equals the eager result."""
    vocab, rows = 262144, 2
    x = _rows("normal", rows, vocab, 5)
    xd = hy.DeviceArray.from_host(x, stream)
    eager = hy.DeviceArray((rows, 20), np.uint32)
    hy.sample_greedy_topk(xd, rows, vocab, eager, stream)
    want = eager.to_host(stream)
    out = hy.DeviceArray((rows, 20), np.uint32)
    g = hy.DeviceArray((rows, 3), np.uint32)
    with hy.Graph.capture(stream) as graph:
        hy.sample_greedy_topk(xd, rows, vocab, out, stream)
    for rep in range(3):
        out.upload(np.zeros((rows, 20), np.uint32), stream)
        hy.sample_greedy(xd, rows, vocab, g, stream)       # eager work on the same workspace
        graph.launch(stream)
        stream.synchronize()
        np.testing.assert_array_equal(out.to_host(stream), want, err_msg=f"replay {rep}")
    graph.close()
    for a in (xd, eager, out, g):
        a.close()
