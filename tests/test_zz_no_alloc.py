"""hyp_qmatmul_noalloc, the entry point that allocates nothing, against hyp_qmatmul.

Both are called through the C ABI (ctypes). The no-allocation form runs the same kernels
and k splits, with the split-k partial sums in the library's fixed device scratch, so its
output must equal hyp_qmatmul's bit for bit. Two calls in a row share the scratch, the
second with a smaller input; a call whose partials exceed the scratch is refused before
anything runs; and the entry can be recorded into a graph and replayed.
"""
import ctypes
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


def _noalloc(w, x, m, y, stream):
    hy.check(hy.lib().hyp_qmatmul_noalloc(w.handle, x.ptr, m, y.ptr, stream.handle), "hyp_qmatmul_noalloc")


def _both(stream, n, k, m, seed):
    """(hyp_qmatmul output, hyp_qmatmul_noalloc output, x, host weights) for one shape."""
    w, s, b = syn.q4_weights(n, k, seed=seed)
    qw = hy.QWeight.from_host(w, s, b)
    x = syn.activations(m, k, seed=seed + 1)
    xd = hy.DeviceArray.from_host(x, stream)
    ya = hy.DeviceArray((m, n), np.uint16)
    yb = hy.DeviceArray((m, n), np.uint16)
    hy.qmatmul(qw, xd, m, ya, stream)
    _noalloc(qw, xd, m, yb, stream)
    out = ya.to_host(stream), yb.to_host(stream)
    for a in (qw, xd, ya, yb):
        a.close()
    return out[0], out[1], x, (w, s, b)


def test_noalloc_equals_qmatmul_two_calls_second_smaller(stream):
    # down [3840, 15360] at m = 2048: k split 2 ways, 62.9 MB of partials in the scratch;
    # then k [2048, 3840] at m = 512: split 4 ways, 16.8 MB, over the first call's contents.
    for n, k, m, seed in ((3840, 15360, 2048, 3000), (2048, 3840, 512, 3010), (15360, 3840, 1, 3020)):
        say(f"noalloc [{n},{k}] m={m}")
        ya, yb, x, wsb = _both(stream, n, k, m, seed)
        np.testing.assert_array_equal(yb, ya, err_msg=f"[{n},{k}] m={m}")
        rows = np.unique(np.array([0, m // 3, m - 1]))
        truth = O.qmatmul_f64(x[rows], *wsb)
        assert syn.sig_rel(syn.bf16_to_f32(yb[rows]), truth) <= 1e-2


def test_noalloc_refuses_partials_beyond_the_scratch(stream):
    # [4608, 65536] at m = 1024 splits k 4 ways: 75.5 MB of partials > 64 MiB. The call is
    # refused and leaves y untouched; hyp_qmatmul (which allocates) still runs it.
    n, k, m = 4608, 65536, 1024
    say(f"noalloc oversize [{n},{k}] m={m}")
    qw = hy.QWeight.from_host(*syn.q4_weights(n, k, seed=3030))
    xd = hy.DeviceArray.from_host(syn.activations(m, k, seed=3031), stream)
    sentinel = np.full((m, n), 0x7FC1, np.uint16)
    yd = hy.DeviceArray.from_host(sentinel, stream)
    with pytest.raises(hy.HypError) as e:
        _noalloc(qw, xd, m, yd, stream)
    assert e.value.status_name == "INVALID_ARGUMENT"
    assert "scratch" in str(e.value)
    stream.synchronize()
    np.testing.assert_array_equal(yd.to_host(stream), sentinel)
    hy.qmatmul(qw, xd, m, yd, stream)
    assert not np.array_equal(yd.to_host(stream), sentinel)
    for a in (qw, xd, yd):
        a.close()


def test_noalloc_records_into_a_graph(stream):
    """The split-k prefill call recorded into a graph (hyp_qmatmul refuses capture on its
    GEMM path): replays with eager work between them all equal the eager output."""
    n, k, m = 2048, 3840, 512
    w, s, b = syn.q4_weights(n, k, seed=3040)
    qw = hy.QWeight.from_host(w, s, b)
    xd = hy.DeviceArray.from_host(syn.activations(m, k, seed=3041), stream)
    y = hy.DeviceArray((m, n), np.uint16)
    other = hy.DeviceArray((m, n), np.uint16)
    hy.qmatmul(qw, xd, m, y, stream)
    eager = y.to_host(stream)
    _noalloc(qw, xd, m, other, stream)         # first use on this device outside the capture
    stream.synchronize()
    with hy.Graph.capture(stream) as graph:
        _noalloc(qw, xd, m, y, stream)
    for rep in range(3):
        _noalloc(qw, xd, m, other, stream)     # eager use of the same scratch between replays
        stream.synchronize()
        y.upload(np.zeros((m, n), np.uint16), stream)
        graph.launch(stream)
        stream.synchronize()
        np.testing.assert_array_equal(y.to_host(stream), eager, err_msg=f"replay {rep}")
    graph.close()
    for a in (qw, xd, y, other):
        a.close()
