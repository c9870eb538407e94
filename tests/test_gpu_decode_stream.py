"""GPU parity of the full decode weight stream (the 48-layer synthetic 12B plus the tied
LM head [262144, 3840]) and of the 12B global-layer projection shapes.

Bars (stated per test):
  * graph replay of a whole decode step: bit-equal to the eager launch sequence;
  * each projection of layers 0 and 47, on the kernel's own inputs: within half a bf16
    ulp of the fp64 truth plus 2^-18 * max|truth| (fp32 accumulation), and
    sig_rel = max|d| / max|truth| <= 1e-2 (forward_12b_test.cc:148-161);
  * the fused gate/up GELU: sig_rel <= 1e-2 against the oracle's bf16 GELU chain applied
    to the fp64 gate and up;
  * the softcap LM head on all 262144 rows: sig_rel <= 1e-2 against 30 tanh(truth / 30)
    on 4096 sampled rows; against the oracle's softcap of the plain head output at most
    2 bf16 ulps on at most 0.1% of the logits; device greedy sampling bit-exact against
    the oracle's restatement of forward.cc:162-189 on the same logits.
"""
import sys

import numpy as np
import pytest

import hyperion_amd as hy
import oracle as O
from hyperion_amd import decode_chain as dc
from hyperion_amd import synthetic as syn
from test_gpu_parity import assert_within_bf16_rounding, ulp_diff

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a, stream):
    return hy.DeviceArray.from_host(a, stream)


@pytest.fixture(scope="module")
def model(stream):
    say(f"building the synthetic decode model: {syn.NUM_LAYERS} layers + LM head [{syn.VOCAB},{syn.HIDDEN}]")
    mdl = dc.DecodeModel(hy, syn.NUM_LAYERS, log=say)
    yield mdl
    mdl.close()


@pytest.fixture(scope="module")
def head_host():
    say("generating the LM head weights on the host")
    return dc.head_weights()


def _snapshot(b, stream):
    return {name: getattr(b, name).to_host(stream) for name in ("h", "q", "k", "v", "o", "g", "logits", "samples")}


@pytest.mark.parametrize("m", [1, 4])
def test_decode_step_graph_replay_equals_eager(model, stream, m):
    """One whole decode step (192 layer launches + renormalise, softcap head, sampling)
    captured into a graph and replayed three times, with eager work between replays:
    every buffer equals the eager launch sequence's bit for bit."""
    h0 = syn.activations(m, syn.HIDDEN, seed=77 + m)
    b = dc.StepBuffers(hy, m, h0, stream)
    say(f"decode step m={m}: eager")
    dc.decode_step(model, m, b, stream)
    eager = _snapshot(b, stream)
    assert np.all(np.isfinite(syn.bf16_to_f32(eager["h"])))
    b.h.upload(h0, stream)
    with hy.Graph.capture(stream) as graph:
        dc.decode_step(model, m, b, stream)
    for rep in range(3):
        b.h.upload(h0, stream)
        scratch = hy.DeviceArray((m, 2048), np.uint16)
        hy.qmatmul(model.layers[0]["k"], b.h, m, scratch, stream)   # eager work between replays
        stream.synchronize()
        say(f"decode step m={m}: replay {rep}")
        graph.launch(stream)
        stream.synchronize()
        got = _snapshot(b, stream)
        for name, want in eager.items():
            np.testing.assert_array_equal(got[name], want, err_msg=f"m={m} replay {rep}: {name}")
        scratch.close()
    graph.close()
    b.close()


def _check_projection(y, x, wsb, what):
    truth = O.qmatmul_f64(x, *wsb)
    rel = syn.sig_rel(syn.bf16_to_f32(y), truth)
    assert rel <= 1e-2, f"{what}: sig_rel {rel:.3e}"
    assert_within_bf16_rounding(y, truth, what)
    return rel


@pytest.mark.parametrize("m", [1, 4])
def test_decode_layers_0_and_47_against_fp64(model, stream, m):
    """Layers 0 and 47 of the eager stream: every launch's output against the fp64 truth
    on the inputs the kernel actually read (the previous launch's device output)."""
    h0 = syn.activations(m, syn.HIDDEN, seed=177 + m)
    b = dc.StepBuffers(hy, m, h0, stream)
    xn = hy.DeviceArray((m, syn.HIDDEN), np.uint16)
    checked = (0, syn.NUM_LAYERS - 1)
    for li, proj in enumerate(model.layers):
        if li in checked:
            hy.rms_normalize(b.h, m, syn.HIDDEN, xn, stream, eps=dc.RMS_EPS)
            x_norm = xn.to_host(stream)
        dc.decode_layer(hy, proj, m, b, stream)
        if li not in checked:
            continue
        say(f"layer {li} m={m}: oracle checks")
        out = _snapshot(b, stream)
        for name in ("q", "k", "v"):
            rel = _check_projection(out[name], x_norm, dc.layer_weights(li, name), f"layer {li} {name} m={m}")
            say(f"  {name}: sig_rel {rel:.2e}")
        rel = _check_projection(out["o"], out["q"], dc.layer_weights(li, "o"), f"layer {li} o m={m}")
        say(f"  o: sig_rel {rel:.2e}")
        gate = O.qmatmul_f64(out["o"], *dc.layer_weights(li, "gate"))
        up = O.qmatmul_f64(out["o"], *dc.layer_weights(li, "up"))
        chain = O.gelu_tanh_mul(syn.bf16_bits(gate.astype(np.float32)), syn.bf16_bits(up.astype(np.float32)))
        rel = syn.sig_rel(syn.bf16_to_f32(out["g"]), syn.bf16_to_f32(chain))
        say(f"  gate/up gelu: sig_rel {rel:.2e}")
        assert rel <= 1e-2, f"layer {li} gate/up m={m}"
        rel = _check_projection(out["h"], out["g"], dc.layer_weights(li, "down"), f"layer {li} down m={m}")
        say(f"  down: sig_rel {rel:.2e}")
    xn.close()
    b.close()


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_lm_head_full_vocab_softcap_and_sampling(model, head_host, stream, m):
    """The tied head [262144, 3840] with softcap 30 at decode batch m (the m >= 2 launches
    take the head kernel's looping form): sampled rows against the fp64 truth, the whole
    row against the oracle's softcap of the plain launch, then device greedy sampling
    and its top-8 sidecar against the oracle on the same capped logits."""
    w, s, b = head_host
    x = syn.activations(m, syn.HIDDEN, seed=900 + m)
    xd = dev(x, stream)
    capped_d = hy.DeviceArray((m, syn.VOCAB), np.uint16)
    plain_d = hy.DeviceArray((m, syn.VOCAB), np.uint16)
    say(f"lm head m={m}")
    hy.qmatmul(model.embed, xd, m, capped_d, stream, softcap=dc.SOFTCAP)
    hy.qmatmul(model.embed, xd, m, plain_d, stream)
    capped = capped_d.to_host(stream)
    plain = plain_d.to_host(stream)
    rng = np.random.default_rng(910 + m)
    rows = np.sort(rng.choice(syn.VOCAB, size=4096, replace=False))
    rows[0], rows[-1] = 0, syn.VOCAB - 1
    truth = O.qmatmul_f64(x, w[rows], s[rows], b[rows])
    assert_within_bf16_rounding(plain[:, rows], truth, f"head plain m={m}")
    cap_truth = dc.SOFTCAP * np.tanh(truth / dc.SOFTCAP)
    rel = syn.sig_rel(syn.bf16_to_f32(capped[:, rows]), cap_truth)
    say(f"  sampled rows: capped sig_rel {rel:.2e} (bound 1e-2)")
    assert rel <= 1e-2
    # The head launch (one wave per tile) and the plain launch (k split over waves) sum the
    # same fp32 terms in another order; each is within half a bf16 ulp + 2^-18 max|y| of the
    # truth, so after the cap they may differ by up to two ulps of the value plus 2^-17 of
    # the largest logit (near-zero logits can then be many ulps apart in relative terms).
    ref = O.softcap(plain, dc.SOFTCAP)
    d = ulp_diff(capped, ref)
    diff = np.abs(syn.bf16_to_f32(capped).astype(np.float64) - syn.bf16_to_f32(ref))
    ulp = np.abs(syn.bf16_to_f32(ref)).astype(np.float64) * 2.0**-7 + 1e-40
    bound = 2.0 * ulp + 2.0**-17 * float(np.max(np.abs(syn.bf16_to_f32(plain))))
    say(f"  capped vs oracle softcap of the plain launch: {np.count_nonzero(d)} differ, worst "
        f"{float(np.max(diff / bound)):.2f} of the bound")
    assert np.all(diff <= bound)
    assert np.count_nonzero(d) <= d.size // 1000
    out = hy.DeviceArray((m, 3), np.uint32)
    hy.sample_greedy(capped_d, m, syn.VOCAB, out, stream)
    got = hy.greedy_samples(out, m, stream)
    for r in range(m):
        want = O.sample_greedy(capped[r])
        assert (got[r][0], got[r][2]) == (want[0], want[2]), f"row {r}: {got[r]} vs {want}"
        assert np.float32(got[r][1]).tobytes() == np.float32(want[1]).tobytes()
    topk = hy.DeviceArray((m, 20), np.uint32)
    hy.sample_greedy_topk(capped_d, m, syn.VOCAB, topk, stream)
    for r, t in enumerate(hy.topk_samples(topk, m, stream)):
        cnt, ids, vals = O.sample_topk(capped[r])
        assert (t["token_id"], t["near_tie"], t["count"]) == (got[r][0], got[r][2], cnt)
        np.testing.assert_array_equal(t["ids"], ids, err_msg=f"row {r}")
        np.testing.assert_array_equal(t["logprobs"].view(np.uint32), vals.view(np.uint32))
    for a in (xd, capped_d, plain_d, out, topk):
        a.close()


# The global (K = V) layers of the real 12B: q [8192, 3840], k [512, 3840], no v_proj, and
# o [3840, 8192] (forward.cc:403-412; golden shapes layer_05_qproj [1,10,8192], kproj
# [1,10,512]). o's k = 8192 changes the decode kernel's x staging and split choice.
GLOBAL_SHAPES = {"q": (8192, 3840), "k": (512, 3840), "o": (3840, 8192)}


@pytest.mark.parametrize("m", [1, 4, 512, 2048])
def test_global_layer_shapes(stream, m):
    rng = np.random.default_rng(2000 + m)
    for i, (name, (n, k)) in enumerate(GLOBAL_SHAPES.items()):
        say(f"global {name} [{n},{k}] m={m}")
        w, s, b = syn.q4_weights(n, k, seed=2100 + i)
        x = syn.activations(m, k, seed=2110 + i)
        qw = hy.QWeight.from_host(w, s, b)
        xd = dev(x, stream)
        yd = hy.DeviceArray((m, n), np.uint16)
        hy.qmatmul(qw, xd, m, yd, stream)
        y = yd.to_host(stream)
        if m <= 4:
            _check_projection(y, x, (w, s, b), f"global {name} m={m}")
        else:
            rows = np.sort(rng.choice(m, size=12, replace=False))
            rows[0], rows[-1] = 0, m - 1
            assert_within_bf16_rounding(y[rows], O.qmatmul_deq_f64(x[rows], w, s, b, mode=1), f"{name} m={m}")
            assert syn.sig_rel(syn.bf16_to_f32(y[rows]), O.qmatmul_f64(x[rows], w, s, b)) <= 1e-2
        for a in (qw, xd, yd):
            a.close()


@pytest.mark.parametrize("m", [1, 4])
def test_global_layer_grouped_qk(stream, m):
    """A global layer's q and k in one grouped launch with the renormalisation (count 2:
    there is no v_proj), against the fp64 truth on the normalised rows."""
    k = 3840
    ws = [syn.q4_weights(n, k, seed=2200 + i) for i, n in enumerate((8192, 512))]
    x = syn.activations(m, k, seed=2210 + m)
    qws = [hy.QWeight.from_host(*w) for w in ws]
    xd = dev(x, stream)
    xn = hy.DeviceArray((m, k), np.uint16)
    hy.rms_normalize(xd, m, k, xn, stream, eps=dc.RMS_EPS)
    x_norm = xn.to_host(stream)
    yds = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xd, m, yds, stream, rms_eps=dc.RMS_EPS)
    for (w, s, b), yd, name in zip(ws, yds, ("q", "k")):
        _check_projection(yd.to_host(stream), x_norm, (w, s, b), f"global grouped {name} m={m}")
    for a in qws + yds + [xd, xn]:
        a.close()


def test_capture_refuses_allocating_calls(stream):
    """While a stream captures, the calls that could allocate or clear memory return
    INVALID_ARGUMENT before enqueueing anything; the capture stays usable and the graph
    replays the calls that were recorded."""
    n, k = 256, 512
    w, s, b = syn.q4_weights(n, k, seed=2300)
    qw = hy.QWeight.from_host(w, s, b)
    up = hy.QWeight.from_host(*syn.q4_weights(n, k, seed=2301))
    x1 = dev(syn.activations(1, k, seed=2302), stream)
    xm = dev(syn.activations(300, k, seed=2303), stream)
    y1 = hy.DeviceArray((1, n), np.uint16)
    ym = hy.DeviceArray((300, n), np.uint16)
    hy.qmatmul(qw, x1, 1, y1, stream)
    eager = y1.to_host(stream)
    y1.fill_zero(stream)
    stream.synchronize()
    refused = []
    with hy.Graph.capture(stream) as graph:
        hy.qmatmul(qw, x1, 1, y1, stream)
        for what, fn in (
                ("memset", lambda: ym.fill_zero(stream)),
                ("qmatmul m=300", lambda: hy.qmatmul(qw, xm, 300, ym, stream)),
                ("group m=300", lambda: hy.qmatmul_group([qw], xm, 300, [ym], stream)),
                ("group rmsnorm m=300", lambda: hy.qmatmul_group([qw], xm, 300, [ym], stream, rms_eps=1e-6)),
                ("gate/up m=300", lambda: hy.qmlp_gate_up_gelu(qw, up, xm, 300, ym, stream))):
            with pytest.raises(hy.HypError) as e:
                fn()
            assert e.value.status_name == "INVALID_ARGUMENT", what
            assert "capturing" in str(e.value), what
            refused.append(what)
    assert len(refused) == 5
    for _ in range(2):
        y1.fill_zero(stream)
        graph.launch(stream)
        stream.synchronize()
        np.testing.assert_array_equal(y1.to_host(stream), eager)
    graph.close()
    for a in (qw, up, x1, xm, y1, ym):
        a.close()


# ---------------------------------------------------------------- decode-step program

def _zero(arrays, stream):
    for a in arrays:
        a.upload(np.zeros(a.shape, a.dtype), stream)


def _program_vs_eager(model, layers, m, stream, seed, reps=2):
    """Run `layers` layers of the model as a step program and as the eager launch sequence
    from the same input; every buffer must be equal bit for bit, on every run."""
    h0 = syn.activations(m, syn.HIDDEN, seed=seed)
    b = dc.StepBuffers(hy, m, h0, stream)
    for proj in model.layers[:layers]:
        dc.decode_layer(hy, proj, m, b, stream)
    eager = {name: getattr(b, name).to_host(stream) for name in ("h", "q", "k", "v", "o", "g")}
    sub = dc.DecodeModel.__new__(dc.DecodeModel)
    sub.hy, sub.layers = hy, model.layers[:layers]
    prog = dc.layer_program(sub, m, b)
    for rep in range(reps):
        b.h.upload(h0, stream)
        _zero((b.q, b.k, b.v, b.o, b.g), stream)
        say(f"step program: {layers} layers m={m} run {rep}")
        prog.run(stream)
        stream.synchronize()
        prog.check()
        for name, want in eager.items():
            np.testing.assert_array_equal(getattr(b, name).to_host(stream), want,
                                          err_msg=f"{layers} layers m={m} run {rep}: {name}")
    prog.close()
    b.close()


@pytest.mark.parametrize("m", [1, 4])
def test_step_program_two_layers_equals_eager(model, stream, m):
    _program_vs_eager(model, 2, m, stream, seed=3100 + m)


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_step_program_48_layers_equals_eager(model, stream, m):
    """The whole 48-layer stack (192 ops) in one launch, three runs in a row."""
    _program_vs_eager(model, syn.NUM_LAYERS, m, stream, seed=3200 + m, reps=3)


def test_step_program_ragged_segments_and_odd_groups(stream):
    """Ops over small ragged shapes: three segments of 3, 2 and 1 row tiles (n = 40, 24, 8,
    partly empty last tiles), an odd group count (k = 192) and a gate/up pair of n = 40,
    chained through one buffer; against the per-call entry points, bit for bit."""
    k = 192
    ws = [hy.QWeight.from_host(*syn.q4_weights(n, k, seed=3300 + n)) for n in (40, 24, 8)]
    gate = hy.QWeight.from_host(*syn.q4_weights(40, k, seed=3310))
    up = hy.QWeight.from_host(*syn.q4_weights(40, k, seed=3311))
    for m in (1, 2, 3, 4):
        x0 = syn.activations(m, k, seed=3320 + m)
        x = dev(x0, stream)
        ya, yb, yc = (hy.DeviceArray((m, n), np.uint16) for n in (40, 24, 8))
        g = hy.DeviceArray((m, 40), np.uint16)
        hy.qmatmul_group(ws, x, m, [ya, yb, yc], stream, rms_eps=1e-6)
        hy.qmlp_gate_up_gelu(gate, up, x, m, g, stream)
        hy.qmatmul_group(ws[:2], x, m, [ya, yb], stream)
        want = [a.to_host(stream) for a in (ya, yb, yc, g)]
        _zero((ya, yb, yc, g), stream)
        prog = hy.StepProgram([
            (hy.STEP_QMATMUL_RMSNORM, ws, x, [ya, yb, yc], 1e-6),
            (hy.STEP_GATE_UP_GELU, [gate, up], x, [g], 0.0),
            (hy.STEP_QMATMUL, ws[:2], x, [ya, yb], 0.0),
        ], m)
        prog.run(stream)
        stream.synchronize()
        prog.check()
        for got, w, name in zip((ya, yb, yc, g), want, ("a", "b", "c", "gate/up")):
            np.testing.assert_array_equal(got.to_host(stream), w, err_msg=f"m={m} {name}")
        prog.close()
        for a in (x, ya, yb, yc, g):
            a.close()
    for q in ws + [gate, up]:
        q.close()


def test_step_program_gives_up_and_recovers(model, stream):
    """A program whose spin limit is two polls gives up at an op boundary: every
    workgroup leaves the launch, and check reports INTERNAL and resets it. A program with
    the default limit then runs the same ops correctly."""
    m = 1
    h0 = syn.activations(m, syn.HIDDEN, seed=3400)
    b = dc.StepBuffers(hy, m, h0, stream)
    sub = dc.DecodeModel.__new__(dc.DecodeModel)
    sub.hy, sub.layers = hy, model.layers[:8]
    for proj in sub.layers:
        dc.decode_layer(hy, proj, m, b, stream)
    want = b.h.to_host(stream)
    b.h.upload(h0, stream)
    hasty = dc.layer_program(sub, m, b, spin_limit=1)
    hasty.run(stream)
    stream.synchronize()
    with pytest.raises(hy.HypError) as e:
        hasty.check()
    assert e.value.status_name == "INTERNAL" and "gave up" in str(e.value)
    hasty.check()   # reset: nothing pending
    hasty.close()
    prog = dc.layer_program(sub, m, b)
    b.h.upload(h0, stream)
    prog.run(stream)
    stream.synchronize()
    prog.check()
    np.testing.assert_array_equal(b.h.to_host(stream), want)
    prog.close()
    b.close()
