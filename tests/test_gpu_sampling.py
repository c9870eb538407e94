"""GPU parity of temperature sampling: hyp_sample_stochastic (ForwardPass::sample_stochastic,
forward.cc:191-322) and the sampled decoder entry points (hyp_prefill_chunk_sampled,
hyp_decode_block_sampled; model.cc:743-960).

Bars, per test:
  * the draw: token, logit bits and near_tie (0) equal to the oracle's
    (orc_sample_stochastic_bf16 with U = generate_canonical of std::mt19937_64(rng_state),
    pinned on the CPU against the reference's host sampler restated over libstdc++), and the
    top-k sidecar equal to the greedy epilogue's (orc_sample_topk_bf16): bit-exact, on rows
    with ties, +-inf, NaN and -0, at vocabularies from 1 to 262144;
  * the workspace: draws of different rows and configs in sequence, interleaved with the
    greedy epilogue, each equal to the oracle (the bins are cleared by every draw);
  * a captured draw replayed with eager work between the replays equals the eager draw;
  * NULL config or temperature 0: the greedy epilogue's 80 bytes exactly; malformed
    configs: INVALID_ARGUMENT (model.cc:234-257);
  * the decoder (the reference's tiny fixture): top_k = 1 draws the greedy tokens
    (sampler_test.cc:196-204); the same seed gives the same tokens (sampler_test.cc:155-166);
    a sampled decode block of n steps equals n one-step blocks seeded with the advanced RNG
    states (model.cc:926-944); the sampled prefill's token equals hyp_sample_stochastic over
    the LM head logits of its last hidden row with rng_state = seed (model.cc:840-841).
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


def cfg(t, k=0, p=0.0, m=0.0, seed=0):
    return hy.SamplingConfig(t, k, p, m, seed)


CONFIGS = {
    "plain": cfg(1.0),
    "topk": cfg(0.7, 40),
    "topp": cfg(1.3, 0, 0.9),
    "minp": cfg(1.0, 0, 0.0, 0.1),
    "all": cfg(0.8, 50, 0.95, 0.02),
    "greedy_k1": cfg(1.0, 1),
    "hot": cfg(5.0, 0, 0.99),
    "nan_topp": cfg(0.9, 0, float("nan")),
}


def rows_of(kind, vocab, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":       # N(0, 36) in bf16: ties in value are common
        return syn.bf16_bits((rng.standard_normal(vocab) * 6).astype(np.float32))
    if kind == "softcapped":   # an LM head's range after a 30 softcap
        return syn.bf16_bits((30 * np.tanh(rng.standard_normal(vocab) * 0.3)).astype(np.float32))
    if kind == "integers":
        return syn.bf16_bits(rng.integers(-3, 4, vocab).astype(np.float32))
    if kind == "specials":     # -inf, -0 and +0 among normals (no +inf / NaN: those draw the last)
        x = syn.bf16_bits(rng.standard_normal(vocab).astype(np.float32))
        for code, frac in ((0xFF80, 0.05), (0x8000, 0.05), (0x0000, 0.05)):
            x[rng.random(vocab) < frac] = code
        return x
    raise ValueError(kind)


class Drawer:
    def __init__(self, stream, max_vocab):
        self.stream = stream
        self.x = hy.DeviceArray((max(max_vocab, 1),), np.uint16)
        self.out = hy.DeviceArray((20,), np.uint32)

    def draw(self, bits, config, state):
        vocab = bits.size
        if vocab:
            row = np.zeros(self.x.shape, np.uint16)
            row[:vocab] = bits
            self.x.upload(row, self.stream)
        hy.sample_stochastic(self.x, vocab, config, state, self.out, self.stream)
        return hy.topk_samples(self.out, 1, self.stream)[0]

    def close(self):
        self.x.close()
        self.out.close()


def expect(bits, config, state):
    """The oracle's draw and sidecar."""
    if config is None or config.temperature == 0.0:
        tok, logit, tie = O.sample_greedy(bits)
    else:
        tok, logit, _ = O.sample_stochastic(bits, config.temperature, config.top_k, config.top_p, config.min_p,
                                            canon=O.canonical(state))
        tie = False
    cnt, ids, vals = O.sample_topk(bits)
    return tok, np.float32(logit), tie, cnt, ids, vals


def check(got, want, where):
    tok, logit, tie, cnt, ids, vals = want
    assert got["token_id"] == tok, f"{where}: token {got['token_id']} != {tok}"
    assert np.float32(got["logit"]).view(np.uint32) == logit.view(np.uint32), where
    assert got["near_tie"] == tie, where
    assert got["count"] == cnt, where
    np.testing.assert_array_equal(got["ids"], ids, err_msg=where)
    np.testing.assert_array_equal(got["logprobs"].view(np.uint32), vals.view(np.uint32), err_msg=where)


@pytest.mark.parametrize("vocab", [262144, 262143, 4099, 1025, 1024, 1000, 7, 1])
@pytest.mark.parametrize("kind", ["normal", "softcapped", "integers", "specials"])
def test_draw_matches_oracle(stream, vocab, kind):
    say(f"hyp_sample_stochastic: {kind} vocab {vocab}")
    d = Drawer(stream, vocab)
    bits = rows_of(kind, vocab, seed=vocab + len(kind))
    for name, c in CONFIGS.items():
        if c.top_k > vocab:
            continue
        for state in (0, 12345, 2 ** 64 - 1):
            check(d.draw(bits, c, state), expect(bits, c, state), f"{kind} {vocab} {name} state {state}")
    d.close()


@pytest.mark.parametrize("case", ["all_neg_inf", "nan", "pos_inf", "tiny_temp", "inf_temp_neg_inf", "overflow",
                                  "inf_temp"])
def test_non_finite_rows(stream, case):
    """+inf / NaN scaled logits draw the last index, no finite scaled logit index 0, as the
    reference's arithmetic gives (the oracle is pinned to it on the CPU)."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(5000) * 2).astype(np.float32)
    t = 1.0
    if case == "all_neg_inf":
        x[:] = -np.inf
    elif case == "nan":
        x[17] = np.nan
    elif case == "pos_inf":
        x[4000] = np.inf
    elif case == "tiny_temp":
        t = 1e-45
    elif case == "inf_temp_neg_inf":
        x[3] = -np.inf
        t = float("inf")
    elif case == "overflow":
        x[5] = 3.0e38
        t = 0.5
    else:
        t = float("inf")
    bits = syn.bf16_bits(x)
    d = Drawer(stream, bits.size)
    for state in (1, 77):
        c = cfg(t, 0, 0.0, 0.0)
        check(d.draw(bits, c, state), expect(bits, c, state), f"{case} state {state}")
    d.close()


def test_many_states_small_row(stream):
    """2,000 RNG states over one row: every draw equal to the oracle's."""
    rng = np.random.default_rng(21)
    bits = syn.bf16_bits((rng.standard_normal(300) * 1.5).astype(np.float32))
    d = Drawer(stream, bits.size)
    c = cfg(0.9, 30, 0.9, 0.01)
    for state in range(2000):
        got = d.draw(bits, c, state)
        want = O.sample_stochastic(bits, 0.9, 30, 0.9, 0.01, canon=O.canonical(state))[0]
        assert got["token_id"] == want, state
    d.close()


def test_sequence_leaves_the_workspace_clean(stream):
    """Draws of different rows and configs in a row, with greedy epilogues between them on
    the same stream: each equals the oracle (a draw that left bins behind would not)."""
    vocab = 70000
    d = Drawer(stream, vocab)
    greedy_out = hy.DeviceArray((20,), np.uint32)
    names = list(CONFIGS)
    for i in range(12):
        bits = rows_of(["normal", "integers", "softcapped"][i % 3], vocab - 997 * i, seed=100 + i)
        c = CONFIGS[names[i % len(names)]]
        check(d.draw(bits, c, i), expect(bits, c, i), f"draw {i}")
        hy.sample_greedy_topk(d.x, 1, bits.size, greedy_out, stream)
        g = hy.topk_samples(greedy_out, 1, stream)[0]
        check(g, expect(bits, None, 0), f"greedy {i}")
    greedy_out.close()
    d.close()


def test_greedy_default_and_contract(stream):
    """NULL config or temperature 0: exactly hyp_sample_greedy_topk's record; malformed
    configs are INVALID_ARGUMENT and write nothing."""
    bits = rows_of("normal", 5000, seed=3)
    d = Drawer(stream, bits.size)
    want = expect(bits, None, 0)
    check(d.draw(bits, None, 5), want, "NULL config")
    check(d.draw(bits, cfg(0.0, 5, 0.5, 0.5, 9), 5), want, "temperature 0")
    for bad in (cfg(-1.0), cfg(0.7, 5001), cfg(0.7, -1), cfg(0.7, 0, 1.5), cfg(0.7, 0, -0.1), cfg(0.7, 0, 0.0, 1.0),
                cfg(0.7, 0, 0.0, -0.5)):
        with pytest.raises(hy.HypError) as e:
            hy.sample_stochastic(d.x, bits.size, bad, 1, d.out, stream)
        assert e.value.status_name == "INVALID_ARGUMENT"
    with pytest.raises(hy.HypError) as e:
        hy.sample_stochastic(d.x, (1 << 23) + 1, cfg(1.0), 1, d.out, stream)
    assert e.value.status_name == "INVALID_ARGUMENT"
    d.close()


def test_captured_draw_replays(stream):
    """A draw captured in a graph keeps its config and RNG state: every replay, with other
    draws and synchronisation between them, equals the eager draw."""
    bits = rows_of("softcapped", 262144, seed=5)
    other = rows_of("normal", 262144, seed=6)
    d = Drawer(stream, bits.size)
    x2 = hy.DeviceArray((bits.size,), np.uint16)
    x2.upload(other, stream)
    out2 = hy.DeviceArray((20,), np.uint32)
    c = cfg(0.8, 64, 0.9, 0.0)
    eager = d.draw(bits, c, 4242)
    want = expect(bits, c, 4242)
    check(eager, want, "eager")
    with hy.Graph.capture(stream) as graph:
        hy.sample_stochastic(d.x, bits.size, c, 4242, d.out, stream)
    for rep in range(4):
        hy.sample_stochastic(x2, other.size, cfg(1.1, 0, 0.8), rep, out2, stream)
        stream.synchronize()
        graph.launch(stream)
        stream.synchronize()
        check(hy.topk_samples(d.out, 1, stream)[0], want, f"replay {rep}")
        check(hy.topk_samples(out2, 1, stream)[0], expect(other, cfg(1.1, 0, 0.8), rep), f"between {rep}")
    graph.close()
    for a in (x2, out2):
        a.close()
    d.close()


# ---- the decoder ------------------------------------------------------------------------

@pytest.fixture(scope="module")
def tiny(fixture_dir):
    import json
    import os
    with open(os.path.join(fixture_dir, "config.json")) as f:
        tc = json.load(f)["text_config"]
    model = hy.Model(hy.geometry_from_config(tc), fixture_dir)
    yield model, tc, fixture_dir
    model.close()


PROMPT = [7, 3, 40, 100]


def run(model, sampling_prefill, sampling_decode, n_decode, per_step=True):
    st = model.kvstate()
    res = hy.StepResult()
    f = st.prefill(PROMPT, res, sampling=sampling_prefill)
    toks = [f.token_id]
    if per_step:
        for _ in range(n_decode):
            toks.append(st.decode(1, res, sampling=sampling_decode).token_id)
    else:
        toks.append(st.decode(n_decode, res, sampling=sampling_decode).token_id)
    st.close()
    res.close()
    return toks


def test_decoder_top_k_one_is_greedy(tiny):
    model, _, _ = tiny
    say("tiny fixture: sampled top_k=1 vs greedy")
    greedy = run(model, None, None, 5)
    for seed in (0, 999):
        c = cfg(1.0, 1, 0.0, 0.0, seed)
        assert run(model, c, c, 5) == greedy


def test_decoder_same_seed_same_tokens(tiny):
    model, _, _ = tiny
    say("tiny fixture: seeded reproducibility")
    c = cfg(1.0, 0, 0.0, 0.0, 12345)
    a = run(model, c, c, 6, per_step=False)
    b = run(model, c, c, 6, per_step=False)
    assert a == b
    # interleaving greedy and sampled blocks on one state (two captured steps)
    st = model.kvstate()
    res = hy.StepResult()
    st.prefill(PROMPT, res)
    st.decode(2, res)
    st.decode(2, res, sampling=c)
    st.decode(1, res)
    st.close()
    res.close()


def test_decoder_block_equals_advanced_single_steps(tiny):
    """A block of n sampled steps from seed s equals n one-step blocks seeded with s,
    adv(s), adv(adv(s)), ... (the block restarts from the seed each call)."""
    model, _, _ = tiny
    say("tiny fixture: sampled block vs advanced single steps")
    n = 5
    s = 2024
    st = model.kvstate()
    res = hy.StepResult()
    st.prefill(PROMPT, res)
    block = st.decode(n, res, sampling=cfg(2.0, 0, 0.0, 0.0, s))
    st.close()
    st = model.kvstate()
    st.prefill(PROMPT, res)
    state = s
    for _ in range(n):
        one = st.decode(1, res, sampling=cfg(2.0, 0, 0.0, 0.0, state))
        state = O.advance_rng(state)
    st.close()
    res.close()
    assert one.token_id == block.token_id
    assert np.float32(one.logit).view(np.uint32) == np.float32(block.logit).view(np.uint32)
    assert list(one.top_k_logprob_ids) == list(block.top_k_logprob_ids)


def test_decoder_sampled_prefill_is_the_draw_over_its_logits(tiny, stream):
    """The sampled prefill's token = hyp_sample_stochastic over softcap(LM head(last hidden
    row)) with rng_state = seed; its sidecar = the greedy epilogue's over the same logits."""
    model, tc, fixture_dir = tiny
    say("tiny fixture: sampled prefill vs the draw over its logits")
    st = model.kvstate()
    hidden = st.forward_hidden(PROMPT, 0)
    st.close()
    qm = hy.QModel(fixture_dir, len(tc["layer_types"]))
    head = qm.embed()
    vocab = tc["vocab_size"]
    x = hy.DeviceArray((1, tc["hidden_size"]), np.uint16)
    x.upload(hidden[-1:].copy(), stream)
    logits = hy.DeviceArray((1, vocab), np.uint16)
    softcap = float(syn.bf16_to_f32(syn.bf16_bits(np.float32([tc["final_logit_softcapping"]])))[0])
    hy.qmatmul(head, x, 1, logits, stream, softcap=softcap)
    out = hy.DeviceArray((20,), np.uint32)
    lbits = logits.to_host(stream).reshape(-1)
    for c in (cfg(1.0, 0, 0.0, 0.0, 31), cfg(0.5, 20, 0.9, 0.0, 7), cfg(1.0, 0, 0.0, 0.0, 2 ** 63 + 5)):
        st = model.kvstate()
        res = hy.StepResult()
        f = st.prefill(PROMPT, res, sampling=c)
        st.close()
        res.close()
        hy.sample_stochastic(logits, vocab, c, c.seed, out, stream)
        want = hy.topk_samples(out, 1, stream)[0]
        assert f.token_id == want["token_id"]
        assert np.float32(f.logit).view(np.uint32) == np.float32(want["logit"]).view(np.uint32)
        assert list(f.top_k_logprob_ids) == list(want["ids"])
        assert f.token_id == O.sample_stochastic(lbits, c.temperature, c.top_k, c.top_p, c.min_p,
                                                 canon=O.canonical(c.seed))[0]
    for a in (x, logits, out, head):
        a.close()
    qm.close()
