"""GPU parity of the decoder around the Q4 projections: hyp_model_load / hyp_prefill_chunk /
hyp_decode_block / hyp_model_forward_hidden (model.cc:359-740; ForwardPass::forward,
forward.cc:509-563) against the oracle's restatement (oracle/oracle.py DecoderOracle, built
from the pinned primitives), and the two fused layer kernels bit-exact against the calls
they fuse.

Bars, written per test:
  * the tiny fixture's final-normalised hidden rows: the reference's own forward parity
    bar, allclose with rtol = atol = 1e-2 (forward_test.cc:258,406,473-477), and in
    addition sig_rel = max|got - ref| / max|ref| <= 3e-2, which binds there, because the
    fixture's hidden values (normal(0.02) norm weights, build_gemma4_unified_tiny.py:47-51)
    sit far below atol. Both sides round every op to bf16; they differ in summation order
    (fp32 on the device, fp64 in the oracle) and in the attention's bf16 P.
  * random-init artifacts with unit-gain rows: see BRANCH_GAIN below.
  * greedy tokens: equal to the oracle's at every step whose oracle top-2 gap is at least
    GAP (random-init artifacts, unit-scale logits) or 5% of the step's logit (the tiny
    fixture, whose logits are below 0.01; every one of its 6 steps is compared); the
    comparison ends at the first step below it (both sides then legitimately pick either
    token).
  * a decode that fails after its first replay consumes its KV state (model.cc:79-105,
    :149-160): later steps on it return INTERNAL until it is freed.
  * hyp_attention_prepare and hyp_residual_rms_norm: bit-exact.
"""
import ctypes
import json
import os
import sys

import numpy as np
import pytest

import hyperion_amd as hy
import oracle as O
import st_reader
from hyperion_amd import synthetic as syn

pytestmark = pytest.mark.gpu

GAP = 0.05


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def load_tensors(d):
    return {k: v for k, (_, v) in st_reader.read_dir(d).items()}


def text_config(d):
    with open(os.path.join(d, "config.json")) as f:
        return json.load(f)["text_config"]


def check_hidden(got_bits, ref_bits, what, sig_bound=3e-2, rtol_atol=1e-2):
    got = syn.bf16_to_f32(got_bits).astype(np.float64)
    ref = syn.bf16_to_f32(ref_bits).astype(np.float64)
    rel = syn.sig_rel(got, ref)
    ok = np.abs(got - ref) <= (rtol_atol or np.inf) * (1.0 + np.abs(ref))
    say(f"  {what}: sig_rel {rel:.2e}, max|ref| {np.max(np.abs(ref)):.3g}, allclose misses {int((~ok).sum())}")
    assert ok.all(), what
    assert rel <= sig_bound, what


def compare_tokens(gpu_steps, oracle_steps, what, gap_rel=None):
    """gpu_steps: [(token, logit)], oracle_steps: [(token, logit, gap)]. Returns steps compared.

    gap_rel None: a step is compared while the oracle's top-2 gap is at least GAP and the
    logits agree to 0.05 + 2% (unit-scale logits). gap_rel given: the bars scale with the
    step's logit instead - a gap of at least gap_rel * |logit|, logits within gap_rel / 2 *
    |logit| (so a compared token is decided by more than both sides' logit error)."""
    compared = 0
    for j, ((gt, gl), (ot, ol, gap)) in enumerate(zip(gpu_steps, oracle_steps)):
        need = GAP if gap_rel is None else gap_rel * abs(ol)
        if gap < need:
            say(f"  {what}: step {j} oracle gap {gap:.3g} < {need:.3g}: comparison ends")
            break
        tol = 0.05 + 0.02 * abs(ol) if gap_rel is None else 0.5 * gap_rel * abs(ol)
        assert abs(gl - ol) <= tol, f"{what}: step {j}: logit {gl} vs oracle {ol} (bound {tol:.3g})"
        assert gt == ot, f"{what}: step {j}: token {gt} != oracle {ot} (gap {gap:.3g})"
        compared += 1
    say(f"  {what}: {compared} of {len(oracle_steps)} greedy steps equal to the oracle's")
    return compared


def gpu_greedy(model, prompt, n_decode, sampled=False):
    st = model.kvstate()
    res = hy.StepResult()
    f = st.prefill(prompt, res, sampled=sampled)
    steps = [(f.token_id, f.logit)]
    for _ in range(n_decode):
        f = st.decode(1, res, sampled=sampled)
        steps.append((f.token_id, f.logit))
    st.close()
    res.close()
    return steps


# ---- the reference's tiny fixture -------------------------------------------------------

@pytest.fixture(scope="module")
def tiny(fixture_dir):
    cfg = text_config(fixture_dir)
    geo = hy.geometry_from_config(cfg)
    model = hy.Model(geo, fixture_dir)
    yield model, load_tensors(fixture_dir), cfg
    model.close()


def test_tiny_fixture_forward_matches_oracle(tiny):
    """forward_test.cc:390-409: the prompt [7, 3, 40, 100] at offset 0."""
    model, T, cfg = tiny
    say("tiny fixture forward, prompt [7, 3, 40, 100]")
    st = model.kvstate()
    got = st.forward_hidden([7, 3, 40, 100], 0)
    st.close()
    ref = O.DecoderOracle(T, cfg).forward([7, 3, 40, 100], 0)
    check_hidden(got, ref, "tiny L=4")


def test_tiny_fixture_continuation_matches_one_shot(tiny):
    """forward_test.cc:412-482: prefix 12 (> window 8) then an 8-token continuation equals
    rows 12..19 of the 20-token sequence in one shot (rtol = atol = 1e-2), and both the oracle."""
    model, T, cfg = tiny
    ids = [(i * 17 + 7) % cfg["vocab_size"] for i in range(20)]
    say("tiny fixture continuation prefill: 12 + 8 vs 20")
    one = model.kvstate()
    whole = one.forward_hidden(ids, 0)
    one.close()
    split = model.kvstate()
    split.forward_hidden(ids[:12], 0)
    cont = split.forward_hidden(ids[12:], 12)
    split.close()
    a = syn.bf16_to_f32(cont).astype(np.float64)
    b = syn.bf16_to_f32(whole[12:]).astype(np.float64)
    assert np.all(np.abs(a - b) <= 1e-2 + 1e-2 * np.abs(b))
    say(f"  continuation vs one shot: max|delta| {np.max(np.abs(a - b)):.3g}")
    ref = O.DecoderOracle(T, cfg).forward(ids, 0)
    check_hidden(whole, ref, "tiny one shot L=20")
    check_hidden(cont, ref[12:], "tiny continuation rows")


def test_tiny_fixture_prefill_decode(tiny):
    """test_abi_load (forward_test.cc:484-560): prefill a short prompt, then decode; the
    result fields as write_step_result fills them (model.cc:310-331)."""
    model, T, cfg = tiny
    say("tiny fixture prefill [7, 3, 40, 100] + 5 decode steps")
    st = model.kvstate()
    res = hy.StepResult()
    f = st.prefill([7, 3, 40, 100], res)
    assert f.token_id < cfg["vocab_size"]
    assert f.governor_state == 0 and f.top_k_logprob_count == 0
    # one ring of window + 2048 positions (capped at max_position_embeddings) per sliding
    # layer, max_position_embeddings per global layer; K and V, bf16
    cap = min(cfg["sliding_window"] + 2048, cfg["max_position_embeddings"])
    n_sl = cfg["layer_types"].count("sliding_attention")
    n_gl = len(cfg["layer_types"]) - n_sl
    assert f.local_kv_bytes == n_sl * cap * cfg["num_key_value_heads"] * cfg["head_dim"] * 4
    assert f.global_kv_bytes == n_gl * cfg["max_position_embeddings"] * cfg["num_global_key_value_heads"] * \
        cfg["global_head_dim"] * 4
    steps = [(f.token_id, f.logit)]
    for _ in range(5):
        f = st.decode(1, res)
        steps.append((f.token_id, f.logit))
    st.close()
    res.close()
    ref = O.DecoderOracle(T, cfg).greedy([7, 3, 40, 100], 5)
    say(f"  gpu {steps}\n  oracle {ref}")
    # The fixture's logits are small (|logit| < 0.01, normal(0.02) weights), so the bars are
    # relative to each step's logit: its top-2 gaps are 13-24% of the top logit, and the
    # hidden rows agree to about 1% (test_tiny_fixture_forward_matches_oracle).
    assert compare_tokens(steps, ref, "tiny greedy", gap_rel=0.05) == len(ref)


def test_failed_decode_consumes_the_kv_state(fixture_dir):
    """hyperion_mlx.h:197,205-206 and DirectKvExecutionGuard (model.cc:79-105, :149-160): a
    decode that fails after its first replay is enqueued leaves the state unusable - every
    later prefill or decode on it returns INTERNAL until it is freed - while a fresh state of
    the same model still decodes the oracle's tokens. The failure is a host-side throw from
    the test build of the library (libhyperion_hip_faults.so), as the reference's
    HYPERION_TEST_FAULTS build injects one; the GPU work itself is ordinary."""
    L = hy.load_library(hy.FAULTS_LIB_PATH)
    L.hyp_test_fault_after_first_replay.argtypes = []
    L.hyp_test_fault_after_first_replay.restype = None
    INTERNAL = 6

    def st(status_code, expect, what):
        buf = ctypes.create_string_buffer(512)
        L.hyp_last_error(buf, len(buf))
        assert status_code == expect, f"{what}: status {status_code} ({buf.value.decode()}), expected {expect}"
        return buf.value.decode()

    cfg = text_config(fixture_dir)
    geo = hy.geometry_from_config(cfg)
    model, kv, kv2, res = (ctypes.c_void_p() for _ in range(4))
    prompt = np.array([7, 3, 40, 100], np.uint32)
    ts = hy.TokenStream(prompt.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), prompt.size, 1)
    fields = hy.StepResultFields()
    say("consumed state: tiny fixture through the fault-hook build")
    st(L.hyp_model_create(ctypes.byref(model)), 0, "model_create")
    try:
        st(L.hyp_model_load(model, ctypes.byref(geo[0]), fixture_dir.encode()), 0, "model_load")
        st(L.hyp_step_result_create(ctypes.byref(res)), 0, "step_result_create")
        st(L.hyp_kvstate_create(model, ctypes.byref(kv)), 0, "kvstate_create")
        st(L.hyp_prefill_chunk(model, kv, ctypes.byref(ts), res), 0, "prefill")
        st(L.hyp_decode_block(model, kv, 1, res), 0, "decode before the fault")
        L.hyp_test_fault_after_first_replay()
        msg = st(L.hyp_decode_block(model, kv, 3, res), INTERNAL, "decode with the fault")
        assert "injected" in msg
        msg = st(L.hyp_decode_block(model, kv, 1, res), INTERNAL, "decode on the consumed state")
        assert "free and recreate" in msg
        st(L.hyp_prefill_chunk(model, kv, ctypes.byref(ts), res), INTERNAL, "prefill on the consumed state")
        st(L.hyp_decode_block_sampled(model, kv, 1, None, res), INTERNAL, "sampled decode on the consumed state")
        st(L.hyp_kvstate_free(ctypes.byref(kv)), 0, "free the consumed state")
        assert not kv.value
        # a fresh state of the same model is unaffected: it decodes the oracle's tokens
        st(L.hyp_kvstate_create(model, ctypes.byref(kv2)), 0, "kvstate_create again")
        st(L.hyp_prefill_chunk(model, kv2, ctypes.byref(ts), res), 0, "prefill on a fresh state")
        st(L.hyp_step_result_fields(res, ctypes.byref(fields)), 0, "fields")
        steps = [(fields.token_id, fields.logit)]
        for _ in range(3):
            st(L.hyp_decode_block(model, kv2, 1, res), 0, "decode on a fresh state")
            st(L.hyp_step_result_fields(res, ctypes.byref(fields)), 0, "fields")
            steps.append((fields.token_id, fields.logit))
        ref = O.DecoderOracle(load_tensors(fixture_dir), cfg).greedy(prompt.tolist(), 3)
        assert compare_tokens(steps, ref, "fresh state after a consumed one", gap_rel=0.05) == len(ref)
    finally:
        for h, fn in ((kv, "hyp_kvstate_free"), (kv2, "hyp_kvstate_free"), (res, "hyp_step_result_free"),
                      (model, "hyp_model_free")):
            if h.value:
                getattr(L, fn)(ctypes.byref(h))


# ---- synthetic artifacts with unit-gain weights ------------------------------------------

def tiny_dims_config(max_positions):
    return {
        "model_type": "gemma4_unified_text", "hidden_size": 128, "intermediate_size": 256, "num_hidden_layers": 6,
        "layer_types": ["sliding_attention"] * 5 + ["full_attention"], "num_attention_heads": 4, "head_dim": 64,
        "global_head_dim": 128, "num_key_value_heads": 2, "num_global_key_value_heads": 1, "attention_k_eq_v": True,
        "num_kv_shared_layers": 0, "sliding_window": 8,
        "rope_parameters": {"sliding_attention": {"rope_theta": 10000.0, "rope_type": "default"},
                            "full_attention": {"rope_theta": 1000000.0, "partial_rotary_factor": 0.25,
                                               "rope_type": "proportional"}},
        "final_logit_softcapping": 30.0, "rms_norm_eps": 1e-6, "attention_bias": False, "vocab_size": 512,
        "max_position_embeddings": max_positions, "tie_word_embeddings": True, "hidden_size_per_layer_input": 0,
        "vocab_size_per_layer_input": 0, "use_double_wide_mlp": False, "enable_moe_block": False,
    }


# Random-init weights make a sensitive network: the oracle run with once-rounded instead
# of exact weights (a 2^-9 relative change per weight) moves its own hidden rows by ~2% of
# their maximum at these gains over 6 layers, and by up to 120% at unit post-norm and
# q/k-norm gains. So a stack of layers is compared with the oracle following the device's
# weight semantics (weights="per_m") by sig_rel <= 3e-2, the exact-weight oracle by
# sig_rel <= 0.1. Single layers are also held element by element, to allclose with rtol =
# atol = 3e-2: the device rounds the softmax weights to bf16 for the P.V products (up to
# 2^-8 relative each, which the oracle does not), and the post-attention norm and the
# MLP's GELU pass that on to every element of the layer's output.
BRANCH_GAIN, QK_GAIN = 0.5, 0.7


def check_both(got, T, cfg, ids, what, per_element=False):
    per_m = O.DecoderOracle(T, cfg, weights="per_m").forward(ids, 0)
    check_hidden(got, per_m, what + " (per-size weights)", rtol_atol=3e-2 if per_element else None)
    exact = O.DecoderOracle(T, cfg).forward(ids, 0)
    check_hidden(got, exact, what + " (exact weights)", sig_bound=0.1, rtol_atol=None)


def test_long_context_ring_wrap(tmp_path):
    """Tiny dims, max_position_embeddings 4096: a 2100-token prompt is two prefill chunks
    (2048 + 52) and wraps the sliding rings (window 8 + 2048 = 2056 slots); 40 decode steps
    read windows across the wrap."""
    cfg = tiny_dims_config(4096)
    T = syn.write_model(str(tmp_path), cfg, seed=11, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg["vocab_size"], size=2100).astype(np.uint32)
    say("long context: forward_hidden over 2100 tokens")
    st = model.kvstate()
    got = st.forward_hidden(prompt, 0)
    st.close()
    per_m = O.DecoderOracle(T, cfg, weights="per_m").forward(prompt, 0)
    for lo, hi in ((0, 16), (1020, 1040), (2040, 2100)):
        check_hidden(got[lo:hi], per_m[lo:hi], f"rows {lo}..{hi}", rtol_atol=None)
    say("long context: prefill 2100 + 40 decode steps")
    steps = gpu_greedy(model, prompt, 40)
    ref_steps = O.DecoderOracle(T, cfg, weights="per_m").greedy(prompt, 40)
    assert compare_tokens(steps, ref_steps, "long context greedy") >= 1
    model.close()


def test_12b_shaped_layers(tmp_path):
    """The 12B's layer shapes (hidden 3840, 16 heads, head_dim 256 / 512, 8 / 1 KV heads,
    window 1024, MLP 15360) as one sliding and one global layer, vocab 1024."""
    cfg = syn.gemma4_text_config(num_layers=2, vocab=1024, max_positions=2048,
                                 layer_types=["sliding_attention", "full_attention"])
    say("12B-shaped layers: writing the artifact")
    T = syn.write_model(str(tmp_path), cfg, seed=12, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, cfg["vocab_size"], size=37).astype(np.uint32)
    st = model.kvstate()
    got = st.forward_hidden(prompt, 0)
    st.close()
    check_both(got, T, cfg, prompt, "12B-shaped L=37")
    say("12B-shaped layers: prefill 37 + 6 decode steps")
    steps = gpu_greedy(model, prompt, 6)
    ref_steps = O.DecoderOracle(T, cfg, weights="per_m").greedy(prompt, 6)
    assert compare_tokens(steps, ref_steps, "12B-shaped greedy") >= 1
    model.close()


def test_12b_global_layer_split_chunk(tmp_path):
    """One 12B-shaped global layer (16 heads of 512, one KV head) over a 300-token prompt:
    the chunk attention splits its keys in two (75 tiles, 300 keys) and merges them."""
    cfg = syn.gemma4_text_config(num_layers=1, vocab=1024, max_positions=2048, layer_types=["full_attention"])
    T = syn.write_model(str(tmp_path), cfg, seed=14, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    prompt = np.random.default_rng(8).integers(0, cfg["vocab_size"], size=300).astype(np.uint32)
    say("12B global layer: forward_hidden over 300 tokens (split chunk attention)")
    st = model.kvstate()
    got = st.forward_hidden(prompt, 0)
    st.close()
    per_m = O.DecoderOracle(T, cfg, weights="per_m").forward(prompt, 0)
    for lo, hi in ((0, 8), (140, 160), (290, 300)):
        check_hidden(got[lo:hi], per_m[lo:hi], f"rows {lo}..{hi}", rtol_atol=None)
    model.close()


@pytest.mark.parametrize("dims,kind", [("tiny", "full_attention"), ("tiny", "sliding_attention"),
                                       ("12b", "full_attention"), ("12b", "sliding_attention")])
def test_single_layer_per_element(tmp_path, dims, kind):
    """One decoder layer (a sliding one closed by a global one where the geometry requires
    a global last layer), compared element by element: allclose rtol = atol = 3e-2 and
    sig_rel <= 3e-2 at L = 3 (decode kernels) and L = 70 (GEMMs)."""
    types = [kind] if kind == "full_attention" else [kind, "full_attention"]
    if dims == "tiny":
        cfg = tiny_dims_config(256)
        cfg["layer_types"], cfg["num_hidden_layers"] = types, len(types)
    else:
        cfg = syn.gemma4_text_config(num_layers=len(types), vocab=512, max_positions=256, layer_types=types)
    say(f"single layer {dims} {types}")
    T = syn.write_model(str(tmp_path), cfg, seed=14, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    prompt = np.random.default_rng(9).integers(0, cfg["vocab_size"], size=70).astype(np.uint32)
    for L in (3, 70):
        st = model.kvstate()
        got = st.forward_hidden(prompt[:L], 0)
        st.close()
        check_both(got, T, cfg, prompt[:L], f"{dims} {types} L={L}", per_element=True)
    model.close()


def test_decode_sizes_tiny_dims(tmp_path):
    """Prompts of 1 to 4 tokens take the decode kernels for every projection (exact weights)
    and 5 the GEMMs: each against both oracles."""
    cfg = tiny_dims_config(256)
    T = syn.write_model(str(tmp_path), cfg, seed=13, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    prompt = np.random.default_rng(8).integers(0, cfg["vocab_size"], size=5).astype(np.uint32)
    for L in (1, 2, 4, 5):
        st = model.kvstate()
        got = st.forward_hidden(prompt[:L], 0)
        st.close()
        check_both(got, T, cfg, prompt[:L], f"tiny dims L={L}")
    model.close()


def test_wide_query_groups_decode(tmp_path):
    """32 query heads over one KV head on every layer (G = 32 > 16): a one-token step cannot
    take the decode attention form, so the prepare runs as its own launch and the chunk form
    attends (attention_prep_fits). A 1-token prefill, a 5-token prefill and 6 decode steps
    (graph replays) against the oracle."""
    cfg = tiny_dims_config(256)
    cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["num_global_key_value_heads"] = 32, 1, 1
    T = syn.write_model(str(tmp_path), cfg, seed=15, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    prompt = np.random.default_rng(10).integers(0, cfg["vocab_size"], size=5).astype(np.uint32)
    say("wide query groups (G = 32): forward_hidden at L = 1 and 5")
    for L in (1, 5):
        st = model.kvstate()
        got = st.forward_hidden(prompt[:L], 0)
        st.close()
        check_both(got, T, cfg, prompt[:L], f"G=32 L={L}")
    say("wide query groups (G = 32): prefill 5 + 6 decode steps")
    steps = gpu_greedy(model, prompt, 6)
    ref_steps = O.DecoderOracle(T, cfg, weights="per_m").greedy(prompt, 6)
    assert compare_tokens(steps, ref_steps, "G=32 greedy") >= 1
    model.close()


def test_sampled_greedy_sidecar_and_contract(tiny, tmp_path):
    """hyp_*_sampled at temperature 0 is the greedy path plus the top-k sidecar
    (model.cc:262-301); temperature > 0 draws (its parity is tests/test_gpu_sampling.py's);
    malformed configs, decode before prefill, a second prefill and a foreign state are
    rejected."""
    model, T, cfg = tiny
    st = model.kvstate()
    res = hy.StepResult()
    with pytest.raises(hy.HypError) as e:
        st.decode(1, res)
    assert e.value.status_name == "INVALID_ARGUMENT"
    f = st.prefill([7, 3, 40, 100], res, sampled=True)
    assert f.top_k_logprob_count == hy.TOP_K_LOGPROBS and f.near_tie_events == 0
    assert f.top_k_logprob_ids[0] == f.token_id and f.top_k_logprob_values[0] == f.logit
    vals = list(f.top_k_logprob_values)
    assert vals == sorted(vals, reverse=True)
    with pytest.raises(hy.HypError) as e:
        st.prefill([1, 2], res)
    assert e.value.status_name == "INVALID_ARGUMENT"
    f2 = st.decode(2, res, sampling=hy.SamplingConfig(0.0, 0, 0.0, 0.0, 7))
    assert f2.top_k_logprob_count == hy.TOP_K_LOGPROBS
    f3 = st.decode(1, res, sampling=hy.SamplingConfig(0.7, 0, 0.0, 0.0, 1))
    assert f3.token_id < cfg["vocab_size"] and f3.top_k_logprob_count == hy.TOP_K_LOGPROBS
    assert f3.near_tie_events == 0
    for bad, status in ((hy.SamplingConfig(-1.0, 0, 0.0, 0.0, 1), "INVALID_ARGUMENT"),
                        (hy.SamplingConfig(0.7, cfg["vocab_size"] + 1, 0.0, 0.0, 1), "INVALID_ARGUMENT"),
                        (hy.SamplingConfig(0.7, 0, 1.5, 0.0, 1), "INVALID_ARGUMENT"),
                        (hy.SamplingConfig(0.7, 0, 0.0, 1.0, 1), "INVALID_ARGUMENT")):
        with pytest.raises(hy.HypError) as e:
            st.decode(1, res, sampling=bad)
        assert e.value.status_name == status
    with pytest.raises(hy.HypError) as e:
        st.prefill([cfg["vocab_size"]], res)   # out of the vocabulary (and not fresh)
    assert e.value.status_name == "INVALID_ARGUMENT"
    fresh = model.kvstate()
    with pytest.raises(hy.HypError) as e:
        fresh.prefill([cfg["vocab_size"]], res)
    assert e.value.status_name == "INVALID_ARGUMENT"
    other = hy.Model(hy.geometry_from_config(cfg), os.path.dirname(os.path.abspath(__file__)) +
                     "/golden/gemma4-unified-tiny")
    foreign = other.kvstate()
    ts = hy.TokenStream((ctypes.c_uint32 * 1)(7), 1, 1)
    st_code = hy.lib().hyp_prefill_chunk(model.handle, foreign.handle, ctypes.byref(ts), res.handle)
    assert hy.HYP_STATUS[st_code] == "INVALID_ARGUMENT"
    for h in (foreign, other, fresh, st, res):
        h.close()


# ---- the fused layer kernels, bit-exact -------------------------------------------------

@pytest.mark.parametrize("L,H,KVH,D,rotated,base,offset,kv_eq", [
    (1, 16, 8, 256, 256, 1e4, 700, False),
    (37, 16, 8, 256, 256, 1e4, 0, False),
    (5, 16, 1, 512, 128, 1e6, 4000, True),
    (300, 16, 1, 512, 128, 1e6, 3, True),
    (9, 4, 2, 64, 64, 1e4, 20, False),
    (3, 4, 1, 128, 32, 1e6, 11, True),
    (40, 4, 2, 64, 64, 1e4, 20, False),    # above 16 tokens: the packed-row form
    (33, 4, 1, 128, 32, 1e6, 70, True),
])
def test_attention_prepare_bit_exact(stream, L, H, KVH, D, rotated, base, offset, kv_eq):
    """hyp_attention_prepare == hyp_rms_normalize + hyp_rope on q, the same on k, the
    weightless norm on v (of k_raw when K = V), hyp_kv_cache_write of the results."""
    say(f"attention prepare L={L} H={H} KVH={KVH} D={D} offset={offset} k_eq_v={kv_eq}")
    rng = np.random.default_rng(L * 31 + D)
    b = lambda scale, *shape: syn.bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))  # noqa: E731
    q, k_raw, v_raw = b(2.0, L, H, D), b(2.0, L, KVH, D), b(2.0, L, KVH, D)
    qw, kw = b(0.3, D), b(0.3, D)
    qw = syn.bf16_bits(1.0 + syn.bf16_to_f32(qw))
    cap = max(L + offset % 64 + 1, 64)
    eps = 1e-6
    dev = lambda a: hy.DeviceArray.from_host(a, stream)  # noqa: E731
    # fused
    c1 = hy.KvCache(cap, KVH, D)
    qd, kd, vd, qwd, kwd = dev(q), dev(k_raw), dev(v_raw), dev(qw), dev(kw)
    hy.attention_prepare(qd, kd, None if kv_eq else vd, L, H, c1, qwd, kwd, eps, rotated, base, offset, stream)
    # separate
    c2 = hy.KvCache(cap, KVH, D)
    kp1, vp1 = c1.buffers()
    q2, k2, v2 = dev(q), dev(k_raw), dev(v_raw if not kv_eq else k_raw)
    vn = hy.DeviceArray((L, KVH, D), np.uint16)
    hy.rms_normalize(q2, L * H, D, q2, stream, eps=eps, weight=qwd)
    hy.rope(q2, L, H, D, rotated, base, offset, q2, stream)
    hy.rms_normalize(v2, L * KVH, D, vn, stream, eps=eps)
    hy.rms_normalize(k2, L * KVH, D, k2, stream, eps=eps, weight=kwd)
    hy.rope(k2, L, KVH, D, rotated, base, offset, k2, stream)
    c2.write(k2, vn, L, offset, stream)
    stream.synchronize()
    np.testing.assert_array_equal(qd.to_host(stream), q2.to_host(stream))
    kp2, vp2 = c2.buffers()
    for p1, p2, what in ((kp1, kp2, "K"), (vp1, vp2, "V")):
        a = np.zeros((cap, KVH, D), np.uint16)
        bb = np.zeros((cap, KVH, D), np.uint16)
        hy.call("hyp_memcpy_dtoh", a.ctypes.data_as(ctypes.c_void_p), p1, a.nbytes, stream.handle)
        hy.call("hyp_memcpy_dtoh", bb.ctypes.data_as(ctypes.c_void_p), p2, bb.nbytes, stream.handle)
        stream.synchronize()
        slots = [(offset + t) % cap for t in range(L)]
        np.testing.assert_array_equal(a[slots], bb[slots], err_msg=what)
    for x in (qd, kd, vd, qwd, kwd, q2, k2, v2, vn):
        x.close()
    c1.close()
    c2.close()


@pytest.mark.parametrize("m,hidden,scalar,nxt", [(1, 3840, False, True), (4, 3840, True, False),
                                                  (300, 3840, True, True), (7, 128, True, True),
                                                  (2, 16384, False, False),
                                                  # from 64 rows on: the coalesced tiled form
                                                  (1024, 3840, False, True), (65, 128, True, False),
                                                  (130, 4096, True, True)])
def test_residual_rms_norm_bit_exact(stream, m, hidden, scalar, nxt):
    """hyp_residual_rms_norm == hyp_rms_normalize(branch, w_post), the bf16 add (and layer
    scalar product) of the oracle, then hyp_rms_normalize(residual, w_next)."""
    say(f"residual rms norm m={m} hidden={hidden} scalar={scalar} next={nxt}")
    rng = np.random.default_rng(m + hidden)
    b = lambda scale, *shape: syn.bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))  # noqa: E731
    branch, resid = b(3.0, m, hidden), b(5.0, m, hidden)
    wp = syn.bf16_bits(1.0 + syn.bf16_to_f32(b(0.2, hidden)))
    wn = syn.bf16_bits(1.0 + syn.bf16_to_f32(b(0.2, hidden)))
    sc = syn.bf16_bits(np.array([0.8125], np.float32))
    dev = lambda a: hy.DeviceArray.from_host(a, stream)  # noqa: E731
    bd, rd, wpd, wnd, scd = dev(branch), dev(resid), dev(wp), dev(wn), dev(sc)
    nd = hy.DeviceArray((m, hidden), np.uint16)
    hy.residual_rms_norm(bd, rd, wpd, scd if scalar else None, wnd if nxt else None, nd if nxt else None, m, hidden,
                         1e-6, stream)
    got_r = rd.to_host(stream)
    # composition
    hn = hy.DeviceArray((m, hidden), np.uint16)
    hy.rms_normalize(bd, m, hidden, hn, stream, eps=1e-6, weight=wpd)
    expect = O.add_bf16(resid, hn.to_host(stream))
    if scalar:
        expect = O.mul_bf16(expect, sc)
    np.testing.assert_array_equal(got_r, expect)
    if nxt:
        ed = dev(expect)
        en = hy.DeviceArray((m, hidden), np.uint16)
        hy.rms_normalize(ed, m, hidden, en, stream, eps=1e-6, weight=wnd)
        np.testing.assert_array_equal(nd.to_host(stream), en.to_host(stream))
        ed.close()
        en.close()
    for x in (bd, rd, wpd, wnd, scd, nd, hn):
        x.close()


@pytest.mark.parametrize("prefix", [20, 31, 32, 63, 64])
@pytest.mark.parametrize("head_dims", [(64, 128), (256, 512)])
def test_folded_prepare_equals_separate(tmp_path, prefix, head_dims):
    """A one-token step folds the q/k norms, RoPE and the cache append into the decode
    attention launch; a two-token step at the same position runs them as their own launch
    (attn_prepare_kernel) with every other kernel the same per row. Row 0 of the two-token
    step has the bits of the one-token step, on both layer kinds, with the new key first,
    last and inside a 32-key block. Head dims 64 and 256 take the folded form with each
    64-value unit spread over 8 and 4 lanes, 128 and 512 (four query rows per kv head) the
    unit-per-lane form."""
    cfg = tiny_dims_config(256)
    cfg["head_dim"], cfg["global_head_dim"] = head_dims
    T = syn.write_model(str(tmp_path), cfg, seed=16, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    ids = np.random.default_rng(prefix).integers(0, cfg["vocab_size"], size=prefix + 2).astype(np.uint32)
    say(f"folded prepare: prefix {prefix}, head dims {head_dims}")
    one, two = model.kvstate(), model.kvstate()
    one.forward_hidden(ids[:prefix], 0)
    two.forward_hidden(ids[:prefix], 0)
    a = one.forward_hidden(ids[prefix:prefix + 1], prefix)
    b = two.forward_hidden(ids[prefix:prefix + 2], prefix)
    np.testing.assert_array_equal(a[0], b[0])
    # and the next step reads the folded step's cache entries as the oracle does (the
    # six-layer stack's bar against the per-size-weight oracle: sig_rel <= 3e-2)
    nxt = one.forward_hidden(ids[prefix + 1:prefix + 2], prefix + 1)
    check_hidden(nxt, O.DecoderOracle(T, cfg, weights="per_m").forward(ids[:prefix + 2], 0)[prefix + 1:],
                 f"step after the folded one, prefix {prefix}", rtol_atol=None)
    for h in (one, two, model):
        h.close()


def test_decode_block_equals_single_steps(tmp_path):
    """hyp_decode_block(n) (n graph replays in one call) ends where n calls of
    hyp_decode_block(1) end: the same token, logit and near-tie count; two states of one
    model each keep their own captured step."""
    cfg = tiny_dims_config(512)
    syn.write_model(str(tmp_path), cfg, seed=15, branch_gain=BRANCH_GAIN, qk_gain=QK_GAIN)
    model = hy.Model(hy.geometry_from_config(cfg), str(tmp_path))
    prompt = np.random.default_rng(10).integers(0, cfg["vocab_size"], size=30).astype(np.uint32)
    res = hy.StepResult()
    a, b = model.kvstate(), model.kvstate()
    a.prefill(prompt, res)
    b.prefill(prompt, res)
    fa = a.decode(12, res)
    ties = 0
    for _ in range(12):
        fb = b.decode(1, res)
        ties += fb.near_tie_events
    say(f"  block: token {fa.token_id} logit {fa.logit} ties {fa.near_tie_events}; steps: token {fb.token_id} "
        f"ties {ties}")
    assert (fa.token_id, fa.logit, fa.near_tie_events) == (fb.token_id, fb.logit, ties)
    assert a.decode(3, res).token_id == b.decode(3, res).token_id
    for h in (a, b, res, model):
        h.close()


def test_model_memory_matches_the_geometry_plan(tiny, tmp_path):
    """hyp_model_memory (the loaded model's buffers, summed) equals hyp_geometry_memory (the
    plan from the geometry alone), field by field, on the fixture and on 12B-shaped layers."""
    model, T, cfg = tiny
    got = model.memory()
    plan = hy.geometry_memory(hy.geometry_from_config(cfg))
    for f, _ in hy.MemoryReport._fields_:
        assert getattr(got, f) == getattr(plan, f), f
    cfg12 = syn.gemma4_text_config(num_layers=2, vocab=1024, max_positions=2048,
                                   layer_types=["sliding_attention", "full_attention"])
    syn.write_model(str(tmp_path), cfg12, seed=16)
    m12 = hy.Model(hy.geometry_from_config(cfg12), str(tmp_path))
    got, plan = m12.memory(), hy.geometry_memory(hy.geometry_from_config(cfg12))
    say(f"  12B-shaped 2 layers: weights {got.weight_bytes} B (dense bf16 {got.dense_bf16_weight_bytes} B), "
        f"scratch {got.scratch_bytes} B")
    for f, _ in hy.MemoryReport._fields_:
        assert getattr(got, f) == getattr(plan, f), f
    m12.close()
