"""GPU parity of the RMS norms and the rotary embedding around attention (the start of the
full decode step): mx::fast::rms_norm with and without its learned weight
(forward.cc:23-26, 400-412, 521-529) and mx::fast::rope in both of the reference's schemes
(rope.cc:16-75). Bars: bit-exact against the oracle's restatements (oracle/q4_oracle.c),
which the CPU tests pin against closed forms; the fused and step-program forms bit-exact
against the separate calls.
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


def dev(a, stream):
    return hy.DeviceArray.from_host(a, stream)


def _weight(k, seed):
    rng = np.random.default_rng(seed)
    return syn.bf16_bits((1.0 + 0.25 * rng.standard_normal(k)).astype(np.float32))


@pytest.mark.parametrize("m,k", [(5, 3840), (48, 256), (16, 512), (3, 1000), (3, 19200), (1, 4096)])
@pytest.mark.parametrize("weighted", [False, True])
def test_rms_norm_matches_oracle(stream, m, k, weighted):
    say(f"rms norm m={m} k={k} weighted={weighted}")
    rng = np.random.default_rng(m * 7 + k)
    x = syn.bf16_bits((rng.standard_normal((m, k)) * rng.choice([1e-2, 1.0, 30.0], (m, 1))).astype(np.float32))
    w = _weight(k, k) if weighted else None
    xd = dev(x, stream)
    wd = dev(w, stream) if weighted else None
    yd = hy.DeviceArray((m, k), np.uint16)
    hy.rms_normalize(xd, m, k, yd, stream, eps=1e-6, weight=wd)
    np.testing.assert_array_equal(yd.to_host(stream), O.rms_norm(x, w, 1e-6))
    hy.rms_normalize(xd, m, k, xd, stream, eps=1e-6, weight=wd)   # in place
    np.testing.assert_array_equal(xd.to_host(stream), yd.to_host(stream))


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5])
def test_group_rmsnorm_with_weight_equals_two_calls(stream, m):
    """The pre-attention input_layernorm fused into the q/k/v launch (m <= 4) or run into a
    temporary (m > 4) equals hyp_rms_normalize with the weight then hyp_qmatmul_group."""
    k = 3840
    ws = [syn.q4_weights(n, k, seed=4000 + i) for i, n in enumerate((4096, 2048, 2048))]
    qws = [hy.QWeight.from_host(*w) for w in ws]
    x = syn.activations(m, k, seed=4010 + m)
    xd = dev(x, stream)
    wd = dev(_weight(k, 4020), stream)
    fused = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xd, m, fused, stream, rms_eps=1e-6, norm_weight=wd)
    xn = hy.DeviceArray((m, k), np.uint16)
    hy.rms_normalize(xd, m, k, xn, stream, eps=1e-6, weight=wd)
    sep = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xn, m, sep, stream)
    for a, b, name in zip(fused, sep, "qkv"):
        np.testing.assert_array_equal(a.to_host(stream), b.to_host(stream), err_msg=f"m={m} {name}")
    np.testing.assert_array_equal(xd.to_host(stream), x)
    for a in qws + fused + sep + [xd, wd, xn]:
        a.close()


@pytest.mark.parametrize("m", [1, 4])
def test_step_program_weighted_norm_op(stream, m):
    k = 3840
    ws = [hy.QWeight.from_host(*syn.q4_weights(n, k, seed=4100 + n)) for n in (4096, 2048, 2048)]
    x = syn.activations(m, k, seed=4110 + m)
    xd = dev(x, stream)
    wd = dev(_weight(k, 4120), stream)
    ys = [hy.DeviceArray((m, n), np.uint16) for n in (4096, 2048, 2048)]
    hy.qmatmul_group(ws, xd, m, ys, stream, rms_eps=1e-6, norm_weight=wd)
    want = [y.to_host(stream) for y in ys]
    for y in ys:
        y.upload(np.zeros(y.shape, np.uint16), stream)
    prog = hy.StepProgram([(hy.STEP_QMATMUL_RMSNORM, ws, xd, ys, 1e-6, wd)], m)
    prog.run(stream)
    stream.synchronize()
    prog.check()
    for y, w in zip(ys, want):
        np.testing.assert_array_equal(y.to_host(stream), w)
    prog.close()
    for a in ws + ys + [xd, wd]:
        a.close()


ROPE_CASES = [
    # rows, heads, head_dim, rotated, base, offset
    (1, 16, 256, 256, 1e4, 0),          # decode, local layer, first token
    (1, 16, 256, 256, 1e4, 4095),       # decode later in the sequence
    (4, 8, 256, 256, 1e4, 123456),      # long context
    (1, 16, 512, 128, 1e6, 77),         # global layer, proportional scheme
    (300, 2, 512, 128, 1e6, 0),         # prefill, global
    (2048, 1, 256, 256, 1e4, 2048),     # prefill chunk, local
]


@pytest.mark.parametrize("rows,heads,d,rotated,base,offset", ROPE_CASES)
def test_rope_matches_oracle(stream, rows, heads, d, rotated, base, offset):
    say(f"rope rows={rows} heads={heads} d={d} rotated={rotated} base={base:g} offset={offset}")
    rng = np.random.default_rng(rows + heads + d + offset)
    x = syn.bf16_bits(rng.standard_normal((rows, heads * d)).astype(np.float32))
    xd = dev(x, stream)
    yd = hy.DeviceArray((rows, heads * d), np.uint16)
    hy.rope(xd, rows, heads, d, rotated, base, offset, yd, stream)
    want = O.rope(x, rows, heads, d, rotated, base, offset).reshape(rows, heads * d)
    np.testing.assert_array_equal(yd.to_host(stream), want)
    hy.rope(xd, rows, heads, d, rotated, base, offset, xd, stream)   # in place
    np.testing.assert_array_equal(xd.to_host(stream), want)


def test_q_k_v_prep_of_a_global_layer(stream):
    """A global layer's attention inputs at decode as the reference forms them
    (forward.cc:395-418): q = rope(q_norm(q_proj x)), k = rope(k_norm(k_proj x)) with the
    proportional scheme, v = v_norm(k_proj x) (K = V: no v_proj, weightless norm), each
    norm per head of 512."""
    m, k, d = 1, 3840, 512
    qw = hy.QWeight.from_host(*syn.q4_weights(8192, k, seed=4200))
    kw = hy.QWeight.from_host(*syn.q4_weights(512, k, seed=4201))
    x = dev(syn.activations(m, k, seed=4202), stream)
    q = hy.DeviceArray((m, 8192), np.uint16)
    kr = hy.DeviceArray((m, 512), np.uint16)
    hy.qmatmul_group([qw, kw], x, m, [q, kr], stream, rms_eps=1e-6)
    qh, kh = q.to_host(stream), kr.to_host(stream)
    q_norm, k_norm = _weight(d, 4203), _weight(d, 4204)
    qn, kn = dev(q_norm, stream), dev(k_norm, stream)
    qo = hy.DeviceArray((m, 8192), np.uint16)
    ko = hy.DeviceArray((m, 512), np.uint16)
    vo = hy.DeviceArray((m, 512), np.uint16)
    hy.rms_normalize(q, m * 16, d, qo, stream, eps=1e-6, weight=qn)
    hy.rms_normalize(kr, m, d, ko, stream, eps=1e-6, weight=kn)
    hy.rms_normalize(kr, m, d, vo, stream, eps=1e-6)
    hy.rope(qo, m, 16, d, 128, 1e6, 9, qo, stream)
    hy.rope(ko, m, 1, d, 128, 1e6, 9, ko, stream)
    want_q = O.rope(O.rms_norm(qh.reshape(16, d), q_norm, 1e-6).reshape(m, 8192), m, 16, d, 128, 1e6, 9)
    want_k = O.rope(O.rms_norm(kh.reshape(1, d), k_norm, 1e-6).reshape(m, 512), m, 1, d, 128, 1e6, 9)
    np.testing.assert_array_equal(qo.to_host(stream), want_q.reshape(m, 8192))
    np.testing.assert_array_equal(ko.to_host(stream), want_k.reshape(m, 512))
    np.testing.assert_array_equal(vo.to_host(stream), O.rms_norm(kh, None, 1e-6))
    for a in (qw, kw, x, q, kr, qn, kn, qo, ko, vo):
        a.close()


# ---- MLX's own 12B keys and values (the reference's hidden golden) ------------------------

@pytest.mark.parametrize("layer", [0, 5])
def test_norms_and_rope_reproduce_the_reference_12b_keys(stream, layer):
    """The reference's 12B golden keys (k_norm then RoPE at positions 0..9) and, on the global
    layer, values (v_norm of k_proj), from the golden k_proj output (forward.cc:395-418,
    forward_12b_test.cc:193-211), with the k_norm weight recovered as the CPU tests do
    (tests/test_golden_norm_rope.py): hyp_rms_normalize + hyp_rope, and the decoder's own
    hyp_attention_prepare into a cache, equal the oracle bit for bit, so they reproduce MLX's
    keys wherever the oracle does (all 5,120 of the global layer, 20,479 of 20,480 on the
    sliding one) and its values exactly."""
    import ctypes

    import norm_rope_fit as F
    from test_golden_norm_rope import resolved_weight
    g = F.load()
    D, heads, rot, theta = F.LAYERS[layer]
    kp = g[f"kproj{layer}"]
    L = kp.shape[0]
    w, _ = resolved_weight(g, layer)
    say(f"12B golden keys: layer {layer}, D={D}, kv heads={heads}")
    ref = O.rope(O.rms_norm(kp.reshape(-1, D), w, 1e-6), L, heads, D, rot, theta, 0)
    xd, wd = dev(kp, stream), dev(w, stream)
    yd = hy.DeviceArray((L, heads, D), np.uint16)
    hy.rms_normalize(xd, L * heads, D, yd, stream, eps=1e-6, weight=wd)
    hy.rope(yd, L, heads, D, rot, theta, 0, yd, stream)
    got = yd.to_host(stream)
    np.testing.assert_array_equal(got, ref)
    assert int((got != g[f"k{layer}"]).sum()) <= (1 if layer == 0 else 0)
    # the decoder's fused prepare: q <- rope(q_norm(q)) and the cache slots <- K, V
    cache = hy.KvCache(64, heads, D)
    qd = dev(kp, stream)
    hy.attention_prepare(qd, xd, None, L, heads, cache, wd, wd, 1e-6, rot, theta, 0, stream)
    np.testing.assert_array_equal(qd.to_host(stream).reshape(L, heads, D), ref)
    kbuf, vbuf = cache.buffers()
    ck = np.zeros((64, heads, D), np.uint16)
    cv = np.zeros((64, heads, D), np.uint16)
    hy.call("hyp_memcpy_dtoh", ck.ctypes.data_as(ctypes.c_void_p), kbuf, ck.nbytes, stream.handle)
    hy.call("hyp_memcpy_dtoh", cv.ctypes.data_as(ctypes.c_void_p), vbuf, cv.nbytes, stream.handle)
    stream.synchronize()
    np.testing.assert_array_equal(ck[:L], ref)
    vn = O.rms_norm(kp.reshape(-1, D), None, 1e-6).reshape(L, heads, D)
    np.testing.assert_array_equal(cv[:L], vn)
    if layer == 5:
        np.testing.assert_array_equal(cv[:L, 0], g["v5"])
    cache.close()
