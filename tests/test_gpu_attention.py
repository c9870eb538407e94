"""GPU parity of the attention around the Q4 linears (ForwardPass::attention,
forward.cc:376-508) and the KV cache writes (LocalKvCache / GlobalKvCache append,
kv_cache.h:33,143): hyp_attention against the oracle's fp64 restatement
(oracle/q4_oracle.c orc_attention_f64, pinned on the CPU against dense numpy attention and
closed forms), hyp_kv_cache_write against the slot rule p % capacity.

Bar (written per test): every output within 2^-8 |ref| + 2^-9 max|v| of the fp64 truth
(the output's bf16 rounding, plus the P.V products' bf16 P), and sig_rel <= 1e-2. MLX's
own SDPA bits are parity unpinned (no reference vectors).
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


def dev(a, stream):
    return hy.DeviceArray.from_host(a, stream)


def _fill_cache(cache, ck, cv, stream):
    kp, vp = cache.buffers()
    for ptr, host in ((kp, ck), (vp, cv)):
        hy.call("hyp_memcpy_htod", ptr, host.ctypes.data_as(ctypes.c_void_p), host.nbytes, stream.handle)
    stream.synchronize()


def _check(got_bits, ref, v_all, what):
    got = syn.bf16_to_f32(got_bits).astype(np.float64)
    vmax = float(np.max(np.abs(syn.bf16_to_f32(v_all)))) if v_all.size else 0.0
    bound = 2.0**-8 * np.abs(ref) + 2.0**-9 * vmax
    err = np.abs(got - ref)
    worst = float(np.max(err / bound))
    rel = syn.sig_rel(got, ref)
    say(f"  {what}: worst {worst:.3f} of the bound, sig_rel {rel:.2e}")
    assert np.all(err <= bound), what
    assert rel <= 1e-2, what


CASES = [
    # L, H, KVH, D, cap, offset, prefix, window, q scale
    (1, 16, 8, 256, 1032, 0, 0, 1024, 0.25),        # sliding decode, first token
    (1, 16, 8, 256, 1032, 700, 700, 1024, 0.25),    # sliding decode inside the window
    (1, 16, 8, 256, 1032, 5000, 1024, 1024, 0.25),  # sliding decode, ring wrapped
    (4, 16, 8, 256, 1032, 3000, 1024, 1024, 0.25),  # batch-4-token decode
    (1, 16, 1, 512, 8192, 4000, 4000, 0, 0.18),     # global decode (K = V layers)
    (4, 16, 1, 512, 8192, 100, 100, 0, 0.18),
    (300, 16, 8, 256, 1032, 0, 0, 1024, 0.25),      # prefill chunk
    (300, 16, 8, 256, 1032, 2000, 1024, 1024, 0.25),   # continuation prefill over the ring
    (2048, 16, 8, 256, 2048, 0, 0, 1024, 0.25),     # a full prefill chunk, window inside it
    (300, 16, 1, 512, 4096, 0, 0, 0, 0.18),         # global prefill
    (257, 16, 1, 512, 4096, 1000, 1000, 0, 0.18),
    (10, 4, 2, 64, 16, 0, 0, 8, 0.5),               # the tiny fixture's shapes
    (1, 4, 2, 64, 16, 20, 8, 8, 0.5),
    (5, 4, 1, 128, 64, 30, 30, 0, 0.4),
]


@pytest.mark.parametrize("L,H,KVH,D,cap,offset,prefix,window,qs", CASES)
def test_attention_matches_oracle(stream, L, H, KVH, D, cap, offset, prefix, window, qs):
    say(f"attention L={L} H={H} KVH={KVH} D={D} cap={cap} offset={offset} prefix={prefix} window={window}")
    rng = np.random.default_rng(L * 7919 + offset * 13 + D)
    b = lambda scale, *shape: syn.bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))  # noqa: E731
    q, k, v = b(qs, L, H, D), b(1.0, L, KVH, D), b(1.0, L, KVH, D)
    ck, cv = b(1.0, cap, KVH, D), b(1.0, cap, KVH, D)
    cache = hy.KvCache(cap, KVH, D)
    _fill_cache(cache, ck, cv, stream)
    qd, kd, vd = dev(q, stream), dev(k, stream), dev(v, stream)
    out = hy.DeviceArray((L, H, D), np.uint16)
    hy.attention(qd, kd, vd, L, H, cache, offset, prefix, window, out, stream)
    ref = O.attention_f64(q, k, v, ck, cv, offset, prefix, window)
    _check(out.to_host(stream), ref, np.concatenate([v.reshape(-1), cv.reshape(-1)]), f"L={L} D={D} offset={offset}")
    for a in (qd, kd, vd, out):
        a.close()
    cache.close()


def test_kv_cache_write_slots_and_ring_overwrite(stream):
    """Tokens land in slot p % capacity; a write longer than the ring keeps its last
    `capacity` tokens; attention over the written prefix equals attention over the same
    rows uploaded directly."""
    cap, KVH, D = 24, 2, 64
    rng = np.random.default_rng(3)
    cache = hy.KvCache(cap, KVH, D)
    kp, vp = cache.buffers()
    expect_k = np.zeros((cap, KVH, D), np.uint16)
    expect_v = np.zeros((cap, KVH, D), np.uint16)
    _fill_cache(cache, expect_k, expect_v, stream)
    pos = 0
    for n in (5, 1, 30, 7, 3):      # 30 > cap wraps past a whole ring
        k = syn.bf16_bits(rng.standard_normal((n, KVH, D)).astype(np.float32))
        v = syn.bf16_bits(rng.standard_normal((n, KVH, D)).astype(np.float32))
        kd, vd = dev(k, stream), dev(v, stream)
        cache.write(kd, vd, n, pos, stream)
        for t in range(n):
            expect_k[(pos + t) % cap] = k[t]
            expect_v[(pos + t) % cap] = v[t]
        pos += n
        kd.close()
        vd.close()
    stream.synchronize()
    got_k = np.zeros_like(expect_k)
    got_v = np.zeros_like(expect_v)
    for ptr, host in ((kp, got_k), (vp, got_v)):
        hy.call("hyp_memcpy_dtoh", host.ctypes.data_as(ctypes.c_void_p), ptr, host.nbytes, stream.handle)
    stream.synchronize()
    np.testing.assert_array_equal(got_k, expect_k)
    np.testing.assert_array_equal(got_v, expect_v)
    # decode one token over the last 20 written positions
    q = syn.bf16_bits((rng.standard_normal((1, 4, D)) * 0.5).astype(np.float32))
    k1 = syn.bf16_bits(rng.standard_normal((1, KVH, D)).astype(np.float32))
    v1 = syn.bf16_bits(rng.standard_normal((1, KVH, D)).astype(np.float32))
    qd, kd, vd = dev(q, stream), dev(k1, stream), dev(v1, stream)
    out = hy.DeviceArray((1, 4, D), np.uint16)
    hy.attention(qd, kd, vd, 1, 4, cache, pos, 20, 21, out, stream)
    ref = O.attention_f64(q, k1, v1, expect_k, expect_v, pos, 20, 21)
    _check(out.to_host(stream), ref, np.concatenate([v1.reshape(-1), expect_v.reshape(-1)]), "after writes")
    for a in (qd, kd, vd, out):
        a.close()
    cache.close()


def test_attention_rejects_bad_arguments(stream):
    cache = hy.KvCache(16, 2, 64)
    x = hy.DeviceArray((4, 4, 64), np.uint16)
    for args, what in (((x, x, x, 1, 3, cache, 5, 5, 0, x), "heads"),       # 3 heads over 2 kv heads
                       ((x, x, x, 1, 4, cache, 5, 6, 0, x), "prefix"),      # prefix beyond offset
                       ((x, x, x, 1, 4, cache, 50, 17, 0, x), "capacity")):  # prefix beyond capacity
        with pytest.raises(hy.HypError) as e:
            hy.attention(*args, stream)
        assert e.value.status_name == "INVALID_ARGUMENT", what
    x.close()
    cache.close()
