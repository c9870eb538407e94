"""RMSNorm and RoPE held to the keys and values of MLX's own 12B forward.

The reference's 12B hidden golden carries, for the first sliding layer (0) and the first global
layer (5), the raw k_proj output beside the keys (k_norm then RoPE, positions 0..9) and, on the
global layer, the values (v_norm of k_proj) (forward.cc:395-418, rope.cc:16-75;
forward_12b_test.cc:193-211 holds the reference's forward to them). `norm_rope_fit` explains
how the absent k_norm weights are pinned down from the unrotated positions.
"""
import numpy as np
import pytest

import norm_rope_fit as F
import oracle as O


@pytest.fixture(scope="module")
def g():
    return F.load()


def resolved_weight(g, layer):
    """The k_norm weight of a layer: per dimension the candidate (from norm_rope_fit) under
    which the oracle's weighted norm and RoPE reproduce the most golden values of that
    dimension's rotation pair (the candidates differ only where a product rounds alike)."""
    D, heads, rot, theta = F.LAYERS[layer]
    kp, k = g[f"kproj{layer}"], g[f"k{layer}"]
    L = kp.shape[0]
    n = O.rms_norm(kp.reshape(-1, D), None, F.EPS).reshape(L, heads, D)
    cands = F.recover_k_norm_weight(n, k, D, rot)
    assert all(len(c) for c in cands.values()), "a dimension with no consistent k_norm weight"
    w = np.array([cands[d][0] for d in range(D)], np.uint16)
    half = D // 2
    for i in range(rot // 2):
        best = None
        for a in cands[i]:
            for b in cands[i + half]:
                w2 = w.copy()
                w2[i], w2[i + half] = a, b
                y = O.rope(O.rms_norm(kp.reshape(-1, D), w2, F.EPS), L, heads, D, rot, theta, 0)
                miss = int((y[:, :, [i, i + half]] != k[:, :, [i, i + half]]).sum())
                if best is None or miss < best[0]:
                    best = (miss, a, b)
        w[i], w[i + half] = best[1], best[2]
    return w, cands


def test_weightless_norm_equals_mlx_v_norm(g):
    """v_norm of the global layer (forward.cc:403-412): the oracle's weightless rms_norm of
    k_proj equals MLX's values on all 5,120 of them."""
    got = O.rms_norm(g["kproj5"], None, F.EPS)
    np.testing.assert_array_equal(got, g["v5"])


def test_a_planted_error_in_the_norm_is_caught(g):
    """The comparison is strict: the norm of a row with one value changed by one ulp differs."""
    kp = g["kproj5"].copy()
    kp[3, 17] += 1
    assert (O.rms_norm(kp, None, F.EPS) != g["v5"]).any()


@pytest.mark.parametrize("layer", [0, 5])
def test_one_k_norm_weight_fits_every_unrotated_value(g, layer):
    """Each dimension's weight is pinned by position 0 (all heads); the dimensions RoPE never
    rotates must then fit all ten positions with that same weight under the oracle's
    weighted rounding, bf16(w * bf16(x * rms)) - a wrong rounding order leaves dimensions
    with no consistent weight."""
    D, heads, rot, _ = F.LAYERS[layer]
    _, cands = resolved_weight(g, layer)
    free = F.unrotated_dims(D, rot)
    print(f"layer {layer}: {len(free)} unrotated dims, candidates per dim {min(map(len, cands.values()))}.."
          f"{max(map(len, cands.values()))}")
    assert all(len(cands[d]) >= 1 for d in range(D))


def test_global_layer_keys_bit_exact(g):
    """k_norm then the proportional RoPE (128 of 512 dims rotated, theta 1e6): the oracle
    reproduces MLX's keys at positions 0..9 bit for bit (5,120 values)."""
    D, heads, rot, theta = F.LAYERS[5]
    w, _ = resolved_weight(g, 5)
    kp = g["kproj5"]
    y = O.rope(O.rms_norm(kp, w, F.EPS), kp.shape[0], heads, D, rot, theta, 0)
    np.testing.assert_array_equal(y, g["k5"])


def test_sliding_layer_keys_within_one_trig_ulp(g):
    """k_norm then RoPE over all 256 dims (theta 1e4), 8 kv heads: 20,479 of MLX's 20,480 keys
    bit for bit. The one other (position 8, kv head 6, dim 11) is one bf16 ulp off: the
    oracle's fp32 result sits one fp32 ulp above a bf16 rounding midpoint, and MLX's Metal cos
    differs from the correctly rounded cosine the oracle uses by an fp32 ulp or more there."""
    D, heads, rot, theta = F.LAYERS[0]
    w, _ = resolved_weight(g, 0)
    kp = g["kproj0"]
    L = kp.shape[0]
    y = O.rope(O.rms_norm(kp.reshape(-1, D), w, F.EPS), L, heads, D, rot, theta, 0).reshape(L, heads, D)
    miss = np.argwhere(y != g["k0"])
    print(f"sliding layer keys: {len(miss)} of {y.size} differ: {miss.tolist()}")
    assert len(miss) <= 1
    for t, h, d in miss:
        a, b = int(y[t, h, d]), int(g["k0"][t, h, d])
        assert abs(a - b) == 1 and (a ^ b) & 0x8000 == 0
        # the fp32 value before the bf16 rounding lies within 2 fp32 ulps of the midpoint
        x = F.from_bf16(O.rms_norm(kp.reshape(-1, D), w, F.EPS).reshape(L, heads, D))
        i = d % (D // 2)
        inv = np.float32(np.power(theta, -2.0 * i / D))
        th = np.float32(np.float32(t) * inv)
        c, s = np.float32(np.cos(np.float64(th))), np.float32(np.sin(np.float64(th)))
        x1, x2 = x[t, h, i], x[t, h, i + D // 2]
        v = np.float32(x1 * c) - np.float32(x2 * s) if d < D // 2 else np.float32(x1 * s) + np.float32(x2 * c)
        low16 = int(np.float32(v).view(np.uint32)) & 0xFFFF
        assert abs(low16 - 0x8000) <= 2
