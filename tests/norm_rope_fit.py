"""The reference's 12B keys and values as checks of RMSNorm and RoPE.

The golden (`tests/golden/gemma4-12b-hidden/golden.safetensors`) holds, for the first sliding
layer (0) and the first global layer (5) of MLX's own 12B forward, the raw k_proj output next
to the keys formed from it - k_norm (RMSNorm with a learned weight), then RoPE at positions
0..9 - and, on the global layer, the values, v_norm (weightless RMSNorm) of the same k_proj
output (forward.cc:395-418; rope.cc:16-75; gen_12b_hidden_golden.py). The k_norm weights are
part of the 12B checkpoint and absent here, but RoPE leaves position 0 unrotated, so each
dimension's weight is pinned down by its position-0 values (8 heads share it on the sliding
layer); the dimensions RoPE never rotates (75% of the global layer's) must then fit all ten
positions with that one weight, and the rotated ones test RoPE at positions 1..9.

`recover_k_norm_weight` finds, per dimension, the bf16 weights w with bf16(w * n) equal to the
golden key wherever the dimension is unrotated, n being the weightless normalisation (the
oracle's, itself held to the golden values separately); numpy only.
"""
import os

import numpy as np

import st_reader

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemma4-12b-hidden",
                      "golden.safetensors")

# (layer, head_dim, kv heads, rotated dims, rope theta) as the 12B's config gives them.
LAYERS = {0: (256, 8, 256, 10000.0), 5: (512, 1, 128, 1000000.0)}
EPS = 1e-6


def load():
    """{name: bf16 bits}: kproj [L, heads * D], k [L, heads, D] per layer, and v5 [L, D]."""
    t = {k: v for k, (_, v) in st_reader.read(GOLDEN).items()}
    out = {}
    for layer, (D, heads, _, _) in LAYERS.items():
        kp = t[f"layer_{layer:02d}_kproj"][0]
        out[f"kproj{layer}"] = kp.copy()
        out[f"k{layer}"] = t[f"layer_{layer:02d}_k"][0].transpose(1, 0, 2).copy()   # [L, heads, D]
    out["v5"] = t["layer_05_v"][0, 0].copy()
    return out


def to_bf16(x) -> np.ndarray:
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bf16(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def unrotated_dims(D: int, rotated: int) -> np.ndarray:
    """Dimensions RoPE leaves alone at every position: pairs (i, i + D/2) with 2 i >= rotated."""
    half = D // 2
    i = np.arange(half)
    keep = 2 * i >= rotated
    return np.concatenate([i[keep], i[keep] + half])


def recover_k_norm_weight(n_bits: np.ndarray, k_bits: np.ndarray, D: int, rotated: int):
    """n_bits, k_bits [L, heads, D]. Returns {dim: array of bf16 weight bits} with every weight
    w such that bf16(w * n) == k at position 0 (all heads) and, for unrotated dims, at every
    position."""
    n = from_bf16(n_bits)
    free = set(unrotated_dims(D, rotated).tolist())
    out = {}
    for d in range(D):
        rows = slice(None) if d in free else slice(0, 1)
        nn = n[rows, :, d].reshape(-1)
        kk = k_bits[rows, :, d].reshape(-1)
        live = nn != 0
        if not live.any():
            out[d] = np.zeros(0, np.uint16)
            continue
        j = int(np.argmax(np.abs(nn)))
        est = to_bf16(from_bf16(kk[j:j + 1]) / nn[j])[0]
        sign = est & 0x8000
        mag = np.arange(max(0, int(est & 0x7FFF) - 6), min(0x7F80, int(est & 0x7FFF) + 7), dtype=np.uint32)
        cand = (mag | sign).astype(np.uint16)
        with np.errstate(over="ignore", invalid="ignore"):
            prod = to_bf16(from_bf16(cand)[:, None] * nn[None, :])
        ok = (prod == kk[None, :]).all(axis=1)
        out[d] = cand[ok]
    return out
