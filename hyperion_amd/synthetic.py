"""Seeded synthetic workloads for the Q4/g64 path (numpy, host side).

The reference's own benchmark draws its inputs with mx.random (scripts/nax-probe.py:67-90);
MLX's generator cannot run here, so these generators use numpy's PCG64 with fixed
seeds. Shapes and distributions are the benchmark configurations of this path:

  decode GEMV      x bf16 N(0,1); codes q ~ U{0..15} packed 8 per uint32, lowest k in
                   the lowest nibble; scale = bf16(|N(0,1)| * 0.02 / 7.5); bias = -8 * scale
  quantize/pack    W bf16 N(0, 0.02^2) with 1% of entries multiplied by 8 (outliers)
  layer stack      q [4096,3840], k/v [2048,3840], o [3840,4096], gate/up [15360,3840],
                   down [3840,15360]
"""
from __future__ import annotations

import numpy as np

# Gemma-class 12B decoder layer projections: name -> (out_features n, in_features k).
LAYER_SHAPES = {
    "q": (4096, 3840),
    "k": (2048, 3840),
    "v": (2048, 3840),
    "o": (3840, 4096),
    "gate": (15360, 3840),
    "up": (15360, 3840),
    "down": (3840, 15360),
}
HIDDEN = 3840
VOCAB = 262144
NUM_LAYERS = 48


def bf16_bits(a) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (NaN stays NaN)."""
    f = np.ascontiguousarray(a, dtype=np.float32)
    u = f.view(np.uint32)
    rounded = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        rounded = np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), rounded)
    return rounded


def bf16_to_f32(h) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def pack_codes(q: np.ndarray) -> np.ndarray:
    """codes uint8 [n, k] (0..15) -> MLX packed uint32 [n, k/8], low nibble first."""
    n, k = q.shape
    q = q.reshape(n, k // 8, 8).astype(np.uint32)
    out = np.zeros((n, k // 8), np.uint32)
    for e in range(8):
        out |= q[:, :, e] << np.uint32(4 * e)
    return out


def unpack_codes(w: np.ndarray) -> np.ndarray:
    n, kw = w.shape
    out = np.empty((n, kw, 8), np.uint8)
    for e in range(8):
        out[:, :, e] = (w >> np.uint32(4 * e)) & np.uint32(0xF)
    return out.reshape(n, kw * 8)


def activations(m: int, k: int, seed: int) -> np.ndarray:
    """x bf16 [m, k] ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    return bf16_bits(rng.standard_normal((m, k), dtype=np.float32))


def q4_weights(n: int, k: int, seed: int):
    """(w uint32 [n,k/8], scales bf16 [n,k/64], biases bf16 [n,k/64]) as the decode config."""
    assert k % 64 == 0
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    s = bf16_bits(np.abs(rng.standard_normal((n, k // 64), dtype=np.float32)) * np.float32(0.02 / 7.5))
    b = bf16_bits(bf16_to_f32(s) * np.float32(-8.0))   # exact: a power-of-two multiple
    return w, s, b


def quantize_input(n: int, k: int, seed: int) -> np.ndarray:
    """bf16 [n, k] ~ N(0, 0.02^2), 1% of entries (Bernoulli 0.01) multiplied by 8 (exact)."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    w = bf16_to_f32(bf16_bits(w))
    outlier = rng.random((n, k), dtype=np.float32) < np.float32(0.01)
    w = np.where(outlier, w * np.float32(8.0), w)
    return bf16_bits(w)


def sig_rel(got, ref) -> float:
    """max|got - ref| / max|ref| (native/hyperion_mlx/tests/forward_12b_test.cc:148-161)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    md = float(np.max(np.abs(got - ref))) if got.size else 0.0
    mo = float(np.max(np.abs(ref))) if ref.size else 0.0
    return md / mo if mo > 0 else md
