"""Which bf16 rounding MLX's dequantize uses, recovered from the reference's 12B embed golden.

The golden (`tests/golden/gemma4-12b-hidden/golden.safetensors`, copied from the reference's
`native/hyperion_mlx/tests/fixtures/12b_hidden_golden.safetensors`) holds MLX's
`ForwardPass::embed` of ten prompt tokens on the real 12B (forward.cc:126-131,
weights_loader.cc:52-69): e = bf16(d * 62) for every element, where d is the bf16 output of
`mx::dequantize` and 62 = bf16(sqrt(3840)). The 12B weights themselves are absent, but each
64-element group of a row holds at most 16 distinct levels, one bf16 scale s and one bf16 bias
b, and the quantize rule puts q = 0 on one extreme of the group (the bias is the edge value,
d(0) = b exactly under either rounding). So for every group the candidates are few:

- b: every bf16 value with bf16(b * 62) equal to the group's smallest or largest value;
- s: every bf16 value of the matching sign whose magnitude lies between 1/15 and 1 of the
  group's range (a 3% margin each side), since the far extreme is q * s away with 1 <= q <= 15.

A group "fits" a rounding when some candidate pair maps every observed value onto one of its
16 levels bf16(dequant(s, q, b) * 62). The two roundings compared are

- "single": bf16(s*q + b) in fp32 (s*q is exact in fp32: 8-bit times 4-bit significands);
- "double": bf16(bf16(s*q) + b), one rounding per composed MLX op.

Everything here is numpy, independent of the oracle's C code, so it can check that code.
"""
import os

import numpy as np

import st_reader

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemma4-12b-hidden",
                      "golden.safetensors")
HIDDEN = 3840
EMBED_SCALE = np.float32(62.0)   # bf16(sqrt(3840)): 61.97 rounds to 62 with 8 significant bits


def load():
    """(ids int32 [10], embed bf16 bits [10, 3840]) of the golden."""
    t = st_reader.read(GOLDEN)
    return t["ids"][1].copy(), t["embed"][1].reshape(-1, HIDDEN).copy()


def to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (no NaN inputs arise here)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bf16(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


_ALL = np.arange(65536, dtype=np.uint32).astype(np.uint16)
_ALLF = from_bf16(_ALL)
_FIN = np.isfinite(_ALLF) & (_ALLF != 0)
with np.errstate(over="ignore", invalid="ignore"):
    _SCALED = to_bf16(np.where(np.isfinite(_ALLF), _ALLF * EMBED_SCALE, 0))
_Q = np.arange(16, dtype=np.float32)


def levels(s, b, rounding: str) -> np.ndarray:
    """bf16 bits of bf16(dequant(s, q, b) * 62) for q = 0..15; s, b float32 arrays of one shape."""
    sq = s[..., None] * _Q                     # exact in fp32
    if rounding == "single":
        d = from_bf16(to_bf16(sq + b[..., None]))
    else:
        d = from_bf16(to_bf16(from_bf16(to_bf16(sq)) + b[..., None]))
    return to_bf16(d * EMBED_SCALE)


def fit_group(obs_bits: np.ndarray, rounding: str):
    """(s_bits, b_bits, levels[16]) of the first candidate pair that reproduces every value of
    one group under `rounding`, or None."""
    obs = np.unique(obs_bits)
    of = from_bf16(obs)
    lo, hi = float(of.min()), float(of.max())
    span = (hi - lo) / float(EMBED_SCALE)
    if span == 0.0:
        return None
    for edge, sign in ((lo, 1.0), (hi, -1.0)):
        bc = _ALL[_FIN & (_SCALED == to_bf16(np.float32(edge)))]
        mag = np.abs(_ALLF)
        sc = _ALL[_FIN & (mag >= span / 15 * 0.97) & (mag <= span * 1.03) & (np.sign(_ALLF) == sign)]
        if bc.size == 0 or sc.size == 0:
            continue
        sb = np.broadcast_to(from_bf16(sc)[None, :], (bc.size, sc.size))
        bb = np.broadcast_to(from_bf16(bc)[:, None], (bc.size, sc.size))
        lev = levels(sb, bb, rounding)                                  # [nb, ns, 16]
        ok = (lev[..., :, None] == obs).any(axis=-2).all(axis=-1)       # [nb, ns]
        hits = np.argwhere(ok)
        if hits.size:
            i, j = hits[0]
            return int(sc[j]), int(bc[i]), lev[i, j]
    return None


def classify(embed_bits: np.ndarray):
    """Counts of groups fitting only single, only double, both, neither rounding."""
    out = {"single": 0, "double": 0, "both": 0, "neither": 0}
    rows, k = embed_bits.shape
    for r in range(rows):
        for g in range(k // 64):
            obs = embed_bits[r, g * 64:(g + 1) * 64]
            a = fit_group(obs, "single") is not None
            b = fit_group(obs, "double") is not None
            out["both" if a and b else "single" if a else "double" if b else "neither"] += 1
    return out


def fitted_rows(embed_bits: np.ndarray):
    """Q4/g64 rows (codes packed low nibble first [rows, k/8] uint32, scales and biases bf16
    [rows, k/64]) whose single-rounded dequantize times 62 reproduces embed_bits; raises if a
    group does not fit."""
    rows, k = embed_bits.shape
    codes = np.zeros((rows, k), np.uint32)
    scales = np.zeros((rows, k // 64), np.uint16)
    biases = np.zeros((rows, k // 64), np.uint16)
    for r in range(rows):
        for g in range(k // 64):
            obs = embed_bits[r, g * 64:(g + 1) * 64]
            f = fit_group(obs, "single")
            if f is None:
                raise AssertionError(f"row {r} group {g} fits no single-rounded dequantize")
            s, b, lev = f
            scales[r, g], biases[r, g] = s, b
            codes[r, g * 64:(g + 1) * 64] = np.argmax(lev[None, :] == obs[:, None], axis=1)
    packed = np.zeros((rows, k // 8), np.uint32)
    for e in range(8):
        packed |= codes[:, e::8] << np.uint32(4 * e)
    return packed, scales, biases
