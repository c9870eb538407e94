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

import os

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


# Gemma 4 text_config of the 12B (crates/hyperion-model/src/geometry.rs:466-500) with the
# layer count and context as parameters; the tiny fixture's config.json has the same keys.
def gemma4_text_config(num_layers: int = 48, vocab: int = VOCAB, max_positions: int = 262144,
                       layer_types=None) -> dict:
    if layer_types is None:   # five sliding layers, then a global one
        layer_types = ["full_attention" if (i + 1) % 6 == 0 else "sliding_attention" for i in range(num_layers)]
    return {
        "model_type": "gemma4_unified_text", "hidden_size": HIDDEN, "intermediate_size": 15360,
        "num_hidden_layers": num_layers, "layer_types": list(layer_types), "num_attention_heads": 16,
        "head_dim": 256, "global_head_dim": 512, "num_key_value_heads": 8, "num_global_key_value_heads": 1,
        "attention_k_eq_v": True, "num_kv_shared_layers": 0, "sliding_window": 1024,
        "rope_parameters": {"sliding_attention": {"rope_theta": 10000.0, "rope_type": "default"},
                            "full_attention": {"rope_theta": 1000000.0, "partial_rotary_factor": 0.25,
                                               "rope_type": "proportional"}},
        "final_logit_softcapping": 30.0, "rms_norm_eps": 1e-6, "attention_bias": False, "vocab_size": vocab,
        "max_position_embeddings": max_positions, "tie_word_embeddings": True, "hidden_size_per_layer_input": 0,
        "vocab_size_per_layer_input": 0, "use_double_wide_mlp": False, "enable_moe_block": False,
    }


def _q4_random(rng, n: int, k: int):
    """Random Q4/g64 codes whose dequantized rows have std ~ 1/sqrt(k): q ~ U{0..15},
    scale = bf16(u / (4.61 sqrt(k))) with u ~ U(0.5, 1.5), bias = bf16(-7.5 * scale)."""
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    u = rng.uniform(0.5, 1.5, size=(n, k // 64)).astype(np.float32)
    s = bf16_bits(u / np.float32(4.61 * np.sqrt(k)))
    b = bf16_bits(bf16_to_f32(s) * np.float32(-7.5))
    return w, s, b


def write_safetensors(path: str, tensors: dict, holes=()) -> None:
    """{name: numpy array} -> one safetensors file (U32 for uint32, BF16 for uint16 bit
    patterns). Tensors named in `holes` are not written: the file keeps a hole there, which
    reads as zeros (their arrays give only the shape and dtype)."""
    import json
    header, offset, blobs = {}, 0, []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a)
        dt = {np.dtype(np.uint32): "U32", np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32"}[a.dtype]
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [offset, offset + a.nbytes]}
        offset += a.nbytes
        blobs.append((name, a))
    raw = json.dumps(header).encode()
    raw += b" " * (-len(raw) % 8)
    holes = set(holes)
    with open(path, "wb") as f:
        f.write(np.uint64(len(raw)).tobytes())
        f.write(raw)
        for name, a in blobs:
            if name in holes:
                f.seek(a.nbytes, os.SEEK_CUR)
            else:
                a.tofile(f)
        f.truncate(8 + len(raw) + offset)


def write_model(directory: str, text_config: dict, seed: int, branch_gain: float = 1.0,
                qk_gain: float = 1.0, share_layers: bool = False, zero_layer_codes: bool = False) -> dict:
    """A random-init Gemma 4 artifact in the mlx-lm layout (config.json + one safetensors
    shard): Q4/g64 projections of unit-gain rows; input, pre-feedforward and final norm
    weights bf16(1 + 0.1 N(0,1)); the post-attention and post-feedforward norms (the
    branches added to the residual stream) around branch_gain; q_norm and k_norm around
    qk_gain * head_dim^-1/4 (so the scale-1 attention scores have a standard deviation of
    about qk_gain^2); layer scalars bf16(U(0.6, 1.0)). share_layers writes the first sliding
    and the first global layer's arrays again for every later layer of the same kind (a
    48-layer artifact is then generated at the cost of two layers; each layer still has its
    own tensors in the file). zero_layer_codes leaves every layer's packed codes as holes in
    the file (all codes 0: each weight is its group's bias), which keeps a 6.6 GB artifact
    cheap to write where only the byte traffic matters. Returns the tensors written."""
    import json
    t = text_config
    rng = np.random.default_rng(seed)
    hidden, inter, heads = t["hidden_size"], t["intermediate_size"], t["num_attention_heads"]
    P = "language_model.model."
    out = {}

    def proj(name, n, k):
        w, s, b = _q4_random(rng, n, k)
        out[name + ".weight"], out[name + ".scales"], out[name + ".biases"] = w, s, b

    def vec(name, n, around=1.0, spread=0.1):
        out[name] = bf16_bits(np.float32(around) + np.float32(spread) * rng.standard_normal(n).astype(np.float32))

    proj(P + "embed_tokens", t["vocab_size"], hidden)
    first = {}
    for i, kind in enumerate(t["layer_types"]):
        sliding = kind == "sliding_attention"
        if share_layers and kind in first:
            src = f"{P}layers.{first[kind]}."
            for name in [n for n in out if n.startswith(src)]:
                out[f"{P}layers.{i}." + name[len(src):]] = out[name]
            continue
        first[kind] = i
        d = t["head_dim"] if sliding else t.get("global_head_dim", t["head_dim"])
        kvh = t["num_key_value_heads"] if sliding else t.get("num_global_key_value_heads", t["num_key_value_heads"])
        a = f"{P}layers.{i}.self_attn."
        proj(a + "q_proj", heads * d, hidden)
        proj(a + "k_proj", kvh * d, hidden)
        if sliding:
            proj(a + "v_proj", kvh * d, hidden)
        proj(a + "o_proj", hidden, heads * d)
        qk = qk_gain * d ** -0.25
        vec(a + "q_norm.weight", d, qk, 0.1 * qk)
        vec(a + "k_norm.weight", d, qk, 0.1 * qk)
        m = f"{P}layers.{i}."
        proj(m + "mlp.gate_proj", inter, hidden)
        proj(m + "mlp.up_proj", inter, hidden)
        proj(m + "mlp.down_proj", hidden, inter)
        for norm in ("input_layernorm", "pre_feedforward_layernorm"):
            vec(m + norm + ".weight", hidden)
        for norm in ("post_attention_layernorm", "post_feedforward_layernorm"):
            vec(m + norm + ".weight", hidden, branch_gain, 0.1 * branch_gain)
        out[m + "layer_scalar"] = bf16_bits(rng.uniform(0.6, 1.0, size=1).astype(np.float32))
    vec(P + "norm.weight", hidden)
    os.makedirs(directory, exist_ok=True)
    holes = [n for n in out if zero_layer_codes and ".layers." in n and n.endswith("_proj.weight")]
    write_safetensors(os.path.join(directory, "model.safetensors"), out, holes)
    for n in holes:   # what the file holds there (a read-only view, no memory)
        out[n] = np.broadcast_to(np.uint32(0), out[n].shape)
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump({"model_type": "gemma4_unified", "tie_word_embeddings": True,
                   "quantization": {"group_size": 64, "bits": 4, "mode": "affine"}, "text_config": t}, f)
    return out
