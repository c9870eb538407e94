"""The synthetic 12B decode step over the C ABI: 48 decoder layers of Q4/g64 linears plus
the tied LM head, with the activation chain reduced to plain matmuls between layers.

This is the full-decode weight stream of the benchmark workload (random-init weights of
the Gemma-class 12B shapes, seeded per projection) as the reference's decode loop drives
it: the layer loop of ForwardPass::forward (native/hyperion_mlx/src/forward.cc:558-563)
inside hyp_decode_block (model.cc:703-718), then the greedy epilogue with its top-8
sidecar (run_epilogue_sampled at temperature 0, model.cc:262-288: LM head, softcap, greedy
sample, the 8 largest logits and their ids). Attention, the KV cache and the
residual adds are not on the quantized-linear path; between the projections each
output feeds the next projection directly, and the hidden state is renormalised
(weightless RMS norm) before each layer's q/k/v, so values stay N(0, 1)-sized over 48
layers.

Per layer, in launch order:
  1. q, k, v of the renormalised hidden state h      (hyp_qmatmul_group_rmsnorm)
  2. o from q's output                               (hyp_qmatmul)
  3. gelu_tanh(gate(o)) * up(o)                       (hyp_qmlp_gate_up_gelu)
  4. down of that into h                              (hyp_qmatmul)
then h renormalised, the softcap LM head and greedy sampling of every row with the top-8
sidecar (hyp_sample_greedy_topk): nothing of the logits leaves the device.
"""
from __future__ import annotations

import time

import numpy as np

from . import synthetic as syn

RMS_EPS = 1e-6
SOFTCAP = 30.0
LAUNCHES_PER_LAYER = 4
HEAD_SEED = 9_999


def layer_seed(layer: int, proj_index: int) -> int:
    """Seed of projection `proj_index` (the order of synthetic.LAYER_SHAPES) of `layer`."""
    return 10_000 + 16 * layer + proj_index


def layer_weights(layer: int, name: str):
    """(w, scales, biases) of one projection of the synthetic model (MLX layout, host)."""
    idx = list(syn.LAYER_SHAPES).index(name)
    n, k = syn.LAYER_SHAPES[name]
    return syn.q4_weights(n, k, seed=layer_seed(layer, idx))


def head_weights():
    return syn.q4_weights(syn.VOCAB, syn.HIDDEN, seed=HEAD_SEED)


def q4_bytes(n: int, k: int) -> int:
    """Packed codes (0.5 B/weight) + bf16 scale and bias per 64 weights."""
    return n * k // 2 + 4 * n * (k // 64)


class DecodeModel:
    """Random-init Q4 weights of a Gemma-class 12B decoder's linear layers (every layer
    with v_proj) and its tied embedding table, resident in HBM."""

    def __init__(self, hy, layers: int, log=None):
        self.hy = hy
        self.layers = []
        t0 = time.perf_counter()
        for li in range(layers):
            self.layers.append({name: hy.QWeight.from_host(*layer_weights(li, name)) for name in syn.LAYER_SHAPES})
        self.embed = hy.QWeight.from_host(*head_weights())
        self.weight_bytes = layers * sum(q4_bytes(n, k) for n, k in syn.LAYER_SHAPES.values()) + \
            q4_bytes(syn.VOCAB, syn.HIDDEN)
        if log is not None:
            log(f"decode model: {layers} layers + LM head, {self.weight_bytes / 1e9:.2f} GB of Q4 weights "
                f"({time.perf_counter() - t0:.1f} s to build)")

    def close(self):
        for proj in self.layers:
            for q in proj.values():
                q.close()
        self.embed.close()


class StepBuffers:
    """Device buffers of one decode step at batch m: the hidden state h, the q/k/v, o
    and gate/up outputs, the logits and the greedy samples."""

    def __init__(self, hy, m: int, h0: np.ndarray, stream):
        self.m = m
        self.h = hy.DeviceArray.from_host(h0, stream)
        self.q = hy.DeviceArray((m, 4096), np.uint16)
        self.k = hy.DeviceArray((m, 2048), np.uint16)
        self.v = hy.DeviceArray((m, 2048), np.uint16)
        self.o = hy.DeviceArray((m, syn.HIDDEN), np.uint16)
        self.g = hy.DeviceArray((m, 15360), np.uint16)
        self.logits = hy.DeviceArray((m, syn.VOCAB), np.uint16)
        self.samples = hy.DeviceArray((m, 20), np.uint32)   # HypTopKSample, 80 bytes a row

    def close(self):
        for a in (self.h, self.q, self.k, self.v, self.o, self.g, self.logits, self.samples):
            a.close()


def decode_layer(hy, proj, m: int, b: StepBuffers, stream) -> None:
    """One layer's four launches (module docstring)."""
    hy.qmatmul_group([proj["q"], proj["k"], proj["v"]], b.h, m, [b.q, b.k, b.v], stream, rms_eps=RMS_EPS)
    hy.qmatmul(proj["o"], b.q, m, b.o, stream)
    hy.qmlp_gate_up_gelu(proj["gate"], proj["up"], b.o, m, b.g, stream)
    hy.qmatmul(proj["down"], b.g, m, b.h, stream)


def decode_layers(model: DecodeModel, m: int, b: StepBuffers, stream) -> None:
    for proj in model.layers:
        decode_layer(model.hy, proj, m, b, stream)


def lm_head(model: DecodeModel, m: int, b: StepBuffers, stream) -> None:
    """The last hidden state renormalised, the tied LM head with softcap 30, then greedy
    sampling of every row with its top-8 sidecar on the device (model.cc:262-288)."""
    hy = model.hy
    hy.rms_normalize(b.h, m, syn.HIDDEN, b.h, stream, eps=RMS_EPS)
    hy.qmatmul(model.embed, b.h, m, b.logits, stream, softcap=SOFTCAP)
    hy.sample_greedy_topk(b.logits, m, syn.VOCAB, b.samples, stream)


def layer_program(model: DecodeModel, m: int, b: StepBuffers, spin_limit: int = 0):
    """The layer stack as one decode-step program (hyp_step_program_*): the same four ops
    per layer as decode_layer, run by one persistent launch with the same output bits."""
    hy = model.hy
    ops = []
    for proj in model.layers:
        ops.append((hy.STEP_QMATMUL_RMSNORM, [proj["q"], proj["k"], proj["v"]], b.h, [b.q, b.k, b.v], RMS_EPS))
        ops.append((hy.STEP_QMATMUL, [proj["o"]], b.q, [b.o], 0.0))
        ops.append((hy.STEP_GATE_UP_GELU, [proj["gate"], proj["up"]], b.o, [b.g], 0.0))
        ops.append((hy.STEP_QMATMUL, [proj["down"]], b.g, [b.h], 0.0))
    return hy.StepProgram(ops, m, spin_limit)


def decode_step(model: DecodeModel, m: int, b: StepBuffers, stream) -> None:
    decode_layers(model, m, b, stream)
    lm_head(model, m, b, stream)


def step_activation_bytes(layers: int, m: int) -> int:
    """Activation bytes of one step: per layer x, q/k/v, o, gate/up, down read or
    written; then the head's x, logits written and read back by the sampler, and 80
    bytes of sample per row."""
    h = syn.HIDDEN
    return 2 * m * (layers * (h * 3 + 4096 * 2 + 2048 * 2 + h * 2 + 15360 * 3) + h + 2 * syn.VOCAB) + 80 * m
