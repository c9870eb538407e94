"""ctypes view of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker and by bench.py's CPU-baseline leg. The product library never imports it.
Arrays are numpy; bf16 values travel as their uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int64


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_bf16_from_f32.restype = ctypes.c_uint16
        L.orc_bf16_from_f32.argtypes = [ctypes.c_float]
        L.orc_f32_from_bf16.restype = ctypes.c_float
        L.orc_f32_from_bf16.argtypes = [ctypes.c_uint16]
        L.orc_bf16_from_f32_array.argtypes = [_P, _I, _P]
        L.orc_f32_from_bf16_array.argtypes = [_P, _I, _P]
        L.orc_quantize_q4g64.argtypes = [_P, _I, _I, _P, _P, _P]
        L.orc_dequantize_q4g64.argtypes = [_P, _P, _P, _P, _I, _I, ctypes.c_int, _P]
        L.orc_qmatmul_f64.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P]
        L.orc_qmatmul_deq_f64.argtypes = [_P, _P, _P, _P, _I, _I, _I, ctypes.c_int, _P]
        L.orc_qmatmul_f32_grouped.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P]
        L.orc_qmatmul_mlx_cpu.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P]
        L.orc_qmatmul_mlx_cpu_rows.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _P]
        L.orc_qmatmul_mlx_cpu_mt.argtypes = [_P, _P, _P, _P, _I, _I, _I, ctypes.c_int, _P]
        L.orc_sample_greedy_bf16.argtypes = [_P, _I, _P, _P, _P]
        L.orc_sample_topk_bf16.restype = ctypes.c_uint32
        L.orc_sample_topk_bf16.argtypes = [_P, _I, ctypes.c_uint32, _P, _P]
        L.orc_gelu_tanh_bf16.argtypes = [_P, _I, _P]
        L.orc_gelu_tanh_mul_bf16.argtypes = [_P, _P, _I, _P]
        L.orc_softcap_bf16.argtypes = [_P, _I, ctypes.c_float, _P]
        L.orc_scale_bf16.argtypes = [_P, _I, ctypes.c_float, _P]
        L.orc_rms_norm_bf16.argtypes = [_P, _P, _I, _I, ctypes.c_float, _P]
        L.orc_rope_bf16.argtypes = [_P, _I, _I, _I, _I, ctypes.c_double, _I, _P]
        L.orc_attention_f64.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P]
        L.orc_det_exp.restype = ctypes.c_float
        L.orc_det_exp.argtypes = [ctypes.c_float]
        L.orc_sample_stochastic_bf16.argtypes = [_P, ctypes.c_uint32, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                                 ctypes.c_int32, ctypes.c_float, _P, _P, _P]
        _lib = L
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_P)


def bf16_from_f32(a) -> np.ndarray:
    a = _c(np.asarray(a, dtype=np.float32), np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_bf16_from_f32_array(_p(a), a.size, _p(out))
    return out


def f32_from_bf16(a) -> np.ndarray:
    a = _c(a, np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().orc_f32_from_bf16_array(_p(a), a.size, _p(out))
    return out


def quantize(w_bf16: np.ndarray):
    """mx.quantize(w, 64, 4, 'affine') -> (wq uint32 [n,k/8], scales bf16 [n,k/64], biases)."""
    w = _c(w_bf16, np.uint16)
    n, k = w.shape
    assert k % 64 == 0
    wq = np.empty((n, k // 8), np.uint32)
    s = np.empty((n, k // 64), np.uint16)
    b = np.empty((n, k // 64), np.uint16)
    lib().orc_quantize_q4g64(_p(w), n, k, _p(wq), _p(s), _p(b))
    return wq, s, b


def dequantize(wq, s, b, rows=None, mode: int = 1) -> np.ndarray:
    """mx.dequantize to bf16 bits; mode 1 (default) is MLX's single rounding bf16(s*q + b),
    mode 0 the op-composed bf16(bf16(s*q) + b) kept for comparison."""
    wq = _c(wq, np.uint32)
    s = _c(s, np.uint16)
    b = _c(b, np.uint16)
    k = wq.shape[1] * 8
    if rows is None:
        n_rows = wq.shape[0]
        rp = None
    else:
        rows = _c(rows, np.uint32)
        n_rows = rows.size
        rp = _p(rows)
    out = np.empty((n_rows, k), np.uint16)
    lib().orc_dequantize_q4g64(_p(wq), _p(s), _p(b), rp, n_rows, k, mode, _p(out))
    return out


def _mm_args(x, wq, s, b):
    x = _c(x, np.uint16)
    wq = _c(wq, np.uint32)
    s = _c(s, np.uint16)
    b = _c(b, np.uint16)
    m, k = x.shape
    n = wq.shape[0]
    assert wq.shape[1] * 8 == k and s.shape == (n, k // 64) and b.shape == s.shape
    return x, wq, s, b, m, n, k


def qmatmul_f64(x, wq, s, b) -> np.ndarray:
    x, wq, s, b, m, n, k = _mm_args(x, wq, s, b)
    y = np.empty((m, n), np.float64)
    lib().orc_qmatmul_f64(_p(x), _p(wq), _p(s), _p(b), m, n, k, _p(y))
    return y


def qmatmul_deq_f64(x, wq, s, b, mode: int = 1) -> np.ndarray:
    """fp64 matmul over the bf16-dequantized weights (mode as in dequantize)."""
    x, wq, s, b, m, n, k = _mm_args(x, wq, s, b)
    y = np.empty((m, n), np.float64)
    lib().orc_qmatmul_deq_f64(_p(x), _p(wq), _p(s), _p(b), m, n, k, mode, _p(y))
    return y


def qmatmul_f32_grouped(x, wq, s, b) -> np.ndarray:
    x, wq, s, b, m, n, k = _mm_args(x, wq, s, b)
    y = np.empty((m, n), np.float32)
    lib().orc_qmatmul_f32_grouped(_p(x), _p(wq), _p(s), _p(b), m, n, k, _p(y))
    return y


def qmatmul_mlx_cpu(x, wq, s, b, rows=None) -> np.ndarray:
    """bf16-accumulating restatement of MLX's CPU loop (parity unpinned)."""
    x, wq, s, b, m, n, k = _mm_args(x, wq, s, b)
    n0, n1 = (0, n) if rows is None else rows
    y = np.empty((m, n1 - n0), np.uint16)
    lib().orc_qmatmul_mlx_cpu_rows(_p(x), _p(wq), _p(s), _p(b), m, n0, n1, k, _p(y))
    return y


def qmatmul_mlx_cpu_mt(x, wq, s, b, threads) -> np.ndarray:
    """qmatmul_mlx_cpu over `threads` OpenMP threads (bit-identical; parity unpinned)."""
    x, wq, s, b, m, n, k = _mm_args(x, wq, s, b)
    y = np.empty((m, n), np.uint16)
    lib().orc_qmatmul_mlx_cpu_mt(_p(x), _p(wq), _p(s), _p(b), m, n, k, int(threads), _p(y))
    return y


def sample_greedy(logits):
    """ForwardPass::sample_greedy of a 1-D bf16 row -> (token_id, logit, near_tie)."""
    x = _c(logits, np.uint16).reshape(-1)
    tok = ctypes.c_uint32()
    val = ctypes.c_float()
    tie = ctypes.c_int32()
    lib().orc_sample_greedy_bf16(_p(x), x.size, ctypes.byref(tok), ctypes.byref(val), ctypes.byref(tie))
    return tok.value, val.value, bool(tie.value)


TOP_K = 8   # HYP_TOP_K_LOGPROBS (hyperion_mlx.h:145)


def sample_topk(logits, k: int = TOP_K):
    """The greedy epilogue's top-k sidecar of a 1-D bf16 row -> (count, ids uint32[k],
    values float32[k]); order: larger value, then lower index, NaN last."""
    x = _c(logits, np.uint16).reshape(-1)
    ids = np.zeros(k, np.uint32)
    vals = np.zeros(k, np.float32)
    cnt = lib().orc_sample_topk_bf16(_p(x), x.size, k, _p(ids), _p(vals))
    return int(cnt), ids, vals


def det_exp(x: float) -> float:
    """exp(x), x <= 0, as the sampling kernels compute it."""
    return float(lib().orc_det_exp(float(x)))


def sample_stochastic(logits, temperature: float, top_k: int = 0, top_p: float = 0.0, min_p: float = 0.0,
                      canon: float = 0.5):
    """ForwardPass::sample_stochastic's draw of a 1-D bf16 row with the HIP kernels' defined
    orders -> (token_id, logit, kept): kept is the size of the kept prefix (value
    descending, index ascending), 0 for a row drawn without weights. canon: the uniform in
    [0, 1) (canonical(state) for an RNG state)."""
    x = _c(logits, np.uint16).reshape(-1)
    with np.errstate(over="ignore", divide="ignore"):
        inv_temp = np.float32(1.0) / np.float32(temperature)
    tok = ctypes.c_uint32()
    val = ctypes.c_float()
    kept = ctypes.c_uint32()
    lib().orc_sample_stochastic_bf16(_p(x), x.size, float(inv_temp), float(top_p), float(min_p), int(top_k),
                                     float(canon), ctypes.byref(tok), ctypes.byref(val), ctypes.byref(kept))
    return tok.value, val.value, kept.value


_stl = None


def stl():
    """oracle/libstlsort.so: the reference's standard-library calls (libstdc++)."""
    global _stl
    if _stl is None:
        path = os.path.join(os.path.dirname(_LIB_PATH), "libstlsort.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library not built: {path} (run __graft_entry__.build())")
        S = ctypes.CDLL(path)
        S.stl_partial_sort_topk.restype = ctypes.c_uint32
        S.stl_partial_sort_topk.argtypes = [_P, _I, ctypes.c_uint32, _P]
        S.stl_canonical_mt19937_64.restype = ctypes.c_float
        S.stl_canonical_mt19937_64.argtypes = [ctypes.c_uint64]
        S.stl_uniform_real_mt19937_64.restype = ctypes.c_float
        S.stl_uniform_real_mt19937_64.argtypes = [ctypes.c_uint64, ctypes.c_float]
        S.stl_mt19937_64_nth.restype = ctypes.c_uint64
        S.stl_mt19937_64_nth.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        S.stl_sample_stochastic.restype = ctypes.c_uint32
        S.stl_sample_stochastic.argtypes = [_P, ctypes.c_uint32, ctypes.c_float, ctypes.c_int32, ctypes.c_float,
                                            ctypes.c_float, ctypes.c_uint64, _P, _P]
        _stl = S
    return _stl


def stl_partial_sort_topk(p_f32, k: int = TOP_K) -> np.ndarray:
    """libstdc++ std::partial_sort of the indices by p[a] > p[b] (model.cc:278-288): the
    first min(k, n) indices."""
    p = _c(p_f32, np.float32).reshape(-1)
    ids = np.zeros(k, np.uint32)
    cnt = stl().stl_partial_sort_topk(_p(p), p.size, k, _p(ids))
    return ids[:cnt]


def canonical(state: int) -> float:
    """std::generate_canonical<float, 24> of std::mt19937_64(state) (libstdc++)."""
    return float(stl().stl_canonical_mt19937_64(state & 0xFFFFFFFFFFFFFFFF))


def stl_uniform_real(state: int, b: float) -> float:
    """std::uniform_real_distribution<float>(0, b) drawn once from std::mt19937_64(state)."""
    return float(stl().stl_uniform_real_mt19937_64(state & 0xFFFFFFFFFFFFFFFF, b))


def mt19937_64_nth(seed: int, n: int) -> int:
    return int(stl().stl_mt19937_64_nth(seed & 0xFFFFFFFFFFFFFFFF, n))


def advance_rng(state: int) -> int:
    """The per-step RNG state advance of the sampled decode loop (model.cc:944)."""
    return (state * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF


def stl_sample_stochastic(logits_f32, temperature: float, top_k: int = 0, top_p: float = 0.0, min_p: float = 0.0,
                          rng_state: int = 0):
    """The reference's host sampler restated over libstdc++ -> (token, kept mask bool[n], u)."""
    x = _c(logits_f32, np.float32).reshape(-1)
    kept = np.zeros(x.size, np.uint8)
    u = ctypes.c_float()
    tok = stl().stl_sample_stochastic(_p(x), x.size, float(temperature), int(top_k), float(top_p), float(min_p),
                                      rng_state & 0xFFFFFFFFFFFFFFFF, _p(kept), ctypes.byref(u))
    return int(tok), kept.astype(bool), u.value


def gelu_tanh(x) -> np.ndarray:
    x = _c(x, np.uint16)
    out = np.empty(x.shape, np.uint16)
    lib().orc_gelu_tanh_bf16(_p(x), x.size, _p(out))
    return out


def gelu_tanh_mul(gate, up) -> np.ndarray:
    g = _c(gate, np.uint16)
    u = _c(up, np.uint16)
    assert g.shape == u.shape
    out = np.empty(g.shape, np.uint16)
    lib().orc_gelu_tanh_mul_bf16(_p(g), _p(u), g.size, _p(out))
    return out


def softcap(x, cap: float = 30.0) -> np.ndarray:
    x = _c(x, np.uint16)
    out = np.empty(x.shape, np.uint16)
    lib().orc_softcap_bf16(_p(x), x.size, cap, _p(out))
    return out


def scale(x, c: float) -> np.ndarray:
    x = _c(x, np.uint16)
    out = np.empty(x.shape, np.uint16)
    lib().orc_scale_bf16(_p(x), x.size, c, _p(out))
    return out


def rms_norm(x, w=None, eps: float = 1e-6) -> np.ndarray:
    """mx::fast::rms_norm over the rows of x [rows, k] (bf16 bits), w [k] or None."""
    x = _c(x, np.uint16)
    rows, k = x.shape
    out = np.empty_like(x)
    wp = _p(_c(w, np.uint16)) if w is not None else None
    lib().orc_rms_norm_bf16(_p(x), wp, rows, k, ctypes.c_float(eps), _p(out))
    return out


def rope(x, rows: int, heads: int, head_dim: int, rotated: int, base: float, offset: int) -> np.ndarray:
    """mx::fast::rope (non-traditional) of x [rows, heads, head_dim] (bf16 bits)."""
    x = _c(x, np.uint16).reshape(rows, heads, head_dim)
    out = np.empty_like(x)
    lib().orc_rope_bf16(_p(x), rows, heads, head_dim, rotated, ctypes.c_double(base), offset, _p(out))
    return out


def attention_f64(q, k, v, cache_k, cache_v, offset: int, prefix_len: int, window: int) -> np.ndarray:
    """ForwardPass::attention's SDPA (scale 1, causal + sliding window, GQA) in fp64:
    q [L, H, D], k/v [L, KVH, D] (the chunk), cache_k/cache_v [cap, KVH, D] (slot = pos % cap,
    positions [offset - prefix_len, offset) read) -> [L, H, D] float64."""
    q = _c(q, np.uint16)
    k = _c(k, np.uint16)
    v = _c(v, np.uint16)
    ck = _c(cache_k, np.uint16)
    cv = _c(cache_v, np.uint16)
    L, H, D = q.shape
    KVH = k.shape[1]
    cap = ck.shape[0]
    out = np.zeros((L, H, D), np.float64)
    lib().orc_attention_f64(_p(q), _p(k), _p(v), _p(ck), _p(cv), cap, L, H, KVH, D, offset, prefix_len, window, _p(out))
    return out


def add_bf16(a, b) -> np.ndarray:
    """mx::add of two bf16 arrays: the fp32 sum rounded to bf16."""
    return bf16_from_f32(f32_from_bf16(a) + f32_from_bf16(b))


def mul_bf16(a, b) -> np.ndarray:
    """mx::multiply of two bf16 arrays (b broadcast): the fp32 product rounded to bf16."""
    return bf16_from_f32(f32_from_bf16(a) * f32_from_bf16(b))


class DecoderOracle:
    """ForwardPass (native/hyperion_mlx/src/forward.cc) restated over this module's pinned
    primitives, every MLX op's bf16 result rounded where the reference's graph rounds it:

      embed           forward.cc:126-131   dequantize (double rounding) x bf16(sqrt(hidden))
      decoder_layer   forward.cc:509-541   the sandwich norms, the residual adds, layer_scalar
      attention       forward.cc:376-508   q/k/v projections (fp64 products rounded to bf16),
                                           q_norm/k_norm (weighted), v_norm (weightless, of
                                           k_raw on K = V layers), RoPE on q and k, SDPA at
                                           scale 1 over the cached prefix and the chunk
                                           (attention_f64, rounded to bf16), o_proj
      mlp             forward.cc:338-343   gate/up, the GELU chain times up, down
      forward         forward.cc:543-563   every layer at one offset, then final_norm
      lm_head/epilogue forward.cc:137-189, model.cc:215-228: tied head, softcap, greedy

    `tensors` maps the artifact's mlx-lm names to arrays (uint32 codes, bf16 bits as
    uint16). Caches are linear per layer (position p in row p); the masks alone bound a
    sliding layer's window, which is what the reference's ring read returns.

    weights="exact" multiplies by the exactly dequantized weights at every size;
    weights="per_m" follows the device path's documented weight semantics - exact below
    five rows (the decode kernel), each weight rounded once to bf16 from five rows on (the
    prefill GEMM) - so that a comparison with the device isolates everything else.
    """

    PREFIX = "language_model.model."

    def __init__(self, tensors: dict, text_config: dict, weights: str = "exact"):
        assert weights in ("exact", "per_m")
        self.weights = weights
        t = text_config
        self.T = tensors
        self.hidden = t["hidden_size"]
        self.heads = t["num_attention_heads"]
        self.kinds = ["sliding" if k == "sliding_attention" else "full" for k in t["layer_types"]]
        self.d_local, self.d_global = t["head_dim"], t.get("global_head_dim", t["head_dim"])
        self.kv_local = t["num_key_value_heads"]
        self.kv_global = t.get("num_global_key_value_heads", self.kv_local)
        self.window = t["sliding_window"]
        rp = t["rope_parameters"]
        self.theta_local = rp["sliding_attention"]["rope_theta"]
        self.theta_global = rp["full_attention"]["rope_theta"]
        prf = np.float32(rp["full_attention"].get("partial_rotary_factor", 1.0))
        rotated = int(np.float32(prf * np.float32(self.d_global)))   # rope.cc:44-49
        self.rotated_global = rotated - rotated % 2
        self.eps = t["rms_norm_eps"]
        self.softcap_cap = t["final_logit_softcapping"]
        self.vocab = t["vocab_size"]
        self.max_pos = t["max_position_embeddings"]
        self.caches = []
        for kind in self.kinds:
            d, kvh = (self.d_local, self.kv_local) if kind == "sliding" else (self.d_global, self.kv_global)
            self.caches.append((np.zeros((self.max_pos, kvh, d), np.uint16), np.zeros((self.max_pos, kvh, d), np.uint16)))

    def _t(self, name):
        return self.T[self.PREFIX + name]

    def _proj(self, x, base):
        wq, s, b = (self._t(base + suffix) for suffix in (".weight", ".scales", ".biases"))
        if self.weights == "per_m" and x.shape[0] > 4:
            return bf16_from_f32(qmatmul_deq_f64(x, wq, s, b, mode=1).astype(np.float32))
        return bf16_from_f32(qmatmul_f64(x, wq, s, b).astype(np.float32))

    def embed(self, ids):
        base = "embed_tokens"
        rows = dequantize(self._t(base + ".weight"), self._t(base + ".scales"), self._t(base + ".biases"),
                          rows=np.asarray(ids, np.uint32))
        return scale(rows, float(np.sqrt(np.float32(self.hidden))))

    def layer(self, x, i, offset):
        L = x.shape[0]
        pre = f"layers.{i}."
        sliding = self.kinds[i] == "sliding"
        d, kvh = (self.d_local, self.kv_local) if sliding else (self.d_global, self.kv_global)
        rotated = d if sliding else self.rotated_global
        theta = self.theta_local if sliding else self.theta_global
        h = rms_norm(x, self._t(pre + "input_layernorm.weight"), self.eps)
        q = self._proj(h, pre + "self_attn.q_proj")
        k_raw = self._proj(h, pre + "self_attn.k_proj")
        v_raw = self._proj(h, pre + "self_attn.v_proj") if sliding else k_raw
        q = rms_norm(q.reshape(L * self.heads, d), self._t(pre + "self_attn.q_norm.weight"), self.eps)
        k = rms_norm(k_raw.reshape(L * kvh, d), self._t(pre + "self_attn.k_norm.weight"), self.eps)
        v = rms_norm(v_raw.reshape(L * kvh, d), None, self.eps).reshape(L, kvh, d)
        q = rope(q, L, self.heads, d, rotated, theta, offset)
        k = rope(k, L, kvh, d, rotated, theta, offset)
        ck, cv = self.caches[i]
        prefix = min(self.window, offset) if sliding else offset
        att = attention_f64(q, k, v, ck, cv, offset, prefix, self.window if sliding else 0)
        ck[offset:offset + L] = k
        cv[offset:offset + L] = v
        att = bf16_from_f32(att.astype(np.float32)).reshape(L, self.heads * d)
        o = self._proj(att, pre + "self_attn.o_proj")
        x = add_bf16(x, rms_norm(o, self._t(pre + "post_attention_layernorm.weight"), self.eps))
        h = rms_norm(x, self._t(pre + "pre_feedforward_layernorm.weight"), self.eps)
        gu = gelu_tanh_mul(self._proj(h, pre + "mlp.gate_proj"), self._proj(h, pre + "mlp.up_proj"))
        dn = self._proj(gu, pre + "mlp.down_proj")
        x = add_bf16(x, rms_norm(dn, self._t(pre + "post_feedforward_layernorm.weight"), self.eps))
        return mul_bf16(x, self._t(pre + "layer_scalar"))

    def forward(self, ids, offset: int):
        """Final-normalised hidden rows [L, hidden] (bf16 bits); appends the K/V."""
        x = self.embed(ids)
        for i in range(len(self.kinds)):
            x = self.layer(x, i, offset)
        return rms_norm(x, self._t("norm.weight"), self.eps)

    def logits(self, last_row):
        """Tied LM head + softcap of one final-normalised row (bf16 bits [vocab])."""
        return softcap(self._proj(last_row.reshape(1, -1), "embed_tokens"), self.softcap_cap).reshape(-1)

    def greedy(self, ids, n_decode: int):
        """hyp_prefill_chunk then n_decode single-token steps: [(token, logit, top1 - top2)]."""
        steps = []
        h = self.forward(ids, 0)
        pos = len(ids)
        for j in range(n_decode + 1):
            lg = self.logits(h[-1])
            f = f32_from_bf16(lg).astype(np.float64)
            order = np.argsort(-f, kind="stable")
            tok = int(order[0])
            steps.append((tok, float(f[tok]), float(f[order[0]] - f[order[1]]) if f.size > 1 else np.inf))
            if j == n_decode:
                break
            h = self.forward([tok], pos)
            pos += 1
        return steps
