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


def dequantize(wq, s, b, rows=None, mode: int = 0) -> np.ndarray:
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


_stl = None


def stl_partial_sort_topk(p_f32, k: int = TOP_K) -> np.ndarray:
    """libstdc++ std::partial_sort of the indices by p[a] > p[b] (model.cc:278-288): the
    first min(k, n) indices."""
    global _stl
    if _stl is None:
        path = os.path.join(os.path.dirname(_LIB_PATH), "libstlsort.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library not built: {path} (run __graft_entry__.build())")
        _stl = ctypes.CDLL(path)
        _stl.stl_partial_sort_topk.restype = ctypes.c_uint32
        _stl.stl_partial_sort_topk.argtypes = [_P, _I, ctypes.c_uint32, _P]
    p = _c(p_f32, np.float32).reshape(-1)
    ids = np.zeros(k, np.uint32)
    cnt = _stl.stl_partial_sort_topk(_p(p), p.size, k, _p(ids))
    return ids[:cnt]


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
