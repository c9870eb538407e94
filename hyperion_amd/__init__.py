"""Python binding of the gfx950 Q4/g64 quantized-linear engine (libhyperion_hip.so).

This is the ctypes counterpart of the reference's safe FFI crate
(crates/hyperion-ffi/src/lib.rs: raw externs :225-269, RAII handles :513-690,
status mapping :303): every call checks the HypStatus, raises HypError with the
thread-local message, and handles free themselves exactly once.

The native library is the product; this module only marshals pointers. It never
falls back to another implementation: if the library is missing or no GPU is
present, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhyperion_hip.so")
# The same library with a host-side fault hook (hyp_test_fault_after_first_replay), for tests.
FAULTS_LIB_PATH = os.path.join(_HERE, "libhyperion_hip_faults.so")

HYP_STATUS = {
    0: "OK",
    1: "INVALID_ARGUMENT",
    2: "NOT_FOUND",
    3: "IO",
    4: "OOM_GOVERNOR",
    5: "UNSUPPORTED",
    6: "INTERNAL",
    7: "CANCELLED",
}
PROJ = {"q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "up": 5, "down": 6}
EPILOGUE_NONE = 0
EPILOGUE_SOFTCAP = 1

# Every symbol declared in include/hyperion_hip.h.
EXPORTED = [
    "hyp_last_error", "hyp_runtime_info",
    "hyp_device_alloc", "hyp_device_free",
    "hyp_stream_create", "hyp_stream_destroy", "hyp_stream_synchronize",
    "hyp_memcpy_htod", "hyp_memcpy_dtoh", "hyp_memcpy_dtod", "hyp_memset_device",
    "hyp_event_create", "hyp_event_destroy", "hyp_event_record", "hyp_event_elapsed_ms",
    "hyp_graph_capture_begin", "hyp_graph_capture_end", "hyp_graph_launch", "hyp_graph_free",
    "hyp_qweight_create", "hyp_qweight_create_device", "hyp_qweight_free",
    "hyp_qweight_shape", "hyp_qweight_export",
    "hyp_qmatmul", "hyp_qmatmul_noalloc", "hyp_qmatmul_ex", "hyp_qmatmul_group", "hyp_qmatmul_group_rmsnorm",
    "hyp_qmlp_gate_up_gelu",
    "hyp_quantize_q4g64", "hyp_dequantize_q4g64", "hyp_embed", "hyp_rms_normalize",
    "hyp_rope", "hyp_sample_greedy", "hyp_sample_greedy_topk", "hyp_sample_stochastic",
    "hyp_kv_cache_create", "hyp_kv_cache_free", "hyp_kv_cache_buffers", "hyp_kv_cache_write", "hyp_attention",
    "hyp_attention_prepare", "hyp_residual_rms_norm",
    "hyp_model_create", "hyp_model_free", "hyp_model_load", "hyp_kvstate_create", "hyp_kvstate_free",
    "hyp_prefill_chunk", "hyp_decode_block", "hyp_prefill_chunk_sampled", "hyp_decode_block_sampled",
    "hyp_step_result_create", "hyp_step_result_free", "hyp_step_result_fields", "hyp_model_forward_hidden",
    "hyp_geometry_memory", "hyp_model_memory",
    "hyp_step_program_create", "hyp_step_program_run", "hyp_step_program_check", "hyp_step_program_free",
    "hyp_qmodel_load", "hyp_qmodel_free", "hyp_qmodel_num_layers",
    "hyp_qmodel_linear", "hyp_qmodel_embed",
]


class HypError(RuntimeError):
    def __init__(self, status: int, op: str, message: str):
        self.status = status
        self.status_name = HYP_STATUS.get(status, f"UNKNOWN({status})")
        super().__init__(f"{op}: {self.status_name}: {message}")


class RuntimeInfo(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("device_count", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("compute_units", ctypes.c_uint32),
        ("hbm_bytes", ctypes.c_uint64),
        ("clock_khz", ctypes.c_uint32),
        ("l2_bytes", ctypes.c_uint32),
        ("arch_name", ctypes.c_char * 64),
        ("device_name", ctypes.c_char * 128),
    ]


STEP_QMATMUL = 0
STEP_QMATMUL_RMSNORM = 1
STEP_GATE_UP_GELU = 2


class StepOp(ctypes.Structure):
    """HypStepOp: one op of a decode-step program."""
    _fields_ = [
        ("kind", ctypes.c_uint32),
        ("count", ctypes.c_uint32),
        ("weights", ctypes.c_void_p * 3),
        ("x", ctypes.c_void_p),
        ("y", ctypes.c_void_p * 3),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_uint32),
        ("norm_weight", ctypes.c_void_p),
    ]


TOP_K_LOGPROBS = 8   # HYP_TOP_K_LOGPROBS (hyperion_mlx.h:145)


class TopKSample(ctypes.Structure):
    """HypTopKSample: ForwardPass::StochasticSample (forward.h:125-131) as the greedy
    epilogue fills it (model.cc:272-288), plus GreedySample's near_tie."""
    _fields_ = [
        ("token_id", ctypes.c_uint32),
        ("logit", ctypes.c_float),
        ("near_tie", ctypes.c_uint32),
        ("top_k_count", ctypes.c_uint32),
        ("top_k_ids", ctypes.c_uint32 * TOP_K_LOGPROBS),
        ("top_k_logprobs", ctypes.c_float * TOP_K_LOGPROBS),
    ]


class GreedySample(ctypes.Structure):
    """HypGreedySample: ForwardPass::GreedySample (forward.h:104-108)."""
    _fields_ = [
        ("token_id", ctypes.c_uint32),
        ("logit", ctypes.c_float),
        ("near_tie", ctypes.c_uint32),
    ]


LAYER_SLIDING = 0   # HypLayerType (hyperion_mlx.h:63-66)
LAYER_FULL = 1
GEMMA4_TEXT = 0     # HypTextModelType
GEMMA4_UNIFIED_TEXT = 1


class RopeSpec(ctypes.Structure):
    """HypRopeSpec (hyperion_mlx.h:75-80)."""
    _fields_ = [
        ("theta", ctypes.c_double),
        ("has_partial_rotary_factor", ctypes.c_int),
        ("partial_rotary_factor", ctypes.c_float),
        ("proportional", ctypes.c_int),
    ]


class MoeConfig(ctypes.Structure):
    _fields_ = [("num_experts", ctypes.c_uint32), ("top_k", ctypes.c_uint32),
                ("moe_intermediate_size", ctypes.c_uint32)]


class GeometryParams(ctypes.Structure):
    """HypGeometryParams (hyperion_mlx.h:89-116)."""
    _fields_ = [
        ("model_type", ctypes.c_int),
        ("hidden_size", ctypes.c_uint32),
        ("intermediate_size", ctypes.c_uint32),
        ("num_hidden_layers", ctypes.c_uint32),
        ("layer_types", ctypes.POINTER(ctypes.c_int)),
        ("num_attention_heads", ctypes.c_uint32),
        ("head_dim_local", ctypes.c_uint32),
        ("head_dim_global", ctypes.c_uint32),
        ("num_kv_heads_local", ctypes.c_uint32),
        ("num_kv_heads_global", ctypes.c_uint32),
        ("attention_k_eq_v_global", ctypes.c_int),
        ("num_kv_shared_layers", ctypes.c_uint32),
        ("sliding_window", ctypes.c_uint32),
        ("rope_local", RopeSpec),
        ("rope_global", RopeSpec),
        ("final_logit_softcapping", ctypes.c_float),
        ("rms_norm_eps", ctypes.c_float),
        ("attention_bias", ctypes.c_int),
        ("vocab_size", ctypes.c_uint32),
        ("max_position_embeddings", ctypes.c_uint32),
        ("tie_word_embeddings", ctypes.c_int),
        ("ple_hidden_per_layer_input", ctypes.c_uint32),
        ("ple_vocab_per_layer_input", ctypes.c_uint32),
        ("use_double_wide_mlp", ctypes.c_int),
        ("has_moe", ctypes.c_int),
        ("moe", MoeConfig),
    ]


class TokenStream(ctypes.Structure):
    """HypTokenStream (hyperion_mlx.h:119-123)."""
    _fields_ = [("tokens", ctypes.POINTER(ctypes.c_uint32)), ("count", ctypes.c_uint32),
                ("is_prompt", ctypes.c_int)]


class SamplingConfig(ctypes.Structure):
    """HypSamplingConfig (hyperion_mlx.h:134-140)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("top_p", ctypes.c_float),
                ("min_p", ctypes.c_float), ("seed", ctypes.c_uint64)]


class StepResultFields(ctypes.Structure):
    """HypStepResultFields (hyperion_mlx.h:157-176)."""
    _fields_ = [
        ("token_id", ctypes.c_uint32),
        ("logit", ctypes.c_float),
        ("peak_mlx_bytes", ctypes.c_uint64),
        ("active_mlx_bytes", ctypes.c_uint64),
        ("phys_footprint_bytes", ctypes.c_uint64),
        ("local_kv_bytes", ctypes.c_uint64),
        ("global_kv_bytes", ctypes.c_uint64),
        ("local_kv_eval_ms", ctypes.c_float),
        ("global_kv_eval_ms", ctypes.c_float),
        ("governor_state", ctypes.c_int),
        ("near_tie_events", ctypes.c_uint32),
        ("top_k_logprob_count", ctypes.c_uint32),
        ("top_k_logprob_ids", ctypes.c_uint32 * TOP_K_LOGPROBS),
        ("top_k_logprob_values", ctypes.c_float * TOP_K_LOGPROBS),
    ]


class MemoryReport(ctypes.Structure):
    """HypMemoryReport: device bytes of a model and one KV state, quantization-aware."""
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "weight_bytes", "norm_bytes", "kv_local_bytes", "kv_global_bytes", "state_bytes", "scratch_bytes",
        "dense_bf16_weight_bytes")]


_lib = None
_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_U32 = ctypes.c_uint32
_SZ = ctypes.c_size_t


def lib() -> ctypes.CDLL:
    """Load libhyperion_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        _lib = load_library(LIB_PATH)
    return _lib


def load_library(path: str) -> ctypes.CDLL:
    """A ctypes handle of one build of the library (the product, or the test build
    FAULTS_LIB_PATH) with the signature of every ABI function set."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with __graft_entry__.build()")
    L = ctypes.CDLL(path)
    sig = {
        "hyp_last_error": [ctypes.c_char_p, _SZ],
        "hyp_runtime_info": [ctypes.POINTER(RuntimeInfo)],
        "hyp_device_alloc": [_SZ, _PP],
        "hyp_device_free": [_PP],
        "hyp_stream_create": [_PP],
        "hyp_stream_destroy": [_PP],
        "hyp_stream_synchronize": [_P],
        "hyp_memcpy_htod": [_P, _P, _SZ, _P],
        "hyp_memcpy_dtoh": [_P, _P, _SZ, _P],
        "hyp_memcpy_dtod": [_P, _P, _SZ, _P],
        "hyp_memset_device": [_P, ctypes.c_int, _SZ, _P],
        "hyp_event_create": [_PP],
        "hyp_event_destroy": [_PP],
        "hyp_event_record": [_P, _P],
        "hyp_event_elapsed_ms": [_P, _P, ctypes.POINTER(ctypes.c_float)],
        "hyp_graph_capture_begin": [_P],
        "hyp_graph_capture_end": [_P, _PP],
        "hyp_graph_launch": [_P, _P],
        "hyp_graph_free": [_PP],
        "hyp_qweight_create": [_P, _P, _P, _U32, _U32, _U32, _U32, _PP],
        "hyp_qweight_create_device": [_P, _P, _P, _U32, _U32, _U32, _U32, _P, _PP],
        "hyp_qweight_free": [_PP],
        "hyp_qweight_shape": [_P, ctypes.POINTER(_U32), ctypes.POINTER(_U32)],
        "hyp_qweight_export": [_P, _P, _P, _P],
        "hyp_qmatmul": [_P, _P, _U32, _P, _P],
        "hyp_qmatmul_noalloc": [_P, _P, _U32, _P, _P],
        "hyp_qmatmul_ex": [_P, _P, _U32, _P, ctypes.c_int, ctypes.c_float, _P],
        "hyp_qmatmul_group": [_P, _U32, _P, _U32, _P, _P],
        "hyp_qmatmul_group_rmsnorm": [_P, _U32, _P, _P, _U32, ctypes.c_float, _P, _P],
        "hyp_qmlp_gate_up_gelu": [_P, _P, _P, _U32, _P, _P],
        "hyp_quantize_q4g64": [_P, _U32, _U32, _P, _P, _P, _P],
        "hyp_dequantize_q4g64": [_P, _P, _P, _U32, _U32, _P, _U32, ctypes.c_float, _P, _P],
        "hyp_embed": [_P, _P, _U32, _P, _P],
        "hyp_rms_normalize": [_P, _P, _U32, _U32, ctypes.c_float, _P, _P],
        "hyp_rope": [_P, _U32, _U32, _U32, _U32, ctypes.c_float, _U32, _P, _P],
        "hyp_sample_greedy": [_P, _U32, _U32, _P, _P],
        "hyp_sample_greedy_topk": [_P, _U32, _U32, _P, _P],
        "hyp_sample_stochastic": [_P, _U32, ctypes.POINTER(SamplingConfig), ctypes.c_uint64, _P, _P],
        "hyp_kv_cache_create": [_U32, _U32, _U32, _PP],
        "hyp_kv_cache_free": [_PP],
        "hyp_kv_cache_buffers": [_P, _PP, _PP],
        "hyp_kv_cache_write": [_P, _P, _P, _U32, _U32, _P],
        "hyp_attention": [_P, _P, _P, _U32, _U32, _P, _U32, _U32, _U32, _P, _P],
        "hyp_attention_prepare": [_P, _P, _P, _U32, _U32, _P, _P, _P, ctypes.c_float, _U32, ctypes.c_float, _U32,
                                  _P],
        "hyp_residual_rms_norm": [_P, _P, _P, _P, _P, _P, _U32, _U32, ctypes.c_float, _P],
        "hyp_model_create": [_PP],
        "hyp_model_free": [_PP],
        "hyp_model_load": [_P, ctypes.POINTER(GeometryParams), ctypes.c_char_p],
        "hyp_kvstate_create": [_P, _PP],
        "hyp_kvstate_free": [_PP],
        "hyp_prefill_chunk": [_P, _P, ctypes.POINTER(TokenStream), _P],
        "hyp_decode_block": [_P, _P, _U32, _P],
        "hyp_prefill_chunk_sampled": [_P, _P, ctypes.POINTER(TokenStream), ctypes.POINTER(SamplingConfig), _P],
        "hyp_decode_block_sampled": [_P, _P, _U32, ctypes.POINTER(SamplingConfig), _P],
        "hyp_step_result_create": [_PP],
        "hyp_step_result_free": [_PP],
        "hyp_step_result_fields": [_P, ctypes.POINTER(StepResultFields)],
        "hyp_model_forward_hidden": [_P, _P, ctypes.POINTER(ctypes.c_uint32), _U32, _U32, _P],
        "hyp_geometry_memory": [ctypes.POINTER(GeometryParams), ctypes.POINTER(MemoryReport)],
        "hyp_model_memory": [_P, ctypes.POINTER(MemoryReport)],
        "hyp_step_program_create": [_P, _U32, _U32, _U32, _PP],
        "hyp_step_program_run": [_P, _P],
        "hyp_step_program_check": [_P],
        "hyp_step_program_free": [_PP],
        "hyp_qmodel_load": [ctypes.c_char_p, _U32, _PP],
        "hyp_qmodel_free": [_PP],
        "hyp_qmodel_num_layers": [_P, ctypes.POINTER(_U32)],
        "hyp_qmodel_linear": [_P, _U32, ctypes.c_int, _PP],
        "hyp_qmodel_embed": [_P, _PP],
    }
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    return L


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().hyp_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(status: int, op: str) -> None:
    if status != 0:
        raise HypError(status, op, last_error())


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def runtime_info() -> RuntimeInfo:
    info = RuntimeInfo()
    call("hyp_runtime_info", ctypes.byref(info))
    return info


class Stream:
    """An explicit HIP stream (the reference passes mx::Stream explicitly)."""

    def __init__(self):
        self._h = ctypes.c_void_p()
        call("hyp_stream_create", ctypes.byref(self._h))

    @property
    def handle(self):
        return self._h

    def synchronize(self) -> None:
        call("hyp_stream_synchronize", self._h)

    def close(self) -> None:
        if self._h:
            call("hyp_stream_destroy", ctypes.byref(self._h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        self._h = ctypes.c_void_p()
        call("hyp_event_create", ctypes.byref(self._h))

    def record(self, stream: Stream) -> None:
        call("hyp_event_record", self._h, stream.handle)

    def elapsed_ms(self, end: "Event") -> float:
        out = ctypes.c_float()
        call("hyp_event_elapsed_ms", self._h, end._h, ctypes.byref(out))
        return float(out.value)

    def close(self) -> None:
        if self._h:
            call("hyp_event_destroy", ctypes.byref(self._h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """A captured launch sequence: `with Graph.capture(stream) as g: ...`, then g.launch()."""

    def __init__(self):
        self._h = ctypes.c_void_p()

    @classmethod
    def capture(cls, stream: "Stream") -> "_Capture":
        return _Capture(cls(), stream)

    def launch(self, stream: "Stream") -> None:
        call("hyp_graph_launch", self._h, stream.handle)

    def close(self) -> None:
        if self._h:
            call("hyp_graph_free", ctypes.byref(self._h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _Capture:
    def __init__(self, graph: Graph, stream: "Stream"):
        self.graph = graph
        self.stream = stream

    def __enter__(self) -> Graph:
        call("hyp_graph_capture_begin", self.stream.handle)
        return self.graph

    def __exit__(self, exc_type, exc, tb):
        status = lib().hyp_graph_capture_end(self.stream.handle, ctypes.byref(self.graph._h))
        if exc_type is None:
            check(status, "hyp_graph_capture_end")
        return False


class DeviceArray:
    """A device allocation with a numpy dtype and shape (bf16 travels as uint16)."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self._p = ctypes.c_void_p()
        call("hyp_device_alloc", max(self.nbytes, 1), ctypes.byref(self._p))

    @property
    def ptr(self):
        return self._p

    @classmethod
    def from_host(cls, a: np.ndarray, stream: Stream) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            call("hyp_memcpy_htod", d.ptr, a.ctypes.data_as(_P), a.nbytes, stream.handle)
            stream.synchronize()
        return d

    def to_host(self, stream: Stream) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("hyp_memcpy_dtoh", out.ctypes.data_as(_P), self.ptr, self.nbytes, stream.handle)
            stream.synchronize()
        return out

    def upload(self, a: np.ndarray, stream: Stream) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        call("hyp_memcpy_htod", self.ptr, a.ctypes.data_as(_P), a.nbytes, stream.handle)
        stream.synchronize()

    def fill_zero(self, stream: Stream) -> None:
        call("hyp_memset_device", self.ptr, 0, self.nbytes, stream.handle)

    def close(self) -> None:
        if self._p:
            call("hyp_device_free", ctypes.byref(self._p))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QWeight:
    """A device-resident Q4/g64 projection (QuantizedLinear, weights.h:18-37)."""

    def __init__(self, handle: ctypes.c_void_p, owner=None):
        self._h = handle
        self._owner = owner   # a QModel for borrowed handles

    @classmethod
    def from_host(cls, w: np.ndarray, scales: np.ndarray, biases: np.ndarray,
                  group_size: int = 64, bits: int = 4) -> "QWeight":
        w = np.ascontiguousarray(w, np.uint32)
        s = np.ascontiguousarray(scales, np.uint16)
        b = np.ascontiguousarray(biases, np.uint16)
        n = w.shape[0]
        k = s.shape[1] * group_size
        h = ctypes.c_void_p()
        call("hyp_qweight_create", w.ctypes.data_as(_P), s.ctypes.data_as(_P), b.ctypes.data_as(_P),
             n, k, group_size, bits, ctypes.byref(h))
        return cls(h)

    @property
    def handle(self):
        return self._h

    @property
    def shape(self):
        n, k = _U32(), _U32()
        call("hyp_qweight_shape", self._h, ctypes.byref(n), ctypes.byref(k))
        return int(n.value), int(k.value)

    def export(self):
        n, k = self.shape
        w = np.empty((n, k // 8), np.uint32)
        s = np.empty((n, k // 64), np.uint16)
        b = np.empty((n, k // 64), np.uint16)
        call("hyp_qweight_export", self._h, w.ctypes.data_as(_P), s.ctypes.data_as(_P), b.ctypes.data_as(_P))
        return w, s, b

    def close(self) -> None:
        if self._h and self._owner is None:
            call("hyp_qweight_free", ctypes.byref(self._h))
        self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QModel:
    """All resident Q4 projections of an MLX artifact (load_model_weights)."""

    def __init__(self, path: str, num_layers: int = 0):
        self._h = ctypes.c_void_p()
        call("hyp_qmodel_load", path.encode(), num_layers, ctypes.byref(self._h))

    @property
    def num_layers(self) -> int:
        out = _U32()
        call("hyp_qmodel_num_layers", self._h, ctypes.byref(out))
        return int(out.value)

    def linear(self, layer: int, proj: str) -> QWeight:
        h = ctypes.c_void_p()
        call("hyp_qmodel_linear", self._h, layer, PROJ[proj], ctypes.byref(h))
        return QWeight(h, owner=self)

    def embed(self) -> QWeight:
        h = ctypes.c_void_p()
        call("hyp_qmodel_embed", self._h, ctypes.byref(h))
        return QWeight(h, owner=self)

    def close(self) -> None:
        if self._h:
            call("hyp_qmodel_free", ctypes.byref(self._h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class StepProgram:
    """A decode-step program (hyp_step_program_*): ops is a list of (kind, weights, x, ys,
    eps[, norm_weight]) with QWeight weights and DeviceArray buffers, all borrowed for the
    program's life."""

    def __init__(self, ops, m: int, spin_limit: int = 0):
        arr = (StepOp * len(ops))()
        self._keep = []
        for i, op in enumerate(ops):
            kind, ws, x, ys, eps = op[:5]
            norm_w = op[5] if len(op) > 5 else None
            o = arr[i]
            o.kind = kind
            o.count = len(ws)
            for q, w in enumerate(ws):
                o.weights[q] = w.handle.value
            o.x = x.ptr.value
            for q, y in enumerate(ys):
                o.y[q] = y.ptr.value
            o.eps = eps
            o.norm_weight = norm_w.ptr.value if norm_w is not None else None
            self._keep.append((ws, x, ys, norm_w))
        self._h = ctypes.c_void_p()
        call("hyp_step_program_create", ctypes.cast(arr, _P), len(ops), m, spin_limit, ctypes.byref(self._h))

    def run(self, stream: "Stream") -> None:
        call("hyp_step_program_run", self._h, stream.handle)

    def check(self) -> None:
        call("hyp_step_program_check", self._h)

    def close(self) -> None:
        if self._h:
            call("hyp_step_program_free", ctypes.byref(self._h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def qmatmul(w: QWeight, x: DeviceArray, m: int, y: DeviceArray, stream: Stream,
            softcap: Optional[float] = None) -> None:
    if softcap is None:
        call("hyp_qmatmul", w.handle, x.ptr, m, y.ptr, stream.handle)
    else:
        call("hyp_qmatmul_ex", w.handle, x.ptr, m, y.ptr, EPILOGUE_SOFTCAP, softcap, stream.handle)


def qmatmul_group(ws, x: DeviceArray, m: int, ys, stream: Stream, rms_eps: Optional[float] = None,
                  norm_weight: Optional[DeviceArray] = None) -> None:
    """ys[i] = x . dequant(ws[i])^T for up to three weights sharing k (one launch at m <= 4);
    with rms_eps, x is rms-normalised first, with norm_weight if given
    (hyp_qmatmul_group_rmsnorm)."""
    if len(ws) != len(ys):
        raise ValueError("qmatmul_group: one output per weight")
    handles = (ctypes.c_void_p * len(ws))(*[w.handle for w in ws])
    outs = (ctypes.c_void_p * len(ys))(*[y.ptr for y in ys])
    if rms_eps is None:
        call("hyp_qmatmul_group", handles, len(ws), x.ptr, m, outs, stream.handle)
    else:
        call("hyp_qmatmul_group_rmsnorm", handles, len(ws), x.ptr, norm_weight.ptr if norm_weight is not None else None,
             m, rms_eps, outs, stream.handle)


def qmlp_gate_up_gelu(gate: QWeight, up: QWeight, x: DeviceArray, m: int, h: DeviceArray,
                      stream: Stream) -> None:
    call("hyp_qmlp_gate_up_gelu", gate.handle, up.handle, x.ptr, m, h.ptr, stream.handle)


def quantize(w: DeviceArray, n: int, k: int, wq: DeviceArray, s: DeviceArray, b: DeviceArray,
             stream: Stream) -> None:
    call("hyp_quantize_q4g64", w.ptr, n, k, wq.ptr, s.ptr, b.ptr, stream.handle)


def dequantize(wq: DeviceArray, s: DeviceArray, b: DeviceArray, n_total: int, k: int,
               rows: Optional[DeviceArray], n_rows: int, out: DeviceArray, stream: Stream,
               out_scale: float = 0.0) -> None:
    call("hyp_dequantize_q4g64", wq.ptr, s.ptr, b.ptr, n_total, k,
         rows.ptr if rows is not None else None, n_rows, out_scale, out.ptr, stream.handle)


def embed(table: QWeight, ids: DeviceArray, n_ids: int, out: DeviceArray, stream: Stream) -> None:
    call("hyp_embed", table.handle, ids.ptr, n_ids, out.ptr, stream.handle)


def rms_normalize(x: DeviceArray, m: int, k: int, y: DeviceArray, stream: Stream, eps: float = 1e-6,
                  weight: Optional[DeviceArray] = None) -> None:
    """mx::fast::rms_norm over m rows of k (hyp_rms_normalize); weight None is the
    parameterless form."""
    call("hyp_rms_normalize", x.ptr, weight.ptr if weight is not None else None, m, k, eps, y.ptr, stream.handle)


def rope(x: DeviceArray, rows: int, heads: int, head_dim: int, rotated: int, base: float, offset: int,
         y: DeviceArray, stream: Stream) -> None:
    """mx::fast::rope (non-traditional) of x [rows, heads, head_dim] (hyp_rope)."""
    call("hyp_rope", x.ptr, rows, heads, head_dim, rotated, base, offset, y.ptr, stream.handle)


def sample_greedy(logits: DeviceArray, rows: int, vocab: int, out: DeviceArray, stream: Stream,
                  row_offset: int = 0) -> None:
    """out[r] = HypGreedySample of logits row row_offset + r, for r < rows (hyp_sample_greedy);
    out is a device array of at least rows * 12 bytes."""
    ptr = ctypes.c_void_p((logits.ptr.value or 0) + 2 * row_offset * vocab) if row_offset else logits.ptr
    call("hyp_sample_greedy", ptr, rows, vocab, out.ptr, stream.handle)


class KvCache:
    """HypKvCache: one layer's K/V cache [capacity, n_kv_heads, head_dim] bf16 on the device
    (slot = position % capacity)."""

    def __init__(self, capacity: int, n_kv_heads: int, head_dim: int):
        self.capacity, self.n_kv_heads, self.head_dim = capacity, n_kv_heads, head_dim
        self.handle = ctypes.c_void_p()
        call("hyp_kv_cache_create", capacity, n_kv_heads, head_dim, ctypes.byref(self.handle))

    def buffers(self):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        call("hyp_kv_cache_buffers", self.handle, ctypes.byref(k), ctypes.byref(v))
        return k, v

    def write(self, k: "DeviceArray", v: "DeviceArray", n: int, pos0: int, stream: "Stream") -> None:
        call("hyp_kv_cache_write", self.handle, k.ptr, v.ptr, n, pos0, stream.handle)

    def close(self) -> None:
        if self.handle:
            call("hyp_kv_cache_free", ctypes.byref(self.handle))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def attention(q: "DeviceArray", k: "DeviceArray", v: "DeviceArray", L: int, n_heads: int, cache: KvCache,
              offset: int, prefix_len: int, window: int, out: "DeviceArray", stream: "Stream") -> None:
    """hyp_attention: scale-1 SDPA of q [L, n_heads, d] over the cache's positions
    [offset - prefix_len, offset) and the chunk k/v [L, n_kv, d]; causal, sliding when
    window > 0."""
    call("hyp_attention", q.ptr, k.ptr, v.ptr, L, n_heads, cache.handle, offset, prefix_len, window, out.ptr,
         stream.handle)


def attention_prepare(q: "DeviceArray", k_raw: "DeviceArray", v_raw: Optional["DeviceArray"], L: int, n_heads: int,
                      cache: KvCache, q_norm: "DeviceArray", k_norm: "DeviceArray", eps: float, rotated: int,
                      base: float, offset: int, stream: "Stream") -> None:
    """hyp_attention_prepare: q <- rope(q_norm(q)) in place; the cache's slots of positions
    offset.. <- rope(k_norm(k_raw)) and v_norm(v_raw) (v_raw None: of k_raw)."""
    call("hyp_attention_prepare", q.ptr, k_raw.ptr, None if v_raw is None else v_raw.ptr, L, n_heads, cache.handle,
         q_norm.ptr, k_norm.ptr, eps, rotated, base, offset, stream.handle)


def residual_rms_norm(branch: "DeviceArray", residual: "DeviceArray", post_w: "DeviceArray",
                      scalar: Optional["DeviceArray"], next_w: Optional["DeviceArray"], nxt: Optional["DeviceArray"],
                      m: int, hidden: int, eps: float, stream: "Stream") -> None:
    """hyp_residual_rms_norm: residual <- bf16(residual + rms_norm(branch, post_w)), times the
    layer scalar when given, then nxt <- rms_norm(residual, next_w) when given."""
    opt = lambda a: None if a is None else a.ptr  # noqa: E731
    call("hyp_residual_rms_norm", branch.ptr, residual.ptr, post_w.ptr, opt(scalar), opt(next_w), opt(nxt), m, hidden,
         eps, stream.handle)


def geometry_from_config(cfg: dict):
    """HypGeometryParams from an mlx-lm config.json's text_config (the reference builds it
    from hyperion-model's Geometry, crates/hyperion-core/src/geometry_abi.rs). Returns the
    structure and the layer-type array it points into (keep both alive)."""
    t = cfg.get("text_config", cfg)
    kinds = [LAYER_SLIDING if k == "sliding_attention" else LAYER_FULL for k in t["layer_types"]]
    types = (ctypes.c_int * len(kinds))(*kinds)
    rp = t["rope_parameters"]
    sl, fu = rp["sliding_attention"], rp["full_attention"]
    g = GeometryParams()
    g.model_type = GEMMA4_UNIFIED_TEXT if t.get("model_type", "").startswith("gemma4_unified") else GEMMA4_TEXT
    g.hidden_size = t["hidden_size"]
    g.intermediate_size = t["intermediate_size"]
    g.num_hidden_layers = t["num_hidden_layers"]
    g.layer_types = ctypes.cast(types, ctypes.POINTER(ctypes.c_int))
    g.num_attention_heads = t["num_attention_heads"]
    g.head_dim_local = t["head_dim"]
    g.head_dim_global = t.get("global_head_dim", t["head_dim"])
    g.num_kv_heads_local = t["num_key_value_heads"]
    g.num_kv_heads_global = t.get("num_global_key_value_heads", t["num_key_value_heads"])
    g.attention_k_eq_v_global = int(bool(t.get("attention_k_eq_v", True)))
    g.num_kv_shared_layers = t.get("num_kv_shared_layers", 0) or 0
    g.sliding_window = t["sliding_window"]
    g.rope_local = RopeSpec(sl["rope_theta"], 0, 0.0, 0)
    g.rope_global = RopeSpec(fu["rope_theta"], 1, fu.get("partial_rotary_factor", 1.0),
                             int(fu.get("rope_type") == "proportional"))
    g.final_logit_softcapping = t["final_logit_softcapping"]
    g.rms_norm_eps = t["rms_norm_eps"]
    g.attention_bias = int(bool(t.get("attention_bias", False)))
    g.vocab_size = t["vocab_size"]
    g.max_position_embeddings = t["max_position_embeddings"]
    g.tie_word_embeddings = int(bool(t.get("tie_word_embeddings", cfg.get("tie_word_embeddings", True))))
    g.ple_hidden_per_layer_input = t.get("hidden_size_per_layer_input", 0) or 0
    g.ple_vocab_per_layer_input = t.get("vocab_size_per_layer_input", 0) or 0
    g.use_double_wide_mlp = int(bool(t.get("use_double_wide_mlp", False)))
    g.has_moe = int(bool(t.get("enable_moe_block", False)))
    return g, types


def geometry_memory(geometry) -> MemoryReport:
    """hyp_geometry_memory: what loading a model of this geometry and one state allocate."""
    g = geometry[0] if isinstance(geometry, tuple) else geometry
    r = MemoryReport()
    call("hyp_geometry_memory", ctypes.byref(g), ctypes.byref(r))
    return r


class StepResult:
    """HypStepResult: a reusable per-step result handle."""

    def __init__(self):
        self.handle = ctypes.c_void_p()
        call("hyp_step_result_create", ctypes.byref(self.handle))

    def fields(self) -> StepResultFields:
        f = StepResultFields()
        call("hyp_step_result_fields", self.handle, ctypes.byref(f))
        return f

    def close(self) -> None:
        if self.handle:
            call("hyp_step_result_free", ctypes.byref(self.handle))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """HypModel loaded from an artifact directory for a geometry (hyp_model_create + load)."""

    def __init__(self, geometry, weights_path: str):
        self.handle = ctypes.c_void_p()
        call("hyp_model_create", ctypes.byref(self.handle))
        self._geometry = geometry
        try:
            call("hyp_model_load", self.handle, ctypes.byref(geometry[0] if isinstance(geometry, tuple) else geometry),
                 weights_path.encode())
        except Exception:
            self.close()
            raise
        g = geometry[0] if isinstance(geometry, tuple) else geometry
        self.hidden, self.vocab = g.hidden_size, g.vocab_size

    def kvstate(self) -> "KvState":
        return KvState(self)

    def memory(self) -> MemoryReport:
        r = MemoryReport()
        call("hyp_model_memory", self.handle, ctypes.byref(r))
        return r

    def close(self) -> None:
        if self.handle:
            call("hyp_model_free", ctypes.byref(self.handle))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _sampling(cfg: Optional[SamplingConfig]):
    return None if cfg is None else ctypes.byref(cfg)


class KvState:
    """HypKvState of a Model: its KV caches and cursor."""

    def __init__(self, model: Model):
        self.model = model
        self.handle = ctypes.c_void_p()
        call("hyp_kvstate_create", model.handle, ctypes.byref(self.handle))

    def prefill(self, tokens, result: StepResult, sampling: Optional[SamplingConfig] = None,
                sampled: bool = False) -> StepResultFields:
        ids = np.ascontiguousarray(tokens, dtype=np.uint32)
        ts = TokenStream(ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), ids.size, 1)
        if sampled or sampling is not None:
            call("hyp_prefill_chunk_sampled", self.model.handle, self.handle, ctypes.byref(ts), _sampling(sampling),
                 result.handle)
        else:
            call("hyp_prefill_chunk", self.model.handle, self.handle, ctypes.byref(ts), result.handle)
        return result.fields()

    def decode(self, n_tokens: int, result: StepResult, sampling: Optional[SamplingConfig] = None,
               sampled: bool = False) -> StepResultFields:
        if sampled or sampling is not None:
            call("hyp_decode_block_sampled", self.model.handle, self.handle, n_tokens, _sampling(sampling),
                 result.handle)
        else:
            call("hyp_decode_block", self.model.handle, self.handle, n_tokens, result.handle)
        return result.fields()

    def forward_hidden(self, tokens, offset: int) -> np.ndarray:
        """hyp_model_forward_hidden: the final-normalised hidden rows (bf16 bits [n, hidden])."""
        ids = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros((ids.size, self.model.hidden), np.uint16)
        call("hyp_model_forward_hidden", self.model.handle, self.handle,
             ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), ids.size, offset, out.ctypes.data_as(_P))
        return out

    def close(self) -> None:
        if self.handle:
            call("hyp_kvstate_free", ctypes.byref(self.handle))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sample_greedy_topk(logits: DeviceArray, rows: int, vocab: int, out: DeviceArray, stream: Stream,
                       row_offset: int = 0) -> None:
    """out[r] = HypTopKSample of logits row row_offset + r, for r < rows
    (hyp_sample_greedy_topk); out is a device array of at least rows * 80 bytes."""
    ptr = ctypes.c_void_p((logits.ptr.value or 0) + 2 * row_offset * vocab) if row_offset else logits.ptr
    call("hyp_sample_greedy_topk", ptr, rows, vocab, out.ptr, stream.handle)


def sample_stochastic(logits: DeviceArray, vocab: int, sampling: Optional[SamplingConfig], rng_state: int,
                      out: DeviceArray, stream: Stream, row_offset: int = 0) -> None:
    """out[0] = the temperature draw of logits row row_offset with the top-k sidecar
    (hyp_sample_stochastic): ForwardPass::sample_stochastic (forward.cc:191-322) with the RNG
    state rng_state; sampling None or temperature 0 is the greedy result."""
    ptr = ctypes.c_void_p((logits.ptr.value or 0) + 2 * row_offset * vocab) if row_offset else logits.ptr
    call("hyp_sample_stochastic", ptr, vocab, _sampling(sampling), rng_state & 0xFFFFFFFFFFFFFFFF, out.ptr,
         stream.handle)


def topk_samples(out: DeviceArray, rows: int, stream: Stream):
    """The first `rows` HypTopKSample records of a device array as dicts (one
    synchronizing copy of rows * 80 bytes); ids/logprobs are numpy arrays of
    TOP_K_LOGPROBS entries, the values as bit-exact float32."""
    raw = out.to_host(stream).reshape(-1).view(np.uint8)[: rows * ctypes.sizeof(TopKSample)]
    recs = np.frombuffer(raw.tobytes(), np.uint32).reshape(rows, ctypes.sizeof(TopKSample) // 4)
    k = TOP_K_LOGPROBS
    return [{
        "token_id": int(r[0]), "logit": r[1:2].view(np.float32)[0], "near_tie": bool(r[2]),
        "count": int(r[3]), "ids": r[4:4 + k].copy(), "logprobs": r[4 + k:4 + 2 * k].view(np.float32).copy(),
    } for r in recs]


def greedy_samples(out: DeviceArray, rows: int, stream: Stream):
    """The first `rows` HypGreedySample records of a device array, as (token_id, logit,
    near_tie) tuples (one synchronizing copy of rows * 12 bytes)."""
    raw = out.to_host(stream).reshape(-1).view(np.uint8)[: rows * ctypes.sizeof(GreedySample)]
    recs = (GreedySample * rows).from_buffer_copy(raw.tobytes())
    return [(r.token_id, r.logit, bool(r.near_tie)) for r in recs]
