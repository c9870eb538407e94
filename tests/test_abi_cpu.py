"""C-ABI contract without a GPU: the library loads, exports exactly what the header
declares, and rejects bad arguments before touching a device. Mirrors the reference's
model-free ABI lifecycle tests (crates/hyperion-ffi/src/lib.rs:697-1000: null
out-pointers, double free, wrong-type handles, load on a missing directory -> NotFound
before any GPU call)."""
import ctypes
import json
import os
import re
import struct
import subprocess

import pytest

import hyperion_amd as hy

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hyperion_hip.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^HypStatus\s+(hyp_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_what_the_binding_lists():
    assert header_functions() == sorted(hy.EXPORTED)


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", hy.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\sT\s(hyp_\w+)$", out.stdout, flags=re.M))
    missing = [f for f in header_functions() if f not in exported]
    assert not missing, missing
    lib = hy.lib()
    for f in header_functions():
        assert getattr(lib, f) is not None


def test_header_compiles_as_c():
    src = '#include "hyperion_hip.h"\nint main(void){ HypStatus s = HYP_STATUS_OK; return (int)s; }\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-pedantic", "-I", os.path.dirname(HEADER),
                        "-x", "c", "-", "-fsyntax-only"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_status_values_match_reference_numbering():
    assert hy.HYP_STATUS == {0: "OK", 1: "INVALID_ARGUMENT", 2: "NOT_FOUND", 3: "IO", 4: "OOM_GOVERNOR",
                             5: "UNSUPPORTED", 6: "INTERNAL", 7: "CANCELLED"}
    text = open(HEADER).read()
    for code, name in hy.HYP_STATUS.items():
        assert re.search(rf"HYP_STATUS_{name}\s*=\s*{code}\b", text)


def _status(name, *args):
    return getattr(hy.lib(), name)(*args)


def test_unsupported_quantization_is_rejected_before_device():
    w = (ctypes.c_uint32 * 16)()
    s = (ctypes.c_uint16 * 2)()
    h = ctypes.c_void_p()
    assert _status("hyp_qweight_create", w, s, s, 1, 128, 32, 4, ctypes.byref(h)) == 5
    assert "group_size=32" in hy.last_error()
    assert _status("hyp_qweight_create", w, s, s, 1, 128, 64, 8, ctypes.byref(h)) == 5
    assert _status("hyp_qweight_create", w, s, s, 1, 100, 64, 4, ctypes.byref(h)) == 1
    assert "multiple of 64" in hy.last_error()
    assert _status("hyp_qweight_create", w, s, s, 0, 128, 64, 4, ctypes.byref(h)) == 1
    assert _status("hyp_qweight_create", w, s, s, 1, 128, 64, 4, None) == 1
    assert _status("hyp_qweight_create", None, s, s, 1, 128, 64, 4, ctypes.byref(h)) == 1
    assert not h.value


def test_free_is_idempotent_and_checks_magic():
    h = ctypes.c_void_p()
    assert _status("hyp_qweight_free", ctypes.byref(h)) == 0          # NULL handle: no-op
    assert hy.last_error() == ""                                        # OK clears the message
    assert _status("hyp_qweight_free", None) == 1
    fake = (ctypes.c_uint32 * 64)()                                     # magic 0: wrong type
    hf = ctypes.c_void_p(ctypes.addressof(fake))
    assert _status("hyp_qweight_free", ctypes.byref(hf)) == 1
    assert "magic" in hy.last_error()
    assert hf.value == ctypes.addressof(fake)                           # not nulled on failure
    for free_fn in ("hyp_qmodel_free", "hyp_stream_destroy", "hyp_event_destroy"):
        z = ctypes.c_void_p()
        assert _status(free_fn, ctypes.byref(z)) == 0
        assert _status(free_fn, ctypes.byref(hf)) == 1


def test_calls_reject_null_and_foreign_handles():
    fake = (ctypes.c_uint32 * 64)()
    hf = ctypes.c_void_p(ctypes.addressof(fake))
    assert _status("hyp_qmatmul", None, None, 1, None, None) == 1
    assert "null" in hy.last_error()
    assert _status("hyp_qmatmul", hf, None, 1, None, hf) == 1
    assert "magic" in hy.last_error()
    assert _status("hyp_qmlp_gate_up_gelu", hf, hf, None, 1, None, None) == 1
    n, k = ctypes.c_uint32(), ctypes.c_uint32()
    assert _status("hyp_qweight_shape", None, ctypes.byref(n), ctypes.byref(k)) == 1
    assert _status("hyp_stream_synchronize", None) == 1
    assert "explicit stream" in hy.last_error()
    assert _status("hyp_quantize_q4g64", None, 1, 64, None, None, None, hf) == 1
    assert _status("hyp_sample_greedy", None, 1, 262144, None, None) == 1   # explicit stream
    assert "explicit stream" in hy.last_error()
    assert _status("hyp_sample_greedy", None, 1, 262144, None, hf) == 1     # foreign stream handle
    assert "magic" in hy.last_error()


def test_last_error_buffer_contract():
    assert _status("hyp_qweight_create", None, None, None, 1, 64, 32, 4, None) == 1
    small = ctypes.create_string_buffer(8)
    assert _status("hyp_last_error", small, 8) == 0
    assert len(small.value) == 7                                        # truncated, NUL-terminated
    assert _status("hyp_last_error", None, 0) == 1


def test_load_missing_directory_is_not_found_without_gpu(tmp_path):
    h = ctypes.c_void_p()
    assert _status("hyp_qmodel_load", str(tmp_path / "nope").encode(), 0, ctypes.byref(h)) == 2
    assert "does not exist" in hy.last_error()
    assert _status("hyp_qmodel_load", str(tmp_path).encode(), 0, ctypes.byref(h)) == 2
    assert "no .safetensors" in hy.last_error()
    assert _status("hyp_qmodel_load", None, 0, ctypes.byref(h)) == 1


def _write_st(path, header: dict, data: bytes):
    hb = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + data)


def test_load_rejects_malformed_artifacts_on_host(tmp_path):
    h = ctypes.c_void_p()
    bad = tmp_path / "bad"
    bad.mkdir()
    (bad / "model.safetensors").write_bytes(struct.pack("<Q", 4) + b"{oops")
    assert _status("hyp_qmodel_load", str(bad).encode(), 0, ctypes.byref(h)) == 1
    assert "malformed" in hy.last_error()

    short = tmp_path / "short"
    short.mkdir()
    _write_st(short / "a.safetensors", {"t": {"dtype": "U32", "shape": [4, 4], "data_offsets": [0, 64]}}, b"\0" * 16)
    assert _status("hyp_qmodel_load", str(short).encode(), 0, ctypes.byref(h)) == 1
    assert "past the end" in hy.last_error()

    missing = tmp_path / "missing"
    missing.mkdir()
    base = "language_model.model.layers.0.self_attn.q_proj"
    hdr = {base + ".weight": {"dtype": "U32", "shape": [2, 8], "data_offsets": [0, 64]}}
    _write_st(missing / "a.safetensors", hdr, b"\0" * 64)
    assert _status("hyp_qmodel_load", str(missing).encode(), 0, ctypes.byref(h)) == 1
    assert "missing tensor" in hy.last_error()


def test_fixture_manifest_validates_on_host(fixture_dir):
    """The reference's tiny artifact passes every host-side check; without a GPU the
    load then stops at the device step (UNSUPPORTED), with a GPU it succeeds."""
    h = ctypes.c_void_p()
    st = _status("hyp_qmodel_load", fixture_dir.encode(), 0, ctypes.byref(h))
    if st == 0:
        assert _status("hyp_qmodel_free", ctypes.byref(h)) == 0
    else:
        assert st == 5 and "no HIP device" in hy.last_error()
    assert _status("hyp_qmodel_load", fixture_dir.encode(), 7, ctypes.byref(h)) == 1
    assert "shards hold 6" in hy.last_error()


def test_runtime_info_reports_abi_version():
    info = hy.RuntimeInfo()
    st = _status("hyp_runtime_info", ctypes.byref(info))
    assert info.abi_version == 1
    assert st in (0, 5)
    assert _status("hyp_runtime_info", None) == 1


def test_step_op_layout_matches_the_header():
    """HypStepOp: 4 + 4 + 3 pointers + x + 3 pointers + eps + reserved + norm_weight = 80
    bytes on LP64 (the Rust binding asserts the same size)."""
    assert ctypes.sizeof(hy.StepOp) == 80
    assert hy.StepOp.norm_weight.offset == 72
    src = ('#include <stddef.h>\n#include "hyperion_hip.h"\n'
           '_Static_assert(sizeof(HypStepOp) == 80, "size");\n'
           '_Static_assert(offsetof(HypStepOp, norm_weight) == 72, "offset");\nint main(void){return 0;}\n')
    r = subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), "-x", "c", "-", "-fsyntax-only"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_topk_sample_layout_matches_the_header():
    """HypTopKSample: token, logit, near_tie, count, 8 ids, 8 values = 80 bytes, and the
    sidecar size is the reference's HYP_TOP_K_LOGPROBS (8)."""
    assert ctypes.sizeof(hy.TopKSample) == 80
    assert hy.TopKSample.top_k_logprobs.offset == 48
    src = ('#include <stddef.h>\n#include "hyperion_hip.h"\n'
           '_Static_assert(HYP_TOP_K_LOGPROBS == 8, "k");\n'
           '_Static_assert(sizeof(HypTopKSample) == 80, "size");\n'
           '_Static_assert(offsetof(HypTopKSample, top_k_logprobs) == 48, "offset");\nint main(void){return 0;}\n')
    r = subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), "-x", "c", "-", "-fsyntax-only"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_step_program_create_rejects_bad_arguments_before_the_device():
    out = ctypes.c_void_p()
    assert _status("hyp_step_program_create", None, 0, 1, 0, ctypes.byref(out)) == 1
    ops = (hy.StepOp * 1)()
    assert _status("hyp_step_program_create", ctypes.cast(ops, ctypes.c_void_p), 1, 5, 0, ctypes.byref(out)) == 1
    ops[0].kind = 9
    ops[0].count = 1
    assert _status("hyp_step_program_create", ctypes.cast(ops, ctypes.c_void_p), 1, 1, 0, ctypes.byref(out)) == 1
    assert "unknown op kind" in hy.last_error()
    assert _status("hyp_step_program_free", None) == 1
    h = ctypes.c_void_p()
    assert _status("hyp_step_program_free", ctypes.byref(h)) == 0


# ---- the model-level ABI (hyperion_mlx.h:50-248) -------------------------------------------

REF_HEADER = "/root/reference/native/hyperion_mlx/include/hyperion_mlx.h"
MODEL_STRUCTS = {
    "HypRopeSpec": ["theta", "has_partial_rotary_factor", "partial_rotary_factor", "proportional"],
    "HypGeometryParams": ["model_type", "hidden_size", "intermediate_size", "num_hidden_layers", "layer_types",
                          "num_attention_heads", "head_dim_local", "head_dim_global", "num_kv_heads_local",
                          "num_kv_heads_global", "attention_k_eq_v_global", "num_kv_shared_layers", "sliding_window",
                          "rope_local", "rope_global", "final_logit_softcapping", "rms_norm_eps", "attention_bias",
                          "vocab_size", "max_position_embeddings", "tie_word_embeddings",
                          "ple_hidden_per_layer_input", "ple_vocab_per_layer_input", "use_double_wide_mlp", "has_moe",
                          "moe"],
    "HypTokenStream": ["tokens", "count", "is_prompt"],
    "HypSamplingConfig": ["temperature", "top_k", "top_p", "min_p", "seed"],
    "HypStepResultFields": ["token_id", "logit", "peak_mlx_bytes", "active_mlx_bytes", "phys_footprint_bytes",
                            "local_kv_bytes", "global_kv_bytes", "local_kv_eval_ms", "global_kv_eval_ms",
                            "governor_state", "near_tie_events", "top_k_logprob_count", "top_k_logprob_ids",
                            "top_k_logprob_values"],
}


def _layout(header_dir, include):
    """sizeof and every field offset of the model-level structs, compiled with gcc."""
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{include}"', 'int main(void) {']
    for s, fields in MODEL_STRUCTS.items():
        lines.append(f'printf("{s} %zu\\n", sizeof({s}));')
        for f in fields:
            lines.append(f'printf("{s}.{f} %zu\\n", offsetof({s}, {f}));')
    lines.append('return 0; }')
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "layout")
        r = subprocess.run(["gcc", "-std=c11", "-I", header_dir, "-x", "c", "-", "-o", exe], input="\n".join(lines),
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    return dict(line.rsplit(" ", 1) for line in out.split("\n") if line)


def test_model_structs_match_the_binding():
    got = _layout(os.path.dirname(HEADER), "hyperion_hip.h")
    py = {"HypRopeSpec": hy.RopeSpec, "HypGeometryParams": hy.GeometryParams, "HypTokenStream": hy.TokenStream,
          "HypSamplingConfig": hy.SamplingConfig, "HypStepResultFields": hy.StepResultFields}
    for s, cls in py.items():
        assert int(got[s]) == ctypes.sizeof(cls), s
        for f in MODEL_STRUCTS[s]:
            assert int(got[f"{s}.{f}"]) == getattr(cls, f).offset, f"{s}.{f}"


@pytest.mark.skipif(not os.path.exists(REF_HEADER), reason="the reference's header is not present")
def test_model_structs_match_the_reference_header():
    """The drop-in claim: the same sizes and field offsets as hyperion_mlx.h."""
    mine = _layout(os.path.dirname(HEADER), "hyperion_hip.h")
    ref = _layout(os.path.dirname(REF_HEADER), "hyperion_mlx.h")
    assert mine == ref


def _tiny_geometry(fixture_dir, **overrides):
    with open(os.path.join(fixture_dir, "config.json")) as f:
        cfg = json.load(f)
    g, types = hy.geometry_from_config(cfg)
    for k, v in overrides.items():
        setattr(g, k, v)
    return g, types


def test_model_lifecycle_and_validation_before_the_device(fixture_dir, tmp_path):
    m = ctypes.c_void_p()
    assert _status("hyp_model_create", None) == 1
    assert _status("hyp_model_create", ctypes.byref(m)) == 0
    g, types = _tiny_geometry(fixture_dir)
    assert _status("hyp_model_load", m, None, fixture_dir.encode()) == 1
    assert _status("hyp_model_load", m, ctypes.byref(g), None) == 1
    # Geometry::validate (geometry.cc:78-130) before any file or device access
    bad_types = (ctypes.c_int * 6)(*([hy.LAYER_SLIDING] * 6))
    g2, _ = _tiny_geometry(fixture_dir)
    g2.layer_types = ctypes.cast(bad_types, ctypes.POINTER(ctypes.c_int))
    assert _status("hyp_model_load", m, ctypes.byref(g2), fixture_dir.encode()) == 1
    assert "full_attention" in hy.last_error()
    for field, value, status in (("sliding_window", 0, 1), ("vocab_size", 0, 1), ("tie_word_embeddings", 0, 1),
                                 ("has_moe", 1, 1), ("use_double_wide_mlp", 1, 5), ("attention_bias", 1, 5),
                                 ("head_dim_local", 96, 5), ("num_kv_shared_layers", 2, 5)):
        gb, _ = _tiny_geometry(fixture_dir, **{field: value})
        assert _status("hyp_model_load", m, ctypes.byref(gb), fixture_dir.encode()) == status, field
    gm, _ = _tiny_geometry(fixture_dir, has_moe=1)
    gm.moe = hy.MoeConfig(4, 2, 64)
    assert _status("hyp_model_load", m, ctypes.byref(gm), fixture_dir.encode()) == 5
    # the artifact: missing directory, too few layers
    assert _status("hyp_model_load", m, ctypes.byref(g), str(tmp_path / "nope").encode()) == 2
    types7 = (ctypes.c_int * 7)(*([hy.LAYER_SLIDING] * 6 + [hy.LAYER_FULL]))
    g7, _ = _tiny_geometry(fixture_dir)
    g7.num_hidden_layers = 7
    g7.layer_types = ctypes.cast(types7, ctypes.POINTER(ctypes.c_int))
    assert _status("hyp_model_load", m, ctypes.byref(g7), fixture_dir.encode()) == 1
    # a valid load reaches the device check last
    st = _status("hyp_model_load", m, ctypes.byref(g), fixture_dir.encode())
    assert st in (0, 5)
    if st == 5:
        kv = ctypes.c_void_p()
        assert _status("hyp_kvstate_create", m, ctypes.byref(kv)) == 1
        assert "not loaded" in hy.last_error()
    assert _status("hyp_model_free", ctypes.byref(m)) == 0 and not m.value
    assert _status("hyp_model_free", ctypes.byref(m)) == 0


def test_step_result_lifecycle():
    r = ctypes.c_void_p()
    assert _status("hyp_step_result_create", ctypes.byref(r)) == 0
    f = hy.StepResultFields()
    f.token_id = 99
    assert _status("hyp_step_result_fields", r, ctypes.byref(f)) == 0
    assert f.token_id == 0 and f.top_k_logprob_count == 0
    assert _status("hyp_step_result_fields", r, None) == 1
    assert _status("hyp_step_result_fields", None, ctypes.byref(f)) == 1
    # a handle of another type is refused by magic
    m = ctypes.c_void_p()
    assert _status("hyp_model_create", ctypes.byref(m)) == 0
    assert _status("hyp_step_result_fields", m, ctypes.byref(f)) == 1
    assert _status("hyp_step_result_free", ctypes.byref(m)) == 1
    assert _status("hyp_model_free", ctypes.byref(m)) == 0
    assert _status("hyp_step_result_free", ctypes.byref(r)) == 0 and not r.value
    ts = hy.TokenStream(None, 0, 1)
    assert _status("hyp_prefill_chunk", None, None, ctypes.byref(ts), None) == 1
    assert _status("hyp_decode_block", None, None, 1, None) == 1


def test_geometry_memory_is_quantization_aware():
    """hyp_geometry_memory on the 12B geometry (geometry.rs:466-500): every projection shape is
    a multiple of 16 rows and 128 columns, so the tiled Q4/g64 layout holds exactly 0.5625 B
    per weight - 6.70 GB for 40 sliding and 8 global layers plus the tied 262144 x 3840 table,
    against the 24.7 GB of governor.cc:601-640's dense bf16 formula (4 h^2 + 3 h i per layer)."""
    from hyperion_amd import synthetic as syn
    cfg = syn.gemma4_text_config()
    g, types = hy.geometry_from_config(cfg)
    r = hy.geometry_memory((g, types))
    h, inter, H = 3840, 15360, 16
    sl = [(H * 256, h), (8 * 256, h), (8 * 256, h), (h, H * 256), (inter, h), (inter, h), (h, inter)]
    gl = [(H * 512, h), (1 * 512, h), (h, H * 512), (inter, h), (inter, h), (h, inter)]
    n_gl = cfg["layer_types"].count("full_attention")
    assert n_gl == 8
    weights = (262144 * h + 40 * sum(n * k for n, k in sl) + 8 * sum(n * k for n, k in gl))
    assert r.weight_bytes * 16 == weights * 9          # 0.5625 B per weight, exactly
    assert r.dense_bf16_weight_bytes == 2 * weights
    assert r.norm_bytes == 2 * (40 * (4 * h + 2 * 256 + 1) + 8 * (4 * h + 2 * 512 + 1) + h)
    assert r.kv_local_bytes == 40 * 2 * (1024 + 2048) * 8 * 256 * 2
    assert r.kv_global_bytes == 8 * 2 * 262144 * 1 * 512 * 2
    governor_dense = 2 * (262144 * h + 48 * (4 * h * h + 3 * h * inter))
    assert round(governor_dense / 1e9, 1) == 24.7 and round(r.weight_bytes / 1e9, 2) == 6.70
    g.layer_types = None
    assert _status("hyp_geometry_memory", ctypes.byref(g), ctypes.byref(r)) == 1
