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
