"""Read-only safetensors reader for the committed fixtures (numpy; bf16 as uint16)."""
import glob
import json
import os
import struct

import numpy as np

_DT = {"U32": np.uint32, "BF16": np.uint16, "F32": np.float32, "F16": np.float16, "I32": np.int32}


def read(path):
    with open(path, "rb") as f:
        raw = f.read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    base = 8 + n
    out = {}
    for name, v in header.items():
        if name == "__metadata__":
            continue
        s, e = v["data_offsets"]
        out[name] = (v["dtype"], np.frombuffer(raw[base + s:base + e], dtype=_DT[v["dtype"]]).reshape(v["shape"]))
    return out


def read_dir(d):
    out = {}
    for p in sorted(glob.glob(os.path.join(d, "*.safetensors"))):
        out.update(read(p))
    return out


def q4_tensors(d):
    """{base name: (w uint32, scales bf16, biases bf16)} for every Q4 projection."""
    t = read_dir(d)
    out = {}
    for name, (dt, v) in t.items():
        if dt == "U32" and name.endswith(".weight"):
            base = name[: -len(".weight")]
            out[base] = (v, t[base + ".scales"][1], t[base + ".biases"][1])
    return dict(sorted(out.items()))
