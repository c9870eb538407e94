"""Extract a subset of the reference's 12B hidden-state fixture.

Reads `native/hyperion_mlx/tests/fixtures/12b_hidden_golden.safetensors` under the reference
checkout (default /root/reference; written by the reference's
native/hyperion_mlx/tests/gen_12b_hidden_golden.py with mlx-lm on the real 12B) and writes
`gemma4-12b-hidden/golden.safetensors` beside this script with seven of its tensors, byte for
byte:

- `ids`            I32 [10]            the prompt token ids the golden was taken on;
- `embed`          BF16 [1,10,3840]    MLX's embedding of those ids: `mx::dequantize(...,
  dtype=bfloat16)` of the gathered Q4/g64 rows times bf16(sqrt(3840)) (forward.cc:126-131,
  weights_loader.cc:52-69; forward_12b_test.cc:218);
- `layer_00_kproj` BF16 [1,10,2048]    the first (sliding) layer's k_proj output;
- `layer_00_k`     BF16 [1,8,10,256]   its keys: k_norm (weighted RMSNorm) then RoPE, theta
  10000 over all 256 dims (forward.cc:395-418; forward_12b_test.cc:199);
- `layer_05_kproj` BF16 [1,10,512]     the first global layer's k_proj output;
- `layer_05_k`     BF16 [1,1,10,512]   its keys: k_norm then the proportional RoPE (25% of
  512 dims rotated, theta 1e6, rope.cc:16-75);
- `layer_05_v`     BF16 [1,1,10,512]   its values: v_norm (weightless RMSNorm) of k_proj (the
  K = V global layer, forward.cc:403-412).

Run it where the reference is present: `python tests/golden/make_12b_hidden_golden.py [ROOT]`.
"""
import json
import os
import struct
import sys

KEYS = ("ids", "embed", "layer_00_kproj", "layer_00_k", "layer_05_kproj", "layer_05_k", "layer_05_v")
SRC = "native/hyperion_mlx/tests/fixtures/12b_hidden_golden.safetensors"


def main() -> None:
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    with open(os.path.join(root, SRC), "rb") as f:
        raw = f.read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    base = 8 + n
    out_header, blobs, off = {}, [], 0
    for key in KEYS:
        v = header[key]
        s, e = v["data_offsets"]
        blobs.append(raw[base + s:base + e])
        out_header[key] = {"dtype": v["dtype"], "shape": v["shape"], "data_offsets": [off, off + (e - s)]}
        off += e - s
    hb = json.dumps(out_header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemma4-12b-hidden", "golden.safetensors")
    with open(dst, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + b"".join(blobs))
    print(f"wrote {dst} ({8 + len(hb) + off} bytes)")


if __name__ == "__main__":
    main()
