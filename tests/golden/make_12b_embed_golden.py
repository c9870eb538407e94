"""Extract the embed golden from the reference's 12B hidden-state fixture.

Reads `native/hyperion_mlx/tests/fixtures/12b_hidden_golden.safetensors` under the reference
checkout (default /root/reference) and writes `gemma4-12b-embed/embed.safetensors` beside
this script with two of its tensors, byte for byte:

- `ids`   I32 [10]          the prompt token ids the golden was taken on;
- `embed` BF16 [1,10,3840]  MLX's `ForwardPass::embed` of those ids on the real 12B:
  `mx::dequantize(..., dtype=bfloat16)` of the gathered Q4/g64 rows times bf16(sqrt(3840))
  (native/hyperion_mlx/src/forward.cc:126-131, weights_loader.cc:52-69), which
  native/hyperion_mlx/tests/forward_12b_test.cc:218 holds the reference to.

Run it where the reference is present: `python tests/golden/make_12b_embed_golden.py [ROOT]`.
"""
import json
import os
import struct
import sys

KEYS = ("ids", "embed")
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
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemma4-12b-embed", "embed.safetensors")
    with open(dst, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + b"".join(blobs))
    print(f"wrote {dst} ({8 + len(hb) + off} bytes)")


if __name__ == "__main__":
    main()
