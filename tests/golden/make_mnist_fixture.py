"""Writes tests/golden/mnist_hw.safetensors: the tensors of the reference's MNIST answer key.

The reference's test (furiosa-opt-examples/tests/mnist_tests.rs:7-53) runs its MLP forward on the ten
images of furiosa-opt-examples/data/mnist/mnist.safetensors (Apache-2.0 data) and checks the argmax
of the first ten logits against the stored labels. This script copies the tensors that test reads
-- hw.fc1.weight [256, 800], fc1.bias [256], hw.fc2.weight [16, 256], hw.fc2.bias [16],
hw.image_0..9 [800] (bf16) and label_0..9 [1] (i32) -- byte for byte into a smaller safetensors
file. The source is parsed as data (its JSON header and raw little-endian bytes); nothing in it is
executed. Run once, in a container that has the reference checkout:

    python tests/golden/make_mnist_fixture.py /root/reference/furiosa-opt-examples/data/mnist/mnist.safetensors
"""
import json
import struct
import sys
from pathlib import Path

NAMES = (["hw.fc1.weight", "fc1.bias", "hw.fc2.weight", "hw.fc2.bias"] + [f"hw.image_{i}" for i in range(10)]
         + [f"label_{i}" for i in range(10)])


def main(src: str) -> None:
    raw = Path(src).read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    base = 8 + n
    out_header, blobs, off = {}, [], 0
    for name in NAMES:
        ent = header[name]
        b, e = ent["data_offsets"]
        data = raw[base + b:base + e]
        out_header[name] = {"dtype": ent["dtype"], "shape": ent["shape"], "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    out_header["__metadata__"] = {"source": "furiosa-opt-examples/data/mnist/mnist.safetensors (Apache-2.0)"}
    h = json.dumps(out_header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    dst = Path(__file__).resolve().parent / "mnist_hw.safetensors"
    dst.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))
    print(dst, dst.stat().st_size)


if __name__ == "__main__":
    main(sys.argv[1])
