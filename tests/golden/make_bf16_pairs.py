"""Extract the reference's bf16 conversion vectors as a data fixture.

Reads the (f32 bits, bf16 bits) pairs that packages/bf16/vectors.zig of the
reference holds (generated there by PyTorch 2.13.0, tools/gen_bf16_vectors.py)
and writes them as a uint32 array [n, 2] to bf16_pairs.npy. Only the numbers
are kept. Run in a container where the reference is mounted:

    python tests/golden/make_bf16_pairs.py /root/reference
"""
import os
import re
import sys

import numpy as np


def main(ref_root: str) -> None:
    path = os.path.join(ref_root, "packages", "bf16", "vectors.zig")
    text = open(path, encoding="utf-8").read()
    pairs = re.findall(r"\.\{\s*0x([0-9A-Fa-f]{8}),\s*0x([0-9A-Fa-f]{4})\s*\}", text)
    arr = np.array([[int(a, 16), int(b, 16)] for a, b in pairs], dtype=np.uint32)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bf16_pairs.npy")
    np.save(out, arr)
    print(f"{arr.shape[0]} pairs -> {out}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
