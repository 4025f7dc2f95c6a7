"""Write the golden fixture of the small RVQ configuration with the oracle.

Configuration: one sequence, t=128, d=256, 4 levels at full resolution
(strides 1,1,1,1), 512 codes per level; x ~N(0,1) (seed 0), codebooks
~N(0, 1/d) in bf16. Stored: the int32 codes [4, 128], the gaps, the
reconstruction's SHA-256 and a slice of it. No reference code is involved
(the reference has no RVQ implementation); this pins the oracle against
regressions and the GPU path against the same numbers.

    python tests/golden/make_rvq_golden.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from ncmorph_amd import synth  # noqa: E402
from oracle import pyoracle  # noqa: E402


def main():
    c = synth.RVQ_SMALL
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    r = pyoracle.rvq_encode(x, cb, c["strides"])
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rvq_small.npz")
    np.savez(out, codes=r["codes"].reshape(c["levels"], c["t"]), gap=r["gap"],
             recon_sha256=np.frombuffer(hashlib.sha256(r["recon"].tobytes()).digest(), np.uint8),
             recon_row0=r["recon"][0, 0], x_sha256=np.frombuffer(
                 hashlib.sha256(x.tobytes()).digest(), np.uint8),
             cb_sha256=np.frombuffer(hashlib.sha256(cb.tobytes()).digest(), np.uint8))
    print("wrote", out)


if __name__ == "__main__":
    main()
