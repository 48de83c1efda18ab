"""Writes the committed fixtures of tests/golden from the CPU oracle (run from the repo root:
python tests/golden/make_golden.py).  The oracle itself is pinned by tests/test_oracle.py; these
fixtures freeze its outputs so later changes to either side show up as diffs.

  codebook_sha256.json   SHA-256 of the three 65536-entry fp16 codebook tables (cb 0, 1, 2)
  reconstruct_small.npz  trellis (seeded uniform words) and W_hat fp16 bits for 32x256 weights,
                         every bit width 1..8 x codebooks 0..2
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402

HERE = Path(__file__).resolve().parent


def main():
    sha = {str(cb): hashlib.sha256(O.codebook_table(cb).tobytes()).hexdigest() for cb in range(3)}
    (HERE / "codebook_sha256.json").write_text(json.dumps(sha, indent=1) + "\n")
    arrs = {}
    K, N = 32, 256
    for bits in range(1, 9):
        r = np.random.default_rng(1000 + bits)
        tr = r.integers(0, 65536, size=(K // 16, N // 16, 16 * bits), dtype=np.uint16)
        for cb in range(3):
            arrs[f"trellis_b{bits}_cb{cb}"] = tr
            arrs[f"w_b{bits}_cb{cb}"] = O.reconstruct(tr, K, N, bits, cb)
    np.savez_compressed(HERE / "reconstruct_small.npz", **arrs)


if __name__ == "__main__":
    main()
