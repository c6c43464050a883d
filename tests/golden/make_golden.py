"""Writes the small golden fixtures under tests/golden/ from data files the reference holds.

    python tests/golden/make_golden.py [--reference /root/reference]

dit_rope_subset.npz
    A token subset of the reference's recorded DiT 3-D RoPE table
    ``scripts/oracle_out/dit_rope_oracle.npz`` (32x32 grid, 1024 tokens x 64 slots x 2x2,
    fp32, produced by scripts/dit_rope_oracle.py from the pinned ComfyUI
    VideoRopePosition3DEmb).  Only data is copied: the rows listed in ``TOKENS`` plus the
    recorded h_theta / dim split / pinned commit.  Loaded with ``allow_pickle=False``.

The fixtures are committed; this script only documents how they were made and is not run
by the tests.
"""

from __future__ import annotations

import argparse
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# Anchor tokens of AnimaXSTests/DitRoPETests.swift:43-88 (0, 1, 17, 31, 32, 37), grid
# corners and rows, plus every 29th token for broad coverage.
TOKENS = sorted(set([0, 1, 17, 31, 32, 37, 63, 64, 511, 512, 992, 1023] + list(range(0, 1024, 29))))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    src = os.path.join(args.reference, "scripts", "oracle_out", "dit_rope_oracle.npz")
    z = np.load(src, allow_pickle=False)
    rope = z["rope"]
    assert rope.shape == (1024, 64, 2, 2) and rope.dtype == np.float32
    tokens = np.asarray(TOKENS, dtype=np.int32)
    np.savez_compressed(
        os.path.join(HERE, "dit_rope_subset.npz"),
        tokens=tokens,
        rope=rope[tokens],
        grid=np.asarray([1, 32, 32], dtype=np.int32),
        h_theta=np.asarray(z["h_theta"], dtype=np.float32),
        dims=np.asarray([int(z["dim_t"]), int(z["dim_h"]), int(z["dim_w"])], dtype=np.int32),
        commit=np.asarray(str(z["commit"])),
    )
    print(f"wrote dit_rope_subset.npz: {len(tokens)} tokens")


if __name__ == "__main__":
    main()
