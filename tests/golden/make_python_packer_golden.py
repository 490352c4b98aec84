#!/usr/bin/env python3
"""Write the fixtures of the reference's canonical Python packer.

The published sidecar was made by source/pack_q4rdna_sidecar.py, whose
`quantize` (:44-73) is a vectorised torch restatement of the native packer's
scale search, and whose `pack_tensor` (:77-98) lays the result out as tiles.
Nothing else pins it: its float32 sums run in torch's reduction order and
its candidate scales are decoded as IEEE fp16 (subnormals exact), where the
native packer sums sequentially and halves subnormal scales.  This script
imports that module from the reference tree (in a container where it is
mounted; torch and safetensors are installed), runs `pack_tensor` on bf16
inputs exactly as the packer's `main` feeds it (bf16 weights, tile chunks of
4 row tiles), and stores what it produced next to the native packer's
output for the same inputs:

  q4rdna_python_packer.npz
    <case>_tiles        uint8 tiles of the Python packer for the golden cases
                        edge / small / outlier of q4rdna_golden.npz (whose
                        <case>_sidecar arrays are the native packer's tiles)
    large_shape_seed    rows, cols, seed of a bf16 N(0, 0.02) sample
                        (oracle.gaussian_weights rounded to bf16)
    large_sha256        sha256 of the Python packer's tiles for that sample
    large_groups        int32 (row, group) indices of the groups where the
                        Python and native packers' tiles differ
    large_scales        uint16 fp16 bits of the Python packer's scale there
    large_codes         uint8 [n, 32]: the group's 32 code bytes (k-pairs
                        0..31), Python packer
    disagree_counts     int64 [4]: groups that differ in edge, small,
                        outlier, large

Run from the repository root in a container with the reference mounted:

    python3 tests/golden/make_python_packer_golden.py
"""
from __future__ import annotations

import hashlib
import io
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402

REFERENCE_SOURCE = "/root/reference/source"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4rdna_python_packer.npz")
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4rdna_golden.npz")
LARGE = (4096, 4096, 0x51EE0202)
TILE_CHUNK = 4  # the packer's --tile-chunk default (pack_q4rdna_sidecar.py:105)


def python_tiles(pack_tensor, bf16_bits: np.ndarray) -> np.ndarray:
    import torch
    w = torch.from_numpy(bf16_bits.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    buf = io.BytesIO()
    pack_tensor(buf, w, TILE_CHUNK)
    return np.frombuffer(buf.getvalue(), dtype=np.uint8).copy()


def group_bytes(tiles: np.ndarray, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """Per (row, group): the fp16 scale bits and the 32 code bytes."""
    g = cols // 64
    t = tiles.reshape(rows // 32, g, 1088)
    scales = t[:, :, :64].copy().view(np.uint16).reshape(rows // 32, g, 32).transpose(0, 2, 1).reshape(rows, g)
    codes = t[:, :, 64:].reshape(rows // 32, g, 32, 32).transpose(0, 3, 1, 2).reshape(rows, g, 32)
    return scales, codes


def differing_groups(a: np.ndarray, b: np.ndarray, rows: int, cols: int) -> np.ndarray:
    sa, ca = group_bytes(a, rows, cols)
    sb, cb = group_bytes(b, rows, cols)
    diff = (sa != sb) | (ca != cb).any(axis=2)
    return np.argwhere(diff).astype(np.int32)


def main() -> int:
    # The reference tree is read-only to this script: no bytecode cache is
    # written next to the module it imports.
    sys.dont_write_bytecode = True
    sys.path.insert(0, REFERENCE_SOURCE)
    from pack_q4rdna_sidecar import pack_tensor  # the reference's canonical packer

    golden = np.load(GOLDEN)
    out = {}
    counts = []
    for case in ("edge", "small", "outlier"):
        bits = golden[f"{case}_bf16"]
        rows, cols = bits.shape
        tiles = python_tiles(pack_tensor, bits)
        out[f"{case}_tiles"] = tiles
        n = len(differing_groups(tiles, golden[f"{case}_sidecar"], rows, cols))
        counts.append(n)
        print(f"{case}: {rows}x{cols}, {n} of {rows * cols // 64} groups differ from the native packer")
    rows, cols, seed = LARGE
    bits, values = O.bf16_round(O.gaussian_weights(rows, cols, seed))
    tiles = python_tiles(pack_tensor, bits.reshape(rows, cols))
    native, _ = O.pack_mt(values.reshape(rows, cols), O.ALGO_SIDECAR)
    idx = differing_groups(tiles, native, rows, cols)
    scales, codes = group_bytes(tiles, rows, cols)
    out["large_shape_seed"] = np.array(LARGE, dtype=np.int64)
    out["large_sha256"] = np.array(hashlib.sha256(tiles.tobytes()).hexdigest())
    out["large_groups"] = idx
    out["large_scales"] = scales[idx[:, 0], idx[:, 1]].astype(np.uint16)
    out["large_codes"] = codes[idx[:, 0], idx[:, 1]].astype(np.uint8)
    counts.append(len(idx))
    out["disagree_counts"] = np.array(counts, dtype=np.int64)
    print(f"large: {rows}x{cols} bf16 N(0, 0.02), {len(idx)} of {rows * cols // 64} groups differ")
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
