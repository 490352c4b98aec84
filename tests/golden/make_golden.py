#!/usr/bin/env python3
"""Write the golden fixtures of the Q4_RDNA packers.

Runs the reference's own CPU tools (compiled from the reference sources into
oracle/_ref/ by oracle/Makefile) on seeded, bf16-representable inputs and
stores their outputs:

  q4rdna_golden.npz
    <case>_bf16          uint16 [rows, cols] input (bf16 bits)
    <case>_sidecar       uint8 tiles from q4rdna_sidecar_pack (scale search of
                         source/q4rdna_sidecar_pack.cpp:126-179)
    <case>_absmax|range|mse  uint8 raw tile stream from q4rdna_cpu_experiment
                         (source/q4rdna_cpu_experiment.cpp:136-273)
    sidecar_image        a complete 3-tensor sidecar file from the native packer
    large_sha256         sha256 of the tiles of a larger seeded case, per algorithm

Cases: "edge" (engineered groups: zeros, single values, ties, subnormal and
overflowing scales, outliers, sign-skewed groups), "small" (N(0, 0.02), 64 x 512),
"outlier" (N(0, 0.02) with 1% of groups scaled x20, 96 x 1024).

Run from the repository root, in a container where the reference tree is
mounted and `make -C oracle` has built oracle/_ref/:

    python3 tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4rdna_golden.npz")
LARGE = dict(rows=256, cols=4096, seed=0x51EE0101)


def bf16_bits(values: np.ndarray) -> np.ndarray:
    bits, _ = O.bf16_round(values.astype(np.float32))
    return bits


def edge_groups() -> np.ndarray:
    """32 rows x 64*8 columns of engineered groups (one group per (row, g))."""
    rng = np.random.default_rng(0xED6E)
    groups = []
    base = rng.standard_normal(64).astype(np.float32) * 0.02
    groups.append(np.zeros(64, np.float32))                                   # all zero
    g = np.zeros(64, np.float32); g[5] = 0.03125; groups.append(g)           # one positive
    g = np.zeros(64, np.float32); g[63] = -0.5; groups.append(g)             # one negative
    groups.append(np.full(64, 0.0078125, np.float32))                        # constant
    groups.append(np.full(64, -3.0, np.float32))                             # constant negative
    groups.append((np.arange(64, dtype=np.float32) - 32) * 0.0625)           # ramp, ties at .5 steps
    groups.append(((np.arange(64) % 16) - 8).astype(np.float32) * 0.25)      # exact codes -8..7
    groups.append(((np.arange(64) % 16) - 7.5).astype(np.float32) * 0.5)     # exact half ties
    groups.append(base * np.float32(1e-4))                                   # subnormal fp16 scales
    groups.append(base * np.float32(1e-6))                                   # deeper subnormal
    groups.append(base * np.float32(1e-9))                                   # below fp16 range
    groups.append(base * np.float32(5e4))                                    # large scales
    groups.append(base * np.float32(2e7))                                    # fp16 scale overflow
    g = base.copy(); g[17] *= 20; groups.append(g)                           # single outlier
    g = np.abs(base); groups.append(g)                                       # all positive
    g = -np.abs(base); groups.append(g)                                      # all negative
    g = base.copy(); g[::2] = 0; groups.append(g)                            # half zeros
    g = np.where(np.arange(64) % 2 == 0, 1.0, -1.0).astype(np.float32); groups.append(g)  # alternating
    g = base.copy(); g[0] = 7 * 0.015625; g[1] = -8 * 0.015625; groups.append(g)  # range corners
    g = base.copy(); g[3] = -0.25; groups.append(g)                          # negative-dominant
    g = base.copy(); g[3] = 0.25; groups.append(g)                           # positive-dominant
    g = np.zeros(64, np.float32); g[0] = 1e-30; groups.append(g)             # tiny single
    while len(groups) < 32 * 8:
        scale = np.float32(10.0 ** rng.uniform(-6, 3))
        g = rng.standard_normal(64).astype(np.float32) * scale
        if rng.random() < 0.3:
            g[rng.integers(0, 64)] *= np.float32(rng.uniform(5, 50))
        if rng.random() < 0.2:
            g[rng.random(64) < 0.5] = 0
        groups.append(g)
    arr = np.stack(groups[:256]).reshape(32, 8, 64).reshape(32, 512)
    return arr


def outlier_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    w = O.gaussian_weights(rows, cols, seed)
    g = w.reshape(rows, cols // 64, 64)
    n = g.shape[0] * g.shape[1]
    pick = np.random.default_rng(seed + 1).permutation(n)[: max(1, n // 100)]
    g.reshape(n, 64)[pick] *= np.float32(20.0)
    return w


def run_case(bits: np.ndarray) -> dict:
    out = {}
    img = O.ref_sidecar_pack([("blk.0.ffn_up.weight", bits)])
    off = O.ENTRY.unpack(img[48:144])[3]
    rows, cols = bits.shape
    out["sidecar"] = np.frombuffer(img[off:off + O.packed_size(rows, cols)], np.uint8).copy()
    for algo in ("absmax", "range", "mse"):
        out[algo] = np.frombuffer(O.ref_cpu_experiment(bits, algo), np.uint8).copy()
    return out


def main() -> None:
    if not O.ref_available():
        raise SystemExit("oracle/_ref tools missing: run `make -C oracle` with the reference mounted")
    cases = {
        "edge": bf16_bits(edge_groups()),
        "small": bf16_bits(O.gaussian_weights(64, 512, 0x51EE0001)),
        "outlier": bf16_bits(outlier_matrix(96, 1024, 0x51EE0002)),
    }
    data = {}
    for name, bits in cases.items():
        data[f"{name}_bf16"] = bits
        for algo, tiles in run_case(bits).items():
            data[f"{name}_{algo}"] = tiles
    # A multi-tensor sidecar image from the native packer.
    three = [("blk.0.attn_q.weight", cases["small"]), ("blk.0.attn_k.weight", cases["edge"]),
             ("blk.0.ffn_down.weight", cases["outlier"])]
    data["sidecar_image"] = np.frombuffer(O.ref_sidecar_pack(three), np.uint8).copy()
    # Larger seeded case: inputs regenerate from the seed, outputs as sha256.
    big = bf16_bits(O.gaussian_weights(LARGE["rows"], LARGE["cols"], LARGE["seed"]))
    hashes = []
    for algo, tiles in run_case(big).items():
        hashes.append(f"{algo}:{hashlib.sha256(tiles.tobytes()).hexdigest()}")
    data["large_sha256"] = np.array(hashes)
    data["large_shape_seed"] = np.array([LARGE["rows"], LARGE["cols"], LARGE["seed"]], dtype=np.int64)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
