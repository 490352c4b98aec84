#!/usr/bin/env python3
"""Write the fixture of the reference bench's own correctness case.

source/q4rdna_gemv_bench.hip checks its GPU kernel once (:215-262): a
12288 x 4096 tile stream written by the CPU experiment with its default
absmax scale search (source/q4rdna_cpu_experiment.cpp:348), the
deterministic activation x_i = sin(0.013 i) * 0.25 + cos(0.007 i) * 0.125
(:224-227), and the gate relative L2 <= 1e-5 against its sequential fp32 loop
(:189-211, 259-261).  The reference ran it on real Qwen3-8B weights, which
are not available; this case feeds the CPU experiment bf16-rounded N(0, 0.02)
weights of a gate projection's shape instead (oracle.gaussian_weights, seed
SEED, rounded to bf16 as the experiment reads bf16).

The script runs the reference's own CPU experiment (compiled from its
sources into oracle/_ref by oracle/Makefile) on those weights, checks that
the oracle's absmax packer writes the same bytes, and stores

  q4rdna_bench_case.json
    rows, cols, seed    the weights: oracle.gaussian_weights(rows, cols, seed)
                        rounded to bf16
    algorithm           "absmax"
    tiles_sha256        sha256 of the experiment's raw tile stream
    x_sha256            sha256 of oracle.bench_activation(cols) (fp32 bytes)
    scales_normal       true when no fp16 scale of the tiles is subnormal, so
                        the bench's own fp16 decode (:163-187) equals IEEE

Run from the repository root in a container where the reference tree is
mounted and `make -C oracle` has built oracle/_ref:

    python3 tests/golden/make_bench_case_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4rdna_bench_case.json")
ROWS, COLS = 12288, 4096          # source/q4rdna_gemv_bench.hip:17-18
SEED = 0x51EE0004                 # layer 0's gate projection in the stack's seed scheme


def main() -> int:
    if not O.ref_available():
        print("oracle/_ref is not built: run `make -C oracle` with the reference mounted", file=sys.stderr)
        return 1
    bits, w = O.bf16_round(O.gaussian_weights(ROWS, COLS, SEED))
    ref = np.frombuffer(O.ref_cpu_experiment(bits, "absmax"), np.uint8)
    mine, _ = O.pack_mt(w, O.ALGO_ABSMAX)
    if not np.array_equal(ref, mine):
        print("the oracle's absmax packer differs from the reference experiment", file=sys.stderr)
        return 1
    scales = ref.reshape(-1, 1088)[:, :64].copy().view(np.uint16)
    normal = bool((((scales & 0x7C00) != 0) | ((scales & 0x3FF) == 0)).all())
    x = O.bench_activation(COLS)
    doc = dict(rows=ROWS, cols=COLS, seed=SEED, algorithm="absmax",
               tiles_sha256=hashlib.sha256(ref.tobytes()).hexdigest(),
               x_sha256=hashlib.sha256(x.tobytes()).hexdigest(), scales_normal=normal)
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1)
        f.write("\n")
    print(json.dumps(doc, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
