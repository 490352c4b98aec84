"""The reference bench's own GPU-versus-CPU correctness case
(source/q4rdna_gemv_bench.hip:215-262), on this build's entry points.

The reference checks one 12288 x 4096 tile stream written by its CPU
experiment with the default absmax search (q4rdna_cpu_experiment.cpp:348)
against its sequential fp32 loop (:189-211) for the activation
x_i = sin(0.013 i) * 0.25 + cos(0.007 i) * 0.125 (:224-227), and fails when
the relative L2 error exceeds 1e-5 (:259-261).  Its weights were real
Qwen3-8B tensors; here they are bf16-rounded N(0, 0.02) weights of the same
shape, packed on the GPU with the absmax search.  The sha256 of the tiles
the reference's own experiment wrote for those weights is committed in
tests/golden/q4rdna_bench_case.json (tests/golden/make_bench_case_golden.py),
so the GPU packer must reproduce them byte for byte before the GEMV runs.

The GEMV then runs through q4rdna_mul_mat, q4rdna_mul_mat_add (zero add),
q4rdna_mul_mat_group and a plan, and each result is gated exactly as the
reference gates its kernel: relative L2 <= 1e-5 against the bench's own
loop, with the bench's fp16 decode (oracle gemv_seq_f32 with the reference
CPU decode; every scale here is a normal fp16 number).  The fp64 per-row bar
of tests/conftest.py applies too.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import oracle as O
import q4rdna
from q4rdna import api
from conftest import assert_gemv_parity

pytestmark = pytest.mark.gpu

CASE = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4rdna_bench_case.json")))
REL_L2_GATE = 1e-5  # source/q4rdna_gemv_bench.hip:259


@pytest.fixture(scope="module")
def bench_case(cuda):
    rows, cols = CASE["rows"], CASE["cols"]
    _, w = O.bf16_round(O.gaussian_weights(rows, cols, CASE["seed"]))
    tiles_dev = api.pack(torch.from_numpy(w).cuda(), q4rdna.ALGO_ABSMAX)
    tiles = tiles_dev.cpu().numpy()
    x = O.bench_activation(cols)
    assert hashlib.sha256(x.tobytes()).hexdigest() == CASE["x_sha256"]
    reference = O.gemv_seq_f32(tiles, rows, cols, x, ref_cpu_decode=True)
    return api.QWeight.from_tiles(tiles_dev, rows, cols), tiles, x, reference


def bench_gate(y: torch.Tensor, reference: np.ndarray, label: str) -> float:
    """The reference bench's check, restated (:250-262)."""
    actual = y.cpu().numpy().astype(np.float64)
    ref = reference.astype(np.float64)
    err = actual - ref
    rel = float(np.sqrt(np.sum(err * err) / np.sum(ref * ref)))
    assert rel <= REL_L2_GATE, (label, rel)
    return rel


def test_gpu_packer_reproduces_the_reference_tiles(bench_case):
    _, tiles, _, _ = bench_case
    assert hashlib.sha256(tiles.tobytes()).hexdigest() == CASE["tiles_sha256"]


def test_bench_case_per_tensor(bench_case):
    w, tiles, x, reference = bench_case
    xd = torch.from_numpy(x).cuda()
    y = api.mul_mat(w, xd)
    assert y is not None
    torch.cuda.synchronize()
    bench_gate(y, reference, "q4rdna_mul_mat")
    assert_gemv_parity(y.cpu().numpy(), tiles, w.rows, w.cols, x, label="q4rdna_mul_mat")
    y2 = api.mul_mat_add(w, xd, torch.zeros(w.rows, device="cuda"))
    torch.cuda.synchronize()
    bench_gate(y2, reference, "q4rdna_mul_mat_add")
    # every split the policy could pick, and the reference's own S = 8
    for split in (1, 2, 3, 4, 6, 8):
        ys = torch.full((w.rows,), float("nan"), device="cuda")
        assert api.mul_mat_ex(w, xd, ys, split_k=split)
        torch.cuda.synchronize()
        bench_gate(ys, reference, f"split {split}")


def test_bench_case_group(bench_case):
    """The weight twice in one shared-x group (two outputs, one launch)."""
    w, tiles, x, reference = bench_case
    ys = [torch.full((w.rows,), float("nan"), device="cuda") for _ in range(2)]
    assert api.mul_mat_group([(w, ys[0]), (w, ys[1])], torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    for i, y in enumerate(ys):
        bench_gate(y, reference, f"group member {i}")
        assert_gemv_parity(y.cpu().numpy(), tiles, w.rows, w.cols, x, label=("group", i))


def test_bench_case_plan(bench_case):
    """The weight in a plan (the int8-digit sweep), next to itself with a
    second output."""
    w, tiles, x, reference = bench_case
    xd = torch.from_numpy(x).cuda()
    ys = [torch.full((w.rows,), float("nan"), device="cuda") for _ in range(2)]
    plan = api.Plan([(w, xd, ys[0]), (w, xd, ys[1])])
    assert plan.launch()
    torch.cuda.synchronize()
    for i, y in enumerate(ys):
        bench_gate(y, reference, f"plan output {i}")
        assert_gemv_parity(y.cpu().numpy(), tiles, w.rows, w.cols, x, label=("plan", i))
    plan.close()
