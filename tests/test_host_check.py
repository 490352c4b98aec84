"""The runtime's host-only logic under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/host_check): the sidecar index parser on
valid, mutated, truncated and random images (statuses against the oracle's
restatement of the reference loader, source/q4rdna.cu:129-170), and the plan
layout with its item deal on the Qwen3-8B stacks, batched plans and mixed
plans (every item dealt exactly once, each workgroup's list ascending,
scratch regions aligned and disjoint), and the split-K exchange tree's
protocol with the kernels' own shape functions.  CPU only."""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
DIR = os.path.join(HERE, "host_check")
BIN = os.path.join(DIR, "host_check")


@pytest.fixture(scope="module")
def host_check():
    subprocess.run(["make", "-C", DIR, "-s"], check=True)
    return BIN


def run(binary, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([binary, *args], capture_output=True, text=True, timeout=300, env=env)
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    return r, [json.loads(line) for line in r.stdout.splitlines() if line.startswith("{")]


def test_plan_layout_and_deal_under_sanitizers(host_check):
    r, lines = run(host_check, "layout")
    assert r.returncode == 0, r.stdout + r.stderr
    by = {d["plan"]: d for d in lines if "plan" in d and "failed" not in d}
    assert [d for d in lines if "failed" in d] == []
    assert lines[-1] == {"failures": 0}
    s = by["qwen3_252"]
    # Per layer: the 4096-wide projections run pair items of 128 rows (q, o
    # 32 each, k, v 8 each, gate, up 96 each), down 64 items of 64 rows with
    # its whole 192-group row in one chunk: 336 items, 12,096 for 36 layers.
    assert (s["gemvs"], s["items"], s["groups"], s["workgroups"]) == (252, 12096, 20736, 512)
    assert s["all_per_one"] and not s["both_streams"]
    assert s["max_load"] <= 1.06 * s["mean_load"]
    f = by["qwen3_216_swiglu"]
    assert f["gemvs"] == 216 and f["both_streams"] and f["all_per_one"]
    assert by["qwen3_252_batch8"]["items"] == by["qwen3_252_batch4"]["items"]
    # Batched, 256-row blocks: q, o 16 each, k, v 4 each, the SwiGLU GEMV 48
    # (up and gate in one item), down 16: 104 items per layer, no partials.
    g8 = by["qwen3_216_swiglu_batch8"]
    assert g8["gemvs"] == 216 and g8["all_per_one"] and g8["both_streams"] and g8["items"] == 104 * 36
    assert not by["mixed"]["all_per_one"] and by["mixed"]["both_streams"]
    assert by["mixed_small_gpu"]["workgroups"] == 16
    assert by["one_gemv"]["items"] == 1


def test_sidecar_parser_under_sanitizers(host_check, golden, tmp_path):
    img = bytes(golden["sidecar_image"].tobytes())
    rng = np.random.default_rng(5)
    cases = {"valid": img, "empty": b"", "header_only": img[:48], "index_cut": img[:48 + 96 + 10],
             "data_cut": img[:-300], "random": rng.integers(0, 256, 5000, dtype=np.uint8).tobytes()}
    huge_count = bytearray(img)
    huge_count[12:16] = (0xFFFFFFFF).to_bytes(4, "little")
    cases["huge_count"] = bytes(huge_count)
    wrap = bytearray(img)
    wrap[40:48] = (2**64 - 16).to_bytes(8, "little")            # data_bytes near 2^64
    cases["data_bytes_wraps"] = bytes(wrap)
    off_wrap = bytearray(img)
    off_wrap[32:40] = (2**64 - 64).to_bytes(8, "little")        # data_offset near 2^64
    cases["data_offset_wraps"] = bytes(off_wrap)
    for i, (off, data) in enumerate([(0, b"Q4RDNA2"), (48 + 64, (33).to_bytes(4, "little")),
                                     (48 + 72, (2**64 - 8).to_bytes(8, "little")),
                                     (48 + 80, (2**63).to_bytes(8, "little")), (48, b"x" * 64)]):
        m = bytearray(img)
        m[off:off + len(data)] = data
        cases[f"mutation{i}"] = bytes(m)
    paths = []
    for name, data in cases.items():
        p = tmp_path / f"{name}.q4rdna"
        p.write_bytes(data)
        paths.append(str(p))
    r, lines = run(host_check, "inspect", *paths)
    assert r.returncode == 0, r.stderr
    got = {os.path.basename(d["file"])[:-len(".q4rdna")]: d for d in lines}
    assert got["valid"]["status"] == 0 and got["valid"]["count"] == 3
    for name, data in cases.items():
        if name == "valid":
            continue
        assert got[name]["status"] < 0, name
        # The oracle's loader restatement rejects the same images.
        assert O.validate_sidecar(bytearray(data)) < 0, name


def test_exchange_tree_protocol_under_sanitizers(host_check):
    """The kernels' exchange-tree shape (exchange_leaves / exchange_meets in
    csrc/q4rdna_internal.h) under random interleavings of the chunks'
    exchanges for every split 2..64: one root, every slot used exactly twice
    and left empty, split - 1 regions used, one sum expression.  Two planted
    mistakes in the shape rule (an off-by-one bound; meeting at every node)
    must fail it for every split that is not a power of two."""
    r, lines = run(host_check, "tree")
    assert r.returncode == 0, r.stdout + r.stderr
    assert {"split": 6, "root": "(((p0+p1)+(p2+p3))+(p4+p5))"} in lines
    assert lines[-1] == {"tree_splits": 63, "failures": 0}
    non_powers = sum(1 for s in range(2, 65) if s & (s - 1))
    for planted in ("tree-planted-off-by-one", "tree-planted-always"):
        r, lines = run(host_check, planted)
        assert r.returncode == 1
        assert lines[-1] == {"tree_splits": 63, "failures": non_powers}, planted
