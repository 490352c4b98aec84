"""The reference's old mapping (Q4RDNA_KERNEL_SEQUENTIAL, source/q4rdna.cu:
190-234,626-634) and its launch statistics and exit report
(source/q4rdna.cu:57,73-112,176,706-709,742,764,789-791).

The old mapping sums each row in one thread, its weights in k order with one
fp32 fma each: the reference bench's CPU loop (q4rdna_gemv_bench.hip:189-210)
step for step, so the GPU result is that loop's bits, which the oracle's
q4o_gemv_seq_f32 reproduces."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import oracle as O
from q4rdna import _lib, api

from test_gpu_parity import dev_f32, dev_u8, random_tiles

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("rows,cols,subnormal", [(96, 4096, False), (160, 12288, True), (4096, 1024, False),
                                                 (32, 64, False)])
def test_sequential_kernel_is_the_cpu_loop_bit_for_bit(cuda, rows, cols, subnormal):
    t = random_tiles(rows, cols, 900 + rows + cols, subnormal=subnormal)
    x = O.gaussian_x(cols, 901 + cols)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    y = torch.full((rows,), float("nan"), device="cuda")
    assert api.mul_mat_ex(w, dev_f32(x), y, kernel=_lib.KERNEL_SEQUENTIAL)
    torch.cuda.synchronize()
    want = O.gemv_seq_f32(t, rows, cols, x)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # The add epilogue is one fp32 addition after the loop.
    add = O.gaussian_x(rows, 902 + rows)
    assert api.mul_mat_ex(w, dev_f32(x), y, add=dev_f32(add), kernel=_lib.KERNEL_SEQUENTIAL, split_k=1)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), (want + add.astype(np.float32)).view(np.uint32))


def test_sequential_swiglu_against_both_bars(cuda):
    rows, cols = 256, 4096
    up_t, gate_t = random_tiles(rows, cols, 910), random_tiles(rows, cols, 911)
    x = O.gaussian_x(cols, 912)
    up = api.QWeight.from_tiles(dev_u8(up_t), rows, cols)
    gate = api.QWeight.from_tiles(dev_u8(gate_t), rows, cols)
    y = torch.full((rows,), float("nan"), device="cuda")
    assert api.mul_mat_ex(up, dev_f32(x), y, gate=gate, kernel=_lib.KERNEL_SEQUENTIAL)
    torch.cuda.synchronize()
    from conftest import assert_gemv_parity
    assert_gemv_parity(y.cpu().numpy(), up_t, rows, cols, x, gate_tiles=gate_t, label="sequential glu")
    # Before the epilogue both sums are the CPU loop's: silu is the only
    # difference (GPU expf against the oracle's), a few ulps.
    u = O.gemv_seq_f32(up_t, rows, cols, x).astype(np.float64)
    g = O.gemv_seq_f32(gate_t, rows, cols, x).astype(np.float64)
    ref = u * O.silu(g)
    assert np.max(np.abs(y.cpu().numpy() - ref) / np.maximum(np.abs(ref), 1e-30)) < 1e-6


def test_sequential_options_batch_and_group(cuda):
    rows, cols, n = 64, 2048, 3
    t = random_tiles(rows, cols, 920)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    xs = np.stack([O.gaussian_x(cols, 921 + v) for v in range(n)])
    y = torch.full((n, rows), float("nan"), device="cuda")
    assert api.mul_mat_batch(w, dev_f32(xs), y, kernel=_lib.KERNEL_SEQUENTIAL)
    torch.cuda.synchronize()
    for v in range(n):
        want = O.gemv_seq_f32(t, rows, cols, xs[v])
        assert np.array_equal(y[v].cpu().numpy().view(np.uint32), want.view(np.uint32)), v
    with pytest.raises(_lib.Q4RdnaError):  # only split 1 exists for it
        api.mul_mat_ex(w, dev_f32(xs[0]), y[0], kernel=_lib.KERNEL_SEQUENTIAL, split_k=2)
    with pytest.raises(_lib.Q4RdnaError):  # a group launch is the split-K kernel
        api.mul_mat_group([(w, y[0])], dev_f32(xs[0]), kernel=_lib.KERNEL_SEQUENTIAL)
    with pytest.raises(_lib.Q4RdnaError):
        api.mul_mat_ex(w, dev_f32(xs[0]), y[0], kernel=2)


def test_launch_count_and_entry_hits(cuda, golden):
    sc = api.Sidecar.from_bytes(golden["sidecar_image"].tobytes())
    entries = sc.entries()
    (n0, r0, c0, _, _), (n1, r1, c1, _, _) = entries[0], entries[1]
    w0 = sc.find(n0, c0, r0)
    w1 = sc.find(n1, c1, r1)
    before = api.launch_count()
    assert [sc.hits(i) for i in range(len(entries))] == [0] * len(entries)
    x0 = dev_f32(O.gaussian_x(c0, 930))
    api.mul_mat(w0, x0)
    api.mul_mat(w0, x0)
    api.mul_mat_ex(w0, x0, torch.empty(r0, device="cuda"), kernel=_lib.KERNEL_SEQUENTIAL)
    if (r0, c0) == (r1, c1):
        api.mul_mat_glu(w0, w1, x0)
        expect0, expect1 = 4, 1
    else:
        api.mul_mat(w1, dev_f32(O.gaussian_x(c1, 931)))
        expect0, expect1 = 3, 1
    torch.cuda.synchronize()
    assert api.launch_count() - before == 4
    assert sc.hits(0) == expect0 and sc.hits(1) == expect1
    assert sc.hits(len(entries)) == 0  # out of range
    # Weights that are not sidecar entries count launches, no hits.
    t = random_tiles(32, 64, 932)
    api.mul_mat(api.QWeight.from_tiles(dev_u8(t), 32, 64), dev_f32(O.gaussian_x(64, 933)))
    torch.cuda.synchronize()
    assert api.launch_count() - before == 5
    assert sc.hits(0) == expect0
    sc.close()


REPORT_SCRIPT = r"""
import sys
sys.path[:0] = [{root!r}, {pkg!r}]
import torch
import q4rdna
from q4rdna import api
from q4rdna._lib import Weight
import ctypes
L = q4rdna.load()
h = L.q4rdna_default_sidecar(0)
assert h
w = Weight()
assert L.q4rdna_find(ctypes.c_void_p(h), {name!r}.encode(), {cols}, {rows}, ctypes.byref(w)) == 0
x = torch.randn({cols}, device="cuda")
for _ in range(3):
    api.mul_mat(api.QWeight(w), x)
torch.cuda.synchronize()
"""


@pytest.mark.parametrize("trace", [False, True])
def test_exit_report_in_the_reference_words(cuda, golden, tmp_path, trace):
    """At exit, once the default sidecar has loaded, the report lists the
    launches, the per-entry hits under LLAMA_Q4_RDNA_TRACE, and the
    hits-by-shape summary, in the reference's lines."""
    p = tmp_path / "three.q4rdna"
    p.write_bytes(golden["sidecar_image"].tobytes())
    sc = api.Sidecar.from_bytes(golden["sidecar_image"].tobytes())
    name, rows, cols, _, _ = sc.entries()[0]
    sc.close()
    env = dict(os.environ)
    env["LLAMA_Q4_RDNA_SIDECAR"] = str(p)
    env.pop("LLAMA_Q4_RDNA_TRACE", None)
    if trace:
        env["LLAMA_Q4_RDNA_TRACE"] = "1"
    code = REPORT_SCRIPT.format(root=ROOT, pkg=os.path.join(ROOT, "rdna-gfx1201-v0.1_amd"), name=name, rows=rows,
                                cols=cols)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [ln for ln in r.stderr.splitlines() if ln.startswith("Q4_RDNA:")]
    assert "Q4_RDNA: launched 3 decode GEMV kernels" in lines, lines
    buckets = {(12288, 4096): 0, (4096, 12288): 0, (4096, 4096): 0, (1024, 4096): 0}
    other = 3 if (rows, cols) not in buckets else 0
    if (rows, cols) in buckets:
        buckets[(rows, cols)] = 3
    summary = ("Q4_RDNA: unique=1, hits by rows x columns: 12288x4096=%d, 4096x12288=%d, 4096x4096=%d, "
               "1024x4096=%d, other=%d" % (buckets[(12288, 4096)], buckets[(4096, 12288)], buckets[(4096, 4096)],
                                           buckets[(1024, 4096)], other))
    assert lines[-1] == summary, lines
    hit = "Q4_RDNA: hit %-31s %d" % (name, 3)
    assert (hit in lines) == trace, lines
