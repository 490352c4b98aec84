"""The clock build of the library (libq4rdna_sweep_clocks_gfx950.so,
-DQ4RDNA_SWEEP_CLOCKS, read by bench.py --clocks): its sweep still meets
both parity bars, and q4rdna_sweep_clocks returns one (start, end) pair of
100 MHz counter values per workgroup of the latest sweep, every start before
its end and the whole launch within a plausible window.  It runs in a fresh
process, since a process binds one build of the library."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
VARIANT = os.path.join(ROOT, "rdna-gfx1201-v0.1_amd", "q4rdna", "libq4rdna_sweep_clocks_gfx950.so")

SCRIPT = r"""
import ctypes, sys
sys.path[:0] = [{root!r}, {pkg!r}, {tests!r}]
import numpy as np, torch
import q4rdna._lib as L
L.LIB_PATH = {lib!r}
import oracle as O
from q4rdna import api
from conftest import assert_gemv_parity
from test_gpu_parity import dev_f32, dev_u8, random_tiles
lib = L.load()
assert lib._name == {lib!r}
fn = lib.q4rdna_sweep_clocks
fn.restype = ctypes.c_int
fn.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
shapes = [(128, 4096, None), (4096, 4096, None), (96, 12288, "add"), (160, 8192, "glu")]
items, checks = [], []
for i, (rows, cols, kind) in enumerate(shapes):
    t = random_tiles(rows, cols, 1100 + i)
    x = O.gaussian_x(cols, 1200 + i)
    y = torch.full((rows,), np.nan, device="cuda")
    gate = add = gt = add_np = None
    if kind == "glu":
        gt = random_tiles(rows, cols, 1300 + i)
        gate = api.QWeight.from_tiles(dev_u8(gt), rows, cols)
    if kind == "add":
        add_np = O.gaussian_x(rows, 1400 + i)
        add = dev_f32(add_np)
    items.append((api.QWeight.from_tiles(dev_u8(t), rows, cols), dev_f32(x), y, gate, add))
    checks.append((t, gt, x, add_np, rows, cols, y))
plan = api.Plan(items)
wg = plan.workgroups
buf = np.zeros(2 * wg, dtype=np.uint64)
for rep in range(2):
    assert plan.launch()
    torch.cuda.synchronize()
    assert fn(buf.ctypes.data, wg) == 0
    start, end = buf[0::2].astype(np.int64), buf[1::2].astype(np.int64)
    # workgroups with no items in this small plan record nothing: only the
    # ones with items are checked
    have = end > 0
    assert have.sum() >= 1
    assert (start[have] <= end[have]).all()
    span_us = (end[have].max() - start[have].min()) / 100.0
    assert 0 < span_us < 10000, span_us
    for t, gt, x, add_np, rows, cols, y in checks:
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, gate_tiles=gt, add=add_np, label=(rows, cols))
assert fn(buf.ctypes.data, 1 << 20) != 0  # beyond the recorded workgroups: refused
plan.close()
print("ok")
"""


def test_clock_build_records_every_workgroup(cuda):
    assert os.path.exists(VARIANT), "build it with make -C rdna-gfx1201-v0.1_amd sweep-clocks"
    code = SCRIPT.format(root=ROOT, pkg=os.path.join(ROOT, "rdna-gfx1201-v0.1_amd"), tests=os.path.join(ROOT, "tests"),
                         lib=VARIANT)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok"), r.stdout
