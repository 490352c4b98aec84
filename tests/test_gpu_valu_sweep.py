"""The multi-tensor sweep in the VALU formulation (libq4rdna_valu_sweep_gfx950.so,
the library built with -DQ4RDNA_SWEEP_VALU for the MFMA-against-VALU
measurement of the sweep): same items, deal and finish as the int8-MFMA
sweep, the per-tensor kernels' arithmetic on fp32 activations.  Its plans
must meet both parity bars like the product's.  It runs in a fresh process,
since a process binds one build of the library."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
VARIANT = os.path.join(ROOT, "rdna-gfx1201-v0.1_amd", "q4rdna", "libq4rdna_valu_sweep_gfx950.so")

SCRIPT = r"""
import sys
sys.path[:0] = [{root!r}, {pkg!r}, {tests!r}]
import numpy as np, torch
import q4rdna._lib as L
L.LIB_PATH = {lib!r}
import oracle as O
from q4rdna import api
from conftest import assert_gemv_parity
from test_gpu_parity import dev_f32, dev_u8, random_tiles, wide_x
assert L.load()._name == {lib!r}
# Pair items (rows of one chunk, no gate), a SwiGLU GEMV of one chunk
# (both streams in one item), split-K chains (12288 and 28672 columns, with
# and without a gate), short tails and odd row-tile counts, the add epilogue.
shapes = [(128, 512, None), (96, 4736, None), (4096, 4096, None), (1024, 4096, "add"), (384, 512, "glu"),
          (160, 8192, "glu"), (96, 12288, "add"), (224, 28672, None), (64, 12800, "glu"), (32, 4096, "glu")]
items, checks = [], []
for i, (rows, cols, kind) in enumerate(shapes):
    t = random_tiles(rows, cols, 700 + i)
    x = O.gaussian_x(cols, 800 + i)
    y = torch.full((rows,), np.nan, device="cuda")
    gate = add = gt = add_np = None
    if kind == "glu":
        gt = random_tiles(rows, cols, 900 + i)
        gate = api.QWeight.from_tiles(dev_u8(gt), rows, cols)
    if kind == "add":
        add_np = O.gaussian_x(rows, 1000 + i)
        add = dev_f32(add_np)
    items.append((api.QWeight.from_tiles(dev_u8(t), rows, cols), dev_f32(x), y, gate, add))
    checks.append((t, gt, x, add_np, rows, cols, y))
plan = api.Plan(items)
for _ in range(2):  # a second launch repeats the first (counters left clean)
    assert plan.launch()
    torch.cuda.synchronize()
    for t, gt, x, add_np, rows, cols, y in checks:
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, gate_tiles=gt, add=add_np, label=(rows, cols))
plan.close()
# Subnormal fp16 scales, activation groups eight decades apart and a zero group.
t = random_tiles(256, 4096, 71, subnormal=True)
x = wide_x(4096, 72)
y = torch.full((256,), np.nan, device="cuda")
plan = api.Plan([(api.QWeight.from_tiles(dev_u8(t), 256, 4096), dev_f32(x), y)])
assert plan.launch()
torch.cuda.synchronize()
assert_gemv_parity(y.cpu().numpy(), t, 256, 4096, x, label="wide")
plan.close()
print("ok")
"""


def test_valu_sweep_plans_meet_both_bars(cuda):
    assert os.path.exists(VARIANT), "build it with make -C rdna-gfx1201-v0.1_amd valu-sweep"
    code = SCRIPT.format(root=ROOT, pkg=os.path.join(ROOT, "rdna-gfx1201-v0.1_amd"), tests=os.path.join(ROOT, "tests"),
                         lib=VARIANT)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok"), r.stdout
