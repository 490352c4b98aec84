"""q4rdna_mul_mat_ex_noalloc through the C ABI: the allocation-free variant
of q4rdna_mul_mat_ex, whose split-K workspace is a fixed per-GPU device
array.  Its outputs must equal q4rdna_mul_mat_ex's at the same split bit for
bit (same kernels, same summation order), on consecutive calls with the
second smaller than the first, with every epilogue; a launch that needs more
than the array holds is refused and touches nothing; and calls captured into
a HIP graph replay correctly."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
import q4rdna
from q4rdna import _lib, api
from conftest import assert_gemv_parity

pytestmark = pytest.mark.gpu


def random_tiles(rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    g = cols // 64
    t = rng.integers(0, 256, (rows // 32, g, 1088), dtype=np.uint8)
    s = (rng.uniform(1e-3, 3e-2, (rows // 32, g, 32)) * rng.choice([-1.0, 1.0], (rows // 32, g, 32))).astype(np.float16)
    t[:, :, :64] = s.view(np.uint8).reshape(rows // 32, g, 64)
    return t.reshape(-1)


def weight(rows, cols, seed):
    t = random_tiles(rows, cols, seed)
    return t, api.QWeight.from_tiles(torch.from_numpy(t).cuda(), rows, cols)


def call(fn, w, gate, x, add, y, split, stream):
    opts = _lib.LaunchOptions()
    opts.split_k = split
    return fn(ctypes.byref(w.raw), ctypes.byref(gate.raw) if gate is not None else None, x.data_ptr(),
              None if add is None else add.data_ptr(), y.data_ptr(), ctypes.byref(opts), stream)


CASES = [
    # rows, cols, split, gate, add: a larger launch, then a smaller one
    (4096, 12288, 6, True, True),
    (1024, 4096, 4, False, False),
    (12288, 4096, 2, True, False),
    (4096, 4096, 2, False, True),
    (96, 8192, 16, True, False),
]


def test_noalloc_equals_mul_mat_ex(cuda):
    L = q4rdna.load()
    s = torch.cuda.current_stream().cuda_stream
    for i, (rows, cols, split, with_gate, with_add) in enumerate(CASES):
        t, w = weight(rows, cols, 10 + i)
        gt, g = weight(rows, cols, 20 + i) if with_gate else (None, None)
        x_np = O.gaussian_x(cols, 30 + i)
        add_np = O.gaussian_x(rows, 40 + i) if with_add else None
        x = torch.from_numpy(x_np).cuda()
        add = None if add_np is None else torch.from_numpy(add_np).cuda()
        y_ref = torch.full((rows,), float("nan"), device="cuda")
        y_na = torch.full((rows,), float("nan"), device="cuda")
        assert call(L.q4rdna_mul_mat_ex, w, g, x, add, y_ref, split, s) == q4rdna.OK
        assert call(L.q4rdna_mul_mat_ex_noalloc, w, g, x, add, y_na, split, s) == q4rdna.OK, q4rdna.last_error()
        torch.cuda.synchronize()
        assert torch.equal(y_na, y_ref), (rows, cols, split)
        assert_gemv_parity(y_na.cpu().numpy(), t, rows, cols, x_np, gate_tiles=gt, add=add_np, label=(rows, cols))


def test_noalloc_refuses_what_does_not_fit(cuda):
    """151936 x 4096 at split 16 meets in a tree of 15 slot regions:
    2,279,040 slots, more than the 2,097,152 the array holds: refused,
    nothing launched.  Likewise a split-2 launch with more rows than slots."""
    L = q4rdna.load()
    rows, cols = 151936, 4096
    assert 15 * rows > _lib.NOALLOC_SLOTS
    w = api.QWeight.from_tiles(torch.zeros(api.packed_size(rows, cols), dtype=torch.uint8, device="cuda"), rows, cols)
    x = torch.zeros(cols, device="cuda")
    y = torch.full((rows,), 7.0, device="cuda")
    rc = call(L.q4rdna_mul_mat_ex_noalloc, w, None, x, None, y, 16, torch.cuda.current_stream().cuda_stream)
    assert rc == q4rdna.ERR_ARGUMENT
    assert "no-alloc scratch" in q4rdna.last_error()
    torch.cuda.synchronize()
    assert (y == 7.0).all()
    # split 1 needs no workspace at all and runs at any size
    rc = call(L.q4rdna_mul_mat_ex_noalloc, w, None, x, None, y, 1, torch.cuda.current_stream().cuda_stream)
    assert rc == q4rdna.OK
    torch.cuda.synchronize()
    assert (y == 0.0).all()
    del w, y
    # split 2 exchanges through one slot per row: 2,097,184 rows need more
    # than the 2,097,152 slots
    rows, cols = 2097184, 128
    assert rows > _lib.NOALLOC_SLOTS
    w = api.QWeight.from_tiles(torch.zeros(api.packed_size(rows, cols), dtype=torch.uint8, device="cuda"), rows, cols)
    x = torch.zeros(cols, device="cuda")
    y = torch.full((rows,), 7.0, device="cuda")
    rc = call(L.q4rdna_mul_mat_ex_noalloc, w, None, x, None, y, 2, torch.cuda.current_stream().cuda_stream)
    assert rc == q4rdna.ERR_ARGUMENT
    assert "slots" in q4rdna.last_error()
    torch.cuda.synchronize()
    assert (y == 7.0).all()


def test_noalloc_calls_replay_from_a_hip_graph(cuda):
    """Two allocation-free launches captured into one graph (after a first
    call has set the GPU up), replayed with new activations and eager work in
    between: every replay equals the eager results bit for bit."""
    L = q4rdna.load()
    t1, w1 = weight(4096, 4096, 50)
    t2, w2 = weight(1024, 12288, 51)
    x1 = torch.empty(4096, device="cuda")
    x2 = torch.empty(12288, device="cuda")
    y1 = torch.empty(4096, device="cuda")
    y2 = torch.empty(1024, device="cuda")
    st = torch.cuda.Stream()

    def work():
        assert call(L.q4rdna_mul_mat_ex_noalloc, w1, None, x1, None, y1, 2, st.cuda_stream) == q4rdna.OK
        assert call(L.q4rdna_mul_mat_ex_noalloc, w2, None, x2, None, y2, 6, st.cuda_stream) == q4rdna.OK

    with torch.cuda.stream(st):
        x1.normal_()
        x2.normal_()
        work()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        work()
    for rep in range(3):
        with torch.cuda.stream(st):
            x1.normal_()
            x2.normal_()
            work()
        st.synchronize()
        want = [y1.clone(), y2.clone()]
        y1.fill_(float("nan"))
        y2.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            g.replay()
        st.synchronize()
        assert torch.equal(y1, want[0]) and torch.equal(y2, want[1]), rep
    assert_gemv_parity(y2.cpu().numpy(), t2, 1024, 12288, x2.cpu().numpy(), label="graph replay")


FIRST_CALL_CAPTURED = r"""
import ctypes, sys
sys.path[:0] = [{root!r}, {pkg!r}]
import numpy as np
import torch
import q4rdna
from q4rdna import _lib, api
L = q4rdna.load()


def weight(rows, cols, seed):
    rng = np.random.default_rng(seed)
    t = rng.integers(0, 256, (rows // 32, cols // 64, 1088), dtype=np.uint8)
    s = (rng.uniform(1e-3, 3e-2, (rows // 32, cols // 64, 32)) * rng.choice([-1.0, 1.0], (rows // 32, cols // 64, 32)))
    t[:, :, :64] = s.astype(np.float16).view(np.uint8).reshape(rows // 32, cols // 64, 64)
    return api.QWeight.from_tiles(torch.from_numpy(t.reshape(-1)).cuda(), rows, cols)


def call(fn, w, gate, x, y, split, stream):
    o = _lib.LaunchOptions()
    o.split_k = split
    return fn(ctypes.byref(w.raw), None if gate is None else ctypes.byref(gate.raw), x.data_ptr(), None,
              y.data_ptr(), ctypes.byref(o), stream)


big, small = (weight(4096, 4096, 1), weight(4096, 4096, 2)), (weight(1024, 4096, 3), weight(1024, 4096, 4))
st = torch.cuda.Stream()
xg = torch.randn(4096, device="cuda")
yg = [torch.full((4096,), float("nan"), device="cuda") for _ in range(2)]
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
# The process's first no-alloc calls, split 2 (exchange slots), plain and
# SwiGLU, are captured: nothing runs until the graph is replayed.
with torch.cuda.graph(g, stream=st):
    assert call(L.q4rdna_mul_mat_ex_noalloc, big[0], None, xg, yg[0], 2, st.cuda_stream) == 0, q4rdna.last_error()
    assert call(L.q4rdna_mul_mat_ex_noalloc, big[0], big[1], xg, yg[1], 2, st.cuda_stream) == 0, q4rdna.last_error()
cur = torch.cuda.current_stream().cuda_stream
# Eager split-2 calls before the first replay, larger then smaller, each
# equal bit for bit to q4rdna_mul_mat_ex at the same split.
for up, gate in (big, small, big):
    for gt in (None, gate):
        x = torch.randn(up.cols, device="cuda")
        y_na = torch.full((up.rows,), float("nan"), device="cuda")
        y_ex = torch.full((up.rows,), float("nan"), device="cuda")
        assert call(L.q4rdna_mul_mat_ex_noalloc, up, gt, x, y_na, 2, cur) == 0, q4rdna.last_error()
        assert call(L.q4rdna_mul_mat_ex, up, gt, x, y_ex, 2, cur) == 0, q4rdna.last_error()
        torch.cuda.synchronize()
        assert torch.equal(y_na, y_ex), (up.rows, gt is not None)
want = [torch.empty(4096, device="cuda") for _ in range(2)]
assert call(L.q4rdna_mul_mat_ex, big[0], None, xg, want[0], 2, cur) == 0
assert call(L.q4rdna_mul_mat_ex, big[0], big[1], xg, want[1], 2, cur) == 0
torch.cuda.synchronize()
for rep in range(3):
    for y in yg:
        y.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        g.replay()
    st.synchronize()
    assert torch.equal(yg[0], want[0]) and torch.equal(yg[1], want[1]), rep
print("ok")
"""


def test_noalloc_first_call_captured_then_eager_calls(cuda):
    """In a fresh process, the first allocation-free calls (split 2, plain
    and SwiGLU) are captured into a graph, so they do not run; eager split-2
    calls made before the first replay must still equal q4rdna_mul_mat_ex
    bit for bit (the empty exchange slot is all-zero memory, which the device
    array holds from the start), and the replays must too."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = FIRST_CALL_CAPTURED.format(root=root, pkg=os.path.join(root, "rdna-gfx1201-v0.1_amd"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok"), r.stdout
