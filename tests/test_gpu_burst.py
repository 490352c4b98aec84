"""The burst kernel (int8 MFMA, tiles loaded straight into LDS, the
activation converted in the kernel) through the C ABI: per-tensor launches
with Q4RDNA_KERNEL_BURST and q4rdna_mul_mat_group (GEMVs sharing one x)
against the fp64 oracle and the reference bench's rel-L2 gate, over K
tails (groups that are not whole 16-group steps), split K chunks meeting in
the arrival chain, odd row counts, and the add / SwiGLU epilogues."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
import q4rdna
from q4rdna import _lib, api
from conftest import assert_gemv_parity

pytestmark = pytest.mark.gpu


def random_tiles(rows: int, cols: int, seed: int, subnormal: bool = False) -> np.ndarray:
    rng = np.random.default_rng(seed)
    g = cols // 64
    t = rng.integers(0, 256, (rows // 32, g, 1088), dtype=np.uint8)
    mag = rng.uniform(1e-3, 3e-2, (rows // 32, g, 32))
    if subnormal:
        mag[..., ::7] = rng.uniform(1e-7, 6e-5, mag[..., ::7].shape)
    s = (mag * rng.choice([-1.0, 1.0], mag.shape)).astype(np.float16)
    t[:, :, :64] = s.view(np.uint8).reshape(rows // 32, g, 64)
    return t.reshape(-1)


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).cuda()


def opts(kernel=_lib.KERNEL_BURST, steps=0, split=0):
    o = _lib.LaunchOptions()
    o.kernel = kernel
    o.burst_steps = steps
    o.split_k = split
    return o


def burst(w, x, y, gate=None, add=None, steps=0):
    L = q4rdna.load()
    o = opts(steps=steps)
    return L.q4rdna_mul_mat_ex(ctypes.byref(w.raw), ctypes.byref(gate.raw) if gate else None, x.data_ptr(),
                               None if add is None else add.data_ptr(), y.data_ptr(), ctypes.byref(o),
                               torch.cuda.current_stream().cuda_stream)


SHAPES = [(32, 64), (64, 512), (96, 1024), (1024, 4096), (4096, 4096), (160, 4736), (4096, 12288), (224, 28672)]


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("kind", ["plain", "add", "glu", "glu+add"])
def test_burst_per_tensor_matches_oracle(cuda, rows, cols, kind):
    t = random_tiles(rows, cols, rows + 3 * cols, subnormal=True)
    x = O.gaussian_x(cols, rows + cols)
    w = api.QWeight.from_tiles(dev(t, np.uint8), rows, cols)
    gt = gate = add_np = add = None
    if "glu" in kind:
        gt = random_tiles(rows, cols, rows + 5 * cols)
        gate = api.QWeight.from_tiles(dev(gt, np.uint8), rows, cols)
    if "add" in kind:
        add_np = O.gaussian_x(rows, 7 * rows + cols)
        add = dev(add_np, np.float32)
    xd = dev(x, np.float32)
    for steps in ((1,) if gate is not None else (1, 2)):
        y = torch.full((rows,), float("nan"), device="cuda")
        assert burst(w, xd, y, gate, add, steps) == q4rdna.OK, q4rdna.last_error()
        torch.cuda.synchronize()
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, gate_tiles=gt, add=add_np, label=(rows, cols, kind, steps))


def test_burst_is_deterministic_and_independent_of_steps_for_one_chunk(cuda):
    """Repeated launches are bit-identical; a K of at most 16 groups is one
    chunk at one or two steps, so both give the same bits."""
    rows, cols = 1024, 1024
    t = random_tiles(rows, cols, 5)
    w = api.QWeight.from_tiles(dev(t, np.uint8), rows, cols)
    xd = dev(O.gaussian_x(cols, 6), np.float32)
    outs = []
    for steps in (1, 1, 2, 2):
        y = torch.empty(rows, device="cuda")
        assert burst(w, xd, y, steps=steps) == q4rdna.OK
        torch.cuda.synchronize()
        outs.append(y.clone())
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def group_call(descs, x, steps=0):
    L = q4rdna.load()
    arr = (_lib.GroupDesc * len(descs))()
    for i, (w, gate, add, y) in enumerate(descs):
        arr[i].weight = w.raw
        arr[i].gate_tiles = gate.raw.tiles if gate is not None else None
        arr[i].add = None if add is None else add.data_ptr()
        arr[i].y = y.data_ptr()
    o = opts(steps=steps)
    return L.q4rdna_mul_mat_group(arr, len(descs), x.data_ptr(), x.numel(), ctypes.byref(o),
                                  torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("steps", [0, 1, 2])
def test_group_qkv_matches_oracle_and_single_launches(cuda, steps):
    """q, k and v of a layer (4096 / 1024 / 1024 rows x 4096) plus an odd
    96-row GEMV with an add, sharing one x, in one launch: each output
    against both bars and bit-identical to the same GEMV's own burst launch
    at the same steps."""
    cols = 4096
    specs = [(4096, None), (1024, None), (1024, None), (96, "add")]
    x = O.gaussian_x(cols, 77)
    xd = dev(x, np.float32)
    descs, checks = [], []
    for i, (rows, kind) in enumerate(specs):
        t = random_tiles(rows, cols, 300 + i)
        w = api.QWeight.from_tiles(dev(t, np.uint8), rows, cols)
        add_np = O.gaussian_x(rows, 400 + i) if kind == "add" else None
        add = None if add_np is None else dev(add_np, np.float32)
        y = torch.full((rows,), float("nan"), device="cuda")
        descs.append((w, None, add, y))
        checks.append((t, rows, add_np))
    assert group_call(descs, xd, steps) == q4rdna.OK, q4rdna.last_error()
    torch.cuda.synchronize()
    resolved = steps or None
    for (w, _, add, y), (t, rows, add_np) in zip(descs, checks):
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, add=add_np, label=(rows, steps))
        if resolved is not None:
            y1 = torch.full((rows,), float("nan"), device="cuda")
            assert burst(w, xd, y1, add=add, steps=resolved) == q4rdna.OK
            torch.cuda.synchronize()
            assert torch.equal(y1, y), (rows, steps)


def test_group_swiglu_gate_up(cuda):
    """gate and up of a layer as one SwiGLU descriptor (12288 x 4096), plus a
    second SwiGLU pair of 160 rows with an add, in one launch."""
    cols = 4096
    x = O.gaussian_x(cols, 91)
    xd = dev(x, np.float32)
    descs, checks = [], []
    for i, (rows, with_add) in enumerate([(12288, False), (160, True)]):
        t = random_tiles(rows, cols, 500 + i)
        gt = random_tiles(rows, cols, 600 + i)
        w = api.QWeight.from_tiles(dev(t, np.uint8), rows, cols)
        g = api.QWeight.from_tiles(dev(gt, np.uint8), rows, cols)
        add_np = O.gaussian_x(rows, 700 + i) if with_add else None
        add = None if add_np is None else dev(add_np, np.float32)
        y = torch.full((rows,), float("nan"), device="cuda")
        descs.append((w, g, add, y))
        checks.append((t, gt, rows, add_np))
    assert group_call(descs, xd) == q4rdna.OK, q4rdna.last_error()
    torch.cuda.synchronize()
    for (_, _, _, y), (t, gt, rows, add_np) in zip(descs, checks):
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, gate_tiles=gt, add=add_np, label=rows)


def test_group_long_k_down_projection(cuda):
    """down (4096 x 12288) and a 64-row GEMV of the same K with an add: 12
    or 6 chunks per block meeting in the arrival chain."""
    cols = 12288
    x = O.gaussian_x(cols, 93)
    xd = dev(x, np.float32)
    for steps in (1, 2):
        descs, checks = [], []
        for i, (rows, with_add) in enumerate([(4096, True), (64, False)]):
            t = random_tiles(rows, cols, 800 + i)
            w = api.QWeight.from_tiles(dev(t, np.uint8), rows, cols)
            add_np = O.gaussian_x(rows, 900 + i) if with_add else None
            add = None if add_np is None else dev(add_np, np.float32)
            y = torch.full((rows,), float("nan"), device="cuda")
            descs.append((w, None, add, y))
            checks.append((t, rows, add_np))
        assert group_call(descs, xd, steps) == q4rdna.OK
        torch.cuda.synchronize()
        for (_, _, _, y), (t, rows, add_np) in zip(descs, checks):
            assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, add=add_np, label=(rows, steps))


def test_group_argument_checks(cuda):
    L = q4rdna.load()
    t = random_tiles(64, 128, 1)
    w = api.QWeight.from_tiles(dev(t, np.uint8), 64, 128)
    w2 = api.QWeight.from_tiles(dev(random_tiles(64, 192, 2), np.uint8), 64, 192)
    x = torch.zeros(128, device="cuda")
    y = torch.full((64,), 3.0, device="cuda")
    # K differs from x: not applicable, nothing launched
    assert group_call([(w, None, None, y), (w2, None, None, y)], x) == q4rdna.NOT_APPLICABLE
    # gate for some descriptors only, y overlapping x, empty and oversized groups: argument errors
    assert group_call([(w, w, None, y), (w, None, None, y)], x) == q4rdna.ERR_ARGUMENT
    big = torch.zeros(256, device="cuda")
    assert group_call([(w, None, None, big[64:128])], big[:128]) == q4rdna.ERR_ARGUMENT
    arr = (_lib.GroupDesc * 9)()
    assert L.q4rdna_mul_mat_group(arr, 0, x.data_ptr(), 128, None, None) == q4rdna.ERR_ARGUMENT
    assert L.q4rdna_mul_mat_group(arr, 9, x.data_ptr(), 128, None, None) == q4rdna.ERR_ARGUMENT
    torch.cuda.synchronize()
    assert (y == 3.0).all()


def test_group_and_burst_replay_from_a_hip_graph(cuda):
    """A qkv group launch and a split-K burst launch captured into one graph
    (after eager calls set up the stream's workspace), replayed with new
    activations and eager work in between: every replay equals the eager
    results bit for bit."""
    cols = 4096
    ts = [random_tiles(r, cols, 1000 + r) for r in (4096, 1024, 1024)]
    ws = [api.QWeight.from_tiles(dev(t, np.uint8), r, cols) for t, r in zip(ts, (4096, 1024, 1024))]
    td = random_tiles(4096, 12288, 1003)
    wd = api.QWeight.from_tiles(dev(td, np.uint8), 4096, 12288)
    x = torch.empty(cols, device="cuda")
    xdn = torch.empty(12288, device="cuda")
    ys = [torch.empty(r, device="cuda") for r in (4096, 1024, 1024)]
    yd = torch.empty(4096, device="cuda")
    st = torch.cuda.Stream()

    def work():
        L = q4rdna.load()
        arr = (_lib.GroupDesc * 3)()
        for i in range(3):
            arr[i].weight = ws[i].raw
            arr[i].y = ys[i].data_ptr()
        o = opts()
        assert L.q4rdna_mul_mat_group(arr, 3, x.data_ptr(), cols, ctypes.byref(o), st.cuda_stream) == q4rdna.OK
        o2 = opts(steps=1)
        assert L.q4rdna_mul_mat_ex(ctypes.byref(wd.raw), None, xdn.data_ptr(), None, yd.data_ptr(), ctypes.byref(o2),
                                   st.cuda_stream) == q4rdna.OK

    with torch.cuda.stream(st):
        x.normal_()
        xdn.normal_()
        work()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        work()
    for rep in range(3):
        with torch.cuda.stream(st):
            x.normal_()
            xdn.normal_()
            work()
        st.synchronize()
        want = [y.clone() for y in ys + [yd]]
        for y in ys + [yd]:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            g.replay()
        st.synchronize()
        for got, w_ in zip(ys + [yd], want):
            assert torch.equal(got, w_), rep
    assert_gemv_parity(yd.cpu().numpy(), td, 4096, 12288, xdn.cpu().numpy(), label="graph down")
