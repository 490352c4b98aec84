"""q4rdna_mul_mat_group on the VALU kernel (the group policy): GEMVs sharing
one activation in one launch, their row tiles in one index space.  Every
output is checked against the fp64 oracle and the sequential-fp32 gate, and
against q4rdna_mul_mat_ex of the same GEMV at the same split bit for bit
(same kernel arithmetic, same reduction order); at split 2 the chunks meet
in one exchange slot per row, at larger splits in a tree of them."""
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


@pytest.mark.parametrize("split", [0, 2, 3, 4])
def test_valu_group_qkv_with_an_odd_member(cuda, split):
    """q, k, v of a layer plus a 96-row GEMV with an add, one x."""
    cols = 4096
    shapes = [(4096, False), (1024, False), (1024, False), (96, True)]
    members = []
    for i, (rows, with_add) in enumerate(shapes):
        t, w = weight(rows, cols, 700 + i)
        add_np = O.gaussian_x(rows, 710 + i) if with_add else None
        members.append((t, w, add_np, None if add_np is None else torch.from_numpy(add_np).cuda(), rows))
    x_np = O.gaussian_x(cols, 720)
    x = torch.from_numpy(x_np).cuda()
    ys = [torch.full((rows,), float("nan"), device="cuda") for *_, rows in members]
    items = [(w, y, None, add) for (t, w, add_np, add, rows), y in zip(members, ys)]
    assert api.mul_mat_group(items, x, split_k=split)
    torch.cuda.synchronize()
    for (t, w, add_np, add, rows), y in zip(members, ys):
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, add=add_np, label=(rows, split))
    if split:
        for (t, w, add_np, add, rows), y in zip(members, ys):
            y1 = torch.empty(rows, device="cuda")
            assert api.mul_mat_ex(w, x, y1, add=add, split_k=split, kernel=_lib.KERNEL_VALU)
            torch.cuda.synchronize()
            assert torch.equal(y, y1), (rows, split)


def test_valu_group_swiglu_equals_mul_mat_glu(cuda):
    """gate/up of a layer as a one-GEMV group with a gate, and two such GEMVs
    in one group: equal to q4rdna_mul_mat_glu bit for bit."""
    rows, cols = 12288, 4096
    ut, up = weight(rows, cols, 730)
    gt, gate = weight(rows, cols, 731)
    ut2, up2 = weight(1024, cols, 732)
    gt2, gate2 = weight(1024, cols, 733)
    x_np = O.gaussian_x(cols, 734)
    x = torch.from_numpy(x_np).cuda()
    y = torch.empty(rows, device="cuda")
    y2 = torch.empty(1024, device="cuda")
    assert api.policy_split_k(rows, cols) == 2 and api.policy_split_k(rows + 1024, cols) == 2
    assert api.mul_mat_group([(up, y, gate), (up2, y2, gate2)], x)
    ref = torch.empty(rows, device="cuda")
    ref2 = torch.empty(1024, device="cuda")
    assert api.mul_mat_glu(up, gate, x, ref) is not None
    assert api.mul_mat_ex(up2, x, ref2, gate=gate2, split_k=2)
    torch.cuda.synchronize()
    assert torch.equal(y, ref) and torch.equal(y2, ref2)
    assert_gemv_parity(y.cpu().numpy(), ut, rows, cols, x_np, gate_tiles=gt, label="glu")
    assert_gemv_parity(y2.cpu().numpy(), ut2, 1024, cols, x_np, gate_tiles=gt2, label="glu 1024")


def test_valu_group_long_k_exchange_tree(cuda):
    """A down projection (K = 12288, split 6 by the policy) and a smaller
    long-K GEMV with an add: the exchange tree, equal to single launches."""
    cols = 12288
    t1, w1 = weight(4096, cols, 740)
    t2, w2 = weight(512, cols, 741)
    add_np = O.gaussian_x(512, 742)
    add = torch.from_numpy(add_np).cuda()
    x_np = O.gaussian_x(cols, 743)
    x = torch.from_numpy(x_np).cuda()
    y1 = torch.empty(4096, device="cuda")
    y2 = torch.empty(512, device="cuda")
    split = api.policy_split_k(4096 + 512, cols)
    assert split > 2
    assert api.mul_mat_group([(w1, y1), (w2, y2, None, add)], x)
    r1 = torch.empty(4096, device="cuda")
    r2 = torch.empty(512, device="cuda")
    assert api.mul_mat_ex(w1, x, r1, split_k=split, kernel=_lib.KERNEL_VALU)
    assert api.mul_mat_ex(w2, x, r2, add=add, split_k=split, kernel=_lib.KERNEL_VALU)
    torch.cuda.synchronize()
    assert torch.equal(y1, r1) and torch.equal(y2, r2)
    assert_gemv_parity(y1.cpu().numpy(), t1, 4096, cols, x_np, label="down")
    assert_gemv_parity(y2.cpu().numpy(), t2, 512, cols, x_np, add=add_np, label="512 + add")


def test_valu_group_replays_from_a_hip_graph(cuda):
    """A VALU group launch and a per-tensor launch on one stream captured
    into a graph, replayed with fresh activations and eager work in
    between: every replay equals the eager results bit for bit."""
    cols = 4096
    _, wq = weight(4096, cols, 750)
    _, wk = weight(1024, cols, 751)
    _, wo = weight(4096, cols, 752)
    x = torch.empty(cols, device="cuda")
    yq, yk, yo = torch.empty(4096, device="cuda"), torch.empty(1024, device="cuda"), torch.empty(4096, device="cuda")
    st = torch.cuda.Stream()

    def work():
        assert api.mul_mat_group([(wq, yq), (wk, yk)], x, stream=st.cuda_stream)
        assert api.mul_mat_add(wo, yq, x, yo, stream=st.cuda_stream) is not None

    with torch.cuda.stream(st):
        x.normal_()
        work()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        work()
    for rep in range(3):
        with torch.cuda.stream(st):
            x.normal_()
            work()
        st.synchronize()
        want = [yq.clone(), yk.clone(), yo.clone()]
        for y in (yq, yk, yo):
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            g.replay()
        st.synchronize()
        for y, w_ in zip((yq, yk, yo), want):
            assert torch.equal(y, w_), rep


def test_valu_group_options(cuda):
    """An explicit VALU kernel equals the policy; unknown kernels (2, the
    withdrawn burst kernel, and 4), nonzero reserved words and oversize
    splits are argument errors that launch nothing."""
    L = q4rdna.load()
    cols = 4096
    _, w = weight(1024, cols, 760)
    x = torch.from_numpy(O.gaussian_x(cols, 761)).cuda()
    y_valu = torch.empty(1024, device="cuda")
    y_policy = torch.empty(1024, device="cuda")
    assert api.mul_mat_group([(w, y_valu)], x, kernel=_lib.KERNEL_VALU)
    assert api.mul_mat_group([(w, y_policy)], x)
    torch.cuda.synchronize()
    assert torch.equal(y_valu, y_policy)
    arr = (_lib.GroupDesc * 1)()
    arr[0].weight = w.raw
    arr[0].y = y_valu.data_ptr()
    for kernel, split, reserved in ((2, 0, 0), (4, 0, 0), (_lib.KERNEL_VALU, 65, 0), (0, 0, 1)):
        o = _lib.LaunchOptions()
        o.kernel = kernel
        o.split_k = split
        o.reserved[0] = reserved
        y_valu.fill_(7.0)
        rc = L.q4rdna_mul_mat_group(arr, 1, x.data_ptr(), cols, ctypes.byref(o), torch.cuda.current_stream().cuda_stream)
        assert rc == q4rdna.ERR_ARGUMENT, (kernel, split, reserved)
        torch.cuda.synchronize()
        assert (y_valu == 7.0).all()
        y1 = torch.full((1024,), 7.0, device="cuda")
        rc = L.q4rdna_mul_mat_ex(ctypes.byref(w.raw), None, x.data_ptr(), None, y1.data_ptr(), ctypes.byref(o),
                                 torch.cuda.current_stream().cuda_stream)
        assert rc == q4rdna.ERR_ARGUMENT, (kernel, split, reserved)
        torch.cuda.synchronize()
        assert (y1 == 7.0).all()


def test_valu_group_rejects_overlapping_outputs(cuda):
    """Members run unordered, so an output overlapping another member's
    output or bias is an argument error, and nothing is launched; the same
    buffers without overlap run."""
    L = q4rdna.load()
    cols = 4096
    _, w = weight(256, cols, 770)
    x = torch.from_numpy(O.gaussian_x(cols, 771)).cuda()
    buf = torch.full((1024,), 7.0, device="cuda")
    add = torch.zeros(256, device="cuda")

    def run(y0, y1, add1):
        arr = (_lib.GroupDesc * 2)()
        for i, (y, a) in enumerate(((y0, None), (y1, add1))):
            arr[i].weight = w.raw
            arr[i].y = y.data_ptr()
            arr[i].add = None if a is None else a.data_ptr()
        return L.q4rdna_mul_mat_group(arr, 2, x.data_ptr(), cols, None, torch.cuda.current_stream().cuda_stream)

    assert run(buf[0:256], buf[128:384], None) == q4rdna.ERR_ARGUMENT          # outputs overlap
    assert "overlap" in q4rdna.last_error()
    assert run(buf[0:256], buf[512:768], buf[200:456]) == q4rdna.ERR_ARGUMENT  # y0 overlaps member 1's add
    torch.cuda.synchronize()
    assert (buf == 7.0).all()
    assert run(buf[0:256], buf[256:512], add) == q4rdna.OK
    torch.cuda.synchronize()
    assert torch.equal(buf[0:256], buf[256:512])


def test_valu_group_past_the_eight_wave_threshold(cuda):
    """Two gate-projection-shaped members at split 2 make 1,536 workgroups,
    more than four per CU, so the group runs four-wave workgroups while a
    single 12288 x 4096 launch at split 2 (768) runs eight: the outputs may
    differ from q4rdna_mul_mat_ex in the last bits, and both meet the bars."""
    rows, cols = 12288, 4096
    assert 2 * (2 * rows // 32) > 4 * torch.cuda.get_device_properties(0).multi_processor_count
    t1, w1 = weight(rows, cols, 780)
    t2, w2 = weight(rows, cols, 781)
    x_np = O.gaussian_x(cols, 782)
    x = torch.from_numpy(x_np).cuda()
    ys = [torch.full((rows,), float("nan"), device="cuda") for _ in range(2)]
    assert api.mul_mat_group([(w1, ys[0]), (w2, ys[1])], x, split_k=2)
    r = torch.full((rows,), float("nan"), device="cuda")
    assert api.mul_mat_ex(w1, x, r, split_k=2)
    torch.cuda.synchronize()
    for t, y in ((t1, ys[0]), (t2, ys[1])):
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, label="group of two")
    assert_gemv_parity(r.cpu().numpy(), t1, rows, cols, x_np, label="single")
