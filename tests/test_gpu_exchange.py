"""Split-K in the per-tensor VALU kernel: the K chunks of a row meet in a
binary tree of exchange slots (one slot at split 2) that every launch must
leave empty (all-zero memory; a partial is stored XOR a signaling-NaN key).
Launches of both slot layouts (one word per row; a (sum, SwiGLU gate sum)
pair per row) alternate on one stream over the same slots: every result is
bit-identical from round to round and within both parity bars, at split 2
and at every tree shape up to 64 chunks.  NaN partials, including the slots'
own signaling-NaN key fed in as an activation, still finish every row, and
the launches after them are unaffected."""
import numpy as np
import pytest
import torch

import oracle as O
from q4rdna import _lib, api
from conftest import assert_gemv_parity

pytestmark = pytest.mark.gpu

SLOT_KEY = 0x7FA5A5A5  # the kernel's slot key (a signaling NaN); a partial with these bits would store as zero


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


# rows, cols, gate, add: every site the policy runs at split 2
SITES = [
    (4096, 4096, False, False),
    (12288, 4096, True, False),
    (1024, 4096, False, True),
    (4096, 4096, True, True),
    (12288, 4096, False, False),
]


def test_split2_slot_layouts_alternate_on_one_stream(cuda):
    for rows, cols, _, _ in SITES:
        assert api.policy_split_k(rows, cols) == 2, (rows, cols)
    prepared = []
    for i, (rows, cols, with_gate, with_add) in enumerate(SITES):
        t, w = weight(rows, cols, 300 + i)
        gt, g = weight(rows, cols, 310 + i) if with_gate else (None, None)
        x_np = O.gaussian_x(cols, 320 + i)
        add_np = O.gaussian_x(rows, 330 + i) if with_add else None
        prepared.append((t, w, gt, g, x_np, torch.from_numpy(x_np).cuda(), add_np,
                         None if add_np is None else torch.from_numpy(add_np).cuda(), rows, cols))
    st = torch.cuda.Stream()
    first = None
    for rnd in range(3):
        outs = []
        with torch.cuda.stream(st):
            for t, w, gt, g, x_np, x, add_np, add, rows, cols in prepared:
                y = torch.full((rows,), 7.0, device="cuda")
                assert api.mul_mat_ex(w, x, y, gate=g, add=add, stream=st.cuda_stream)
                outs.append(y)
        st.synchronize()
        if first is None:
            first = outs
            for (t, w, gt, g, x_np, x, add_np, add, rows, cols), y in zip(prepared, outs):
                assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, gate_tiles=gt, add=add_np,
                                   label=(rows, cols, g is not None, add is not None))
        else:
            for a, b in zip(first, outs):
                assert torch.equal(a, b), rnd


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("chunk", [0, 1])
def test_split2_nan_partials_finish_every_row(cuda, gated, chunk):
    """An activation in chunk `chunk` set to the slot key's bit pattern makes
    that chunk's partial of every row NaN: every row still gets written (NaN),
    and a clean launch right after on the same stream is exact again."""
    rows, cols = 4096, 4096
    t, w = weight(rows, cols, 400)
    gt, g = weight(rows, cols, 401) if gated else (None, None)
    x_np = O.gaussian_x(cols, 402)
    bad = x_np.copy()
    bad.view(np.uint32)[chunk * (cols // 2) + 5] = SLOT_KEY
    st = torch.cuda.Stream()
    y_bad = torch.full((rows,), 7.0, device="cuda")
    y = torch.full((rows,), 7.0, device="cuda")
    with torch.cuda.stream(st):
        assert api.mul_mat_ex(w, torch.from_numpy(bad).cuda(), y_bad, gate=g, split_k=2, stream=st.cuda_stream)
        assert api.mul_mat_ex(w, torch.from_numpy(x_np).cuda(), y, gate=g, split_k=2, stream=st.cuda_stream)
    st.synchronize()
    assert torch.isnan(y_bad).all()
    assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, gate_tiles=gt, label=("after NaN", gated, chunk))


def test_split2_noalloc_shares_the_protocol(cuda):
    """The allocation-free entry point at split 2 (its own slots) after a NaN
    launch and between launches of the stream workspace: equal bit for bit."""
    import ctypes
    import q4rdna
    L = q4rdna.load()
    rows, cols = 12288, 4096
    t, w = weight(rows, cols, 500)
    gt, g = weight(rows, cols, 501)
    x = torch.from_numpy(O.gaussian_x(cols, 502)).cuda()
    bad = x.clone()
    bad[17] = float("nan")
    opts = _lib.LaunchOptions()
    opts.split_k = 2
    s = torch.cuda.current_stream().cuda_stream

    def na(xx, yy, gate):
        return L.q4rdna_mul_mat_ex_noalloc(ctypes.byref(w.raw), ctypes.byref(gate.raw) if gate else None,
                                           xx.data_ptr(), None, yy.data_ptr(), ctypes.byref(opts), s)

    for gate in (None, g):
        y_ref = torch.empty(rows, device="cuda")
        y_bad = torch.full((rows,), 7.0, device="cuda")
        y_na = torch.empty(rows, device="cuda")
        assert api.mul_mat_ex(w, x, y_ref, gate=gate, split_k=2)
        assert na(bad, y_bad, gate) == q4rdna.OK, q4rdna.last_error()
        assert na(x, y_na, gate) == q4rdna.OK, q4rdna.last_error()
        torch.cuda.synchronize()
        assert torch.isnan(y_bad).all()
        assert torch.equal(y_na, y_ref)


@pytest.mark.parametrize("rows,cols", [(32, 128), (96, 192), (64, 4096), (160, 28672)])
@pytest.mark.parametrize("kind", ["plain", "add", "glu", "glu+add"])
def test_split2_edge_shapes(cuda, rows, cols, kind):
    """Split 2 at the smallest shapes (one row tile; one group per chunk; an
    odd group count) and a long K, with every epilogue: both parity bars."""
    t, w = weight(rows, cols, rows + cols)
    gt, g = weight(rows, cols, rows + cols + 1) if "glu" in kind else (None, None)
    add_np = O.gaussian_x(rows, rows + 2 * cols) if "add" in kind else None
    x_np = O.gaussian_x(cols, rows + 3 * cols)
    y = torch.full((rows,), 7.0, device="cuda")
    assert api.mul_mat_ex(w, torch.from_numpy(x_np).cuda(), y, gate=g,
                          add=None if add_np is None else torch.from_numpy(add_np).cuda(), split_k=2)
    torch.cuda.synchronize()
    assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, gate_tiles=gt, add=add_np, label=(rows, cols, kind))


def test_group_of_eight_mixed_rows(cuda):
    """The largest group (8 GEMVs of different row counts, some with a bias)
    on the VALU kernel at split 2: every output within both bars."""
    cols = 4096
    rows_list = [32, 64, 96, 1024, 4096, 128, 2048, 160]
    members = []
    for i, rows in enumerate(rows_list):
        t, w = weight(rows, cols, 600 + i)
        add_np = O.gaussian_x(rows, 610 + i) if i % 3 == 0 else None
        members.append((t, w, add_np, rows))
    x_np = O.gaussian_x(cols, 620)
    x = torch.from_numpy(x_np).cuda()
    ys = [torch.full((rows,), 7.0, device="cuda") for *_, rows in members]
    items = [(w, y, None, None if a is None else torch.from_numpy(a).cuda()) for (t, w, a, rows), y in zip(members, ys)]
    assert api.mul_mat_group(items, x, split_k=2)
    torch.cuda.synchronize()
    for (t, w, a, rows), y in zip(members, ys):
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, add=a, label=rows)


TREE_SPLITS = [3, 4, 5, 6, 7, 8, 9, 12, 16, 17, 31, 33, 64]


@pytest.mark.parametrize("split", TREE_SPLITS)
def test_exchange_tree_every_shape(cuda, split):
    """Splits above 2 meet in the exchange tree (leaves passed through where
    a subtree holds no chunk).  Plain and SwiGLU + bias launches alternate on
    one stream for three rounds: each round equals the first bit for bit (so
    every slot was left empty), and the first is within both bars."""
    rows, cols = 96, 4096
    cases = []
    for i, kind in enumerate(("plain", "glu+add")):
        t, w = weight(rows, cols, 700 + 10 * split + i)
        gt, g = weight(rows, cols, 701 + 10 * split + i) if "glu" in kind else (None, None)
        add_np = O.gaussian_x(rows, 702 + 10 * split + i) if "add" in kind else None
        x_np = O.gaussian_x(cols, 703 + 10 * split + i)
        cases.append((kind, t, w, gt, g, add_np, None if add_np is None else torch.from_numpy(add_np).cuda(),
                      x_np, torch.from_numpy(x_np).cuda()))
    st = torch.cuda.Stream()
    first = None
    for rnd in range(3):
        outs = []
        with torch.cuda.stream(st):
            for kind, t, w, gt, g, add_np, add, x_np, x in cases:
                y = torch.full((rows,), 7.0, device="cuda")
                assert api.mul_mat_ex(w, x, y, gate=g, add=add, split_k=split, stream=st.cuda_stream)
                outs.append(y)
        st.synchronize()
        if first is None:
            first = outs
            for (kind, t, w, gt, g, add_np, add, x_np, x), y in zip(cases, outs):
                assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, gate_tiles=gt, add=add_np,
                                   label=(split, kind))
        else:
            for a, b in zip(first, outs):
                assert torch.equal(a, b), (split, rnd)


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("chunk", [0, 3, 5])
def test_exchange_tree_nan_partials_finish_every_row(cuda, gated, chunk):
    """At split 6 (leaves 0..3 three exchanges deep, 4 and 5 two), the slot
    key's bits as an activation in chunk `chunk`: every row is still written
    (NaN), and a clean launch right after on the same stream is exact."""
    rows, cols, split = 4096, 12288, 6
    t, w = weight(rows, cols, 800)
    gt, g = weight(rows, cols, 801) if gated else (None, None)
    x_np = O.gaussian_x(cols, 802)
    bad = x_np.copy()
    bad.view(np.uint32)[chunk * (cols // split) + 9] = SLOT_KEY
    st = torch.cuda.Stream()
    y_bad = torch.full((rows,), 7.0, device="cuda")
    y = torch.full((rows,), 7.0, device="cuda")
    with torch.cuda.stream(st):
        assert api.mul_mat_ex(w, torch.from_numpy(bad).cuda(), y_bad, gate=g, split_k=split, stream=st.cuda_stream)
        assert api.mul_mat_ex(w, torch.from_numpy(x_np).cuda(), y, gate=g, split_k=split, stream=st.cuda_stream)
    st.synchronize()
    assert torch.isnan(y_bad).all()
    assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x_np, gate_tiles=gt, label=("after NaN", split, gated, chunk))
