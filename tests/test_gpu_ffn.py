"""q4rdna_mul_mat_ffn: the SwiGLU (up, gate) and down GEMVs of an FFN block in
one launch, down's workgroups waiting for the SwiGLU rows of their K chunk.

Each phase's arithmetic and chunk reduction are the per-tensor kernel's, so
mid and y must equal q4rdna_mul_mat_ex of the SwiGLU and of down (+ add) at
the same splits bit for bit (where those launches run eight-wave
workgroups), and meet both parity bars against the oracle.  Launches in a
row with new activations, graph replays and an in-place residual check that
the launch leaves its counters and slots clean."""
import numpy as np
import pytest
import torch

import oracle as O
from q4rdna import _lib, api
from conftest import assert_gemv_parity
from test_gpu_parity import dev_f32, dev_u8, random_tiles

pytestmark = pytest.mark.gpu


def ffn_splits(m: int, k: int, n: int) -> tuple[int, int]:
    """The splits the FFN launch runs: each phase's policy split, raised
    until every K chunk holds at most 64 groups."""
    ga, gm = k // 64, m // 64
    pa = max(1, min(api.policy_split_k(m, k), ga, 64))
    pb = max(1, min(api.policy_split_k(n, m), gm, 64))
    return min(max(pa, -(-ga // 64)), min(ga, 64)), min(max(pb, -(-gm // 64)), min(gm, 64))


def eight_waves(rows: int, split: int) -> bool:
    """Whether a per-tensor launch of `rows` at `split` (chunks of at most 64
    groups) runs eight-wave workgroups (at most four per CU)."""
    return rows // 32 * split <= 4 * torch.cuda.get_device_properties(0).multi_processor_count


class Ffn:
    def __init__(self, m: int, k: int, n: int, seed: int):
        self.m, self.k, self.n = m, k, n
        self.tu = random_tiles(m, k, seed)
        self.tg = random_tiles(m, k, seed + 1)
        self.td = random_tiles(n, m, seed + 2)
        self.up = api.QWeight.from_tiles(dev_u8(self.tu), m, k)
        self.gate = api.QWeight.from_tiles(dev_u8(self.tg), m, k)
        self.down = api.QWeight.from_tiles(dev_u8(self.td), n, m)

    def check(self, x_np, mid, y, add_np=None, label=""):
        """mid against the SwiGLU's bars; y against down's on the mid the
        launch actually produced."""
        mid_np = mid.cpu().numpy()
        assert_gemv_parity(mid_np, self.tu, self.m, self.k, x_np, gate_tiles=self.tg, label=("mid", label))
        assert_gemv_parity(y.cpu().numpy(), self.td, self.n, self.m, mid_np, add=add_np, label=("y", label))

    def per_tensor(self, x, add):
        """The same block as two per-tensor launches at the FFN's splits."""
        sa, sb = ffn_splits(self.m, self.k, self.n)
        mid = torch.full((self.m,), float("nan"), device="cuda")
        y = torch.full((self.n,), float("nan"), device="cuda")
        assert api.mul_mat_ex(self.up, x, mid, gate=self.gate, split_k=sa, kernel=_lib.KERNEL_VALU)
        assert api.mul_mat_ex(self.down, mid, y, add=add, split_k=sb, kernel=_lib.KERNEL_VALU)
        return mid, y


# (m, k, n): the Qwen3-8B FFN; a small block; uneven down chunks (33 groups
# of mid) after a SwiGLU split over 65 groups; a 128-group SwiGLU row (split
# raised to 2); a block whose down phase has one row tile.
SHAPES = [(12288, 4096, 4096), (1024, 512, 256), (2112, 4160, 96), (4096, 8192, 1024), (2048, 1024, 32)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("with_add", [False, True])
def test_ffn_equals_the_two_launches(cuda, shape, with_add):
    m, k, n = shape
    f = Ffn(m, k, n, 3100 + sum(shape) % 97)
    x_np = O.gaussian_x(k, 3200 + m % 89)
    add_np = O.gaussian_x(n, 3300) if with_add else None
    x = dev_f32(x_np)
    add = dev_f32(add_np) if with_add else None
    out = api.mul_mat_ffn(f.up, f.gate, f.down, x, add=add)
    assert out is not None
    y, mid = out
    torch.cuda.synchronize()
    f.check(x_np, mid, y, add_np, label=shape)
    sa, sb = ffn_splits(m, k, n)
    if eight_waves(m, sa) and eight_waves(n, sb):
        mid1, y1 = f.per_tensor(x, add)
        torch.cuda.synchronize()
        assert torch.equal(mid, mid1), (shape, sa)
        assert torch.equal(y, y1), (shape, sb)


def test_ffn_launches_in_a_row_and_in_place_residual(cuda):
    """Three launches with new activations each: a launch that left a
    chunk's count behind would let down read the previous launch's rows.
    The last one adds the residual in place (add is y)."""
    f = Ffn(12288, 4096, 4096, 3400)
    mid = torch.empty(f.m, device="cuda")
    y = torch.empty(f.n, device="cuda")
    for i in range(3):
        x_np = O.gaussian_x(f.k, 3500 + i)
        add_np = O.gaussian_x(f.n, 3600 + i)
        y.copy_(dev_f32(add_np))
        assert api.mul_mat_ffn(f.up, f.gate, f.down, dev_f32(x_np), add=y, mid=mid, y=y) is not None
        torch.cuda.synchronize()
        f.check(x_np, mid, y, add_np, label=i)


def test_ffn_replays_from_a_hip_graph(cuda):
    """The FFN launch captured into a HIP graph (its workspace allocated by an
    eager call first), replayed with new activations and eager launches in
    between: every replay equals the eager result bit for bit."""
    f = Ffn(12288, 4096, 4096, 3700)
    x = torch.empty(f.k, device="cuda")
    add = torch.empty(f.n, device="cuda")
    mid = torch.empty(f.m, device="cuda")
    y = torch.empty(f.n, device="cuda")
    s = torch.cuda.Stream()

    def work():
        assert api.mul_mat_ffn(f.up, f.gate, f.down, x, add=add, mid=mid, y=y, stream=s.cuda_stream) is not None

    with torch.cuda.stream(s):
        x.normal_()
        add.normal_()
        work()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        work()
    for rep in range(3):
        with torch.cuda.stream(s):
            x.normal_()
            add.normal_()
            work()
        s.synchronize()
        want_mid, want_y = mid.clone(), y.clone()
        mid.fill_(float("nan"))
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(mid, want_mid), rep
        assert torch.equal(y, want_y), rep
    f.check(x.cpu().numpy(), mid, y, add.cpu().numpy(), label="replay")


def test_ffn_refuses_what_does_not_fit(cuda):
    """Mismatched shapes are not applicable (nothing launched); overlapping
    buffers are argument errors."""
    f = Ffn(1024, 512, 256, 3800)
    x = torch.randn(512, device="cuda")
    other_down = api.QWeight.from_tiles(dev_u8(random_tiles(256, 2048, 3801)), 256, 2048)
    assert api.mul_mat_ffn(f.up, f.gate, other_down, x) is None           # down's K is not up's rows
    assert api.mul_mat_ffn(f.up, f.gate, f.down, torch.randn(1024, device="cuda")) is None   # x_ne0 != K
    assert api.mul_mat_ffn(f.up, f.gate, f.down, x, y=torch.empty(128, device="cuda")) is None  # y_ne0 != N
    buf = torch.zeros(1024 + 256, device="cuda")
    assert api.mul_mat_ffn(f.up, f.gate, f.down, buf[768:], mid=torch.empty(1024, device="cuda")) is not None
    with pytest.raises(_lib.Q4RdnaError):  # mid's last 256 floats are x's first
        api.mul_mat_ffn(f.up, f.gate, f.down, buf[768:], mid=buf[:1024])
    with pytest.raises(_lib.Q4RdnaError):  # y overlaps add without being it
        api.mul_mat_ffn(f.up, f.gate, f.down, x, add=buf[:256], y=buf[128:384])
    torch.cuda.synchronize()
