"""Small-batch decode at the Qwen3-8B projection shapes: N = 2, 4 and 8
activation vectors against one decoder layer's seven projections (q/o
4096 x 4096, k/v 1024 x 4096, gate/up 12288 x 4096, down 4096 x 12288),
N(0, 0.02) weights packed on the GPU with the sidecar search and N(0, 1)
activations, as the small-batch configuration states.

Through q4rdna_mul_mat_batch (one launch per weight, every tile read once
for all N vectors) at gate/up plain, gate/up as the SwiGLU site and down
with the residual add; and through batched plans: the same three sites, and
one whole layer (q, k, v, o + add, the gate/up SwiGLU site, down + add).
Every vector of every output meets both bars of tests/conftest.py: per row
1e-3 of max(|y64|, 0.01 rms) against the fp64 oracle, and relative L2
<= 1e-5 against the reference bench's sequential fp32 loop
(source/q4rdna_gemv_bench.hip:189-211, 259-261).
"""
import numpy as np
import pytest
import torch

import oracle as O
from q4rdna import api
from conftest import assert_gemv_parity

pytestmark = pytest.mark.gpu

# name -> (rows, cols, seed index within layer 0 of the stack's seed scheme)
LAYER = {"q": (4096, 4096, 0), "k": (1024, 4096, 1), "v": (1024, 4096, 2), "o": (4096, 4096, 3),
         "gate": (12288, 4096, 4), "up": (12288, 4096, 5), "down": (4096, 12288, 6)}


@pytest.fixture(scope="module")
def layer(cuda):
    """One decoder layer's seven projections packed on the GPU: name ->
    (QWeight, tiles on the host)."""
    out = {}
    gen = torch.Generator(device="cuda")
    for name, (rows, cols, i) in LAYER.items():
        gen.manual_seed(0x51EE0000 + i)
        w = torch.randn(rows, cols, generator=gen, device="cuda").mul_(0.02)
        tiles = api.pack(w)
        del w
        out[name] = (api.QWeight.from_tiles(tiles, rows, cols), tiles.cpu().numpy())
    torch.cuda.synchronize()
    return out


def xs_for(cols: int, n: int, seed: int) -> np.ndarray:
    return np.stack([O.gaussian_x(cols, seed + v) for v in range(n)])


def check_batch(y: torch.Tensor, tiles, rows, cols, xs, gate_tiles=None, add=None, label=""):
    yh = y.cpu().numpy().reshape(xs.shape[0], rows)
    for v in range(xs.shape[0]):
        assert_gemv_parity(yh[v], tiles, rows, cols, xs[v], gate_tiles=gate_tiles,
                           add=None if add is None else add[v], label=(label, v))


@pytest.mark.parametrize("n", [2, 4, 8])
def test_mul_mat_batch_at_the_ffn_sites(cuda, layer, n):
    """q4rdna_mul_mat_batch at gate/up 12288 x 4096 (plain and SwiGLU) and
    down 4096 x 12288 + add."""
    up, up_t = layer["up"]
    gate, gate_t = layer["gate"]
    down, down_t = layer["down"]
    x = xs_for(4096, n, 0x5B00 + n)
    xd = torch.from_numpy(x).cuda()
    y = torch.full((n, 12288), float("nan"), device="cuda")
    assert api.mul_mat_batch(up, xd, y)
    torch.cuda.synchronize()
    check_batch(y, up_t, 12288, 4096, x, label=("up", n))
    y.fill_(float("nan"))
    assert api.mul_mat_batch(up, xd, y, gate=gate)
    torch.cuda.synchronize()
    check_batch(y, up_t, 12288, 4096, x, gate_tiles=gate_t, label=("swiglu", n))
    xh = xs_for(12288, n, 0x5C00 + n)
    res = xs_for(4096, n, 0x5D00 + n)
    yd = torch.full((n, 4096), float("nan"), device="cuda")
    assert api.mul_mat_batch(down, torch.from_numpy(xh).cuda(), yd, add=torch.from_numpy(res).cuda())
    torch.cuda.synchronize()
    check_batch(yd, down_t, 4096, 12288, xh, add=res, label=("down + add", n))


@pytest.mark.parametrize("n", [2, 4, 8])
def test_batched_plan_at_the_ffn_sites(cuda, layer, n):
    """A batched plan of gate/up plain, the gate/up SwiGLU site and down +
    add, each with its own N activation vectors."""
    up, up_t = layer["up"]
    gate, gate_t = layer["gate"]
    down, down_t = layer["down"]
    x_up = xs_for(4096, n, 0x6B00 + n)
    x_glu = xs_for(4096, n, 0x6C00 + n)
    x_down = xs_for(12288, n, 0x6D00 + n)
    res = xs_for(4096, n, 0x6E00 + n)
    y_up = torch.full((n, 12288), float("nan"), device="cuda")
    y_glu = torch.full((n, 12288), float("nan"), device="cuda")
    y_down = torch.full((n, 4096), float("nan"), device="cuda")
    dev = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    plan = api.Plan([(up, dev(x_up), y_up), (up, dev(x_glu), y_glu, gate, None),
                     (down, dev(x_down), y_down, None, dev(res))], batch=n)
    assert plan.launch()
    torch.cuda.synchronize()
    check_batch(y_up, up_t, 12288, 4096, x_up, label=("plan up", n))
    check_batch(y_glu, up_t, 12288, 4096, x_glu, gate_tiles=gate_t, label=("plan swiglu", n))
    check_batch(y_down, down_t, 4096, 12288, x_down, add=res, label=("plan down + add", n))
    plan.close()


@pytest.mark.parametrize("n", [2, 4, 8])
def test_batched_plan_of_one_layer(cuda, layer, n):
    """One decoder layer's projections as one batched plan: q, k and v on the
    layer input, o + add (the residual), the gate/up SwiGLU site, down + add.
    Launched twice: the second launch repeats the first bit for bit."""
    dev = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    h = xs_for(4096, n, 0x7A00 + n)              # the layer input (q, k, v)
    attn = xs_for(4096, n, 0x7B00 + n)           # attention output (o)
    h2 = xs_for(4096, n, 0x7C00 + n)             # post-attention norm output (gate/up)
    act = xs_for(12288, n, 0x7D00 + n)           # SwiGLU output (down)
    res1 = xs_for(4096, n, 0x7E00 + n)
    res2 = xs_for(4096, n, 0x7F00 + n)
    ys = {name: torch.full((n, rows), float("nan"), device="cuda")
          for name, (rows, _, _) in LAYER.items() if name != "gate"}
    hd = dev(h)
    items = [(layer["q"][0], hd, ys["q"]), (layer["k"][0], hd, ys["k"]), (layer["v"][0], hd, ys["v"]),
             (layer["o"][0], dev(attn), ys["o"], None, dev(res1)),
             (layer["up"][0], dev(h2), ys["up"], layer["gate"][0], None),
             (layer["down"][0], dev(act), ys["down"], None, dev(res2))]
    plan = api.Plan(items, batch=n)
    assert plan.launch()
    torch.cuda.synchronize()
    first = {k: v.clone() for k, v in ys.items()}
    assert plan.launch()
    torch.cuda.synchronize()
    for k in ys:
        assert torch.equal(first[k], ys[k]), k
    for name, xs, add, gate in (("q", h, None, None), ("k", h, None, None), ("v", h, None, None),
                                ("o", attn, res1, None), ("up", h2, None, "gate"), ("down", act, res2, None)):
        rows, cols, _ = LAYER[name]
        check_batch(ys[name], layer[name][1], rows, cols, xs, add=add,
                    gate_tiles=layer[gate][1] if gate else None, label=("layer", name, n))
    plan.close()
