"""GPU parity at the bench's own scale, through the C ABI: the lm_head shape
(151936 x 4096) through the per-tensor kernel and a plan, the full Qwen3-8B
36-layer stack as the 252-GEMV plan and as the 216-GEMV SwiGLU-fused plan
at their real item deal (512 workgroups, two per CU), plans of more
items than workgroups with every item kind, single-vector and batched, and
one decoder layer at an 8-way tensor-parallel GPU's shard shapes.

Bars (tests/conftest.py): per row 1e-3 of max(|y64|, 0.01 rms) against the
fp64 oracle, and relative L2 <= 1e-5 against the reference bench's
sequential fp32 loop (source/q4rdna_gemv_bench.hip:189-211, 259-261).
"""
import numpy as np
import pytest
import torch

import oracle as O
import q4rdna
from q4rdna import api
from conftest import assert_gemv_parity

pytestmark = pytest.mark.gpu


def dev_u8(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def dev_f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def random_tiles(rows: int, cols: int, seed: int, subnormal: bool = False) -> np.ndarray:
    """Uniform random code bytes and random fp16 scales of both signs."""
    rng = np.random.default_rng(seed)
    g = cols // 64
    t = rng.integers(0, 256, (rows // 32, g, 1088), dtype=np.uint8)
    mag = rng.uniform(1e-3, 3e-2, (rows // 32, g, 32))
    if subnormal:
        mag[..., ::7] = rng.uniform(1e-7, 6e-5, mag[..., ::7].shape)
    s = (mag * rng.choice([-1.0, 1.0], mag.shape)).astype(np.float16)
    t[:, :, :64] = s.view(np.uint8).reshape(rows // 32, g, 64)
    return t.reshape(-1)


# ----------------------------------------------------------------- lm_head

LM_ROWS, LM_COLS = 151936, 4096


@pytest.fixture(scope="module")
def lm_head():
    up = random_tiles(LM_ROWS, LM_COLS, 0x1A0, subnormal=True)
    gate = random_tiles(LM_ROWS, LM_COLS, 0x1A1)
    x = O.gaussian_x(LM_COLS, 0x1A2)
    add = O.gaussian_x(LM_ROWS, 0x1A3)
    return up, gate, x, add


@pytest.mark.parametrize("kind", ["plain", "add", "glu"])
def test_lm_head_per_tensor(cuda, lm_head, kind):
    """151936 x 4096 at batch 1 through the per-tensor entry points: the
    shape policy gives split 1 (4,748 workgroups, more than four per CU), so
    the launch runs four-wave workgroups of 16 tiles per wave."""
    up_t, gate_t, x, add = lm_head
    assert api.policy_split_k(LM_ROWS, LM_COLS) == 1
    assert LM_ROWS // 32 > 4 * torch.cuda.get_device_properties(0).multi_processor_count
    up = api.QWeight.from_tiles(dev_u8(up_t), LM_ROWS, LM_COLS)
    xd = dev_f32(x)
    y = torch.full((LM_ROWS,), float("nan"), device="cuda")
    if kind == "plain":
        assert api.mul_mat(up, xd, y) is not None
        assert_gemv_parity(y.cpu().numpy(), up_t, LM_ROWS, LM_COLS, x, label="lm_head")
    elif kind == "add":
        assert api.mul_mat_add(up, xd, dev_f32(add), y) is not None
        assert_gemv_parity(y.cpu().numpy(), up_t, LM_ROWS, LM_COLS, x, add=add, label="lm_head + add")
    else:
        gate = api.QWeight.from_tiles(dev_u8(gate_t), LM_ROWS, LM_COLS)
        assert api.mul_mat_glu(up, gate, xd, y) is not None
        assert_gemv_parity(y.cpu().numpy(), up_t, LM_ROWS, LM_COLS, x, gate_tiles=gate_t, label="lm_head swiglu")


def test_lm_head_plan(cuda, lm_head):
    """lm_head through a plan (pair items, the MFMA sweep), next to a q
    projection so two GEMVs share the deal."""
    up_t, _, x, _ = lm_head
    q_t = random_tiles(4096, 4096, 0x1A4)
    xq = O.gaussian_x(4096, 0x1A5)
    up = api.QWeight.from_tiles(dev_u8(up_t), LM_ROWS, LM_COLS)
    q = api.QWeight.from_tiles(dev_u8(q_t), 4096, 4096)
    y = torch.full((LM_ROWS,), float("nan"), device="cuda")
    yq = torch.full((4096,), float("nan"), device="cuda")
    plan = api.Plan([(up, dev_f32(x), y), (q, dev_f32(xq), yq)])
    assert plan.launch()
    torch.cuda.synchronize()
    assert_gemv_parity(y.cpu().numpy(), up_t, LM_ROWS, LM_COLS, x, label="lm_head plan")
    assert_gemv_parity(yq.cpu().numpy(), q_t, 4096, 4096, xq, label="q next to lm_head")
    plan.close()


# ----------------------------------------------------------------- the 36-layer stack

@pytest.fixture(scope="module")
def stack(cuda):
    """The Qwen3-8B 36-layer stack as the bench builds it: N(0, 0.02)
    weights packed on the GPU in layer order, N(0, 1) x per tensor."""
    from q4rdna.sidecar import layout, qwen3_8b_stack
    names = qwen3_8b_stack(36)
    data_offset, entries, end = layout(names)
    data = torch.empty(end - data_offset, dtype=torch.uint8, device="cuda")
    gen = torch.Generator(device="cuda")
    tensors = []
    for i, (name, rows, cols, off, size) in enumerate(entries):
        gen.manual_seed(0x51EE0000 + i)
        w = torch.randn(rows, cols, generator=gen, device="cuda").mul_(0.02)
        view = data[off - data_offset: off - data_offset + size]
        api.pack(w, out=view)
        del w
        gen.manual_seed(0x51EE8000 + i)
        x = torch.randn(cols, generator=gen, device="cuda")
        tensors.append(dict(name=name, rows=rows, cols=cols, w=api.QWeight.from_tiles(view, rows, cols), x=x))
    torch.cuda.synchronize()
    yield tensors
    del data


CHECK_LAYERS = (0, 17, 35)


def test_full_stack_252_gemv_plan(cuda, stack):
    """The bench's plan: 252 GEMVs, 12,096 items dealt to two workgroups per
    CU; every projection of the first, a middle and the last layer against
    both bars, and a second launch bit-identical to the first."""
    ys = [torch.full((t["rows"],), float("nan"), device="cuda") for t in stack]
    plan = api.Plan([(t["w"], t["x"], y) for t, y in zip(stack, ys)])
    assert plan.workgroups == 2 * torch.cuda.get_device_properties(0).multi_processor_count
    assert plan.launch()
    torch.cuda.synchronize()
    first = [y.clone() for y in ys]
    assert plan.launch()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(first, ys))
    assert not any(torch.isnan(y).any().item() for y in ys)
    for layer in CHECK_LAYERS:
        for j in range(7):
            t = stack[7 * layer + j]
            assert_gemv_parity(ys[7 * layer + j].cpu().numpy(), t["w"].tiles.cpu().numpy(), t["rows"], t["cols"],
                               t["x"].cpu().numpy(), label=t["name"])
    plan.close()


def test_full_stack_216_swiglu_plan(cuda, stack):
    """The reference's fused dispatch over the same bytes: per layer q, k, v,
    o, one SwiGLU GEMV for up with the gate, and down (216 GEMVs); the
    SwiGLU GEMVs stream both weights in one item per block."""
    by = {t["name"]: t for t in stack}
    items, checks = [], []
    for t in stack:
        if t["name"].endswith("ffn_gate.weight"):
            continue
        y = torch.full((t["rows"],), float("nan"), device="cuda")
        if t["name"].endswith("ffn_up.weight"):
            g = by[t["name"].replace("ffn_up", "ffn_gate")]
            items.append((t["w"], t["x"], y, g["w"]))
            checks.append((t, g, y))
        else:
            items.append((t["w"], t["x"], y))
            checks.append((t, None, y))
    assert len(items) == 216
    plan = api.Plan(items)
    assert plan.workgroups == 2 * torch.cuda.get_device_properties(0).multi_processor_count
    assert plan.launch()
    torch.cuda.synchronize()
    for layer in CHECK_LAYERS:
        for j in range(6):
            t, g, y = checks[6 * layer + j]
            assert_gemv_parity(y.cpu().numpy(), t["w"].tiles.cpu().numpy(), t["rows"], t["cols"], t["x"].cpu().numpy(),
                               gate_tiles=None if g is None else g["w"].tiles.cpu().numpy(), label=t["name"])
    plan.close()


def rms_norm(x: torch.Tensor, out: torch.Tensor) -> None:
    """A decoder's RMS normalization without a weight (eps 1e-6), written
    into a fixed buffer; it keeps the chain's activations O(1)."""
    out.copy_(torch.nn.functional.rms_norm(x, (x.numel(),), eps=1e-6))


@pytest.mark.parametrize("dispatch", ["reference", "grouped"])
def test_decoder_layer_chain(cuda, stack, dispatch):
    """The stack as a decoder runs it, every layer's input the previous
    layer's output: x_l normalized (RMS) feeds q, k and v; o on q's output
    plus the residual x_l gives h; h normalized feeds the gate/up SwiGLU
    site; down on that plus the residual h gives x_{l+1}.  (Without the
    normalizations the N(0, 0.02) weights grow the activations
    quadratically through SwiGLU and they overflow within five layers.)
    "reference" is the reference's per-tensor dispatch (six launches per
    layer, source/q4rdna.cu:713-793 from the hooks of
    llama-cpp-q4rdna-integration.patch); "grouped" runs q/k/v as one
    shared-x group (four launches).  All 36 layers run eagerly on one
    stream, then are captured into one HIP graph and replayed: every output
    of the replays equals the eager run bit for bit, and every launch of
    layers 0, 17 and 35 meets both bars on the inputs it read."""
    by = {t["name"]: t for t in stack}
    layers = len(stack) // 7
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x51EEC000)
    x0 = torch.randn(4096, generator=gen, device="cuda")
    bufs = [dict(xn=torch.empty(4096, device="cuda"), q=torch.empty(4096, device="cuda"),
                 k=torch.empty(1024, device="cuda"), v=torch.empty(1024, device="cuda"),
                 h=torch.empty(4096, device="cuda"), hn=torch.empty(4096, device="cuda"),
                 act=torch.empty(12288, device="cuda"), out=torch.empty(4096, device="cuda")) for _ in range(layers)]

    def w(l, part):
        return by[f"blk.{l}.{part}.weight"]["w"]

    def run(stream):
        for l in range(layers):
            b = bufs[l]
            x = x0 if l == 0 else bufs[l - 1]["out"]
            rms_norm(x, b["xn"])
            if dispatch == "reference":
                assert api.mul_mat(w(l, "attn_q"), b["xn"], b["q"], stream=stream) is not None
                assert api.mul_mat(w(l, "attn_k"), b["xn"], b["k"], stream=stream) is not None
                assert api.mul_mat(w(l, "attn_v"), b["xn"], b["v"], stream=stream) is not None
            else:
                assert api.mul_mat_group([(w(l, "attn_q"), b["q"]), (w(l, "attn_k"), b["k"]),
                                          (w(l, "attn_v"), b["v"])], b["xn"], stream=stream)
            assert api.mul_mat_add(w(l, "attn_output"), b["q"], x, b["h"], stream=stream) is not None
            rms_norm(b["h"], b["hn"])
            assert api.mul_mat_glu(w(l, "ffn_up"), w(l, "ffn_gate"), b["hn"], b["act"], stream=stream) is not None
            assert api.mul_mat_add(w(l, "ffn_down"), b["act"], b["h"], b["out"], stream=stream) is not None

    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        run(st.cuda_stream)
    torch.cuda.synchronize()
    eager = [{k: v.clone() for k, v in b.items()} for b in bufs]
    assert all(torch.isfinite(v).all() for b in eager for v in b.values())
    for l in CHECK_LAYERS:
        b = {k: v.cpu().numpy() for k, v in eager[l].items()}
        x = (x0 if l == 0 else eager[l - 1]["out"]).cpu().numpy()

        def tiles(part):
            return by[f"blk.{l}.{part}.weight"]["w"].tiles.cpu().numpy()

        for part, rows in (("attn_q", 4096), ("attn_k", 1024), ("attn_v", 1024)):
            assert_gemv_parity(b[part[-1]], tiles(part), rows, 4096, b["xn"], label=(dispatch, l, part))
        assert_gemv_parity(b["h"], tiles("attn_output"), 4096, 4096, b["q"], add=x, label=(dispatch, l, "o + add"))
        assert_gemv_parity(b["act"], tiles("ffn_up"), 12288, 4096, b["hn"], gate_tiles=tiles("ffn_gate"),
                           label=(dispatch, l, "swiglu"))
        assert_gemv_parity(b["out"], tiles("ffn_down"), 4096, 12288, b["act"], add=b["h"],
                           label=(dispatch, l, "down + add"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        run(st.cuda_stream)
    for rep in range(2):
        for b in bufs:
            for v in b.values():
                v.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            graph.replay()
        st.synchronize()
        for l in range(layers):
            for k in bufs[l]:
                assert torch.equal(bufs[l][k], eager[l][k]), (dispatch, rep, l, k)


# ----------------------------------------------------------------- many items per workgroup

KINDS = {
    # rows, cols, gate, add: the item kinds of the single-vector sweep
    "pair": (128, 512, False, False),          # one pair item (two 64-row blocks, one K chunk)
    "pair_add": (256, 4096, False, True),      # two pair items with the add epilogue
    "glu_one_item": (192, 4096, True, False),  # SwiGLU, both weight streams in one item per block
    "split_k": (64, 12800, False, False),      # two chunks meeting in the arrival chain
    "split_k_glu": (64, 12800, True, True),    # two chunks x two streams, add then SwiGLU
    "tail": (96, 4736, False, False),          # 74 groups: full steps and a short tail
}
COUNTS = {"pair": 600, "pair_add": 150, "glu_one_item": 150, "split_k": 150, "split_k_glu": 60, "tail": 60}


def make_gemvs(batch: int, seed: int):
    rng = np.random.default_rng(seed)
    order = [k for k, n in COUNTS.items() for _ in range(n)]
    rng.shuffle(order)
    gemvs = []
    for i, kind in enumerate(order):
        rows, cols, gate, add = KINDS[kind]
        t = random_tiles(rows, cols, seed * 1000 + i)
        gt = random_tiles(rows, cols, seed * 1000 + 500000 + i) if gate else None
        xs = np.stack([O.gaussian_x(cols, seed * 7 + 11 * i + v) for v in range(batch)])
        adds = np.stack([O.gaussian_x(rows, seed * 5 + 13 * i + v) for v in range(batch)]) if add else None
        gemvs.append(dict(kind=kind, rows=rows, cols=cols, t=t, gt=gt, xs=xs, adds=adds,
                          w=api.QWeight.from_tiles(dev_u8(t), rows, cols),
                          g=None if gt is None else api.QWeight.from_tiles(dev_u8(gt), rows, cols),
                          xd=dev_f32(xs if batch > 1 else xs[0]),
                          ad=None if adds is None else dev_f32(adds if batch > 1 else adds[0])))
    return gemvs


def run_plan(gemvs, batch: int):
    ys = [torch.full((batch, g["rows"]) if batch > 1 else (g["rows"],), float("nan"), device="cuda") for g in gemvs]
    plan = api.Plan([(g["w"], g["xd"], y, g["g"], g["ad"]) for g, y in zip(gemvs, ys)], batch=batch)
    assert plan.launch()
    torch.cuda.synchronize()
    wg = plan.workgroups
    plan.close()
    return ys, wg


def test_plan_with_many_items_per_workgroup(cuda):
    """1,170 GEMVs of every single-vector item kind, 2,010 items for 512
    workgroups, so workgroups run several items of mixed kinds in turn (the
    prefetch across item ends, alternating reduction buffers, pair, one-pass
    and both-stream items).  Every output against both bars, and each GEMV
    bit-identical to the same GEMV run alone in a plan of its own (one item
    per workgroup)."""
    gemvs = make_gemvs(1, 3)
    ys, wg = run_plan(gemvs, 1)
    items = sum({"pair": 1, "pair_add": 2, "glu_one_item": 3, "split_k": 2, "split_k_glu": 4, "tail": 2}[g["kind"]]
                for g in gemvs)
    assert items > 3 * wg
    for g, y in zip(gemvs, ys):
        assert_gemv_parity(y.cpu().numpy(), g["t"], g["rows"], g["cols"], g["xs"][0], gate_tiles=g["gt"],
                           add=None if g["adds"] is None else g["adds"][0], label=g["kind"])
    for i in range(0, len(gemvs), 23):
        alone, _ = run_plan([gemvs[i]], 1)
        assert torch.equal(alone[0], ys[i]), (i, gemvs[i]["kind"])


def test_batched_plan_with_many_items(cuda):
    """The batched sweep's queue with more items than workgroups (three
    vectors per GEMV): every vector of every GEMV against both bars."""
    gemvs = make_gemvs(3, 4)
    ys, wg = run_plan(gemvs, 3)
    assert len(gemvs) > wg
    for g, y in zip(gemvs, ys):
        yh = y.cpu().numpy()
        for v in range(3):
            assert_gemv_parity(yh[v], g["t"], g["rows"], g["cols"], g["xs"][v], gate_tiles=g["gt"],
                               add=None if g["adds"] is None else g["adds"][v], label=(g["kind"], v))


@pytest.mark.gpu
def test_tensor_parallel_shard_layer(cuda):
    """One decoder layer at an 8-way tensor-parallel GPU's shard shapes (the
    shapes bench.py --shards measures): q / k / v / gate / up split by rows
    (512, 128, 128, 1536, 1536 rows of K = 4096), o and down split along K
    (4096 x 512 with the residual add, 4096 x 1536 + add), gate/up as one
    SwiGLU GEMV.  Per-tensor launches and one plan, every output against
    both bars; the plan's outputs equal each other across two launches."""
    shapes = [("q", 512, 4096, None), ("k", 128, 4096, None), ("v", 128, 4096, None), ("o", 4096, 512, "add"),
              ("ffn", 1536, 4096, "glu"), ("down", 4096, 1536, "add")]
    items, checks = [], []
    for i, (name, rows, cols, kind) in enumerate(shapes):
        t = random_tiles(rows, cols, 2100 + i)
        x = O.gaussian_x(cols, 2200 + i)
        gt = add_np = None
        w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
        gate = add = None
        if kind == "glu":
            gt = random_tiles(rows, cols, 2300 + i)
            gate = api.QWeight.from_tiles(dev_u8(gt), rows, cols)
        if kind == "add":
            add_np = O.gaussian_x(rows, 2400 + i)
            add = dev_f32(add_np)
        xd = dev_f32(x)
        y1 = torch.full((rows,), float("nan"), device="cuda")
        assert api.mul_mat_ex(w, xd, y1, gate=gate, add=add)
        y = torch.full((rows,), float("nan"), device="cuda")
        items.append((w, xd, y, gate, add))
        checks.append((name, t, gt, x, add_np, rows, cols, y, y1))
    plan = api.Plan(items)
    assert plan.launch()
    torch.cuda.synchronize()
    first = [c[7].clone() for c in checks]
    assert plan.launch()
    torch.cuda.synchronize()
    for (name, t, gt, x, add_np, rows, cols, y, y1), f in zip(checks, first):
        assert torch.equal(y, f), name
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, gate_tiles=gt, add=add_np, label=("plan", name))
        assert_gemv_parity(y1.cpu().numpy(), t, rows, cols, x, gate_tiles=gt, add=add_np, label=("per tensor", name))
    plan.close()
