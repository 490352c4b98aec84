"""GPU parity of the gfx950 kernels against the CPU oracle, through the C ABI.

Bars: dequant and packing bit-exact; GEMV within the gate
|y - y64| <= 1e-3 * max(|y64|, 0.01 * rms(y64)) per row against the fp64
oracle (fp32 accumulation), plus the reference bench's own gate, relative L2
<= 1e-5 against the sequential fp32 oracle (source/q4rdna_gemv_bench.hip:259).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
import q4rdna
from q4rdna import _lib, api
from conftest import GATE_TOL, REL_L2_TOL, assert_gemv_parity, bf16_to_f32

pytestmark = pytest.mark.gpu

ALGOS = [(q4rdna.ALGO_SIDECAR, "sidecar"), (q4rdna.ALGO_ABSMAX, "absmax"), (q4rdna.ALGO_RANGE, "range"),
         (q4rdna.ALGO_MSE, "mse")]


def dev_u8(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def dev_f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def random_tiles(rows: int, cols: int, seed: int, subnormal: bool = False) -> np.ndarray:
    """Uniform random code bytes and random fp16 scales (both signs)."""
    rng = np.random.default_rng(seed)
    g = cols // 64
    t = rng.integers(0, 256, (rows // 32, g, 1088), dtype=np.uint8)
    mag = rng.uniform(1e-3, 3e-2, (rows // 32, g, 32))
    if subnormal:
        mag[..., ::7] = rng.uniform(1e-7, 6e-5, mag[..., ::7].shape)
    s = (mag * rng.choice([-1.0, 1.0], mag.shape)).astype(np.float16)
    t[:, :, :64] = s.view(np.uint8).reshape(rows // 32, g, 64)
    return t.reshape(-1)


def check_gemv(y: torch.Tensor, tiles: np.ndarray, rows: int, cols: int, x: np.ndarray, label=""):
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    y64, a64 = O.gemv_f64(tiles, rows, cols, x)
    err = O.gemv_errors(yh, y64, a64)
    assert err["gate"] <= GATE_TOL, (label, err)
    yseq = O.gemv_seq_f32(tiles, rows, cols, x)
    assert O.rel_l2(yh, yseq) <= REL_L2_TOL, (label, O.rel_l2(yh, yseq))
    return err


# ----------------------------------------------------------------- dequant

def test_dequant_bit_exact_every_fp16_scale(cuda):
    from test_oracle import all_scales_tiles
    tiles, rows, cols = all_scales_tiles()
    w = api.QWeight.from_tiles(dev_u8(tiles), rows, cols)
    got = api.dequantize(w).cpu().numpy()
    want = O.dequant(tiles, rows, cols)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("case", ["edge", "small", "outlier"])
@pytest.mark.parametrize("name", ["sidecar", "absmax", "range", "mse"])
def test_dequant_of_reference_packed_tiles(cuda, golden, case, name):
    tiles = golden[f"{case}_{name}"]
    rows, cols = golden[f"{case}_bf16"].shape
    got = api.dequantize(api.QWeight.from_tiles(dev_u8(tiles), rows, cols)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), O.dequant(tiles, rows, cols).view(np.uint32))
    # Identical to the CPU experiment's own dequantized values wherever the
    # stored scale is a normal fp16 number (it halves subnormal scales).
    ref_cpu = O.dequant(tiles, rows, cols, ref_cpu_decode=True)
    t = tiles.reshape(rows // 32, cols // 64, 1088)[:, :, :64].copy().view(np.uint16)
    normal = ((t & 0x7C00) != 0) | ((t & 0x3FF) == 0)                  # [rt, g, lane]
    mask = np.repeat(normal.transpose(0, 2, 1).reshape(rows, cols // 64), 64, axis=1)
    assert np.array_equal(got[mask].view(np.uint32), ref_cpu[mask].view(np.uint32))


# ----------------------------------------------------------------- packing

@pytest.mark.parametrize("case", ["edge", "small", "outlier"])
@pytest.mark.parametrize("algo,name", ALGOS)
def test_gpu_pack_matches_reference_golden(cuda, golden, case, algo, name):
    w = dev_f32(bf16_to_f32(golden[f"{case}_bf16"]))
    got = api.pack(w, algo).cpu().numpy()
    assert np.array_equal(got, golden[f"{case}_{name}"])


@pytest.mark.parametrize("algo,name", ALGOS)
def test_gpu_pack_matches_oracle_fp32_inputs(cuda, algo, name):
    rows, cols = 256, 2048
    w = O.gaussian_weights(rows, cols, 77 + algo)
    w.reshape(-1, 64)[::97] *= 20
    w.reshape(-1, 64)[5::211] *= 1e-4
    got = api.pack(dev_f32(w), algo).cpu().numpy()
    assert np.array_equal(got, O.pack(w, algo))


# ----------------------------------------------------------------- GEMV

SHAPES = [(32, 64), (64, 512), (96, 1024), (1024, 4096), (4096, 4096), (12288, 4096), (4096, 12288)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_gemv_matches_oracle(cuda, rows, cols):
    tiles = random_tiles(rows, cols, rows + cols, subnormal=True)
    x = O.gaussian_x(cols, rows * 7 + cols)
    w = api.QWeight.from_tiles(dev_u8(tiles), rows, cols)
    y = api.mul_mat(w, dev_f32(x))
    assert y is not None
    check_gemv(y, tiles, rows, cols, x, f"{rows}x{cols}")


def test_gemv_packed_gaussian_weights(cuda):
    rows, cols = 4096, 4096
    wf = O.gaussian_weights(rows, cols, 0x51EE0000)
    tiles_dev = api.pack(dev_f32(wf))
    tiles = tiles_dev.cpu().numpy()
    # the GPU packer output equals the oracle's on a sample of row tiles
    sample = O.pack(wf[:128], q4rdna.ALGO_SIDECAR)
    assert np.array_equal(tiles[: sample.size], sample)
    x = O.gaussian_x(cols, 0x51EE8000)
    y = api.mul_mat(api.QWeight.from_tiles(tiles_dev, rows, cols), dev_f32(x))
    check_gemv(y, tiles, rows, cols, x, "gaussian 4096x4096")


@pytest.mark.parametrize("rows,cols", [(4096, 12288), (2048, 28672)])
def test_split_k_sweep_with_outlier_groups(cuda, rows, cols):
    wf = O.gaussian_weights(rows, cols, rows ^ cols)
    g = wf.reshape(-1, 64)
    g[np.random.default_rng(1).permutation(g.shape[0])[: g.shape[0] // 100]] *= 20
    tiles_dev = api.pack(dev_f32(wf))
    tiles = tiles_dev.cpu().numpy()
    w = api.QWeight.from_tiles(tiles_dev, rows, cols)
    x = O.gaussian_x(cols, 5)
    xd = dev_f32(x)
    y64, a64 = O.gemv_f64(tiles, rows, cols, x)
    yseq = O.gemv_seq_f32(tiles, rows, cols, x)
    for split in (1, 2, 3, 4, 5, 8, 12, 16, 24, 32):
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        assert api.mul_mat_ex(w, xd, y, split_k=split)
        torch.cuda.synchronize()
        yh = y.cpu().numpy()
        assert O.gemv_errors(yh, y64, a64)["gate"] <= GATE_TOL, split
        assert O.rel_l2(yh, yseq) <= REL_L2_TOL, split


def test_gemv_is_deterministic(cuda):
    rows, cols = 1024, 4096
    tiles = random_tiles(rows, cols, 3)
    w = api.QWeight.from_tiles(dev_u8(tiles), rows, cols)
    xd = dev_f32(O.gaussian_x(cols, 4))
    ys = [api.mul_mat(w, xd).cpu().numpy() for _ in range(5)]
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32))


def test_mul_mat_add(cuda):
    rows, cols = 4096, 4096
    tiles = random_tiles(rows, cols, 11)
    x = O.gaussian_x(cols, 12)
    add = O.gaussian_x(rows, 13)
    w = api.QWeight.from_tiles(dev_u8(tiles), rows, cols)
    y = api.mul_mat_add(w, dev_f32(x), dev_f32(add))
    torch.cuda.synchronize()
    assert_gemv_parity(y.cpu().numpy(), tiles, rows, cols, x, add=add, label="mul_mat_add")


@pytest.mark.parametrize("rows,cols", [(12288, 4096), (1024, 4096)])
def test_mul_mat_glu_swiglu(cuda, rows, cols):
    up_t = random_tiles(rows, cols, 21)
    gate_t = random_tiles(rows, cols, 22)
    x = O.gaussian_x(cols, 23)
    up = api.QWeight.from_tiles(dev_u8(up_t), rows, cols)
    gate = api.QWeight.from_tiles(dev_u8(gate_t), rows, cols)
    y = api.mul_mat_glu(up, gate, dev_f32(x))
    torch.cuda.synchronize()
    assert_gemv_parity(y.cpu().numpy(), up_t, rows, cols, x, gate_tiles=gate_t, label=("swiglu", rows, cols))


@pytest.mark.parametrize("kind", ["plain", "add", "glu", "glu+add"])
def test_every_kernel_path_matches_oracle(cuda, kind):
    """Each per-tensor kernel path: K chunks of at most 64 groups (4, 8, 16,
    32, 64, 43 and 48 groups: 1, 2, 4 and 8 tiles per wave of eight, every
    load issued before the first wait), chunks of 65 to 128 groups on the
    16-wave workgroup (65 and 80 groups: 6 tiles per wave, some waves' last
    tile a clamped duplicate; 96 at splits 1 and 2; 128: 8 tiles per wave)
    and longer chunks (192 groups: the pipelined loop), each with the plain,
    add, SwiGLU and SwiGLU-after-add epilogues, against both parity bars."""
    rows = 96
    for cols, splits in [(4096, (16, 8, 4, 2, 1)), (8192, (1, 3)), (6144, (1, 2)), (4160, (1,)), (5120, (1,)),
                         (12288, (2, 1))]:
        up_t = random_tiles(rows, cols, 31 + cols)
        x = O.gaussian_x(cols, 32 + cols)
        up = api.QWeight.from_tiles(dev_u8(up_t), rows, cols)
        gate = add = gate_t = add_np = None
        if "add" in kind:
            add_np = O.gaussian_x(rows, 33 + cols)
            add = dev_f32(add_np)
        if "glu" in kind:
            gate_t = random_tiles(rows, cols, 34 + cols)
            gate = api.QWeight.from_tiles(dev_u8(gate_t), rows, cols)
        for split in splits:
            y = torch.full((rows,), float("nan"), device="cuda")
            assert api.mul_mat_ex(up, dev_f32(x), y, gate=gate, add=add, split_k=split)
            torch.cuda.synchronize()
            assert_gemv_parity(y.cpu().numpy(), up_t, rows, cols, x, gate_tiles=gate_t, add=add_np,
                               label=(kind, cols, split))


@pytest.mark.parametrize("n", [2, 3, 4, 5, 8])
def test_mul_mat_batch_matches_oracle(cuda, n):
    """q4rdna_mul_mat_batch: every vector against both parity bars, on short
    and long K (28672 columns: 448 groups in 16- or 32-group chunks), odd
    row-tile counts, with the add, SwiGLU and SwiGLU-after-add epilogues."""
    cases = [(96, 1024, "plain"), (4096, 4096, "add"), (1024, 12288, "glu"), (256, 28672, "glu+add"),
             (160, 4096, "plain")]
    for rows, cols, kind in cases:
        up_t = random_tiles(rows, cols, 41 + rows + n)
        xs = np.stack([O.gaussian_x(cols, 42 + cols + 7 * v) for v in range(n)])
        up = api.QWeight.from_tiles(dev_u8(up_t), rows, cols)
        gate = add = gate_t = add_np = None
        if "add" in kind:
            add_np = np.stack([O.gaussian_x(rows, 43 + rows + v) for v in range(n)])
            add = dev_f32(add_np)
        if "glu" in kind:
            gate_t = random_tiles(rows, cols, 44 + rows + n)
            gate = api.QWeight.from_tiles(dev_u8(gate_t), rows, cols)
        y = torch.full((n, rows), float("nan"), device="cuda")
        assert api.mul_mat_batch(up, dev_f32(xs), y, gate=gate, add=add)
        torch.cuda.synchronize()
        yh = y.cpu().numpy()
        for v in range(n):
            assert_gemv_parity(yh[v], up_t, rows, cols, xs[v], gate_tiles=gate_t,
                               add=None if add_np is None else add_np[v], label=(rows, cols, kind, n, v))


@pytest.mark.parametrize("n,split", [(2, 2), (4, 2), (8, 4), (3, 4), (3, 6), (5, 7)])
def test_mul_mat_batch_equals_single_vector_launches(cuda, n, split):
    """Each vector of a batched launch equals q4rdna_mul_mat_ex of that vector
    with the same split, bit for bit (same staging, fma order and summation
    order; both run eight-wave workgroups at this shape)."""
    rows, cols = 4096, 4096
    t = random_tiles(rows, cols, 51)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    gt = api.QWeight.from_tiles(dev_u8(random_tiles(rows, cols, 52)), rows, cols)
    xs = dev_f32(np.stack([O.gaussian_x(cols, 53 + v) for v in range(n)]))
    for gate in (None, gt):
        y = torch.empty((n, rows), device="cuda")
        assert api.mul_mat_batch(w, xs, y, gate=gate, split_k=split)
        for v in range(n):
            y1 = torch.empty(rows, device="cuda")
            assert api.mul_mat_ex(w, xs[v].contiguous(), y1, gate=gate, split_k=split)
            torch.cuda.synchronize()
            assert torch.equal(y[v], y1), (n, split, v, gate is not None)


def test_mul_mat_batch_long_rows_fall_back_per_vector(cuda):
    """Rows longer than 64 chunks of the n-vector kernel's stage (here 1025
    groups at n = 5: 16-group chunks would need 65) run one launch per
    vector, still against the oracle; n outside 1..8 is an argument error."""
    rows, cols, n = 32, 1025 * 64, 5
    t = random_tiles(rows, cols, 61)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    xs = np.stack([O.gaussian_x(cols, 62 + v) for v in range(n)])
    y = torch.full((n, rows), float("nan"), device="cuda")
    assert api.mul_mat_batch(w, dev_f32(xs), y)
    torch.cuda.synchronize()
    for v in range(n):
        check_gemv(y[v], t, rows, cols, xs[v], f"fallback vector {v}")
    lib = q4rdna.load()
    xd = dev_f32(xs)
    for bad in (0, 9):
        rc = lib.q4rdna_mul_mat_batch(ctypes.byref(w.raw), None, xd.data_ptr(), bad, None, y.data_ptr(), None,
                                      api._stream(xd.device))
        assert rc == q4rdna.ERR_ARGUMENT


def test_not_applicable_leaves_output_untouched(cuda):
    rows, cols = 64, 512
    w = api.QWeight.from_tiles(dev_u8(random_tiles(rows, cols, 1)), rows, cols)
    y = torch.full((rows + 32,), 7.0, device="cuda")
    assert api.mul_mat(w, dev_f32(np.ones(cols, np.float32)), y) is None
    x_short = dev_f32(np.ones(cols - 64, np.float32))
    y2 = torch.full((rows,), 7.0, device="cuda")
    assert api.mul_mat(w, x_short, y2) is None
    torch.cuda.synchronize()
    assert (y.cpu() == 7.0).all() and (y2.cpu() == 7.0).all()
    assert "shape mismatch" in q4rdna.last_error()


def test_overlapping_buffers_are_refused(cuda):
    """y overlapping x, and an add that overlaps y without being y, are
    argument errors that launch nothing (the kernels read x and add while
    other workgroups write y); so are a group's outputs that overlap each
    other or another descriptor's add.  add may be y itself, the in-place
    residual, per tensor and in a group."""
    rows, cols = 256, 512
    t = random_tiles(rows, cols, 31)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    buf = torch.full((cols + rows,), 7.0, device="cuda")
    with pytest.raises(_lib.Q4RdnaError):          # y's first rows are x's last columns
        api.mul_mat(w, buf[:cols], buf[cols - 16:cols - 16 + rows])
    y = torch.full((rows,), 7.0, device="cuda")
    add = torch.full((rows + 8,), 1.0, device="cuda")
    with pytest.raises(_lib.Q4RdnaError):          # add shifted by 8 rows against y
        api.mul_mat_add(w, dev_f32(O.gaussian_x(cols, 32)), add[8:], add[:rows])
    xb = torch.zeros(2, cols, device="cuda")
    with pytest.raises(_lib.Q4RdnaError):          # n vectors: y inside x's second vector
        api.mul_mat_batch(w, xb, xb.view(-1)[cols:cols + 2 * rows].view(2, rows))
    xg = dev_f32(O.gaussian_x(cols, 35))
    y2 = torch.full((rows,), 7.0, device="cuda")
    with pytest.raises(_lib.Q4RdnaError):          # group: a descriptor's add shifted against its own y
        api.mul_mat_group([(w, add[:rows], None, add[8:])], xg)
    with pytest.raises(_lib.Q4RdnaError):          # group: one descriptor's y is another's add
        api.mul_mat_group([(w, y, None, None), (w, y2, None, y)], xg)
    with pytest.raises(_lib.Q4RdnaError):          # group: two outputs overlap
        api.mul_mat_group([(w, add[:rows]), (w, add[8:])], xg)
    torch.cuda.synchronize()
    assert (buf.cpu() == 7.0).all() and (y.cpu() == 7.0).all() and (xb.cpu() == 0.0).all()
    assert (y2.cpu() == 7.0).all() and (add.cpu() == 1.0).all()
    x = O.gaussian_x(cols, 33)
    res = O.gaussian_x(rows, 34)
    y_in = dev_f32(res)                             # add is y: the residual in place
    assert api.mul_mat_add(w, dev_f32(x), y_in, y_in) is not None
    torch.cuda.synchronize()
    assert_gemv_parity(y_in.cpu().numpy(), t, rows, cols, x, add=res, label="in place")
    g_in = dev_f32(res)                             # the same in a group
    assert api.mul_mat_group([(w, g_in, None, g_in)], dev_f32(x))
    torch.cuda.synchronize()
    assert torch.equal(g_in, y_in)


# ----------------------------------------------------------------- sidecar

def test_sidecar_open_find_and_gemv(cuda, golden, tmp_path):
    img = golden["sidecar_image"].tobytes()
    path = tmp_path / "three.q4rdna"
    path.write_bytes(img)
    for sc in (api.Sidecar.open(str(path)), api.Sidecar.from_bytes(img)):
        ents = sc.entries()
        assert [e[0] for e in ents] == ["blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.ffn_down.weight"]
        for name, rows, cols, off, size in ents:
            w = sc.find(name, cols, rows)
            assert w is not None
            assert sc.find(name, rows + 32, cols) is None            # shape check (ne0 = cols)
            tiles = np.frombuffer(img[off:off + size], np.uint8)
            x = O.gaussian_x(cols, rows)
            y = api.mul_mat(w, dev_f32(x))
            check_gemv(y, tiles, rows, cols, x, name)
            y2 = api.mul_mat(api.QWeight.from_tiles(dev_u8(tiles), rows, cols), dev_f32(x))
            torch.cuda.synchronize()
            assert torch.equal(y, y2)
        assert sc.find("blk.9.attn_q.weight", 512, 64) is None
        sc.close()


# ----------------------------------------------------------------- multi-tensor plan

def test_plan_matches_oracle(cuda):
    # K chunks (up to 192 groups) of whole 16-group steps with and without a
    # short tail, tail-only chunks, several chunks (split-K) with a short
    # last one, odd row-tile counts, and the add / SwiGLU epilogues: SwiGLU
    # GEMVs of one chunk stream both weights in one item, longer ones meet
    # in the split-K chain (12800 and 28672 columns).
    shapes = [(128, 512, None), (32, 512, None), (32, 512, "add"), (128, 512, None), (384, 512, "glu"),
              (128, 1536, None), (4096, 4096, None), (1024, 4096, "add"), (96, 4736, None),
              (160, 8192, "glu"), (96, 12288, "add"), (32, 4096, "glu"), (224, 28672, None),
              (64, 12800, None), (96, 8320, "add"), (160, 4096, None), (224, 2048, "glu"),
              (64, 12800, "glu"), (32, 28672, "glu"), (96, 12288, "glu")]
    items, checks = [], []
    for i, (rows, cols, kind) in enumerate(shapes):
        t = random_tiles(rows, cols, 100 + i)
        x = O.gaussian_x(cols, 200 + i)
        w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
        y = torch.full((rows,), np.nan, device="cuda")
        gate = add = None
        gt = None
        if kind == "glu":
            gt = random_tiles(rows, cols, 300 + i)
            gate = api.QWeight.from_tiles(dev_u8(gt), rows, cols)
        if kind == "add":
            add_np = O.gaussian_x(rows, 400 + i)
            add = dev_f32(add_np)
        xd = dev_f32(x)
        items.append((w, xd, y, gate, add))
        checks.append((t, gt, x, add_np if kind == "add" else None, rows, cols, y))
    plan = api.Plan(items)
    assert plan.workgroups >= 1
    assert plan.launch()
    torch.cuda.synchronize()
    first = [c[-1].clone() for c in checks]
    for c in checks:
        c[-1].fill_(np.nan)
    assert plan.prepare() and plan.sweep()
    torch.cuda.synchronize()
    for f, c in zip(first, checks):  # the counters were left clean: a second sweep repeats the first
        assert torch.equal(f, c[-1])
    for t, gt, x, add_np, rows, cols, y in checks:
        assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x, gate_tiles=gt, add=add_np, label=(rows, cols))
    plan.close()


def wide_x(cols: int, seed: int) -> np.ndarray:
    """N(0, 1) activations with groups scaled by 1e4 and by 1e-4, and one
    all-zero group: block exponents far apart and a zero block."""
    x = O.gaussian_x(cols, seed)
    g = x.reshape(-1, 64)
    g[1::5] *= 1e4
    g[3::7] *= 1e-4
    g[2] = 0.0
    return x


@pytest.mark.parametrize("batch", [1, 3])
def test_plan_subnormal_scales_and_wide_activations(cuda, batch):
    """Plans (one vector and a batch of three) on tiles with subnormal fp16
    scales and activations whose groups span eight decades plus a zero group;
    a vector of zeros gives exact zeros."""
    rows, cols = 256, 4096
    t = random_tiles(rows, cols, 71, subnormal=True)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    xs = [wide_x(cols, 72 + v) for v in range(batch)]
    if batch > 1:
        xs[-1] = np.zeros(cols, np.float32)
    xd = dev_f32(np.stack(xs)) if batch > 1 else dev_f32(xs[0])
    y = torch.full((batch, rows) if batch > 1 else (rows,), float("nan"), device="cuda")
    plan = api.Plan([(w, xd, y)], batch=batch)
    assert plan.launch()
    torch.cuda.synchronize()
    yh = y.cpu().numpy().reshape(batch, rows)
    for v, x in enumerate(xs):
        if not x.any():
            assert (yh[v] == 0).all()
            continue
        assert_gemv_parity(yh[v], t, rows, cols, x, label=v)
    plan.close()


@pytest.mark.gpu
def test_plan_nonfinite_activation(cuda):
    """A NaN in x makes every row NaN, as in the fp32 reference.  An infinity
    makes every row non-finite (the reference gives +-inf or NaN per row
    depending on the weight it meets; the digit path gives NaN).  The other
    GEMVs of the plan are unaffected."""
    rows, cols = 64, 4096
    t = random_tiles(rows, cols, 7)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    xs = [O.gaussian_x(cols, 8 + i) for i in range(3)]
    xs[0][100] = np.nan
    xs[1][4000] = np.inf
    ys = [torch.zeros(rows, device="cuda") for _ in xs]
    plan = api.Plan([(w, dev_f32(x), y) for x, y in zip(xs, ys)])
    assert plan.launch()
    torch.cuda.synchronize()
    assert torch.isnan(ys[0]).all() and not torch.isfinite(ys[1]).any()
    assert_gemv_parity(ys[2].cpu().numpy(), t, rows, cols, xs[2])
    plan.close()


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [2, 3, 4, 5, 8])
def test_batched_plan_matches_oracle(cuda, batch):
    """Every vector of a batched plan against the fp64 oracle: short and
    full chunks, several chunks, odd row-tile counts, row counts that are not
    a multiple of 256, add and SwiGLU epilogues."""
    shapes = [(256, 4096, None), (96, 512, None), (1024, 4096, "add"), (160, 8192, "glu"),
              (4096, 4096, None), (288, 12288, "add"), (32, 4736, "glu"), (512, 1536, None),
              (64, 16384, "glu")]
    # SwiGLU rows of up to 12288 columns run up and gate in one item; the
    # 16384-column SwiGLU GEMV meets its chunks and streams in the partials.
    items, checks = [], []
    for i, (rows, cols, kind) in enumerate(shapes):
        t = random_tiles(rows, cols, 500 + 17 * batch + i)
        xs = np.stack([O.gaussian_x(cols, 600 + 31 * batch + 7 * i + v) for v in range(batch)])
        w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
        y = torch.full((batch, rows), np.nan, device="cuda")
        gate = add = None
        gt = add_np = None
        if kind == "glu":
            gt = random_tiles(rows, cols, 700 + i)
            gate = api.QWeight.from_tiles(dev_u8(gt), rows, cols)
        if kind == "add":
            add_np = np.stack([O.gaussian_x(rows, 800 + i + v) for v in range(batch)])
            add = dev_f32(add_np)
        items.append((w, dev_f32(xs), y, gate, add))
        checks.append((t, gt, xs, add_np, rows, cols, y))
    plan = api.Plan(items, batch=batch)
    for _ in range(2):
        assert plan.launch()
    torch.cuda.synchronize()
    for t, gt, xs, add_np, rows, cols, y in checks:
        yh = y.cpu().numpy()
        for v in range(batch):
            assert_gemv_parity(yh[v], t, rows, cols, xs[v], gate_tiles=gt,
                               add=None if add_np is None else add_np[v], label=(rows, cols, v))
    plan.close()


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 4])
def test_plan_result_is_independent_of_descriptor_order(cuda, batch):
    """The plan sweeps its GEMVs in an order of its own (longest K chunks
    first); a GEMV's arithmetic does not depend on that order, so the same
    descriptors given forwards and backwards give bit-identical outputs."""
    shapes = [(256, 4096, None), (64, 12288, "add"), (96, 512, "glu"), (128, 8320, None), (32, 28672, None)]
    descs = []
    for i, (rows, cols, kind) in enumerate(shapes):
        w = api.QWeight.from_tiles(dev_u8(random_tiles(rows, cols, 1200 + i)), rows, cols)
        gate = api.QWeight.from_tiles(dev_u8(random_tiles(rows, cols, 1300 + i)), rows, cols) if kind == "glu" else None
        add = dev_f32(np.stack([O.gaussian_x(rows, 1400 + i + v) for v in range(batch)])) if kind == "add" else None
        x = dev_f32(np.stack([O.gaussian_x(cols, 1500 + i + v) for v in range(batch)]))
        descs.append((w, x, gate, add, rows))
    outs = []
    for order in (list(range(len(descs))), list(reversed(range(len(descs))))):
        ys = [torch.full((batch, d[4]), np.nan, device="cuda") for d in descs]
        plan = api.Plan([(descs[i][0], descs[i][1], ys[i], descs[i][2], descs[i][3]) for i in order], batch=batch)
        assert plan.launch()
        torch.cuda.synchronize()
        plan.close()
        outs.append(ys)
    for a, b in zip(*outs):
        assert not torch.isnan(a).any()
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_batched_plan_rows_are_independent_of_batch(cuda):
    """A vector's result depends only on that vector: the batch-4 result of
    vector v equals the batch-8 result of the same vector bit for bit (both
    run the same digits and the same per-row summation order)."""
    rows, cols = 512, 4096
    t = random_tiles(rows, cols, 901)
    w = api.QWeight.from_tiles(dev_u8(t), rows, cols)
    xs = np.stack([O.gaussian_x(cols, 910 + v) for v in range(8)])
    y4 = torch.empty((4, rows), device="cuda")
    y8 = torch.empty((8, rows), device="cuda")
    p4 = api.Plan([(w, dev_f32(xs[:4]), y4)], batch=4)
    p8 = api.Plan([(w, dev_f32(xs), y8)], batch=8)
    assert p4.launch() and p8.launch()
    torch.cuda.synchronize()
    assert torch.equal(y4, y8[:4])
    p4.close()
    p8.close()


@pytest.mark.gpu
def test_plan_and_mul_mat_replay_from_a_hip_graph(cuda):
    """A plan launch, a per-tensor launch and a four-vector launch captured
    into one HIP graph (the plan allocates nothing per launch; the per-tensor
    workspace is allocated by an eager call first).  Replayed several times
    with new activations and eager work in between; every replay must equal
    the eager results bit for bit."""
    rows, cols = 1024, 4096
    tiles = [random_tiles(rows, cols, 1200 + i) for i in range(3)]
    ws = [api.QWeight.from_tiles(dev_u8(t), rows, cols) for t in tiles]
    xs = [torch.empty(cols, device="cuda") for _ in ws]
    ys_plan = [torch.empty(rows, device="cuda") for _ in ws]
    y_single = torch.empty(rows, device="cuda")
    xb = torch.empty(4, cols, device="cuda")
    yb = torch.empty(4, rows, device="cuda")
    s = torch.cuda.Stream()
    plan = api.Plan([(w, x, y) for w, x, y in zip(ws, xs, ys_plan)])

    def work():
        assert plan.launch(s.cuda_stream)
        api.mul_mat(ws[0], xs[1], y_single, stream=s.cuda_stream)
        assert api.mul_mat_batch(ws[1], xb, yb, stream=s.cuda_stream)

    with torch.cuda.stream(s):
        for x in xs + [xb]:
            x.normal_()
        work()  # allocates the per-tensor split-K workspace of stream s
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        work()
    for rep in range(4):
        with torch.cuda.stream(s):
            for x in xs + [xb]:
                x.normal_()
            work()
        s.synchronize()
        outs = ys_plan + [y_single, yb]
        eager = [y.clone() for y in outs]
        for y in outs:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        for got, want in zip(outs, eager):
            assert torch.equal(got, want), rep
        # and the replays are right, not just repeatable
        for t, x, y in zip(tiles, xs, ys_plan):
            assert_gemv_parity(y.cpu().numpy(), t, rows, cols, x.cpu().numpy(), label=("plan replay", rep))
        assert_gemv_parity(y_single.cpu().numpy(), tiles[0], rows, cols, xs[1].cpu().numpy(), label=("single", rep))
        for v in range(4):
            assert_gemv_parity(yb[v].cpu().numpy(), tiles[1], rows, cols, xb[v].cpu().numpy(), label=("batch", rep, v))
    plan.close()


@pytest.mark.gpu
def test_graph_replays_after_the_split_k_workspace_grows(cuda):
    """A per-tensor launch captured into a HIP graph keeps the stream's
    split-K workspace of that moment.  A larger shape on the same stream
    afterwards grows the workspace; the outgrown buffers are kept, so the
    graph still replays correctly (bit-identical to an eager call), and the
    larger call is right too."""
    small_rows, small_cols = 1024, 4096
    big_rows, big_cols = 4096, 28672
    assert api.policy_split_k(small_rows, small_cols) > 1
    assert api.policy_split_k(big_rows, big_cols) * big_rows > api.policy_split_k(small_rows, small_cols) * small_rows
    t_small = random_tiles(small_rows, small_cols, 1600)
    t_big = random_tiles(big_rows, big_cols, 1601)
    w_small = api.QWeight.from_tiles(dev_u8(t_small), small_rows, small_cols)
    w_big = api.QWeight.from_tiles(dev_u8(t_big), big_rows, big_cols)
    x_small = torch.empty(small_cols, device="cuda")
    y_small = torch.empty(small_rows, device="cuda")
    x_big = dev_f32(O.gaussian_x(big_cols, 1602))
    y_big = torch.empty(big_rows, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        x_small.normal_()
        api.mul_mat(w_small, x_small, y_small, stream=s.cuda_stream)  # allocates the small workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        api.mul_mat(w_small, x_small, y_small, stream=s.cuda_stream)
    for rep in range(3):
        with torch.cuda.stream(s):
            api.mul_mat(w_big, x_big, y_big, stream=s.cuda_stream)  # grows the workspace on the first pass
            x_small.normal_()
            api.mul_mat(w_small, x_small, y_small, stream=s.cuda_stream)
        s.synchronize()
        want = y_small.clone()
        y_small.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(y_small, want), rep
        assert_gemv_parity(y_small.cpu().numpy(), t_small, small_rows, small_cols, x_small.cpu().numpy(),
                           label=("small replay", rep))
    assert_gemv_parity(y_big.cpu().numpy(), t_big, big_rows, big_cols, x_big.cpu().numpy(), label="grown")


@pytest.mark.gpu
def test_plan_rejects_bad_descriptors(cuda):
    """Argument errors return a negative status from the library and create
    nothing; the Python layer refuses short or misplaced buffers first."""
    t = random_tiles(64, 128, 5)
    w = api.QWeight.from_tiles(dev_u8(t), 64, 128)
    x = torch.zeros(129, device="cuda")
    y = torch.zeros(64, device="cuda")
    L = q4rdna.load()
    from q4rdna._lib import GemvDesc
    descs = (GemvDesc * 1)()
    descs[0].weight = w.raw
    descs[0].x = x.data_ptr()
    descs[0].y = y.data_ptr()
    h = ctypes.c_void_p()
    for batch in (0, 9):
        assert L.q4rdna_plan_create_batch(descs, 1, batch, 0, ctypes.byref(h)) == q4rdna.ERR_ARGUMENT
    descs[0].x = x[1:].data_ptr()  # misaligned activation
    assert L.q4rdna_plan_create_batch(descs, 1, 1, 0, ctypes.byref(h)) == q4rdna.ERR_ARGUMENT
    assert "alignment" in q4rdna.last_error()
    assert not h.value
    with pytest.raises(ValueError):
        api.Plan([(w, x, y)])            # x holds 129 floats, 128 are needed
    with pytest.raises(ValueError):
        api.Plan([(w, x[:128], y)], batch=2)
    with pytest.raises(ValueError):
        api.dequantize(w, out=torch.empty(64 * 127, device="cuda"))


def test_pack_refuses_a_bad_output_buffer(cuda):
    """api.pack checks the output buffer before the library sees its address:
    short, long, mistyped and non-contiguous buffers are refused, nothing is
    written."""
    w = dev_f32(O.gaussian_weights(64, 128, 3))
    need = api.packed_size(64, 128)
    for bad in (torch.zeros(need - 1, dtype=torch.uint8, device="cuda"),
                torch.zeros(need + 1, dtype=torch.uint8, device="cuda"),
                torch.zeros(need, dtype=torch.int8, device="cuda"),
                torch.zeros(2 * need, dtype=torch.uint8, device="cuda")[::2],
                torch.zeros(need, dtype=torch.uint8)):
        with pytest.raises(ValueError):
            api.pack(w, out=bad)
        assert not bad.any()
    good = torch.zeros(need, dtype=torch.uint8, device="cuda")
    assert np.array_equal(api.pack(w, out=good).cpu().numpy(), O.pack(w.cpu().numpy()))
