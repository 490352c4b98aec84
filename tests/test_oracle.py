"""Pins the CPU oracle (oracle/q4oracle.c) before anything is checked against it.

Each function is checked against something other than itself: the reference's
compiled tools (oracle/_ref) and the golden fixtures they wrote, textbook
definitions evaluated independently (numpy), exhaustive enumeration, and
closed forms.  Tests that plant a mistake plant it in a copy of the oracle's
computation here on the CPU and show the checks catch it.
"""
import hashlib
import os

import numpy as np
import pytest

import oracle as O
from conftest import bf16_to_f32

ALGOS = [(O.ALGO_SIDECAR, "sidecar"), (O.ALGO_ABSMAX, "absmax"), (O.ALGO_RANGE, "range"), (O.ALGO_MSE, "mse")]


# ----------------------------------------------------------------- fp16 decode

def textbook_fp16(h: int) -> float:
    s = -1.0 if h & 0x8000 else 1.0
    e = (h >> 10) & 0x1F
    m = h & 0x3FF
    if e == 0:
        return s * m * 2.0 ** -24
    if e == 31:
        return s * np.inf if m == 0 else np.nan
    return s * (1.0 + m / 1024.0) * 2.0 ** (e - 15)


def test_fp16_decode_exhaustive():
    lib = O.lib()
    for h in range(65536):
        got = lib.q4o_fp16_to_f32(h)
        want = textbook_fp16(h)
        if np.isnan(want):
            assert np.isnan(got)
        else:
            assert got == want, hex(h)
            assert np.signbit(got) == bool(h & 0x8000)


def test_reference_cpu_decode_halves_subnormals():
    """The reference CPU tools' decode equals the textbook value for normal
    numbers, zeros and infinities and half of it for subnormals
    (source/q4rdna_sidecar_pack.cpp:87 uses 127-15-shift)."""
    lib = O.lib()
    for h in range(65536):
        got = lib.q4o_fp16_to_f32_ref(h)
        want = textbook_fp16(h)
        if np.isnan(want):
            assert np.isnan(got)
        elif (h & 0x7C00) == 0 and (h & 0x3FF) != 0:
            assert got == want / 2, hex(h)
        else:
            assert got == want, hex(h)


def test_fp16_encode_matches_ieee_rne():
    rng = np.random.default_rng(7)
    bits = np.concatenate([
        rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32),
        np.arange(0x33000000, 0x33800000, 997, dtype=np.uint32),  # subnormal boundary region
        np.arange(0x477fe000, 0x47800100, 1, dtype=np.uint32),    # overflow boundary
        np.array([0, 0x80000000, 0x7f800000, 0xff800000], dtype=np.uint32),
    ])
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    # Every constructed value: the random bits and both boundary regions
    # (the subnormal range's edge near 2^-25..2^-24 and the overflow edge at
    # 65504..65536) and the signed zeros and infinities.
    want = f.astype(np.float16).view(np.uint16)
    lib = O.lib()
    got = np.array([lib.q4o_f32_to_fp16(float(v)) for v in f], dtype=np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(int(f[i].view(np.uint32))), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]
    assert got.size > 215000
    # The reference maps NaN to infinity (source/q4rdna_sidecar_pack.cpp:112).
    assert lib.q4o_f32_to_fp16(float("nan")) == 0x7C00


def test_nibble_decode_exhaustive():
    lib = O.lib()
    for b in range(256):
        lo, hi = b & 15, b >> 4
        assert lib.q4o_nibble_low(b) == (lo - 16 if lo >= 8 else lo)
        assert lib.q4o_nibble_high(b) == (hi - 16 if hi >= 8 else hi)


# ----------------------------------------------------------------- layout / dequant

def all_scales_tiles() -> tuple[np.ndarray, int, int]:
    """2048 x 2048 tensor whose 65536 (row, group) pairs carry every fp16 bit
    pattern as scale and the 16 codes cycling in every group."""
    rows, cols = 2048, 2048
    g = cols // 64
    tiles = np.zeros(O.packed_size(rows, cols), np.uint8).reshape(rows // 32, g, 1088)
    scales = np.arange(65536, dtype=np.uint16).reshape(rows // 32, 32, g).transpose(0, 2, 1)
    tiles[:, :, :64] = scales.copy().view(np.uint8).reshape(rows // 32, g, 64)
    codes = (np.arange(1024) % 256).astype(np.uint8)
    tiles[:, :, 64:] = codes
    return tiles.reshape(-1), rows, cols


def dequant_closed_form(tiles, rows, cols):
    g = cols // 64
    t = tiles.reshape(rows // 32, g, 1088)
    s = t[:, :, :64].copy().view(np.float16).astype(np.float32)        # [rt, g, lane]
    c = t[:, :, 64:].reshape(rows // 32, g, 32, 32)                     # [rt, g, i, lane]
    lo = ((c & 15).astype(np.int8) << 4) >> 4
    hi = (c.astype(np.int8) >> 4)
    q = np.stack([lo, hi], axis=3)                                      # [rt, g, i, 2, lane]
    q = q.reshape(rows // 32, g, 64, 32).transpose(0, 3, 1, 2)          # [rt, lane, g, k]
    w = s.transpose(0, 2, 1)[:, :, :, None] * q.astype(np.float32)
    return w.reshape(rows, cols)


def test_dequant_exhaustive_scales_and_signed_zero():
    tiles, rows, cols = all_scales_tiles()
    got = O.dequant(tiles, rows, cols)
    want = dequant_closed_form(tiles, rows, cols)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # code 0 with a negative scale is -0.0
    assert np.signbit(got[~nan & (want == 0) & np.signbit(want)]).all()


def test_layout_offsets_brute_force():
    for rows, cols in [(32, 64), (64, 128), (96, 192)]:
        lib = O.lib()
        g = cols // 64
        seen = set()
        for r in range(rows):
            for gg in range(g):
                off = lib.q4o_scale_offset(cols, r, gg)
                assert off == ((r // 32) * g + gg) * 1088 + 2 * (r % 32)
                seen.update((off, off + 1))
            for k in range(0, cols, 2):
                off = lib.q4o_code_offset(cols, r, k)
                assert off == ((r // 32) * g + k // 64) * 1088 + 64 + 32 * ((k % 64) // 2) + r % 32
                seen.add(off)
        assert seen == set(range(O.packed_size(rows, cols)))  # a bijection onto the tensor bytes


def test_pack_dequant_roundtrip_codes():
    rng = np.random.default_rng(3)
    rows, cols = 64, 256
    codes = rng.integers(-8, 8, (rows, cols))
    scales = rng.choice([0.5, 0.25, -0.125, 2.0], (rows, cols // 64)).astype(np.float32)
    w = (codes.reshape(rows, cols // 64, 64) * scales[:, :, None]).reshape(rows, cols).astype(np.float32)
    for algo in (O.ALGO_SIDECAR, O.ALGO_MSE):
        back = O.dequant(O.pack(w, algo), rows, cols)
        # exactly representable groups quantize losslessly
        assert np.array_equal(back, w)


# ----------------------------------------------------------------- quantizers

@pytest.mark.parametrize("case", ["edge", "small", "outlier"])
@pytest.mark.parametrize("algo,name", ALGOS)
def test_pack_matches_reference_golden(golden, case, algo, name):
    w = bf16_to_f32(golden[f"{case}_bf16"])
    assert np.array_equal(O.pack(w, algo), golden[f"{case}_{name}"])


def test_pack_matches_reference_large_sha(golden):
    rows, cols, seed = (int(v) for v in golden["large_shape_seed"])
    _, w = O.bf16_round(O.gaussian_weights(rows, cols, seed))
    want = dict(s.split(":") for s in golden["large_sha256"])
    for algo, name in ALGOS:
        assert hashlib.sha256(O.pack(w, algo).tobytes()).hexdigest() == want[name], name


@pytest.mark.skipif(not O.ref_available(), reason="reference tools not built (oracle/_ref)")
def test_pack_matches_reference_tools_fresh_seeds():
    for seed in (11, 12):
        w = O.gaussian_weights(32, 1024, seed)
        w.reshape(-1, 64)[np.random.default_rng(seed).permutation(512)[:5]] *= 20
        bits, wf = O.bf16_round(w)
        img = O.ref_sidecar_pack([("t", bits)])
        off = O.ENTRY.unpack(img[48:144])[3]
        assert np.array_equal(O.pack(wf, O.ALGO_SIDECAR), np.frombuffer(img[off:off + O.packed_size(32, 1024)], np.uint8))
        for algo, name in ALGOS[1:]:
            assert np.array_equal(O.pack(wf, algo), np.frombuffer(O.ref_cpu_experiment(bits, name), np.uint8))


def test_quantizer_closed_forms():
    z = np.zeros(64, np.float32)
    for algo, _ in ALGOS:
        assert O.select_scale(z, algo) == 0                       # all-zero group
    for v in (0.875, -1.0, 7 * 2.0 ** -12):
        g = np.zeros(64, np.float32)
        g[9] = v
        for algo, _ in ALGOS:
            if algo == O.ALGO_ABSMAX and v < 0:
                continue  # absmax uses |v|/7 only: -1.0 maps to code -7
            # a single value with an exactly representable range scale
            # (v/7 or -v/8) quantizes exactly, and every other code is 0
            tiles = O.pack(np.tile(g, (32, 1)), algo)
            back = O.dequant(tiles, 32, 64)
            assert back[0, 9] == np.float32(v) and not back[0, np.arange(64) != 9].any(), (v, algo)
    rng = np.random.default_rng(5)
    g = rng.standard_normal(64).astype(np.float32)
    want = np.float32(np.max(np.abs(g))) / np.float32(7.0)
    assert O.select_scale(g, O.ALGO_ABSMAX) == int(np.array([want], np.float32).astype(np.float16).view(np.uint16)[0])


def test_search_beats_every_start():
    """The native search returns the best scale among its candidates: its
    error is never above the plain range-scale error."""
    rng = np.random.default_rng(9)
    lib = O.lib()
    for _ in range(200):
        g = (rng.standard_normal(64) * 0.02).astype(np.float32)
        s = O.fp16_to_f32(O.select_scale(g, O.ALGO_SIDECAR))
        pmax, nmax = max(0.0, g.max()), max(0.0, -g.min())
        r = O.fp16_to_f32(O.f32_to_fp16(np.float32(max(pmax / 7, nmax / 8))))
        def err(sc):
            q = np.array([lib.q4o_quantize_value_rne(float(v), float(sc)) for v in g], np.float32)
            return float(np.sum((np.float32(sc) * q - g) ** 2))
        assert err(s) <= err(r) * (1 + 1e-6)


# ----------------------------------------------------------------- GEMV

def small_problem(rows=64, cols=512, seed=1):
    w = O.gaussian_weights(rows, cols, seed)
    tiles = O.pack(w)
    x = O.gaussian_x(cols, seed + 100)
    return tiles, x


def test_gemv_f64_matches_numpy_matmul():
    tiles, x = small_problem()
    w = O.dequant(tiles, 64, 512).astype(np.float64)
    y64, a64 = O.gemv_f64(tiles, 64, 512, x)
    ref = w @ x.astype(np.float64)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12)
    assert np.allclose(a64, np.abs(w * x.astype(np.float64)).sum(1), rtol=1e-12)


def test_gemv_seq_f32_is_sequential_fma():
    tiles, x = small_problem(32, 128, 4)
    w = O.dequant(tiles, 32, 128)
    y = O.gemv_seq_f32(tiles, 32, 128, x)
    want = np.zeros(32, np.float32)
    for r in range(32):
        acc = np.float32(0)
        for k in range(128):
            acc = np.float32(np.float64(w[r, k]) * np.float64(x[k]) + np.float64(acc))  # fma: one rounding
        want[r] = acc
    assert np.array_equal(y, want)


def test_gemv_seq_f32_threads_match_one_thread():
    tiles, x = small_problem(256, 512, 9)
    y1 = O.gemv_seq_f32(tiles, 256, 512, x)
    ym, used = O.gemv_seq_f32_mt(tiles, 256, 512, x, threads=4)
    assert used >= 1
    assert np.array_equal(y1, ym)


@pytest.mark.parametrize("algorithm", [0, 1, 2, 3])
def test_pack_threads_match_one_thread(algorithm):
    """The all-cores packer writes the same bytes as the one-thread packer,
    on Gaussian weights with outlier and near-zero groups."""
    w = O.gaussian_weights(128, 256, 17 + algorithm)
    w.reshape(-1, 64)[::7] *= 20
    w.reshape(-1, 64)[3::11] *= 1e-5
    one = O.pack(w, algorithm)
    many, used = O.pack_mt(w, algorithm, threads=4)
    assert used >= 1
    assert np.array_equal(one, many)


def test_gemv_gates_accept_oracle_and_catch_planted_mistakes():
    tiles, x = small_problem(256, 1024, 8)
    rows, cols = 256, 1024
    y64, a64 = O.gemv_f64(tiles, rows, cols, x)
    yseq = O.gemv_seq_f32(tiles, rows, cols, x)
    assert O.gemv_errors(yseq, y64, a64)["gate"] <= 1e-3
    assert O.rel_l2(yseq, y64) <= 1e-5
    w = O.dequant(tiles, rows, cols).astype(np.float64)
    xd = x.astype(np.float64)
    mistakes = {
        "swapped nibbles": (w.reshape(rows, -1, 2)[:, :, ::-1].reshape(rows, cols)) @ xd,
        "dropped scale": np.sign(w) @ xd,
        "transposed x pairs": w @ xd.reshape(-1, 2)[:, ::-1].reshape(-1),
        "dropped last group": w[:, :-64] @ xd[:-64],
        "wrong row order": (w @ xd)[np.r_[1:rows, 0]],
        "sign flip": -(w @ xd),
    }
    for name, bad in mistakes.items():
        assert O.gemv_errors(bad, y64, a64)["gate"] > 1e-3, name
        assert O.rel_l2(bad, y64) > 1e-5, name


def test_silu_textbook():
    g = np.array([-20.0, -1.5, 0.0, 0.3, 4.0, 30.0])
    assert np.allclose(O.silu(g), g / (1 + np.exp(-g)), rtol=1e-15, atol=1e-300)


def silu_identities_hold(f) -> bool:
    """Facts of silu(g) = g * sigmoid(g) that do not restate the formula:
    silu(g) - silu(-g) = g (sigmoid(g) + sigmoid(-g) = 1), silu(0) = 0,
    silu'(0) = 1/2 (silu(h) / h = 1/2 + h/4 + O(h^3)), silu(g) -> g for large
    g and -> g e^g for very negative g."""
    g = np.array([0.1, 0.7, 1.5, 3.0, 9.0, 20.0])
    ok = np.allclose(f(g) - f(-g), g, rtol=1e-13, atol=0)
    ok &= f(np.array([0.0]))[0] == 0.0
    for h in (1e-3, 1e-4):
        ok &= abs(f(np.array([h]))[0] / h - (0.5 + h / 4)) < h ** 3
    ok &= abs(f(np.array([40.0]))[0] - 40.0) < 1e-13
    ok &= abs(f(np.array([-40.0]))[0] / (-40.0 * np.exp(-40.0)) - 1.0) < 1e-12
    return bool(ok)


def test_silu_identities():
    assert silu_identities_hold(O.silu)
    # planted mistakes: the sign of the exponent, a dropped g, the sigmoid
    # of -g: each breaks at least one identity
    assert not silu_identities_hold(lambda g: g / (1 + np.exp(g)))
    assert not silu_identities_hold(lambda g: 1 / (1 + np.exp(-g)))
    assert not silu_identities_hold(lambda g: -g / (1 + np.exp(g)))


# ----------------------------------------------------------------- sidecar

def test_stack_known_answers():
    import q4rdna
    names = q4rdna.qwen3_8b_stack()
    assert len(names) == 252
    weights = sum(r * c for _, r, c in names)
    assert weights == 6945767424                                  # results/kernel_profile.json:22
    from q4rdna.sidecar import layout
    data_offset, entries, end = layout(names)
    assert data_offset == 24576
    assert end - data_offset == 3689938944                        # results/provenance.json:34
    assert sum(e[4] for e in entries) == 3689938944


def test_sidecar_validation_rules(golden):
    img = bytearray(golden["sidecar_image"].tobytes())
    assert O.validate_sidecar(img) == 3
    def mutate(off, data):
        m = bytearray(img)
        m[off:off + len(data)] = data
        return O.validate_sidecar(m)
    assert mutate(0, b"Q4RDNA2") == -1                            # magic
    assert mutate(8, (2).to_bytes(4, "little")) == -1             # version
    assert mutate(16, (32).to_bytes(4, "little")) == -1           # group
    assert mutate(12, (1000).to_bytes(4, "little")) == -2         # truncated index
    assert mutate(48, b"x" * 64) == -3                            # name without NUL
    assert mutate(48 + 64, (33).to_bytes(4, "little")) == -3      # rows % 32
    assert mutate(48 + 80, (5).to_bytes(8, "little")) == -3       # size
    assert mutate(48 + 72, (0).to_bytes(8, "little")) == -3       # offset < data_offset
    assert O.validate_sidecar(img[: len(img) - 300]) == -4        # truncated data


# ----------------------------------------------------------------- the reference bench's own case

BENCH_CASE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4rdna_bench_case.json")


def test_bench_case_fixture_pins_the_oracle():
    """The reference bench's correctness case (source/q4rdna_gemv_bench.hip:
    215-262): the oracle's absmax packer (source/q4rdna_cpu_experiment.cpp's
    default search) writes the tile stream whose sha256 the reference's own
    experiment produced for these weights, and the bench activation has the
    recorded bytes."""
    import json
    case = json.load(open(BENCH_CASE))
    _, w = O.bf16_round(O.gaussian_weights(case["rows"], case["cols"], case["seed"]))
    tiles, _ = O.pack_mt(w, O.ALGO_ABSMAX)
    assert hashlib.sha256(tiles.tobytes()).hexdigest() == case["tiles_sha256"]
    x = O.bench_activation(case["cols"])
    assert hashlib.sha256(x.tobytes()).hexdigest() == case["x_sha256"]
    # the formula itself, at points where it is known in closed form
    assert x[0] == np.float32(0.125)
    assert abs(float(x[1]) - (np.sin(0.013) * 0.25 + np.cos(0.007) * 0.125)) < 1e-7
    # every scale is a normal fp16 number, so the bench's fp16 decode
    # (which halves subnormals, :163-187) reads them as IEEE does
    assert case["scales_normal"]
    assert np.array_equal(O.gemv_seq_f32(tiles[:1088 * 64 * 2], 64, case["cols"], x),
                          O.gemv_seq_f32(tiles[:1088 * 64 * 2], 64, case["cols"], x, ref_cpu_decode=True))
