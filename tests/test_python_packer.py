"""The reference's canonical Python packer (source/pack_q4rdna_sidecar.py
quantize :44-73 and pack_tensor :77-98) against the native packer's
algorithm, which the oracle restates and the GPU packer reproduces byte for
byte.  The fixtures in tests/golden/q4rdna_python_packer.npz hold what the
Python packer itself produced (tests/golden/make_python_packer_golden.py
imported it from the reference tree to write them).

What they pin:
  * on N(0, 0.02) bf16 weights (the golden "small" and "outlier" cases and a
    4096 x 4096 sample) the two packers write the same bytes except where a
    scale and its negation tie exactly in the search's squared error (a group
    whose extremes are symmetric), which the two break differently, or where
    two adjacent fp16 scales tie to float32 rounding and the two summation
    orders rank them differently (24 of 262,144 groups: 22 and 2);
  * on the engineered "edge" groups they also differ where a scale is an
    fp16 subnormal (the native packer decodes subnormals at half their value
    inside its search, torch exactly), where the Python search overflows to
    an infinite scale, and in the sign of a zero scale."""
import hashlib

import numpy as np
import pytest

import oracle as O
from conftest import GOLDEN

PYTHON_FIXTURES = GOLDEN.replace("q4rdna_golden.npz", "q4rdna_python_packer.npz")


def group_bytes(tiles: np.ndarray, rows: int, cols: int):
    """Per (row, group): the fp16 scale bits and the 32 code bytes."""
    g = cols // 64
    t = tiles.reshape(rows // 32, g, 1088)
    scales = t[:, :, :64].copy().view(np.uint16).reshape(rows // 32, g, 32).transpose(0, 2, 1).reshape(rows, g)
    codes = t[:, :, 64:].reshape(rows // 32, g, 32, 32).transpose(0, 3, 1, 2).reshape(rows, g, 32)
    return scales, codes


def dequant_group(scale_bits: int, codes: np.ndarray) -> np.ndarray:
    """fp32(scale) * q for the group's 64 weights (IEEE fp16 decode)."""
    s = np.float32(np.uint16(scale_bits).view(np.float16))
    b = codes.astype(np.int32)
    q = np.empty(64, np.float32)
    q[0::2] = ((b & 15) ^ 8) - 8
    q[1::2] = ((b >> 4) ^ 8) - 8
    return s * q


def differing(a, b, rows, cols):
    sa, ca = group_bytes(a, rows, cols)
    sb, cb = group_bytes(b, rows, cols)
    return np.argwhere((sa != sb) | (ca != cb).any(axis=2))


@pytest.fixture(scope="module")
def py():
    return np.load(PYTHON_FIXTURES)


@pytest.mark.parametrize("case,count", [("small", 0), ("outlier", 0), ("edge", 63)])
def test_python_packer_golden_cases(golden, py, case, count):
    bits = golden[f"{case}_bf16"]
    rows, cols = bits.shape
    values = (bits.astype(np.uint32) << 16).view(np.float32)
    native = O.pack(values, O.ALGO_SIDECAR)
    python = py[f"{case}_tiles"]
    assert python.size == native.size
    idx = differing(python, native, rows, cols)
    assert len(idx) == count == int(py["disagree_counts"][["edge", "small", "outlier"].index(case)])
    ps, pc = group_bytes(python, rows, cols)
    ns, nc = group_bytes(native, rows, cols)
    kinds = {"tie": 0, "subnormal": 0, "overflow": 0, "zero sign": 0}
    for r, g in idx:
        p_scale = abs(float(np.uint16(ps[r, g]).view(np.float16)))
        n_scale = abs(float(np.uint16(ns[r, g]).view(np.float16)))
        if np.array_equal(dequant_group(ps[r, g], pc[r, g]), dequant_group(ns[r, g], nc[r, g])):
            kinds["zero sign" if p_scale == n_scale == 0.0 else "tie"] += 1
        elif np.isinf(p_scale):
            kinds["overflow"] += 1
        else:
            # a subnormal scale on at least one side (below 2^-14)
            assert min(p_scale or np.inf, n_scale or np.inf) < 2.0 ** -14, (case, r, g, ps[r, g], ns[r, g])
            kinds["subnormal"] += 1
    if case == "edge":
        assert kinds["subnormal"] == 61 and kinds["overflow"] == 1 and kinds["zero sign"] == 1, kinds


def test_python_packer_large_sample(py):
    """4096 x 4096 bf16 N(0, 0.02): the native algorithm's tiles with the
    fixture's differing groups replaced by the Python packer's bytes hash
    to the Python packer's tiles, so every other group agrees byte for byte;
    every differing group is a tie between a scale and its negation."""
    rows, cols, seed = (int(v) for v in py["large_shape_seed"])
    _, values = O.bf16_round(O.gaussian_weights(rows, cols, seed))
    values = values.reshape(rows, cols)
    native, _ = O.pack_mt(values, O.ALGO_SIDECAR)
    idx = py["large_groups"]
    assert len(idx) == int(py["disagree_counts"][3]) == 24
    g = cols // 64
    t = native.copy().reshape(rows // 32, g, 1088)
    ns, nc = group_bytes(native, rows, cols)
    kinds = {"sign tie": 0, "near tie": 0}
    for (r, gi), sbits, codes in zip(idx, py["large_scales"], py["large_codes"]):
        v = values[r, 64 * gi:64 * gi + 64].astype(np.float64)
        a = dequant_group(sbits, codes).astype(np.float64)
        b = dequant_group(ns[r, gi], nc[r, gi]).astype(np.float64)
        ea, eb = ((v - a) ** 2).sum(), ((v - b) ** 2).sum()
        if sbits == ns[r, gi] ^ 0x8000:
            # The negated scale with exactly the same squared error.  Only
            # weights beyond 7|s| land differently: there the two signs of
            # the scale reach the asymmetric ends of the code range [-8, 7].
            assert ea == eb, (r, gi)
            scale = abs(float(np.uint16(sbits).view(np.float16)))
            assert np.all((a == b) | (np.abs(v) > 7.0 * scale)), (r, gi)
            kinds["sign tie"] += 1
        else:
            # Adjacent fp16 scales whose errors agree to float32 rounding: the
            # summation orders (torch's reduction, the native sequential
            # loop) rank them differently.
            assert abs(int(sbits) - int(ns[r, gi])) == 1, (r, gi)
            assert abs(ea - eb) <= 1e-6 * max(ea, eb), (r, gi)
            kinds["near tie"] += 1
        t[r // 32, gi, 2 * (r % 32):2 * (r % 32) + 2] = np.array([sbits], np.uint16).view(np.uint8)
        t[r // 32, gi, 64 + 32 * np.arange(32) + (r % 32)] = codes
    assert kinds == {"sign tie": 22, "near tie": 2}, kinds
    assert hashlib.sha256(t.tobytes()).hexdigest() == str(py["large_sha256"])
