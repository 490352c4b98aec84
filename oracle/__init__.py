"""CPU oracle for the Q4_RDNA group-64 dequant-GEMV (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package, and only as the checker.  The product library never
loads ``liboracle.so``.

``liboracle.so`` is the C restatement in ``q4oracle.c``; every function there
cites the reference file:line it restates.  ``_ref/`` holds the reference's own
CPU tools (``q4rdna_sidecar_pack``, ``q4rdna_cpu_experiment``) compiled from
their sources by ``Makefile`` when the reference tree is mounted; helpers here
drive them to pin the restatement.
"""
from __future__ import annotations

import ctypes
import os
import struct
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")
REF_PACK = os.path.join(REF_DIR, "q4rdna_sidecar_pack")
REF_EXPERIMENT = os.path.join(REF_DIR, "q4rdna_cpu_experiment")

GROUP = 64
TILE_ROWS = 32
TILE_BYTES = 1088

ALGO_SIDECAR = 0
ALGO_ABSMAX = 1
ALGO_RANGE = 2
ALGO_MSE = 3
ALGO_NAMES = {ALGO_ABSMAX: "absmax", ALGO_RANGE: "range", ALGO_MSE: "mse"}

_lib = None


def lib() -> ctypes.CDLL:
    """Load liboracle.so (build it with ``make -C oracle``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        _lib = load_build(LIB_PATH)
    return _lib


def build_native(out_dir: str) -> str:
    """Compile q4oracle.c with -O3 -march=native for the host this runs on
    (the CPU baseline's optimised build; contraction stays off, so every
    result is bit-identical to liboracle.so's).  Returns the library path."""
    out = os.path.join(out_dir, "liboracle_native.so")
    subprocess.run(["gcc", "-O3", "-march=native", "-std=c11", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared",
                    "-o", out, os.path.join(HERE, "q4oracle.c"), "-lm"], check=True)
    return out


def load_build(path: str) -> ctypes.CDLL:
    """Load a build of q4oracle.c and declare its prototypes."""
    L = ctypes.CDLL(path)
    u8p = ctypes.POINTER(ctypes.c_uint8)
    f32p = ctypes.POINTER(ctypes.c_float)
    f64p = ctypes.POINTER(ctypes.c_double)
    u32 = ctypes.c_uint32
    L.q4o_fp16_to_f32.argtypes = [ctypes.c_uint16]
    L.q4o_fp16_to_f32.restype = ctypes.c_float
    L.q4o_fp16_to_f32_ref.argtypes = [ctypes.c_uint16]
    L.q4o_fp16_to_f32_ref.restype = ctypes.c_float
    L.q4o_f32_to_fp16.argtypes = [ctypes.c_float]
    L.q4o_f32_to_fp16.restype = ctypes.c_uint16
    L.q4o_f32_to_bf16.argtypes = [ctypes.c_float]
    L.q4o_f32_to_bf16.restype = ctypes.c_uint16
    L.q4o_nibble_low.argtypes = [ctypes.c_uint8]
    L.q4o_nibble_high.argtypes = [ctypes.c_uint8]
    L.q4o_quantize_value_rne.argtypes = [ctypes.c_float, ctypes.c_float]
    L.q4o_quantize_value_round.argtypes = [ctypes.c_float, ctypes.c_float]
    L.q4o_select_scale.argtypes = [f32p, ctypes.c_int]
    L.q4o_select_scale.restype = ctypes.c_uint16
    L.q4o_pack.argtypes = [f32p, u32, u32, ctypes.c_int, u8p]
    L.q4o_pack_mt.argtypes = [f32p, u32, u32, ctypes.c_int, u8p, ctypes.c_int]
    L.q4o_pack_mt.restype = ctypes.c_int
    L.q4o_dequant.argtypes = [u8p, u32, u32, f32p]
    L.q4o_dequant_ref_cpu.argtypes = [u8p, u32, u32, f32p]
    L.q4o_gemv_seq_f32.argtypes = [u8p, u32, u32, f32p, f32p, u32, u32, ctypes.c_int]
    L.q4o_gemv_seq_f32_mt.argtypes = [u8p, u32, u32, f32p, f32p, ctypes.c_int]
    L.q4o_gemv_seq_f32_mt.restype = ctypes.c_int
    L.q4o_gemv_f64.argtypes = [u8p, u32, u32, f32p, f64p, f64p]
    L.q4o_silu.argtypes = [ctypes.c_double]
    L.q4o_silu.restype = ctypes.c_double
    L.q4o_validate_sidecar.argtypes = [u8p, ctypes.c_uint64]
    L.q4o_validate_sidecar.restype = ctypes.c_long
    L.q4o_scale_offset.argtypes = [u32, u32, u32]
    L.q4o_scale_offset.restype = ctypes.c_uint64
    L.q4o_code_offset.argtypes = [u32, u32, u32]
    L.q4o_code_offset.restype = ctypes.c_uint64
    return L


def _ptr(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def packed_size(rows: int, cols: int) -> int:
    return rows * cols * 34 // GROUP


def fp16_to_f32(h: int) -> float:
    """Exact IEEE decode (the runtime's __half2float)."""
    return lib().q4o_fp16_to_f32(h)


def fp16_to_f32_ref(h: int) -> float:
    """The reference CPU tools' decode (subnormals halved)."""
    return lib().q4o_fp16_to_f32_ref(h)


def f32_to_fp16(f: float) -> int:
    return lib().q4o_f32_to_fp16(f)


def select_scale(group: np.ndarray, algorithm: int = ALGO_SIDECAR) -> int:
    g = np.ascontiguousarray(group, dtype=np.float32)
    assert g.shape == (GROUP,)
    return lib().q4o_select_scale(_ptr(g, ctypes.c_float), algorithm)


def pack(w: np.ndarray, algorithm: int = ALGO_SIDECAR) -> np.ndarray:
    """Quantize fp32 [rows, cols] into Q4_RDNA tile bytes."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.zeros(packed_size(rows, cols), dtype=np.uint8)
    rc = lib().q4o_pack(_ptr(w, ctypes.c_float), rows, cols, algorithm, _ptr(out, ctypes.c_uint8))
    if rc != 0:
        raise ValueError(f"unsupported shape {w.shape} or algorithm {algorithm}")
    return out


def pack_mt(w: np.ndarray, algorithm: int = ALGO_SIDECAR, threads: int = 0):
    """pack() with row tiles spread over OpenMP threads (0 = the OpenMP
    default); returns (tiles, threads used)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.zeros(packed_size(rows, cols), dtype=np.uint8)
    used = lib().q4o_pack_mt(_ptr(w, ctypes.c_float), rows, cols, algorithm, _ptr(out, ctypes.c_uint8), threads)
    if used < 0:
        raise ValueError(f"unsupported shape {w.shape} or algorithm {algorithm}")
    return out, used


def dequant(tiles: np.ndarray, rows: int, cols: int, ref_cpu_decode: bool = False) -> np.ndarray:
    """fp32(scale) * code; ref_cpu_decode uses the CPU experiment's decode."""
    tiles = np.ascontiguousarray(tiles, dtype=np.uint8)
    assert tiles.size == packed_size(rows, cols)
    out = np.empty((rows, cols), dtype=np.float32)
    fn = lib().q4o_dequant_ref_cpu if ref_cpu_decode else lib().q4o_dequant
    fn(_ptr(tiles, ctypes.c_uint8), rows, cols, _ptr(out, ctypes.c_float))
    return out


def gemv_seq_f32(tiles: np.ndarray, rows: int, cols: int, x: np.ndarray,
                 row_begin: int = 0, row_end: int | None = None, ref_cpu_decode: bool = False) -> np.ndarray:
    """Sequential fp32 fma GEMV in the reference bench's loop order."""
    tiles = np.ascontiguousarray(tiles, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape == (cols,)
    row_end = rows if row_end is None else row_end
    y = np.zeros(rows, dtype=np.float32)
    lib().q4o_gemv_seq_f32(_ptr(tiles, ctypes.c_uint8), rows, cols, _ptr(x, ctypes.c_float),
                           _ptr(y, ctypes.c_float), row_begin, row_end, int(ref_cpu_decode))
    return y


def gemv_seq_f32_mt(tiles: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 0):
    """q4o_gemv_seq_f32 over all rows with OpenMP threads (0 = the OpenMP
    default); returns (y, threads used)."""
    tiles = np.ascontiguousarray(tiles, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape == (cols,)
    y = np.zeros(rows, dtype=np.float32)
    used = lib().q4o_gemv_seq_f32_mt(_ptr(tiles, ctypes.c_uint8), rows, cols, _ptr(x, ctypes.c_float),
                                     _ptr(y, ctypes.c_float), threads)
    return y, used


def gemv_f64(tiles: np.ndarray, rows: int, cols: int, x: np.ndarray):
    """fp64 GEMV and the conditioning sum of |w*x| per row."""
    tiles = np.ascontiguousarray(tiles, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float64)
    a = np.empty(rows, dtype=np.float64)
    lib().q4o_gemv_f64(_ptr(tiles, ctypes.c_uint8), rows, cols, _ptr(x, ctypes.c_float),
                       _ptr(y, ctypes.c_double), _ptr(a, ctypes.c_double))
    return y, a


def silu(g: np.ndarray) -> np.ndarray:
    f = lib().q4o_silu
    return np.array([f(float(v)) for v in np.asarray(g, dtype=np.float64).ravel()]).reshape(np.shape(g))


def validate_sidecar(image: bytes | np.ndarray) -> int:
    buf = np.frombuffer(bytes(image), dtype=np.uint8).copy()
    return lib().q4o_validate_sidecar(_ptr(buf, ctypes.c_uint8), buf.size)


# ---------------------------------------------------------------------------
# GEMV error gate
# ---------------------------------------------------------------------------

def gemv_errors(y: np.ndarray, y64: np.ndarray, absdot: np.ndarray) -> dict:
    """Error figures of a GEMV result against the fp64 oracle.

    ``gate``: max over rows of |y - y64| / max(|y64|, 0.01 * rms(y64)); the
    parity bar is gate <= 1e-3.  ``conditioned``: max |y - y64| / sum|w*x|.
    ``naive_fail``: rows with |y - y64| > 1e-3 * |y64| (reported, not gated).
    """
    y = np.asarray(y, dtype=np.float64)
    diff = np.abs(y - y64)
    rms = float(np.sqrt(np.mean(y64 * y64))) if y64.size else 0.0
    denom = np.maximum(np.abs(y64), 0.01 * rms)
    denom = np.where(denom == 0, 1.0, denom)
    cond = np.where(absdot == 0, diff, diff / np.where(absdot == 0, 1.0, absdot))
    return {
        "gate": float(np.max(diff / denom)) if y.size else 0.0,
        "conditioned": float(np.max(cond)) if y.size else 0.0,
        "naive_fail": int(np.sum(diff > 1e-3 * np.abs(y64))),
        "max_abs": float(np.max(diff)) if y.size else 0.0,
    }


def rel_l2(y: np.ndarray, ref: np.ndarray) -> float:
    """Relative L2 error, the reference bench's GPU-vs-CPU gate
    (source/q4rdna_gemv_bench.hip:250-262, bar 1e-5)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.sum(ref * ref))
    return float(np.sqrt(np.sum((y - ref) ** 2) / den)) if den > 0 else float(np.sqrt(np.sum((y - ref) ** 2)))


# ---------------------------------------------------------------------------
# sidecar container (struct layout of source/q4rdna.cu:26-50)
# ---------------------------------------------------------------------------

HEADER = struct.Struct("<8sIIIIIIQQ")
ENTRY = struct.Struct("<64sIIQQQ")


def align_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def build_sidecar(tensors) -> bytes:
    """Sidecar image for [(name, rows, cols, tile_bytes)], laid out as the
    reference writers do (source/pack_q4rdna_sidecar.py:127-161,
    source/q4rdna_sidecar_pack.cpp:223-245,289)."""
    data_offset = align_up(HEADER.size + ENTRY.size * len(tensors), 4096)
    offset = data_offset
    entries = []
    for name, rows, cols, tiles in tensors:
        size = rows * cols * 34 // GROUP
        assert len(tiles) == size
        entries.append((name, rows, cols, offset, size, tiles))
        offset = align_up(offset + size, 256)
    out = bytearray(offset)
    out[:HEADER.size] = HEADER.pack(b"Q4RDNA1", 1, len(entries), GROUP, TILE_ROWS, TILE_BYTES, 0,
                                    data_offset, offset - data_offset)
    for i, (name, rows, cols, off, size, tiles) in enumerate(entries):
        e = ENTRY.pack(name.encode("ascii"), rows, cols, off, size, 0)
        out[HEADER.size + i * ENTRY.size: HEADER.size + (i + 1) * ENTRY.size] = e
        out[off:off + size] = bytes(np.asarray(tiles, dtype=np.uint8))
    return bytes(out)


# ---------------------------------------------------------------------------
# reference tools (oracle/_ref), available where the reference tree was mounted
# ---------------------------------------------------------------------------

def ref_available() -> bool:
    return os.path.exists(REF_PACK) and os.path.exists(REF_EXPERIMENT)


def ref_sidecar_pack(tensors) -> bytes:
    """Run the reference native packer on [(name, bf16 uint16 [rows, cols])]
    and return the sidecar file bytes."""
    with tempfile.TemporaryDirectory() as d:
        lines = []
        for i, (name, bf16) in enumerate(tensors):
            p = os.path.join(d, f"t{i}.bf16")
            np.ascontiguousarray(bf16, dtype=np.uint16).tofile(p)
            rows, cols = bf16.shape
            lines.append(f"{p}\t0\t{rows}\t{cols}\t{name}\n")
        man = os.path.join(d, "manifest.tsv")
        with open(man, "w") as f:
            f.writelines(lines)
        out = os.path.join(d, "out.q4rdna")
        subprocess.run([REF_PACK, man, out], check=True, capture_output=True,
                       env={**os.environ, "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS", "4")})
        with open(out, "rb") as f:
            return f.read()


def ref_cpu_experiment(bf16: np.ndarray, algorithm: str) -> bytes:
    """Run the reference CPU experiment on bf16 [rows, cols] and return the raw
    tile stream it writes (zero Q4_K blocks feed only its comparison metrics)."""
    rows, cols = bf16.shape
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "w.bf16")
        np.ascontiguousarray(bf16, dtype=np.uint16).tofile(src)
        q4k = os.path.join(d, "q4k.bin")
        with open(q4k, "wb") as f:
            f.write(bytes(rows * cols // 256 * 144))
        out = os.path.join(d, "out.q4rdna")
        js = os.path.join(d, "out.json")
        subprocess.run([REF_EXPERIMENT, src, "0", q4k, "0", str(rows), str(cols), out, js, algorithm],
                       check=True, capture_output=True)
        with open(out, "rb") as f:
            return f.read()


# ---------------------------------------------------------------------------
# seeded inputs
# ---------------------------------------------------------------------------

def bf16_round(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Round fp32 to bf16 (ties to even); return (bf16 bits, fp32 values)."""
    b = np.ascontiguousarray(w, dtype=np.float32).view(np.uint32)
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) >> 16).astype(np.uint16)
    return r, (r.astype(np.uint32) << 16).view(np.float32)


def gaussian_weights(rows: int, cols: int, seed: int, std: float = 0.02) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal((rows, cols), dtype=np.float32) * np.float32(std))


def gaussian_x(cols: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(cols, dtype=np.float32)


def bench_activation(cols: int) -> np.ndarray:
    """The reference bench's deterministic activation
    (source/q4rdna_gemv_bench.hip:224-227): x_i = sinf(float(i) * 0.013f) *
    0.25f + cosf(float(i) * 0.007f) * 0.125f, all in fp32.  The arguments are
    fp32 products, sinf/cosf are the C library's (the reference's std::sin
    and std::cos on float), and since the two scalings by powers of two are
    exact, the sum rounds once whether or not the compiler fuses it."""
    libm = ctypes.CDLL("libm.so.6")
    libm.sinf.restype = libm.cosf.restype = ctypes.c_float
    libm.sinf.argtypes = libm.cosf.argtypes = [ctypes.c_float]
    i = np.arange(cols, dtype=np.float32)
    a = i * np.float32(0.013)
    b = i * np.float32(0.007)
    s = np.array([libm.sinf(float(v)) for v in a], dtype=np.float32)
    c = np.array([libm.cosf(float(v)) for v in b], dtype=np.float32)
    return (s * np.float32(0.25) + c * np.float32(0.125)).astype(np.float32)
