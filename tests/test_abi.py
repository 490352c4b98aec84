"""CPU-side checks of the C-ABI library: it loads, exports every function
include/q4rdna.h declares, and its host-only paths (sidecar validation, the
scope filter, argument checks that return before any HIP call) behave as the
reference's loader and entry points do.  No compute call is made here."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle as O
import q4rdna
from q4rdna import _lib
from q4rdna.sidecar import write_sidecar

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q4rdna.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q4rdna_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = q4rdna.load()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(L, name), name
    assert set(names) == set(_lib.EXPORTS)
    assert L.q4rdna_abi_version() == 4


def test_library_is_gfx950_code_object():
    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert b"gfx1201" not in data


def test_scope_filter_matches_reference_rules():
    # source/q4rdna.cu:685-696, written out per scope for one layer
    q, k, v, o, g, u, d = [n for n, _, _ in q4rdna.qwen3_8b_stack(1)]
    admitted = {
        None: {q, k, v, o, g, u, d},
        "": {q, k, v, o, g, u, d},
        "ffn": {g, u, d},
        "qkv-fallback": {o, g, u, d},
        "hotspot": {g, u},
        "attn": {q, k, v, o},
        "unknown-scope": {q, k, v, o, g, u, d},
    }
    for scope, names in admitted.items():
        for n in (q, k, v, o, g, u, d):
            assert q4rdna.api.scope_allows(scope, n) == (n in names), (scope, n)


def test_sidecar_writer_matches_reference_image(golden):
    img = golden["sidecar_image"].tobytes()
    entries = []
    for i in range(3):
        name, rows, cols, off, size, _ = O.ENTRY.unpack(img[48 + 96 * i: 144 + 96 * i])
        entries.append((name.rstrip(b"\0").decode(), rows, cols, img[off:off + size]))
    import io
    buf = io.BytesIO()
    n = write_sidecar(buf, entries)
    assert n == len(img)
    assert buf.getvalue() == img


def test_inspect_accepts_and_rejects_like_the_loader(golden):
    img = bytearray(golden["sidecar_image"].tobytes())
    assert q4rdna.api.inspect_sidecar(bytes(img)) == 3
    mutations = [
        (0, b"Q4RDNA2"), (8, (2).to_bytes(4, "little")), (16, (32).to_bytes(4, "little")),
        (20, (16).to_bytes(4, "little")), (24, (1024).to_bytes(4, "little")),
        (12, (1000).to_bytes(4, "little")), (48, b"x" * 64), (48 + 64, (33).to_bytes(4, "little")),
        (48 + 68, (65).to_bytes(4, "little")), (48 + 80, (5).to_bytes(8, "little")),
        (48 + 72, (0).to_bytes(8, "little")), (48 + 72, (2**64 - 8).to_bytes(8, "little")),
    ]
    for off, data in mutations:
        m = bytearray(img)
        m[off:off + len(data)] = data
        expect = O.validate_sidecar(m)
        assert expect < 0
        with pytest.raises(q4rdna.Q4RdnaError) as e:
            q4rdna.api.inspect_sidecar(bytes(m))
        assert e.value.code == q4rdna.ERR_FORMAT, (off, q4rdna.last_error())
    short = bytes(img[:-300])
    assert O.validate_sidecar(short) == -4
    with pytest.raises(q4rdna.Q4RdnaError):
        q4rdna.api.inspect_sidecar(short)


def test_argument_errors_before_any_device_call():
    L = q4rdna.load()
    w = _lib.Weight()
    # NULL weight: not applicable, as the reference returns false.
    assert L.q4rdna_mul_mat(None, None, 0, None, 0, None) == q4rdna.NOT_APPLICABLE
    assert L.q4rdna_weight_from_device(None, 32, 64, 0, ctypes.byref(w)) == q4rdna.ERR_ARGUMENT
    assert L.q4rdna_weight_from_device(ctypes.c_void_p(4096), 33, 64, 0, ctypes.byref(w)) == q4rdna.ERR_ARGUMENT
    assert L.q4rdna_weight_from_device(ctypes.c_void_p(4096), 32, 96, 0, ctypes.byref(w)) == q4rdna.ERR_ARGUMENT
    assert L.q4rdna_weight_from_device(ctypes.c_void_p(4097), 32, 64, 0, ctypes.byref(w)) == q4rdna.ERR_ARGUMENT
    assert L.q4rdna_weight_from_device(ctypes.c_void_p(4096), 32, 64, 0, ctypes.byref(w)) == q4rdna.OK
    assert (w.rows, w.columns, w.device) == (32, 64, 0)
    assert L.q4rdna_pack(None, 32, 64, 0, None, None) == q4rdna.ERR_ARGUMENT
    assert L.q4rdna_pack(ctypes.c_void_p(4096), 32, 64, 9, ctypes.c_void_p(4096), None) == q4rdna.ERR_ARGUMENT
    assert "algorithm" in q4rdna.last_error()
    assert L.q4rdna_plan_create(None, 1, 0, ctypes.byref(ctypes.c_void_p())) == q4rdna.ERR_ARGUMENT
    assert L.q4rdna_sidecar_open(b"/nonexistent/file.q4rdna", 0, ctypes.byref(ctypes.c_void_p())) == q4rdna.ERR_IO
    assert L.q4rdna_sidecar_count(None) == 0
    assert L.q4rdna_find(None, b"x", 64, 32, ctypes.byref(w)) == q4rdna.NOT_APPLICABLE


def test_glu_op_other_than_swiglu_is_not_applicable():
    L = q4rdna.load()
    assert L.q4rdna_mul_mat_glu(None, None, None, 0, 7, None, 0, None) == q4rdna.NOT_APPLICABLE


def test_python_constants_match_the_header():
    """Every Q4RDNA_* constant the header defines that the ctypes harness
    mirrors (status codes, format, algorithms, kernels, limits, the no-alloc
    slot count) has the header's value, so the two cannot drift apart."""
    import re
    from q4rdna import _lib
    header = open(os.path.join(ROOT, "include", "q4rdna.h")).read()
    seen = 0
    for name, expr in re.findall(r"^#define Q4RDNA_(\w+)\s+([^/\n]+)", header, flags=re.M):
        if name in ("H", "ABI_VERSION") or not hasattr(_lib, name):
            continue
        value = eval(re.sub(r"(\d+)u\b", r"\1", expr.strip()), {})
        assert getattr(_lib, name) == value, (name, getattr(_lib, name), value)
        seen += 1
    assert seen >= 18, seen
