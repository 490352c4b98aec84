"""Sidecar container writer and the Qwen3-8B tensor inventory.

The file layout is the reference's (source/pack_q4rdna_sidecar.py:16-23,
127-161; source/q4rdna_sidecar_pack.cpp:23-47,223-245,289): a 48-byte header
``<8sIIIIIIQQ`` (magic "Q4RDNA1\\0", version 1, count, 64, 32, 1088, 0,
data_offset, data_bytes), ``count`` 96-byte entries ``<64sIIQQQ`` (name,
rows, columns, absolute offset, size, 0), zero padding up to
data_offset = align(48 + 96*count, 4096), then each tensor at a 256-byte
aligned offset with zero fill between tensors.
"""
from __future__ import annotations

import struct
from typing import Iterable

HEADER = struct.Struct("<8sIIIIIIQQ")
ENTRY = struct.Struct("<64sIIQQQ")
MAGIC = b"Q4RDNA1"
GROUP, TILE_ROWS, TILE_BYTES = 64, 32, 1088
DATA_ALIGNMENT = 4096
TENSOR_ALIGNMENT = 256

# One Qwen3-8B decoder block's linear tensors in the reference's order
# (source/pack_q4rdna_sidecar.py:25-33): (ggml suffix, rows = out, cols = in).
QWEN3_8B_LAYER = (
    ("attn_q.weight", 4096, 4096),
    ("attn_k.weight", 1024, 4096),
    ("attn_v.weight", 1024, 4096),
    ("attn_output.weight", 4096, 4096),
    ("ffn_gate.weight", 12288, 4096),
    ("ffn_up.weight", 12288, 4096),
    ("ffn_down.weight", 4096, 12288),
)


def qwen3_8b_stack(layers: int = 36):
    """(name, rows, cols) of the scoped tensors in layer-major order."""
    return [(f"blk.{layer}.{suffix}", rows, cols) for layer in range(layers) for suffix, rows, cols in QWEN3_8B_LAYER]


def _align(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def layout(tensors: Iterable[tuple[str, int, int]]):
    """(data_offset, [(name, rows, cols, offset, size)], end) of a sidecar."""
    tensors = list(tensors)
    data_offset = _align(HEADER.size + ENTRY.size * len(tensors), DATA_ALIGNMENT)
    offset = data_offset
    entries = []
    for name, rows, cols in tensors:
        if rows % TILE_ROWS or cols % GROUP:
            raise ValueError(f"unsupported Q4_RDNA shape {rows}x{cols} for {name}")
        if len(name.encode("ascii")) >= 64:
            raise ValueError(f"tensor name too long: {name}")
        size = rows * cols * 34 // GROUP
        entries.append((name, rows, cols, offset, size))
        offset = _align(offset + size, TENSOR_ALIGNMENT)
    return data_offset, entries, offset


def write_sidecar(path_or_file, tensors: Iterable[tuple[str, int, int, bytes]]) -> int:
    """Write (name, rows, cols, packed tile bytes) tensors; returns file size."""
    tensors = list(tensors)
    data_offset, entries, end = layout((n, r, c) for n, r, c, _ in tensors)
    own = isinstance(path_or_file, (str, bytes)) or hasattr(path_or_file, "__fspath__")
    f = open(path_or_file, "wb") if own else path_or_file
    try:
        f.write(HEADER.pack(MAGIC, 1, len(entries), GROUP, TILE_ROWS, TILE_BYTES, 0, data_offset, end - data_offset))
        for name, rows, cols, off, size in entries:
            f.write(ENTRY.pack(name.encode("ascii"), rows, cols, off, size, 0))
        pos = HEADER.size + ENTRY.size * len(entries)
        for (name, rows, cols, off, size), (_, _, _, data) in zip(entries, tensors):
            f.write(bytes(off - pos))
            data = bytes(data)
            if len(data) != size:
                raise ValueError(f"{name}: {len(data)} bytes, expected {size}")
            f.write(data)
            pos = off + size
        f.write(bytes(end - pos))
    finally:
        if own:
            f.close()
    return end


class SidecarWriter:
    """Streams a sidecar to disk: header and index first, then each tensor's
    packed tiles in index order (same bytes as :func:`write_sidecar`)."""

    def __init__(self, path, tensors: Iterable[tuple[str, int, int]]):
        self.data_offset, self.entries, self.end = layout(tensors)
        self._f = open(path, "wb")
        self._next = 0
        self._f.write(HEADER.pack(MAGIC, 1, len(self.entries), GROUP, TILE_ROWS, TILE_BYTES, 0, self.data_offset,
                                  self.end - self.data_offset))
        for name, rows, cols, off, size in self.entries:
            self._f.write(ENTRY.pack(name.encode("ascii"), rows, cols, off, size, 0))
        self._pos = HEADER.size + ENTRY.size * len(self.entries)

    def add(self, name: str, data) -> None:
        """Append the next tensor's packed bytes (index order)."""
        if self._next >= len(self.entries):
            raise ValueError("more tensors than the index holds")
        ename, rows, cols, off, size = self.entries[self._next]
        if name != ename:
            raise ValueError(f"expected {ename}, got {name}")
        data = memoryview(data).cast("B")
        if data.nbytes != size:
            raise ValueError(f"{name}: {data.nbytes} bytes, expected {size}")
        self._f.write(bytes(off - self._pos))
        self._f.write(data)
        self._pos = off + size
        self._next += 1

    def close(self) -> int:
        if self._f is None:
            return self.end
        try:
            if self._next != len(self.entries):
                raise ValueError(f"{len(self.entries) - self._next} tensors were not written")
            self._f.write(bytes(self.end - self._pos))
        finally:
            self._f.close()
            self._f = None
        return self.end

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        if exc[0] is None:
            self.close()
        elif self._f is not None:
            self._f.close()
            self._f = None
        return False
