"""Python harness over the C ABI, with torch tensors as device buffers.

Mirrors the reference's entry points (source/q4rdna.cuh:5-24): each GEMV
call returns True when it launched and False when the call is not
applicable (the reference's ``return false``: nothing was launched and the
caller should use its own path).  Errors raise :class:`Q4RdnaError`.
Launches are asynchronous on torch's current stream of the tensors' device.
"""
from __future__ import annotations

import ctypes
from typing import Iterable, Sequence

import torch

from . import _lib
from ._lib import (ALGO_SIDECAR, GLU_SWIGLU, GROUP, TILE_BYTES, TILE_ROWS, GemvDesc, LaunchOptions,
                   Q4RdnaError, Weight, check, load)


def packed_size(rows: int, cols: int) -> int:
    """Bytes of one packed tensor: rows*cols*34/64 (source/q4rdna.cu:149)."""
    return rows * cols * 34 // GROUP


def _stream(device: torch.device | int | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _f32_vec(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 CUDA tensor")
    return t


def _on_device(device: int, **tensors: torch.Tensor | None) -> None:
    """The weight's device is where the kernels read and write: a buffer on
    another device is refused here rather than passed by address."""
    for name, t in tensors.items():
        if t is not None and t.device.index != device:
            raise ValueError(f"{name} lives on cuda:{t.device.index}, the weight on cuda:{device}")


def _f32_buf(t: torch.Tensor, name: str, numel: int, device: int) -> torch.Tensor:
    """A device buffer the kernels read or write numel floats of: checked
    here, since the library sees only its address and a short or misplaced
    buffer would be read or written past its end on the GPU."""
    _f32_vec(t, name)
    if t.numel() != numel:
        raise ValueError(f"{name} holds {t.numel()} floats, {numel} are needed")
    if t.device.index != device:
        raise ValueError(f"{name} lives on cuda:{t.device.index}, the weight on cuda:{device}")
    return t


class QWeight:
    """A packed Q4_RDNA tensor resident on a GPU.

    ``tiles`` keeps the device buffer alive (a uint8 tensor of
    rows*cols*34/64 bytes) unless the weight views a sidecar's buffer, which
    the sidecar owns.
    """

    def __init__(self, raw: Weight, tiles: torch.Tensor | None = None, owner=None):
        self.raw = raw
        self.tiles = tiles
        self._owner = owner

    @classmethod
    def from_tiles(cls, tiles: torch.Tensor, rows: int, cols: int) -> "QWeight":
        if tiles.dtype != torch.uint8 or not tiles.is_cuda or not tiles.is_contiguous():
            raise ValueError("tiles must be a contiguous uint8 CUDA tensor")
        if tiles.numel() != packed_size(rows, cols):
            raise ValueError(f"tiles hold {tiles.numel()} bytes, {rows}x{cols} needs {packed_size(rows, cols)}")
        raw = Weight()
        check(load().q4rdna_weight_from_device(tiles.data_ptr(), rows, cols, tiles.device.index, ctypes.byref(raw)))
        return cls(raw, tiles)

    @property
    def rows(self) -> int:
        return self.raw.rows

    @property
    def cols(self) -> int:
        return self.raw.columns

    @property
    def device(self) -> int:
        return self.raw.device

    @property
    def nbytes(self) -> int:
        return packed_size(self.rows, self.cols)


def mul_mat(w: QWeight, x: torch.Tensor, y: torch.Tensor | None = None, stream: int | None = None):
    """y = W x.  Returns y, or None when the call is not applicable."""
    x = _f32_vec(x, "x")
    if y is None:
        y = torch.empty(w.rows, dtype=torch.float32, device=x.device)
    _f32_vec(y, "y")
    _on_device(w.device, x=x, y=y)
    s = _stream(x.device) if stream is None else stream
    ok = check(load().q4rdna_mul_mat(ctypes.byref(w.raw), x.data_ptr(), x.numel(), y.data_ptr(), y.numel(), s))
    return y if ok else None


def mul_mat_add(w: QWeight, x: torch.Tensor, add: torch.Tensor, y: torch.Tensor | None = None,
                stream: int | None = None):
    """y = W x + add.  Returns y, or None when not applicable."""
    x = _f32_vec(x, "x")
    add = _f32_vec(add, "add")
    if y is None:
        y = torch.empty(w.rows, dtype=torch.float32, device=x.device)
    _f32_vec(y, "y")
    _on_device(w.device, x=x, add=add, y=y)
    s = _stream(x.device) if stream is None else stream
    ok = check(load().q4rdna_mul_mat_add(ctypes.byref(w.raw), x.data_ptr(), x.numel(), add.data_ptr(), add.numel(),
                                         y.data_ptr(), y.numel(), s))
    return y if ok else None


def mul_mat_glu(up: QWeight, gate: QWeight, x: torch.Tensor, y: torch.Tensor | None = None,
                glu_op: int = GLU_SWIGLU, stream: int | None = None):
    """y = (W_up x) * silu(W_gate x).  Returns y, or None when not applicable."""
    x = _f32_vec(x, "x")
    if y is None:
        y = torch.empty(up.rows, dtype=torch.float32, device=x.device)
    _f32_vec(y, "y")
    _on_device(up.device, x=x, y=y)
    s = _stream(x.device) if stream is None else stream
    ok = check(load().q4rdna_mul_mat_glu(ctypes.byref(up.raw), ctypes.byref(gate.raw), x.data_ptr(), x.numel(),
                                         glu_op, y.data_ptr(), y.numel(), s))
    return y if ok else None


def mul_mat_ex(w: QWeight, x: torch.Tensor, y: torch.Tensor, gate: QWeight | None = None,
               add: torch.Tensor | None = None, split_k: int = 0, stream: int | None = None,
               kernel: int = _lib.KERNEL_POLICY) -> bool:
    """GEMV with explicit launch options: split_k (0 = the shape policy),
    kernel (KERNEL_VALU, or 0 = the policy, which is that kernel, or
    KERNEL_SEQUENTIAL: the reference's old mapping, split_k 0 or 1)."""
    _f32_buf(x, "x", w.cols, w.device)
    _f32_buf(y, "y", w.rows, w.device)
    if add is not None:
        _f32_buf(add, "add", w.rows, w.device)
    if gate is not None and (gate.rows, gate.cols) != (w.rows, w.cols):
        raise ValueError("gate and weight shapes differ")
    opts = LaunchOptions()
    opts.split_k = split_k
    opts.kernel = kernel
    s = _stream(x.device) if stream is None else stream
    return check(load().q4rdna_mul_mat_ex(ctypes.byref(w.raw), ctypes.byref(gate.raw) if gate else None,
                                          x.data_ptr(), _ptr(add), y.data_ptr(), ctypes.byref(opts), s))


def mul_mat_batch(w: QWeight, x: torch.Tensor, y: torch.Tensor, gate: QWeight | None = None,
                  add: torch.Tensor | None = None, split_k: int = 0, stream: int | None = None,
                  kernel: int = _lib.KERNEL_POLICY) -> bool:
    """n activation vectors against one weight, one launch: x [n][cols], y and
    add [n][rows] (contiguous float32 on the weight's device)."""
    if x.dim() != 2 or not x.is_contiguous() or x.dtype != torch.float32:
        raise ValueError("x must be a contiguous float32 [n, cols] tensor")
    if y.dim() != 2 or not y.is_contiguous() or y.dtype != torch.float32 or y.shape[0] != x.shape[0]:
        raise ValueError("y must be a contiguous float32 [n, rows] tensor")
    if x.shape[1] != w.cols or y.shape[1] != w.rows:
        raise ValueError("x / y shapes do not match the weight")
    if add is not None and (add.shape != y.shape or not add.is_contiguous() or add.dtype != torch.float32):
        raise ValueError("add must match y")
    for t, name in ((x, "x"), (y, "y"), (add, "add")):
        if t is not None and (not t.is_cuda or t.device.index != w.device):
            raise ValueError(f"{name} must live on the weight's device cuda:{w.device}")
    opts = LaunchOptions()
    opts.split_k = split_k
    opts.kernel = kernel
    s = _stream(x.device) if stream is None else stream
    return check(load().q4rdna_mul_mat_batch(ctypes.byref(w.raw), ctypes.byref(gate.raw) if gate else None,
                                             x.data_ptr(), x.shape[0], _ptr(add), y.data_ptr(),
                                             ctypes.byref(opts), s))


def mul_mat_group(items: Sequence[tuple], x: torch.Tensor, stream: int | None = None,
                  kernel: int = _lib.KERNEL_POLICY, split_k: int = 0) -> bool:
    """GEMVs sharing one activation x in one launch.  items: (weight, y) or
    (weight, y, gate_weight_or_None, add_or_None); every weight has
    x.numel() columns.  split_k: 0 = the shape policy for the group's total
    rows.  Returns False when not applicable."""
    if not 1 <= len(items) <= _lib.MAX_GROUP:
        raise ValueError(f"a group holds 1..{_lib.MAX_GROUP} GEMVs")
    descs = (_lib.GroupDesc * len(items))()
    for i, it in enumerate(items):
        w, y = it[0], it[1]
        gate = it[2] if len(it) > 2 else None
        add = it[3] if len(it) > 3 else None
        _f32_buf(x, "x", w.cols, w.device)
        _f32_buf(y, f"item {i} y", w.rows, w.device)
        if add is not None:
            _f32_buf(add, f"item {i} add", w.rows, w.device)
        if gate is not None and (gate.rows, gate.cols, gate.device) != (w.rows, w.cols, w.device):
            raise ValueError(f"item {i}: gate and weight differ in shape or device")
        descs[i].weight = w.raw
        descs[i].gate_tiles = gate.raw.tiles if gate is not None else None
        descs[i].add = _ptr(add)
        descs[i].y = y.data_ptr()
    opts = LaunchOptions()
    opts.kernel = kernel
    opts.split_k = split_k
    s = _stream(x.device) if stream is None else stream
    return check(load().q4rdna_mul_mat_group(descs, len(items), x.data_ptr(), x.numel(), ctypes.byref(opts), s))


def policy_split_k(rows: int, cols: int, device: int = 0) -> int:
    return load().q4rdna_policy_split_k(rows, cols, device)


def pack(w: torch.Tensor, algorithm: int = ALGO_SIDECAR, out: torch.Tensor | None = None,
         stream: int | None = None) -> torch.Tensor:
    """Quantize fp32 W [rows, cols] on the GPU into Q4_RDNA tiles (uint8)."""
    if w.dtype != torch.float32 or not w.is_cuda or not w.is_contiguous() or w.dim() != 2:
        raise ValueError("w must be a contiguous 2-D float32 CUDA tensor")
    rows, cols = w.shape
    if out is None:
        out = torch.empty(packed_size(rows, cols), dtype=torch.uint8, device=w.device)
    # The library sees only out's address: a short, mistyped or misplaced
    # buffer would be written past its end on the GPU.
    if out.dtype != torch.uint8 or not out.is_cuda or not out.is_contiguous():
        raise ValueError("out must be a contiguous uint8 CUDA tensor")
    if out.numel() != packed_size(rows, cols):
        raise ValueError(f"out holds {out.numel()} bytes, {rows}x{cols} packs into {packed_size(rows, cols)}")
    if out.device != w.device:
        raise ValueError(f"out lives on {out.device}, w on {w.device}")
    s = _stream(w.device) if stream is None else stream
    check(load().q4rdna_pack(w.data_ptr(), rows, cols, algorithm, out.data_ptr(), s))
    return out


def dequantize(w: QWeight, out: torch.Tensor | None = None, stream: int | None = None) -> torch.Tensor:
    """fp32 [rows, cols] = scale * code (the exact product)."""
    if out is None:
        out = torch.empty((w.rows, w.cols), dtype=torch.float32, device=torch.device("cuda", w.device))
    _f32_buf(out, "out", w.rows * w.cols, w.device)
    s = _stream(out.device) if stream is None else stream
    check(load().q4rdna_dequantize(ctypes.byref(w.raw), out.data_ptr(), s))
    return out


class Sidecar:
    """A sidecar file uploaded to one device (library-owned weights)."""

    def __init__(self, handle: int, device: int):
        self._h = ctypes.c_void_p(handle)
        self.device = device

    @classmethod
    def open(cls, path: str, device: int = 0) -> "Sidecar":
        h = ctypes.c_void_p()
        check(load().q4rdna_sidecar_open(path.encode(), device, ctypes.byref(h)))
        return cls(h.value, device)

    @classmethod
    def from_bytes(cls, image: bytes, device: int = 0) -> "Sidecar":
        h = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(image, len(image))
        check(load().q4rdna_sidecar_open_memory(ctypes.cast(buf, ctypes.c_void_p), len(image), device, ctypes.byref(h)))
        return cls(h.value, device)

    def close(self) -> None:
        if self._h is not None and self._h.value:
            load().q4rdna_sidecar_close(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return load().q4rdna_sidecar_count(self._h)

    def entries(self):
        L = load()
        out = []
        for i in range(len(self)):
            name = ctypes.create_string_buffer(64)
            r, c = ctypes.c_uint32(), ctypes.c_uint32()
            off, size = ctypes.c_uint64(), ctypes.c_uint64()
            check(L.q4rdna_sidecar_entry(self._h, i, name, ctypes.byref(r), ctypes.byref(c), ctypes.byref(off),
                                         ctypes.byref(size)))
            out.append((name.value.decode(), r.value, c.value, off.value, size.value))
        return out

    def find(self, name: str, ne0: int, ne1: int) -> QWeight | None:
        """Weight by ggml name with the ne0 = columns, ne1 = rows check."""
        raw = Weight()
        if not check(load().q4rdna_find(self._h, name.encode(), ne0, ne1, ctypes.byref(raw))):
            return None
        return QWeight(raw, owner=self)

    def hits(self, index: int) -> int:
        """GEMV launches that streamed entry `index` (q4rdna_sidecar_hits)."""
        return int(load().q4rdna_sidecar_hits(self._h, index))


def launch_count() -> int:
    """GEMV kernel launches made through the library (q4rdna_launch_count)."""
    return int(load().q4rdna_launch_count())


def report_stats() -> None:
    """The reference's launch report on stderr (q4rdna_report_stats)."""
    load().q4rdna_report_stats()


def inspect_sidecar(image: bytes, file_size: int | None = None) -> int:
    """Validate a sidecar header + index on the host; returns the entry count."""
    count = ctypes.c_uint32()
    buf = ctypes.create_string_buffer(bytes(image), len(image))
    check(load().q4rdna_sidecar_inspect(ctypes.cast(buf, ctypes.c_void_p), len(image),
                                        len(image) if file_size is None else file_size, ctypes.byref(count)))
    return count.value


def scope_allows(scope: str | None, name: str) -> bool:
    return bool(load().q4rdna_scope_allows(None if scope is None else scope.encode(), name.encode()))


class Plan:
    """A multi-tensor GEMV sweep launched as one kernel."""

    def __init__(self, items: Sequence[tuple], device: int = 0, batch: int = 1):
        """items: (weight, x, y) or (weight, x, y, gate_weight_or_None, add_or_None).

        batch > 1: each x holds `batch` activation vectors ([batch, cols],
        contiguous), y and add hold [batch, rows]."""
        descs = (GemvDesc * len(items))()
        self._keep = []
        for i, it in enumerate(items):
            w, x, y = it[0], it[1], it[2]
            gate = it[3] if len(it) > 3 else None
            add = it[4] if len(it) > 4 else None
            if w.device != device:
                raise ValueError(f"item {i}: the weight lives on cuda:{w.device}, the plan on cuda:{device}")
            _f32_buf(x, f"item {i} x", batch * w.cols, device)
            _f32_buf(y, f"item {i} y", batch * w.rows, device)
            if add is not None:
                _f32_buf(add, f"item {i} add", batch * w.rows, device)
            if gate is not None and (gate.rows, gate.cols, gate.device) != (w.rows, w.cols, w.device):
                raise ValueError(f"item {i}: gate and weight differ in shape or device")
            descs[i].weight = w.raw
            descs[i].gate_tiles = gate.raw.tiles if gate is not None else None
            descs[i].x = x.data_ptr()
            descs[i].add = _ptr(add)
            descs[i].y = y.data_ptr()
            self._keep.append(it)
        h = ctypes.c_void_p()
        check(load().q4rdna_plan_create_batch(descs, len(items), batch, device, ctypes.byref(h)))
        self._h = h
        self.device = device
        self.batch = batch

    @property
    def workgroups(self) -> int:
        return load().q4rdna_plan_workgroups(self._h)

    def launch(self, stream: int | None = None) -> bool:
        """prepare() + sweep() on one stream."""
        s = _stream(self.device) if stream is None else stream
        return check(load().q4rdna_plan_launch(self._h, s))

    def prepare(self, stream: int | None = None) -> bool:
        """Convert every activation into the plan's int8 digit buffers."""
        s = _stream(self.device) if stream is None else stream
        return check(load().q4rdna_plan_prepare(self._h, s))

    def sweep(self, stream: int | None = None) -> bool:
        """Run the GEMVs (after a prepare of the same activations)."""
        s = _stream(self.device) if stream is None else stream
        return check(load().q4rdna_plan_sweep(self._h, s))

    def close(self) -> None:
        if self._h is not None and self._h.value:
            load().q4rdna_plan_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
