"""MI355X (gfx950) Q4_RDNA group-64 dequant-GEMV: Python harness.

The compute lives in ``libq4rdna_gfx950.so`` (hand-written HIP kernels behind
the C ABI of ``include/q4rdna.h``); this package binds it with ctypes.
"""
from ._lib import (ALGO_ABSMAX, ALGO_MSE, ALGO_RANGE, ALGO_SIDECAR, ERR_ARGUMENT, ERR_FORMAT, ERR_HIP, ERR_IO,
                   ERR_MEMORY, EXPORTS, GLU_SWIGLU, GROUP, LIB_PATH, NOT_APPLICABLE, OK, TILE_BYTES, TILE_ROWS,
                   Q4RdnaError, last_error, load)
from .build import build
from .sidecar import QWEN3_8B_LAYER, qwen3_8b_stack, write_sidecar

__all__ = [
    "ALGO_ABSMAX", "ALGO_MSE", "ALGO_RANGE", "ALGO_SIDECAR", "ERR_ARGUMENT", "ERR_FORMAT", "ERR_HIP", "ERR_IO",
    "ERR_MEMORY", "EXPORTS", "GLU_SWIGLU", "GROUP", "LIB_PATH", "NOT_APPLICABLE", "OK", "TILE_BYTES", "TILE_ROWS",
    "Q4RdnaError", "last_error", "load", "build", "QWEN3_8B_LAYER", "qwen3_8b_stack", "write_sidecar",
]


def __getattr__(name):
    # The torch-dependent API is imported on first use so the CPU-only pieces
    # (format constants, sidecar writer, build) load without torch.
    import importlib
    api = importlib.import_module(__name__ + ".api")
    if name == "api":
        return api
    if hasattr(api, name):
        return getattr(api, name)
    raise AttributeError(name)
