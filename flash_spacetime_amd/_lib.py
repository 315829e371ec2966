"""ctypes binding of the gfx950 HIP library (include/flash_spacetime.h).

The library is built in-tree by `python -m flash_spacetime_amd.build` (or
`__graft_entry__.build()`). There is no fallback: when the shared library is
missing or no ROCm GPU is present, every operator raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libflash_spacetime.so"

FST_BF16 = 0
FST_F32 = 1
FST_ATTN_BIAS = 1
FST_ACT_BIAS = 2
FST_PACKED = 4
FST_TOKEN_MAJOR = 8
FST_QKV_INTERLEAVED = 16
# Plan bits (include/flash_spacetime.h): one group per kernel knob, at most
# one bit of a group set.
FST_PLAN_FWD_OCC2 = 1 << 8
FST_PLAN_FWD_OCC3 = 1 << 9
FST_PLAN_ROWS_W4 = 1 << 10
FST_PLAN_ROWS_W8 = 1 << 11
FST_PLAN_COLS_OCC2 = 1 << 12
FST_PLAN_COLS_OCC3 = 1 << 13
FST_PLAN_ROWS_W8X2 = 1 << 14
FST_PLAN_ROWS_KV_REG = 1 << 15
FST_PLAN_ROWS_KV_LDS = 1 << 16
FST_PLAN_FWD_KC16 = 1 << 17
FST_PLAN_FWD_KC32 = 1 << 18
FST_PLAN_FWD_T16 = 1 << 19
FST_PLAN_FWD_T32 = 1 << 20
FST_PLAN_FWD_T64 = 1 << 21
FST_PLAN_BWD_T16 = 1 << 22
FST_PLAN_BWD_T32 = 1 << 23
FST_PLAN_BWD_T64 = 1 << 24
FST_PLAN_BWD_KC16 = 1 << 25
FST_PLAN_BWD_KC32 = 1 << 26
FST_PLAN_BWD_PASS1 = 1 << 27
FST_PLAN_BWD_PASS2 = 1 << 28
FST_PLAN_FWD_W8 = 1 << 29
FST_PLAN_BWD_W8 = 1 << 30
FST_PLAN_MASK = 0x7FFFFF00

FST_PHASE_WORKLIST = 1
FST_PHASE_FWD = 2
FST_PHASE_BWD_ROWS = 4
FST_PHASE_BWD_COLS = 8
FST_PHASE_REDUCE = 16
FST_FWD_ALL = FST_PHASE_WORKLIST | FST_PHASE_FWD
FST_BWD_ALL = FST_PHASE_WORKLIST | FST_PHASE_BWD_ROWS | FST_PHASE_BWD_COLS | FST_PHASE_REDUCE

FST_OK = 0
FST_EINVAL = -1
FST_EUNSUPPORTED = -2
FST_EWORKSPACE = -3
FST_ELAUNCH = -4

# Every symbol the C header declares, with its ctypes signature.
_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "fst_supported": (_i, [_i, _i, _i, _i]),
    "fst_plans": (_i, [_i, _i, _i, _i]),
    "fst_plan_supported": (_i, [_i, _i, _i, _i, _i]),
    "fst_forward_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i, _i]),
    "fst_forward": (
        _i,
        [_i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _sz, _vp],
    ),
    "fst_forward_noalloc": (
        _i,
        [_i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp],
    ),
    "fst_backward_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i, _i]),
    "fst_backward": (
        _i,
        [_i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "fst_forward_phases": (
        _i,
        [_i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _sz, _vp],
    ),
    "fst_backward_phases": (
        _i,
        [_i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "fst_max_event_len": (_i, [_i, _i, _i, _i, _i]),
    "fst_frequencies": (None, [_i, ctypes.POINTER(ctypes.c_float)]),
    "fst_last_error": (ctypes.c_char_p, []),
    "fst_version": (ctypes.c_char_p, []),
}

_LIB = None


class LibraryMissing(RuntimeError):
    """The HIP library has not been built (run flash_spacetime_amd.build)."""


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library with typed signatures."""
    global _LIB
    if _LIB is None:
        path = Path(os.environ.get("FST_LIBRARY", LIB_PATH))
        if not path.exists():
            raise LibraryMissing(
                f"{path} not found: build it with `python -m flash_spacetime_amd.build`"
            )
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def last_error() -> str:
    return load().fst_last_error().decode()


def check(rc: int, what: str) -> None:
    """Map a C status code onto the Python exception the reference raises."""
    if rc == FST_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc in (FST_EINVAL, FST_EUNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            "flash-spacetime runs on the GPU only: the HIP kernels need device tensors "
            f"(got a tensor on {t.device}); there is no CPU path"
        )


def frequencies(c: int) -> torch.Tensor:
    """The fp32 ladder the kernels embed with (host-side, no GPU needed)."""
    buf = (ctypes.c_float * (c // 2))()
    load().fst_frequencies(c, buf)
    return torch.tensor(list(buf), dtype=torch.float32)
