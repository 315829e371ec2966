"""Measured choice of kernel variants ("plans") per problem shape.

The bf16 kernels are compiled in variants that compute every output row
with the same arithmetic and differ only in their register and LDS budget:
two or three workgroups per CU for the forward and the backward cols
kernel, four or eight waves per workgroup for the backward rows kernel
(the FST_PLAN_* bits of include/flash_spacetime.h; `fst_plans` lists the
ones compiled for a shape). Without tuning the library runs its static
choice per (H, D, C). With tuning on, the first call of a shape times every
compiled variant of each kernel and the static choice on the caller's own
inputs, and later calls of that shape run the fastest variant where it
beats the static choice by 3 % or more (timings vary by a few per cent
from run to run), else the static choice.

out, lse, dq, dk, dv and rowsum are the same for every plan; dW and db
depend on the rows plan only through the order in which fp32 partial sums
are added. A shape is keyed by dtype, H, D, C, the layout and bias flags,
and the bit lengths of its batch and length (padded) or token count
(packed), so the ragged batches of one training run share a choice.

The reference's Triton kernels take fixed tile constants
(src/flash_spacetime/_tiles.py) and are not autotuned (README.md:86-95).
"""

from __future__ import annotations

import contextlib
import json
import os
from typing import Callable, Dict, Iterable, List, Optional, Tuple

import torch

from . import _lib

_FWD_BITS = (_lib.FST_PLAN_FWD_OCC2, _lib.FST_PLAN_FWD_OCC3)
_ROWS_BITS = (_lib.FST_PLAN_ROWS_W4, _lib.FST_PLAN_ROWS_W8)
_COLS_BITS = (_lib.FST_PLAN_COLS_OCC2, _lib.FST_PLAN_COLS_OCC3)
_KEY_FLAGS = (_lib.FST_ATTN_BIAS | _lib.FST_ACT_BIAS | _lib.FST_PACKED | _lib.FST_TOKEN_MAJOR
              | _lib.FST_QKV_INTERLEAVED)

_enabled = os.environ.get("FST_AUTOTUNE", "0") == "1"
_reps = 3
_cache: Dict[Tuple, int] = {}
_fixed: Optional[int] = None
# FST_AUTOTUNE_CACHE=<path>: choices are loaded from that JSON file (when it
# exists) on first use and written back after every new choice, so the
# processes of a training job time each shape once.
_cache_path: Optional[str] = os.environ.get("FST_AUTOTUNE_CACHE") or None
_cache_loaded = False


def set_autotune(enabled: bool, reps: int = 3) -> None:
    """Turn the measured plan choice on or off; `reps` timed runs per variant."""
    global _enabled, _reps
    if reps < 1:
        raise ValueError("reps must be at least 1")
    _enabled = bool(enabled)
    _reps = int(reps)


def autotune_enabled() -> bool:
    return _enabled


@contextlib.contextmanager
def fixed_plan(bits: int):
    """Run every call inside the block with these FST_PLAN_* bits (each call
    takes the bits of the kernels it launches), bypassing the timing and the
    cache. Bits a shape does not have make its calls raise ValueError."""
    global _fixed
    if bits & ~_lib.FST_PLAN_MASK:
        raise ValueError(f"not plan bits: {bits:#x}")
    prev, _fixed = _fixed, int(bits)
    try:
        yield
    finally:
        _fixed = prev


def plans(dtype: int, heads: int, dim: int, channels: int) -> int:
    """The FST_PLAN_* bits compiled for a shape (0: one static variant only)."""
    return int(_lib.load().fst_plans(dtype, heads, dim, channels))


def chosen() -> Dict[Tuple, int]:
    """The plans chosen so far: shape key -> FST_PLAN_* bits."""
    return dict(_cache)


def clear() -> None:
    _cache.clear()


def save(path: str) -> None:
    """Write the chosen plans to a JSON file (keys as lists), replacing it in
    one rename so a reader never sees a partial file."""
    tmp = f"{path}.{os.getpid()}.tmp"
    with open(tmp, "w") as fh:
        json.dump([[list(k), v] for k, v in _cache.items()], fh)
    os.replace(tmp, path)


def load(path: str) -> None:
    """Add the plans of a JSON file written by `save` (a later choice wins)."""
    with open(path) as fh:
        for key, value in json.load(fh):
            _cache[tuple(key)] = int(value)


def shape_key(kind: str, dims: Tuple[int, ...]) -> Tuple:
    """Key of a call: kind ("fwd" / "bwd"), dtype, H, D, C, layout and bias
    flags, and the bit lengths of (B, L) padded or (T, B) packed."""
    dtype, flags, batch, heads, length, tokens, dim, channels = dims
    size = (tokens.bit_length(), batch.bit_length()) if flags & _lib.FST_PACKED else \
        (batch.bit_length(), length.bit_length())
    return (kind, dtype, heads, dim, channels, flags & _KEY_FLAGS) + size


def _candidates(mask: int, bits: Iterable[int]) -> List[int]:
    return [b for b in bits if mask & b]


def _time_ms(run: Callable[[int], int], plan: int, what: str) -> float:
    _lib.check(run(plan), what)  # first launch of the variant, untimed
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(_reps):
        _lib.check(run(plan), what)
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / _reps


# A variant replaces the static choice only when it is this much faster:
# timings of one kernel vary by a few per cent from run to run.
_MARGIN = 0.97


def _fastest(run: Callable[[int], int], cands: List[int], base: int, what: str) -> int:
    """The plan bits of the fastest variant, or 0 (the static choice, which is
    one of the variants) unless some variant beats it by the margin."""
    if len(cands) < 2:
        return 0
    times = {c: float("inf") for c in [0, *cands]}
    for _ in range(3):  # interleaved rounds; the minimum drops a cold first one
        for c in times:
            times[c] = min(times[c], _time_ms(run, base | c, what))
    best = min(cands, key=lambda c: (times[c], c))
    return best if times[best] < _MARGIN * times[0] else 0


def _record(key: Tuple, plan: int) -> None:
    _cache[key] = plan
    if _cache_path:
        save(_cache_path)


def _lookup(key: Tuple) -> Optional[int]:
    global _cache_loaded
    if _cache_path and not _cache_loaded:
        _cache_loaded = True
        if os.path.exists(_cache_path):
            load(_cache_path)
    return _cache.get(key)


def _usable() -> bool:
    # No timing (which synchronises) while the caller captures a graph.
    return _enabled and not torch.cuda.is_current_stream_capturing()


def forward_plan(dims: Tuple[int, ...], run: Callable[[int], int]) -> int:
    """Plan bits for a forward call; `run(flags)` launches the whole forward
    with those flags (dims[1] plus plan bits) and returns the status."""
    if _fixed is not None:
        return _fixed & sum(_FWD_BITS)
    key = shape_key("fwd", dims)
    known = _lookup(key)
    if known is not None or not _usable():
        # a file written by another build may name variants this one lacks
        return known & plans(dims[0], dims[3], dims[6], dims[7]) if known else 0
    cands = _candidates(plans(dims[0], dims[3], dims[6], dims[7]), _FWD_BITS)
    choice = _fastest(run, cands, dims[1], "flash_spacetime_forward (tuning)")
    _record(key, choice)
    return choice


def backward_plan(dims: Tuple[int, ...], run: Callable[[int, int], int]) -> int:
    """Plan bits for a backward call; `run(phases, flags)` launches those
    phases of the backward with those flags and returns the status. The rows
    kernel is timed first (after one work-list phase), then the cols kernel,
    which reads what the rows kernel wrote; the caller's own launch follows
    with the chosen plan."""
    if _fixed is not None:
        return _fixed & sum(_ROWS_BITS + _COLS_BITS)
    key = shape_key("bwd", dims)
    known = _lookup(key)
    if known is not None or not _usable():
        return known & plans(dims[0], dims[3], dims[6], dims[7]) if known else 0
    mask = plans(dims[0], dims[3], dims[6], dims[7])
    rows, cols = _candidates(mask, _ROWS_BITS), _candidates(mask, _COLS_BITS)
    what = "flash_spacetime_backward (tuning)"
    if len(rows) > 1 or len(cols) > 1:
        _lib.check(run(_lib.FST_PHASE_WORKLIST, dims[1]), what)
    r = _fastest(lambda f: run(_lib.FST_PHASE_BWD_ROWS, f), rows, dims[1], what)
    if len(cols) > 1 and len(rows) < 2:  # the cols kernel reads the rows kernel's scratch
        _lib.check(run(_lib.FST_PHASE_BWD_ROWS, dims[1] | r), what)
    c = _fastest(lambda f: run(_lib.FST_PHASE_BWD_COLS, f), cols, dims[1] | r, what)
    _record(key, r | c)
    return r | c


def plan_names(plan: int) -> Optional[str]:
    """Readable form of plan bits ("fwd:occ3 rows:w8 cols:occ2")."""
    names = []
    for bit, name in ((_lib.FST_PLAN_FWD_OCC2, "fwd:occ2"), (_lib.FST_PLAN_FWD_OCC3, "fwd:occ3"),
                      (_lib.FST_PLAN_ROWS_W4, "rows:w4"), (_lib.FST_PLAN_ROWS_W8, "rows:w8"),
                      (_lib.FST_PLAN_COLS_OCC2, "cols:occ2"), (_lib.FST_PLAN_COLS_OCC3, "cols:occ3")):
        if plan & bit:
            names.append(name)
    return " ".join(names) if names else None
