"""Measured choice of kernel variants ("plans") per problem shape.

The kernels are compiled in variants (the FST_PLAN_* bits of
include/flash_spacetime.h, one group of bits per kernel knob; `plans` lists
the bits compiled for a shape and `_lib.fst_plan_supported` whether one
combination is):

* bf16 forward: two or three workgroups per CU, 16- or 32-key chunks;
* bf16 backward rows kernel: four waves, eight waves in one workgroup per CU,
  or eight waves in two; K and V of a key chunk in registers or in LDS;
* bf16 backward cols kernel: two or three workgroups per CU;
* float32 forward: 16, 32 or 64 query rows per workgroup, 16- or 32-key
  chunks; float32 backward: 16, 32 or 64 rows (keys) per workgroup and
  16- or 32-key (row) chunks, for the rows and cols kernels together, and
  one or two passes of the rows kernel over the keys.

Without tuning the library runs its static choice per (dtype, H, D, C). With
tuning on, the first call of a shape times every supported combination of
each kernel's groups and the static choice on the caller's own inputs, and
later calls of that shape run the fastest where it beats the static choice
by 3 % or more (timings vary by a few per cent from run to run), else the
static choice.

The occupancy, wave, K/V-staging and tile-height variants leave out, lse,
dq, dk, dv and rowsum unchanged bit for bit (dW and db change only in the
order their fp32 partial sums are added); the key-chunk and pass variants
agree with the static choice to rounding. A shape is keyed by the GPU architecture, the
library version, kind, dtype, H, D, C, the layout and bias flags, and the
bit lengths of its batch and length (padded) or token count (packed), so the
ragged batches of one training run share a choice.

The reference's Triton kernels take fixed tile constants
(src/flash_spacetime/_tiles.py) and are not autotuned (README.md:86-95); its
launchers' block_m / block_n / num_warps arguments are mapped onto these
groups by `plan_from_tiles`.
"""

from __future__ import annotations

import contextlib
import contextvars
import fcntl
import itertools
import json
import os
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib

# Plan-bit groups of each kernel (at most one bit of a group per plan).
_FWD_GROUPS = ((_lib.FST_PLAN_FWD_OCC2, _lib.FST_PLAN_FWD_OCC3),
               (_lib.FST_PLAN_FWD_KC16, _lib.FST_PLAN_FWD_KC32),
               (_lib.FST_PLAN_FWD_T16, _lib.FST_PLAN_FWD_T32, _lib.FST_PLAN_FWD_T64, _lib.FST_PLAN_FWD_W8))
_ROWS_GROUPS = ((_lib.FST_PLAN_ROWS_W4, _lib.FST_PLAN_ROWS_W8, _lib.FST_PLAN_ROWS_W8X2),
                (_lib.FST_PLAN_ROWS_KV_REG, _lib.FST_PLAN_ROWS_KV_LDS))
_COLS_GROUPS = ((_lib.FST_PLAN_COLS_OCC2, _lib.FST_PLAN_COLS_OCC3),)
# float32 backward groups: they set the rows and the cols kernel together.
_BWD_GROUPS = ((_lib.FST_PLAN_BWD_T16, _lib.FST_PLAN_BWD_T32, _lib.FST_PLAN_BWD_T64, _lib.FST_PLAN_BWD_W8),
               (_lib.FST_PLAN_BWD_KC16, _lib.FST_PLAN_BWD_KC32),
               (_lib.FST_PLAN_BWD_PASS1, _lib.FST_PLAN_BWD_PASS2))


def _bits(groups: Sequence[Sequence[int]]) -> int:
    return sum(b for g in groups for b in g)


_FWD_BITS = _bits(_FWD_GROUPS)
_BWD_ALL_BITS = _bits(_ROWS_GROUPS) | _bits(_COLS_GROUPS) | _bits(_BWD_GROUPS)
_KEY_FLAGS = (_lib.FST_ATTN_BIAS | _lib.FST_ACT_BIAS | _lib.FST_PACKED | _lib.FST_TOKEN_MAJOR
              | _lib.FST_QKV_INTERLEAVED)

_enabled = os.environ.get("FST_AUTOTUNE", "0") == "1"
_reps = 3
_cache: Dict[Tuple, int] = {}
_fixed: Optional[int] = None
# FST_AUTOTUNE_CACHE=<path>: choices are loaded from that JSON file (when it
# exists) on the first tuned call and merged into it after every new choice,
# under a lock, so the processes of a training job time each shape once and
# none overwrites another's choices.
_cache_path: Optional[str] = os.environ.get("FST_AUTOTUNE_CACHE") or None
_cache_loaded = False
# (block_m, block_n, num_warps) of the launcher call in progress, if given.
_tiles: contextvars.ContextVar = contextvars.ContextVar("fst_tiles", default=None)


def set_autotune(enabled: bool, reps: int = 3) -> None:
    """Turn the measured plan choice on or off; `reps` timed runs per variant.
    Off, every call runs the static choice (choices made while it was on are
    kept for when it is turned on again)."""
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


@contextlib.contextmanager
def tile_request(block_m: Optional[int] = None, block_n: Optional[int] = None, num_warps: Optional[int] = None):
    """The launchers' tile arguments for the calls inside the block: each
    call takes `plan_from_tiles` of them instead of the tuned or static
    choice (and of a fixed_plan). None everywhere changes nothing."""
    for name, value in (("block_m", block_m), ("block_n", block_n), ("num_warps", num_warps)):
        if value is not None and (not isinstance(value, int) or isinstance(value, bool) or value < 1):
            raise ValueError(f"{name} must be a positive int or None, got {value!r}")
    if block_m is None and block_n is None and num_warps is None:
        yield
        return
    token = _tiles.set((block_m, block_n, num_warps))
    try:
        yield
    finally:
        _tiles.reset(token)


def _tiled(kind: str, dims: Tuple[int, ...]) -> Optional[int]:
    req = _tiles.get()
    return None if req is None else plan_from_tiles(dims[0], dims[3], dims[6], dims[7], kind, *req)


def plans(dtype: int, heads: int, dim: int, channels: int) -> int:
    """The FST_PLAN_* bits compiled for a shape (0: one static variant only)."""
    return int(_lib.load().fst_plans(dtype, heads, dim, channels))


def plan_supported(dtype: int, heads: int, dim: int, channels: int, plan: int) -> bool:
    """Whether this combination of plan bits is compiled for the shape."""
    return bool(_lib.load().fst_plan_supported(dtype, heads, dim, channels, plan))


def chosen() -> Dict[Tuple, int]:
    """The plans chosen so far: shape key -> FST_PLAN_* bits."""
    return dict(_cache)


def clear() -> None:
    _cache.clear()


def save(path: str) -> None:
    """Merge the chosen plans into a JSON file (keys as lists): under an
    exclusive lock on `path`.lock the file is read, this process's choices
    are added (a choice made here wins), and the result replaces the file in
    one rename, so a reader never sees a partial file and concurrent writers
    lose nothing."""
    with open(f"{path}.lock", "a") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        try:
            merged: Dict[Tuple, int] = {}
            if os.path.exists(path):
                merged.update(_read(path))
            merged.update(_cache)
            tmp = f"{path}.{os.getpid()}.tmp"
            with open(tmp, "w") as fh:
                json.dump([[list(k), v] for k, v in merged.items()], fh)
            os.replace(tmp, path)
        finally:
            fcntl.flock(lock, fcntl.LOCK_UN)


def _read(path: str) -> Dict[Tuple, int]:
    with open(path) as fh:
        return {tuple(key): int(value) for key, value in json.load(fh)}


def load(path: str) -> None:
    """Add the plans of a JSON file written by `save` (a later choice wins)."""
    _cache.update(_read(path))


def _build_id() -> Tuple[str, str]:
    """(GPU architecture, library version) of this process's device and build:
    a choice timed elsewhere does not apply here."""
    arch = "cpu"
    if torch.cuda.is_available():
        arch = getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", "gpu")
    version = _lib.load().fst_version()
    return arch, version.decode() if isinstance(version, bytes) else str(version)


def shape_key(kind: str, dims: Tuple[int, ...], build: Optional[Tuple[str, str]] = None) -> Tuple:
    """Key of a call: the build (architecture, library version; this
    process's when not given), kind ("fwd" / "bwd"), dtype, H, D, C, layout
    and bias flags, and the bit lengths of (B, L) padded or (T, B) packed."""
    dtype, flags, batch, heads, length, tokens, dim, channels = dims
    size = (tokens.bit_length(), batch.bit_length()) if flags & _lib.FST_PACKED else \
        (batch.bit_length(), length.bit_length())
    return (*(build or _build_id()), kind, dtype, heads, dim, channels, flags & _KEY_FLAGS) + size


def _combos(dims: Tuple[int, ...], groups: Sequence[Sequence[int]]) -> List[int]:
    """Every supported combination of one offered bit per group (groups the
    shape offers nothing in stay empty)."""
    dtype, heads, dim, chans = dims[0], dims[3], dims[6], dims[7]
    mask = plans(dtype, heads, dim, chans)
    choices = [[b for b in g if mask & b] or [0] for g in groups]
    out = []
    for combo in itertools.product(*choices):
        plan = sum(combo)
        if plan and plan_supported(dtype, heads, dim, chans, plan):
            out.append(plan)
    return out


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
    """The plan bits of the fastest variant, or 0 (the static choice) unless
    some variant beats it by the margin."""
    if not cands:
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
    return not torch.cuda.is_current_stream_capturing()


def forward_plan(dims: Tuple[int, ...], run: Callable[[int], int]) -> int:
    """Plan bits for a forward call; `run(flags)` launches the whole forward
    with those flags (dims[1] plus plan bits) and returns the status."""
    tiled = _tiled("fwd", dims)
    if tiled is not None:
        return tiled
    if _fixed is not None:
        return _fixed & _FWD_BITS
    if not _enabled:
        return 0
    key = shape_key("fwd", dims)
    known = _lookup(key)
    if known is not None:
        return known if plan_supported(dims[0], dims[3], dims[6], dims[7], known) else 0
    if not _usable():
        return 0
    choice = _fastest(run, _combos(dims, _FWD_GROUPS), dims[1], "flash_spacetime_forward (tuning)")
    _record(key, choice)
    return choice


def backward_plan(dims: Tuple[int, ...], run: Callable[[int, int], int]) -> int:
    """Plan bits for a backward call; `run(phases, flags)` launches those
    phases of the backward with those flags and returns the status. The
    float32 groups, which set both kernels and their rows per workgroup, are
    timed over the two together, each run with its own work list; then the
    rows kernel's groups (after one work-list phase for the plan so far), then
    the cols kernel's, which reads what the rows kernel wrote. The caller's
    own launch follows with the chosen plan."""
    tiled = _tiled("bwd", dims)
    if tiled is not None:
        return tiled
    if _fixed is not None:
        return _fixed & _BWD_ALL_BITS
    if not _enabled:
        return 0
    key = shape_key("bwd", dims)
    known = _lookup(key)
    if known is not None:
        return known if plan_supported(dims[0], dims[3], dims[6], dims[7], known) else 0
    if not _usable():
        return 0
    what = "flash_spacetime_backward (tuning)"
    rows, cols, both = (_combos(dims, g) for g in (_ROWS_GROUPS, _COLS_GROUPS, _BWD_GROUPS))
    # The float32 groups change the rows per workgroup, which the work list
    # is built for: each of their timed runs builds its own.
    plan = _fastest(lambda f: run(_lib.FST_PHASE_WORKLIST | _lib.FST_PHASE_BWD_ROWS | _lib.FST_PHASE_BWD_COLS, f),
                    both, dims[1], what)
    if rows or cols:
        _lib.check(run(_lib.FST_PHASE_WORKLIST, dims[1] | plan), what)
    r = _fastest(lambda f: run(_lib.FST_PHASE_BWD_ROWS, f), rows, dims[1] | plan, what)
    plan |= r
    if cols and not rows:  # the cols kernel reads the rows kernel's scratch
        _lib.check(run(_lib.FST_PHASE_BWD_ROWS, dims[1] | plan), what)
    c = _fastest(lambda f: run(_lib.FST_PHASE_BWD_COLS, f), cols, dims[1] | plan, what)
    plan |= c
    _record(key, plan)
    return plan


def plan_from_tiles(dtype: int, heads: int, dim: int, channels: int, kind: str,
                    block_m: Optional[int] = None, block_n: Optional[int] = None,
                    num_warps: Optional[int] = None) -> Optional[int]:
    """Plan bits for the reference launchers' tile arguments, or None when
    none is given (the library's choice, tuned or static).

    block_m (query rows per program) selects the tile height of the float32
    kernels (16, 32, 64 rows per workgroup); the bf16 tile kernels have one
    height, 16 rows. block_n (keys per inner step) selects the key chunk of
    the forward (16 or 32) and of the float32 backward. num_warps selects the
    bf16 rows kernel's waves per workgroup (4, or 8 in two workgroups per CU
    where offered, else in one) and, for float32, the waves of a 16-row
    tile (4, or 8 where offered; the 32- and 64-row tiles have four waves).
    Each takes the offered value nearest the request (the smaller on a tie),
    and a combination the shape does not compile drops num_warps, then
    block_n, then block_m, in that order. num_stages has no counterpart: the
    kernels' loads run one chunk ahead."""
    if block_m is None and block_n is None and num_warps is None:
        return None
    mask = plans(dtype, heads, dim, channels)
    fwd = kind == "fwd"

    def nearest(value: Optional[int], options: Sequence[Tuple[int, int]]) -> int:
        offered = [(v, b) for v, b in options if mask & b]
        if value is None or not offered:
            return 0
        return min(offered, key=lambda vb: (abs(vb[0] - value), vb[0]))[1]

    m_opts = ((16, _lib.FST_PLAN_FWD_T16), (32, _lib.FST_PLAN_FWD_T32), (64, _lib.FST_PLAN_FWD_T64)) if fwd else \
        ((16, _lib.FST_PLAN_BWD_T16), (32, _lib.FST_PLAN_BWD_T32), (64, _lib.FST_PLAN_BWD_T64))
    n_opts = ((16, _lib.FST_PLAN_FWD_KC16), (32, _lib.FST_PLAN_FWD_KC32)) if fwd else \
        ((16, _lib.FST_PLAN_BWD_KC16), (32, _lib.FST_PLAN_BWD_KC32))
    m, n = nearest(block_m, m_opts), nearest(block_n, n_opts)
    if dtype == _lib.FST_F32:
        # num_warps refines the tile-height group: eight waves replace the
        # 16-row bit, four waves pick it where no height was asked for.
        t16, w8 = (_lib.FST_PLAN_FWD_T16, _lib.FST_PLAN_FWD_W8) if fwd else \
            (_lib.FST_PLAN_BWD_T16, _lib.FST_PLAN_BWD_W8)
        w = nearest(num_warps, ((4, t16), (8, w8)))
        mw = w8 if w == w8 and m in (0, t16) else (t16 if w == t16 and m == 0 else m)
        candidates = [mw + n, m + n, m]
    else:
        w8 = _lib.FST_PLAN_ROWS_W8X2 if mask & _lib.FST_PLAN_ROWS_W8X2 else _lib.FST_PLAN_ROWS_W8
        w_opts = () if fwd else ((4, _lib.FST_PLAN_ROWS_W4), (8, w8))
        candidates = [m + n + nearest(num_warps, w_opts), m + n, m]
    for plan in candidates:
        if plan == 0 or plan_supported(dtype, heads, dim, channels, plan):
            return plan
    return 0


_NAMES = ((_lib.FST_PLAN_FWD_OCC2, "fwd:occ2"), (_lib.FST_PLAN_FWD_OCC3, "fwd:occ3"),
          (_lib.FST_PLAN_FWD_KC16, "fwd:kc16"), (_lib.FST_PLAN_FWD_KC32, "fwd:kc32"),
          (_lib.FST_PLAN_FWD_T16, "fwd:t16"), (_lib.FST_PLAN_FWD_T32, "fwd:t32"),
          (_lib.FST_PLAN_FWD_T64, "fwd:t64"), (_lib.FST_PLAN_FWD_W8, "fwd:w8"),
          (_lib.FST_PLAN_ROWS_W4, "rows:w4"), (_lib.FST_PLAN_ROWS_W8, "rows:w8"),
          (_lib.FST_PLAN_ROWS_W8X2, "rows:w8x2"), (_lib.FST_PLAN_ROWS_KV_REG, "rows:kvreg"),
          (_lib.FST_PLAN_ROWS_KV_LDS, "rows:kvlds"),
          (_lib.FST_PLAN_COLS_OCC2, "cols:occ2"), (_lib.FST_PLAN_COLS_OCC3, "cols:occ3"),
          (_lib.FST_PLAN_BWD_T16, "bwd:t16"), (_lib.FST_PLAN_BWD_T32, "bwd:t32"),
          (_lib.FST_PLAN_BWD_T64, "bwd:t64"), (_lib.FST_PLAN_BWD_KC16, "bwd:kc16"),
          (_lib.FST_PLAN_BWD_KC32, "bwd:kc32"), (_lib.FST_PLAN_BWD_PASS1, "bwd:pass1"),
          (_lib.FST_PLAN_BWD_PASS2, "bwd:pass2"), (_lib.FST_PLAN_BWD_W8, "bwd:w8"))


def plan_names(plan: int) -> Optional[str]:
    """Readable form of plan bits ("fwd:occ3 rows:w8 cols:occ2")."""
    names = [name for bit, name in _NAMES if plan & bit]
    return " ".join(names) if names else None
