"""Measured choice of the split (tiles per workgroup) of each kernel family,
and of the block height (64 or 128 query rows per workgroup, which also sets
the waves per SIMD and LDS buffer sets of the kernel that runs) of the O + LSE
forward.

The library picks a split by simulating the launch (csrc/ttt_capi.hip,
``choose_split``).  With autotuning on, the first call of a kernel family on a
given problem shape instead times the library's pick and a few splits around
it on the call's own operands, and keeps the fastest for every later call of
that shape, as the reference's Triton kernels pick their tile configuration
per shape with ``triton.autotune`` (ttt_kernels/triton_attention.py:78-85,
keyed on the sequence length and head dim).

Off by default: a different split changes the fp32 summation order of the
split partials, so results stay bitwise repeatable only for a fixed split, and
a measured choice may differ between runs.  ``enable()`` or the environment
variable ``TTT_AUTOTUNE=1`` turns it on.  Tuning synchronizes the device
(HIP events) and is skipped while a HIP graph is being captured; the library's
own pick is used then.
"""
from __future__ import annotations

import os
from typing import Callable, Dict, List, Tuple

import torch

_enabled = os.environ.get("TTT_AUTOTUNE", "0") not in ("", "0")
_cache: Dict[tuple, object] = {}
# Splits tried around the library's pick c0: c0 * these, and no split at all.
_FACTORS = (0.5, 0.75, 1.25, 1.5, 2.0)
_MIN_CHUNK = 4  # the library's smallest split (kMinChunk)
_REPS = 3


def enable(on: bool = True) -> None:
    global _enabled
    _enabled = bool(on)


def enabled() -> bool:
    return _enabled


def clear() -> None:
    _cache.clear()


def choices() -> Dict[tuple, object]:
    """The choices so far: {(family, shape key): tiles per workgroup, or
    (block rows, tiles) for the O + LSE forward}, 0 / (0, 0) where the
    library's own pick won."""
    return dict(_cache)


def candidates(c0: int, lmax: int) -> List[int]:
    """The library's pick c0 first, then the splits around it and the whole
    walk (lmax tiles: no split), each within [min(4, lmax), lmax], without
    repeats."""
    lo = min(_MIN_CHUNK, lmax)
    out: List[int] = []
    for c in [c0] + [int(round(c0 * f)) for f in _FACTORS] + [lmax]:
        c = max(lo, min(lmax, c))
        if c not in out:
            out.append(c)
    return out


def _capturing() -> bool:
    return torch.cuda.is_current_stream_capturing()


def _time(run: Callable[[int], None], c: int) -> float:
    run(c)  # warm-up (and first-use setup) outside the timed launches
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(_REPS):
        run(c)
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / _REPS


def choose(key: tuple, options: Callable[[], Tuple[tuple, List[tuple]]], run: Callable[[tuple], None]) -> tuple:
    """A kernel configuration beyond the split (for the O + LSE forward:
    (block rows, split)): the cached choice, or the fastest of the candidate
    configurations timed with `run(cfg)` on the current stream.  `options()`
    gives (the library's own configuration, the candidates, which include
    it); (0, 0), meaning the library's choice, is returned when tuning is
    off, a graph is being captured, or the library's own configuration
    wins."""
    if not _enabled or _capturing():
        return (0, 0)
    c = _cache.get(key)
    if c is not None:
        return c
    lib, cands = options()
    if lib not in cands:
        cands = [lib] + cands
    if len(cands) == 1:
        best = cands[0]
    else:
        times = [(_time(run, cfg), i, cfg) for i, cfg in enumerate(cands)]
        best = min(times)[2]
    best = (0, 0) if best == lib else best
    _cache[key] = best
    return best


def chunk(key: tuple, pick: Callable[[], Tuple[int, int]], run: Callable[[int], None]) -> int:
    """The split to launch family/shape `key` with: 0 (the library's choice)
    when tuning is off or a graph is being captured; otherwise the cached
    choice, or the fastest of ``candidates`` timed with `run(c)` on the
    current stream, with 0 again when that is the library's own pick (the
    same launches, and the fused entry points, which take the library's
    splits, stay usable).  `pick()` gives (the library's split, the longest
    walk in tiles)."""
    if not _enabled:
        return 0
    c = _cache.get(key)
    if c is not None:
        return c
    if _capturing():
        return 0
    c0, lmax = pick()
    cands = candidates(c0, lmax)
    if len(cands) == 1:
        best = cands[0]
    else:
        times = [(_time(run, c), i, c) for i, c in enumerate(cands)]
        best = min(times)[2]
    if best == cands[0]:
        best = 0
    _cache[key] = best
    return best
