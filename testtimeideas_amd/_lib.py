"""ctypes binding of ``libttt_attn.so`` (the C ABI in ``include/ttt_attn.h``).

This module is the thin layer between torch tensors and the HIP kernels:
it checks devices, dtypes and shapes, makes operands kernel-compatible
(unit stride in the last dimension, 16-byte aligned rows, head dim padded to
64 or 128), allocates outputs with torch's caching allocator, and calls the
C entry points on torch's current HIP stream.  There is no fallback: if the
library is missing or an operand is not on a ROCm device, it raises.

Every public function mirrors a launcher of the reference
(``ttt_kernels/backward_stubs.py`` and the forward in
``ttt_kernels/triton_attention.py``); see the docstrings for the lines.
"""
from __future__ import annotations

import contextlib
import ctypes
import dataclasses
import importlib.util
import os
from typing import Dict, List, Optional, Tuple

import torch

from . import autotune

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libttt_attn.so")
# torch binding of the three fused entry points (csrc/ttt_torch.cpp): the same
# C calls with the per-call Python work (views, outputs, workspace, stream)
# done in C++.  The per-kernel entry points and the launchers stay on ctypes.
EXT_PATH = os.path.join(_HERE, "_ttt_torch.so")

_DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


class ExtensionMissingError(RuntimeError):
    """libttt_attn.so has not been built (run ``__graft_entry__.build()``)."""


class _View(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_t", ctypes.c_int64),
    ]


class _Problem(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("scale", ctypes.c_float),
        ("split_chunk", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("window_kind", ctypes.c_int32),
        ("bias", _View),
        ("block_rows", ctypes.c_int32),
    ]


# ttt_window_kind (include/ttt_attn.h)
WINDOW_SLIDING, WINDOW_LOCAL = 0, 1


@dataclasses.dataclass(frozen=True)
class Mask:
    """Which scores a problem masks.

    causal: keys after the query are masked.  window (> 0, needs causal): a
    key window of kind WINDOW_SLIDING (query m sees keys m-W+1..m,
    cloud_ttt_e2e/ttt_e2e/utils.py:40-54) or WINDOW_LOCAL (the chunked loop
    of cloud_ttt_e2e/ttt_e2e/attention.py:111-128 as one problem).  bias: an
    additive score bias already in kernel layout (see ``prep_bias``), or None.
    """
    causal: bool = False
    window: int = 0
    window_kind: int = WINDOW_SLIDING
    bias: Optional[torch.Tensor] = None


def as_mask(m) -> Mask:
    """A Mask, given a Mask or a plain causal flag."""
    return m if isinstance(m, Mask) else Mask(causal=bool(m))


_P = ctypes.POINTER
_VP = _P(_View)
_FP = ctypes.c_void_p  # float* / workspace passed as an address
_WS = [_FP, ctypes.c_int64]  # workspace, workspace_bytes
_ST = [ctypes.c_void_p]  # stream
_SIGS = {
    "ttt_attn_fwd": [_P(_Problem), _VP, _VP, _VP, _VP, _FP, _VP] + _WS + _ST,
    "ttt_attn_bwd_dq": [_P(_Problem), _VP, _VP, _VP, _VP, _VP, _FP, _VP, _FP, _FP, _VP] + _WS + _ST,
    "ttt_attn_bwd_dkdv": [_P(_Problem), _VP, _VP, _VP, _VP, _FP, _VP, _FP, _VP, _VP] + _WS + _ST,
    "ttt_attn_bwd": [_P(_Problem), _VP, _VP, _VP, _VP, _VP, _FP, _VP, _FP, _VP, _VP, _VP] + _WS + _ST,
    "ttt_attn_bwd_rowsum": [_P(_Problem), _VP, _VP, _VP, _FP] + _ST,
    "ttt_attn_fill_masked_p": [_P(_Problem), _VP] + _ST,
    "ttt_attn_gg_row": [_P(_Problem), _VP, _VP, _VP, _VP, _FP, _VP, _FP, _VP, _VP, _VP, _VP, _VP, _VP, _FP,
                        _FP] + _WS + _ST,
    "ttt_attn_gg_col": [_P(_Problem), _VP, _VP, _VP, _VP, _FP, _VP, _FP, _FP, _FP, _VP, _VP, _VP, _VP, _VP]
                       + _WS + _ST,
    "ttt_attn_gg": [_P(_Problem), _VP, _VP, _VP, _VP, _FP, _VP, _FP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                    _FP, _FP] + _WS + _ST,
    "ttt_attn_gg_noalloc": [_P(_Problem), _VP, _VP, _VP, _VP, _FP, _VP, _FP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                            _VP] + _ST,
}

# ttt_entry codes (include/ttt_attn.h)
ENTRY_FWD, ENTRY_FWD_P, ENTRY_BWD_DQ, ENTRY_BWD_DKDV, ENTRY_BWD, ENTRY_GG_ROW, ENTRY_GG_COL, ENTRY_GG = range(8)

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libttt_attn.so once and bind the entry points' signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ExtensionMissingError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or `make -C testtimeideas_amd/csrc`)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.ttt_last_error.argtypes = []
    lib.ttt_last_error.restype = ctypes.c_char_p
    lib.ttt_version.argtypes = []
    lib.ttt_version.restype = ctypes.c_int
    lib.ttt_attn_workspace_size.argtypes = [_P(_Problem), ctypes.c_int32, ctypes.c_int32]
    lib.ttt_attn_workspace_size.restype = ctypes.c_int64
    lib.ttt_attn_split_info.argtypes = [_P(_Problem), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                        _P(ctypes.c_int32), _P(ctypes.c_int32), _P(ctypes.c_int64)]
    lib.ttt_attn_split_info.restype = ctypes.c_int
    lib.ttt_attn_launch_item.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P(ctypes.c_int32),
                                         _P(ctypes.c_int32)]
    lib.ttt_attn_launch_item.restype = ctypes.c_int
    lib.ttt_kernel_timing.argtypes = [ctypes.c_int32]
    lib.ttt_kernel_timing.restype = ctypes.c_int
    lib.ttt_kernel_timing_read.argtypes = [ctypes.c_int32, _P(ctypes.c_float), _P(ctypes.c_int32)]
    lib.ttt_kernel_timing_read.restype = ctypes.c_int
    _lib = lib
    return lib


_ext_mod = None


def ext():
    """The torch binding module (loaded once, after libttt_attn.so)."""
    global _ext_mod
    if _ext_mod is None:
        load()
        if not os.path.exists(EXT_PATH):
            raise ExtensionMissingError(
                f"{EXT_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        spec = importlib.util.spec_from_file_location("testtimeideas_amd._ttt_torch", EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _ext_mod = mod
    return _ext_mod


def _call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.ttt_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


# ---------------------------------------------------------------------------
# Optional per-kernel timing with HIP events on the launch stream.
# ---------------------------------------------------------------------------
_timing: Optional[Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event]]]] = None


@contextlib.contextmanager
def kernel_timing():
    """Record a (start, end) HIP event pair around every launch while active.

    Yields a dict ``name -> [(start, end), ...]``; call
    ``torch.cuda.synchronize()`` before reading elapsed times.  While timing
    is active, the fused entry points are issued as their per-kernel entry
    points so that each kernel is bracketed on its own.
    """
    global _timing
    prev = _timing
    _timing = {}
    try:
        yield _timing
    finally:
        _timing = prev


def _timed(name: str, *args) -> None:
    if _timing is None:
        _call(name, *args)
        return
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    _call(name, *args)
    e.record()
    _timing.setdefault(name, []).append((s, e))


def mean_ms(rec: Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event]]]) -> Dict[str, float]:
    return {k: sum(a.elapsed_time(b) for a, b in v) / len(v) for k, v in rec.items() if v}


# ---------------------------------------------------------------------------
# Operand preparation.
# ---------------------------------------------------------------------------
def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _view(t: Optional[torch.Tensor]):
    if t is None:
        return None
    s = t.stride()
    return ctypes.byref(_View(t.data_ptr(), s[0], s[1], s[2]))


def _fptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def padded_head_dim(d: int) -> int:
    if d <= 64:
        return 64
    if d <= 128:
        return 128
    raise NotImplementedError(f"head_dim {d} > 128 is not supported (the reference's kernels stop at 128 too)")


def _kernel_ok(t: torch.Tensor) -> bool:
    """The C ABI takes `t` as it is: unit last stride, a positive T stride (an
    operand expanded along T has stride 0 there and is copied), 16-byte
    aligned base and strides."""
    st = t.stride()
    if len(st) == 4 and st[3] == 1:
        # the common case in one pass: [B,H,T,D] with row-major strides
        b, h, n, d = t.shape
        if st[2] == d and st[1] == n * d and st[0] == h * n * d and d > 0:
            return (d * t.element_size()) % 16 == 0 and t.data_ptr() % 16 == 0
    if t.stride(-1) != 1 and t.size(-1) > 1:
        return False
    if t.stride(2) <= 0:
        return False
    eb = t.element_size()
    if t.data_ptr() % 16:
        return False
    return all((s * eb) % 16 == 0 for s in t.stride()[:-1])


def _ready(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """`t`, or a copy with fresh contiguous strides when the C ABI would not
    take it as it is (the torch binding does the same in C++ for its own
    calls; this is for the ctypes calls)."""
    if t is None or _kernel_ok(t):
        return t
    return t.clone(memory_format=torch.contiguous_format)


def prep(t: torch.Tensor, d_pad: int) -> torch.Tensor:
    """Return a [B,H,T,d_pad] tensor the kernels accept (copy only if needed)."""
    d = t.size(-1)
    if d != d_pad:
        out = t.new_zeros(t.shape[:-1] + (d_pad,))
        out[..., :d] = t
        return out
    if _kernel_ok(t):
        return t
    return t.contiguous()


def prep_rows(t: torch.Tensor, d_pad: int, front: int, back: int) -> torch.Tensor:
    """``prep`` plus `front` zero rows before and `back` zero rows after the T
    dimension (copies only when there is padding to add)."""
    if front == 0 and back == 0:
        return prep(t, d_pad)
    b, h, n, d = t.shape
    out = t.new_zeros((b, h, front + n + back, d_pad))
    out[:, :, front:front + n, :d] = t
    return out


def check_inputs(*ts: torch.Tensor) -> None:
    ref = ts[0]
    if ref.dim() != 4:
        raise ValueError(f"expected [B, H, T, D] tensors, got shape {tuple(ref.shape)}")
    if ref.device.type != "cuda":
        raise RuntimeError(
            "ttt_kernels runs on a ROCm GPU; got a tensor on device "
            f"'{ref.device}' (there is no CPU path)")
    if ref.dtype not in _DTYPE_CODE:
        raise TypeError(f"unsupported dtype {ref.dtype}; expected float16, bfloat16 or float32")
    for t in ts[1:]:
        if t.shape != ref.shape:
            raise ValueError(f"shape mismatch: {tuple(t.shape)} vs {tuple(ref.shape)}")
        if t.dtype != ref.dtype or t.device != ref.device:
            raise ValueError("all operands must share dtype and device")


# Tiles per workgroup of the split streamed loop; 0 lets the library choose.
_split_chunk = 0


@contextlib.contextmanager
def split_chunk(n: int):
    """Force the chunk length (tiles per workgroup) of every launch inside the
    block; used by tests to exercise the split/combine path at small sizes."""
    global _split_chunk
    prev = _split_chunk
    _split_chunk = int(n)
    try:
        yield
    finally:
        _split_chunk = prev


# Query rows per workgroup of the O + LSE forward (ttt_problem.block_rows);
# 0 lets the library (or the autotuner) choose.
_block_rows = 0


@contextlib.contextmanager
def block_rows(n: int):
    """Force the block height of the O + LSE forward (64, or 128 for 16-bit
    problems without a window or bias) inside the block; used by tests to
    run either kernel."""
    global _block_rows
    prev = _block_rows
    _block_rows = int(n)
    try:
        yield
    finally:
        _block_rows = prev


def _problem(x: torch.Tensor, mask, scale: float, split: Optional[int] = None, rows: int = 0) -> _Problem:
    b, h, t, d = x.shape
    m = as_mask(mask)
    bv = _View(None, 0, 0, 0)
    if m.bias is not None:
        s = m.bias.stride()
        bv = _View(m.bias.data_ptr(), s[0], s[1], s[2])
    return _Problem(_DTYPE_CODE[x.dtype], 1 if m.causal else 0, b, h, t, d, float(scale),
                    _split_chunk if split is None else int(split), int(m.window), int(m.window_kind), bv, int(rows))


def _split_for(entry: int, x: torch.Tensor, m, scale: float, load_p: bool, gdo: bool, run) -> int:
    """The split to launch kernel family `entry` with: a split forced by
    ``split_chunk``, else the autotuned one (``autotune``; `run(c)` launches
    the call with split c), else 0, the library's choice."""
    if _split_chunk or not autotune.enabled():
        return _split_chunk
    key = (entry, x.dtype, m.causal, tuple(x.shape), int(m.window), int(m.window_kind), m.bias is not None,
           bool(load_p), bool(gdo))

    def pick():
        pr = _problem(x, m, scale, 0)
        c0 = split_info(pr, entry, load_p, gdo)[0]
        pr.split_chunk = 1 << 30  # clipped to the longest walk
        return c0, split_info(pr, entry, load_p, gdo)[0]

    return autotune.chunk(key, pick, run)


def _fwd_config(x: torch.Tensor, m, scale: float, run) -> Tuple[int, int]:
    """(block_rows, split) of the O + LSE forward: (0, split_chunk) when a
    split is forced, (0, 0) -- the library's choice -- with tuning off, else
    the fastest of the library's choice and, for each block height the
    problem allows (64 rows; 128 for 16-bit types without a window or bias),
    the splits around that height's own pick, timed with `run((rows,
    split))`; (0, 0) again when the library's choice wins."""
    if _block_rows or _split_chunk or not autotune.enabled():
        return _block_rows, _split_chunk
    key = ("fwd_rows", x.dtype, m.causal, tuple(x.shape), int(m.window), int(m.window_kind), m.bias is not None)
    t = x.shape[2]
    pairs_ok = x.dtype != torch.float32 and m.bias is None and not (0 < int(m.window) < t)

    def options():
        opts = []
        for rows in ((64, 128) if pairs_ok else (64,)):
            pr = _problem(x, m, scale, 0, rows)
            c0 = split_info(pr, ENTRY_FWD, False)[0]
            pr.split_chunk = 1 << 30  # clipped to the longest walk
            lmax = split_info(pr, ENTRY_FWD, False)[0]
            for c in autotune.candidates(c0, lmax):
                pr.split_chunk = c
                ce = split_info(pr, ENTRY_FWD, False)[0]  # as launched (causal row pairs: even)
                if (rows, ce) not in opts:
                    opts.append((rows, ce))
        pr = _problem(x, m, scale, 0, 0)
        lib_rows = 128 if pairs_ok and x.shape[3] <= 64 else 64
        return (lib_rows, split_info(pr, ENTRY_FWD, False)[0]), opts

    return autotune.choose(key, options, run)


def prep_bias(bias: torch.Tensor, b: int, h: int, t: int, dtype: torch.dtype, device) -> torch.Tensor:
    """An additive score bias broadcastable to [b,h,t,t] as the kernels read
    it: `dtype` (the input dtype), an expanded [b,h,t,t] view whose broadcast
    dimensions have stride 0, unit column stride, 16-byte aligned base and
    strides, and rows readable up to t rounded up to 8 elements.  Copies only when the given
    tensor does not already satisfy this.  The bias receives no gradient."""
    x = bias.detach()
    if x.dtype != dtype:
        x = x.to(dtype)
    if x.device != torch.device(device):
        x = x.to(device)
    if x.dim() > 4:
        raise ValueError(f"attn_mask of shape {tuple(bias.shape)} does not broadcast to [B, H, T, T]")
    while x.dim() < 4:
        x = x.unsqueeze(0)
    try:
        full = x.expand(b, h, t, t)
    except RuntimeError as e:
        raise ValueError(f"attn_mask of shape {tuple(bias.shape)} does not broadcast to "
                         f"{(b, h, t, t)}") from e
    eb = x.element_size()
    tp = (t + ROW_READ - 1) // ROW_READ * ROW_READ
    if (full.stride(-1) == 1 and full.data_ptr() % 16 == 0
            and all((s * eb) % 16 == 0 for s in full.stride()[:3]) and _rows_readable(full)):
        return full
    keep = tuple(1 if x.size(i) == 1 else n for i, n in enumerate((b, h, t)))
    buf = torch.empty(keep + (tp,), dtype=x.dtype, device=x.device)
    buf[..., :t].copy_(x.expand(keep + (t,)))
    return buf[..., :t].expand(b, h, t, t)


_ws_sizes: Dict[tuple, int] = {}


def workspace_bytes(pr: _Problem, entry: int, gdo: bool = False) -> int:
    key = (pr.dtype, pr.causal, pr.batch, pr.heads, pr.seqlen, pr.head_dim, pr.split_chunk, pr.window,
           pr.window_kind, pr.bias.data is not None, entry, gdo)
    n = _ws_sizes.get(key)
    if n is None:
        n = int(load().ttt_attn_workspace_size(ctypes.byref(pr), entry, 1 if gdo else 0))
        if n < 0:
            raise RuntimeError(f"ttt_attn_workspace_size: {load().ttt_last_error().decode(errors='replace')}")
        _ws_sizes[key] = n
    return n


def _workspace(pr: _Problem, entry: int, device, gdo: bool = False):
    """(pointer, bytes, tensor) of a fresh workspace from torch's caching allocator."""
    n = workspace_bytes(pr, entry, gdo)
    if n == 0:
        return None, 0, None
    buf = torch.empty(n, dtype=torch.uint8, device=device)
    return buf.data_ptr(), n, buf


# The kernels read rows of P and of the bias in runs of 8 elements from
# multiples of 8, so a row is read up to T rounded up to 8 elements.
ROW_READ = 8


def _rows_readable(x: torch.Tensor) -> bool:
    """The last element the kernels read of a [B,H,T,N] operand (row T-1 of
    the last (b, h), column roundup(N, 8) - 1) lies inside its storage."""
    n = x.size(-1)
    span = (n + ROW_READ - 1) // ROW_READ * ROW_READ
    last = x.storage_offset() + sum((d - 1) * st for d, st in zip(x.shape[:-1], x.stride()[:-1])) + span
    return last * x.element_size() <= x.untyped_storage().nbytes()


def alloc_p(like: torch.Tensor) -> torch.Tensor:
    """[B,H,T,T] P buffer whose rows start on 16-byte boundaries and hold T
    rounded up to 8 elements."""
    b, h, t, _ = like.shape
    tp = (t + ROW_READ - 1) // ROW_READ * ROW_READ
    buf = torch.empty((b, h, t, tp), dtype=like.dtype, device=like.device)
    return buf if tp == t else buf[..., :t]


def _stats(like: torch.Tensor) -> torch.Tensor:
    b, h, t, _ = like.shape
    return torch.empty((b, h, t), dtype=torch.float32, device=like.device)


def prep_p(p: torch.Tensor) -> torch.Tensor:
    if p.stride(-1) == 1 and p.data_ptr() % 16 == 0 and all(
            (s * p.element_size()) % 16 == 0 for s in p.stride()[:-1]) and _rows_readable(p):
        return p
    out = alloc_p(p)
    out.copy_(p)
    return out


def _empty_like_out(x: torch.Tensor) -> torch.Tensor:
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


# ---------------------------------------------------------------------------
# Tensor-level entry points (inputs already padded and validated).  `mask` is
# a Mask, or a bool for a plain causal flag.
# ---------------------------------------------------------------------------
def _library_choice() -> bool:
    """Every launch takes the library's own split: nothing forced, no tuning,
    no per-kernel timing (the entry points then call the binding directly)."""
    return not _split_chunk and not _block_rows and _timing is None and not autotune.enabled()


def fwd(q, k, v, mask, scale: float, want_p: bool):
    """Forward: O, LSE and (save_p) P.  Reference: TritonAttentionFn.forward,
    ttt_kernels/triton_attention.py:261-337 (P path :51-59, :270-273)."""
    if q.numel() == 0:
        return _empty_like_out(q), _stats(q), alloc_p(q) if want_p else None
    m = as_mask(mask)
    if _library_choice():
        return tuple(ext().fwd(q, k, v, m.causal, float(scale), bool(want_p), 0, int(m.window), int(m.window_kind),
                               m.bias, 0))
    ent = ENTRY_FWD_P if want_p else ENTRY_FWD

    def run(c, rows=0):
        return ext().fwd(q, k, v, m.causal, float(scale), bool(want_p), c, int(m.window), int(m.window_kind), m.bias,
                         rows)

    if want_p:
        rows, c = 0, _split_for(ent, q, m, scale, want_p, False, run)
    else:
        rows, c = _fwd_config(q, m, scale, lambda rc: run(rc[1], rc[0]))
    if _timing is None:
        return tuple(run(c, rows))
    q, k, v = _ready(q), _ready(k), _ready(v)
    o = _empty_like_out(q)
    lse = _stats(q)
    p = alloc_p(q) if want_p else None
    pr = _problem(q, mask, scale, c, rows)
    wp, wn, _wbuf = _workspace(pr, ENTRY_FWD_P if want_p else ENTRY_FWD, q.device)
    _timed("ttt_attn_fwd", ctypes.byref(pr), _view(q), _view(k), _view(v), _view(o), lse.data_ptr(),
           _view(p), wp, wn, _stream())
    return o, lse, p


def bwd(q, k, v, o, do, lse, p, mask, scale: float):
    """First backward: dQ, dK, dV and the row statistic D = rowsum(dO o O).
    Reference: TritonAttentionFn.backward, triton_attention.py:351-379 and
    :416-420; launchers backward_stubs.py:154-181, 224-255, 362-425."""
    if q.numel() == 0:
        return _empty_like_out(q), _empty_like_out(k), _empty_like_out(v), _stats(q)
    m = as_mask(mask)
    lp = p is not None
    if _library_choice():
        return tuple(ext().bwd_fused(q, k, v, o, do, lse, p, m.causal, float(scale), int(m.window),
                                     int(m.window_kind), m.bias))

    def run(cq, ck):
        return ext().bwd(q, k, v, o, do, lse, p, m.causal, float(scale), cq, ck, int(m.window), int(m.window_kind),
                         m.bias)

    cq = _split_for(ENTRY_BWD_DQ, q, m, scale, lp, False, lambda c: run(c, 0))
    ck = _split_for(ENTRY_BWD_DKDV, q, m, scale, lp, False, lambda c: run(cq, c))
    if _timing is None:
        if cq == 0 and ck == 0:
            return tuple(ext().bwd_fused(q, k, v, o, do, lse, p, m.causal, float(scale), int(m.window),
                                         int(m.window_kind), m.bias))
        return tuple(run(cq, ck))
    q, k, v, o, do = _ready(q), _ready(k), _ready(v), _ready(o), _ready(do)
    dq = _empty_like_out(q)
    dk = _empty_like_out(k)
    dv = _empty_like_out(v)
    rowsum = _stats(q)
    st = _stream()
    lse_p = _fptr(lse)
    pq = _problem(q, mask, scale, cq)
    pk = _problem(q, mask, scale, ck)
    wp, wn, _wbuf = _workspace(pq, ENTRY_BWD_DQ, q.device)
    _timed("ttt_attn_bwd_dq", ctypes.byref(pq), _view(q), _view(k), _view(v), _view(o), _view(do), lse_p, _view(p),
           None, rowsum.data_ptr(), _view(dq), wp, wn, st)
    wp, wn, _wbuf2 = _workspace(pk, ENTRY_BWD_DKDV, q.device)
    _timed("ttt_attn_bwd_dkdv", ctypes.byref(pk), _view(q), _view(k), _view(v), _view(do), lse_p, _view(p),
           rowsum.data_ptr(), _view(dk), _view(dv), wp, wn, st)
    return dq, dk, dv, rowsum


def bwd_dq(q, k, v, do, p, lse, rowsum, mask, scale: float, o=None):
    """dQ alone (D from rowsum, or formed from O).  Reference: _attn_bwd_dq_kernel,
    backward_stubs.py:259-309."""
    dq = _empty_like_out(q)
    if q.numel() == 0:
        return dq
    prob = _problem(q, mask, scale)
    wp, wn, _wbuf = _workspace(prob, ENTRY_BWD_DQ, q.device)
    _timed("ttt_attn_bwd_dq", ctypes.byref(prob), _view(q), _view(k), _view(v), _view(o), _view(do),
           _fptr(lse), _view(p), _fptr(rowsum), None, _view(dq), wp, wn, _stream())
    return dq


def bwd_dkdv(q, k, v, do, p, lse, rowsum, mask, scale: float, want_dk: bool = True):
    """dK and dV (or dV alone).  Reference: backward_stubs.py:22-181, 313-359."""
    dk = _empty_like_out(do) if want_dk else None
    dv = _empty_like_out(do)
    if do.numel() == 0:
        return dk, dv
    prob = _problem(do, mask, scale)
    wp, wn, _wbuf = _workspace(prob, ENTRY_BWD_DKDV, do.device)
    _timed("ttt_attn_bwd_dkdv", ctypes.byref(prob), _view(q), _view(k), _view(v), _view(do), _fptr(lse),
           _view(p), _fptr(rowsum), _view(dk), _view(dv), wp, wn, _stream())
    return dk, dv


def fill_masked_p(p, mask) -> None:
    """Zero the tiles of a forward's P that the forward leaves unwritten
    (causal: past the diagonal; window: before the first visible key), so P
    holds the softmax everywhere, as the reference's P kernel writes it
    (ttt_kernels/triton_attention.py:208-256)."""
    m = as_mask(mask)
    if not m.causal or p.numel() == 0:
        return
    b, h, t, _ = p.shape
    like = torch.empty((b, h, t, 64), dtype=p.dtype, device="meta")
    pr = ctypes.byref(_problem(like, m, 1.0))
    _timed("ttt_attn_fill_masked_p", pr, _view(p), _stream())


def rowsum_from_p(p, do, v, mask):
    """rowsum = sum_n P o (dO V^T).  Reference: backward_stubs.py:184-255."""
    rs = _stats(do)
    if do.numel() == 0:
        return rs
    pr = ctypes.byref(_problem(do, mask, 1.0))
    _timed("ttt_attn_bwd_rowsum", pr, _view(p), _view(do), _view(v), rs.data_ptr(), _stream())
    return rs


def gg(q, k, v, do, lse, p, rowsum, gq, gk, gv, mask, scale: float, want_gdo: bool, dq=None):
    """Double backward: (GQ, GK, GV, GdO or None).  `dq`: the first
    backward's dQ for the same inputs (``bwd``'s first output), or None; given,
    the row pass reads it instead of forming one of its products (GQ agrees
    to rounding).  Reference stubs backward_stubs.py:539-548; torch version
    :434-514 (corrected)."""
    if q.numel() == 0:
        return (_empty_like_out(q), _empty_like_out(k), _empty_like_out(v),
                _empty_like_out(do) if want_gdo else None)
    m = as_mask(mask)
    lp = p is not None
    if dq is not None:
        if dq.shape != q.shape or dq.dtype != q.dtype or dq.device != q.device:
            raise ValueError(f"dq: expected the shape, dtype and device of q {tuple(q.shape)}, got "
                             f"{tuple(dq.shape)} {dq.dtype} {dq.device}")
    if _library_choice():
        return tuple(ext().gg_fused(q, k, v, do, lse, p, rowsum, dq, gq, gk, gv, m.causal, float(scale),
                                    bool(want_gdo), int(m.window), int(m.window_kind), m.bias))

    def run(cr, cc):
        return ext().gg(q, k, v, do, lse, p, rowsum, dq, gq, gk, gv, m.causal, float(scale), bool(want_gdo), cr,
                        cc, int(m.window), int(m.window_kind), m.bias)

    cr = _split_for(ENTRY_GG_ROW, q, m, scale, lp, want_gdo, lambda c: run(c, 0))
    cc = _split_for(ENTRY_GG_COL, q, m, scale, lp, False, lambda c: run(cr, c))
    if _timing is None:
        if cr == 0 and cc == 0:
            return tuple(ext().gg_fused(q, k, v, do, lse, p, rowsum, dq, gq, gk, gv, m.causal, float(scale),
                                        bool(want_gdo), int(m.window), int(m.window_kind), m.bias))
        return tuple(run(cr, cc))
    q, k, v, do, dq, gq, gk, gv = (_ready(t) for t in (q, k, v, do, dq, gq, gk, gv))
    gq_out = _empty_like_out(q)
    gk_out = _empty_like_out(k)
    gv_out = _empty_like_out(v)
    gdo = _empty_like_out(do) if want_gdo else None
    e = _stats(q)
    f = _stats(q)
    st = _stream()
    lse_p = _fptr(lse)
    prr = _problem(q, mask, scale, cr)
    prc = _problem(q, mask, scale, cc)
    wp, wn, _wbuf = _workspace(prr, ENTRY_GG_ROW, q.device, want_gdo)
    _timed("ttt_attn_gg_row", ctypes.byref(prr), _view(q), _view(k), _view(v), _view(do), lse_p, _view(p),
           rowsum.data_ptr(), _view(dq), _view(gq), _view(gk), _view(gv), _view(gq_out), _view(gdo),
           e.data_ptr(), f.data_ptr(), wp, wn, st)
    wp, wn, _wbuf2 = _workspace(prc, ENTRY_GG_COL, q.device)
    _timed("ttt_attn_gg_col", ctypes.byref(prc), _view(q), _view(k), _view(v), _view(do), lse_p, _view(p),
           rowsum.data_ptr(), e.data_ptr(), f.data_ptr(), _view(gq), _view(gk), _view(gv), _view(gk_out),
           _view(gv_out), wp, wn, st)
    return gq_out, gk_out, gv_out, gdo


def gg_noalloc(q, k, v, do, lse, p, rowsum, gq, gk, gv, mask, scale: float, want_gdo: bool, dq=None):
    """``gg`` through ttt_attn_gg_noalloc: the library's static device scratch
    instead of a workspace and E/F buffers (outputs are still allocated
    here); `dq` as in ``gg``.  No counterpart in the reference."""
    gq_out = _empty_like_out(q)
    gk_out = _empty_like_out(k)
    gv_out = _empty_like_out(v)
    gdo = _empty_like_out(do) if want_gdo else None
    if q.numel() == 0:
        return gq_out, gk_out, gv_out, gdo
    prob = _problem(q, mask, scale)
    _timed("ttt_attn_gg_noalloc", ctypes.byref(prob), _view(q), _view(k), _view(v), _view(do), _fptr(lse),
           _view(p), rowsum.data_ptr(), _view(dq), _view(gq), _view(gk), _view(gv), _view(gq_out), _view(gk_out),
           _view(gv_out), _view(gdo), _stream())
    return gq_out, gk_out, gv_out, gdo


def split_info(pr: _Problem, entry: int, load_p: bool, gdo: bool = False) -> Tuple[int, int, int]:
    """(tiles per workgroup, chunks of the longest block, workgroup slots) the
    library would use for `entry` on the current device."""
    c, n, sl = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    _call("ttt_attn_split_info", ctypes.byref(pr), entry, 1 if load_p else 0, 1 if gdo else 0, ctypes.byref(c),
          ctypes.byref(n), ctypes.byref(sl))
    return c.value, n.value, sl.value


def launch_item(nblk: int, chunk: int, column: int) -> Tuple[int, int]:
    """(block, chunk index) that grid column `column` of a split plain-causal
    slice runs (block -1: none)."""
    b, c = ctypes.c_int32(), ctypes.c_int32()
    _call("ttt_attn_launch_item", nblk, chunk, column, ctypes.byref(b), ctypes.byref(c))
    return b.value, c.value


# ttt_kernel codes (include/ttt_attn.h): the main kernels per-kernel timing tells apart
KERNELS = ("fwd_online", "fwd_stats", "fwd_p", "bwd_dq", "bwd_dkdv", "gg_row", "gg_col")


@contextlib.contextmanager
def launch_timing(capacity: int = 4096):
    """Time every main-kernel launch inside the block with HIP events on its
    stream (ttt_kernel_timing), whichever entry point launches it, fused ones
    included.  Yields a function returning {kernel: (mean ms, launches)};
    call it after the work has been issued (it waits for the events)."""
    _call("ttt_kernel_timing", capacity)

    def read() -> Dict[str, Tuple[float, int]]:
        out = {}
        ms, n = ctypes.c_float(), ctypes.c_int32()
        for i, name in enumerate(KERNELS):
            _call("ttt_kernel_timing_read", i, ctypes.byref(ms), ctypes.byref(n))
            if n.value:
                out[name] = (ms.value, n.value)
        return out

    try:
        yield read
    finally:
        _call("ttt_kernel_timing", 0)


def exported_symbols() -> List[str]:
    """Names of the C entry points this binding uses (for ABI checks)."""
    return list(_SIGS) + ["ttt_last_error", "ttt_version", "ttt_attn_workspace_size", "ttt_attn_split_info",
                          "ttt_attn_launch_item", "ttt_kernel_timing", "ttt_kernel_timing_read"]
