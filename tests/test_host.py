"""Host-side logic on the CPU: the C ABI library loads and exports every
declared symbol, argument validation fails before anything is enqueued,
workspace sizing, the roofline model, the bwd_mode registry, the number of
launches per grad-grad step, and the C1 golden fixture."""
import ctypes
import importlib
import os
import re

import numpy as np
import pytest
import torch

from testtimeideas_amd import _lib, workloads

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "ttt_attn.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(ttt_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert "ttt_attn_fwd" in names and "ttt_attn_gg" in names
    for n in names:
        assert hasattr(lib, n), n
    assert set(_lib.exported_symbols()) == set(names)
    assert lib.ttt_version() >= 200


def test_ctypes_signatures_match_header():
    """Each ctypes argument list of _lib has as many parameters as the
    header's declaration of that entry point."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, args in _lib._SIGS.items():
        m = re.search(r"\b" + name + r"\s*\(([^)]*)\)\s*;", text)
        assert m, name
        assert len(m.group(1).split(",")) == len(args), name


def test_torch_binding_loads():
    """The torch binding of the fused entry points is built next to the
    library and exposes them (no call: there is no GPU here)."""
    mod = _lib.ext()
    assert os.path.dirname(mod.__file__) == os.path.dirname(_lib.LIB_PATH)
    for name in ("fwd", "bwd", "gg"):
        assert callable(getattr(mod, name))


def _prob(**kw):
    d = dict(dtype=0, causal=1, batch=1, heads=1, seqlen=128, head_dim=64, scale=0.125, split_chunk=0, window=0,
             window_kind=0, block_rows=0)
    d.update(kw)
    pr = _lib._Problem(d["dtype"], d["causal"], d["batch"], d["heads"], d["seqlen"], d["head_dim"],
                       d["scale"], d["split_chunk"], d["window"], d["window_kind"])
    pr.block_rows = d["block_rows"]
    return pr


def _v(addr=0x10000, st=64):
    return ctypes.byref(_lib._View(addr, 128 * st, 128 * st, st))


def _fwd_rc(pr, q=None, ws=None, wsn=0, p=None):
    lib = _lib.load()
    q = q if q is not None else _v()
    return lib.ttt_attn_fwd(ctypes.byref(pr), q, _v(), _v(), _v(), 0x20000, p, ws, wsn, None)


def test_validation_errors_without_gpu():
    lib = _lib.load()
    # unsupported head dim / dtype
    assert _fwd_rc(_prob(head_dim=96)) == 2
    assert b"head_dim" in lib.ttt_last_error()
    assert _fwd_rc(_prob(dtype=7)) == 2
    # bad sizes
    assert _fwd_rc(_prob(seqlen=0)) == 1
    assert _fwd_rc(_prob(batch=70000)) == 1
    # null and misaligned operands
    assert lib.ttt_attn_fwd(ctypes.byref(_prob()), None, _v(), _v(), _v(), 0x20000, None, None, 0, None) == 1
    assert _fwd_rc(_prob(), q=_v(addr=0x10002)) == 1
    assert b"aligned" in lib.ttt_last_error()
    assert _fwd_rc(_prob(), q=_v(st=60)) == 1
    # a split problem without a workspace
    big = _prob(seqlen=8192)
    assert _lib.workspace_bytes(big, _lib.ENTRY_FWD) > 0
    assert _fwd_rc(big) == 4
    assert b"workspace" in lib.ttt_last_error()
    # rowsum missing for dK
    assert lib.ttt_attn_bwd_dkdv(ctypes.byref(_prob()), _v(), _v(), _v(), _v(), 0x20000, None, None, _v(), _v(),
                                 None, 0, None) == 1


def _slice_workgroups(n, c, causal):
    """Workgroups of one (b,h) slice with chunks of c tiles, by brute force."""
    return sum(-(-ln // c) for ln in (range(1, n + 1) if causal else [n] * n))


def _visible(t, causal, window=0, kind=0):
    """[T, T] bool: query i sees key j, from the mask definitions (a window
    of T or more is none)."""
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    vis = np.ones((t, t), bool) if not causal else j <= i
    if 0 < window < t:
        lo = i - window + 1 if kind == 0 else np.minimum(t, (i // window + 1) * window) - window
        vis = vis & (j >= lo)
    return vis


def _block_tiles(t, causal, window=0, kind=0, col=False):
    """Streamed tiles of each block in launch order, by brute force: the
    span between the first and last tile holding a visible pair (row kernels
    issue the last row block first when causal)."""
    vis = _visible(t, causal, window, kind)
    nblk = -(-t // 64)
    out = []
    for i in range(nblk):
        b = i if col or not causal else nblk - 1 - i
        strip = vis[:, b * 64:(b + 1) * 64] if col else vis[b * 64:(b + 1) * 64, :]
        hit = strip.any(axis=1 if col else 0)
        tiles = sorted({n // 64 for n in np.nonzero(hit)[0]})
        out.append(tiles[-1] - tiles[0] + 1)
    return out


def _grid_order(lens, c, longest_first):
    """(block, chunk) run by each grid column of a slice, None where a column
    runs nothing.  Chunk index by chunk index, blocks in launch order; with
    `longest_first` (plain causal) every full chunk that way first, then the
    blocks' shorter last chunks by length, longest first, ties in launch
    order."""
    k = -(-max(lens) // c)
    cols = len(lens) * k
    if not longest_first or k == 1:
        return [(b, ch) if ch * c < lens[b] else None for ch in range(k) for b in range(len(lens))]
    full = [(b, ch) for ch in range(k) for b in range(len(lens)) if lens[b] - ch * c >= c]
    last = sorted(((b, lens[b] // c) for b in range(len(lens)) if lens[b] % c), key=lambda it: -(lens[it[0]] % c))
    return full + last + [None] * (cols - len(full) - len(last))


def test_kernel_timing_validation():
    """ttt_kernel_timing rejects a capacity past 65536 and
    ttt_kernel_timing_read an unknown kernel; capacity 0 (off) always
    succeeds, and with nothing timed a read reports no launches."""
    lib = _lib.load()
    assert lib.ttt_kernel_timing(70000) == 1 and b"capacity" in lib.ttt_last_error()
    assert lib.ttt_kernel_timing(0) == 0
    ms, n = ctypes.c_float(1.0), ctypes.c_int32(7)
    assert lib.ttt_kernel_timing_read(len(_lib.KERNELS), ctypes.byref(ms), ctypes.byref(n)) == 1
    assert lib.ttt_kernel_timing_read(5, ctypes.byref(ms), ctypes.byref(n)) == 0 and n.value == 0


def test_launch_order_longest_first():
    """ttt_attn_launch_item (the kernels' causal_item) against the order
    written out directly, exhaustively for small slices: each chunk of each
    block exactly once, full chunks first, then the last chunks longest
    first, columns past them empty."""
    for n in range(1, 70):
        lens = [n - b for b in range(n)]
        for c in range(1, n + 3):
            want = _grid_order(lens, c, True)
            got = [_lib.launch_item(n, c, x) for x in range(len(want))]
            assert got == [(-1, 0) if w is None else w for w in want], (n, c)
    with pytest.raises(RuntimeError):
        _lib.launch_item(8, 3, 8 * 3)


def _xcd_local(x, gx):
    """Column x's item in a grid of gx columns whose slices do not spread
    evenly over the 8 XCDs: within each full group of 64 columns, the XCD of
    column x (x mod 8) takes 8 consecutive items, the XCDs in reverse order
    in odd groups; a last partial group keeps its order."""
    grp = x // 64
    if (grp + 1) * 64 > gx:
        return x
    r = x % 64
    k = r % 8
    return grp * 64 + 8 * (7 - k if grp % 2 else k) + r // 8


def _simulated_chunk(nblk, causal, bh, slots, min_chunk=4, lengths=None, longest_first=None):
    """Independent restatement of the library's split chooser: list-schedule
    the grid (x = block + nblk*chunk, y = b*h; blocks in launch order with
    `lengths` tiles, by default nblk..1 when causal) onto `slots` workgroup
    slots spread round-robin over 8 XCDs (slice y to XCD y % 8 when b*h is a
    multiple of 8; otherwise, when column x of every slice runs on XCD x % 8
    (one slice, or a grid width that is a multiple of 8), column x runs the
    item of _xcd_local(x)), cost =
    makespan + 0.015 per non-empty workgroup, each non-empty workgroup taking
    its tiles + 0.5 and an empty one 0.05, plus 8 for any split.  Blocks are
    split only while they fill fewer than the slots (twice the slots when
    causal)."""
    import heapq

    lens = lengths or ([nblk - b for b in range(nblk)] if causal else [nblk] * nblk)
    lmax = max(lens)
    if longest_first is None:
        longest_first = causal and lengths is None

    def cost(c):
        per = max(1, slots // 8)
        heaps = [[0.0] * per for _ in range(8)]
        end, used, idx = 0.0, 0, 0
        order = _grid_order(lens, c, longest_first)
        if bh % 8 and (bh == 1 or len(order) % 8 == 0):
            order = [order[_xcd_local(x, len(order))] for x in range(len(order))]
        for y in range(bh):
            for item in order:
                t = 0 if item is None else min(c, lens[item[0]] - item[1] * c)
                h = heaps[y % 8 if bh % 8 == 0 else idx % 8]
                f = heapq.heappop(h) + (t + 0.5 if t else 0.05)
                heapq.heappush(h, f)
                end, used, idx = max(end, f), used + (t > 0), idx + 1
        return end + 0.015 * used

    if bh * nblk >= (2 if causal else 1) * slots:
        return lmax
    best_c, best = lmax, cost(lmax)
    c = min(min_chunk, lmax)
    while c < lmax:
        if bh * sum(-(-ln // c) for ln in lens) <= 16 * slots:
            v = cost(c) + 8.0
            if v < best:
                best_c, best = c, v
        c = c + 1 if c < 64 else c + max(1, c // 32)
    return best_c


def _simulated_pair_chunk(nblk, causal, bh, slots):
    """The split of the O + LSE forward over row-block pairs (16-bit, d64, no
    window or bias): the same chooser over npair = ceil(nblk/2) pairs of
    2(npair - i) tiles in launch order when causal, simulated in units of two
    tiles (longest-first order) with chunks of at least 8 units, else nblk
    tiles each with chunks of at least 8 tiles; a causal chunk is even."""
    npair = -(-nblk // 2)
    if causal:
        c = 2 * _simulated_chunk(npair, True, bh, slots, min_chunk=8, lengths=[npair - i for i in range(npair)],
                                 longest_first=True)
    else:
        c = _simulated_chunk(npair, False, bh, slots, min_chunk=8, lengths=[nblk] * npair)
    return min(c, nblk)


@pytest.mark.parametrize("t,window,kind", [(8192, 512, 1), (8192, 512, 0), (1100, 512, 1), (1100, 300, 0),
                                           (4096, 64, 0), (4096, 100, 1), (2048, 4096, 0)])
def test_window_workspace_matches_brute_force_ranges(t, window, kind):
    """The library's tile ranges under a window (seen through the workspace
    it asks for) equal the brute-force spans of visible pairs."""
    slots = 512
    nblk = -(-t // 64)
    for col, entry, nacc_nsc in ((False, _lib.ENTRY_FWD, 64 + 2), (True, _lib.ENTRY_GG_COL, 2 * 64)):
        lens = _block_tiles(t, True, window, kind, col)
        if entry == _lib.ENTRY_FWD and window >= t:  # no window: the row-pair forward
            c = _simulated_pair_chunk(nblk, True, 1, slots)
        else:
            c = _simulated_chunk(nblk, True, 1, slots, lengths=lens)
        k = -(-max(lens) // min(c, max(lens)))
        pr = _prob(seqlen=t, window=window, window_kind=kind)
        parts = nblk * k if k > 1 else 0
        assert _lib.workspace_bytes(pr, entry) == parts * 64 * nacc_nsc * 4, (col, lens[:4], c)
    # plain causal: the brute-force spans are nblk, nblk-1, ..., 1 (rows) and the same (columns)
    assert _block_tiles(640, True) == list(range(10, 0, -1)) == _block_tiles(640, True, col=True)


def test_split_info_matches_workspace():
    """ttt_attn_split_info reports the split the workspace is sized for (no
    GPU here: 256 CUs x 2 workgroups, all usable)."""
    pr = _prob(seqlen=8192)
    assert _lib.split_info(pr, _lib.ENTRY_GG_ROW, True) == (17, 8, 512)
    assert _lib.workspace_bytes(pr, _lib.ENTRY_GG_ROW) == 128 * 8 * 64 * (3 * 64 + 3) * 4
    with pytest.raises(RuntimeError, match="single kernel family"):
        _lib.split_info(pr, _lib.ENTRY_GG, True)
    # the chunk itself (not only the workspace it implies) against the restatement,
    # XCD-local column order included (b*h not a multiple of 8)
    for t in (8192, 16384, 3712, 5120, 8704):
        for bh in (1, 2, 3):
            nblk = t // 64
            pr = _prob(seqlen=t, heads=bh)
            assert _lib.split_info(pr, _lib.ENTRY_GG_ROW, True)[0] == _simulated_chunk(nblk, True, bh, 512), (t, bh)
            assert _lib.split_info(pr, _lib.ENTRY_FWD, False)[0] == _simulated_pair_chunk(nblk, True, bh, 512), (t, bh)
    assert _lib.split_info(_prob(seqlen=16384), _lib.ENTRY_GG_ROW, True)[0] == 64
    # the row-pair forward at C3 and T16k: 16- and 34-tile chunks (even: whole pairs of tiles)
    assert _lib.split_info(_prob(seqlen=8192), _lib.ENTRY_FWD, False)[:2] == (16, 8)
    assert _lib.split_info(_prob(seqlen=16384), _lib.ENTRY_FWD, False)[:2] == (34, 8)
    # a forced odd chunk of a causal row-pair launch is rounded up to whole pairs of tiles
    assert _lib.split_info(_prob(seqlen=300, split_chunk=1), _lib.ENTRY_FWD, False)[:2] == (2, 3)
    assert _lib.split_info(_prob(seqlen=300, split_chunk=1, causal=0), _lib.ENTRY_FWD, False)[:2] == (1, 5)
    # fp32 and d128 keep the 64-row forward and its chooser
    assert _lib.split_info(_prob(seqlen=300, split_chunk=1, dtype=2), _lib.ENTRY_FWD, False)[:2] == (1, 5)


def test_window_and_bias_validation():
    lib = _lib.load()
    assert _fwd_rc(_prob(window=-1)) == 1
    assert _fwd_rc(_prob(window=16, causal=0)) == 1
    assert b"causal" in lib.ttt_last_error()
    assert _fwd_rc(_prob(window=16, window_kind=5)) == 1
    pr = _prob()
    pr.bias = _lib._View(0x10002, 0, 0, 128)
    assert _fwd_rc(pr) == 1 and b"bias" in lib.ttt_last_error()
    pr.bias = _lib._View(0x10000, 0, 0, 100)
    assert _fwd_rc(pr) == 1 and b"bias" in lib.ttt_last_error()
    pr.bias = _lib._View(0x10000, -128, 0, 128)
    assert _fwd_rc(pr) == 1
    # a window of T or more is none: the same workspace as plain causal
    big = _prob(seqlen=8192)
    assert _lib.workspace_bytes(_prob(seqlen=8192, window=8192), _lib.ENTRY_GG) == \
        _lib.workspace_bytes(big, _lib.ENTRY_GG)


def test_prep_bias_layouts():
    """Bias operands: broadcast dims keep stride 0, rows whose storage ends
    short of 16 bytes are copied into padded rows, aligned ones are used as
    they are."""
    m = torch.zeros(512, 512, dtype=torch.float16)
    out = _lib.prep_bias(m, 2, 8, 512, torch.float16, "cpu")
    assert out.shape == (2, 8, 512, 512) and out.stride()[:2] == (0, 0) and out.data_ptr() == m.data_ptr()
    odd = torch.randn(1, 1, 100, 100).half()
    out = _lib.prep_bias(odd, 1, 2, 100, torch.float16, "cpu")
    assert out.stride(2) == 104 and torch.equal(out[0, 1], odd[0, 0])
    kp = torch.zeros(3, 1, 1, 64)  # key padding mask, fp32 -> fp16
    out = _lib.prep_bias(kp, 3, 4, 64, torch.float16, "cpu")
    assert out.dtype == torch.float16 and out.stride()[1:3] == (0, 0)
    with pytest.raises(ValueError):
        _lib.prep_bias(torch.zeros(5, 7), 1, 1, 8, torch.float16, "cpu")


def test_workspace_sizes():
    # Without a GPU the split assumes 256 CUs x 2 workgroups, all usable = 512
    # slots.  Partial accumulators per chunk: nacc x 64 x D fp32 + nsc scalars
    # per row (forward 1 acc + 2, dQ 1, dK/dV 2, GQ 3 + 3, GQ+GdO 5 + 3).
    slots = 512
    for (t, causal, bh) in [(8192, 1, 1), (16384, 1, 1), (8192, 0, 1), (4096, 1, 2), (2048, 1, 1)]:
        nblk = t // 64
        c = _simulated_chunk(nblk, bool(causal), bh, slots)
        k = -(-nblk // c)
        pr = _prob(seqlen=t, causal=causal, heads=bh)
        parts = bh * nblk * k if k > 1 else 0
        # the O + LSE forward of 16-bit d64 problems runs over row-block pairs (its own split); fp32 does not
        cp = _simulated_pair_chunk(nblk, bool(causal), bh, slots)
        kp = -(-nblk // cp)
        parts_p = bh * nblk * kp if kp > 1 else 0
        assert _lib.workspace_bytes(pr, _lib.ENTRY_FWD) == parts_p * 64 * (64 + 2) * 4, (t, causal, bh, cp)
        pr32 = _prob(seqlen=t, causal=causal, heads=bh, dtype=2)
        assert _lib.workspace_bytes(pr32, _lib.ENTRY_FWD) == parts * 64 * (64 + 2) * 4, (t, causal, bh, c)
        assert _lib.workspace_bytes(pr, _lib.ENTRY_GG_ROW) == parts * 64 * (3 * 64 + 3) * 4
        # the fused double backward holds the row pass's partials (five accumulators, three row scalars)
        # and the column pass's (two accumulators) at once
        assert _lib.workspace_bytes(pr, _lib.ENTRY_GG, True) == parts * 64 * (5 * 64 + 3 + 2 * 64) * 4
        # the fused backward holds dQ's partials (one accumulator) and dK/dV's (two) at once
        assert _lib.workspace_bytes(pr, _lib.ENTRY_BWD) == parts * 64 * (3 * 64) * 4
    # C3: 17-tile chunks; of the 548 workgroups the 36 beyond the 512 slots
    # are the shortest last chunks, which the longest-first order runs last
    assert _simulated_chunk(128, True, 1, slots) == 17 and _slice_workgroups(128, 17, True) == 548
    # C5 fills the chip with blocks alone: no split, no workspace
    c5 = _prob(batch=4, heads=16, seqlen=8192, head_dim=128, dtype=1)
    assert all(_lib.workspace_bytes(c5, e) == 0 for e in range(8))
    # no chunk is shorter than 4 tiles: 4 blocks never split; split_chunk forces a length
    assert _lib.workspace_bytes(_prob(seqlen=256), _lib.ENTRY_GG_COL) == 0
    assert _lib.workspace_bytes(_prob(seqlen=300, split_chunk=2), _lib.ENTRY_GG_COL) == 5 * 3 * 64 * 128 * 4
    assert _lib.load().ttt_attn_workspace_size(ctypes.byref(_prob()), 99, 0) == -1


def test_roofline_model_matches_baseline_table():
    r = workloads.roofline_us(workloads.CONFIGS["C3"])
    assert round(r["flops"] / 1e9, 2) == 60.60 and round(r["bytes"] / 1e6, 1) == 225.0
    assert round(r["roofline_us"], 1) == 28.1 and r["bound"] == "hbm"
    r = workloads.roofline_us(workloads.CONFIGS["C5"])
    assert round(r["flops"] / 1e9, 1) == 7756.7 and r["bound"] == "mfma"
    r = workloads.roofline_us(workloads.CONFIGS["C2"])
    assert round(r["flops"] / 1e9, 2) == 51.54 and round(r["bytes"] / 1e6, 1) == 180.5
    r = workloads.roofline_us(workloads.CONFIGS["C4_16k"])
    assert round(r["roofline_us"], 1) == 106.6
    assert workloads.active_area(8192, True) == 64 * 64 * 128 * 129 // 2


def test_inputs_are_seeded_and_ordered():
    cfg = workloads.CONFIGS["C1"]
    a = workloads.make_inputs(cfg, seed=0)
    b = workloads.make_inputs(cfg, seed=0)
    g = torch.Generator().manual_seed(0)
    first = torch.randn((1, 1, 64, 64), generator=g)
    assert torch.equal(a["q"], first) and all(torch.equal(a[n], b[n]) for n in a)
    c5 = workloads.Config("x", 1, 1, 64, 64, "fp32", True, qkv_scale=0.5)
    assert torch.allclose(workloads.make_inputs(c5)["q"], first * 0.5)


def test_mode_registry():
    ta = importlib.import_module("testtimeideas_amd.ttt_kernels.triton_attention")
    for m in ("save_p", "save_p_triton", "save_p_triton_bwd", "save_p_triton_full"):
        assert ta.mode_kind(m) == "save_p"
    for m in ("recompute", "recompute_manual", "recompute_sdp", "recompute_sdp_mem", "recompute_sdp_auto",
              "recompute_compiled", "dv_only", "anything else"):
        assert ta.mode_kind(m) == "recompute"
    assert ta.mode_kind("custom") == "custom"
    # the reference CLI's twelve choices (tests/bench_gradgrad.py:53-54) are all accepted
    assert len(ta.BWD_MODES) == 12


def test_cpu_tensors_raise():
    from ttt_kernels import triton_attention
    q = torch.randn(1, 1, 8, 64)
    with pytest.raises(RuntimeError, match="ROCm"):
        triton_attention(q, q, q)
    with pytest.raises(NotImplementedError):
        _lib.padded_head_dim(160)
    assert _lib.padded_head_dim(32) == 64 and _lib.padded_head_dim(80) == 128


def test_one_launch_of_each_pass_per_gradgrad_step(monkeypatch):
    """Regression: the first backward ran a second time during the grad-grad
    when the forward output reached the backward Function with its graph."""
    ta = importlib.import_module("testtimeideas_amd.ttt_kernels.triton_attention")
    calls = {"fwd": 0, "bwd": 0, "gg": 0}
    monkeypatch.setattr(_lib, "check_inputs", lambda *a: None)

    def fwd(q, k, v, causal, scale, want_p):
        calls["fwd"] += 1
        t = q.shape[2]
        return torch.zeros_like(q), torch.zeros(q.shape[:3]), torch.zeros(q.shape[:3] + (t,)) if want_p else None

    made = {}

    def bwd(q, k, v, o, do, lse, p, causal, scale):
        calls["bwd"] += 1
        made["dq"] = torch.zeros_like(q)
        return made["dq"], torch.zeros_like(k), torch.zeros_like(v), torch.zeros(q.shape[:3])

    def gg(q, k, v, do, lse, p, rowsum, gq, gk, gv, causal, scale, want_gdo, dq=None):
        calls["gg"] += 1
        # the double backward reads the first backward's dQ
        assert dq is not None and dq.data_ptr() == made["dq"].data_ptr() and dq.shape == made["dq"].shape
        return torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v), None

    monkeypatch.setattr(_lib, "fwd", fwd)
    monkeypatch.setattr(_lib, "bwd", bwd)
    monkeypatch.setattr(_lib, "gg", gg)
    q, k, v, do, rq, rk, rv = (torch.randn(1, 1, 64, 64) for _ in range(7))
    for mode in ("save_p_triton_full", "recompute"):
        for key in calls:
            calls[key] = 0
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        o = ta.triton_attention(qq, kk, vv, causal=True, bwd_mode=mode)
        dq, dk, dv = torch.autograd.grad(o, (qq, kk, vv), do, create_graph=True)
        s = (dq * rq).sum() + (dk * rk).sum() + (dv * rv).sum()
        torch.autograd.grad(s, (qq, kk, vv))
        assert calls == {"fwd": 1, "bwd": 1, "gg": 1}, (mode, calls)


def test_golden_fixture_reproduces():
    """The committed C1 fixture equals what the oracle produces now."""
    golden = importlib.import_module("tests.golden.make_c1")
    ref = np.load(os.path.join(ROOT, "tests", "golden", "c1_b1h1_t64_d64_fp32.npz"))
    now = golden.build()
    for key in ref.files:
        assert np.array_equal(ref[key], now[key]), key


def test_expanded_operand_is_copied():
    """An operand expanded along T (stride 0 there) is not what the C ABI
    takes (it needs a positive T stride), so the binding copies it."""
    x = torch.randn(2, 3, 1, 64).expand(2, 3, 5, 64)
    assert x.stride(2) == 0
    assert not _lib._kernel_ok(x)
    y = _lib.prep(x, 64)
    assert y.stride(2) > 0 and torch.equal(y, x)
    assert _lib._kernel_ok(y)


def test_noalloc_rejects_too_many_rows_without_gpu():
    """ttt_attn_gg_noalloc keeps E and F in its static scratch (B*H*T <= 2^21)
    and says so before touching the device."""
    lib = _lib.load()
    pr = _prob(batch=64, seqlen=32769)
    rc = lib.ttt_attn_gg_noalloc(ctypes.byref(pr), _v(), _v(), _v(), _v(), 0x20000, None, 0x20000, None, _v(), _v(),
                                 _v(), _v(), _v(), _v(), None, None)
    assert rc == 1
    assert b"B*H*T" in lib.ttt_last_error()


def test_block_rows_choice():
    """ttt_problem.block_rows: the library runs 128-row pairs for 16-bit d64
    problems without a window or bias and 64-row blocks otherwise; 64 and
    128 can be asked for (128 only where pairs run); the split follows the
    kernel that runs."""
    slots = 512
    nblk = 8192 // 64
    c64 = _simulated_chunk(nblk, True, 1, slots)
    cp = _simulated_pair_chunk(nblk, True, 1, slots)
    assert _lib.split_info(_prob(seqlen=8192), _lib.ENTRY_FWD, False)[0] == cp
    assert _lib.split_info(_prob(seqlen=8192, block_rows=128), _lib.ENTRY_FWD, False)[0] == cp
    assert _lib.split_info(_prob(seqlen=8192, block_rows=64), _lib.ENTRY_FWD, False)[0] == c64
    # d128: 64-row blocks unless asked for, then pairs (the same pair chooser)
    assert _lib.split_info(_prob(seqlen=8192, head_dim=128), _lib.ENTRY_FWD, False)[0] == c64
    assert _lib.split_info(_prob(seqlen=8192, head_dim=128, block_rows=128), _lib.ENTRY_FWD, False)[0] == cp
    # workspaces follow the same splits
    k64, kp = -(-nblk // c64), -(-nblk // cp)
    assert _lib.workspace_bytes(_prob(seqlen=8192, block_rows=64), _lib.ENTRY_FWD) == nblk * k64 * 64 * 66 * 4
    assert _lib.workspace_bytes(_prob(seqlen=8192), _lib.ENTRY_FWD) == nblk * kp * 64 * 66 * 4
    # the forward with P and the other entries ignore it
    assert _lib.split_info(_prob(seqlen=8192, block_rows=64), _lib.ENTRY_FWD_P, True) == \
        _lib.split_info(_prob(seqlen=8192), _lib.ENTRY_FWD_P, True)
    lib = _lib.load()
    assert _fwd_rc(_prob(block_rows=96)) == 1 and b"block_rows" in lib.ttt_last_error()
    assert _fwd_rc(_prob(block_rows=128, dtype=2)) == 2 and b"block_rows" in lib.ttt_last_error()
    assert _fwd_rc(_prob(block_rows=128, window=16)) == 2
    assert lib.ttt_version() >= 400
