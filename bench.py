"""Benchmark of the grad-grad attention step on one MI355X.

Workload: b=1 h=1 T=8192 d=64 fp16, causal with 64x64
block-sparse tiles, bwd_mode='save_p_triton_full'.  One step is

    O = triton_attention(q, k, v, causal=True, bwd_mode='save_p_triton_full')
    dQ, dK, dV = grad(O, (q, k, v), dO, create_graph=True)
    GQ, GK, GV = grad(sum(dQ*rq + dK*rk + dV*rv), (q, k, v))

with q, k, v, dO, rq, rk, rv ~ N(0,1) drawn from a seeded CPU generator and
resident in HBM before timing starts.  Prints one JSON line (rank 0).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3]
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

from testtimeideas_amd import _lib, autotune, workloads  # noqa: E402
from testtimeideas_amd.ttt_e2e import windowed_attention  # noqa: E402
from ttt_kernels import triton_attention  # noqa: E402

METRIC = "fwd+bwd+grad-grad ms at T=8k/16k d=64 fp16 causal; MFMA/HBM % of peak"
REFERENCE_H100_MS = {"C3": 4.054, "C4_16k": 13.649}  # artifacts/gradgrad_sweep.csv (reduced grad-grad)
# The reference's published sweep (artifacts/gradgrad_sweep.csv:2-13, triton_ms_mean; b1 h1 d64 fp16,
# save_p_triton_full, its mean-loss harness, H100): (T, causal) -> ms.  Context only: its grad-grad
# holds P constant.
REFERENCE_SWEEP_H100_MS = {
    (512, False): 1.901, (1024, False): 2.012, (2048, False): 1.981, (4096, False): 2.010,
    (8192, False): 3.503, (16384, False): 11.466, (512, True): 1.994, (1024, True): 1.953,
    (2048, True): 1.995, (4096, True): 2.083, (8192, True): 4.054, (16384, True): 13.649}
# The reference's forward at C2 (artifacts/modal_bench_h100_latest.txt:3-5; triton_attention(q, k, v)
# with the default mode, no grad): ms on H100.
REFERENCE_C2_FWD_H100_MS = 0.137


def _two_stage_sum(t: torch.Tensor) -> torch.Tensor:
    """Sum as 256 row sums then one 256-element sum: torch's single-output
    reduction over a large tensor clears a semaphore buffer with a memset,
    which must not be recorded into a HIP graph; this form launches two reduce
    kernels and no memset.  Its gradient is the same all-ones broadcast."""
    return t.reshape(256, -1).sum(1).sum()


def make_step(cfg: workloads.Config, x, graph_safe: bool = False, scalar_loss: bool = False):
    """One step: O, then (dQ, dK, dV) with create_graph=True, then the
    gradient of sum(dQ*rq + dK*rk + dV*rv) with respect to (q, k, v).  By
    default that last gradient is asked for as the vector-Jacobian product of
    (dQ, dK, dV) with cotangents (rq, rk, rv), which is the same gradient
    (the sum is linear in dQ, dK, dV with those coefficients) and launches
    only the attention kernels; `scalar_loss` instead forms the scalar with
    torch products and reductions and differentiates it, as a script would."""
    q, k, v = (x[n].requires_grad_(True) for n in ("q", "k", "v"))
    do, rq, rk, rv = x["do"], x["rq"], x["rk"], x["rv"]
    red = _two_stage_sum if graph_safe else torch.sum

    def attend():
        if cfg.window:
            return windowed_attention(q, k, v, cfg.window, local=cfg.window_kind == "local", bwd_mode=cfg.bwd_mode)
        return triton_attention(q, k, v, causal=cfg.causal, bwd_mode=cfg.bwd_mode)

    def step():
        o = attend()
        dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=cfg.gradgrad)
        if not cfg.gradgrad:
            return (dq,)
        if not scalar_loss:
            return torch.autograd.grad((dq, dk, dv), (q, k, v), (rq, rk, rv))
        s = red(dq * rq) + red(dk * rk) + red(dv * rv)
        return torch.autograd.grad(s, (q, k, v))

    return step


def graph_steps(cfg: workloads.Config, x, steps: int, warmup: int, checks: int = 3) -> float:
    """ms per step of the same step replayed from a HIP graph (captured once;
    every replay reruns every kernel from the resident inputs).  Before timing,
    `checks` replays, each followed by eager steps and a synchronisation, are
    compared bitwise with the eager result; a mismatch raises."""
    step = make_step(cfg, x, graph_safe=True)
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ref = [t.clone() for t in step()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for i in range(checks):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, ref):
            if not torch.equal(a, b):
                raise RuntimeError(f"graph replay {i} differs from the eager step")
        step()  # eager work between replays
        torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    del graph
    return ms


def time_steps(step, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def kernel_times(step, reps: int = 10):
    """Mean duration (ms) of each kernel, from HIP events recorded on the launch stream."""
    with _lib.kernel_timing() as rec:
        for _ in range(reps):
            step()
        torch.cuda.synchronize()
        return _lib.mean_ms(rec)


SAVE_P = ("save_p", "save_p_triton", "save_p_triton_bwd", "save_p_triton_full")


def launch_times(step, steps: int) -> dict:
    """Mean duration (ms) of each main kernel's launches while `steps` steps
    run as in the timed region (fused entry points included), from the two HIP
    events the library records on the launch stream around every main-kernel
    launch while timing is on (ttt_kernel_timing)."""
    with _lib.launch_timing(16 * steps + 64) as read:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        return {k: v[0] for k, v in read().items()}


# the main kernel of each entry point (the launch-timing names)
ENTRY_KERNEL = {"ttt_attn_gg_row": "gg_row", "ttt_attn_gg_col": "gg_col", "ttt_attn_bwd_dq": "bwd_dq",
                "ttt_attn_bwd_dkdv": "bwd_dkdv"}


def roofline_entry(cfg, ktimes, launch_ms=None, with_p=None):
    """Roofline of the dominant entry point (the longest in the per-entry
    timing `ktimes`), priced on its main kernel's own launches in the step
    (`launch_ms`) when they were timed, else on the entry's time."""
    if with_p is None:
        with_p = cfg.bwd_mode in SAVE_P
    name = max(ktimes, key=ktimes.get)
    model = workloads.kernel_model(name, cfg, with_p)
    kern = ENTRY_KERNEL.get(name)  # the forward entry runs two kernels with P: priced whole
    kernel_ms = (launch_ms or {}).get(kern) if kern else None
    dur_s = (kernel_ms if kernel_ms else ktimes[name]) * 1e-3
    tag = workloads.DTYPE_TAG[cfg.torch_dtype]
    if model["bound"] == "mfma":
        achieved = model["flops"] / dur_s / 1e12
        peak, unit = workloads.PEAK_TFLOPS[tag], "TFLOP/s"
    else:
        achieved = model["bytes"] / dur_s / 1e9
        peak, unit = workloads.PEAK_HBM_GBS, "GB/s"
    traffic, label = measured_traffic(name, cfg, kern if kernel_ms else None, with_label=True)
    kname = (label.split("<")[0] if label else f"k_{kern}") if kernel_ms else name
    return {"kernel": kname, "entry": name, "bound": model["bound"],
            "achieved": round(achieved, 2), "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "avg_us": round(dur_s * 1e6, 2), "entry_us": round(ktimes[name] * 1e3, 2),
            "algorithmic_flops": model["flops"], "algorithmic_bytes": model["bytes"]}


def measured_traffic(entry: str, cfg: workloads.Config, kernel=None, with_label: bool = False):
    """HBM bytes per launch from the committed rocprof PMC summary
    (FETCH_SIZE + WRITE_SIZE scaled by a plain-copy calibration): of the main
    kernel `kernel` alone as the step launches it (its fused form, with
    combine workgroups appended, where there is one; its eight-wave form
    k_<kernel>8 where the step runs that), or else summed over the kernels the
    summary attributes to the entry point, its combine kernels included; None
    without a summary.  With `with_label`, (bytes, the summary's kernel label
    or None)."""
    def out(v, label=None):
        return (v, label) if with_label else v

    path = os.path.join(ROOT, "profiles", f"pmc_traffic_{cfg.name}.json")
    if not os.path.exists(path):
        return out(None)
    with open(path) as f:
        data = json.load(f)["kernels"]
    if kernel is not None:
        labels = [k for k in data if (k.startswith(f"k_{kernel}<") or k.startswith(f"k_{kernel}8<")) and "@" not in k]
        fused = [k for k in labels if "+" in k]
        pick = (fused or labels)[:1]
        if not pick:
            return out(None)
        return out(round(data[pick[0]]["fetch_bytes"] + data[pick[0]]["write_bytes"]), pick[0])
    total, found = 0.0, False
    for rec in data.values():
        if rec.get("entry") == entry:
            total += rec["fetch_bytes"] + rec["write_bytes"]
            found = True
    return out(round(total) if found else None)


def fwd_mfma(cfg: workloads.Config, dev, reps: int = 50) -> dict:
    """The O + LSE forward (recompute modes; the reference's default forward)
    alone and its MFMA utilisation by algorithmic FLOPs (QK^T and PV over the
    active tiles).  `us` is the mean time per call of `reps` calls issued back
    to back, between two HIP events on the launch stream: the GPU time of the
    entry (its kernels and the gap between them) without the host's time to
    submit one call, which a pair of events around a lone call also counts
    (`entry_us`, the per-entry form used for the step's entries)."""
    x = workloads.make_inputs(cfg, seed=0, device=dev)
    q, k, v = x["q"], x["k"], x["v"]
    stream = torch.cuda.current_stream()
    with torch.no_grad():
        for _ in range(5):
            _lib.fwd(q, k, v, cfg.causal, cfg.scale, False)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            _lib.fwd(q, k, v, cfg.causal, cfg.scale, False)
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / reps
        with _lib.kernel_timing() as rec:
            for _ in range(10):
                _lib.fwd(q, k, v, cfg.causal, cfg.scale, False)
            torch.cuda.synchronize()
            entry_ms = _lib.mean_ms(rec)["ttt_attn_fwd"]
    flops = 4.0 * cfg.b * cfg.h * cfg.d * workloads.cfg_area(cfg)
    peak = workloads.PEAK_TFLOPS[workloads.DTYPE_TAG[cfg.torch_dtype]]
    return {"us": round(ms * 1e3, 2), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "mfma_frac": round(flops / (ms * 1e-3) / (peak * 1e12), 4), "entry_us": round(entry_ms * 1e3, 2)}


def sweep_bench(dev, steps: int, warmup: int) -> list:
    """The reference's published sweep (C4): b1 h1 d64 fp16, T = 512 ... 16384,
    non-causal and causal, the full step per point: eager (`ms`) and replayed
    from a HIP graph (`graph_ms`: the device time of the same launches
    without the host's submission of each)."""
    out = []
    for causal in (False, True):
        for t in (512, 1024, 2048, 4096, 8192, 16384):
            cfg = workloads.sweep_config(t, causal)
            x = workloads.make_inputs(cfg, seed=0, device=dev)
            ms = time_steps(make_step(cfg, x), steps, warmup)
            gms = graph_steps(cfg, x, steps, warmup)
            roof = workloads.roofline_us(cfg)
            out.append({"t": t, "causal": causal, "ms": round(ms, 4), "graph_ms": round(gms, 4),
                        "tflops": round(roof["flops"] / (ms * 1e-3) / 1e12, 2),
                        "step_roofline_frac": round(roof["roofline_us"] * 1e-3 / ms, 4),
                        "reference_h100_ms": REFERENCE_SWEEP_H100_MS[(t, causal)]})
            del x
    return out


# The reference's per-mode table at b1 h1 T8192 d64 fp16 non-causal
# (artifacts/modal_bench_h100_latest.txt:79-93): ms on H100 for its Triton
# path; its grad-grad in the save_p modes holds P constant.
REFERENCE_MODES_T8192_H100_MS = {"recompute": 4.899, "save_p": 3.423, "save_p_triton_bwd": 3.511,
                                 "save_p_triton_full": 3.591}


def modes_bench(dev, steps: int, warmup: int) -> dict:
    """The full step at b1 h1 T8192 d64 fp16 non-causal in each of the
    reference's timed modes (all with the exact grad-grad here)."""
    out = {}
    base = workloads.sweep_config(8192, False)
    x = workloads.make_inputs(base, seed=0, device=dev)
    for mode, ref in REFERENCE_MODES_T8192_H100_MS.items():
        cfg = dataclasses.replace(base, name=f"T8192_{mode}", bwd_mode=mode)
        out[mode] = {"ms": round(time_steps(make_step(cfg, x), steps, warmup), 4), "reference_h100_ms": ref}
    return out


def c2_bench(dev, steps: int, warmup: int) -> dict:
    """C2 (b2 h4 T2048 d128 fp16 non-causal): the forward alone as the
    reference's forward benchmark runs it (default mode, no grad), the save_p
    forward (P written), and save_p forward + first backward."""
    cfg = workloads.CONFIGS["C2"]
    x = workloads.make_inputs(cfg, seed=0, device=dev)
    q, k, v = x["q"], x["k"], x["v"]

    def fwd(mode):
        def run():
            with torch.no_grad():
                return triton_attention(q, k, v, causal=cfg.causal, bwd_mode=mode)
        return run

    fwd_ms = time_steps(fwd("recompute"), steps, warmup)
    fwd_p_ms = time_steps(fwd("save_p"), steps, warmup)
    step = make_step(cfg, x)
    ms = time_steps(step, steps, warmup)
    roof = workloads.roofline_us(cfg)
    return {"fwd_ms": round(fwd_ms, 4), "fwd_save_p_ms": round(fwd_p_ms, 4), "fwd_bwd_ms": round(ms, 4),
            "fwd_bwd_tflops": round(roof["flops"] / (ms * 1e-3) / 1e12, 2),
            "fwd_bwd_roofline_frac": round(roof["roofline_us"] * 1e-3 / ms, 4),
            "kernel_us": {k: round(v * 1e3, 2) for k, v in sorted(kernel_times(step, 5).items())},
            "reference_h100_fwd_ms": REFERENCE_C2_FWD_H100_MS}


def autotuned(step, steps: int):
    """(ms per step, choices) of the same step with every kernel family's
    configuration measured per shape (testtimeideas_amd.autotune; the first
    step tunes, untimed).  Tuning is left as it was found."""
    was = autotune.enabled()
    autotune.enable(True)
    try:
        step()
        torch.cuda.synchronize()
        tuned_ms = time_steps(step, steps, 1)
        tuned = {str(k[0]): v for k, v in autotune.choices().items()}
    finally:
        autotune.enable(was)
        autotune.clear()
    return tuned_ms, tuned


def c5_bench(dev, steps: int, warmup: int) -> dict:
    """C5 (b4 h16 T8192 d128 bf16 causal, q, k, v x 0.5): the full step."""
    cfg = workloads.CONFIGS["C5"]
    x = workloads.make_inputs(cfg, seed=0, device=dev)
    step = make_step(cfg, x)
    ms = time_steps(step, steps, warmup)
    roof = workloads.roofline_us(cfg)
    kt = kernel_times(step, 3)
    lt = launch_times(step, 3)
    tuned_ms, tuned = autotuned(step, steps)
    return {"ms": round(ms, 3), "autotuned_ms": round(tuned_ms, 3), "autotuned_choices": tuned,
            "tflops": round(roof["flops"] / (ms * 1e-3) / 1e12, 1),
            "step_roofline_us": round(roof["roofline_us"], 1),
            "step_roofline_frac": round(roof["roofline_us"] * 1e-3 / ms, 4),
            "kernel_us": {k: round(v * 1e3, 1) for k, v in sorted(kt.items())},
            "launch_us": {k: round(v * 1e3, 1) for k, v in lt.items()},
            "roofline": roofline_entry(cfg, kt, lt)}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host_cpus() -> dict:
    """The host's CPU as lscpu reports it (model, sockets x physical cores,
    hardware threads) and the CPUs this process may use (its affinity and
    cgroup quota)."""
    info = {"model": _cpu_model(), "sockets": None, "physical_cores": None, "hw_threads": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, timeout=10).stdout
        pairs = {tuple(line.split(",")[:2]) for line in out.splitlines() if line and not line.startswith("#")}
        info["physical_cores"] = len(pairs)
        info["sockets"] = len({s for _, s in pairs})
    except (OSError, subprocess.SubprocessError):
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            usable = min(usable, max(1, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    info["usable"] = usable
    return info


def cpu_baseline(cfg: workloads.Config, budget_s: float = 20.0):
    """The math path (oracle.math_path, the reference's _attention_math + autograd
    restated) on the host CPU, on the same seeded inputs in the config dtype,
    with one thread per physical core of the host, or as many as this process
    may use if that is fewer.  Bounded sample: one warmup step, then whole
    steps until ~budget_s of timed CPU work (at least one)."""
    from oracle import math_path
    cpus = _host_cpus()
    threads = max(1, min(cpus["physical_cores"] or cpus["usable"], cpus["usable"]))
    torch.set_num_threads(threads)
    x = workloads.make_inputs(cfg, seed=0)
    args = [x[n] for n in ("q", "k", "v", "do", "rq", "rk", "rv")]
    if cfg.window:
        # the reference's chunk loop (WindowedSelfAttention) through its masked math, with autograd
        def run():
            return math_path.window_gradgrad_step(*args, cfg.window)
        what = f"the reference's {cfg.window}-row chunk loop of masked math with autograd"
    else:
        def run():
            return math_path.gradgrad_step(*args, cfg.causal, cfg.scale)
        what = "torch CPU math path with autograd"
    run()  # warmup
    times = []
    while not times or (sum(times) < budget_s * 1e3 and len(times) < 20):
        t0 = time.perf_counter()
        run()
        times.append((time.perf_counter() - t0) * 1e3)
    return {"value": round(statistics.median(times), 3), "unit": "ms", "cores": threads, "kind": "port",
            "host": cpus,
            "sample": f"{len(times)} full {cfg.name} steps (b{cfg.b} h{cfg.h} T{cfg.t} d{cfg.d} {cfg.dtype} "
                      f"causal={cfg.causal}{f' window={cfg.window}' if cfg.window else ''}) after 1 warmup, "
                      f"median; {what}; {threads} threads; host (lscpu): {cpus['model']}, "
                      f"{cpus['sockets']} socket(s), {cpus['physical_cores']} physical cores, "
                      f"{cpus['hw_threads']} hardware threads; this process may use {cpus['usable']}"}


# The reference's meta-training configuration (cloud_ttt_e2e/configs/meta_8k_v2.yaml) and its H100 rate
# (cloud_ttt_e2e/meta_8k_v2.log: 1.26-1.28 s/it over 5000 iterations).
META_8K = dict(vocab_size=512, num_keys=64, max_seq_len=8192, context_len=6144, query_len=2048, window_size=512,
               d_model=384, n_heads=6, n_layers=8, d_ff=1536, suffix_layers=2, dual_mlp=True,
               ttt_param_filter="mlp_fast", chunk_size=1024, far_frac=0.75, batch_size=8, lr=5e-4, inner_steps=4,
               inner_lr=0.1)
META_8K_H100_S_PER_IT = 1.27


def meta_bench(steps: int, warmup: int, dev) -> dict:
    """Seconds per meta-training iteration of the reference TTT model at
    meta_8k_v2 on this GPU, timed as the reference's loop is
    (scripts/train_meta.py:133-160): synthetic batch, meta_step, backward of
    the outer loss through every inner update, AdamW step."""
    from ttt_e2e import data, meta
    from ttt_e2e.model import ModelConfig, TTTModel
    c = META_8K
    torch.manual_seed(1337)
    model = TTTModel(ModelConfig(vocab_size=c["vocab_size"], max_seq_len=c["max_seq_len"],
                                 window_size=c["window_size"], d_model=c["d_model"], n_heads=c["n_heads"],
                                 n_layers=c["n_layers"], d_ff=c["d_ff"], suffix_layers=c["suffix_layers"],
                                 dual_mlp=c["dual_mlp"])).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=c["lr"], weight_decay=0.0)
    gen = torch.Generator().manual_seed(1337)

    def it():
        bt = data.generate_kv_batch(c["batch_size"], c["context_len"], c["query_len"], c["vocab_size"],
                                    num_keys=c["num_keys"], device=dev, pad_to=c["max_seq_len"],
                                    far_frac=c["far_frac"], generator=gen)
        inner, outer = meta.meta_step(model, bt.input_ids, bt.targets, bt.inner_mask, bt.outer_mask,
                                      inner_lr=c["inner_lr"], inner_steps=c["inner_steps"],
                                      param_filter=c["ttt_param_filter"], chunk_size=c["chunk_size"])
        opt.zero_grad(set_to_none=True)
        outer.backward()
        opt.step()
        return inner, outer

    for _ in range(warmup):
        it()
    torch.cuda.synchronize()
    times = []
    for _ in range(steps):
        t0 = time.perf_counter()
        inner, outer = it()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    return {"s_per_it": round(statistics.median(times), 4), "iterations": steps, "warmup": warmup,
            "inner_loss": round(float(inner), 4), "outer_loss": round(float(outer), 4),
            "reference_h100_s_per_it": META_8K_H100_S_PER_IT,
            "config": "meta_8k_v2: b8 T8192 d_model 384 6 heads 8 layers (2 suffix) window 512 chunks 1024, "
                      "4 inner steps on mlp_fast, fp32, AdamW"}


def copy_calibration(mb: int, reps: int = 5) -> None:
    """A plain device copy of `mb` MiB (read mb, write mb), for scaling rocprof's
    FETCH_SIZE / WRITE_SIZE counters to bytes."""
    src = torch.empty(mb << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--config", default="C3", choices=sorted(workloads.CONFIGS) + ["META_8K"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the T=16k point and forward-only metrics")
    ap.add_argument("--forward-only", action="store_true",
                    help="time only the O + LSE forward of --config (--steps calls) and print its line")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay of the step")
    ap.add_argument("--autotune", action="store_true",
                    help="measured split per kernel family and shape (testtimeideas_amd.autotune), tuned in warmup")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="also run a plain device copy of this many MiB (counter calibration for rocprof)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the (b,h) slices would shard across GPUs with no communication); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda", 0)
    autotune.enable(args.autotune)
    if args.copy_mb:
        copy_calibration(args.copy_mb)
    if args.config == "META_8K":
        torch.autograd.set_multithreading_enabled(False)
        r = meta_bench(args.steps, args.warmup, dev)
        print(json.dumps({"metric": "meta-train s/it (reference TTT model, meta_8k_v2)", "value": r["s_per_it"],
                          "unit": "s/it", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": round(r["s_per_it"] * 1e3, 2), "higher_is_better": False,
                          "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                          "data": "synthetic key-value batches (the reference's generator, restated)",
                          "config": {"workload": r["config"]}, "meta": r}), flush=True)
        return
    cfg = workloads.CONFIGS[args.config]
    if args.forward_only:
        fm = fwd_mfma(cfg, dev, reps=args.steps)
        print(json.dumps({"metric": "O+LSE forward us per call", "value": fm["us"], "unit": "us", "n_gpus": 1,
                          "steps": args.steps, "warmup": 5, "higher_is_better": False, "scaling": "weak",
                          "vs_baseline": None, "dtype": {"fp16": "f16", "bf16": "bf16", "fp32": "f32"}[cfg.dtype],
                          "data": "synthetic", "config": {"workload": f"{cfg.name} O+LSE forward"}, "forward": fm}),
              flush=True)
        return
    x = workloads.make_inputs(cfg, seed=0, device=dev)
    step = make_step(cfg, x)
    # Backward passes run on the calling thread: the engine's default hand-off
    # to a per-device worker thread costs more host time per step than the
    # kernels take at this size.  The work done per step is the same.
    torch.autograd.set_multithreading_enabled(False)
    ms = time_steps(step, args.steps, args.warmup)
    # the same step with the scalar sum(dQ*rq + dK*rk + dV*rv) formed and differentiated
    ms_scalar = time_steps(make_step(cfg, x, scalar_loss=True), args.steps, args.warmup) if cfg.gradgrad else None
    ktimes = kernel_times(step)
    launch_ms = launch_times(step, args.steps)
    graph_ms = graph_steps(cfg, x, args.steps, args.warmup) if not args.no_graph else None
    roof = workloads.roofline_us(cfg)
    # beside the library's own splits (value): the same step with them measured per shape (not in
    # --no-extra runs, which the profiles use: tuning launches every candidate split)
    tuned_ms, tuned_choices = (None, None) if args.autotune or args.no_extra else autotuned(step, args.steps)

    out = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp16": "f16", "bf16": "bf16", "fp32": "f32"}[cfg.dtype],
        "data": "synthetic N(0,1) q,k,v,dO,rq,rk,rv from a seeded CPU generator",
        "config": {"workload": f"{cfg.name}: b{cfg.b} h{cfg.h} T{cfg.t} d{cfg.d} {cfg.dtype} "
                               f"{'causal 64x64 block-sparse' if cfg.causal else 'non-causal'} "
                               f"{f'{cfg.window_kind} window {cfg.window} ' if cfg.window else ''}"
                               f"{cfg.bwd_mode} fwd+bwd{'+grad-grad' if cfg.gradgrad else ''}",
                   "batch": cfg.b, "heads": cfg.h, "seq_len": cfg.t, "head_dim": cfg.d,
                   "window": cfg.window or None, "bwd_mode": cfg.bwd_mode,
                   "autograd": "eager, backward on the calling thread",
                   "splits": "autotuned" if args.autotune else "library choice"},
        "tflops": round(roof["flops"] / (ms * 1e-3) / 1e12, 3),
        "step_roofline_us": round(roof["roofline_us"], 2),
        "step_roofline_frac": round(roof["roofline_us"] * 1e-3 / ms, 5),
        "graph_ms_per_step": None if graph_ms is None else round(graph_ms, 4),
        "autotuned_ms_per_step": None if tuned_ms is None else round(tuned_ms, 4),
        "autotuned_choices": tuned_choices,
        "scalar_loss_ms_per_step": None if ms_scalar is None else round(ms_scalar, 4),
        "kernel_us": {k: round(v * 1e3, 2) for k, v in sorted(ktimes.items())},
        "kernel_sum_us": round(sum(ktimes.values()) * 1e3, 2),
        "launch_us": {k: round(v * 1e3, 2) for k, v in launch_ms.items()},
        "roofline": roofline_entry(cfg, ktimes, launch_ms),
        "reference_h100_ms": REFERENCE_H100_MS.get(cfg.name),
    }

    if not args.no_extra and cfg.name == "C3":
        # forward-only, O + LSE (recompute mode): MFMA utilisation of the contraction kernel
        fm = fwd_mfma(cfg, dev)
        out["fwd_lse_us"] = fm["us"]
        out["fwd_lse_mfma_frac"] = fm["mfma_frac"]
        out["fwd_lse"] = {name: fwd_mfma(workloads.CONFIGS[name], dev) for name in ("C3", "C4_16k", "C2", "C5")}
        # the reference's published points: the C4 sweep (its T=16384 causal point is the T16k figure),
        # the per-mode table at T=8192 non-causal, the C2 forward and first backward, and C5
        out["c4_sweep"] = sweep_bench(dev, max(30, args.steps // 3), 30)
        out["t16k_causal_ms"] = next(p["ms"] for p in out["c4_sweep"] if p["t"] == 16384 and p["causal"])
        out["modes_t8192_noncausal"] = modes_bench(dev, max(30, args.steps // 3), 30)
        out["c2"] = c2_bench(dev, max(10, args.steps // 5), 5)
        out["c5"] = c5_bench(dev, 5, 2)
        # the reference TTT model's windowed attention (one launch per pass for its chunk loop)
        for name in ("TTT_W512", "TTT_W512_8K"):
            cw = workloads.CONFIGS[name]
            xw = workloads.make_inputs(cw, seed=0, device=dev)
            out[name.lower() + "_ms"] = round(time_steps(make_step(cw, xw), max(5, args.steps // 2), 3), 4)
            del xw
        # the whole meta-training iteration of the reference TTT model (one GPU)
        out["meta_8k"] = meta_bench(3, 1, dev)

    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
