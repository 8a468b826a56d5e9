"""Benchmark configurations, seeded synthetic inputs and the FLOP/byte model.

Configurations are the reference's headline cases for this path (C1-C5 of the
baseline).  Inputs are drawn from a CPU ``torch.Generator`` in the fixed order
q, k, v, dO, rq, rk, rv as float32 ``randn([B,H,T,D])`` (C5 scales q, k, v by
0.5), then cast to the config dtype, so CPU and GPU runs see identical values.

Roofline model (algorithmic work; recomputation inside kernels is not counted):
  A = T^2 (non-causal) or 64^2 * nb(nb+1)/2 with nb = ceil(T/64) (causal, the
      active 64x64 tiles)
  step FLOPs  F = c * B*H * d * A, c = 4 (forward) + 8 (backward) + 16 (grad-grad)
  step bytes  B = 3 e BH A + 21 e BH T d + 12 BH T  (P written, read by the
      backward and by the grad-grad; 21 [T,d] tensors; fp32 LSE, D, E/F)
  with the first-backward-only variant (c = 12; 2 e BH A + 11 e BH T d + 8 BH T).
Per-kernel figures (``kernel_model``) count each distinct product a kernel must
form for its outputs once, and each tensor it must read or write once.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Dict, Optional

import torch

PEAK_TFLOPS = {"f16": 2516.6, "bf16": 2516.6, "f32": 157.3}  # dense MFMA, MI355X
PEAK_HBM_GBS = 8000.0  # HBM3E, MI355X

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
DTYPE_TAG = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


@dataclasses.dataclass(frozen=True)
class Config:
    name: str
    b: int
    h: int
    t: int
    d: int
    dtype: str
    causal: bool
    qkv_scale: float = 1.0
    gradgrad: bool = True
    bwd_mode: str = "save_p_triton_full"
    window: int = 0           # key window (needs causal); 0 = none
    window_kind: str = "local"  # "local": WindowedSelfAttention's chunks; "sliding": make_window_mask

    @property
    def torch_dtype(self) -> torch.dtype:
        return DTYPES[self.dtype]

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.d)


CONFIGS: Dict[str, Config] = {
    "C1": Config("C1", 1, 1, 64, 64, "fp32", False),
    "C2": Config("C2", 2, 4, 2048, 128, "fp16", False, gradgrad=False, bwd_mode="save_p"),
    "C3": Config("C3", 1, 1, 8192, 64, "fp16", True),
    # C3 with P recomputed from the LSE (the reference's default mode): the online forward
    "C3_recompute": Config("C3_recompute", 1, 1, 8192, 64, "fp16", True, bwd_mode="recompute"),
    "C4_16k": Config("C4_16k", 1, 1, 16384, 64, "fp16", True),
    "C5": Config("C5", 4, 16, 8192, 128, "bf16", True, qkv_scale=0.5),
    # The reference TTT model's attention (cloud_ttt_e2e/configs/meta_8k_v2.yaml: batch 8, d_model 384,
    # 6 heads, window 512, inner-loop chunks of 1024 tokens, fp32): WindowedSelfAttention on one chunk,
    # differentiated twice by the meta-gradient.
    "TTT_W512": Config("TTT_W512", 8, 6, 1024, 64, "fp32", True, bwd_mode="recompute", window=512),
    # The same attention over a whole 8k sequence in bf16 (the prefix pass's shape).
    "TTT_W512_8K": Config("TTT_W512_8K", 8, 6, 8192, 64, "bf16", True, bwd_mode="recompute", window=512),
}


def sweep_config(t: int, causal: bool) -> Config:
    return Config(f"C4_T{t}_{'causal' if causal else 'full'}", 1, 1, t, 64, "fp16", causal)


def make_inputs(cfg: Config, seed: int = 0, device: Optional[torch.device] = None,
                dtype: Optional[torch.dtype] = None) -> Dict[str, torch.Tensor]:
    """q, k, v, do, rq, rk, rv drawn in that order from a CPU generator."""
    gen = torch.Generator().manual_seed(seed)
    shape = (cfg.b, cfg.h, cfg.t, cfg.d)
    out = {}
    for name in ("q", "k", "v", "do", "rq", "rk", "rv"):
        x = torch.randn(shape, generator=gen, dtype=torch.float32)
        if name in ("q", "k", "v") and cfg.qkv_scale != 1.0:
            x = x * cfg.qkv_scale
        out[name] = x.to(dtype or cfg.torch_dtype)
    if device is not None:
        out = {k: v.to(device) for k, v in out.items()}
    return out


def _window_lo(m: int, t: int, w: int, kind: str) -> int:
    """First key query m sees under a window (0 without one)."""
    if w <= 0 or w >= t:
        return 0
    if kind == "sliding":
        return max(0, m - w + 1)
    return max(0, min(t, (m // w + 1) * w) - w)


def active_area(t: int, causal: bool, blk: int = 64, window: int = 0, kind: str = "local") -> int:
    """Elements of the 64x64 score tiles the kernels process: all, the lower
    block triangle (causal), or, with a window, the tiles between each row
    block's first visible key and its diagonal."""
    if not causal:
        return t * t
    nb = (t + blk - 1) // blk
    if window <= 0 or window >= t:
        return blk * blk * nb * (nb + 1) // 2
    return blk * blk * sum(mb - _window_lo(mb * blk, t, window, kind) // blk + 1 for mb in range(nb))


def cfg_area(cfg: Config) -> int:
    return active_area(cfg.t, cfg.causal, window=cfg.window, kind=cfg.window_kind)


def step_flops(cfg: Config) -> float:
    c = 28 if cfg.gradgrad else 12
    return float(c * cfg.b * cfg.h * cfg.d * cfg_area(cfg))


def step_bytes(cfg: Config) -> float:
    e = torch.tensor([], dtype=cfg.torch_dtype).element_size()
    bh, a, t, d = cfg.b * cfg.h, cfg_area(cfg), cfg.t, cfg.d
    if cfg.bwd_mode not in ("save_p", "save_p_triton", "save_p_triton_bwd", "save_p_triton_full"):
        # recompute: no P in HBM; q, k, v, o, dO, cotangents and gradients, LSE, D, E, F
        return float(21 * e * bh * t * d + 16 * bh * t) if cfg.gradgrad else float(11 * e * bh * t * d + 8 * bh * t)
    if cfg.gradgrad:
        return float(3 * e * bh * a + 21 * e * bh * t * d + 12 * bh * t)
    return float(2 * e * bh * a + 11 * e * bh * t * d + 8 * bh * t)


def roofline_us(cfg: Config) -> Dict[str, float]:
    tag = DTYPE_TAG[cfg.torch_dtype]
    f, b = step_flops(cfg), step_bytes(cfg)
    t_f = f / (PEAK_TFLOPS[tag] * 1e12) * 1e6
    t_b = b / (PEAK_HBM_GBS * 1e9) * 1e6
    return {"flops": f, "bytes": b, "t_mfma_us": t_f, "t_hbm_us": t_b, "roofline_us": max(t_f, t_b),
            "bound": "mfma" if t_f >= t_b else "hbm"}


# Per-kernel algorithmic model: (flop coefficient c: flops = c*BH*d*A,
# P passes (fraction of A*e bytes), number of [T,d] tensors moved, fp32 row vectors moved).
_KERNEL = {
    # forward writing P: products QK^T, PV; P written once; q,k,v read, o written; lse written
    "ttt_attn_fwd/p": (4, 1, 4, 1),
    # forward without P: QK^T, PV; q,k,v,o; lse
    "ttt_attn_fwd": (4, 0, 4, 1),
    # dQ from P: dP = dO V^T, dQ = dS K; P read; k, v, do, o read, dq written; D written
    "ttt_attn_bwd_dq/p": (4, 1, 5, 1),
    "ttt_attn_bwd_dq": (6, 0, 6, 2),
    # dK,dV from P: dV, dP, dK; P read; q, v, do read, dk, dv written; D read
    "ttt_attn_bwd_dkdv/p": (6, 1, 5, 1),
    "ttt_attn_bwd_dkdv": (8, 0, 6, 2),
    # grad-grad row pass: dP, gdS (2), gP1, dS gK, gS K; P read; q,k,v,do,gq,gk,gv and the first
    # backward's dQ read (the dQ form, which the autograd path runs), GQ written; D read, E and F written
    "ttt_attn_gg_row/p": (12, 1, 9, 3),
    "ttt_attn_gg_row": (14, 0, 9, 4),
    # grad-grad column pass: dP, gdS (2), gP1, dS^T gQ, gS^T Q, gdP^T dO; P read;
    # 7 inputs, GK and GV written; D, E, F read
    "ttt_attn_gg_col/p": (14, 1, 9, 3),
    "ttt_attn_gg_col": (16, 0, 9, 4),
}


def kernel_model(name: str, cfg: Config, with_p: bool) -> Dict[str, float]:
    key = name + ("/p" if with_p else "")
    c, ppass, ntd, nvec = _KERNEL[key]
    e = torch.tensor([], dtype=cfg.torch_dtype).element_size()
    bh, a = cfg.b * cfg.h, cfg_area(cfg)
    flops = float(c * bh * cfg.d * a)
    byts = float(ppass * e * bh * a + ntd * e * bh * cfg.t * cfg.d + 4 * nvec * bh * cfg.t)
    tag = DTYPE_TAG[cfg.torch_dtype]
    t_f = flops / (PEAK_TFLOPS[tag] * 1e12)
    t_b = byts / (PEAK_HBM_GBS * 1e9)
    return {"flops": flops, "bytes": byts, "bound": "mfma" if t_f >= t_b else "hbm"}
