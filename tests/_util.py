"""Comparison helpers shared by the tests (tolerances are stated where used)."""
import numpy as np
import torch

# fp16/bf16: relative Frobenius error against the float64 math on the same
# (rounded) inputs; fp32: max-abs error.
REL_FRO_16 = 2e-2
MAX_ABS_32 = 1e-5


def to_np(x):
    if isinstance(x, torch.Tensor):
        return x.detach().to("cpu", torch.float64).numpy()
    return np.asarray(x, dtype=np.float64)


def rel_fro(got, ref) -> float:
    g, r = to_np(got), to_np(ref)
    den = np.linalg.norm(r.ravel())
    return float(np.linalg.norm((g - r).ravel()) / max(den, 1e-30))


def max_abs(got, ref) -> float:
    return float(np.max(np.abs(to_np(got) - to_np(ref)))) if np.size(to_np(ref)) else 0.0


# A reference whose RMS is below this is treated as zero: relative error is
# then meaningless and the check falls back to max-abs against this floor
# (e.g. dQ at T=1, where the softmax has a single entry and dS = 0 exactly).
ZERO_RMS = 1e-6
ZERO_ABS_16 = 1e-3


def check_f32_scaled(name, got, ref, abs_tol=MAX_ABS_32):
    """fp32 max-abs error against abs_tol times the reference's largest
    magnitude where that exceeds 1 (values of the helper Functions' VJPs reach
    ~10, where fp32 rounding of their own dot products is ~1e-6 relative)."""
    r = to_np(ref)
    scale = max(1.0, float(np.max(np.abs(r)))) if r.size else 1.0
    err = max_abs(got, ref)
    assert err <= abs_tol * scale, f"{name}: max-abs {err:.3e} > {abs_tol:.1e} x {scale:.2f}"
    return err


def check(name, got, ref, dtype, rel_tol=REL_FRO_16, abs_tol=MAX_ABS_32):
    r = to_np(ref)
    if dtype == torch.float32:
        err = max_abs(got, ref)
        assert err <= abs_tol, f"{name}: max-abs {err:.3e} > {abs_tol:.1e}"
    elif r.size and np.sqrt(np.mean(r * r)) < ZERO_RMS:
        err = max_abs(got, ref)
        assert err <= ZERO_ABS_16, f"{name}: reference is ~0 and max-abs {err:.3e} > {ZERO_ABS_16:.1e}"
    else:
        err = rel_fro(got, ref)
        assert err <= rel_tol, f"{name}: rel-Frobenius {err:.3e} > {rel_tol:.1e}"
    return err
