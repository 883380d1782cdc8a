"""Comparison helpers shared by the tests."""
import numpy as np
import torch

FP32_TOL = 1e-5   # relative tolerance for float32 results (outputs and gradients)


def to_np(x):
    if isinstance(x, torch.Tensor):
        return x.detach().to("cpu").double().numpy()
    return np.asarray(x, dtype=np.float64)


def rel_err(got, ref) -> float:
    """max(|got-ref|) / max(|ref|): the infinity-norm relative error of a whole tensor."""
    g, r = to_np(got), to_np(ref)
    assert g.shape == r.shape, (g.shape, r.shape)
    if r.size == 0:
        return 0.0
    scale = np.abs(r).max()
    diff = np.abs(g - r).max()
    if scale == 0:
        return float(diff)
    return float(diff / scale)


def assert_rel(got, ref, tol=FP32_TOL, what=""):
    e = rel_err(got, ref)
    assert e <= tol, f"{what}: relative error {e:.3e} > {tol:.1e}"
    return e


def assert_equal(got, ref, what=""):
    g = got.detach().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    r = ref.detach().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    bad = np.nonzero(g != r)[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: {g[bad[:5]]} vs {r[bad[:5]]}"
