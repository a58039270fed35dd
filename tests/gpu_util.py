"""Shared helpers for the GPU parity tests (the tests, not the product)."""

from __future__ import annotations

import numpy as np
import pytest
import torch


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")


def announce(msg: str) -> None:
    """Print which case runs before its GPU work starts (flushed)."""
    print(f"[gpu-case] {msg}", flush=True)


def to_dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def assert_close(actual, expected, rtol, atol, what=""):
    np.testing.assert_allclose(np.asarray(actual), np.asarray(expected), rtol=rtol, atol=atol,
                               err_msg=what)


def assert_parity(actual, ref32, ref64, rtol=1e-4, atol=1e-5, what="", factor=2.0):
    """Parity with the reference's fp32 result at (rtol, atol) elementwise.

    Long fp32 recurrences carry rounding error of their own: where an element
    misses the elementwise bound, the check falls back to fp64 truth and
    requires the GPU's worst error against it to be within `factor` of the
    fp32 reference's own worst error (plus atol), i.e. the GPU is as accurate
    as the reference kernel."""
    a = np.asarray(actual)
    r32 = np.asarray(ref32)
    r64 = np.asarray(ref64)
    viol = np.abs(a - r32) > atol + rtol * np.abs(r32)
    if not viol.any():
        return
    e_gpu = float(np.abs(a.astype(r64.dtype) - r64).max())
    e_ref = float(np.abs(r32.astype(r64.dtype) - r64).max())
    assert e_gpu <= factor * e_ref + atol, (
        f"{what}: {int(viol.sum())}/{viol.size} elements outside rtol={rtol}/atol={atol} of the "
        f"fp32 reference and max|gpu-fp64|={e_gpu:.3e} > {factor}*max|ref-fp64|={e_ref:.3e}+atol")


def sum_atol(ref64, k=2e-5) -> float:
    """The magnitude-scaled absolute tolerance of a gradient that is a sum
    over many terms (over batch, time or channels): k * max(1, max|ref|).
    The sum's rounding scales with its terms, not with each element."""
    return k * max(1.0, float(np.abs(np.asarray(ref64)).max()))


def assert_grad_parity(actual, ref32, ref64, what="", rtol=1e-4, k=2e-5):
    """Elementwise gradient parity: assert_parity at rtol and the
    magnitude-scaled atol of sum_atol(ref64, k), i.e. every element within
    tolerance of an fp32 computation of the same gradient or, where that
    computation's own rounding misses, no less accurate than it against fp64
    truth."""
    assert_parity(np.asarray(actual), np.asarray(ref32), np.asarray(ref64), rtol, sum_atol(ref64, k),
                  what)


def rel_fro(a, b) -> float:
    a = np.asarray(a, np.complex128 if np.iscomplexobj(a) else np.float64)
    b = np.asarray(b, a.dtype)
    return float(np.linalg.norm((a - b).ravel()) / max(np.linalg.norm(b.ravel()), 1e-300))


def no_device_errors():
    from ossm_amd import _lib

    bits = _lib.device_error_bits()
    assert bits == 0, f"scan kernels raised device error bits {bits:#x}"


def _dlinoss_M(variant, a, g, dt):
    """Transition matrices [P,2,2] (table of reference _dlinoss_scan.py:54-101),
    used only to keep test inputs inside each variant's stable region."""
    one = np.ones_like(a)
    if variant == "imex1":
        S = 1 + dt * g
        m = [[one / S, -dt * dt * a / S], [one / S, 1 - dt * dt * a / S]]
    elif variant == "imex2":
        m = [[1 - dt * g, -dt * a], [dt * (1 - dt * g), 1 - dt * dt * a]]
    elif variant == "im":
        D = 1 + dt * g + dt * dt * a
        m = [[one / D, -dt * a / D], [dt / D, (1 + dt * g) / D]]
    else:
        m = [[1 - dt * g, -dt * a], [dt, one]]
    return np.stack([np.stack(r, -1) for r in m], -2)


def dlinoss_inputs(L, B, P, seed, stable=True, variant=None):
    """Seeded D-LinOSS inputs with the distributions of BASELINE configs 2/5:
    A ~ U(0.1, 1), G ~ U(0, 1), dt = sigmoid(N(0,1)), A projected into the
    stable band of DampedLinOSSLayer._project_parameters (dlinoss.py:252-267),
    bu complex N(0, 1) (the scan input after the B projection)."""
    rng = np.random.default_rng(seed)
    a = rng.uniform(0.1, 1.0, P)
    g = rng.uniform(0.0, 1.0, P)
    dt = 1.0 / (1.0 + np.exp(-rng.normal(size=P)))
    if stable:
        s = dt * g
        base = np.sqrt(np.maximum(1.0 + s, 1e-6))
        denom = np.maximum(dt * dt, 1e-6)
        lo = (2.0 + s - 2.0 * base) / denom
        hi = (2.0 + s + 2.0 * base) / denom
        a = np.clip(a, lo, hi)
    if variant is not None:
        # keep every oscillator non-expanding for this variant: halve dt
        # until the spectral radius of M is at most 1
        for _ in range(60):
            rho = np.abs(np.linalg.eigvals(_dlinoss_M(variant, a, g, dt))).max(-1)
            bad = rho > 1.0 + 1e-6
            if not bad.any():
                break
            dt = np.where(bad, dt * 0.5, dt)
    bu = (rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))).astype(np.complex64)
    go = (rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))).astype(np.complex64)
    return a.astype(np.float32), g.astype(np.float32), dt.astype(np.float32), bu, go
