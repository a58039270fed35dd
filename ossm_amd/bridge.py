"""Autograd bridges over the MI355X scan library, mirroring the reference's
kernel bridges (the L2 layer above ``ossm._kernels``):

* D-LinOSS: ``run_dlinoss``, ``has_kernels``, ``extension_error``, the
  ``ossm::dlinoss_<v>_{forward,backward}`` torch.library operators with Meta
  implementations (_dlinoss_scan.py:176-406) and one autograd Function per
  variant over them — reference src/ossm/models/_dlinoss_scan.py:416-680.
  Forward saves ``(a, g, step, bu, states)`` and returns ``states[..., 1]``;
  backward passes ``grad_output.contiguous()`` (:461-498).
* Selective D-LinOSS: ``run_sdlinoss`` and ``SdlinossFn``
  (_sdlinoss_scan.py:286-452), same save/return semantics.
* LinOSS: ``try_run_scan`` (_linoss_scan.py:44-63) plus ``LinossScanFn`` whose
  backward is the native ``linoss_scan_backward`` instead of the reference's
  Python loop (models/linoss.py:83-151), and ``LinossMatrixScanFn`` /
  ``run_associative_scan``, the same with the reference's ``_LinossScanFn``
  interface (``a_matrix`` [P, 2, 2], ``b_seq``), which ``ossm_amd.linoss.LinOSSLayer``
  uses and which can replace ``_LinossScanFn`` under the reference's layer.
* Selective scan: ``try_selective_scan`` and ``SelectiveScanFn``
  (_selective_scan.py:127-297): fp32 only, the no-grad shortcut, the
  ``(out, chunk_states, raw_out)`` forward saved for the backward.
* Diagonal scans (LRU, S5): ``try_run_lru_scan`` / ``try_run_s5_scan``
  (_lru_scan.py:21-40, _s5_scan.py:21-40) over ``DiagScanFn``, which saves
  ``(lambda_bar, states)`` like _LRUScanFn / _S5ScanFn (lru.py:33-80,
  s5.py:118-165) and runs the backward on the device instead of their Python
  loop over time.

Differences from the reference bridges, on purpose: there is no pure-PyTorch
fallback and no swallowed RuntimeError.  A missing library is an ImportError
at import time; an unsupported dtype or device raises RuntimeError.  (When this
library is installed as ``ossm._kernels`` under the reference's own bridges,
those bridges keep their fp64 and error fallbacks; this module is for callers
that use the MI355X path directly.)
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _kernels

__all__ = [
    "has_kernels", "extension_error", "run_dlinoss", "run_dlinoss_imex1", "DlinossFn", "CUSTOM_OPS",
    "run_sdlinoss", "SdlinossFn",
    "try_run_scan", "LinossScanFn", "LinossMatrixScanFn", "run_associative_scan",
    "try_selective_scan", "SelectiveScanFn",
    "DiagScanFn", "try_run_lru_scan", "try_run_s5_scan",
]

SUPPORTED_VARIANTS = ("imex1", "imex2", "im", "ex")


def has_kernels(variant: Optional[str] = None) -> bool:
    """True when the device kernels for ``variant`` (or all variants) exist
    (reference _dlinoss_scan.py:416-435)."""
    if variant is None:
        return all(has_kernels(v) for v in SUPPORTED_VARIANTS)
    variant = variant.lower()
    if variant not in SUPPORTED_VARIANTS:
        raise ValueError(f"Unknown D-LinOSS variant '{variant}'.")
    return hasattr(_kernels, f"dlinoss_{variant}_forward")


def extension_error() -> Optional[Exception]:
    """Always None: the library loads at import or the import fails."""
    return None


# ------------------------------------------------------------------ D-LinOSS
# torch.library operators ``ossm::dlinoss_<v>_{forward,backward}`` with the
# reference's schema strings (_dlinoss_scan.py:183-206), so torch.compile can
# trace the scans with fake tensors and still call the device kernels: the
# CompositeExplicitAutograd implementation is the drop-in module's entry
# point, the Meta implementation only produces outputs of the right shape and
# dtype.  When the operators already exist (the reference's bridge imported
# in the same process defines them too, over ``ossm._kernels``), the existing
# definitions and implementations are kept.
_OP_FWD = "dlinoss_{v}_forward(Tensor a_diag, Tensor g_diag, Tensor step, Tensor bu) -> Tensor"
_OP_BWD = ("dlinoss_{v}_backward(Tensor a_diag, Tensor g_diag, Tensor step, Tensor bu, "
           "Tensor states, Tensor grad_output) -> (Tensor, Tensor, Tensor, Tensor)")
_OPS_LIBRARY = None


def _forward_meta(a_diag: Tensor, g_diag: Tensor, step: Tensor, bu: Tensor) -> Tensor:
    return bu.new_empty((*bu.shape, 2))


def _backward_meta(a_diag: Tensor, g_diag: Tensor, step: Tensor, bu: Tensor, states: Tensor,
                   grad_output: Tensor):
    return (torch.empty_like(a_diag), torch.empty_like(g_diag), torch.empty_like(step),
            torch.empty_like(bu))


def _register_ops() -> bool:
    """Define and implement the operators; False when torch.library is missing."""
    global _OPS_LIBRARY
    try:
        from torch.library import Library
    except ImportError:  # pragma: no cover - very old torch
        return False
    try:
        lib = Library("ossm", "DEF")
        for v in SUPPORTED_VARIANTS:
            lib.define(_OP_FWD.format(v=v))
            lib.define(_OP_BWD.format(v=v))
    except RuntimeError:
        lib = Library("ossm", "IMPL")  # defined already: keep the definitions
    for v in SUPPORTED_VARIANTS:
        for name, impl, meta in ((f"dlinoss_{v}_forward", getattr(_kernels, f"dlinoss_{v}_forward"),
                                  _forward_meta),
                                 (f"dlinoss_{v}_backward", getattr(_kernels, f"dlinoss_{v}_backward"),
                                  _backward_meta)):
            for fn, key in ((impl, "CompositeExplicitAutograd"), (meta, "Meta")):
                try:
                    lib.impl(name, fn, key)
                except RuntimeError:
                    pass  # an implementation is registered already
    _OPS_LIBRARY = lib
    return True


CUSTOM_OPS = _register_ops()


def _dlinoss_op(variant: str, direction: str):
    if CUSTOM_OPS:
        return getattr(torch.ops.ossm, f"dlinoss_{variant}_{direction}")
    return getattr(_kernels, f"dlinoss_{variant}_{direction}")


class DlinossFn(torch.autograd.Function):
    """Autograd bridge of one D-LinOSS variant (reference _DlinossImex1Fn and
    siblings, _dlinoss_scan.py:458-600), through the ``ossm::dlinoss_*``
    operators."""

    @staticmethod
    def forward(ctx, variant: str, a_diag: Tensor, g_diag: Tensor, step: Tensor,
                bu: Tensor) -> Tensor:  # type: ignore[override]
        states = _dlinoss_op(variant, "forward")(a_diag, g_diag, step, bu)
        ctx.variant = variant
        ctx.save_for_backward(a_diag, g_diag, step, bu, states)
        return states[..., 1]

    @staticmethod
    def backward(ctx, grad_output: Tensor):  # type: ignore[override]
        a_diag, g_diag, step, bu, states = ctx.saved_tensors
        grad_a, grad_g, grad_step, grad_bu = _dlinoss_op(ctx.variant, "backward")(
            a_diag, g_diag, step, bu, states, grad_output.contiguous())
        return None, grad_a, grad_g, grad_step, grad_bu


def run_dlinoss(variant: str, a_diag: Tensor, g_diag: Tensor, step: Tensor, bu: Tensor) -> Tensor:
    """x = states[..., 1] of the D-LinOSS recurrence for ``variant``
    (reference run_dlinoss, _dlinoss_scan.py:630-680).  bu is [L, B, P]
    complex on the device; a, g, step are [P] real.  The precision follows the
    reference's rule for higher-precision inputs (_dlinoss_scan.py:35-48,
    648-654): float64 / complex128 when any coefficient is float64, else
    float32 / complex64, with every input cast to it; both run on the device
    kernels (the reference sends the float64 case to its Python loop)."""
    variant = variant.lower()
    if variant not in SUPPORTED_VARIANTS:
        raise ValueError(f"Unknown D-LinOSS variant '{variant}'.")
    if bu.numel() == 0:
        return bu
    real = torch.float64 if any(t.dtype == torch.float64 for t in (a_diag, g_diag, step)) \
        else torch.float32
    cplx = torch.complex128 if real == torch.float64 else torch.complex64
    a_diag, g_diag, step = (t.to(dtype=real) for t in (a_diag, g_diag, step))
    return DlinossFn.apply(variant, a_diag, g_diag, step, bu.to(dtype=cplx))


def run_dlinoss_imex1(a_diag: Tensor, g_diag: Tensor, step: Tensor, bu: Tensor) -> Tensor:
    """reference run_dlinoss_imex1 (_dlinoss_scan.py:683-686)."""
    return run_dlinoss("imex1", a_diag, g_diag, step, bu)


# -------------------------------------------------------- selective D-LinOSS
class SdlinossFn(torch.autograd.Function):
    """Autograd bridge of one selective D-LinOSS variant (reference
    _SdlinossImex1Fn and siblings, _sdlinoss_scan.py:286-379): the forward saves
    ``(A, G, step, bu, states)`` and returns ``states[..., 1]``; the backward
    passes ``grad_output.contiguous()``."""

    @staticmethod
    def forward(ctx, variant: str, A: Tensor, G: Tensor, step: Tensor,
                bu: Tensor) -> Tensor:  # type: ignore[override]
        states = getattr(_kernels, f"sdlinoss_{variant}_forward")(A, G, step, bu)
        ctx.variant = variant
        ctx.save_for_backward(A, G, step, bu, states)
        return states[..., 1]

    @staticmethod
    def backward(ctx, grad_output: Tensor):  # type: ignore[override]
        A, G, step, bu, states = ctx.saved_tensors
        grad_A, grad_G, grad_step, grad_bu = getattr(_kernels, f"sdlinoss_{ctx.variant}_backward")(
            A, G, step, bu, states, grad_output.contiguous())
        return None, grad_A, grad_G, grad_step, grad_bu


def run_sdlinoss(variant: str, a_diag: Tensor, g_diag: Tensor, step: Tensor, bu: Tensor) -> Tensor:
    """x = states[..., 1] of the selective D-LinOSS recurrence (reference
    run_sdlinoss, _sdlinoss_scan.py:382-452).  bu is [L, B, M] complex64 (float32
    parameters) or complex128 (float64 parameters) on the device; A, G, step are
    shaped (M,), (L, M), (B, M) or (L|1, B|1, M);
    their gradients come back in the same shapes (summed over broadcast axes)."""
    variant = variant.lower()
    if variant not in SUPPORTED_VARIANTS:
        raise ValueError(
            f"Unsupported variant '{variant}'. Expected one of {', '.join(SUPPORTED_VARIANTS)}.")
    if bu.dim() != 3:
        raise ValueError("bu must be (length, batch, ssm_size) complex.")
    if bu.size(0) == 0:
        return bu.new_empty((0, bu.size(1), bu.size(2)))
    return SdlinossFn.apply(variant, a_diag, g_diag, step, bu)


# -------------------------------------------------------------------- LinOSS
class LinossScanFn(torch.autograd.Function):
    """``s_t = M s_{t-1} + b_t`` with complex M per oscillator (reference
    _LinossScanFn, models/linoss.py:57-157); the backward runs on the device."""

    @staticmethod
    def forward(ctx, m11: Tensor, m12: Tensor, m21: Tensor, m22: Tensor,
                b_seq: Tensor) -> Tensor:  # type: ignore[override]
        states = _kernels.linoss_scan(m11, m12, m21, m22, b_seq)
        ctx.save_for_backward(m11, m12, m21, m22, states)
        return states

    @staticmethod
    def backward(ctx, grad_states: Tensor):  # type: ignore[override]
        m11, m12, m21, m22, states = ctx.saved_tensors
        grad_m, grad_b = _kernels.linoss_scan_backward(m11, m12, m21, m22, states,
                                                       grad_states.contiguous())
        return grad_m[:, 0, 0], grad_m[:, 0, 1], grad_m[:, 1, 0], grad_m[:, 1, 1], grad_b


_M_ENTRIES = ((0, 0), (0, 1), (1, 0), (1, 1))


class LinossMatrixScanFn(torch.autograd.Function):
    """The reference's ``_LinossScanFn(a_matrix, b_seq)`` interface
    (models/linoss.py:57-151) on the device, backward included: ``a_matrix`` is
    [P, 2, 2] (real or complex), ``b_seq`` [L, B, P, 2] complex.  The gradient
    of ``a_matrix`` is the reference's ``sum_b grad_i conj(s_j,t-1)``, kept
    complex for a complex ``a_matrix`` and reduced to its real part for a real
    one (linoss.py:122-132).  Sequences of length 0 or 1 are returned as given,
    as the reference does (s_0 = b_0)."""

    @staticmethod
    def forward(ctx, a_matrix: Tensor, b_seq: Tensor) -> Tensor:  # type: ignore[override]
        if b_seq.size(0) <= 1:
            ctx.save_for_backward(a_matrix, b_seq)
            return b_seq
        b_seq = b_seq.contiguous()
        ms = [a_matrix[:, i, j].to(dtype=b_seq.dtype).contiguous() for i, j in _M_ENTRIES]
        states = _kernels.linoss_scan(*ms, b_seq)
        ctx.save_for_backward(a_matrix, states)
        return states

    @staticmethod
    def backward(ctx, grad_output: Tensor):  # type: ignore[override]
        a_matrix, states = ctx.saved_tensors
        if grad_output.size(0) == 0:
            return torch.zeros_like(a_matrix), grad_output
        ms = [a_matrix[:, i, j].to(dtype=grad_output.dtype).contiguous() for i, j in _M_ENTRIES]
        grad_m, grad_b = _kernels.linoss_scan_backward(*ms, states.contiguous(),
                                                       grad_output.contiguous())
        if not torch.is_complex(a_matrix):
            grad_m = grad_m.real
        return grad_m.to(a_matrix.dtype), grad_b


def run_associative_scan(a_matrix: Tensor, b_seq: Tensor) -> Tensor:
    """reference ``_run_associative_scan`` (models/linoss.py:154-157)."""
    return LinossMatrixScanFn.apply(a_matrix, b_seq)


def try_run_scan(m11: Tensor, m12: Tensor, m21: Tensor, m22: Tensor, b_seq: Tensor) -> Tensor:
    """States [L, B, P, 2] of the LinOSS scan (reference try_run_scan,
    _linoss_scan.py:44-63), differentiable through the native backward."""
    if b_seq.numel() == 0:
        return b_seq
    return LinossScanFn.apply(m11, m12, m21, m22, b_seq)


# ----------------------------------------------------------- selective scan
class SelectiveScanFn(torch.autograd.Function):
    """Reference _SelectiveScanFn (_selective_scan.py:199-297), device path."""

    @staticmethod
    def forward(ctx, inputs: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor,
                gate: Optional[Tensor], chunk_length: int) -> Tensor:  # type: ignore[override]
        if inputs.dtype != torch.float32:
            raise RuntimeError("Selective scan kernels require float32 inputs")
        if dt.dtype != torch.float32 or A.dtype != torch.float32:
            raise RuntimeError("Selective scan kernels require float32 parameters")
        if gate is not None and gate.dtype != torch.float32:
            raise RuntimeError("Selective scan kernels require float32 gate")
        if int(chunk_length) <= 0:
            raise RuntimeError("chunk_length must be positive")
        gate_c = gate.contiguous() if gate is not None else None
        tensors = [x.contiguous() for x in (inputs, dt, A, B, C)]
        out, chunk_states, raw = _kernels.selective_scan_cuda(*tensors, gate_c, int(chunk_length))
        ctx.has_gate = gate_c is not None
        ctx.chunk = int(chunk_length)
        ctx.save_for_backward(*tensors, gate_c if gate_c is not None else inputs.new_empty(0),
                              chunk_states, raw)
        return out

    @staticmethod
    def backward(ctx, grad_output: Tensor):  # type: ignore[override]
        inputs, dt, A, B, C, gate_saved, chunk_states, raw = ctx.saved_tensors
        gate = gate_saved if ctx.has_gate else None
        grads = _kernels.selective_scan_cuda_backward(grad_output.contiguous(), inputs, dt, A, B, C,
                                                      gate, chunk_states, raw, ctx.chunk)
        du, ddt, dA, dB, dC, dz = grads
        return du, ddt, dA, dB, dC, (dz if ctx.has_gate else None), None


def try_selective_scan(inputs: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor,
                       gate: Optional[Tensor], chunk_length: int = 64) -> Tensor:
    """Fused selective scan on the device (reference try_selective_scan,
    _selective_scan.py:127-196): the no-grad case skips the autograd wrapper."""
    if inputs.numel() == 0:
        return inputs
    if not inputs.is_cuda:
        raise RuntimeError("try_selective_scan: the MI355X path needs device tensors")
    requires_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (inputs, dt, A, B, C, gate))
    if not requires_grad:
        return _kernels.selective_scan_cuda(inputs, dt, A, B, C, gate, chunk_length)[0]
    return SelectiveScanFn.apply(inputs, dt, A, B, C, gate, chunk_length)


# ------------------------------------------------------ diagonal scans (LRU, S5)
class DiagScanFn(torch.autograd.Function):
    """``x_t = lambda_bar * x_{t-1} + b_t`` over complex ``b_seq [L, B, P]``
    (reference _LRUScanFn / _S5ScanFn, lru.py:33-80, s5.py:118-165): the forward
    saves ``(lambda_bar, states)``; the backward returns ``(grad_lambda,
    grad_b)`` from the device kernel (grad_b_t = g_t with g_t = grad_t +
    conj(lambda_bar) g_{t+1}; grad_lambda = sum over t, b of g_t conj(x_{t-1}))."""

    @staticmethod
    def forward(ctx, name: str, lambda_bar: Tensor, b_seq: Tensor) -> Tensor:  # type: ignore[override]
        if b_seq.size(0) == 0:
            ctx.save_for_backward(lambda_bar, b_seq)
            return b_seq
        fwd = _kernels.lru_scan if name == "lru" else _kernels.s5_scan
        lam = lambda_bar.resolve_conj()
        result = fwd(lam.real.contiguous(), lam.imag.contiguous(),
                     torch.view_as_real(b_seq.contiguous()))
        states = torch.view_as_complex(result)
        ctx.save_for_backward(lambda_bar, states)
        return states

    @staticmethod
    def backward(ctx, grad_output: Tensor):  # type: ignore[override]
        lambda_bar, states = ctx.saved_tensors
        if grad_output.size(0) == 0:
            return None, torch.zeros_like(lambda_bar), grad_output
        lam = lambda_bar.resolve_conj()
        grad_lambda, grad_b = _kernels.lru_scan_backward(
            lam.real.contiguous(), lam.imag.contiguous(), torch.view_as_real(states),
            torch.view_as_real(grad_output.resolve_conj().contiguous()))
        return None, torch.view_as_complex(grad_lambda), torch.view_as_complex(grad_b)


def try_run_lru_scan(lambda_bar: Tensor, b_seq: Tensor) -> Tensor:
    """Complex states ``[L, B, P]`` of the LRU scan (reference try_run_lru_scan,
    _lru_scan.py:21-40), differentiable through the native backward."""
    if b_seq.numel() == 0:
        return b_seq
    return DiagScanFn.apply("lru", lambda_bar, b_seq)


def try_run_s5_scan(lambda_bar: Tensor, b_seq: Tensor) -> Tensor:
    """Complex states ``[L, B, P]`` of the S5 scan (reference try_run_s5_scan,
    _s5_scan.py:21-40), differentiable through the native backward."""
    if b_seq.numel() == 0:
        return b_seq
    return DiagScanFn.apply("s5", lambda_bar, b_seq)
