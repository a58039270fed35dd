"""Drop-in replacement for the reference extension module ``ossm._kernels``.

Same names, argument order, keyword names, return structure and RuntimeError
messages as the pybind module of the reference (src/ossm/csrc/bindings.cpp:159-224),
so the reference's kernel bridges (models/_dlinoss_scan.py, _linoss_scan.py,
_selective_scan.py) run unchanged on top of it.  Device tensors (ROCm tensors
report ``is_cuda``) run on the MI355X through libossm_scan.so; outputs are
allocated here with torch's caching allocator on the input's device and
stream, and the library only launches kernels.

CPU tensors are not this module's job.  The reference's CPU kernels can be
attached with :func:`set_cpu_delegate` (any object exposing the reference's
CPU entry points, e.g. the reference's own ``ossm._kernels`` build); without a
delegate a CPU call raises RuntimeError, which the reference bridges treat as
"kernel unavailable".

``linear_rnn_scan`` has no HIP implementation in this build: it exists so
attribute lookups behave like the reference's module, and on device tensors it
raises RuntimeError (the reference's bridge then runs its Python loop).
"""

from __future__ import annotations

from typing import Any, List, Optional

import torch

from . import _lib

__all__ = [
    "linoss_scan",
    "linoss_scan_backward",
    "dlinoss_imex1_forward", "dlinoss_imex1_backward",
    "dlinoss_imex2_forward", "dlinoss_imex2_backward",
    "dlinoss_im_forward", "dlinoss_im_backward",
    "dlinoss_ex_forward", "dlinoss_ex_backward",
    "selective_scan", "selective_scan_backward",
    "selective_scan_cuda", "selective_scan_cuda_backward",
    "selective_scan_cuda_bf16", "selective_scan_cuda_bf16_backward",
    "sdlinoss_imex1_forward", "sdlinoss_imex1_backward",
    "sdlinoss_imex2_forward", "sdlinoss_imex2_backward",
    "sdlinoss_im_forward", "sdlinoss_im_backward",
    "sdlinoss_ex_forward", "sdlinoss_ex_backward",
    "lru_scan", "s5_scan", "lru_scan_backward", "s5_scan_backward",
    "linear_rnn_scan",
    "set_cpu_delegate",
]

_VARIANT_CODE = {"imex1": 0, "imex2": 1, "im": 2, "ex": 3}
_MAX_DSTATE = 256  # reference MAX_DSTATE (selective_scan_common.h:41)
_ELEM = {torch.float32: 0, torch.bfloat16: 1}  # OSSM_ELEM_F32, OSSM_ELEM_BF16

_cpu_delegate: Optional[Any] = None


def set_cpu_delegate(module: Optional[Any]) -> None:
    """Route CPU-tensor calls to ``module`` (an object with the reference's CPU
    entry points).  ``None`` removes the delegate."""
    global _cpu_delegate
    _cpu_delegate = module


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _delegate(name: str, *args):
    if _cpu_delegate is None or not hasattr(_cpu_delegate, name):
        raise RuntimeError(
            f"{name}: CPU tensors are not handled by the MI355X scan library "
            "(no CPU delegate attached)")
    return getattr(_cpu_delegate, name)(*args)


def _on_device(*tensors: Optional[torch.Tensor]) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        _check(t.is_cuda, "All tensors must be on the same device")
        if dev is None:
            dev = t.device
        _check(t.device == dev, "All tensors must be on the same device")


# ------------------------------------------------------------------- D-LinOSS
_DLINOSS_ENTRIES = {torch.complex64: (torch.float32, ""), torch.complex128: (torch.float64, "_f64")}
_TYPE_NAMES = {torch.float32: "Float", torch.float64: "Double", torch.complex64: "ComplexFloat",
               torch.complex128: "ComplexDouble"}


def _dlinoss_entry(variant: str, direction: str, bu, coeffs, same_as_bu) -> str:
    """The C entry for bu's dtype, with the reference dispatcher's dtype rules
    (dlinoss_imex1_cuda.cu:196, 234): complex64 or complex128 bu
    (AT_DISPATCH_COMPLEX_TYPES), coefficient diagonals of its value type and
    states / grad_output of its own type (data_ptr<T>)."""
    if bu.dtype not in _DLINOSS_ENTRIES:
        raise RuntimeError(f'"dlinoss_{variant}_{direction}_cuda" not implemented for '
                           f"'{_TYPE_NAMES.get(bu.dtype, str(bu.dtype))}'")
    real, suffix = _DLINOSS_ENTRIES[bu.dtype]
    for t, want in [(c, real) for c in coeffs] + [(c, bu.dtype) for c in same_as_bu]:
        _check(t.dtype == want, f"expected scalar type {_TYPE_NAMES[want]} but found "
                                f"{_TYPE_NAMES.get(t.dtype, str(t.dtype))}")
    return f"ossm_dlinoss_{direction}{suffix}"


def _dlinoss_forward(variant: str, a_diag, g_diag, step, bu):
    # dlinoss_imex1.cpp:317-352 (same checks in the other variants)
    _check(a_diag.dim() == 1 and g_diag.dim() == 1 and step.dim() == 1,
           "Coefficient diagonals must be 1-D tensors")
    _check(bu.dim() == 3, "bu must have shape (length, batch, ssm_size)")
    length, batch, ssm = bu.shape
    _check(a_diag.size(0) == ssm and g_diag.size(0) == ssm and step.size(0) == ssm,
           "Coefficient diagonals must match state size")
    output = torch.empty((length, batch, ssm, 2), dtype=bu.dtype, device=bu.device)
    if length == 0:
        return output
    _check(a_diag.is_contiguous() and g_diag.is_contiguous() and step.is_contiguous(),
           "Coefficient diagonals must be contiguous")
    _check(bu.is_contiguous(), "bu must be contiguous")
    if not bu.is_cuda:
        return _delegate(f"dlinoss_{variant}_forward", a_diag, g_diag, step, bu)
    _on_device(a_diag, g_diag, step, bu)
    entry = _dlinoss_entry(variant, "forward", bu, (a_diag, g_diag, step), ())
    with torch.cuda.device(bu.device):
        _lib.check(getattr(_lib.load(), entry)(
            _VARIANT_CODE[variant], a_diag.data_ptr(), g_diag.data_ptr(), step.data_ptr(),
            bu.data_ptr(), output.data_ptr(), length, batch, ssm, _lib.stream_of(bu)))
    return output


def _dlinoss_backward(variant: str, a_diag, g_diag, step, bu, states, grad_output):
    # dlinoss_imex1.cpp:354-390
    _check(a_diag.dim() == 1 and g_diag.dim() == 1 and step.dim() == 1,
           "Coefficient diagonals must be 1-D tensors")
    _check(states.dim() == 4 and states.size(3) == 2,
           "states must have shape (length, batch, ssm_size, 2)")
    _check(bu.dim() == 3, "bu must have shape (length, batch, ssm_size)")
    _check(grad_output.shape == bu.shape, "grad_output must match bu shape")
    length, batch, ssm = bu.shape
    _check(a_diag.size(0) == ssm and g_diag.size(0) == ssm and step.size(0) == ssm,
           "Coefficient diagonals must match state size")
    _check(tuple(states.shape[:3]) == (length, batch, ssm),
           "states must have shape (length, batch, ssm_size, 2)")
    grad_bu = torch.empty_like(bu)
    if length == 0:
        return [torch.zeros_like(a_diag), torch.zeros_like(g_diag), torch.zeros_like(step), grad_bu]
    # overwritten by the library (it reduces the parameter sums in-kernel)
    grad_a = torch.empty_like(a_diag)
    grad_g = torch.empty_like(g_diag)
    grad_step = torch.empty_like(step)
    _check(a_diag.is_contiguous() and g_diag.is_contiguous() and step.is_contiguous(),
           "Coefficient diagonals must be contiguous")
    _check(bu.is_contiguous(), "bu must be contiguous")
    _check(states.is_contiguous() and grad_output.is_contiguous(),
           "states and grad_output must be contiguous")
    if not bu.is_cuda:
        return _delegate(f"dlinoss_{variant}_backward", a_diag, g_diag, step, bu, states,
                         grad_output)
    _on_device(a_diag, g_diag, step, bu, states, grad_output)
    entry = _dlinoss_entry(variant, "backward", bu, (a_diag, g_diag, step), (states, grad_output))
    with torch.cuda.device(bu.device):
        _lib.check(getattr(_lib.load(), entry)(
            _VARIANT_CODE[variant], a_diag.data_ptr(), g_diag.data_ptr(), step.data_ptr(),
            bu.data_ptr(), states.data_ptr(), grad_output.data_ptr(), grad_a.data_ptr(),
            grad_g.data_ptr(), grad_step.data_ptr(), grad_bu.data_ptr(), length, batch, ssm,
            _lib.stream_of(bu)))
    return [grad_a, grad_g, grad_step, grad_bu]


def dlinoss_imex1_forward(a_diag, g_diag, step, bu):
    return _dlinoss_forward("imex1", a_diag, g_diag, step, bu)


def dlinoss_imex1_backward(a_diag, g_diag, step, bu, states, grad_output):
    return _dlinoss_backward("imex1", a_diag, g_diag, step, bu, states, grad_output)


def dlinoss_imex2_forward(a_diag, g_diag, step, bu):
    return _dlinoss_forward("imex2", a_diag, g_diag, step, bu)


def dlinoss_imex2_backward(a_diag, g_diag, step, bu, states, grad_output):
    return _dlinoss_backward("imex2", a_diag, g_diag, step, bu, states, grad_output)


def dlinoss_im_forward(a_diag, g_diag, step, bu):
    return _dlinoss_forward("im", a_diag, g_diag, step, bu)


def dlinoss_im_backward(a_diag, g_diag, step, bu, states, grad_output):
    return _dlinoss_backward("im", a_diag, g_diag, step, bu, states, grad_output)


def dlinoss_ex_forward(a_diag, g_diag, step, bu):
    return _dlinoss_forward("ex", a_diag, g_diag, step, bu)


def dlinoss_ex_backward(a_diag, g_diag, step, bu, states, grad_output):
    return _dlinoss_backward("ex", a_diag, g_diag, step, bu, states, grad_output)


# --------------------------------------------------------------------- LinOSS
_LINOSS_ENTRIES = {
    torch.complex64: ("ossm_linoss_forward", "ossm_linoss_backward"),
    torch.complex128: ("ossm_linoss_forward_f64", "ossm_linoss_backward_f64"),
}


def linoss_scan(m11, m12, m21, m22, b_seq):
    """linoss_scan.cpp:115-146."""
    output = torch.empty_like(b_seq)
    if b_seq.size(0) == 0:
        return output
    _check(b_seq.dim() == 4,
           f"b_seq must have shape (length, batch, ssm_size, 2), got {list(b_seq.shape)}")
    _check(m11.is_contiguous() and m12.is_contiguous() and m21.is_contiguous()
           and m22.is_contiguous(), "Coefficient tensors must be contiguous")
    _check(b_seq.is_contiguous(), "b_seq must be contiguous")
    if not b_seq.is_cuda:
        return _delegate("linoss_scan", m11, m12, m21, m22, b_seq)
    length, batch, ssm, two = b_seq.shape
    _check(two == 2, "b_seq must have shape (length, batch, ssm_size, 2)")
    _on_device(m11, m12, m21, m22, b_seq)
    # complex64 and complex128, as the reference's device kernel dispatches
    # (AT_DISPATCH_COMPLEX_TYPES, linoss_scan_cuda.cu:139)
    _check(b_seq.dtype in _LINOSS_ENTRIES,
           f"linoss_scan: b_seq must be complex64 or complex128, got {b_seq.dtype}")
    for m in (m11, m12, m21, m22):
        _check(m.dim() == 1 and m.size(0) == ssm, "Coefficient tensors must have shape (ssm_size,)")
        _check(m.dtype == b_seq.dtype, "Coefficient tensors must have b_seq's dtype")
    with torch.cuda.device(b_seq.device):
        _lib.check(getattr(_lib.load(), _LINOSS_ENTRIES[b_seq.dtype][0])(
            m11.data_ptr(), m12.data_ptr(), m21.data_ptr(), m22.data_ptr(), b_seq.data_ptr(),
            output.data_ptr(), length, batch, ssm, _lib.stream_of(b_seq)))
    return output


def linoss_scan_backward(m11, m12, m21, m22, states, grad_output):
    """Native backward of :func:`linoss_scan` (the reference runs it as a Python
    loop, models/linoss.py:83-151).  Returns ``[grad_m [P,2,2], grad_b [L,B,P,2]]``."""
    _check(states.dim() == 4 and states.size(3) == 2,
           "states must have shape (length, batch, ssm_size, 2)")
    _check(grad_output.shape == states.shape, "grad_output must match states shape")
    length, batch, ssm, _ = states.shape
    grad_b = torch.empty_like(grad_output)
    if length == 0:
        return [torch.zeros((ssm, 2, 2), dtype=states.dtype, device=states.device), grad_b]
    grad_m = torch.empty((ssm, 2, 2), dtype=states.dtype, device=states.device)
    _check(states.is_cuda, "linoss_scan_backward: HIP path needs device tensors")
    _on_device(m11, m12, m21, m22, states, grad_output)
    _check(states.dtype in _LINOSS_ENTRIES and grad_output.dtype == states.dtype,
           "linoss_scan_backward: states and grad_output must be both complex64 or both complex128")
    for m in (m11, m12, m21, m22):
        _check(m.dim() == 1 and m.size(0) == ssm and m.is_contiguous() and m.dtype == states.dtype,
               "Coefficient tensors must be contiguous (ssm_size,) of the states' dtype")
    _check(states.is_contiguous() and grad_output.is_contiguous(),
           "states and grad_output must be contiguous")
    with torch.cuda.device(states.device):
        _lib.check(getattr(_lib.load(), _LINOSS_ENTRIES[states.dtype][1])(
            m11.data_ptr(), m12.data_ptr(), m21.data_ptr(), m22.data_ptr(), states.data_ptr(),
            grad_output.data_ptr(), grad_m.data_ptr(), grad_b.data_ptr(), length, batch, ssm,
            _lib.stream_of(states)))
    return [grad_m, grad_b]


# ------------------------------------------------------------- selective scan
def _selective_checks(inputs, dt, A, B, C, gate, name: str,
                      dtype: torch.dtype = torch.float32) -> None:
    # selective_scan_cuda.cu:60-102 (CPU twin: selective_scan_cpu.cpp:15-56);
    # ``dtype`` is the storage type of every tensor but A (float32 for the
    # reference's names, bfloat16 for the *_bf16 extension)
    dn = "float32" if dtype == torch.float32 else "bfloat16"
    _check(inputs.dtype == dtype, f"{name} requires {dn} inputs")
    _check(inputs.dim() == 3, "inputs must have shape (batch, channels, length)")
    _check(dt.device == inputs.device, "dt must be on the same device as inputs")
    _check(dt.dtype == dtype, f"dt must be {dn}")
    _check(dt.shape == inputs.shape, "dt shape mismatch")
    _check(A.device == inputs.device, "A must be on the same device as inputs")
    _check(A.dtype == torch.float32, "A must be float32")
    _check(A.dim() == 2, "A must have shape (channels, state)")
    _check(A.size(0) == inputs.size(1), "A channels mismatch")
    _check(A.size(1) > 0, "state dimension must be positive")
    _check(A.size(1) <= _MAX_DSTATE,
           f"state dimension exceeds supported maximum ({_MAX_DSTATE})")
    _check(B.device == inputs.device, "B must be on the same device as inputs")
    _check(B.dtype == dtype, f"B must be {dn}")
    _check(B.dim() == 3, "B must have shape (batch, length, state)")
    _check(B.size(0) == inputs.size(0) and B.size(1) == inputs.size(2) and B.size(2) == A.size(1),
           "B shape mismatch")
    _check(C.device == inputs.device, "C must be on the same device as inputs")
    _check(C.dtype == dtype, f"C must be {dn}")
    _check(C.dim() == 3, "C must have shape (batch, length, state)")
    _check(C.shape == B.shape, "C shape mismatch")
    if gate is not None:
        _check(gate.device == inputs.device, "gate must be on the same device as inputs")
        _check(gate.dtype == dtype, f"gate must be {dn}")
        _check(gate.shape == inputs.shape, "gate shape mismatch")


def _num_chunks(length: int) -> int:
    return int(_lib.load().ossm_selective_num_chunks(length))


def selective_scan_cuda(inputs, dt, A, B, C, gate=None, chunk_length=16):
    """selective_scan_cuda.cu:253-310: returns ``[outputs, chunk_states, raw_outputs]``.

    ``chunk_length`` is accepted and ignored, as in the reference (:259)."""
    return _selective_forward(inputs, dt, A, B, C, gate, torch.float32, "selective_scan_cuda")


def selective_scan_cuda_bf16(inputs, dt, A, B, C, gate=None, chunk_length=16):
    """bfloat16 storage variant of :func:`selective_scan_cuda` (no counterpart in
    the reference, whose extension is float32 only): inputs, dt, B, C, gate and
    the outputs are bfloat16, A and chunk_states float32; the scan runs in
    float32 and each output is rounded once."""
    return _selective_forward(inputs, dt, A, B, C, gate, torch.bfloat16, "selective_scan_cuda_bf16")


def selective_scan_cuda_skip(inputs, dt, A, B, C, D, gate=None):
    """:func:`selective_scan_cuda` (float32 inputs) or :func:`selective_scan_cuda_bf16`
    (bfloat16) with a per-channel skip ``D`` (float32, shape (channels,)) fused
    into the scan: ``raw = y + D u``, ``out = raw * silu(gate)``.  An extension
    with no counterpart in the reference's kernels (BASELINE configs 3 and 4
    name a D skip); returns ``[outputs, chunk_states, raw_outputs]``."""
    return _selective_forward(inputs, dt, A, B, C, gate, inputs.dtype, "selective_scan_cuda_skip",
                              skip=D)


def _skip_checks(D, inputs, name):
    _check(D is not None, f"{name} needs the skip D")
    _check(D.device == inputs.device, "D must be on the same device as inputs")
    _check(D.dtype == torch.float32, "D must be float32")
    _check(D.dim() == 1 and D.size(0) == inputs.size(1), "D must have shape (channels,)")


def _selective_forward(inputs, dt, A, B, C, gate, dtype, name, skip=None):
    _check(inputs.is_cuda, "inputs must be CUDA tensor")
    if skip is not None:
        _check(dtype in (torch.float32, torch.bfloat16), f"{name} requires float32 or bfloat16 inputs")
        _skip_checks(skip, inputs, name)
    _selective_checks(inputs, dt, A, B, C, gate, name, dtype)
    batch, dim, length = inputs.shape
    dstate = A.size(1)
    if length == 0:
        return [torch.zeros_like(inputs),
                torch.zeros((batch, dim, 0, dstate * 2), dtype=torch.float32, device=inputs.device),
                torch.zeros_like(inputs)]
    u, d, a, b, c = (x.contiguous() for x in (inputs, dt, A, B, C))
    z = gate.contiguous() if gate is not None else None
    raw = torch.empty_like(u)
    out = torch.empty_like(u) if z is not None else raw
    chunks = torch.empty((batch, dim, _num_chunks(length), dstate * 2), dtype=torch.float32,
                         device=u.device)
    with torch.cuda.device(u.device):
        if skip is not None:
            _lib.check(_lib.load().ossm_selective_forward_skip(
                _ELEM[dtype], u.data_ptr(), d.data_ptr(), a.data_ptr(), b.data_ptr(), c.data_ptr(),
                skip.contiguous().data_ptr(), _lib.ptr(z), out.data_ptr(), raw.data_ptr(),
                chunks.data_ptr(), batch, dim, length, dstate, _lib.stream_of(u)))
            return [out, chunks, raw]
        fn = _lib.load().ossm_selective_forward if dtype == torch.float32 else \
            _lib.load().ossm_selective_forward_bf16
        _lib.check(fn(
            u.data_ptr(), d.data_ptr(), a.data_ptr(), b.data_ptr(), c.data_ptr(), _lib.ptr(z),
            out.data_ptr(), raw.data_ptr(), chunks.data_ptr(), batch, dim, length, dstate,
            _lib.stream_of(u)))
    return [out, chunks, raw]


def selective_scan_cuda_backward(grad_output, inputs, dt, A, B, C, gate=None, chunk_states=None,
                                 raw_outputs=None, chunk_length=None):
    """selective_scan_cuda.cu:312-393: returns ``[du, ddt, dA, dB, dC, dgate]``.

    ``chunk_states`` must come from :func:`selective_scan_cuda` on the same
    inputs (its rows are this library's state checkpoints).  ``raw_outputs``
    (y before the gate) is read for ``dgate`` when a gate is given; if it is
    missing the forward is re-run to produce it."""
    return _selective_backward(grad_output, inputs, dt, A, B, C, gate, chunk_states, raw_outputs,
                               torch.float32, "selective_scan_cuda")


def selective_scan_cuda_bf16_backward(grad_output, inputs, dt, A, B, C, gate=None,
                                      chunk_states=None, raw_outputs=None, chunk_length=None):
    """bfloat16 storage variant of :func:`selective_scan_cuda_backward`:
    ``[du, ddt, dA, dB, dC, dgate]`` with dA float32 and the rest bfloat16;
    ``chunk_states`` (float32) and ``raw_outputs`` come from
    :func:`selective_scan_cuda_bf16`."""
    return _selective_backward(grad_output, inputs, dt, A, B, C, gate, chunk_states, raw_outputs,
                               torch.bfloat16, "selective_scan_cuda_bf16")


def selective_scan_cuda_skip_backward(grad_output, inputs, dt, A, B, C, D, gate=None,
                                      chunk_states=None, raw_outputs=None):
    """Backward of :func:`selective_scan_cuda_skip`: ``[du, ddt, dA, dB, dC, dD, dgate]``
    (dA and dD float32, the rest in the inputs' dtype); ``du`` includes
    ``D * gy`` and ``dD`` is the sum over batch and time of ``gy * u``, with
    ``gy = grad_output * silu(gate)``.  ``chunk_states`` and ``raw_outputs``
    come from :func:`selective_scan_cuda_skip` on the same inputs."""
    return _selective_backward(grad_output, inputs, dt, A, B, C, gate, chunk_states, raw_outputs,
                               inputs.dtype, "selective_scan_cuda_skip", skip=D)


def _selective_backward(grad_output, inputs, dt, A, B, C, gate, chunk_states, raw_outputs, dtype,
                        name, skip=None):
    dn = "float32" if dtype == torch.float32 else "bfloat16"
    _check(inputs.is_cuda, "inputs must be CUDA tensor")
    if skip is not None:
        _check(dtype in (torch.float32, torch.bfloat16), f"{name} requires float32 or bfloat16 inputs")
        _skip_checks(skip, inputs, name)
    _selective_checks(inputs, dt, A, B, C, gate, name, dtype)
    _check(grad_output.device == inputs.device, "grad_output must be on the same device as inputs")
    _check(grad_output.dtype == dtype, f"grad_output must be {dn}")
    _check(grad_output.shape == inputs.shape, "grad_output shape mismatch")
    _check(chunk_states is not None, "chunk_states must have shape (batch, channels, num_chunks, state * 2)")
    _check(chunk_states.device == inputs.device, "chunk_states must be on the same device as inputs")
    _check(chunk_states.dtype == torch.float32, "chunk_states must be float32")
    _check(chunk_states.dim() == 4,
           "chunk_states must have shape (batch, channels, num_chunks, state * 2)")
    if raw_outputs is not None:
        _check(raw_outputs.device == inputs.device, "raw_outputs must be on the same device as inputs")
        _check(raw_outputs.dtype == dtype, f"raw_outputs must be {dn}")
        _check(raw_outputs.shape == inputs.shape, "raw_outputs shape mismatch")
    batch, dim, length = inputs.shape
    dstate = A.size(1)
    u, d, a, b, c = (x.contiguous() for x in (inputs, dt, A, B, C))
    z = gate.contiguous() if gate is not None else None
    gout = grad_output.contiguous()
    du, ddt = torch.empty_like(u), torch.empty_like(d)
    dA = torch.empty_like(a)  # float32 in both storage types
    dB, dC = torch.empty_like(b), torch.empty_like(c)
    dz = torch.empty_like(u)
    dD = torch.zeros_like(skip) if skip is not None else None
    if length == 0:
        return [du, ddt, dA.zero_(), dB, dC, dz] if skip is None else [du, ddt, dA.zero_(), dB, dC, dD, dz]
    cs = chunk_states.contiguous()
    _check(tuple(cs.shape) == (batch, dim, _num_chunks(length), 2 * dstate),
           "chunk_states do not match this library's forward for these inputs")
    raw = None
    if z is not None:
        raw = raw_outputs.contiguous() if raw_outputs is not None else \
            _selective_forward(inputs, dt, A, B, C, gate, dtype, name, skip=skip)[2]
    with torch.cuda.device(u.device):
        if skip is not None:
            _lib.check(_lib.load().ossm_selective_backward_skip(
                _ELEM[dtype], gout.data_ptr(), u.data_ptr(), d.data_ptr(), a.data_ptr(),
                b.data_ptr(), c.data_ptr(), skip.contiguous().data_ptr(), _lib.ptr(z),
                cs.data_ptr(), _lib.ptr(raw), du.data_ptr(), ddt.data_ptr(), dA.data_ptr(),
                dB.data_ptr(), dC.data_ptr(), dD.data_ptr(), dz.data_ptr(), batch, dim, length,
                dstate, _lib.stream_of(u)))
            return [du, ddt, dA, dB, dC, dD, dz]
        fn = _lib.load().ossm_selective_backward if dtype == torch.float32 else \
            _lib.load().ossm_selective_backward_bf16
        _lib.check(fn(
            gout.data_ptr(), u.data_ptr(), d.data_ptr(), a.data_ptr(), b.data_ptr(), c.data_ptr(),
            _lib.ptr(z), cs.data_ptr(), _lib.ptr(raw), du.data_ptr(), ddt.data_ptr(),
            dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), dz.data_ptr(), batch, dim, length,
            dstate, _lib.stream_of(u)))
    return [du, ddt, dA, dB, dC, dz]


def selective_scan(inputs, dt, A, B, C, gate=None):
    """selective_scan_cpu.cpp:78-166 entry; device tensors run the HIP kernel."""
    if not inputs.is_cuda:
        return _delegate("selective_scan", inputs, dt, A, B, C, gate)
    return selective_scan_cuda(inputs, dt, A, B, C, gate)[0]


def selective_scan_backward(grad_output, inputs, dt, A, B, C, gate=None):
    """selective_scan_cpu.cpp:168-360 entry; device tensors re-run the forward
    for its checkpoints, then the HIP backward."""
    if not inputs.is_cuda:
        return _delegate("selective_scan_backward", grad_output, inputs, dt, A, B, C, gate)
    _, chunks, raw = selective_scan_cuda(inputs, dt, A, B, C, gate)
    return selective_scan_cuda_backward(grad_output, inputs, dt, A, B, C, gate, chunks, raw, 16)


# ---------------------------------------------------- selective D-LinOSS
def _sdl_param(param: torch.Tensor, name: str, length: int, batch: int, ssm: int):
    """normalize_param_view_cpu (sdlinoss_cpu_utils.h:11-72): the (La, Ba, M)
    view of a parameter given as (M,), (L,M), (B,M) or (L|1, B|1, M);
    returns the contiguous float32 view and (La, Ba)."""
    shape = list(param.shape)
    _check(1 <= param.dim() <= 3,
           f"{name} must be shaped as (M,), (L,M), (B,M), or (L,B,M); got {shape}")
    _check(param.size(-1) == ssm,
           f"{name} must have size {ssm} along the last dimension; got {shape}")
    if param.dim() == 1:
        la, ba = 1, 1
    elif param.dim() == 2:
        if param.size(0) == length:
            la, ba = length, 1
        elif param.size(0) == batch:
            la, ba = 1, batch
        else:
            raise RuntimeError(f"{name} must be shaped as (M,), (L,M), (B,M), or (L,B,M); got {shape}")
    else:
        _check(param.size(0) in (length, 1) and param.size(1) in (batch, 1),
               f"{name} must have shape (L,B,M) with optional singleton L/B axes; got {shape}")
        la, ba = param.size(0), param.size(1)
    return param.contiguous(), la, ba


# complex dtype of bu -> (real parameter dtype, forward entry, backward entry)
_SDL_ENTRIES = {
    torch.complex64: (torch.float32, "ossm_sdlinoss_forward", "ossm_sdlinoss_backward"),
    torch.complex128: (torch.float64, "ossm_sdlinoss_forward_f64", "ossm_sdlinoss_backward_f64"),
}


def _sdl_entries(variant: str, direction: str, bu: torch.Tensor, params):
    """The reference's device kernels dispatch complex64 and complex128
    (AT_DISPATCH_COMPLEX_TYPES, sdlinoss_imex1_cuda.cu:232, 271); parameters
    must be the matching real dtype."""
    _check(bu.dtype in _SDL_ENTRIES,
           f"sdlinoss_{variant}_{direction}: bu must be complex64 or complex128, got {bu.dtype}")
    real, fwd, bwd = _SDL_ENTRIES[bu.dtype]
    for p, name in params:
        _check(p.dtype == real, f"{name} must be {real} to match bu ({bu.dtype}); got {p.dtype}")
    return fwd if direction == "forward" else bwd


def _sdl_forward(variant: str, A, G, step, bu):
    # sdlinoss_imex1.cpp:317-355 (and siblings)
    _check(bu.dim() == 3, "bu must have shape (length, batch, ssm_size)")
    _check(A.device == bu.device and G.device == bu.device and step.device == bu.device,
           "All tensors must live on the same device")
    if not bu.is_cuda:
        return _delegate(f"sdlinoss_{variant}_forward", A, G, step, bu)
    length, batch, ssm = bu.shape
    out = torch.empty((length, batch, ssm, 2), dtype=bu.dtype, device=bu.device)
    if length == 0:
        return out
    named = ((A, "A"), (G, "G"), (step, "step"))
    entry = _sdl_entries(variant, "forward", bu, named)
    views = [_sdl_param(p, n, length, batch, ssm) for p, n in named]
    b = bu.contiguous()
    args = []
    for v, la, ba in views:
        args += [v.data_ptr(), la, ba]
    with torch.cuda.device(bu.device):
        _lib.check(getattr(_lib.load(), entry)(
            _VARIANT_CODE[variant], *args, b.data_ptr(), out.data_ptr(), length, batch, ssm,
            _lib.stream_of(b)))
    return out


def _sdl_backward(variant: str, A, G, step, bu, states, grad_output):
    # sdlinoss_imex1.cpp:357-425 (and siblings); returns [grad_A, grad_G, grad_step, grad_bu]
    _check(states.dim() == 4 and states.size(3) == 2,
           "states must have shape (length, batch, ssm_size, 2)")
    _check(bu.dim() == 3, "bu must have shape (length, batch, ssm_size)")
    _check(grad_output.shape == bu.shape, "grad_output must match bu shape")
    if not bu.is_cuda:
        return _delegate(f"sdlinoss_{variant}_backward", A, G, step, bu, states, grad_output)
    _on_device(A, G, step, bu, states, grad_output)
    _check(states.is_contiguous() and grad_output.is_contiguous(),
           "states and grad_output must be contiguous on CUDA")
    length, batch, ssm = bu.shape
    grads = [torch.empty(p.shape, dtype=p.dtype, device=p.device) for p in (A, G, step)]
    grad_bu = torch.empty_like(bu)
    if length == 0 or batch == 0 or ssm == 0:
        return [g.zero_() for g in grads] + [grad_bu]
    named = ((A, "A"), (G, "G"), (step, "step"))
    entry = _sdl_entries(variant, "backward", bu, named)
    _check(states.dtype == bu.dtype and grad_output.dtype == bu.dtype,
           "states and grad_output must have bu's dtype")
    _check(tuple(states.shape) == (length, batch, ssm, 2),
           "states must have shape (length, batch, ssm_size, 2)")
    views = [_sdl_param(p, n, length, batch, ssm) for p, n in named]
    b = bu.contiguous()
    args = []
    for v, la, ba in views:
        args += [v.data_ptr(), la, ba]
    with torch.cuda.device(bu.device):
        _lib.check(getattr(_lib.load(), entry)(
            _VARIANT_CODE[variant], *args, b.data_ptr(), states.data_ptr(), grad_output.data_ptr(),
            grads[0].data_ptr(), grads[1].data_ptr(), grads[2].data_ptr(), grad_bu.data_ptr(),
            length, batch, ssm, _lib.stream_of(b)))
    return grads + [grad_bu]


def sdlinoss_imex1_forward(A, G, step, bu):
    return _sdl_forward("imex1", A, G, step, bu)


def sdlinoss_imex1_backward(A, G, step, bu, states, grad_output):
    return _sdl_backward("imex1", A, G, step, bu, states, grad_output)


def sdlinoss_imex2_forward(A, G, step, bu):
    return _sdl_forward("imex2", A, G, step, bu)


def sdlinoss_imex2_backward(A, G, step, bu, states, grad_output):
    return _sdl_backward("imex2", A, G, step, bu, states, grad_output)


def sdlinoss_im_forward(A, G, step, bu):
    return _sdl_forward("im", A, G, step, bu)


def sdlinoss_im_backward(A, G, step, bu, states, grad_output):
    return _sdl_backward("im", A, G, step, bu, states, grad_output)


def sdlinoss_ex_forward(A, G, step, bu):
    return _sdl_forward("ex", A, G, step, bu)


def sdlinoss_ex_backward(A, G, step, bu, states, grad_output):
    return _sdl_backward("ex", A, G, step, bu, states, grad_output)


# ------------------------------------------------------ export-only names
def _export_only(name: str):
    def fn(*args, **kwargs):
        tensors = [a for a in args if isinstance(a, torch.Tensor)]
        if tensors and not tensors[0].is_cuda:
            return _delegate(name, *args)
        raise RuntimeError(f"{name} has no HIP implementation in this build")

    fn.__name__ = name
    fn.__doc__ = f"Export-only name of the reference module ({name}); see module docstring."
    return fn


linear_rnn_scan = _export_only("linear_rnn_scan")


# ------------------------------------------------------ diagonal scans (LRU, S5)
def _diag_lambda(lambda_real, lambda_imag, state: int, dtype):
    _check(lambda_real.dim() == 1, "lambda_real must be 1-D")
    _check(lambda_imag.dim() == 1, "lambda_imag must be 1-D")
    _check(lambda_real.size(0) == state, "lambda_real must match state dimension")
    _check(lambda_imag.size(0) == state, "lambda_imag must match state dimension")
    _check(lambda_real.dtype == dtype and lambda_imag.dtype == dtype,
           "lambda_real, lambda_imag and b_seq must share one floating dtype")
    return lambda_real.contiguous(), lambda_imag.contiguous()


def _diag_entry(dtype, direction: str):
    _check(dtype in (torch.float32, torch.float64),
           f"diagonal scan HIP kernel supports float32 and float64, got {dtype}")
    suffix = "" if dtype == torch.float32 else "_f64"
    return getattr(_lib.load(), f"ossm_diag_scan_{direction}{suffix}")


def _diag_forward(name: str, lambda_real, lambda_imag, b_seq):
    """lru_scan.cpp:126-146 / s5_scan.cpp:126-146 (dispatch) with the checks of the
    CPU path (:68-92); the GPU result is the same recurrence on the device."""
    if b_seq.size(0) == 0:
        return torch.empty_like(b_seq)
    _check(b_seq.dim() == 4,
           f"b_seq must have shape (length, batch, state, 2), got {list(b_seq.shape)}")
    if not b_seq.is_cuda:
        return _delegate(name, lambda_real, lambda_imag, b_seq)
    _check(b_seq.size(-1) == 2, "b_seq must have shape (length, batch, state, 2)")
    _on_device(lambda_real, lambda_imag, b_seq)
    length, batch, state, _ = b_seq.shape
    lre, lim = _diag_lambda(lambda_real, lambda_imag, state, b_seq.dtype)
    fn = _diag_entry(b_seq.dtype, "forward")
    b_seq = b_seq.contiguous()
    result = torch.empty_like(b_seq)
    with torch.cuda.device(b_seq.device):
        _lib.check(fn(lre.data_ptr(), lim.data_ptr(), b_seq.data_ptr(), result.data_ptr(),
                      length, batch, state, _lib.stream_of(b_seq)))
    return result


def _diag_backward(lambda_real, lambda_imag, states, grad_output):
    """Native backward of the diagonal scan, in the layout of the forward:
    ``[grad_lambda [P,2], grad_b [L,B,P,2]]`` (real views of complex tensors).
    The reference runs it as a Python loop (lru.py:52-80, s5.py:137-165)."""
    _check(states.dim() == 4 and states.size(-1) == 2,
           "states must have shape (length, batch, state, 2)")
    _check(grad_output.shape == states.shape, "grad_output must match states shape")
    _check(states.is_cuda, "diagonal scan backward: HIP path needs device tensors")
    _on_device(lambda_real, lambda_imag, states, grad_output)
    length, batch, state, _ = states.shape
    _check(grad_output.dtype == states.dtype, "grad_output must match the dtype of states")
    lre, lim = _diag_lambda(lambda_real, lambda_imag, state, states.dtype)
    fn = _diag_entry(states.dtype, "backward")
    states = states.contiguous()
    grad_output = grad_output.contiguous()
    grad_lambda = torch.empty((state, 2), dtype=states.dtype, device=states.device)
    grad_b = torch.empty_like(grad_output)
    with torch.cuda.device(states.device):
        _lib.check(fn(lre.data_ptr(), lim.data_ptr(), states.data_ptr(), grad_output.data_ptr(),
                      grad_lambda.data_ptr(), grad_b.data_ptr(), length, batch, state,
                      _lib.stream_of(states)))
    return [grad_lambda, grad_b]


def lru_scan(lambda_real, lambda_imag, b_seq):
    """``x_t = lambda * x_{t-1} + b_t`` over ``b_seq [L,B,P,2]`` (lru_scan.cpp:126-146)."""
    return _diag_forward("lru_scan", lambda_real, lambda_imag, b_seq)


def s5_scan(lambda_real, lambda_imag, b_seq):
    """Same recurrence under the S5 name (s5_scan.cpp:126-146)."""
    return _diag_forward("s5_scan", lambda_real, lambda_imag, b_seq)


def lru_scan_backward(lambda_real, lambda_imag, states, grad_output):
    """Native backward of :func:`lru_scan` (no counterpart in the reference module)."""
    return _diag_backward(lambda_real, lambda_imag, states, grad_output)


def s5_scan_backward(lambda_real, lambda_imag, states, grad_output):
    """Native backward of :func:`s5_scan` (no counterpart in the reference module)."""
    return _diag_backward(lambda_real, lambda_imag, states, grad_output)


def _load_now() -> List[str]:
    """Load the library (ImportError when missing) and return its exported ABI names."""
    lib = _lib.load()
    return [name for name in _lib.EXPORTED if hasattr(lib, name)]


# Importing this module loads the library: a missing build fails loudly here.
_load_now()
