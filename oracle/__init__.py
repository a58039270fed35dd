"""CPU oracle for the OSSM scan kernels — TEST INFRASTRUCTURE ONLY.

Python face of ``oracle/scan_oracle.c`` (a C restatement of the reference's
CPU kernels) and of ``oracle/_ref`` (the reference's own CPU kernels compiled
from /root/reference by ``oracle/Makefile.ref``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package, and only as the checker or the timed CPU baseline.  The product path
(``ossm_amd``) never imports it.

All functions take and return numpy arrays in the reference's layouts:
D-LinOSS ``bu [L,B,P]`` complex, states ``[L,B,P,2]`` complex (the selective
D-LinOSS alike, with parameters (M,), (L,M), (B,M) or (L|1,B|1,M)); LinOSS
``b_seq [L,B,P,2]`` complex with complex ``m_ij [P]``; diagonal (LRU / S5)
scans ``b_seq [L,B,P]`` complex with complex ``lambda_bar [P]``; selective scan
``u, dt, gate [B,D,L]``, ``A [D,N]``, ``B, C [B,L,N]`` real; the D-LinOSS
layer ``inputs, outputs [B,L,H]`` real with ``B [P,H,2]``, ``C [H,P,2]``; the
Mamba mixer's steps in its ``[B,L,D]`` layout.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libscan_oracle.so"
_REF_DIR = _HERE / "_ref"

VARIANTS = ("imex1", "imex2", "im", "ex")
_VARIANT_CODE = {name: i for i, name in enumerate(VARIANTS)}

_lib: Optional[ctypes.CDLL] = None


def build() -> None:
    """Compile the C restatement (``make -C oracle``)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
    return _lib


def num_threads() -> int:
    return int(_load().oracle_num_threads())


def _ptr(arr: Optional[np.ndarray]):
    if arr is None:
        return None
    assert arr.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return arr.ctypes.data_as(ctypes.c_void_p)


def _real_dtype(precision: str):
    return np.float32 if precision == "f32" else np.float64


def _complex_dtype(precision: str):
    return np.complex64 if precision == "f32" else np.complex128


def _prec_of(arr: np.ndarray) -> str:
    return "f64" if arr.dtype in (np.float64, np.complex128) else "f32"


def _fn(name: str, precision: str):
    return getattr(_load(), f"{name}_{precision}")


def _c(arr, dtype) -> np.ndarray:
    return np.ascontiguousarray(arr, dtype=dtype)


# ---------------------------------------------------------------- D-LinOSS
def dlinoss_forward(variant: str, a_diag, g_diag, step, bu) -> np.ndarray:
    """States ``[L,B,P,2]`` of the D-LinOSS recurrence (dlinoss_<v>.cpp forward)."""
    prec = _prec_of(np.asarray(bu))
    rt, ct = _real_dtype(prec), _complex_dtype(prec)
    bu = _c(bu, ct)
    L, B, P = bu.shape
    a, g, s = _c(a_diag, rt), _c(g_diag, rt), _c(step, rt)
    out = np.empty((L, B, P, 2), dtype=ct)
    I = ctypes.c_int64
    _fn("oracle_dlinoss_forward", prec)(
        ctypes.c_int(_VARIANT_CODE[variant]), _ptr(a), _ptr(g), _ptr(s), _ptr(bu), _ptr(out),
        I(L), I(B), I(P))
    return out


def dlinoss_backward(variant: str, a_diag, g_diag, step, bu, states, grad_output,
                     grad_aux=None):
    """``(grad_a, grad_g, grad_step, grad_bu)`` (dlinoss_<v>.cpp backward).

    ``grad_aux`` is an oracle-only extra gradient w.r.t. state component 0;
    ``None`` gives the reference's arithmetic exactly.
    """
    prec = _prec_of(np.asarray(bu))
    rt, ct = _real_dtype(prec), _complex_dtype(prec)
    bu = _c(bu, ct)
    L, B, P = bu.shape
    a, g, s = _c(a_diag, rt), _c(g_diag, rt), _c(step, rt)
    states = _c(states, ct)
    gout = _c(grad_output, ct)
    gaux = None if grad_aux is None else _c(grad_aux, ct)
    grad_bu = np.empty_like(bu)
    ga, gg, gs = np.zeros(P, rt), np.zeros(P, rt), np.zeros(P, rt)
    I = ctypes.c_int64
    _fn("oracle_dlinoss_backward", prec)(
        ctypes.c_int(_VARIANT_CODE[variant]), _ptr(a), _ptr(g), _ptr(s), _ptr(bu), _ptr(states),
        _ptr(gout), _ptr(gaux), _ptr(grad_bu), _ptr(ga), _ptr(gg), _ptr(gs), I(L), I(B), I(P))
    return ga, gg, gs, grad_bu


# ------------------------------------------------------------ D-LinOSS layer
def dlinoss_layer_forward(variant: str, inputs, B, C, D, a_diag, g_diag, step):
    """``(y, states)`` of DampedLinOSSLayer.forward after the parameter
    projection (dlinoss.py:210-247), in the inputs' precision: ``bu = u B^T``
    with ``B[..., 0] + i B[..., 1]`` (two real GEMMs, dlinoss.py:219-224), the
    scan above on ``bu`` permuted to ``[L,B,P]``, then
    ``y = Re(x) C[..., 0]^T - Im(x) C[..., 1]^T + D u`` (dlinoss.py:237-245) with
    ``x = states[..., 1]``.  ``u, y [B,L,H]``; ``B [P,H,2]``; ``C [H,P,2]``;
    ``D [H]``; states ``[L,B,P,2]``."""
    u = np.asarray(inputs)
    prec = _prec_of(u)
    rt, ct = _real_dtype(prec), _complex_dtype(prec)
    u = _c(u, rt)
    Bw, Cw, Dw = _c(B, rt), _c(C, rt), _c(D, rt)
    nb, L, H = u.shape
    P = Bw.shape[0]
    flat = u.reshape(nb * L, H)
    bu = (flat @ Bw[..., 0].T).astype(rt) + 1j * (flat @ Bw[..., 1].T).astype(rt)
    bu = np.ascontiguousarray(bu.astype(ct).reshape(nb, L, P).transpose(1, 0, 2))
    states = dlinoss_forward(variant, a_diag, g_diag, step, bu)
    x = states[..., 1].transpose(1, 0, 2).reshape(nb * L, P)
    proj = (x.real.astype(rt) @ Cw[..., 0].T).astype(rt) - (x.imag.astype(rt) @ Cw[..., 1].T).astype(rt)
    y = proj.reshape(nb, L, H) + u * Dw
    return y.astype(rt), states


# ------------------------------------------------------------------ LinOSS
def linoss_forward(m11, m12, m21, m22, b_seq) -> np.ndarray:
    """States ``[L,B,P,2]`` of ``s_t = M s_{t-1} + b_t`` (linoss_scan.cpp)."""
    prec = _prec_of(np.asarray(b_seq))
    ct = _complex_dtype(prec)
    b_seq = _c(b_seq, ct)
    L, B, P, _ = b_seq.shape
    ms = [_c(m, ct) for m in (m11, m12, m21, m22)]
    out = np.empty_like(b_seq)
    I = ctypes.c_int64
    _fn("oracle_linoss_forward", prec)(*[_ptr(m) for m in ms], _ptr(b_seq), _ptr(out),
                                       I(L), I(B), I(P))
    return out


def linoss_backward(m11, m12, m21, m22, states, grad_output):
    """``(grad_m [P,2,2], grad_b [L,B,P,2])`` restating linoss.py:83-151."""
    prec = _prec_of(np.asarray(states))
    ct = _complex_dtype(prec)
    states = _c(states, ct)
    gout = _c(grad_output, ct)
    L, B, P, _ = states.shape
    ms = [_c(m, ct) for m in (m11, m12, m21, m22)]
    grad_m = np.zeros((P, 2, 2), dtype=ct)
    grad_b = np.empty_like(states)
    I = ctypes.c_int64
    _fn("oracle_linoss_backward", prec)(*[_ptr(m) for m in ms], _ptr(states), _ptr(gout),
                                        _ptr(grad_m), _ptr(grad_b), I(L), I(B), I(P))
    return grad_m, grad_b


# ------------------------------------------------------ diagonal (LRU, S5)
def diag_forward(lambda_bar, b_seq) -> np.ndarray:
    """Complex states ``[L,B,P]`` of ``x_t = lambda * x_{t-1} + b_t``
    (lru_scan.cpp:10-58 / s5_scan.cpp:10-66); ``lambda_bar [P]`` complex."""
    prec = _prec_of(np.asarray(b_seq))
    rt, ct = _real_dtype(prec), _complex_dtype(prec)
    b_seq = _c(b_seq, ct)
    L, B, P = b_seq.shape
    lam = np.asarray(lambda_bar)
    lre, lim = _c(lam.real, rt), _c(lam.imag, rt)
    out = np.empty_like(b_seq)
    I = ctypes.c_int64
    _fn("oracle_diag_forward", prec)(_ptr(lre), _ptr(lim), _ptr(b_seq), _ptr(out), I(L), I(B), I(P))
    return out


def diag_backward(lambda_bar, states, grad_output):
    """``(grad_lambda [P], grad_b [L,B,P])`` restating lru.py:52-80 (s5.py:137-165)."""
    prec = _prec_of(np.asarray(states))
    rt, ct = _real_dtype(prec), _complex_dtype(prec)
    states = _c(states, ct)
    gout = _c(grad_output, ct)
    L, B, P = states.shape
    lam = np.asarray(lambda_bar)
    lre, lim = _c(lam.real, rt), _c(lam.imag, rt)
    grad_lambda = np.zeros(P, dtype=ct)
    grad_b = np.empty_like(states)
    I = ctypes.c_int64
    _fn("oracle_diag_backward", prec)(_ptr(lre), _ptr(lim), _ptr(states), _ptr(gout),
                                      _ptr(grad_lambda), _ptr(grad_b), I(L), I(B), I(P))
    return grad_lambda, grad_b


# --------------------------------------------------------------- selective
def selective_forward(u, dt, A, Bm, Cm, gate=None) -> np.ndarray:
    """Selective scan output ``[B,D,L]`` (selective_scan_cpu.cpp:78-166)."""
    prec = _prec_of(np.asarray(u))
    rt = _real_dtype(prec)
    u, dt, A, Bm, Cm = (_c(x, rt) for x in (u, dt, A, Bm, Cm))
    gate = None if gate is None else _c(gate, rt)
    Bsz, D, L = u.shape
    N = A.shape[1]
    out = np.empty_like(u)
    I = ctypes.c_int64
    _fn("oracle_selective_forward", prec)(_ptr(u), _ptr(dt), _ptr(A), _ptr(Bm), _ptr(Cm),
                                          _ptr(gate), _ptr(out), I(Bsz), I(D), I(L), I(N))
    return out


# ------------------------------------------------ Mamba mixer pre/post steps
def softplus(x) -> np.ndarray:
    """F.softplus with torch's defaults (beta 1, threshold 20: x itself above),
    as mambarec.py:155 applies it to dt."""
    x = np.asarray(x)
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20)))).astype(x.dtype)


def mamba_conv_silu(x, weight, bias=None) -> np.ndarray:
    """``silu(Conv1d(pad_left(x^T, K-1)))^T`` of mambarec.py:143-150 for x
    ``[B,L,D]``, depthwise weight ``[D,1,K]`` or ``[D,K]``, bias ``[D]``:
    ``pre[b,t,d] = bias[d] + sum_k w[d,k] x[b,t-K+1+k,d]`` (zero before t = 0)."""
    x = np.asarray(x)
    rt = x.dtype
    nb, L, D = x.shape
    w = np.asarray(weight, rt).reshape(D, -1)
    K = w.shape[1]
    pad = np.concatenate([np.zeros((nb, K - 1, D), rt), x], axis=1)
    pre = np.zeros((nb, L, D), rt) + (np.asarray(bias, rt) if bias is not None else 0)
    for k in range(K):
        pre = pre + w[:, k] * pad[:, k:k + L, :]
    return (pre / (1 + np.exp(-pre))).astype(rt)


def selective_forward_bld(u, dt_pre, A, Bm, Cm, gate=None, dt_bias=None) -> np.ndarray:
    """The selective scan in the mixer's ``[B,L,D]`` layout with dt given before
    its softplus (mambarec.py:155-170): transposes to ``[B,D,L]``, the scan
    above, and back."""
    u = np.asarray(u)
    dt = np.asarray(dt_pre) + (0 if dt_bias is None else np.asarray(dt_bias))
    t = lambda a: np.ascontiguousarray(np.asarray(a).transpose(0, 2, 1))
    y = selective_forward(t(u), t(softplus(dt.astype(u.dtype))), A, Bm, Cm,
                          None if gate is None else t(gate))
    return np.ascontiguousarray(y.transpose(0, 2, 1))


def selective_backward(grad_output, u, dt, A, Bm, Cm, gate=None):
    """``(du, ddt, dA, dB, dC, dgate)`` (selective_scan_cpu.cpp:168-360)."""
    prec = _prec_of(np.asarray(u))
    rt = _real_dtype(prec)
    gout, u, dt, A, Bm, Cm = (_c(x, rt) for x in (grad_output, u, dt, A, Bm, Cm))
    gate = None if gate is None else _c(gate, rt)
    Bsz, D, L = u.shape
    N = A.shape[1]
    gu, gdt, ggate = np.empty_like(u), np.empty_like(u), np.empty_like(u)
    gA = np.zeros_like(A)
    gB, gC = np.zeros_like(Bm), np.zeros_like(Cm)
    I = ctypes.c_int64
    _fn("oracle_selective_backward", prec)(
        _ptr(gout), _ptr(u), _ptr(dt), _ptr(A), _ptr(Bm), _ptr(Cm), _ptr(gate), _ptr(gu),
        _ptr(gdt), _ptr(gA), _ptr(gB), _ptr(gC), _ptr(ggate), I(Bsz), I(D), I(L), I(N))
    return gu, gdt, gA, gB, gC, ggate


# ------------------------------------------------------ selective D-LinOSS
def _sdl_view(param, length: int, batch: int, ssm: int) -> np.ndarray:
    """normalize_param_view_cpu (sdlinoss_cpu_utils.h:11-72) as a [La, Ba, M] view."""
    p = np.asarray(param)
    if p.ndim == 1 and p.shape[0] == ssm:
        return p.reshape(1, 1, ssm)
    if p.ndim == 2 and p.shape[1] == ssm:
        if p.shape[0] == length:
            return p.reshape(length, 1, ssm)
        if p.shape[0] == batch:
            return p.reshape(1, batch, ssm)
    if p.ndim == 3 and p.shape[2] == ssm and p.shape[0] in (1, length) and p.shape[1] in (1, batch):
        return p
    raise ValueError(f"parameter must be shaped as (M,), (L,M), (B,M), or (L,B,M); got {p.shape}")


def _sdl_full(param, length, batch, ssm, rt) -> np.ndarray:
    """materialize_param_cpu (sdlinoss_cpu_utils.h:74-82)."""
    return _c(np.broadcast_to(_sdl_view(param, length, batch, ssm), (length, batch, ssm)), rt)


def sdlinoss_forward(variant: str, A, G, step, bu) -> np.ndarray:
    """States ``[L,B,M,2]`` of the selective D-LinOSS recurrence (sdlinoss_<v>.cpp forward);
    A, G, step may be (M,), (L,M), (B,M) or (L|1, B|1, M)."""
    prec = _prec_of(np.asarray(bu))
    rt, ct = _real_dtype(prec), _complex_dtype(prec)
    bu = _c(bu, ct)
    L, B, M = bu.shape
    full = [_sdl_full(x, L, B, M, rt) for x in (A, G, step)]
    out = np.empty((L, B, M, 2), dtype=ct)
    I = ctypes.c_int64
    _fn("oracle_sdlinoss_forward", prec)(
        ctypes.c_int(_VARIANT_CODE[variant]), *[_ptr(x) for x in full], _ptr(bu), _ptr(out),
        I(L), I(B), I(M))
    return out


def sdlinoss_backward(variant: str, A, G, step, bu, states, grad_output):
    """``(grad_A, grad_G, grad_step, grad_bu)`` (sdlinoss_<v>.cpp backward); parameter
    gradients summed over broadcast axes and shaped like the parameters
    (reduce_broadcast_grad, sdlinoss_cpu_utils.h:84-97)."""
    prec = _prec_of(np.asarray(bu))
    rt, ct = _real_dtype(prec), _complex_dtype(prec)
    bu = _c(bu, ct)
    L, B, M = bu.shape
    params = (A, G, step)
    full = [_sdl_full(x, L, B, M, rt) for x in params]
    states = _c(states, ct)
    gout = _c(grad_output, ct)
    grad_bu = np.empty_like(bu)
    g_full = [np.zeros((L, B, M), rt) for _ in range(3)]
    I = ctypes.c_int64
    _fn("oracle_sdlinoss_backward", prec)(
        ctypes.c_int(_VARIANT_CODE[variant]), *[_ptr(x) for x in full], _ptr(bu), _ptr(states),
        _ptr(gout), _ptr(grad_bu), *[_ptr(x) for x in g_full], I(L), I(B), I(M))
    out = []
    for p, gf in zip(params, g_full):
        view = _sdl_view(p, L, B, M)
        g = gf
        if view.shape[0] == 1 and L > 1:
            g = g.sum(0, keepdims=True)
        if view.shape[1] == 1 and B > 1:
            g = g.sum(1, keepdims=True)
        out.append(np.ascontiguousarray(g.reshape(np.asarray(p).shape), dtype=rt))
    return out[0], out[1], out[2], grad_bu


# ------------------------------------------------- reference CPU kernels
def reference_module():
    """The reference's own CPU kernels (``oracle/_ref/_ref_kernels.so``), or None.

    Built in the survey container by ``make -f oracle/Makefile.ref`` from the
    sources under /root/reference; torch must be imported first.
    """
    path = _REF_DIR / "_ref_kernels.so"
    if not path.exists():
        return None
    import importlib.util

    import torch  # noqa: F401  (loads libtorch for the extension)

    spec = importlib.util.spec_from_file_location("_ref_kernels", str(path))
    if spec is None or spec.loader is None:
        return None
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def have_reference() -> bool:
    return (_REF_DIR / "_ref_kernels.so").exists()


os.environ.setdefault("OMP_PROC_BIND", "false")
