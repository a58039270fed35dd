"""The Mamba mixer with its pre/post-processing fused around the selective scan.

The reference mixer (``_MambaMixer``, mambarec.py:63-184) runs, between its
projections, a transpose + pad + depthwise Conv1d + SiLU, a softplus pass over
dt, transposes of x_conv, dt and z to ``[B, D, L]`` for the scan (plus
``.contiguous()`` copies) and a transpose of the output.  Here:

* ``ossm_mamba_conv_forward/backward``: the causal depthwise conv + SiLU in the
  mixer's ``[B, L, D]`` layout, reading x straight out of ``in_proj``'s output;
* ``ossm_selective_mamba_forward/backward``: the selective scan reading u, dt
  (before its softplus, with the dt_proj bias) and the gate z in ``[B, L, D]``
  with row strides (z and B, C stay views into the projection outputs) and
  writing ``[B, L, D]`` for ``out_proj``.

``MambaMixer`` has the reference module's constructor arguments and parameter
names (``in_proj``, ``conv1d``, ``x_proj``, ``dt_proj``, ``out_proj``,
``A_log``), so a reference ``state_dict`` loads unchanged.  Device float32
only; there is no CPU path (CPU inputs raise).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _lib

__all__ = ["MambaMixer", "mamba_conv_silu", "selective_scan_mamba", "ConvSiluFn", "MambaScanFn"]


def _rows(t: Tensor, name: str) -> Tuple[Tensor, int]:
    """A ``[B, L, C]`` float32 device tensor as (tensor, row stride): views whose
    last dimension is contiguous and whose batch stride is L row strides pass
    as they are; anything else is made contiguous."""
    if t.dim() != 3:
        raise RuntimeError(f"{name} must be (batch, length, channels), got {tuple(t.shape)}")
    if t.dtype != torch.float32 or not t.is_cuda:
        raise RuntimeError(f"{name} must be a float32 GPU tensor (got {t.dtype} on {t.device})")
    Bz, L, C = t.shape
    ok = t.stride(2) == 1 and t.stride(1) >= C and (Bz <= 1 or t.stride(0) == L * t.stride(1))
    if not ok:
        t = t.contiguous()
    return t, int(t.stride(1)) if L > 0 else C


def _param(t: Optional[Tensor], name: str) -> Optional[Tensor]:
    """A parameter the kernels read as contiguous float32 on the device."""
    if t is None:
        return None
    if t.dtype != torch.float32 or not t.is_cuda:
        raise RuntimeError(f"{name} must be a float32 GPU tensor (got {t.dtype} on {t.device})")
    return t.contiguous()


def _same_device(*ts: Optional[Tensor]) -> None:
    devs = {t.device for t in ts if t is not None}
    if len(devs) > 1:
        raise RuntimeError(f"tensors on different devices: {sorted(map(str, devs))}")


# ------------------------------------------------------------------ conv + SiLU
def _conv_fwd(x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    x, ld = _rows(x, "x")
    Bz, L, D = x.shape
    w = _param(weight, "conv weight").reshape(D, -1)
    b = _param(bias, "conv bias")
    if b is not None and tuple(b.shape) != (D,):
        raise RuntimeError(f"conv bias must have shape ({D},), got {tuple(b.shape)}")
    _same_device(x, w, b)
    out = torch.empty((Bz, L, D), dtype=torch.float32, device=x.device)
    if out.numel() == 0:
        return out
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().ossm_mamba_conv_forward(
            x.data_ptr(), ld, w.data_ptr(), _lib.ptr(b), out.data_ptr(), Bz, L, D, w.size(1),
            _lib.stream_of(x)))
    return out


class ConvSiluFn(torch.autograd.Function):
    """silu(causal depthwise conv1d(x) + bias) in ``[B, L, D]``."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:  # type: ignore[override]
        ctx.save_for_backward(x, weight, bias)
        ctx.has_bias = bias is not None
        return _conv_fwd(x, weight, bias)

    @staticmethod
    def backward(ctx, grad_out: Tensor):  # type: ignore[override]
        x, weight, bias = ctx.saved_tensors
        x, ld = _rows(x, "x")
        Bz, L, D = x.shape
        w = _param(weight, "conv weight").reshape(D, -1)
        K = w.size(1)
        go = grad_out.contiguous()
        gx = torch.empty((Bz, L, D), dtype=torch.float32, device=x.device)
        gw = torch.empty((D, K), dtype=torch.float32, device=x.device)
        gb = torch.empty((D,), dtype=torch.float32, device=x.device) if ctx.has_bias else None
        with torch.cuda.device(x.device):
            _lib.check(_lib.load().ossm_mamba_conv_backward(
                x.data_ptr(), ld, w.data_ptr(), _lib.ptr(bias), go.data_ptr(), gx.data_ptr(),
                gw.data_ptr(), _lib.ptr(gb), Bz, L, D, K, _lib.stream_of(x)))
        return gx, gw.reshape(weight.shape), gb


def mamba_conv_silu(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    """``silu(Conv1d(pad_left(x^T, K-1)))^T`` of mambarec.py:143-150 for x
    ``[B, L, D]`` (a strided view is read in place); weight ``[D, 1, K]`` or
    ``[D, K]``; returns ``[B, L, D]``."""
    return ConvSiluFn.apply(x, weight, bias)


# ------------------------------------------------------------- selective scan
class MambaScanFn(torch.autograd.Function):
    """Selective scan in ``[B, L, D]`` with dt before its softplus."""

    @staticmethod
    def forward(ctx, u: Tensor, dt: Tensor, A: Tensor, Bm: Tensor, Cm: Tensor,
                z: Optional[Tensor], dt_bias: Optional[Tensor]) -> Tensor:  # type: ignore[override]
        lib = _lib.load()
        u, ld_u = _rows(u, "inputs")
        dt, ld_dt = _rows(dt, "dt")
        Bm, ld_b = _rows(Bm, "B")
        Cm, ld_c = _rows(Cm, "C")
        if ld_b != ld_c or (Cm.data_ptr() - Bm.data_ptr()) % 4 != 0:
            Bm, Cm = Bm.contiguous(), Cm.contiguous()
            ld_b = ld_c = Bm.size(2)
        ld_z = 0
        if z is not None:
            z, ld_z = _rows(z, "gate")
        Bz, L, D = u.shape
        N = A.size(1)
        if tuple(dt.shape) != (Bz, L, D) or tuple(A.shape) != (D, N) or \
                tuple(Bm.shape) != (Bz, L, N) or tuple(Cm.shape) != (Bz, L, N) or \
                (z is not None and tuple(z.shape) != (Bz, L, D)) or \
                (dt_bias is not None and tuple(dt_bias.shape) != (D,)):
            raise RuntimeError("selective_scan_mamba: inconsistent shapes "
                               f"u {tuple(u.shape)} dt {tuple(dt.shape)} A {tuple(A.shape)} "
                               f"B {tuple(Bm.shape)} C {tuple(Cm.shape)}")
        Ac = _param(A, "A")
        bias = _param(dt_bias, "dt_bias")
        _same_device(u, dt, Ac, Bm, Cm, z, bias)
        out = torch.empty((Bz, L, D), dtype=torch.float32, device=u.device)
        raw = torch.empty_like(out) if z is not None else None
        n_chunks = int(lib.ossm_selective_num_chunks(L))
        ck = torch.empty((Bz, D, n_chunks, 2 * N), dtype=torch.float32, device=u.device)
        if out.numel() > 0:
            with torch.cuda.device(u.device):
                _lib.check(lib.ossm_selective_mamba_forward(
                    u.data_ptr(), ld_u, dt.data_ptr(), ld_dt, _lib.ptr(bias), Ac.data_ptr(),
                    Bm.data_ptr(), Cm.data_ptr(), ld_b, _lib.ptr(z), ld_z, out.data_ptr(),
                    _lib.ptr(raw), ck.data_ptr(), Bz, D, L, N, _lib.stream_of(u)))
        ctx.has_z = z is not None
        ctx.has_bias = bias is not None
        ctx.lds = (ld_u, ld_dt, ld_b, ld_z)
        ctx.save_for_backward(u, dt, Ac, Bm, Cm, z, bias, ck, raw)
        return out

    @staticmethod
    def backward(ctx, grad_out: Tensor):  # type: ignore[override]
        u, dt, A, Bm, Cm, z, bias, ck, raw = ctx.saved_tensors
        ld_u, ld_dt, ld_b, ld_z = ctx.lds
        Bz, L, D = u.shape
        N = A.size(1)
        go = grad_out.contiguous()
        dev = u.device
        du = torch.empty((Bz, L, D), dtype=torch.float32, device=dev)
        ddt = torch.empty_like(du)
        dz = torch.empty_like(du) if ctx.has_z else None
        dA = torch.empty((D, N), dtype=torch.float32, device=dev)
        dB = torch.empty((Bz, L, N), dtype=torch.float32, device=dev)
        dC = torch.empty_like(dB)
        with torch.cuda.device(dev):
            _lib.check(_lib.load().ossm_selective_mamba_backward(
                go.data_ptr(), u.data_ptr(), ld_u, dt.data_ptr(), ld_dt, _lib.ptr(bias),
                A.data_ptr(), Bm.data_ptr(), Cm.data_ptr(), ld_b, _lib.ptr(z), ld_z, ck.data_ptr(),
                _lib.ptr(raw), du.data_ptr(), ddt.data_ptr(), dA.data_ptr(), dB.data_ptr(),
                dC.data_ptr(), _lib.ptr(dz), Bz, D, L, N, _lib.stream_of(u)))
        dbias = ddt.sum(dim=(0, 1)) if ctx.has_bias else None
        return du, ddt, dA, dB, dC, dz, dbias


def selective_scan_mamba(inputs: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor,
                         gate: Optional[Tensor] = None, dt_bias: Optional[Tensor] = None) -> Tensor:
    """``y = scan(u, softplus(dt + dt_bias), A, B, C) * silu(gate)`` with every
    ``[B, L, *]`` tensor in the mixer's layout (the reference scan,
    mambarec.py:23-61 and selective_scan_cuda.cu:253-310, on transposes)."""
    return MambaScanFn.apply(inputs, dt, A, B, C, gate, dt_bias)


class _ColumnSplit(torch.autograd.Function):
    """``xz[..., :d], xz[..., d:]`` as views, whose backward writes the gradient
    of ``xz`` in one pass (torch.cat of the two); slicing the tensor directly
    would, in the backward, zero-fill the whole ``[B, L, 2d]`` gradient once per
    slice, copy each slice's gradient in and add the two."""

    @staticmethod
    def forward(ctx, xz: Tensor, d: int):  # type: ignore[override]
        ctx.d = d
        ctx.shape = xz.shape
        return xz[..., :d], xz[..., d:]

    @staticmethod
    def backward(ctx, gx: Optional[Tensor], gz: Optional[Tensor]):  # type: ignore[override]
        d, shape = ctx.d, ctx.shape
        if gx is None and gz is None:
            return None, None
        ref = gx if gx is not None else gz
        if gx is None:
            gx = torch.zeros(*shape[:-1], d, dtype=ref.dtype, device=ref.device)
        if gz is None:
            gz = torch.zeros(*shape[:-1], shape[-1] - d, dtype=ref.dtype, device=ref.device)
        return torch.cat([gx, gz], dim=-1), None


# ------------------------------------------------------------------ the mixer
class MambaMixer(nn.Module):
    """Mamba mixer (reference ``_MambaMixer``, mambarec.py:63-184) whose conv,
    softplus, gate and layout changes run inside this library's kernels."""

    def __init__(self, d_model: int, *, d_state: int, d_conv: int, expand: int,
                 dt_rank: int | str = "auto", dt_min: float = 0.001, dt_max: float = 0.1,
                 dt_init: str = "random", dt_scale: float = 1.0, dt_init_floor: float = 1e-4,
                 conv_bias: bool = True, bias: bool = False) -> None:
        super().__init__()
        if dt_rank == "auto":
            dt_rank = max(1, math.ceil(d_model / 16))
        self.d_model = int(d_model)
        self.d_state = int(d_state)
        self.d_conv = int(d_conv)
        self.expand = int(expand)
        self.d_inner = self.expand * self.d_model
        self.dt_rank = int(dt_rank)
        self.in_proj = nn.Linear(self.d_model, 2 * self.d_inner, bias=bias)
        self.conv1d = nn.Conv1d(self.d_inner, self.d_inner, kernel_size=self.d_conv,
                                groups=self.d_inner, bias=conv_bias, padding=0)
        self.x_proj = nn.Linear(self.d_inner, self.dt_rank + 2 * self.d_state, bias=False)
        self.dt_proj = nn.Linear(self.dt_rank, self.d_inner, bias=True)
        self.out_proj = nn.Linear(self.d_inner, self.d_model, bias=bias)
        # dt_proj: weights uniform or constant at dt_rank^-1/2 * dt_scale; bias =
        # softplus^-1 of dt log-uniform on [dt_min, dt_max] (mambarec.py:111-126)
        std = self.dt_rank ** -0.5 * dt_scale
        if dt_init == "constant":
            nn.init.constant_(self.dt_proj.weight, std)
        elif dt_init == "random":
            nn.init.uniform_(self.dt_proj.weight, -std, std)
        else:
            raise ValueError("dt_init must be 'random' or 'constant'")
        log_lo, log_hi = math.log(dt_min), math.log(dt_max)
        dt = torch.exp(torch.rand(self.d_inner) * (log_hi - log_lo) + log_lo).clamp(min=dt_init_floor)
        with torch.no_grad():
            self.dt_proj.bias.copy_(dt + torch.log(-torch.expm1(-dt)))
        self.dt_proj.bias._no_reinit = True  # type: ignore[attr-defined]
        # A = -(1 .. d_state) per channel, stored as its log (mambarec.py:128-131)
        A = torch.arange(1, self.d_state + 1, dtype=torch.float32).repeat(self.d_inner, 1)
        self.A_log = nn.Parameter(torch.log(A))
        self.A_log._no_weight_decay = True  # type: ignore[attr-defined]
        self.register_parameter("D", None)

    def forward(self, inputs: Tensor) -> Tensor:
        if inputs.ndim != 3:
            raise ValueError("Inputs to Mamba mixer must have shape (batch, length, channels)")
        if inputs.size(1) == 0:
            return torch.zeros_like(inputs)
        if not inputs.is_cuda:
            raise RuntimeError("the fused Mamba mixer runs on the GPU only")
        Di, R, N = self.d_inner, self.dt_rank, self.d_state
        xz = self.in_proj(inputs).float()
        x, z = _ColumnSplit.apply(xz, Di)                 # views, row stride 2 * d_inner
        x_conv = mamba_conv_silu(x, self.conv1d.weight.float(),
                                 None if self.conv1d.bias is None else self.conv1d.bias.float())
        proj = self.x_proj(x_conv.to(self.x_proj.weight.dtype)).float()
        dt_raw, B_gen, C_gen = proj[..., :R], proj[..., R:R + N], proj[..., R + N:]
        dt_pre = F.linear(dt_raw, self.dt_proj.weight.float())   # bias goes into the softplus
        A = -torch.exp(self.A_log.float())
        y = selective_scan_mamba(x_conv, dt_pre, A, B_gen, C_gen, gate=z,
                                 dt_bias=self.dt_proj.bias.float())
        return self.out_proj(y.to(self.out_proj.weight.dtype))
