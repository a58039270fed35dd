"""D-LinOSS layer whose forward is one fused MI355X kernel.

``DampedLinOSSLayer`` has the reference module's interface (dlinoss.py:48-278):
the same constructor arguments, parameter names and shapes (``A_diag``,
``G_diag``, ``steps`` [P]; ``B`` [P, H, 2]; ``C`` [H, P, 2]; ``D`` [H]), the
same stable-region projection and the same forward contract, so a reference
``state_dict`` loads unchanged.

Forward on a GPU float32 (or bf16 / fp16, computed in float32 as the
reference does) input is ``ossm_dlinoss_layer_forward``: the in-projection
``bu = u B^T``, the D-LinOSS scan and ``y = Re(x C^T) + D u`` in one launch,
with bu and the states kept on chip; for training it also saves the state
entering each 32-step chunk.  The backward is ``ossm_dlinoss_layer_backward``
(the projections of the upstream gradient and of u on the matrix cores, the
states re-run from those carries, the scan adjoint, grad_u), followed by the
two weight-gradient GEMMs over the grad_bu and x it returns.  Shapes whose
backward does not fit one workgroup's LDS recompute through the unfused
composition (``unfused_layer_forward``) and differentiate that.

No CPU path computes here: CPU tensors go through the same composition, whose
scan delegates to the reference's CPU module when it is installed (as the
rest of the drop-in does) and raises otherwise.  float64 raises: the device
kernels compute in float32 / complex64.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
from torch import Tensor, nn

from . import _lib
from .bridge import run_dlinoss

__all__ = ["DampedLinOSSLayer", "dlinoss_layer_forward", "dlinoss_layer_backward", "DlinossLayerFn",
           "project_parameters", "unfused_layer_forward"]

_VARIANTS = {"imex1": 0, "imex2": 1, "im": 2, "ex": 3}
_LAYER_MAX = 256  # largest hidden_dim / ssm_size of the fused kernel
_CHUNK = 32       # steps per workgroup chunk (the carries' second dimension)
_LDS = 160 * 1024


def _bwd_fits(hidden: int, ssm: int) -> bool:
    """The fused backward's LDS (u or gy rows with bu over them, grad_bu tiles)
    fits one workgroup (mirrors layer_bwd_lds_bytes in dlinoss_layer.hip; true
    for every size up to 256)."""
    hp, pp = -(-hidden // 32) * 32, -(-ssm // 32) * 32
    return (_CHUNK * max(hp + 4, 2 * pp + 4) + _CHUNK * (2 * pp + 4) + 4 * ssm) * 4 <= _LDS


def project_parameters(A_diag: Tensor, G_diag: Tensor, steps: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """(a, g, dt) inside the stability region (reference _project_parameters,
    dlinoss.py:249-264): dt = sigmoid(steps), g = relu(G), a clamped to
    [(2 + dt g - 2 sqrt(1 + dt g)) / dt^2, (2 + dt g + 2 sqrt(1 + dt g)) / dt^2]
    with the clamp written as relu differences (the same values and gradients)."""
    dt = torch.sigmoid(steps)
    g = torch.relu(G_diag)
    dt2 = torch.clamp(dt * dt, min=1e-6)
    dg = dt * g
    root = torch.sqrt(torch.clamp(1.0 + dg, min=1e-6))
    lo = (2.0 + dg - 2.0 * root) / dt2
    hi = (2.0 + dg + 2.0 * root) / dt2
    a = lo + torch.relu(A_diag - lo) - torch.relu(A_diag - hi)
    return a, g, dt


def _check_layer_args(inputs: Tensor, B: Tensor, C: Tensor, D: Tensor, a: Tensor, g: Tensor,
                      step: Tensor) -> Tuple[int, int, int, int]:
    if inputs.dim() != 3:
        raise ValueError("DampedLinOSSLayer expects input of shape (batch, length, hidden_dim).")
    batch, length, hidden = inputs.shape
    if B.dim() != 3 or B.size(1) != hidden or B.size(2) != 2:
        raise RuntimeError(f"B must have shape (ssm_size, {hidden}, 2), got {tuple(B.shape)}")
    ssm = B.size(0)
    if tuple(C.shape) != (hidden, ssm, 2):
        raise RuntimeError(f"C must have shape ({hidden}, {ssm}, 2), got {tuple(C.shape)}")
    if tuple(D.shape) != (hidden,):
        raise RuntimeError(f"D must have shape ({hidden},), got {tuple(D.shape)}")
    for name, t in (("a_diag", a), ("g_diag", g), ("step", step)):
        if tuple(t.shape) != (ssm,):
            raise RuntimeError(f"{name} must have shape ({ssm},), got {tuple(t.shape)}")
    return batch, length, hidden, ssm


def _check_on_gpu(tensors, hidden: int, ssm: int) -> None:
    if any(t.dtype != torch.float32 for t in tensors):
        raise RuntimeError("the fused D-LinOSS layer computes in float32; got "
                           + ", ".join(str(t.dtype) for t in tensors))
    if not all(t.is_cuda for t in tensors) or len({t.device for t in tensors}) != 1:
        raise RuntimeError("the fused D-LinOSS layer needs every tensor on one GPU")
    if hidden > _LAYER_MAX or ssm > _LAYER_MAX:
        raise RuntimeError(f"the fused D-LinOSS layer supports hidden_dim and ssm_size up to "
                           f"{_LAYER_MAX}, got {hidden} and {ssm}")


def _check_carries(carries: Tensor, batch: int, length: int, ssm: int, device) -> None:
    want = (batch, -(-length // _CHUNK), ssm, 4)
    if tuple(carries.shape) != want or carries.dtype != torch.float32 or \
            not carries.is_contiguous() or carries.device != device:
        raise RuntimeError(f"carries must be a contiguous float32 {want} tensor on {device}")


def dlinoss_layer_forward(variant: str, inputs: Tensor, B: Tensor, C: Tensor, D: Tensor,
                          a_diag: Tensor, g_diag: Tensor, step: Tensor,
                          carries: Optional[Tensor] = None) -> Tensor:
    """y = Re(x C^T) + D u with x the D-LinOSS states driven by bu = u B^T, in
    one kernel launch.  Every tensor float32 on one GPU; a, g, step projected.
    ``carries`` (float32 [batch, ceil(length / 32), ssm, 4]) receives the state
    entering each chunk, for ``dlinoss_layer_backward``."""
    variant = variant.lower()
    if variant not in _VARIANTS:
        raise ValueError(f"Unknown D-LinOSS variant '{variant}'.")
    batch, length, hidden, ssm = _check_layer_args(inputs, B, C, D, a_diag, g_diag, step)
    tensors = (inputs, B, C, D, a_diag, g_diag, step)
    _check_on_gpu(tensors, hidden, ssm)
    u, Bc, Cc, Dc, a, g, s = (t.contiguous() for t in tensors)
    out = torch.empty_like(u)
    if out.numel() == 0:
        return out
    if carries is not None:
        _check_carries(carries, batch, length, ssm, u.device)
    lib = _lib.load()
    with torch.cuda.device(u.device):
        _lib.check(lib.ossm_dlinoss_layer_forward(
            _VARIANTS[variant], u.data_ptr(), Bc.data_ptr(), Cc.data_ptr(), Dc.data_ptr(),
            a.data_ptr(), g.data_ptr(), s.data_ptr(), out.data_ptr(), _lib.ptr(carries), batch,
            length, hidden, ssm, _lib.stream_of(u)))
    return out


def dlinoss_layer_backward(variant: str, inputs: Tensor, grad_output: Tensor, B: Tensor,
                           C: Tensor, D: Tensor, a_diag: Tensor, g_diag: Tensor, step: Tensor,
                           carries: Tensor):
    """Gradients of the fused layer: ``(grad_inputs, grad_B, grad_C, grad_D, grad_a,
    grad_g, grad_step)`` from the forward's ``carries``.  One kernel for
    grad_inputs and the scan's parameter gradients; grad_B and grad_C are GEMMs
    over the grad_bu and conj(x) it returns, grad_D a sum."""
    variant = variant.lower()
    if variant not in _VARIANTS:
        raise ValueError(f"Unknown D-LinOSS variant '{variant}'.")
    batch, length, hidden, ssm = _check_layer_args(inputs, B, C, D, a_diag, g_diag, step)
    if grad_output.shape != inputs.shape:
        raise RuntimeError(f"grad_output must have the inputs' shape {tuple(inputs.shape)}, "
                           f"got {tuple(grad_output.shape)}")
    tensors = (inputs, grad_output, B, C, D, a_diag, g_diag, step)
    _check_on_gpu(tensors, hidden, ssm)
    u, go, Bc, Cc, Dc, a, g, s = (t.contiguous() for t in tensors)
    dev = u.device
    _check_carries(carries, batch, length, ssm, dev)
    gu = torch.empty_like(u)
    gbu = torch.empty((batch, length, ssm, 2), dtype=torch.float32, device=dev)
    xq = torch.empty_like(gbu)
    ga, gg, gs = (torch.empty(ssm, dtype=torch.float32, device=dev) for _ in range(3))
    with torch.cuda.device(dev):
        _lib.check(_lib.load().ossm_dlinoss_layer_backward(
            _VARIANTS[variant], u.data_ptr(), go.data_ptr(), Bc.data_ptr(), Cc.data_ptr(),
            Dc.data_ptr(), a.data_ptr(), g.data_ptr(), s.data_ptr(), carries.data_ptr(),
            gu.data_ptr(), gbu.data_ptr(), xq.data_ptr(), ga.data_ptr(), gg.data_ptr(),
            gs.data_ptr(), batch, length, hidden, ssm, _lib.stream_of(u)))
    rows = batch * length
    uf, gof = u.reshape(rows, hidden), go.reshape(rows, hidden)
    # grad_B[p, h, c] = sum_r grad_bu[r, p, c] u[r, h];  grad_C[h, p, c] = sum_r go[r, h] xq[r, p, c]
    gB = _sum_rows_product(gbu.reshape(rows, 2 * ssm), uf)
    gB = gB.reshape(ssm, 2, hidden).permute(0, 2, 1).contiguous()
    gC = _sum_rows_product(gof, xq.reshape(rows, 2 * ssm)).reshape(hidden, ssm, 2)
    gD = (gof * uf).sum(0)
    return gu, gB, gC, gD, ga, gg, gs


def _sum_rows_product(a: Tensor, b: Tensor, split: int = 32) -> Tensor:
    """a^T b for row-major a [R, M], b [R, N] with R much larger than M, N (the
    weight gradients sum over every (batch, step) row): the first
    split * (R // split) rows are split into ``split`` slices multiplied as one
    batched GEMM and the partials added, the remaining rows (fewer than
    ``split``) by one small GEMM.  That is the shape the library GEMMs run
    well: one GEMM with K = R ran at ~24 TFLOP/s here, 16–64 slices at ~110
    (128 slices 104, 512 slices 80)."""
    R = a.size(0)
    n = R // split
    if n < 4:
        return a.t() @ b
    head = split * n
    out = torch.bmm(a[:head].view(split, n, -1).transpose(1, 2), b[:head].view(split, n, -1)).sum(0)
    if head < R:
        out += a[head:].t() @ b[head:]
    return out


def unfused_layer_forward(variant: str, inputs: Tensor, B: Tensor, C: Tensor, D: Tensor,
                          a_diag: Tensor, g_diag: Tensor, step: Tensor) -> Tensor:
    """The layer as separate steps (dlinoss.py:210-247): two real GEMMs for bu,
    the scan (``run_dlinoss``, this library's kernels), two GEMMs for Re(x C^T)
    and the D skip.  Differentiable; the fused layer's backward runs through it."""
    batch, length, hidden, ssm = _check_layer_args(inputs, B, C, D, a_diag, g_diag, step)
    flat = inputs.reshape(batch * length, hidden)
    bu = torch.complex(flat @ B[..., 0].t().contiguous(), flat @ B[..., 1].t().contiguous())
    bu_seq = bu.reshape(batch, length, ssm).permute(1, 0, 2).contiguous()
    if length == 0:
        x = bu_seq
    else:
        x = run_dlinoss(variant, a_diag, g_diag, step, bu_seq)
    xf = x.permute(1, 0, 2).reshape(batch * length, ssm)
    proj = xf.real @ C[..., 0].t().contiguous() - xf.imag @ C[..., 1].t().contiguous()
    return proj.reshape(batch, length, hidden) + inputs * D


class DlinossLayerFn(torch.autograd.Function):
    """Fused forward and backward (``dlinoss_layer_backward``); shapes whose
    backward does not fit recompute through ``unfused_layer_forward``."""

    @staticmethod
    def forward(ctx, variant: str, inputs: Tensor, B: Tensor, C: Tensor, D: Tensor,
                a_diag: Tensor, g_diag: Tensor, step: Tensor) -> Tensor:  # type: ignore[override]
        ctx.variant = variant
        batch, length, hidden = inputs.shape
        ssm = B.size(0)
        carries = None
        if any(ctx.needs_input_grad[1:]) and _bwd_fits(hidden, ssm):
            carries = torch.empty((batch, -(-length // _CHUNK), ssm, 4), dtype=torch.float32,
                                  device=inputs.device)
        ctx.fused_bwd = carries is not None
        ctx.save_for_backward(inputs, B, C, D, a_diag, g_diag, step, carries)
        return dlinoss_layer_forward(variant, inputs, B, C, D, a_diag, g_diag, step, carries)

    @staticmethod
    def backward(ctx, grad_out: Tensor):  # type: ignore[override]
        *saved, carries = ctx.saved_tensors
        needs = ctx.needs_input_grad[1:]
        if ctx.fused_bwd:
            grads = dlinoss_layer_backward(ctx.variant, *saved[:1], grad_out, *saved[1:], carries)
            return (None, *[gr if n else None for gr, n in zip(grads, needs)])
        with torch.enable_grad():
            leaves = [t.detach().requires_grad_(bool(n)) for t, n in zip(saved, needs)]
            y = unfused_layer_forward(ctx.variant, *leaves)
            wanted = [t for t in leaves if t.requires_grad]
            got = iter(torch.autograd.grad(y, wanted, grad_out)) if wanted else iter(())
        grads = [next(got) if t.requires_grad else None for t in leaves]
        return (None, *grads)


class DampedLinOSSLayer(nn.Module):
    """Single damped LinOSS layer (reference DampedLinOSSLayer, dlinoss.py:48-278)."""

    def __init__(self, ssm_size: int, hidden_dim: int, *, variant: str = "imex1",
                 initialization: str = "ring", r_min: float = 0.9, r_max: float = 1.0,
                 theta_min: float = 0.0, theta_max: float = math.pi, A_min: float = 0.0,
                 A_max: float = 1.0, G_min: float = 0.0, G_max: float = 1.0,
                 dt_std: float = 0.5) -> None:
        super().__init__()
        variant = variant.lower()
        if variant not in _VARIANTS:
            raise ValueError("DampedLinOSSLayer received unsupported variant "
                             f"'{variant}'. Expected one of {', '.join(_VARIANTS)}.")
        self.variant = variant
        self.ssm_size = ssm_size
        self.hidden_dim = hidden_dim
        self.init_config = dict(initialization=initialization.lower(), r_min=float(r_min),
                                r_max=float(r_max), theta_min=float(theta_min),
                                theta_max=float(theta_max), A_min=float(A_min), A_max=float(A_max),
                                G_min=float(G_min), G_max=float(G_max), dt_std=float(dt_std))
        self.A_diag = nn.Parameter(torch.empty(ssm_size))
        self.G_diag = nn.Parameter(torch.empty(ssm_size))
        self.steps = nn.Parameter(torch.empty(ssm_size))
        self.B = nn.Parameter(torch.empty(ssm_size, hidden_dim, 2))
        self.C = nn.Parameter(torch.empty(hidden_dim, ssm_size, 2))
        self.D = nn.Parameter(torch.empty(hidden_dim))
        self.reset_parameters()

    # -- initialisation (dlinoss.py:100-174) ---------------------------------
    def reset_parameters(self) -> None:
        nn.init.uniform_(self.B, -1.0 / math.sqrt(self.hidden_dim), 1.0 / math.sqrt(self.hidden_dim))
        nn.init.uniform_(self.C, -1.0 / math.sqrt(self.ssm_size), 1.0 / math.sqrt(self.ssm_size))
        nn.init.normal_(self.D, mean=0.0, std=1.0)
        kind = self.init_config["initialization"]
        if kind == "ring":
            a, g, steps = self._ring_values()
        elif kind == "uniform":
            a, g, steps = self._uniform_values()
        else:
            raise ValueError(f"Unknown initialization '{kind}'.")
        with torch.no_grad():
            self.A_diag.copy_(a)
            self.G_diag.copy_(g)
            self.steps.copy_(steps)

    def _ring_values(self) -> Tuple[Tensor, Tensor, Tensor]:
        """Eigenvalue pairs r e^{+-i theta} with r^2 uniform on [r_min^2, r_max^2]
        and theta uniform, mapped to (a, g) for dt = sigmoid(N(0, dt_std^2)): the
        pair's product fixes 1 / (1 + dt g), its sum then fixes a."""
        cfg, n = self.init_config, self.ssm_size
        dtype, device = self.A_diag.dtype, self.A_diag.device
        steps = torch.randn(n, dtype=dtype, device=device) * cfg["dt_std"]
        dt = torch.sigmoid(steps)
        r2 = torch.rand(n, dtype=dtype, device=device) * (cfg["r_max"] ** 2 - cfg["r_min"] ** 2) \
            + cfg["r_min"] ** 2
        theta = torch.rand(n, dtype=dtype, device=device) * (cfg["theta_max"] - cfg["theta_min"]) \
            + cfg["theta_min"]
        pair_sum = 2.0 * torch.sqrt(r2) * torch.cos(theta)
        pair_prod = r2
        g = (1.0 / torch.clamp(pair_prod, min=1e-6) - 1.0) / torch.clamp(dt, min=1e-6)
        g = torch.clamp(g, min=cfg["G_min"])
        a = (2.0 + dt * g - pair_sum * (1.0 + dt * g)) / torch.clamp(dt * dt, min=1e-6)
        return a, g, steps

    def _uniform_values(self) -> Tuple[Tensor, Tensor, Tensor]:
        """(A, G) uniform on their boxes and steps ~ N(0, dt_std^2), kept where the
        discrete oscillator is underdamped (G >= 0 and (G - dt A)^2 < 4 A,
        dlinoss.py:177-179), drawn until ssm_size samples are kept."""
        cfg, n = self.init_config, self.ssm_size
        dtype, device = self.A_diag.dtype, self.A_diag.device
        draw = max(4 * n, 512)
        kept: list[Tuple[Tensor, Tensor, Tensor]] = []
        total = 0
        while total < n:
            A = torch.rand(draw, dtype=dtype, device=device) * (cfg["A_max"] - cfg["A_min"]) + cfg["A_min"]
            G = torch.rand(draw, dtype=dtype, device=device) * (cfg["G_max"] - cfg["G_min"]) + cfg["G_min"]
            s = torch.randn(draw, dtype=dtype, device=device) * cfg["dt_std"]
            dt = torch.sigmoid(s)
            ok = (G >= 0) & ((G - dt * A) ** 2 - 4.0 * A < 0)
            if ok.any():
                kept.append((A[ok], G[ok], s[ok]))
                total += int(ok.sum())
        return tuple(torch.cat([k[i] for k in kept])[:n] for i in range(3))  # type: ignore[return-value]

    # -- forward (dlinoss.py:184-247) ----------------------------------------
    def forward(self, inputs: Tensor) -> Tensor:
        if inputs.dim() != 3:
            raise ValueError("DampedLinOSSLayer expects input of shape (batch, length, hidden_dim).")
        if inputs.size(-1) != self.hidden_dim:
            raise ValueError(f"Expected hidden_dim={self.hidden_dim}, received {inputs.size(-1)}.")
        dtype = inputs.dtype
        if dtype == torch.float64:
            raise RuntimeError("the MI355X D-LinOSS kernels compute in float32/complex64; "
                               "got float64 inputs")
        compute = torch.float32
        u = inputs.to(compute)
        params = [t.to(device=u.device, dtype=compute) for t in
                  (self.A_diag, self.G_diag, self.steps, self.B, self.C, self.D)]
        a, g, dt = project_parameters(*params[:3])
        Bw, Cw, Dw = params[3:]
        if u.is_cuda and self.hidden_dim <= _LAYER_MAX and self.ssm_size <= _LAYER_MAX:
            y = DlinossLayerFn.apply(self.variant, u, Bw, Cw, Dw, a, g, dt)
        else:
            y = unfused_layer_forward(self.variant, u, Bw, Cw, Dw, a, g, dt)
        return y if dtype == compute else y.to(dtype)
