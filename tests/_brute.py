"""Brute-force fp64 PyTorch recurrences used to pin the oracle by autograd.

These are sequential loops written from the mathematics of each scan, not
from the oracle's code: their backward passes come from torch.autograd, so a
wrong sign, index or transposition in the oracle's hand-written adjoint shows
up as a mismatch.  CPU only, small sizes.
"""

from __future__ import annotations

import torch


def dlinoss_matrices(variant: str, a, g, dt):
    """``(M [P,2,2], f [P,2])`` of the D-LinOSS recurrence s_t = M s_{t-1} + f bu_t.

    The variant table (reference _dlinoss_scan.py:54-101):
      imex1: S=1+dt g, M=[[1/S, -dt^2 a/S], [1/S, 1-dt^2 a/S]], f=[dt^2/S, dt^2/S]
      imex2: M=[[1-dt g, -dt a], [dt(1-dt g), 1-dt^2 a]], f=[dt, dt^2]
      im:    D=1+dt g+dt^2 a, M=[[1/D, -dt a/D], [dt/D, (1+dt g)/D]], f=[dt/D, dt^2/D]
      ex:    M=[[1-dt g, -dt a], [dt, 1]], f=[dt, 0]
    """
    one = torch.ones_like(a)
    if variant == "imex1":
        S = one + dt * g
        m = [[one / S, -(dt * dt * a) / S], [one / S, one - (dt * dt * a) / S]]
        f = [dt * dt / S, dt * dt / S]
    elif variant == "imex2":
        m = [[one - dt * g, -dt * a], [dt * (one - dt * g), one - dt * dt * a]]
        f = [dt, dt * dt]
    elif variant == "im":
        D = one + dt * g + dt * dt * a
        m = [[one / D, -(dt * a) / D], [dt / D, (one + dt * g) / D]]
        f = [dt / D, dt * dt / D]
    elif variant == "ex":
        m = [[one - dt * g, -dt * a], [dt, one]]
        f = [dt, torch.zeros_like(dt)]
    else:
        raise ValueError(variant)
    M = torch.stack([torch.stack(r, -1) for r in m], -2)
    return M, torch.stack(f, -1)


def dlinoss_states(variant: str, a, g, dt, bu):
    """States ``[L,B,P,2]`` by a plain loop; differentiable in every input."""
    M, f = dlinoss_matrices(variant, a, g, dt)
    L, B, P = bu.shape
    s = torch.zeros(B, P, 2, dtype=bu.dtype)
    out = []
    Mc = M.to(bu.dtype)
    fc = f.to(bu.dtype)
    for t in range(L):
        s = torch.einsum("pij,bpj->bpi", Mc, s) + fc.unsqueeze(0) * bu[t].unsqueeze(-1)
        out.append(s)
    return torch.stack(out, 0)


def linoss_states(a_matrix, b_seq):
    """``s_t = M s_{t-1} + b_t`` with complex ``M [P,2,2]``; ``b_seq [L,B,P,2]``."""
    L, B, P, _ = b_seq.shape
    s = torch.zeros(B, P, 2, dtype=b_seq.dtype)
    out = []
    for t in range(L):
        s = torch.einsum("pij,bpj->bpi", a_matrix, s) + b_seq[t]
        out.append(s)
    return torch.stack(out, 0)


def selective(u, dt, A, Bm, Cm, gate=None):
    """Mamba recurrence h = exp(dt A) h + dt B u, y = C.h, y*silu(z)."""
    Bsz, D, L = u.shape
    h = torch.zeros(Bsz, D, A.shape[1], dtype=u.dtype)
    ys = []
    for t in range(L):
        d = dt[:, :, t].unsqueeze(-1)
        h = torch.exp(d * A.unsqueeze(0)) * h + (d * Bm[:, t].unsqueeze(1)) * u[:, :, t].unsqueeze(-1)
        ys.append((h * Cm[:, t].unsqueeze(1)).sum(-1))
    y = torch.stack(ys, -1)
    if gate is not None:
        y = y * torch.nn.functional.silu(gate)
    return y


def sdlinoss_states(variant: str, A, G, step, bu):
    """States ``[L,B,M,2]`` of the selective D-LinOSS recurrence by a plain loop.

    Parameters broadcast against ``bu [L,B,M]`` the torch way (shapes (M,),
    (L,1,M), (1,B,M), (L,B,M)), so autograd sums their gradients over the
    broadcast axes.  Per step, dt = clamp(step, 1e-6, 1):
      imex1: w = (w + dt^2 (bu - a x)) / max(1 + dt g, 1e-6)
      imex2: w = ((1 - dt g) w + dt^2 (bu - a x)) / max(1 + dt^2 a, 1e-6)
      im:    w = (w + dt^2 (bu - a x)) / max(1 + dt g + dt^2 a, 1e-6)
      ex:    w = (1 - dt g) w + dt^2 (bu - a x)
    then x = x + w (the bridge's fallback, _sdlinoss_scan.py:150-197).
    """
    L, B, M = bu.shape
    shape = (L, B, M)
    a = A.expand(shape) if A.dim() == 3 else A.reshape(1, 1, M).expand(shape)
    g = G.expand(shape) if G.dim() == 3 else G.reshape(1, 1, M).expand(shape)
    st = step.expand(shape) if step.dim() == 3 else step.reshape(1, 1, M).expand(shape)
    dt = torch.clamp(st, min=1e-6, max=1.0)
    w = torch.zeros(B, M, dtype=bu.dtype)
    x = torch.zeros(B, M, dtype=bu.dtype)
    out = []
    for t in range(L):
        d, at, gt = dt[t], a[t], g[t]
        comb = bu[t] - at * x
        if variant == "imex1":
            w = (w + d * d * comb) / torch.clamp(1.0 + d * gt, min=1e-6)
        elif variant == "imex2":
            w = ((1.0 - d * gt) * w + d * d * comb) / torch.clamp(1.0 + d * d * at, min=1e-6)
        elif variant == "im":
            w = (w + d * d * comb) / torch.clamp(1.0 + d * gt + d * d * at, min=1e-6)
        elif variant == "ex":
            w = (1.0 - d * gt) * w + d * d * comb
        else:
            raise ValueError(variant)
        x = x + w
        out.append(torch.stack([w, x], -1))
    return torch.stack(out, 0)


def diag_states(lam, b_seq):
    """x_t = lam * x_{t-1} + b_t over complex b_seq [L, B, P] with complex lam [P]."""
    x = torch.zeros_like(b_seq[0])
    out = []
    for t in range(b_seq.shape[0]):
        x = lam * x + b_seq[t]
        out.append(x)
    return torch.stack(out, 0)


def mamba_mixer(inputs, params, d_conv: int, dt_rank: int, d_state: int):
    """The Mamba mixer forward of mambarec.py:136-184 as plain torch ops in the
    inputs' dtype: in_proj, causal depthwise conv + SiLU (torch's conv1d), x_proj,
    softplus(dt_proj(.)), the selective scan as a per-step loop in the
    reference's [B, C, L] layout (mambarec.py:23-61), the SiLU gate, out_proj.
    ``params`` maps the reference module's parameter names to tensors."""
    F = torch.nn.functional
    xz = inputs @ params["in_proj.weight"].T
    Di = xz.shape[-1] // 2
    x, z = xz[..., :Di], xz[..., Di:]
    xc = F.conv1d(F.pad(x.transpose(1, 2), (d_conv - 1, 0)), params["conv1d.weight"],
                  params.get("conv1d.bias"), groups=Di)
    xc = F.silu(xc)                                   # [B, D, L]
    proj = xc.transpose(1, 2) @ params["x_proj.weight"].T
    dt_raw = proj[..., :dt_rank]
    Bg = proj[..., dt_rank:dt_rank + d_state]
    Cg = proj[..., dt_rank + d_state:]
    dt = F.softplus(dt_raw @ params["dt_proj.weight"].T + params["dt_proj.bias"]).transpose(1, 2)
    A = -torch.exp(params["A_log"])
    h = torch.zeros(xc.shape[0], Di, d_state, dtype=xc.dtype)
    ys = []
    for t in range(xc.shape[2]):
        d = dt[:, :, t, None]
        h = torch.exp(d * A) * h + (d * Bg[:, t, None, :]) * xc[:, :, t, None]
        ys.append((h * Cg[:, t, None, :]).sum(-1))
    y = torch.stack(ys, -1) * F.silu(z.transpose(1, 2))
    return y.transpose(1, 2) @ params["out_proj.weight"].T
