"""LinOSS layer on the MI355X scan, forward and backward.

``LinOSSLayer`` has the reference module's interface (models/linoss.py:172-315):
the constructor ``(ssm_size, hidden_dim, discretization)`` with ``"IM"`` or
``"IMEX"``, the parameters ``A_diag`` and ``steps`` [P], ``B`` [P, H, 2],
``C`` [H, P, 2] and ``D`` [H] with the same initialisation, and the same
forward contract, so a reference ``state_dict`` loads unchanged.

The recurrence ``s_t = M s_{t-1} + b_t`` runs through
``bridge.LinossMatrixScanFn``: the forward is ``linoss_scan`` and the backward
is the native ``linoss_scan_backward``, where the reference runs a Python
loop of about twenty torch operations per time step (linoss.py:83-151).
The layer glue around it (parameter maps, the B and C projections, the D
skip) is the reference's arithmetic in torch operations.

Transition per discretisation (a = relu(A_diag), dt = sigmoid(steps)):
  IM   (linoss.py:244-251): schur = 1 / (1 + dt^2 a),
       M = [[1 - dt^2 a schur, -dt a schur], [dt schur, schur]],
       b = (bu m11 dt, bu m21 dt)
  IMEX (linoss.py:253-258): M = [[1, -dt a], [dt, 1 - dt^2 a]], b = (bu dt, bu dt^2)
The layer output is Re(x C^T) + D u with x = s[..., 1].
"""

from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from .bridge import run_associative_scan

__all__ = ["LinOSSLayer", "linoss_transition"]


def linoss_transition(a_diag: Tensor, step: Tensor, discretization: str):
    """(m11, m12, m21, m22, f1, f2) of one discretisation: M entries and the
    per-oscillator factors that map bu onto the two input components."""
    dt2a = step * step * a_diag
    if discretization == "IM":
        schur = 1.0 / (1.0 + dt2a)
        m11, m12, m21, m22 = 1.0 - dt2a * schur, -step * a_diag * schur, step * schur, schur
        return m11, m12, m21, m22, m11 * step, m21 * step
    m11 = torch.ones_like(a_diag)
    return m11, -step * a_diag, step, 1.0 - dt2a, step, step * step


class LinOSSLayer(nn.Module):
    """Single LinOSS state-space layer (reference LinOSSLayer, linoss.py:172-315)."""

    def __init__(self, ssm_size: int, hidden_dim: int, discretization: str) -> None:
        super().__init__()
        if discretization not in {"IM", "IMEX"}:
            raise ValueError(f"Unsupported discretization '{discretization}'.")
        self.ssm_size = ssm_size
        self.hidden_dim = hidden_dim
        self.discretization = discretization
        self.A_diag = nn.Parameter(torch.empty(ssm_size))
        self.B = nn.Parameter(torch.empty(ssm_size, hidden_dim, 2))
        self.C = nn.Parameter(torch.empty(hidden_dim, ssm_size, 2))
        self.D = nn.Parameter(torch.empty(hidden_dim))
        self.steps = nn.Parameter(torch.empty(ssm_size))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        """reference reset_parameters (linoss.py:190-196)."""
        b_bound = 1.0 / math.sqrt(self.hidden_dim)
        c_bound = 1.0 / math.sqrt(self.ssm_size)
        nn.init.uniform_(self.A_diag, 0.0, 1.0)
        nn.init.uniform_(self.steps, 0.0, 1.0)
        nn.init.uniform_(self.B, -b_bound, b_bound)
        nn.init.uniform_(self.C, -c_bound, c_bound)
        nn.init.normal_(self.D, mean=0.0, std=1.0)

    def forward(self, inputs: Tensor) -> Tensor:
        if inputs.dim() != 3:
            raise ValueError("LinOSSLayer expects input of shape (batch, length, hidden_dim).")
        batch, length, hidden = inputs.shape
        if hidden != self.hidden_dim:
            raise ValueError(f"Expected hidden_dim={self.hidden_dim}, received {hidden}.")
        dtype, device = inputs.dtype, inputs.device
        cast = lambda t: t.to(device=device, dtype=dtype)  # noqa: E731
        a_diag = cast(torch.relu(self.A_diag))
        step = cast(torch.sigmoid(self.steps))
        flat = inputs.reshape(batch * length, hidden)
        # bu = u B^T as two real GEMMs, as the reference forms it (linoss.py:222-227)
        bu = torch.complex(flat @ cast(self.B[..., 0]).t(), flat @ cast(self.B[..., 1]).t())
        bu = bu.reshape(batch, length, self.ssm_size)
        if length == 0:
            x = bu.new_zeros(batch, 0, self.ssm_size)
        else:
            cd = bu.dtype
            m11, m12, m21, m22, f1, f2 = linoss_transition(a_diag, step, self.discretization)
            a_matrix = torch.stack((torch.stack((m11, m12), -1), torch.stack((m21, m22), -1)),
                                   -2).to(cd)
            bu_seq = bu.permute(1, 0, 2)  # [L, B, P]
            b_seq = torch.stack((bu_seq * f1.to(cd), bu_seq * f2.to(cd)), -1).contiguous()
            states = run_associative_scan(a_matrix, b_seq)  # [L, B, P, 2]
            x = states[..., 1].permute(1, 0, 2)  # [B, L, P]
        x = x.reshape(batch * length, self.ssm_size)
        y = x.real @ cast(self.C[..., 0]).t() - x.imag @ cast(self.C[..., 1]).t()
        return y.reshape(batch, length, hidden) + inputs * cast(self.D)
