"""CPU checks of the fused D-LinOSS layer's host side and its oracle: the
oracle's layer forward against the reference's layer fixture, the parameter
projection and the ring initialisation against closed forms.  No GPU call."""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
VARIANTS = oracle.VARIANTS


def _case(variant, dtype):
    cases = json.loads((GOLDEN / "dlinoss_reference_cases.json").read_text())["cases"]
    return cases[variant][dtype]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("dtype", ["float32", "float64"])
def test_oracle_layer_forward_matches_reference_fixture(variant, dtype):
    """oracle.dlinoss_layer_forward vs the outputs and states of the reference's
    layer fixture (tests/dlinoss_reference_cases.json, test_dlinoss_parity.py:73-116)."""
    c = _case(variant, dtype)
    rt = np.float32 if dtype == "float32" else np.float64
    tol = 5e-6 if dtype == "float32" else 1e-9  # the reference test's tolerances
    y, states = oracle.dlinoss_layer_forward(
        variant, np.asarray(c["inputs"], rt), np.asarray(c["B"], rt), np.asarray(c["C"], rt),
        np.asarray(c["D"], rt), np.asarray(c["A_diag"], rt), np.asarray(c["G_diag"], rt),
        np.asarray(c["step"], rt))
    assert y.dtype == rt
    np.testing.assert_allclose(y, np.asarray(c["outputs"]), rtol=tol, atol=tol)
    main = states[..., 1].transpose(1, 0, 2)
    np.testing.assert_allclose(np.stack([main.real, main.imag], -1),
                               np.asarray(c["states"]["main"]), rtol=tol, atol=tol)


def test_oracle_layer_forward_linear_pieces():
    """With the scan silenced (bu = 0 because B = 0) the layer is the D skip;
    with D = 0 it is linear in u (the scan and both projections are)."""
    rng = np.random.default_rng(5)
    nb, L, H, P = 2, 9, 5, 3
    u = rng.normal(size=(nb, L, H))
    Bw = rng.normal(size=(P, H, 2))
    Cw = rng.normal(size=(H, P, 2))
    Dw = rng.normal(size=H)
    a, g, dt = rng.uniform(0.1, 1, P), rng.uniform(0, 1, P), rng.uniform(0.2, 0.8, P)
    y0, _ = oracle.dlinoss_layer_forward("im", u, np.zeros_like(Bw), Cw, Dw, a, g, dt)
    np.testing.assert_allclose(y0, u * Dw, rtol=1e-14, atol=1e-14)
    z = np.zeros(H)
    y1, _ = oracle.dlinoss_layer_forward("im", u, Bw, Cw, z, a, g, dt)
    y2, _ = oracle.dlinoss_layer_forward("im", 2.5 * u, Bw, Cw, z, a, g, dt)
    np.testing.assert_allclose(y2, 2.5 * y1, rtol=1e-12, atol=1e-12)
    # one step, im variant: x_0 = f2 bu_0 with f2 = dt^2 / (1 + dt g + dt^2 a)
    y, _ = oracle.dlinoss_layer_forward("im", u[:, :1], Bw, Cw, z, a, g, dt)
    bu = u[:, 0] @ (Bw[..., 0] + 1j * Bw[..., 1]).T
    x = dt * dt / (1 + dt * g + dt * dt * a) * bu
    np.testing.assert_allclose(y[:, 0], x.real @ Cw[..., 0].T - x.imag @ Cw[..., 1].T,
                               rtol=1e-12, atol=1e-12)


def test_project_parameters_closed_form():
    from ossm_amd.layers import project_parameters

    dt = torch.tensor([0.3, 0.6, 0.9], dtype=torch.float64)
    g = torch.tensor([0.5, -1.0, 2.0], dtype=torch.float64)
    gr = torch.relu(g)
    root = torch.sqrt(1 + dt * gr)
    lo = (2 + dt * gr - 2 * root) / dt ** 2
    hi = (2 + dt * gr + 2 * root) / dt ** 2
    # below the band, inside it, above it
    a_raw = torch.stack([lo[0] - 1.0, 0.5 * (lo[1] + hi[1]), hi[2] + 3.0])
    a, gp, dtp = project_parameters(a_raw, g, torch.logit(dt))
    torch.testing.assert_close(dtp, dt)
    torch.testing.assert_close(gp, gr)
    torch.testing.assert_close(a, torch.stack([lo[0], a_raw[1], hi[2]]))


@pytest.mark.parametrize("variant", VARIANTS)
def test_project_parameters_keeps_fixture(variant):
    """The fixture's parameters lie inside the stable band, so the projection of
    (A, G, logit(step)) returns them (the reference test loads them this way)."""
    from ossm_amd.layers import project_parameters

    c = _case(variant, "float64")
    A, G, step = (torch.tensor(c[k], dtype=torch.float64) for k in ("A_diag", "G_diag", "step"))
    a, g, dt = project_parameters(A, G, torch.logit(step))
    torch.testing.assert_close(dt, step)
    torch.testing.assert_close(g, G)
    torch.testing.assert_close(a, A)


def test_ring_init_places_imex1_eigenvalues_on_the_ring():
    """For imex1, M(a, g, dt) has det 1 / (1 + dt g) and trace
    (2 + dt g - dt^2 a) / (1 + dt g); the ring initialisation solves these for a
    sampled pair r e^{+-i theta}, so M's eigenvalues have |lambda| in
    [r_min, r_max] and argument in [theta_min, theta_max]."""
    from ossm_amd.layers import DampedLinOSSLayer, project_parameters

    torch.manual_seed(0)
    layer = DampedLinOSSLayer(64, 8, variant="imex1", r_min=0.8, r_max=0.95, theta_min=0.2,
                              theta_max=2.5).double()
    a, g, dt = (t.detach().numpy() for t in project_parameters(layer.A_diag, layer.G_diag, layer.steps))
    S = 1 + dt * g
    M = np.stack([np.stack([1 / S, -dt * dt * a / S], -1), np.stack([1 / S, 1 - dt * dt * a / S], -1)], -2)
    lam = np.linalg.eigvals(M)
    r = np.abs(lam)
    assert np.all(r > 0.8 - 1e-6) and np.all(r < 0.95 + 1e-6)
    th = np.abs(np.angle(lam))
    assert np.all(th > 0.2 - 1e-6) and np.all(th < 2.5 + 1e-6)


def test_layer_module_interface():
    from ossm_amd.layers import DampedLinOSSLayer

    layer = DampedLinOSSLayer(6, 4, variant="IM", initialization="uniform")
    assert layer.variant == "im"
    shapes = {k: tuple(v.shape) for k, v in layer.state_dict().items()}
    assert shapes == {"A_diag": (6,), "G_diag": (6,), "steps": (6,), "B": (6, 4, 2),
                      "C": (4, 6, 2), "D": (4,)}
    # uniform init keeps only underdamped oscillators (dlinoss.py:177-179)
    dt = torch.sigmoid(layer.steps)
    assert bool(((layer.G_diag >= 0) & ((layer.G_diag - dt * layer.A_diag) ** 2 - 4 * layer.A_diag < 0)).all())
    with pytest.raises(ValueError, match="unsupported variant"):
        DampedLinOSSLayer(4, 4, variant="rk4")
    with pytest.raises(ValueError, match="shape \\(batch, length, hidden_dim\\)"):
        layer(torch.zeros(3, 4))
    with pytest.raises(ValueError, match="Expected hidden_dim=4"):
        layer(torch.zeros(1, 2, 5))
    with pytest.raises(RuntimeError, match="float32"):
        layer.double()(torch.zeros(1, 2, 4, dtype=torch.float64))
    bound = 1.0 / math.sqrt(4)
    assert float(layer.B.detach().abs().max()) <= bound
    assert float(layer.C.detach().abs().max()) <= 1.0 / math.sqrt(6)


def test_layer_entry_argument_checks():
    """The public fused-layer entries reject what the kernels cannot read before
    any device work: an unknown variant, a grad_output of another shape, and
    tensors that are not float32 on one GPU."""
    from ossm_amd import layers

    b, L, H, P = 2, 5, 4, 3
    args = [torch.zeros(b, L, H), torch.zeros(P, H, 2), torch.zeros(H, P, 2), torch.zeros(H),
            torch.ones(P), torch.ones(P), torch.ones(P)]
    carries = torch.zeros(b, 1, P, 4)
    with pytest.raises(ValueError, match="Unknown D-LinOSS variant"):
        layers.dlinoss_layer_backward("rk4", args[0], args[0], *args[1:], carries)
    with pytest.raises(RuntimeError, match="grad_output must have the inputs' shape"):
        layers.dlinoss_layer_backward("imex1", args[0], args[0][:, :2], *args[1:], carries)
    with pytest.raises(RuntimeError, match="one GPU"):
        layers.dlinoss_layer_backward("imex1", args[0], args[0], *args[1:], carries)
    with pytest.raises(RuntimeError, match="one GPU"):
        layers.dlinoss_layer_forward("imex1", *args)
    with pytest.raises(RuntimeError, match="float32"):
        layers.dlinoss_layer_forward("imex1", args[0].double(), *args[1:])


@pytest.mark.parametrize("rows", [3, 100, 127, 128, 130, 1000, 4096])
def test_weight_gradient_row_sum_split(rows):
    """The fused layer's weight gradients a^T b over every (batch, step) row,
    split into batched slices plus a remainder, equal the plain product."""
    from ossm_amd.layers import _sum_rows_product
    g = torch.Generator().manual_seed(rows)
    a = torch.randn(rows, 12, generator=g, dtype=torch.float64)
    b = torch.randn(rows, 7, generator=g, dtype=torch.float64)
    got = _sum_rows_product(a, b)
    assert got.shape == (12, 7)
    assert torch.allclose(got, a.t() @ b, rtol=1e-12, atol=1e-12)
