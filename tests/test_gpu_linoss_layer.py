"""GPU tests of ``ossm_amd.linoss.LinOSSLayer``, the reference LinOSS layer
(models/linoss.py:172-315) on the device scan with the native backward:
the reference's layer snapshot (REFERENCE_LINOSS), and outputs plus every
parameter gradient against torch.autograd of an fp64 loop, for IM and IMEX."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from tests import _brute
from tests.gpu_util import announce, need_gpu

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def linoss():
    need_gpu()
    from ossm_amd import linoss as mod

    return mod


def test_linoss_layer_matches_reference_snapshot(linoss):
    """REFERENCE_LINOSS (the reference's test_linoss_parity.py:74-204): a
    LinOSS-IM layer with ssm_size 4, hidden_dim 6, its parameters and a
    [2, L, 6] input; the outputs it recorded."""
    ref = json.loads((GOLDEN / "linoss_reference_snapshot.json").read_text())
    layer = linoss.LinOSSLayer(4, 6, "IM").cuda()
    with torch.no_grad():
        layer.A_diag.copy_(torch.tensor(ref["A_diag"]))
        layer.B.copy_(torch.tensor(ref["B"]))
        layer.C.copy_(torch.tensor(ref["C"]).reshape(6, 4, 2))
        layer.D.copy_(torch.tensor(ref["D"]))
        layer.steps.copy_(torch.tensor(ref["steps"]))
    u = torch.tensor(ref["inputs"], dtype=torch.float32).cuda()
    announce("linoss layer snapshot")
    out = layer(u)
    np.testing.assert_allclose(out.detach().cpu().numpy(), np.asarray(ref["outputs"]),
                               rtol=5e-6, atol=5e-6)


def _layer64(params, u, disc):
    """The layer's arithmetic in fp64 over the brute-force loop (the reference's
    own fp64 path: the doubling scan is the same recurrence)."""
    A_diag, Bw, Cw, Dw, steps = params
    a = torch.relu(A_diag)
    dt = torch.sigmoid(steps)
    if disc == "IM":
        schur = 1.0 / (1.0 + dt * dt * a)
        m = (1.0 - dt * dt * a * schur, -dt * a * schur, dt * schur, schur)
        f1, f2 = m[0] * dt, m[2] * dt
    else:
        m = (torch.ones_like(a), -dt * a, dt, 1.0 - dt * dt * a)
        f1, f2 = dt, dt * dt
    Bc = torch.complex(Bw[..., 0], Bw[..., 1])
    bu = torch.matmul(u.to(Bc.dtype), Bc.t()).permute(1, 0, 2)  # [L, B, P]
    M = torch.stack((torch.stack(m[:2], -1), torch.stack(m[2:], -1)), -2).to(Bc.dtype)
    b_seq = torch.stack((bu * f1.to(Bc.dtype), bu * f2.to(Bc.dtype)), -1)
    x = _brute.linoss_states(M, b_seq)[..., 1].permute(1, 0, 2)
    return x.real @ Cw[..., 0].t() - x.imag @ Cw[..., 1].t() + u * Dw


@pytest.mark.parametrize("disc", ["IM", "IMEX"])
@pytest.mark.parametrize("shape", [(2, 1, 5, 3), (3, 300, 12, 20)], ids=lambda s: "x".join(map(str, s)))
def test_linoss_layer_grads_vs_fp64(linoss, disc, shape):
    """Outputs and the gradients of A_diag, B, C, D and steps, through the
    device scan and its native backward, against fp64 autograd."""
    Bsz, L, H, P = shape
    torch.manual_seed(31 + L)
    layer = linoss.LinOSSLayer(P, H, disc)
    u = torch.randn(Bsz, L, H)
    w = torch.randn(Bsz, L, H)
    announce(f"linoss layer {disc} {shape}")
    dev = layer.cuda()
    out = dev(u.cuda())
    (out * w.cuda()).sum().backward()
    ref = [p.detach().double().cpu().requires_grad_() for p in
           (layer.A_diag, layer.B, layer.C, layer.D, layer.steps)]
    out64 = _layer64(ref, u.double(), disc)
    (out64 * w.double()).sum().backward()
    np.testing.assert_allclose(out.detach().cpu().numpy(), out64.detach().numpy(),
                               rtol=5e-4, atol=1e-4)
    for p, r, name in zip((dev.A_diag, dev.B, dev.C, dev.D, dev.steps), ref,
                          ("A_diag", "B", "C", "D", "steps")):
        np.testing.assert_allclose(p.grad.cpu().numpy(), r.grad.numpy(), rtol=5e-4,
                                   atol=1e-4 * max(1.0, float(r.grad.abs().max())), err_msg=name)


def test_linoss_matrix_scan_fn_complex_matrix(linoss):
    """``LinossMatrixScanFn`` with a complex [P, 2, 2] matrix keeps a complex
    gradient (linoss.py:122-126); length-1 sequences pass through as s_0 = b_0."""
    from ossm_amd import bridge

    rng = np.random.default_rng(12)
    L, B, P = 40, 2, 5
    M = (rng.normal(size=(P, 2, 2)) + 1j * rng.normal(size=(P, 2, 2))) * 0.4
    b = rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))
    G = rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))
    announce("linoss matrix scan fn complex")
    tM = torch.tensor(M, dtype=torch.complex64, device="cuda", requires_grad=True)
    tb = torch.tensor(b, dtype=torch.complex64, device="cuda", requires_grad=True)
    s = bridge.run_associative_scan(tM, tb)
    (s * torch.tensor(G, dtype=torch.complex64, device="cuda").conj()).real.sum().backward()
    rM = torch.tensor(M, requires_grad=True)
    rb = torch.tensor(b, requires_grad=True)
    (_brute.linoss_states(rM, rb) * torch.tensor(G).conj()).real.sum().backward()
    assert tM.grad.dtype == torch.complex64
    np.testing.assert_allclose(tM.grad.cpu().numpy(), rM.grad.numpy(), rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(tb.grad.cpu().numpy(), rb.grad.numpy(), rtol=1e-4, atol=1e-4)
    one = torch.tensor(b[:1], dtype=torch.complex64, device="cuda")
    assert torch.equal(bridge.run_associative_scan(tM.detach(), one), one)
