"""Layer-level parity through the autograd bridges (ossm_amd.bridge), in the
shape of the reference's kernel-vs-fallback tests: the reference compares its
kernel path with its pure-PyTorch path on a layer's outputs and every
parameter gradient (tests/test_dlinoss_kernels.py:14-70, fp32 atol 1e-4 /
rtol 5e-4; tests/test_scan_parity.py:138-183 for the selective scan).  Here the
other side is a plain fp64 loop on the CPU (tests/_brute.py) differentiated by
torch.autograd.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import _brute
from tests.gpu_util import announce, need_gpu

pytestmark = pytest.mark.gpu
VARIANTS = ("imex1", "imex2", "im", "ex")


@pytest.fixture(scope="module")
def bridge():
    need_gpu()
    from ossm_amd import bridge

    return bridge


def _layer_params(P, H, seed):
    g = torch.Generator().manual_seed(seed)
    A = torch.rand(P, generator=g) * 0.9 + 0.1
    G = torch.rand(P, generator=g)
    steps = torch.randn(P, generator=g)
    Bw = torch.randn(P, H, 2, generator=g) / H ** 0.5
    Cw = torch.randn(H, P, 2, generator=g) / P ** 0.5
    Dw = torch.randn(H, generator=g)
    return A, G, steps, Bw, Cw, Dw


def _dlinoss_layer(run, variant, A, G, steps, Bw, Cw, Dw, u):
    """DampedLinOSSLayer.forward glue (dlinoss.py:184-278): projected
    parameters, bu = u B^T, x = scan, y = Re(x C^T) + D u."""
    dt = torch.sigmoid(steps)
    g = torch.relu(G)
    s = dt * g
    base = torch.sqrt(torch.clamp(1.0 + s, min=1e-6))
    denom = torch.clamp(dt * dt, min=1e-6)
    a = torch.minimum(torch.maximum(A, (2.0 + s - 2.0 * base) / denom), (2.0 + s + 2.0 * base) / denom)
    Bc = torch.complex(Bw[..., 0], Bw[..., 1])
    Cc = torch.complex(Cw[..., 0], Cw[..., 1])
    bu = torch.matmul(u.to(Bc.dtype), Bc.transpose(0, 1)).permute(1, 0, 2).contiguous()  # [L,B,P]
    x = run(variant, a, g, dt, bu).permute(1, 0, 2)                                        # [B,L,P]
    return torch.matmul(x, Cc.transpose(0, 1)).real + u * Dw


# (B, L, P, H): the reference test's layer (ssm_size=8, hidden_dim=16, inputs
# [3, 12, 16]) and a longer sequence
LAYER_SHAPES = [(3, 12, 8, 16), (3, 300, 24, 16)]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("shape", LAYER_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_dlinoss_layer_outputs_and_grads(bridge, variant, shape):
    Bsz, L, P, H = shape
    announce(f"bridge dlinoss layer {variant} {shape}")
    params = _layer_params(P, H, seed=7)
    if variant == "ex" and L > 50:
        # the explicit variant grows by sqrt(1 + dt^2 a - dt g) per step where
        # dt a > g; keep dt small so 300 steps stay representable in fp32
        params = (params[0], params[1], params[2] - 3.0) + params[3:]
    u = torch.randn(Bsz, L, H, generator=torch.Generator().manual_seed(8))
    w = torch.randn(Bsz, L, H, generator=torch.Generator().manual_seed(9))

    dev = [p.cuda().requires_grad_() for p in params]
    y = _dlinoss_layer(bridge.run_dlinoss, variant, *dev, u.cuda())
    (y * w.cuda()).sum().backward()

    ref = [p.double().requires_grad_() for p in params]

    def brute(variant, a, g, dt, bu):
        return _brute.dlinoss_states(variant, a, g, dt, bu)[..., 1]

    y64 = _dlinoss_layer(brute, variant, *ref, u.double())
    (y64 * w.double()).sum().backward()
    np.testing.assert_allclose(y.detach().cpu().numpy(), y64.detach().numpy(), rtol=5e-4, atol=1e-4)
    for got, r, name in zip(dev, ref, ("A", "G", "steps", "B", "C", "D")):
        np.testing.assert_allclose(got.grad.cpu().numpy(), r.grad.numpy(), rtol=5e-4,
                                   atol=1e-4 * max(1.0, float(r.grad.abs().max())), err_msg=name)


@pytest.mark.parametrize("variant", VARIANTS)
def test_dlinoss_bridge_fp64_runs_complex128_kernels(bridge, variant):
    """float64 coefficients select the complex128 kernels (the reference's
    precision rule, _dlinoss_scan.py:35-48): the layer's outputs and every
    gradient against autograd of the brute fp64 loop, at rtol 1e-9."""
    Bsz, L, P, H = 2, 60, 6, 5
    announce(f"bridge dlinoss fp64 {variant}")
    params = [p.double() for p in _layer_params(P, H, seed=17)]
    u = torch.randn(Bsz, L, H, generator=torch.Generator().manual_seed(18), dtype=torch.float64)
    w = torch.randn(Bsz, L, H, generator=torch.Generator().manual_seed(19), dtype=torch.float64)
    dev = [p.cuda().requires_grad_() for p in params]
    y = _dlinoss_layer(bridge.run_dlinoss, variant, *dev, u.cuda())
    assert y.dtype == torch.float64
    (y * w.cuda()).sum().backward()
    ref = [p.clone().requires_grad_() for p in params]

    def brute(variant, a, g, dt, bu):
        return _brute.dlinoss_states(variant, a, g, dt, bu)[..., 1]

    y64 = _dlinoss_layer(brute, variant, *ref, u)
    (y64 * w).sum().backward()
    np.testing.assert_allclose(y.detach().cpu().numpy(), y64.detach().numpy(), rtol=1e-9, atol=1e-11)
    for got, r, name in zip(dev, ref, ("A", "G", "steps", "B", "C", "D")):
        np.testing.assert_allclose(got.grad.cpu().numpy(), r.grad.numpy(), rtol=1e-9,
                                   atol=1e-11 * max(1.0, float(r.grad.abs().max())), err_msg=name)


def test_dlinoss_bridge_rejects_bad_variant(bridge):
    x = torch.zeros(4, 1, 2, dtype=torch.complex128, device="cuda")
    p = torch.ones(2, dtype=torch.float64, device="cuda")
    with pytest.raises(ValueError, match="Unknown D-LinOSS variant"):
        bridge.run_dlinoss("nope", p, p, p, x)
    assert bridge.has_kernels() and bridge.has_kernels("im")


def test_linoss_im_layer_grads(bridge):
    """LinOSS-IM recurrence (linoss.py:244-251, 260-315) through try_run_scan
    with the native backward, vs autograd of a fp64 loop."""
    Bsz, L, P, H = 2, 400, 20, 12
    announce("bridge linoss IM")
    g = torch.Generator().manual_seed(3)
    A0 = torch.rand(P, generator=g)
    st0 = torch.randn(P, generator=g)
    Bw0 = torch.randn(P, H, 2, generator=g) / H ** 0.5
    u = torch.randn(Bsz, L, H, generator=g)
    w = torch.randn(L, Bsz, P, generator=g)

    def layer(scan, A, steps, Bw, uu):
        dt = torch.sigmoid(steps)
        a = torch.relu(A)
        schur = 1.0 / (1.0 + dt * dt * a)
        m11, m12, m21, m22 = (1.0 - dt * dt * a * schur), (-dt * a * schur), dt * schur, schur
        Bc = torch.complex(Bw[..., 0], Bw[..., 1])
        bu = torch.matmul(uu.to(Bc.dtype), Bc.transpose(0, 1)).permute(1, 0, 2)
        cd = Bc.dtype
        b_seq = torch.stack([bu * (m11 * dt).to(cd), bu * (m21 * dt).to(cd)], -1).contiguous()
        states = scan(m11.to(cd).contiguous(), m12.to(cd).contiguous(), m21.to(cd).contiguous(),
                      m22.to(cd).contiguous(), b_seq)
        return states[..., 1].real

    dev = [x.cuda().requires_grad_() for x in (A0, st0, Bw0)]
    out = layer(bridge.try_run_scan, *dev, u.cuda())
    (out * w.cuda()).sum().backward()

    def brute_scan(m11, m12, m21, m22, b_seq):
        M = torch.stack([torch.stack([m11, m12], -1), torch.stack([m21, m22], -1)], -2)
        return _brute.linoss_states(M, b_seq)

    ref = [x.double().requires_grad_() for x in (A0, st0, Bw0)]
    out64 = layer(brute_scan, *ref, u.double())
    (out64 * w.double()).sum().backward()
    np.testing.assert_allclose(out.detach().cpu().numpy(), out64.detach().numpy(), rtol=5e-4, atol=1e-4)
    for got, r, name in zip(dev, ref, ("A", "steps", "B")):
        np.testing.assert_allclose(got.grad.cpu().numpy(), r.grad.numpy(), rtol=5e-4,
                                   atol=1e-4 * max(1.0, float(r.grad.abs().max())), err_msg=name)


@pytest.mark.parametrize("gated", [True, False], ids=["gate", "nogate"])
def test_selective_bridge_grads(bridge, gated):
    """try_selective_scan with autograd vs the fp64 Mamba loop (the reference's
    CUDA parity test shape: B=2, D=32, L=256, N=32, rtol 2e-4 / atol 1e-4)."""
    Bsz, D, L, N = 2, 32, 256, 32
    announce(f"bridge selective gated={gated}")
    g = torch.Generator().manual_seed(21)
    u = torch.randn(Bsz, D, L, generator=g)
    dt = torch.nn.functional.softplus(torch.randn(Bsz, D, L, generator=g) - 4.0)
    A = -torch.exp(torch.log(torch.arange(1, N + 1, dtype=torch.float32))).repeat(D, 1)
    Bm = torch.randn(Bsz, L, N, generator=g)
    Cm = torch.randn(Bsz, L, N, generator=g)
    z = torch.randn(Bsz, D, L, generator=g) if gated else None
    w = torch.randn(Bsz, D, L, generator=g)
    base = [u, dt, A, Bm, Cm] + ([z] if gated else [])
    dev = [x.cuda().requires_grad_() for x in base]
    y = bridge.try_selective_scan(*dev[:5], dev[5] if gated else None)
    (y * w.cuda()).sum().backward()
    ref = [x.double().requires_grad_() for x in base]
    y64 = _brute.selective(*ref[:5], ref[5] if gated else None)
    (y64 * w.double()).sum().backward()
    np.testing.assert_allclose(y.detach().cpu().numpy(), y64.detach().numpy(), rtol=2e-4, atol=1e-4)
    names = ("u", "dt", "A", "B", "C", "z")
    for got, r, name in zip(dev, ref, names):
        np.testing.assert_allclose(got.grad.cpu().numpy(), r.grad.numpy(), rtol=2e-4,
                                   atol=1e-4 * max(1.0, float(r.grad.abs().max())), err_msg=name)
    with torch.no_grad():
        y_ng = bridge.try_selective_scan(*[x.detach() for x in dev[:5]],
                                         dev[5].detach() if gated else None)
    assert torch.equal(y_ng, y.detach())


def _sdlinoss_layer(run, variant, W, u):
    """SelectiveDLinOSSLayer.forward glue (sdlinoss.py:153-238, without the
    causal conv): per-step (r, theta, dt) heads, the variant's (A, G) from them,
    bu = u B^T, x = scan, y = Re(x C^T) + D u."""
    Wf, Wr, Wth, Wdt, rb, thb, dtb, Bw, Cw, Dw = W
    feats = torch.tanh(u @ Wf)
    r = torch.sigmoid(rb + feats @ Wr)
    theta = np.pi * torch.tanh(thb + feats @ Wth)
    dt = 0.02 + 0.98 * torch.sigmoid(dtb + feats @ Wdt)
    r2 = torch.clamp(r * r, min=1e-8)
    c = torch.cos(theta)
    if variant == "imex1":
        A, G = (r2 - 2 * r * c + 1) / (dt * dt * r2), (1 - r2) / (dt * r2)
    elif variant == "imex2":
        A, G = (r2 - 2 * r * c + 1) / (dt * dt), (1 - r2) / dt
    elif variant == "im":
        A, G = (r2 - 2 * r * c + 1) / (dt * dt * r2), (-2 * r2 + 2 * r * c) / (dt * r2)
    else:
        A, G = (r2 - 2 * r * c + 1) / (dt * dt), (2 - 2 * r * c) / dt
    Bc = torch.complex(Bw[..., 0], Bw[..., 1])
    Cc = torch.complex(Cw[..., 0], Cw[..., 1])
    bu = torch.matmul(u.to(Bc.dtype), Bc.transpose(0, 1))
    perm = lambda t: t.permute(1, 0, 2).contiguous()  # noqa: E731  [B,L,M] -> [L,B,M]
    x = run(variant, perm(A), perm(G), perm(dt), perm(bu)).permute(1, 0, 2)
    return torch.matmul(x, Cc.transpose(0, 1)).real + u * Dw


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("shape", [(2, 12, 8, 16), (3, 257, 24, 16)], ids=lambda s: "x".join(map(str, s)))
def test_sdlinoss_layer_outputs_and_grads(bridge, variant, shape):
    """Selective D-LinOSS layer through ``run_sdlinoss``: outputs and every weight's
    gradient vs torch.autograd of the fp64 loop (tolerances of the D-LinOSS test).
    Pole radii r = sigmoid(.) around 0.4: a radius near 1 integrates the input into
    states of 1e5 and more, whose fp32 rounding alone exceeds these tolerances."""
    Bsz, L, M, H = shape
    announce(f"bridge sdlinoss layer {variant} {shape}")
    g = torch.Generator().manual_seed(21)
    W = [torch.randn(H, H, generator=g) / H ** 0.5, torch.randn(H, M, generator=g) * 0.3,
         torch.randn(H, M, generator=g) * 0.3, torch.randn(H, M, generator=g) * 0.3,
         torch.randn(M, generator=g) * 0.5 - 0.5, torch.randn(M, generator=g) * 0.5,
         torch.randn(M, generator=g) - 1.0, torch.randn(M, H, 2, generator=g) / H ** 0.5,
         torch.randn(H, M, 2, generator=g) / M ** 0.5, torch.randn(H, generator=g)]
    if variant == "ex":
        # the explicit scheme's poles leave the unit disc as theta -> pi
        # (det M = 2 r cos(theta) - 1): keep theta small
        W[2], W[5] = W[2] * 0.2, W[5] * 0.2
    u = torch.randn(Bsz, L, H, generator=torch.Generator().manual_seed(22))
    w = torch.randn(Bsz, L, H, generator=torch.Generator().manual_seed(23))

    dev = [p.cuda().requires_grad_() for p in W]
    y = _sdlinoss_layer(bridge.run_sdlinoss, variant, dev, u.cuda())
    (y * w.cuda()).sum().backward()

    ref = [p.double().requires_grad_() for p in W]

    def brute(variant, A, G, dt, bu):
        return _brute.sdlinoss_states(variant, A, G, dt, bu)[..., 1]

    y64 = _sdlinoss_layer(brute, variant, ref, u.double())
    (y64 * w.double()).sum().backward()
    np.testing.assert_allclose(y.detach().cpu().numpy(), y64.detach().numpy(), rtol=5e-4, atol=1e-4)
    names = ("Wf", "Wr", "Wth", "Wdt", "r_base", "th_base", "dt_base", "B", "C", "D")
    for got, r, name in zip(dev, ref, names):
        np.testing.assert_allclose(got.grad.cpu().numpy(), r.grad.numpy(), rtol=5e-4,
                                   atol=1e-4 * max(1.0, float(r.grad.abs().max())), err_msg=name)


@pytest.mark.parametrize("variant", VARIANTS)
def test_dlinoss_torch_library_ops_opcheck(bridge, variant):
    """``torch.library.opcheck`` on ``ossm::dlinoss_<v>_{forward,backward}``
    (schema, fake-tensor / Meta consistency with the device kernels, AOT
    dispatch), and a ``torch.compile`` trace of ``run_dlinoss`` that agrees
    with the eager call (to the last bits the look-back's association may
    change between runs)."""
    assert bridge.CUSTOM_OPS
    g = torch.Generator().manual_seed(5)
    L, B, P = 70, 2, 9
    a = (torch.rand(P, generator=g) * 0.9 + 0.1).cuda()
    gg = torch.rand(P, generator=g).cuda()
    dt = torch.sigmoid(torch.randn(P, generator=g)).cuda()
    bu = torch.complex(torch.randn(L, B, P, generator=g), torch.randn(L, B, P, generator=g)).cuda()
    go = torch.complex(torch.randn(L, B, P, generator=g), torch.randn(L, B, P, generator=g)).cuda()
    announce(f"torch.library opcheck dlinoss_{variant}")
    fwd = getattr(torch.ops.ossm, f"dlinoss_{variant}_forward")
    bwd = getattr(torch.ops.ossm, f"dlinoss_{variant}_backward")
    torch.library.opcheck(fwd, (a, gg, dt, bu))
    states = fwd(a, gg, dt, bu)
    torch.library.opcheck(bwd, (a, gg, dt, bu, states, go))
    # complex128 with float64 coefficients, as the reference's dispatcher takes
    d64 = [t.double() for t in (a, gg, dt)] + [bu.to(torch.complex128)]
    torch.library.opcheck(fwd, tuple(d64))
    st64 = fwd(*d64)
    assert st64.dtype == torch.complex128
    torch.library.opcheck(bwd, (*d64, st64, go.to(torch.complex128)))
    eager = bridge.run_dlinoss(variant, a, gg, dt, bu)
    compiled = torch.compile(lambda *xs: bridge.run_dlinoss(variant, *xs), backend="aot_eager",
                             fullgraph=True)
    torch.testing.assert_close(compiled(a, gg, dt, bu), eager, rtol=1e-6, atol=1e-6)
