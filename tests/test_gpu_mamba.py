"""GPU parity of the Mamba mixer kernels (ossm_amd.mamba through the C ABI):
the causal depthwise conv + SiLU and the selective scan in the mixer's
[B, L, D] layout against the CPU oracle and fp64 autograd, the scan against
this library's [B, D, L] drop-in scan on transposed inputs, and the whole
mixer against a brute-force fp64 mixer.

Tolerances: forward rtol 1e-4 / atol 1e-5 x magnitude against the fp32 oracle
with the fp64 oracle as arbiter (assert_parity); gradients elementwise against
the same computation in fp32 on the CPU (torch autograd), at rtol 1e-4 and the
magnitude-scaled atol of sums, with fp64 autograd as the arbiter
(assert_grad_parity).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests import _brute
from tests.gpu_util import (announce, assert_grad_parity, assert_parity, need_gpu, no_device_errors,
                            sum_atol, to_dev, to_np)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    need_gpu()
    from ossm_amd import mamba

    return mamba


def _conv_ref64(x, w, b):
    """silu(causal depthwise conv) in fp64 on the CPU with autograd (torch's conv1d)."""
    K = w.shape[-1]
    D = x.shape[-1]
    y = F.silu(F.conv1d(F.pad(x.transpose(1, 2), (K - 1, 0)), w.reshape(D, 1, K), b, groups=D))
    return y.transpose(1, 2)


CONV_SHAPES = [(1, 1, 4, 4), (2, 37, 12, 4), (3, 200, 64, 4), (2, 130, 7, 3), (2, 50, 20, 1),
               (1, 300, 33, 8), (4, 1000, 256, 4)]


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("strided", [False, True])
def test_conv_silu_forward_backward(M, shape, strided):
    nb, L, D, K = shape
    announce(f"mamba conv B={nb} L={L} D={D} K={K} strided={strided}")
    rng = np.random.default_rng(L + D)
    xz = rng.normal(size=(nb, L, 2 * D if strided else D)).astype(np.float32)
    w = (rng.normal(size=(D, 1, K)) * 0.5).astype(np.float32)
    b = (rng.normal(size=D) * 0.1).astype(np.float32)
    go = rng.normal(size=(nb, L, D)).astype(np.float32)
    base = to_dev(xz)
    x = base[..., :D].detach().requires_grad_(True) if not strided else base[..., :D]
    if strided:
        base.requires_grad_(True)
        x = base[..., :D]
    tw, tb = to_dev(w).requires_grad_(True), to_dev(b).requires_grad_(True)
    y = M.mamba_conv_silu(x, tw, tb)
    y.backward(to_dev(go))
    refs = {}
    for dt_ in (torch.float32, torch.float64):
        xr = torch.tensor(xz[..., :D], dtype=dt_, requires_grad=True)
        wr = torch.tensor(w, dtype=dt_, requires_grad=True)
        br = torch.tensor(b, dtype=dt_, requires_grad=True)
        out = _conv_ref64(xr, wr, br)
        out.backward(torch.tensor(go, dtype=dt_))
        refs[dt_] = [out.detach().numpy(), xr.grad.numpy(), wr.grad.numpy(), br.grad.numpy()]
    r32, r64 = refs[torch.float32], refs[torch.float64]
    y32 = oracle.mamba_conv_silu(xz[..., :D], w, b)
    assert_parity(to_np(y), y32, r64[0], rtol=1e-5, atol=1e-6, what="conv out")
    gx = to_np(base.grad[..., :D]) if strided else to_np(x.grad)
    if strided:
        assert np.all(to_np(base.grad[..., D:]) == 0)
    for got, a, b_, n in zip((gx, to_np(tw.grad), to_np(tb.grad)), r32[1:], r64[1:], ("x", "w", "b")):
        assert_grad_parity(got, a, b_, f"conv grad {n}")
    no_device_errors()


def _scan_inputs(nb, L, D, N, R, seed):
    """Mixer-shaped scan inputs: u, z as [B,L,D] (z a view into [B,L,2D]), dt
    before softplus with a bias, B and C views into a [B, L, R + 2N] projection."""
    rng = np.random.default_rng(seed)
    u = rng.normal(size=(nb, L, D)).astype(np.float32)
    xz = rng.normal(size=(nb, L, 2 * D)).astype(np.float32)
    dt_pre = (rng.normal(size=(nb, L, D)) * 0.5).astype(np.float32)
    bias = rng.uniform(-5, -2, D).astype(np.float32)
    A = (-np.arange(1, N + 1, dtype=np.float32)[None, :].repeat(D, 0)
         * rng.uniform(0.5, 1.5, (D, 1))).astype(np.float32)
    proj = rng.normal(size=(nb, L, R + 2 * N)).astype(np.float32)
    return u, xz, dt_pre, bias, A, proj


def _views(M, u, xz, dt_pre, bias, A, proj, D, N, R, grad=False):
    tu, txz, tdt, tb, tA, tp = (to_dev(v) for v in (u, xz, dt_pre, bias, A, proj))
    if grad:
        for t in (tu, txz, tdt, tb, tA, tp):
            t.requires_grad_(True)
    z = txz[..., D:]
    Bv, Cv = tp[..., R:R + N], tp[..., R + N:]
    return (tu, txz, tdt, tb, tA, tp), (tu, tdt, tA, Bv, Cv, z, tb)


SCAN_SHAPES = [(1, 1, 4, 1, 1), (2, 37, 20, 5, 2), (3, 200, 64, 16, 4), (2, 130, 36, 17, 3),
               (2, 64, 70, 33, 1), (1, 1000, 128, 16, 8), (2, 97, 30, 4, 2)]


@pytest.mark.parametrize("shape", SCAN_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_scan_bld_forward_matches_oracle(M, shape):
    nb, L, D, N, R = shape
    announce(f"mamba scan fwd B={nb} L={L} D={D} N={N}")
    u, xz, dt_pre, bias, A, proj = _scan_inputs(nb, L, D, N, R, 3)
    _, args = _views(M, u, xz, dt_pre, bias, A, proj, D, N, R)
    y = to_np(M.selective_scan_mamba(*args[:5], gate=args[5], dt_bias=args[6]))
    Bg, Cg, z = proj[..., R:R + N], proj[..., R + N:], xz[..., D:]
    y32 = oracle.selective_forward_bld(u, dt_pre, A, Bg, Cg, gate=z, dt_bias=bias)
    f64 = lambda a: np.asarray(a, np.float64)
    y64 = oracle.selective_forward_bld(f64(u), f64(dt_pre), f64(A), f64(Bg), f64(Cg), gate=f64(z),
                                       dt_bias=f64(bias))
    scale = max(1.0, float(np.abs(y64).max()))
    assert_parity(y, y32, y64, rtol=1e-4, atol=1e-5 * scale, what=f"scan {shape}")
    no_device_errors()


def _scan_ref64(u, dt_pre, bias, A, Bg, Cg, z):
    """fp64 autograd reference of the gated scan with softplus'd dt (loop)."""
    dt = F.softplus(dt_pre + bias)
    h = torch.zeros(u.shape[0], u.shape[2], A.shape[1], dtype=u.dtype)
    ys = []
    for t in range(u.shape[1]):
        d = dt[:, t, :, None]
        h = torch.exp(d * A) * h + (d * Bg[:, t, None, :]) * u[:, t, :, None]
        ys.append((h * Cg[:, t, None, :]).sum(-1))
    return torch.stack(ys, 1) * F.silu(z)


@pytest.mark.parametrize("shape", [(2, 70, 20, 5, 2), (1, 45, 36, 17, 3)],
                         ids=lambda s: "x".join(map(str, s)))
def test_scan_bld_backward_matches_fp64_autograd(M, shape):
    nb, L, D, N, R = shape
    announce(f"mamba scan bwd B={nb} L={L} D={D} N={N}")
    u, xz, dt_pre, bias, A, proj = _scan_inputs(nb, L, D, N, R, 5)
    go = np.random.default_rng(6).normal(size=(nb, L, D)).astype(np.float32)
    leaves, args = _views(M, u, xz, dt_pre, bias, A, proj, D, N, R, grad=True)
    y = M.selective_scan_mamba(*args[:5], gate=args[5], dt_bias=args[6])
    y.backward(to_dev(go))
    refs = {}
    for dt_ in (torch.float32, torch.float64):
        Lr = [torch.tensor(v, dtype=dt_, requires_grad=True) for v in (u, xz, dt_pre, bias, A, proj)]
        ref = _scan_ref64(Lr[0], Lr[2], Lr[3], Lr[4], Lr[5][..., R:R + N], Lr[5][..., R + N:],
                          Lr[1][..., D:])
        ref.backward(torch.tensor(go, dtype=dt_))
        refs[dt_] = [r.grad.numpy() for r in Lr]
    for t, a, b, n in zip(leaves, refs[torch.float32], refs[torch.float64],
                          ["u", "xz", "dt_pre", "dt_bias", "A", "proj"]):
        assert_grad_parity(to_np(t.grad), a, b, f"{shape} grad {n}")
    no_device_errors()


def test_scan_bld_agrees_with_bdl_dropin(M):
    """At C4's channel count the [B,L,D] scan and the drop-in [B,D,L] scan on
    transposed copies compute the same arithmetic: outputs and every gradient
    agree to rounding (ddt through the softplus: times sigmoid(dt_pre + bias))."""
    from ossm_amd import _kernels as K

    nb, L, D, N, R = 2, 300, 1536, 16, 4
    announce(f"mamba scan vs drop-in B={nb} L={L} D={D} N={N}")
    u, xz, dt_pre, bias, A, proj = _scan_inputs(nb, L, D, N, R, 8)
    go = np.random.default_rng(9).normal(size=(nb, L, D)).astype(np.float32)
    leaves, args = _views(M, u, xz, dt_pre, bias, A, proj, D, N, R, grad=True)
    y = M.selective_scan_mamba(*args[:5], gate=args[5], dt_bias=args[6])
    y.backward(to_dev(go))
    T = lambda a: to_dev(np.ascontiguousarray(np.asarray(a).transpose(0, 2, 1)))
    dt_sp = torch.nn.functional.softplus(to_dev(dt_pre) + to_dev(bias))
    uT, dtT, zT = T(u), dt_sp.transpose(1, 2).contiguous(), T(xz[..., D:])
    Bg, Cg = to_dev(np.ascontiguousarray(proj[..., R:R + N])), to_dev(np.ascontiguousarray(proj[..., R + N:]))
    out, ck, raw = K.selective_scan_cuda(uT, dtT, to_dev(A), Bg, Cg, zT)
    np.testing.assert_allclose(to_np(y), to_np(out.transpose(1, 2)), rtol=1e-5, atol=1e-5)
    du, ddt, dA, dB, dC, dz = K.selective_scan_cuda_backward(T(go), uT, dtT, to_dev(A), Bg, Cg, zT,
                                                             ck, raw, 16)
    sig = torch.sigmoid(to_dev(dt_pre) + to_dev(bias))
    pairs = ((leaves[0].grad, du.transpose(1, 2), "du", False),
             (leaves[2].grad, ddt.transpose(1, 2) * sig, "ddt", False),
             (leaves[4].grad, dA, "dA", True),
             (leaves[5].grad[..., R:R + N], dB, "dB", True),
             (leaves[5].grad[..., R + N:], dC, "dC", True),
             (leaves[1].grad[..., D:], dz.transpose(1, 2), "dz", False))
    for got, ref, n, is_sum in pairs:
        ref = to_np(ref)
        np.testing.assert_allclose(to_np(got), ref, rtol=1e-4,
                                   atol=sum_atol(ref) if is_sum else 1e-5, err_msg=n)
    no_device_errors()


def test_mixer_matches_brute_fp64(M):
    """The whole mixer (MambaMixer) forward and backward against the
    brute-force fp64 mixer on the CPU with the same parameters."""
    announce("mamba mixer vs brute fp64")
    torch.manual_seed(0)
    mixer = M.MambaMixer(24, d_state=8, d_conv=4, expand=2).cuda()
    with torch.no_grad():
        mixer.dt_proj.bias.uniform_(-4.0, -2.0)
    u = torch.randn(2, 60, 24, device="cuda", requires_grad=True)
    y = mixer(u)
    go = torch.randn_like(y)
    y.backward(go)
    refs = {}
    for dt_ in (torch.float32, torch.float64):
        params = {k: v.detach().to(dt_).cpu().requires_grad_(True)
                  for k, v in mixer.state_dict().items()}
        ur = u.detach().to(dt_).cpu().requires_grad_(True)
        out = _brute.mamba_mixer(ur, params, mixer.d_conv, mixer.dt_rank, mixer.d_state)
        out.backward(go.to(dt_).cpu())
        refs[dt_] = (out.detach().numpy(), ur.grad.numpy(),
                     {k: p.grad.numpy() for k, p in params.items()})
    (y32, gu32, gp32), (y64, gu64, gp64) = refs[torch.float32], refs[torch.float64]
    assert_parity(to_np(y), y32, y64, rtol=1e-4, atol=1e-5 * max(1.0, float(np.abs(y64).max())),
                  what="mixer out")
    assert_grad_parity(to_np(u.grad), gu32, gu64, "mixer grad inputs")
    named = dict(mixer.named_parameters())
    for k in gp64:
        assert_grad_parity(to_np(named[k].grad), gp32[k], gp64[k], f"mixer grad {k}")
    no_device_errors()


def test_mamba_edge_cases_and_errors(M):
    announce("mamba edge cases")
    x = torch.randn(2, 5, 8, device="cuda")
    with pytest.raises(RuntimeError, match="kernel width"):
        M.mamba_conv_silu(x, torch.randn(8, 1, 9, device="cuda"))
    with pytest.raises(RuntimeError, match="float32 GPU"):
        M.mamba_conv_silu(x.double(), torch.randn(8, 1, 4, device="cuda", dtype=torch.float64))
    # no bias, no gate, no dt bias
    y = M.mamba_conv_silu(x, torch.randn(8, 1, 4, device="cuda"))
    assert y.shape == x.shape and torch.isfinite(y).all()
    A = -torch.rand(8, 3, device="cuda") - 0.5
    Bm, Cm = torch.randn(2, 5, 3, device="cuda"), torch.randn(2, 5, 3, device="cuda")
    out = M.selective_scan_mamba(x, torch.randn(2, 5, 8, device="cuda"), A, Bm, Cm)
    assert out.shape == x.shape and torch.isfinite(out).all()
    with pytest.raises(RuntimeError, match="inconsistent shapes"):
        M.selective_scan_mamba(x, torch.randn(2, 5, 7, device="cuda"), A, Bm, Cm)
    # parameters of another dtype are rejected, not reinterpreted
    with pytest.raises(RuntimeError, match="conv weight must be a float32 GPU tensor"):
        M.mamba_conv_silu(x, torch.randn(8, 1, 4, device="cuda", dtype=torch.float64))
    with pytest.raises(RuntimeError, match="A must be a float32 GPU tensor"):
        M.selective_scan_mamba(x, torch.randn(2, 5, 8, device="cuda"), A.double(), Bm, Cm)
    # empty sequence
    e = torch.zeros(2, 0, 8, device="cuda")
    assert M.mamba_conv_silu(e, torch.randn(8, 1, 4, device="cuda")).shape == e.shape
    no_device_errors()
