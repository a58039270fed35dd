"""GPU parity of the fused D-LinOSS layer (ossm_dlinoss_layer_forward through
ossm_amd.layers) against the CPU oracle's layer forward, the reference's
layer fixture, and fp64 gradients built from the oracle's adjoint.

Tolerance: rtol 1e-4 / atol 1e-5 scaled by the output's magnitude against the
fp32 oracle (the products and sums of both projections are fp32 on the matrix
cores, in another order than the oracle's BLAS), with the fp64 oracle as the
arbiter where an fp32 recurrence's own rounding dominates (assert_parity).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import (announce, assert_grad_parity, assert_parity, dlinoss_inputs, need_gpu,
                            no_device_errors, rel_fro, sum_atol, to_dev, to_np)

pytestmark = pytest.mark.gpu
VARIANTS = oracle.VARIANTS
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def layers():
    need_gpu()
    from ossm_amd import layers as m

    return m


def _layer_inputs(nb, L, H, P, seed, variant):
    rng = np.random.default_rng(seed)
    a, g, dt, _, _ = dlinoss_inputs(1, 1, P, seed, variant=variant)
    u = rng.normal(size=(nb, L, H)).astype(np.float32)
    Bw = rng.uniform(-1, 1, size=(P, H, 2)).astype(np.float32) / np.float32(np.sqrt(max(H, 1)))
    Cw = rng.uniform(-1, 1, size=(H, P, 2)).astype(np.float32) / np.float32(np.sqrt(max(P, 1)))
    Dw = rng.normal(size=H).astype(np.float32)
    return u, Bw, Cw, Dw, a, g, dt


def _oracle(variant, args, dtype):
    return oracle.dlinoss_layer_forward(variant, *(np.asarray(x, dtype) for x in args))


def _run(layers, variant, args):
    return layers.dlinoss_layer_forward(variant, *(to_dev(x) for x in args))


def _check(layers, variant, args, what):
    y = to_np(_run(layers, variant, args))
    y32, _ = _oracle(variant, args, np.float32)
    y64, _ = _oracle(variant, args, np.float64)
    scale = max(1.0, float(np.abs(y64).max()))
    assert_parity(y, y32, y64, rtol=1e-4, atol=1e-5 * scale, what=what)
    no_device_errors()


# H, P <= 128 run the four-workgroups-per-CU instantiation, larger ones the other
# (two oscillator groups per wave when P > 128); H % 4 or P % 4 != 0 take the scalar loads
SHAPES = [(1, 1, 1, 1), (2, 6, 3, 4), (2, 33, 8, 12), (3, 100, 16, 32), (2, 257, 64, 96),
          (1, 1030, 128, 128), (2, 64, 130, 33), (3, 40, 256, 256), (5, 97, 32, 64),
          (2, 50, 128, 124), (2, 70, 64, 160), (3, 45, 100, 129)]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_layer_matches_oracle(layers, variant, shape):
    nb, L, H, P = shape
    announce(f"layer {variant} B={nb} L={L} H={H} P={P}")
    _check(layers, variant, _layer_inputs(nb, L, H, P, 11, variant), f"{variant} {shape}")


def test_layer_config2_size(layers):
    """BASELINE config 2's shape (B=32, L=4096, H=P=128), imex1: 128 chunks per
    batch row through the look-back."""
    announce("layer imex1 B=32 L=4096 H=128 P=128")
    _check(layers, "imex1", _layer_inputs(32, 4096, 128, 128, 2, "imex1"), "config 2")


@pytest.mark.parametrize("variant", VARIANTS)
def test_layer_module_matches_reference_fixture(layers, variant):
    """The reference's layer fixture run through DampedLinOSSLayer on the GPU,
    parameters loaded as the reference test does (test_dlinoss_parity.py:94-103)."""
    announce(f"layer module fixture {variant}")
    c = json.loads((GOLDEN / "dlinoss_reference_cases.json").read_text())["cases"][variant]["float32"]
    layer = layers.DampedLinOSSLayer(int(c["ssm_size"]), int(c["hidden_dim"]), variant=variant).cuda()
    with torch.no_grad():
        layer.A_diag.copy_(torch.tensor(c["A_diag"]))
        layer.G_diag.copy_(torch.tensor(c["G_diag"]))
        layer.steps.copy_(torch.logit(torch.tensor(c["step"]).clamp(1e-6, 1 - 1e-6)))
        layer.B.copy_(torch.tensor(c["B"]))
        layer.C.copy_(torch.tensor(c["C"]))
        layer.D.copy_(torch.tensor(c["D"]))
    with torch.no_grad():
        y = layer(torch.tensor(c["inputs"], dtype=torch.float32).cuda())
    np.testing.assert_allclose(to_np(y), np.asarray(c["outputs"]), rtol=2e-5, atol=2e-5)


def _oracle_grads(variant, args, gy, dtype=np.float64):
    """Gradients of sum(y * gy) w.r.t. (u, B, C, D, a, g, dt) from the
    oracle's forward and adjoint, in `dtype` (fp64: truth; fp32: the
    reference's arithmetic): g_x = gy (C_re - i C_im) (complex gradient as
    d/dre + i d/dim), the scan adjoint gives grad_bu and (a, g, dt), then the
    two projections' transposes."""
    u, Bw, Cw, Dw, a, g, dt = (np.asarray(x, dtype) for x in args)
    gy = np.asarray(gy, dtype)
    ct = np.complex128 if dtype == np.float64 else np.complex64
    nb, L, H = u.shape
    P = Bw.shape[0]
    y, states = oracle.dlinoss_layer_forward(variant, u, Bw, Cw, Dw, a, g, dt)
    bu = np.einsum("blh,ph->lbp", u, (Bw[..., 0] + 1j * Bw[..., 1]).astype(ct)).astype(ct)
    x = states[..., 1].transpose(1, 0, 2)  # [B, L, P]
    gx = np.einsum("blh,hp->blp", gy, (Cw[..., 0] - 1j * Cw[..., 1]).astype(ct)).astype(ct)
    ga, gg, gs, gbu = oracle.dlinoss_backward(variant, a, g, dt, np.ascontiguousarray(bu), states,
                                              np.ascontiguousarray(gx.transpose(1, 0, 2)))
    gbu = gbu.transpose(1, 0, 2)  # [B, L, P]
    gu = np.einsum("blp,ph->blh", gbu.real, Bw[..., 0]) + np.einsum("blp,ph->blh", gbu.imag, Bw[..., 1]) + gy * Dw
    gB = np.stack([np.einsum("blp,blh->ph", gbu.real, u), np.einsum("blp,blh->ph", gbu.imag, u)], -1)
    gC = np.stack([np.einsum("blh,blp->hp", gy, x.real), -np.einsum("blh,blp->hp", gy, x.imag)], -1)
    gD = (gy * u).sum((0, 1))
    return [gu, gB, gC, gD, ga, gg, gs]


LEAVES = ["inputs", "B", "C", "D", "a_diag", "g_diag", "step"]


def _check_grads(got, args, gy, variant, what):
    """Every gradient elementwise against the fp32 oracle, fp64 as arbiter."""
    r32 = _oracle_grads(variant, args, gy, np.float32)
    r64 = _oracle_grads(variant, args, gy, np.float64)
    for t, a, b, n in zip(got, r32, r64, LEAVES):
        assert_grad_parity(to_np(t), a, b, f"{what} grad {n}")


@pytest.mark.parametrize("variant", VARIANTS)
def test_layer_gradients(layers, variant):
    """Backward of the fused layer (recomputation through the unfused
    composition) against fp64 gradients from the oracle's adjoint."""
    nb, L, H, P = 2, 150, 24, 40
    announce(f"layer grads {variant} B={nb} L={L} H={H} P={P}")
    args = _layer_inputs(nb, L, H, P, 4, variant)
    gy = np.random.default_rng(9).normal(size=(nb, L, H)).astype(np.float32)
    leaves = [to_dev(x).requires_grad_(True) for x in args]
    y = layers.DlinossLayerFn.apply(variant, *leaves)
    y.backward(to_dev(gy))
    _check_grads([t.grad for t in leaves], args, gy, variant, variant)
    no_device_errors()


def test_layer_module_fused_and_unfused_agree(layers):
    """DampedLinOSSLayer forward and backward equal the unfused composition.
    imex1: the ring initialisation places the eigenvalues of imex1's transition
    on the ring (other variants can grow under it and overflow over long rows)."""
    announce("layer module fused vs unfused")
    torch.manual_seed(3)
    layer = layers.DampedLinOSSLayer(48, 20, variant="imex1").cuda()
    u = torch.randn(3, 77, 20, device="cuda", requires_grad=True)
    y = layer(u)
    (y * y).sum().backward()
    g_fused = [p.grad.clone() for p in layer.parameters()] + [u.grad.clone()]
    layer.zero_grad()
    u2 = u.detach().clone().requires_grad_(True)
    a, g, dt = layers.project_parameters(layer.A_diag, layer.G_diag, layer.steps)
    y2 = layers.unfused_layer_forward("imex1", u2, layer.B, layer.C, layer.D, a, g, dt)
    (y2 * y2).sum().backward()
    g_unfused = [p.grad.clone() for p in layer.parameters()] + [u2.grad.clone()]
    yr = to_np(y2)
    np.testing.assert_allclose(to_np(y), yr, rtol=1e-4, atol=1e-5 * max(1.0, float(np.abs(yr).max())))
    for a_, b_ in zip(g_fused, g_unfused):
        ref = to_np(b_)
        np.testing.assert_allclose(to_np(a_), ref, rtol=1e-4, atol=sum_atol(ref))
    no_device_errors()


def test_layer_bf16_input_computes_in_fp32(layers):
    announce("layer module bf16 input")
    torch.manual_seed(1)
    layer = layers.DampedLinOSSLayer(16, 8).cuda()
    u = torch.randn(2, 30, 8, device="cuda")
    y32 = layer(u)
    y16 = layer(u.bfloat16())
    assert y16.dtype == torch.bfloat16
    ref = layer(u.bfloat16().float())
    np.testing.assert_allclose(to_np(y16.float()), to_np(ref.bfloat16().float()), rtol=0, atol=0)
    assert rel_fro(to_np(y32), to_np(ref)) < 1e-2


def test_layer_edge_cases_and_errors(layers):
    announce("layer edge cases")
    v = "imex1"
    # L = 0 and B = 0: empty outputs
    for shape in ((2, 0, 4), (0, 5, 4)):
        u = torch.zeros(shape, device="cuda")
        args = [torch.zeros(3, 4, 2, device="cuda"), torch.zeros(4, 3, 2, device="cuda"),
                torch.zeros(4, device="cuda")] + [torch.full((3,), 0.5, device="cuda")] * 3
        assert layers.dlinoss_layer_forward(v, u, *args).shape == shape
    # P = 0: the layer is the D skip
    u = torch.randn(2, 9, 4, device="cuda")
    D = torch.randn(4, device="cuda")
    z = torch.zeros(0, device="cuda")
    y = layers.dlinoss_layer_forward(v, u, torch.zeros(0, 4, 2, device="cuda"),
                                     torch.zeros(4, 0, 2, device="cuda"), D, z, z, z)
    np.testing.assert_allclose(to_np(y), to_np(u * D), rtol=1e-6, atol=1e-6)
    # limits and checks
    big = torch.zeros(1, 2, 257, device="cuda")
    with pytest.raises(RuntimeError, match="up to 256"):
        layers.dlinoss_layer_forward(v, big, torch.zeros(2, 257, 2, device="cuda"),
                                     torch.zeros(257, 2, 2, device="cuda"),
                                     torch.zeros(257, device="cuda"), *[torch.zeros(2, device="cuda")] * 3)
    with pytest.raises(RuntimeError, match="C must have shape"):
        layers.dlinoss_layer_forward(v, u, torch.zeros(3, 4, 2, device="cuda"),
                                     torch.zeros(3, 4, 2, device="cuda"), D,
                                     *[torch.zeros(3, device="cuda")] * 3)
    with pytest.raises(RuntimeError, match="float32"):
        layers.dlinoss_layer_forward(v, u.double(), torch.zeros(3, 4, 2, device="cuda"),
                                     torch.zeros(4, 3, 2, device="cuda"), D,
                                     *[torch.zeros(3, device="cuda")] * 3)
    with pytest.raises(ValueError, match="Unknown D-LinOSS variant"):
        layers.dlinoss_layer_forward("rk4", u, torch.zeros(3, 4, 2, device="cuda"),
                                     torch.zeros(4, 3, 2, device="cuda"), D,
                                     *[torch.zeros(3, device="cuda")] * 3)
    # a module wider than the fused kernel runs the unfused composition
    wide = layers.DampedLinOSSLayer(300, 8).cuda()
    uw = torch.randn(1, 20, 8, device="cuda")
    a, g, dt = layers.project_parameters(wide.A_diag, wide.G_diag, wide.steps)
    ref = layers.unfused_layer_forward("imex1", uw, wide.B, wide.C, wide.D, a, g, dt)
    np.testing.assert_allclose(to_np(wide(uw)), to_np(ref), rtol=0, atol=0)
    no_device_errors()


def test_layer_repeatable(layers):
    """Two launches give the same bits up to the look-back's association of
    carries (only the chunk carries may regroup; bounded by 1e-6 of |y|)."""
    announce("layer repeatable")
    args = [to_dev(x) for x in _layer_inputs(4, 2000, 64, 64, 7, "im")]
    y1 = to_np(layers.dlinoss_layer_forward("im", *args))
    y2 = to_np(layers.dlinoss_layer_forward("im", *args))
    assert np.abs(y1 - y2).max() <= 1e-6 * max(1.0, np.abs(y1).max())


@pytest.mark.parametrize("shape", [(2, 70, 13, 9), (3, 33, 40, 4), (1, 1, 8, 8)],
                         ids=lambda s: "x".join(map(str, s)))
def test_layer_fused_backward_odd_sizes(layers, shape):
    """The fused backward on sizes that take the unaligned paths (H, P not
    multiples of 4, one-step rows) against fp64 oracle gradients."""
    nb, L, H, P = shape
    announce(f"layer fused bwd odd B={nb} L={L} H={H} P={P}")
    args = _layer_inputs(nb, L, H, P, 12, "im")
    gy = np.random.default_rng(13).normal(size=(nb, L, H)).astype(np.float32)
    leaves = [to_dev(x).requires_grad_(True) for x in args]
    y = layers.DlinossLayerFn.apply("im", *leaves)
    y.backward(to_dev(gy))
    _check_grads([t.grad for t in leaves], args, gy, "im", f"{shape}")
    no_device_errors()


@pytest.mark.parametrize("variant", VARIANTS)
def test_layer_fused_backward_matches_unfused_at_size(layers, variant):
    """At H = P = 128 over 1000 steps (32 chunks through the reverse look-back)
    the fused backward's gradients and the unfused composition's, each
    elementwise against the fp32 oracle with fp64 truth as arbiter."""
    nb, L, H, P = 4, 1000, 128, 128
    announce(f"layer fused vs unfused bwd {variant} B={nb} L={L}")
    host = _layer_inputs(nb, L, H, P, 21, variant)
    args = [to_dev(x) for x in host]
    gy_h = np.random.default_rng(22).normal(size=(nb, L, H)).astype(np.float32)
    gy = to_dev(gy_h)
    l1 = [t.clone().requires_grad_(True) for t in args]
    layers.DlinossLayerFn.apply(variant, *l1).backward(gy)
    l2 = [t.clone().requires_grad_(True) for t in args]
    layers.unfused_layer_forward(variant, *l2).backward(gy)
    _check_grads([t.grad for t in l1], host, gy_h, variant, f"{variant} fused")
    _check_grads([t.grad for t in l2], host, gy_h, variant, f"{variant} unfused")
    no_device_errors()


def test_layer_fused_backward_at_256(layers):
    """H = P = 256, the largest fused size: two oscillator groups per wave in
    the bu projection (bu held in the accumulators until u is read) and the
    fused backward's LDS at its largest, against fp64 oracle gradients."""
    nb, L, H, P = 2, 70, 256, 256
    announce("layer fused backward H=P=256")
    assert layers._bwd_fits(H, P)
    args = _layer_inputs(nb, L, H, P, 31, "imex1")
    gy = np.random.default_rng(32).normal(size=(nb, L, H)).astype(np.float32)
    leaves = [to_dev(x).requires_grad_(True) for x in args]
    layers.DlinossLayerFn.apply("imex1", *leaves).backward(to_dev(gy))
    _check_grads([t.grad for t in leaves], args, gy, "imex1", "H=P=256")
    no_device_errors()


def test_layer_backward_recompute_path(layers, monkeypatch):
    """The recomputing backward (through the unfused composition), taken when
    the fused backward's LDS would not fit, forced here at a small size."""
    nb, L, H, P = 1, 40, 48, 40
    announce("layer backward recompute path")
    monkeypatch.setattr(layers, "_bwd_fits", lambda hidden, ssm: False)
    args = _layer_inputs(nb, L, H, P, 33, "imex1")
    gy = np.random.default_rng(34).normal(size=(nb, L, H)).astype(np.float32)
    leaves = [to_dev(x).requires_grad_(True) for x in args]
    layers.DlinossLayerFn.apply("imex1", *leaves).backward(to_dev(gy))
    _check_grads([t.grad for t in leaves], args, gy, "imex1", "recompute path")
    no_device_errors()
