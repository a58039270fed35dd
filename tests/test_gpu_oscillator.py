"""GPU parity of the D-LinOSS and LinOSS scans (through the drop-in module,
i.e. the C ABI) against the CPU oracle and the reference's kernel vectors.

Tolerance (north star): rtol 1e-4 / atol 1e-5 in fp32/complex64 against the
reference CPU kernel.  Parameter gradients are sums over B*L terms; the
reference accumulates them in one fp32 scalar, so they are compared with an
atol scaled by the gradient's magnitude and checked against fp64 truth.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import (announce, assert_close, assert_parity, dlinoss_inputs, need_gpu,
                            no_device_errors, rel_fro, to_dev, to_np)

pytestmark = pytest.mark.gpu
VARIANTS = oracle.VARIANTS
GOLDEN = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def _fwd(K, v, a, g, dt, bu):
    return getattr(K, f"dlinoss_{v}_forward")(to_dev(a), to_dev(g), to_dev(dt), to_dev(bu))


def _bwd(K, v, a, g, dt, bu, states, go):
    return getattr(K, f"dlinoss_{v}_backward")(to_dev(a), to_dev(g), to_dev(dt), to_dev(bu),
                                               states, to_dev(go))


def _param_atol(ref: np.ndarray) -> float:
    return 2e-5 * max(1.0, float(np.abs(ref).max()))


@pytest.mark.parametrize("variant", VARIANTS)
def test_dlinoss_matches_reference_kernel_vectors(K, variant):
    """GPU vs the outputs the reference's own CPU kernels produced (fixture)."""
    with np.load(GOLDEN / "ref_kernel_vectors.npz") as z:
        v = {k: z[k] for k in z.files}
    announce(f"dlinoss golden {variant} L=53 B=3 P=7")
    st = _fwd(K, variant, v["dl_a"], v["dl_g"], v["dl_step"], v["dl_bu"])
    assert_close(to_np(st), v[f"dl_{variant}_states"], RTOL, ATOL, "states")
    ga, gg, gs, gb = _bwd(K, variant, v["dl_a"], v["dl_g"], v["dl_step"], v["dl_bu"],
                          to_dev(v[f"dl_{variant}_states"]), v["dl_grad"])
    assert_close(to_np(gb), v[f"dl_{variant}_grad_bu"], RTOL, ATOL, "grad_bu")
    for got, key in ((ga, "grad_a"), (gg, "grad_g"), (gs, "grad_step")):
        ref = v[f"dl_{variant}_{key}"]
        assert_close(to_np(got), ref, RTOL, _param_atol(ref), key)
    no_device_errors()


# shapes: tiny, ragged (P and B*P not multiples of 64), many chunks / groups;
# (1000, 32, 64) is the smallest grid (128 workgroups) on which the forward
# takes its 256-step tile (16 steps x 16 waves), with a partial last chunk
SHAPES = [(1, 1, 1), (2, 3, 5), (129, 2, 33), (1000, 3, 70), (2100, 4, 64), (1000, 32, 64)]


def _oracle64(variant, a, g, dt, bu, go):
    a64, g64, d64 = (x.astype(np.float64) for x in (a, g, dt))
    b64, go64 = bu.astype(np.complex128), go.astype(np.complex128)
    st = oracle.dlinoss_forward(variant, a64, g64, d64, b64)
    return st, oracle.dlinoss_backward(variant, a64, g64, d64, b64, st, go64)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_dlinoss_forward_backward_vs_oracle(K, variant, shape):
    L, B, P = shape
    a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=L + 7 * B + 13 * P, variant=variant)
    announce(f"dlinoss {variant} L={L} B={B} P={P}")
    st = _fwd(K, variant, a, g, dt, bu)
    ga, gg, gs, gb = _bwd(K, variant, a, g, dt, bu, st, go)
    ref = oracle.dlinoss_forward(variant, a, g, dt, bu)
    rga, rgg, rgs, rgb = oracle.dlinoss_backward(variant, a, g, dt, bu, ref, go)
    st64, (tga, tgg, tgs, tgb) = _oracle64(variant, a, g, dt, bu, go)
    assert_parity(to_np(st), ref, st64, RTOL, ATOL, "states")
    assert_parity(to_np(gb), rgb, tgb, RTOL, ATOL, "grad_bu")
    # parameter gradients are sums over B*L terms: atol scaled by their size
    for got, r32, r64, key in ((ga, rga, tga, "grad_a"), (gg, rgg, tgg, "grad_g"),
                               (gs, rgs, tgs, "grad_step")):
        assert_parity(to_np(got), r32, r64, RTOL, _param_atol(r64), key)
    no_device_errors()


def test_dlinoss_zero_length_and_empty(K):
    a, g, dt, bu, go = dlinoss_inputs(4, 2, 3, seed=1)
    st = K.dlinoss_imex1_forward(to_dev(a), to_dev(g), to_dev(dt), to_dev(bu[:0]))
    assert tuple(st.shape) == (0, 2, 3, 2)
    grads = K.dlinoss_imex1_backward(to_dev(a), to_dev(g), to_dev(dt), to_dev(bu[:0]),
                                     torch.empty((0, 2, 3, 2), dtype=torch.complex64, device="cuda"),
                                     to_dev(go[:0]))
    assert all(float(t.abs().sum()) == 0 for t in grads[:3])


def test_dlinoss_rejects_bad_inputs(K):
    a, g, dt, bu, _ = dlinoss_inputs(8, 2, 3, seed=2)
    with pytest.raises(RuntimeError, match="bu must have shape"):
        K.dlinoss_imex1_forward(to_dev(a), to_dev(g), to_dev(dt), to_dev(bu[0]))
    with pytest.raises(RuntimeError, match="match state size"):
        K.dlinoss_imex1_forward(to_dev(a[:2]), to_dev(g), to_dev(dt), to_dev(bu))
    with pytest.raises(RuntimeError, match="bu must be contiguous"):
        K.dlinoss_imex1_forward(to_dev(a), to_dev(g), to_dev(dt), to_dev(bu).transpose(0, 1))


# complex128: the reference dispatcher's other complex type (AT_DISPATCH_COMPLEX_TYPES,
# dlinoss_imex1_cuda.cu:196, 234), coefficients float64
F64_SHAPES = [(1, 1, 1), (2, 3, 5), (129, 2, 33), (1000, 3, 70), (300, 5, 130)]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("shape", F64_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_dlinoss_complex128_vs_fp64_oracle(K, variant, shape):
    """complex128 forward and backward against the oracle's fp64 restatement
    of the reference kernels, elementwise at rtol 1e-10 (parameter gradients
    with atol 1e-10 x their magnitude: sums over B*L terms)."""
    L, B, P = shape
    a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=3 * L + B + 5 * P, variant=variant)
    a, g, dt = (x.astype(np.float64) for x in (a, g, dt))
    rng = np.random.default_rng(L + B + P)
    bu = bu.astype(np.complex128) + 1e-3 * rng.normal(size=bu.shape)  # beyond fp32's values
    go = go.astype(np.complex128)
    announce(f"dlinoss complex128 {variant} L={L} B={B} P={P}")
    st = _fwd(K, variant, a, g, dt, bu)
    assert st.dtype == torch.complex128
    ga, gg, gs, gb = _bwd(K, variant, a, g, dt, bu, st, go)
    assert ga.dtype == torch.float64 and gb.dtype == torch.complex128
    ref = oracle.dlinoss_forward(variant, a, g, dt, bu)
    rga, rgg, rgs, rgb = oracle.dlinoss_backward(variant, a, g, dt, bu, ref, go)
    np.testing.assert_allclose(to_np(st), ref, rtol=1e-10, atol=1e-12, err_msg="states")
    np.testing.assert_allclose(to_np(gb), rgb, rtol=1e-10, atol=1e-12, err_msg="grad_bu")
    for got, r, key in ((ga, rga, "grad_a"), (gg, rgg, "grad_g"), (gs, rgs, "grad_step")):
        np.testing.assert_allclose(to_np(got), r, rtol=1e-10,
                                   atol=1e-10 * max(1.0, float(np.abs(r).max())), err_msg=key)
    no_device_errors()


def test_dlinoss_complex128_dtype_rules(K):
    """The reference's data_ptr<value_t> rules: complex128 bu needs float64
    coefficients and complex128 states / grad_output; other bu types are not
    dispatched; L = 0 gives zero float64 gradients."""
    a, g, dt, bu, go = dlinoss_inputs(6, 2, 3, seed=4)
    a64, g64, d64 = (to_dev(x.astype(np.float64)) for x in (a, g, dt))
    bu64 = to_dev(bu.astype(np.complex128))
    with pytest.raises(RuntimeError, match="expected scalar type Double but found Float"):
        K.dlinoss_imex1_forward(to_dev(a), g64, d64, bu64)
    with pytest.raises(RuntimeError, match="expected scalar type Float but found Double"):
        K.dlinoss_imex1_forward(a64, g64, d64, to_dev(bu))
    with pytest.raises(RuntimeError, match="not implemented for 'Float'"):
        K.dlinoss_imex1_forward(a64, g64, d64, to_dev(bu.real.copy()))
    st = K.dlinoss_imex1_forward(a64, g64, d64, bu64)
    with pytest.raises(RuntimeError, match="expected scalar type ComplexDouble but found ComplexFloat"):
        K.dlinoss_imex1_backward(a64, g64, d64, bu64, st, to_dev(go))
    grads = K.dlinoss_imex1_backward(a64, g64, d64, bu64[:0], st[:0], to_dev(go.astype(np.complex128))[:0])
    assert all(t.dtype == torch.float64 and float(t.abs().sum()) == 0 for t in grads[:3])


@pytest.mark.parametrize("variant", ["imex1", "im"])
def test_dlinoss_config2_full_size(K, variant):
    """BASELINE config 2 shape (B=32, L=4096, P=128): every channel of a slice
    of oscillators checked against the oracle at full length, plus linearity
    of the whole scan."""
    L, B, P = 4096, 32, 128
    a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=2024, variant=variant)
    announce(f"dlinoss {variant} full config2")
    st = _fwd(K, variant, a, g, dt, bu)
    gp = _bwd(K, variant, a, g, dt, bu, st, go)
    # channel slice: batches 0, 17, 31 and every oscillator
    bs = [0, 17, 31]
    bus, gos = np.ascontiguousarray(bu[:, bs]), np.ascontiguousarray(go[:, bs])
    ref = oracle.dlinoss_forward(variant, a, g, dt, bus)
    _, _, _, rgb = oracle.dlinoss_backward(variant, a, g, dt, bus, ref, gos)
    st64, (_, _, _, tgb) = _oracle64(variant, a, g, dt, bus, gos)
    assert_parity(to_np(st[:, bs]), ref, st64, RTOL, ATOL, "states slice")
    assert_parity(to_np(gp[3][:, bs]), rgb, tgb, RTOL, ATOL, "grad_bu slice")
    # whole-problem parameter gradients vs the oracle on all channels: relative
    # norm, and elementwise (atol scaled by the sums' size, fp64 fallback)
    full = oracle.dlinoss_forward(variant, a, g, dt, bu)
    rg = oracle.dlinoss_backward(variant, a, g, dt, bu, full, go)
    _, tg = _oracle64(variant, a, g, dt, bu, go)
    for got, r, t, key in zip(gp[:3], rg[:3], tg[:3], ("grad_a", "grad_g", "grad_step")):
        assert rel_fro(to_np(got), r) < 1e-4, key
        assert_parity(to_np(got), r, t, RTOL, _param_atol(t), key)
    # linearity: scan(bu + 2 bu') = scan(bu) + 2 scan(bu')
    bu2 = torch.roll(to_dev(bu), shifts=1, dims=1)
    s2 = _fwd(K, variant, a, g, dt, to_np(bu2))
    s12 = _fwd(K, variant, a, g, dt, to_np(to_dev(bu) + 2 * bu2))
    assert rel_fro(to_np(s12), to_np(st + 2 * s2)) < 1e-5
    no_device_errors()


def test_dlinoss_config5_long_sequence(K):
    """BASELINE config 5 (B=4, L=65536, P=256, forward only): cross-workgroup
    carries over 256 chunks of 256 steps; checked per channel against the oracle and
    against fp64 truth."""
    L, B, P = 65536, 4, 256
    a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=5)
    announce("dlinoss imex1 full config5")
    st = to_np(_fwd(K, "imex1", a, g, dt, bu))
    ref32 = oracle.dlinoss_forward("imex1", a, g, dt, bu)
    ref64 = oracle.dlinoss_forward("imex1", a.astype(np.float64), g.astype(np.float64),
                                   dt.astype(np.float64), bu.astype(np.complex128))
    e_gpu = rel_fro(st, ref64)
    e_cpu = rel_fro(ref32, ref64)
    assert e_gpu <= 4 * e_cpu + 1e-6, (e_gpu, e_cpu)
    assert rel_fro(st, ref32) < 1e-4
    # elementwise on channel slices: batch row 1 (every oscillator, all 65536
    # steps, so every one of the 512 chunk carries of 256 channels) and every
    # 8th oscillator of the other rows
    assert_parity(st[:, 1], ref32[:, 1], ref64[:, 1], RTOL, ATOL, "states row 1")
    for b in (0, 2, 3):
        assert_parity(st[:, b, ::8], ref32[:, b, ::8], ref64[:, b, ::8], RTOL, ATOL,
                      f"states row {b}, every 8th oscillator")
    no_device_errors()


# ------------------------------------------------------------------- LinOSS
def _linoss_inputs(L, B, P, seed):
    rng = np.random.default_rng(seed)
    # LinOSS-IM transition of linoss.py:244-251 with a ~ U(0, 1), dt = sigmoid(N)
    a = rng.uniform(0.0, 1.0, P)
    dt = 1 / (1 + np.exp(-rng.normal(size=P)))
    schur = 1 / (1 + dt * dt * a)
    ms = [(1 - dt * dt * a * schur), (-dt * a * schur), (dt * schur), schur]
    ms = [m + 1j * 0.05 * rng.normal(size=P) for m in ms]
    # rescale so the perturbed transition stays non-expanding (rho <= 0.999)
    M = np.stack([np.stack(ms[:2], -1), np.stack(ms[2:], -1)], -2)
    rho = np.abs(np.linalg.eigvals(M)).max(-1)
    scale = np.minimum(1.0, 0.999 / rho)
    ms = [(m * scale).astype(np.complex64) for m in ms]
    b = (rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))).astype(np.complex64)
    go = (rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))).astype(np.complex64)
    return ms, b, go


def test_linoss_matches_reference_kernel_vectors(K):
    with np.load(GOLDEN / "ref_kernel_vectors.npz") as z:
        v = {k: z[k] for k in z.files}
    announce("linoss golden")
    out = K.linoss_scan(*[to_dev(v[k]) for k in ("lo_m11", "lo_m12", "lo_m21", "lo_m22", "lo_b")])
    assert_close(to_np(out), v["lo_out"], RTOL, ATOL)


@pytest.mark.parametrize("shape", [(1, 1, 1), (37, 3, 5), (1500, 2, 96)],
                         ids=lambda s: "x".join(map(str, s)))
def test_linoss_forward_backward_vs_oracle(K, shape):
    L, B, P = shape
    ms, b, go = _linoss_inputs(L, B, P, seed=L + P)
    announce(f"linoss L={L} B={B} P={P}")
    st = K.linoss_scan(*[to_dev(m) for m in ms], to_dev(b))
    ref = oracle.linoss_forward(*ms, b)
    ms64 = [m.astype(np.complex128) for m in ms]
    st64 = oracle.linoss_forward(*ms64, b.astype(np.complex128))
    assert_parity(to_np(st), ref, st64, RTOL, ATOL, "states")
    gm, gb = K.linoss_scan_backward(*[to_dev(m) for m in ms], st, to_dev(go))
    rgm, rgb = oracle.linoss_backward(*ms, ref, go)
    tgm, tgb = oracle.linoss_backward(*ms64, st64, go.astype(np.complex128))
    assert_parity(to_np(gb), rgb, tgb, RTOL, ATOL, "grad_b")
    assert_parity(to_np(gm), rgm, tgm, RTOL, _param_atol(tgm), "grad_m")
    no_device_errors()


@pytest.mark.parametrize("shape", [(1, 1, 1), (37, 3, 5), (600, 2, 96)],
                         ids=lambda s: "x".join(map(str, s)))
def test_linoss_complex128_vs_oracle(K, shape):
    """complex128 LinOSS runs on the device, as the reference's kernel dispatches
    it (linoss_scan_cuda.cu:139): forward and the native backward against the
    fp64 oracle at rtol 1e-10."""
    import torch

    L, B, P = shape
    ms, b, go = _linoss_inputs(L, B, P, seed=3 * L + P)
    ms = [m.astype(np.complex128) for m in ms]
    b, go = b.astype(np.complex128), go.astype(np.complex128)
    announce(f"linoss c128 L={L} B={B} P={P}")
    st = K.linoss_scan(*[to_dev(m) for m in ms], to_dev(b))
    assert st.dtype == torch.complex128
    ref = oracle.linoss_forward(*ms, b)
    scale = max(1.0, float(np.abs(ref).max()))
    assert_close(to_np(st), ref, 1e-10, 1e-12 * scale, "c128 states")
    gm, gb = K.linoss_scan_backward(*[to_dev(m) for m in ms], st, to_dev(go))
    rgm, rgb = oracle.linoss_backward(*ms, ref, go)
    assert_close(to_np(gb), rgb, 1e-10, 1e-12 * max(1.0, float(np.abs(rgb).max())), "c128 grad_b")
    assert_close(to_np(gm), rgm, 1e-10, 1e-12 * max(1.0, float(np.abs(rgm).max())), "c128 grad_m")
    # mixed dtypes are rejected, not reinterpreted
    with pytest.raises(RuntimeError, match="b_seq's dtype"):
        K.linoss_scan(*[to_dev(m.astype(np.complex64)) for m in ms], to_dev(b))
    no_device_errors()


def _linoss_grad(rng, L, B, P):
    return (rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))).astype(np.complex64)


@pytest.mark.parametrize("B", [4, 32])
def test_linoss_imex_unit_modulus(K, B):
    """LinOSS-IMEX (linoss.py:253-258): M = [[1, -dt a], [dt, 1 - dt^2 a]] has
    det M = 1 and, for dt^2 a < 4, both eigenvalues on the unit circle, so
    neither the chunk powers M^T nor the look-back carries decay.  L = 4096,
    b = (bu dt, bu dt^2); forward and the native backward against the oracle
    and fp64 truth.  B = 4 leaves 64 workgroups, so the forward runs 128-step
    chunks; B = 32 runs its 256-step tile (16 steps x 16 waves, M^256)."""
    L, P = 4096, 64
    rng = np.random.default_rng(4096)
    a = rng.uniform(0.1, 1.0, P)
    dt = 1 / (1 + np.exp(-rng.normal(size=P)))
    ms64 = [np.ones(P), -dt * a, dt, 1 - dt * dt * a]
    lam = np.linalg.eigvals(np.stack([np.stack(ms64[:2], -1), np.stack(ms64[2:], -1)], -2))
    assert np.allclose(np.abs(lam), 1.0, atol=1e-12)  # the regime under test
    ms = [m.astype(np.complex64) for m in ms64]
    bu = (rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))).astype(np.complex64)
    dtc = dt.astype(np.complex64)
    b = np.ascontiguousarray(np.stack([bu * dtc, bu * dtc * dtc], -1).astype(np.complex64))
    go = _linoss_grad(rng, L, B, P)
    announce(f"linoss IMEX |lambda|=1 L={L} B={B} P={P}")
    st = K.linoss_scan(*[to_dev(m) for m in ms], to_dev(b))
    ref = oracle.linoss_forward(*ms, b)
    ms128 = [m.astype(np.complex128) for m in ms]
    st64 = oracle.linoss_forward(*ms128, b.astype(np.complex128))
    assert_parity(to_np(st), ref, st64, RTOL, ATOL, "IMEX states")
    gm, gb = K.linoss_scan_backward(*[to_dev(m) for m in ms], st, to_dev(go))
    rgm, rgb = oracle.linoss_backward(*ms, ref, go)
    tgm, tgb = oracle.linoss_backward(*ms128, st64, go.astype(np.complex128))
    assert_parity(to_np(gb), rgb, tgb, RTOL, ATOL, "IMEX grad_b")
    assert_parity(to_np(gm), rgm, tgm, RTOL, _param_atol(tgm), "IMEX grad_m")
    no_device_errors()


def test_linoss_config1_workload(K):
    """BASELINE config 1 exactly: LinOSS-IM forward, B=8 L=1024 P=64 H=64 with
    A_diag = relu(N(0,1)) + 0.1, dt = sigmoid(N(0,1)), B complex N(0, 1/H),
    u ~ N(0,1), bu = u B^T and b_seq = (bu m11 dt, bu m21 dt) (linoss.py:244-251);
    every state against the oracle (elementwise, fp64 fallback), plus the
    native backward."""
    Bsz, L, P, H = 8, 1024, 64, 64
    rng = np.random.default_rng(1)
    A = np.maximum(rng.normal(size=P), 0.0) + 0.1
    dt = 1 / (1 + np.exp(-rng.normal(size=P)))
    Bw = (rng.normal(size=(P, H)) + 1j * rng.normal(size=(P, H))) / np.sqrt(H)
    u = rng.normal(size=(Bsz, L, H))
    bu = np.ascontiguousarray((u @ Bw.T).transpose(1, 0, 2))  # [L, B, P]
    schur = 1 / (1 + dt * dt * A)
    ms64 = [1 - dt * dt * A * schur, -dt * A * schur, dt * schur, schur]
    b64 = np.stack([bu * ms64[0] * dt, bu * ms64[2] * dt], -1)
    ms = [m.astype(np.complex64) for m in ms64]
    b = np.ascontiguousarray(b64.astype(np.complex64))
    announce(f"linoss IM config1 B={Bsz} L={L} P={P} H={H}")
    st = K.linoss_scan(*[to_dev(m) for m in ms], to_dev(b))
    ref = oracle.linoss_forward(*ms, b)
    ms128 = [m.astype(np.complex128) for m in ms]
    st64 = oracle.linoss_forward(*ms128, b.astype(np.complex128))
    assert tuple(st.shape) == (L, Bsz, P, 2)
    assert_parity(to_np(st), ref, st64, RTOL, ATOL, "config1 states")
    go = _linoss_grad(rng, L, Bsz, P)
    gm, gb = K.linoss_scan_backward(*[to_dev(m) for m in ms], st, to_dev(go))
    rgm, rgb = oracle.linoss_backward(*ms, ref, go)
    tgm, tgb = oracle.linoss_backward(*ms128, st64, go.astype(np.complex128))
    assert_parity(to_np(gb), rgb, tgb, RTOL, ATOL, "config1 grad_b")
    assert_parity(to_np(gm), rgm, tgm, RTOL, _param_atol(tgm), "config1 grad_m")
    no_device_errors()
