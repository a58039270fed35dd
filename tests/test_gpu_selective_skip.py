"""GPU parity of the selective scan with a fused per-channel skip D
(``selective_scan_cuda_skip`` and its backward, the C entry points
``ossm_selective_{forward,backward}_skip``): an extension with no counterpart
in the reference's kernels, which take no D (selective_scan_cuda.cu:253-393);
BASELINE configs 3 and 4 name a D skip.

Expected values are composed from the oracle's ungated scan, which is pinned
to the reference's CPU kernels (selective_scan_cpu.cpp:78-360), and the
skip's definition (the Mamba block's y + D u before the gate).  With y the
ungated scan output and gy = g * silu(z) the gated upstream gradient (g
without a gate):

    raw = y + D u,   out = raw * silu(z),
    du  = du_scan(gy) + D gy,   ddt, dA, dB, dC = the scan's gradients under gy,
    dD  = sum over batch and time of gy u,   dz = g * raw * silu'(z),

each in fp32 (the reference's precision) and in fp64 (the arbiter of
assert_parity).  Sums over batch, time or channels (dA, dB, dC, dD) take the
magnitude-scaled atol.  With D = 0 the skip entry points must return the plain
entry points' results bit for bit (and dD = sum gy u).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.gpu_util import announce, assert_parity, need_gpu, sum_atol, to_dev, to_np
from tests.test_gpu_selective import selective_inputs

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5
NAMES = ("out", "du", "ddt", "dA", "dB", "dC", "dD", "dz")
SUMS = ("dA", "dB", "dC", "dD")
EPS_BF16 = 2.0 ** -8


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def skip_inputs(Bz, D, L, N, seed, gated=True):
    u, dt, A, Bm, Cm, z, g = selective_inputs(Bz, D, L, N, seed, gated)
    Dk = np.random.default_rng(seed + 1000).normal(size=D).astype(np.float32)
    return u, dt, A, Bm, Cm, Dk, z, g


def skip_reference(u, dt, A, Bm, Cm, Dk, z, g):
    """[out, du, ddt, dA, dB, dC, dD, dz] in the inputs' precision (see the
    module docstring); dz is None without a gate."""
    y = oracle.selective_forward(u, dt, A, Bm, Cm, None)
    raw = y + Dk[None, :, None] * u
    if z is not None:
        sg = 1.0 / (1.0 + np.exp(-z))
        out = raw * (z * sg)
        gy = g * (z * sg)
        dz = g * raw * (sg * (1.0 + z * (1.0 - sg)))
    else:
        out, gy, dz = raw, g, None
    du, ddt, dA, dB, dC, _ = oracle.selective_backward(gy.astype(u.dtype), u, dt, A, Bm, Cm, None)
    du = du + Dk[None, :, None] * gy
    dD = (gy * u).sum(axis=(0, 2))
    return [out, du, ddt, dA, dB, dC, dD, dz]


def run_skip(K, u, dt, A, Bm, Cm, Dk, z, g, dtype=None):
    import torch

    conv = (lambda x: to_dev(x)) if dtype is None else (lambda x: to_dev(x).to(dtype))
    zz = None if z is None else conv(z)
    ud, dtd, Bd, Cd = conv(u), conv(dt), conv(Bm), conv(Cm)
    Ad, Dd = to_dev(A), to_dev(Dk)
    out, chunks, raw = K.selective_scan_cuda_skip(ud, dtd, Ad, Bd, Cd, Dd, zz)
    grads = K.selective_scan_cuda_skip_backward(conv(g), ud, dtd, Ad, Bd, Cd, Dd, zz, chunks, raw)
    assert chunks.dtype == torch.float32 and grads[2].dtype == torch.float32
    assert grads[5].dtype == torch.float32 and grads[5].shape == (u.shape[1],)
    return [out] + list(grads)


def check_skip(got, args, what):
    """Every output against the fp32 composition, fp64 as the arbiter."""
    r32 = skip_reference(*args)
    f64 = [None if x is None else x.astype(np.float64) for x in args]
    r64 = skip_reference(*f64)
    for a, x32, x64, name in zip(got, r32, r64, NAMES):
        if x32 is None:
            continue
        atol = sum_atol(x64) if name in SUMS else ATOL
        assert_parity(to_np(a.float()), x32, x64, RTOL, atol, f"{what} {name}")


# (1, 64, 2048, 16): few rows, so both directions split each row's time span
# across workgroups; (2, 48, 192, 32) and (4, 96, 384, 64): several 16-state passes
SHAPES = [(1, 1, 1, 1), (2, 70, 37, 5), (3, 65, 100, 16), (1, 130, 129, 20), (2, 48, 192, 32),
          (4, 96, 384, 64), (1, 64, 2048, 16)]


@pytest.mark.parametrize("gated", [True, False], ids=["gate", "nogate"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_selective_skip_vs_oracle(K, shape, gated):
    args = skip_inputs(*shape, seed=11 + sum(shape), gated=gated)
    announce(f"selective skip {shape} gated={gated}")
    check_skip(run_skip(K, *args), args, f"{shape}")


@pytest.mark.parametrize("npw", [2, 4])
@pytest.mark.parametrize("shape", [(2, 70, 37, 5), (1, 130, 129, 20), (4, 96, 384, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_selective_skip_both_layouts(K, shape, npw, monkeypatch):
    """Forward and backward forced to 2 and to 4 states per lane."""
    monkeypatch.setenv("OSSM_SEL_BWD_NPW", str(npw))
    monkeypatch.setenv("OSSM_SEL_FWD_NPW", str(npw))
    args = skip_inputs(*shape, seed=3 + npw + sum(shape), gated=True)
    announce(f"selective skip layouts {shape} npw={npw}")
    check_skip(run_skip(K, *args), args, f"{shape} npw={npw}")


@pytest.mark.parametrize("npw", [2, 4])
def test_selective_skip_zero_d_is_the_plain_scan(K, npw, monkeypatch):
    """D = 0: the skip entry points return the plain ones' outputs and
    gradients bit for bit (the skip terms add exact zeros and the per-element
    sums keep their order), and dD = sum gy u."""
    import torch

    monkeypatch.setenv("OSSM_SEL_BWD_NPW", str(npw))
    u, dt, A, Bm, Cm, Dk, z, g = skip_inputs(2, 96, 300, 16, seed=17)
    Dk = np.zeros_like(Dk)
    announce(f"selective skip D=0 npw={npw}")
    got = run_skip(K, u, dt, A, Bm, Cm, Dk, z, g)
    dev = [to_dev(x) for x in (u, dt, A, Bm, Cm, z)]
    out, chunks, raw = K.selective_scan_cuda(*dev)
    plain = [out] + list(K.selective_scan_cuda_backward(to_dev(g), *dev, chunks, raw, 16))
    for a, b, name in zip(got[:6] + got[7:], plain, ("out", "du", "ddt", "dA", "dB", "dC", "dz")):
        assert torch.equal(a, b), name
    sg = 1.0 / (1.0 + np.exp(-z.astype(np.float64)))
    dD64 = (g * z * sg * u).sum(axis=(0, 2))
    assert np.abs(to_np(got[6]) - dD64).max() <= sum_atol(dD64)


def test_selective_skip_deterministic(K):
    """Two skip backward calls give bitwise-identical gradients, dD included."""
    import torch

    args = skip_inputs(3, 200, 300, 16, seed=5)
    announce("selective skip determinism")
    g1 = run_skip(K, *args)
    g2 = run_skip(K, *args)
    for a, b, name in zip(g1, g2, NAMES):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("shape", [(2, 70, 37, 5), (3, 65, 100, 16), (4, 96, 384, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_selective_skip_bf16(K, shape):
    """bf16 storage: inputs rounded to bf16, the composition in fp64 on those
    values; every stored output within one bf16 ulp of fp64 truth (dz two, as
    it reads y + D u back from bf16 raw_outputs; dA and dD are fp32 sums)."""
    import torch

    args = list(skip_inputs(*shape, seed=7 + sum(shape), gated=True))
    for i in (0, 1, 3, 4, 6, 7):  # u, dt, B, C, z, g
        args[i] = torch.from_numpy(args[i]).to(torch.bfloat16).float().numpy()
    announce(f"selective skip bf16 {shape}")
    got = run_skip(K, *args, dtype=torch.bfloat16)
    assert got[0].dtype == torch.bfloat16 and got[6].dtype == torch.float32
    r64 = skip_reference(*[x.astype(np.float64) for x in args])
    for a, ref, name in zip(got, r64, NAMES):
        rel = {"dz": 2 * EPS_BF16, "dA": 1e-5, "dD": 1e-5}.get(name, EPS_BF16)
        err = np.abs(to_np(a.float()).astype(np.float64) - ref)
        bound = rel * np.abs(ref) + 2e-5 * max(1.0, float(np.abs(ref).max()))
        assert not (err > bound).any(), f"{name}: {int((err > bound).sum())} beyond the bound"


def test_selective_skip_config3_full_size(K):
    """BASELINE config 3 with its D skip and gate (B=256, L=200, D=128, N=16,
    fp32), every output and gradient elementwise."""
    args = skip_inputs(256, 128, 200, 16, seed=33)
    announce("selective skip config 3")
    got = run_skip(K, *args)
    check_skip(got, args, "config 3")


def _ulp_diff(a_bf16, b_bf16):
    """Distance in bf16 units in the last place (16-bit patterns as ordered integers)."""
    import torch

    def key(t):
        v = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(v < 0, -32768 - v, v)

    return (key(a_bf16) - key(b_bf16)).abs()


def test_selective_skip_bf16_config4(K):
    """BASELINE config 4 as specified (B=16, D=1536, L=2048, N=16, bf16
    storage, gate and D skip): the full tensors against the fp32 skip path on
    the same values (at most one bf16 ulp apart, 99 % equal, dz two ulps; dA
    bit-identical, dD within fp32 summation error), and one batch row (out,
    du, ddt, dB, dC, dz) within one bf16 ulp of the fp64 composition (dz two)."""
    import torch

    args = list(skip_inputs(16, 1536, 2048, 16, seed=47))
    for i in (0, 1, 3, 4, 6, 7):  # u, dt, B, C, z, g to bf16 values
        args[i] = torch.from_numpy(args[i]).to(torch.bfloat16).float().numpy()
    announce("selective skip bf16 config 4")
    got = run_skip(K, *args, dtype=torch.bfloat16)
    ref = run_skip(K, *args)
    for a, r, name in zip(got, ref, NAMES):
        if name == "dA":
            assert torch.equal(a, r), name
            continue
        if name == "dD":
            torch.testing.assert_close(a, r, rtol=1e-5, atol=1e-5 * float(r.abs().max()))
            continue
        d = _ulp_diff(a, r.to(torch.bfloat16))
        assert int(d.max()) <= (2 if name == "dz" else 1), f"{name}: {int(d.max())} ulps"
        if name != "dz":  # dz reads y + D u back from the bf16 raw_outputs
            assert float((d == 0).float().mean()) >= 0.99, name
    del ref
    bs = [5]
    sl = [np.ascontiguousarray(x[bs]).astype(np.float64) if x.ndim == 3 else x.astype(np.float64)
          for x in args]
    r64 = skip_reference(*sl)
    for idx, name in ((0, "out"), (1, "du"), (2, "ddt"), (4, "dB"), (5, "dC"), (7, "dz")):
        rel = 2 * EPS_BF16 if name == "dz" else EPS_BF16
        a = to_np(got[idx].float())[bs].astype(np.float64)
        err = np.abs(a - r64[idx])
        bound = rel * np.abs(r64[idx]) + 2e-5 * max(1.0, float(np.abs(r64[idx]).max()))
        assert not (err > bound).any(), f"{name} slice: {int((err > bound).sum())} beyond the bound"


def test_selective_skip_errors(K):
    """The skip D must be float32 (channels,) on the inputs' device; the [B, D, L]
    entry points only."""
    import torch

    u, dt, A, Bm, Cm, Dk, z, g = skip_inputs(1, 8, 16, 4, seed=1)
    dev = [to_dev(x) for x in (u, dt, A, Bm, Cm)]
    with pytest.raises(RuntimeError, match="D must be float32"):
        K.selective_scan_cuda_skip(*dev, to_dev(Dk).double())
    with pytest.raises(RuntimeError, match=r"D must have shape \(channels,\)"):
        K.selective_scan_cuda_skip(*dev, to_dev(Dk)[:4])
    with pytest.raises(RuntimeError, match="D must be on the same device"):
        K.selective_scan_cuda_skip(*dev, torch.from_numpy(Dk))
