"""GPU parity of the diagonal complex scans (``lru_scan`` / ``s5_scan`` and their
native backward, through the drop-in module, i.e. the C ABI) against the CPU
oracle, the reference's own kernel vectors and the reference test's literals.

Tolerance (north star): rtol 1e-4 / atol 1e-5 against the fp32 reference
arithmetic; where a long fp32 recurrence misses that bound, the GPU must be as
close to fp64 truth as the fp32 oracle is (``assert_parity``).  grad_lambda is a
sum over time and batch: its atol scales with the sum's magnitude.  fp64 runs
are checked against the fp64 oracle at 1e-10.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.gpu_util import announce, assert_close, assert_parity, need_gpu, no_device_errors

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def _dev_real(z):
    """complex numpy [..] -> device real view [.., 2]"""
    import torch

    return torch.view_as_real(torch.from_numpy(np.ascontiguousarray(z))).contiguous().cuda()


def _np_complex(t):
    import torch

    return torch.view_as_complex(t.detach().contiguous()).cpu().numpy()


def diag_inputs(L, B, P, seed, dtype=np.complex64, radius=(0.5, 0.999)):
    """Seeded eigenvalues inside the unit disc (LRU's ring init, lru.py:118-134,
    draws |lambda| in [r_min, r_max] and phases in [0, max_phase]) and complex
    normal inputs and upstream gradients."""
    rng = np.random.default_rng(seed)
    lam = rng.uniform(*radius, P) * np.exp(1j * rng.uniform(0, 6.28, P))
    b = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    go = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    return lam.astype(dtype), b.astype(dtype), go.astype(dtype)


def _run(K, lam, b, go, name="lru"):
    import torch

    fwd = getattr(K, f"{name}_scan")
    bwd = getattr(K, f"{name}_scan_backward")
    rdt = torch.float32 if lam.dtype == np.complex64 else torch.float64
    lre = torch.from_numpy(np.ascontiguousarray(lam.real)).to(rdt).cuda()
    lim = torch.from_numpy(np.ascontiguousarray(lam.imag)).to(rdt).cuda()
    states = fwd(lre, lim, _dev_real(b))
    gl, gb = bwd(lre, lim, states, _dev_real(go))
    return _np_complex(states), _np_complex(gl), _np_complex(gb)


def _check(lam, b, go, states, gl, gb, what):
    if lam.dtype == np.complex128:
        st = oracle.diag_forward(lam, b)
        assert_close(states, st, 1e-10, 1e-10, f"{what} states")
        rl, rb = oracle.diag_backward(lam, st, go)
        assert_close(gb, rb, 1e-10, 1e-10, f"{what} grad_b")
        assert_close(gl, rl, 1e-10, 1e-10 * max(1.0, float(np.abs(rl).max())), f"{what} grad_lambda")
        return
    ref = oracle.diag_forward(lam, b)
    f64 = [x.astype(np.complex128) for x in (lam, b, go)]
    truth = oracle.diag_forward(f64[0], f64[1])
    assert_parity(states, ref, truth, RTOL, ATOL, f"{what} states")
    # the backward from the GPU's own states, as the bridge does
    rl, rb = oracle.diag_backward(lam, states, go)
    tl, tb = oracle.diag_backward(f64[0], truth, f64[2])
    assert_parity(gb, rb, tb, RTOL, ATOL, f"{what} grad_b")
    assert_parity(gl, rl, tl, RTOL, 2e-5 * max(1.0, float(np.abs(tl).max())), f"{what} grad_lambda")


@pytest.mark.parametrize("prec", ["f32", "f64"])
@pytest.mark.parametrize("name", ["lru", "s5"])
def test_diag_matches_reference_kernel_vectors(K, prec, name):
    """GPU forward vs the reference's own CPU kernels (fixture)."""
    with np.load(GOLDEN / "diag_kernel_vectors.npz", allow_pickle=False) as z:
        v = {k: z[k] for k in z.files}
    announce(f"diag golden {name} {prec}")
    lam, b = v[f"{prec}_lambda"], v[f"{prec}_b"]
    states, _, _ = _run(K, lam, b, np.zeros_like(b), name)
    tol = 1e-5 if prec == "f32" else 1e-12
    assert_close(states, v[f"{prec}_{name}"], tol, tol, f"{name} {prec}")
    no_device_errors()


def test_diag_matches_reference_complex_literal(K):
    """The reference test's literal case (test_scan_parity.py:186-349, :465-474)."""
    d = json.loads((GOLDEN / "complex_scan_reference.json").read_text())
    c = lambda k: np.asarray(d[k])[..., 0] + 1j * np.asarray(d[k])[..., 1]  # noqa: E731
    announce("diag reference literal")
    lam = c("REFERENCE_COMPLEX_LAMBDA").astype(np.complex64)
    b = c("REFERENCE_COMPLEX_B").astype(np.complex64)
    for name in ("lru", "s5"):
        states, _, _ = _run(K, lam, b, np.zeros_like(b), name)
        assert_close(states, c("REFERENCE_COMPLEX_STATES"), 5e-6, 5e-6, name)


# (L, B, P): single step, ragged channel counts (B*P not a multiple of 64), one
# and several forward chunks (128 steps), long look-back, one channel; the last
# shape takes the backward's 16 x 16 tile (340 workgroups of 256-step chunks)
# with a ragged last chunk and channel group, the others its 16 x 8 tile
SHAPES = [(1, 1, 1), (5, 2, 3), (70, 3, 5), (128, 1, 64), (300, 3, 70), (1000, 2, 64),
          (129, 5, 33), (4100, 1, 1), (5000, 8, 130)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_diag_vs_oracle_f32(K, shape):
    L, B, P = shape
    lam, b, go = diag_inputs(L, B, P, seed=L + 3 * B + 5 * P)
    announce(f"diag f32 L={L} B={B} P={P}")
    states, gl, gb = _run(K, lam, b, go)
    _check(lam, b, go, states, gl, gb, f"f32 {shape}")


@pytest.mark.parametrize("shape", [(1, 1, 1), (70, 3, 5), (300, 3, 70), (1000, 2, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_diag_vs_oracle_f64(K, shape):
    L, B, P = shape
    lam, b, go = diag_inputs(L, B, P, seed=7 * L + B + P, dtype=np.complex128)
    announce(f"diag f64 L={L} B={B} P={P}")
    states, gl, gb = _run(K, lam, b, go)
    _check(lam, b, go, states, gl, gb, f"f64 {shape}")


def test_diag_eigenvalue_edge_cases(K):
    """lambda = 0 (x = b), |lambda| = 1 on the real axis (running sums), and
    negative / imaginary eigenvalues, across several chunks."""
    L, B = 700, 2
    lam = np.array([0.0, 1.0, -1.0, 1j, -0.999, 0.999j], np.complex64)
    P = lam.size
    rng = np.random.default_rng(4)
    b = (rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))).astype(np.complex64) * 0.1
    go = (rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))).astype(np.complex64)
    announce("diag eigenvalue edge cases")
    states, gl, gb = _run(K, lam, b, go)
    assert_close(states[:, :, 0], b[:, :, 0], 0, 0, "lambda=0")
    _check(lam, b, go, states, gl, gb, "edge eigenvalues")


def test_diag_config_size(K):
    """The benchmark shape (B=32, L=4096, P=128): forward and backward against
    the fp32 oracle and fp64 truth."""
    L, B, P = 4096, 32, 128
    lam, b, go = diag_inputs(L, B, P, seed=2024)
    announce(f"diag config L={L} B={B} P={P}")
    states, gl, gb = _run(K, lam, b, go)
    _check(lam, b, go, states, gl, gb, "config")
    no_device_errors()


def test_diag_empty_and_errors(K):
    import torch

    lam, b, go = diag_inputs(4, 2, 3, seed=1)
    lre = torch.from_numpy(lam.real.copy()).cuda()
    lim = torch.from_numpy(lam.imag.copy()).cuda()
    db = _dev_real(b)
    out = K.lru_scan(lre, lim, db[:0])
    assert tuple(out.shape) == (0, 2, 3, 2)
    out = K.s5_scan(lre, lim, db[:, :0])
    assert tuple(out.shape) == (4, 0, 3, 2)
    gl, gb = K.lru_scan_backward(lre, lim, db[:0], db[:0])
    assert tuple(gl.shape) == (3, 2) and float(gl.abs().sum()) == 0.0
    with pytest.raises(RuntimeError, match="b_seq must have shape"):
        K.lru_scan(lre, lim, db[0])
    with pytest.raises(RuntimeError, match="match state dimension"):
        K.lru_scan(lre[:2], lim, db)
    with pytest.raises(RuntimeError, match="1-D"):
        K.s5_scan(lre[None], lim, db)
    with pytest.raises(RuntimeError, match="share one floating dtype"):
        K.lru_scan(lre.double(), lim.double(), db)
    with pytest.raises(RuntimeError, match="grad_output must match"):
        K.lru_scan_backward(lre, lim, db, db[:2])


def test_diag_bridge_autograd(K):
    """DiagScanFn (the _LRUScanFn / _S5ScanFn counterpart) through torch.autograd
    on complex tensors, against the oracle's restated Python backward."""
    import torch

    from ossm_amd import bridge

    L, B, P = 257, 3, 40
    lam, b, go = diag_inputs(L, B, P, seed=5)
    announce("diag bridge autograd")
    for fn in (bridge.try_run_lru_scan, bridge.try_run_s5_scan):
        tl = torch.from_numpy(lam).cuda().requires_grad_(True)
        tb = torch.from_numpy(b).cuda().requires_grad_(True)
        x = fn(tl, tb)
        gl, gb = torch.autograd.grad(x, (tl, tb), grad_outputs=torch.from_numpy(go).cuda())
        states = x.detach().cpu().numpy()
        _check(lam, b, go, states, gl.cpu().numpy(), gb.cpu().numpy(), fn.__name__)
    empty = torch.from_numpy(b[:0]).cuda()
    assert bridge.try_run_lru_scan(torch.from_numpy(lam).cuda(), empty) is empty


def test_diag_repeatable(K):
    """Two runs agree to rounding (look-back association depends on publish
    timing, and every chunk's share of grad_lambda is added atomically)."""
    lam, b, go = diag_inputs(3000, 4, 96, seed=9)
    announce("diag repeatability")
    s1, l1, b1 = _run(K, lam, b, go)
    s2, l2, b2 = _run(K, lam, b, go)
    # reassociated carries differ by a few ulps of the largest summands (|x| ~ 20 at
    # |lambda| = 0.999), not of each result
    assert_close(s1, s2, 1e-5, 1e-6 * max(1.0, float(np.abs(s2).max())), "states")
    assert_close(b1, b2, 1e-5, 1e-6 * max(1.0, float(np.abs(b2).max())), "grad_b")
    assert_close(l1, l2, 1e-5, 1e-6 * max(1.0, float(np.abs(l2).max())), "grad_lambda")
