"""GPU parity of the selective scan (through the drop-in module, i.e. the C
ABI) against the CPU oracle and the reference kernel vectors.

Tolerance (north star): rtol 1e-4 / atol 1e-5 in fp32 against the reference
CPU kernel, for the per-element outputs (out, du, ddt, dz).  dB and dC are
sums over channels and dA a sum over batch and time: their summation order
differs from the reference's sequential fp32 accumulators, so they are
compared with an atol scaled by the gradient's magnitude and, where the
elementwise bound misses, against fp64 truth (the GPU must be as accurate as
the reference kernel).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.gpu_util import announce, assert_close, assert_parity, need_gpu, rel_fro, to_dev, to_np

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-4, 1e-5
NAMES = ("du", "ddt", "dA", "dB", "dC", "dz")


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def selective_inputs(Bz, D, L, N, seed, gated=True):
    """Seeded inputs with the distributions of BASELINE configs 3/4:
    A = -exp(log(arange(1..N))) for every channel, dt = softplus(N(0,1) - 4),
    u, B, C, z, upstream grad ~ N(0,1); B/C in the API layout [B, L, N]."""
    rng = np.random.default_rng(seed)
    u = rng.normal(size=(Bz, D, L)).astype(np.float32)
    dt = np.log1p(np.exp(rng.normal(size=(Bz, D, L)) - 4.0)).astype(np.float32)
    A = np.tile(-np.exp(np.log(np.arange(1, N + 1, dtype=np.float64))), (D, 1)).astype(np.float32)
    Bm = rng.normal(size=(Bz, L, N)).astype(np.float32)
    Cm = rng.normal(size=(Bz, L, N)).astype(np.float32)
    z = rng.normal(size=(Bz, D, L)).astype(np.float32) if gated else None
    g = rng.normal(size=(Bz, D, L)).astype(np.float32)
    return u, dt, A, Bm, Cm, z, g


def _run(K, u, dt, A, Bm, Cm, z, g):
    dz = None if z is None else to_dev(z)
    out, chunks, raw = K.selective_scan_cuda(to_dev(u), to_dev(dt), to_dev(A), to_dev(Bm),
                                             to_dev(Cm), dz)
    grads = K.selective_scan_cuda_backward(to_dev(g), to_dev(u), to_dev(dt), to_dev(A),
                                           to_dev(Bm), to_dev(Cm), dz, chunks, raw, 16)
    return out, chunks, raw, grads


def _sum_atol(ref):
    return 2e-5 * max(1.0, float(np.abs(ref).max()))


def _check_all(out, grads, u, dt, A, Bm, Cm, z, g, what=""):
    ref_out = oracle.selective_forward(u, dt, A, Bm, Cm, z)
    ref_g = oracle.selective_backward(g, u, dt, A, Bm, Cm, z)
    f64 = [x.astype(np.float64) if x is not None else None for x in (u, dt, A, Bm, Cm, z, g)]
    t_out = oracle.selective_forward(*f64[:6])
    t_g = oracle.selective_backward(f64[6], *f64[:6])
    assert_parity(to_np(out), ref_out, t_out, RTOL, ATOL, f"{what} out")
    for got, r32, r64, name in zip(grads, ref_g, t_g, NAMES):
        atol = _sum_atol(r64) if name in ("dA", "dB", "dC") else ATOL
        assert_parity(to_np(got), r32, r64, RTOL, atol, f"{what} {name}")


@pytest.mark.parametrize("tag", ["gate", "nogate"])
def test_selective_matches_reference_kernel_vectors(K, tag):
    """GPU vs the outputs of the reference's own CPU kernels (fixture)."""
    with np.load(GOLDEN / "ref_kernel_vectors.npz") as zf:
        v = {k: zf[k] for k in zf.files}
    z = v["sel_z"] if tag == "gate" else None
    announce(f"selective golden {tag} B=2 D=5 L=47 N=8")
    out, _, _, grads = _run(K, v["sel_u"], v["sel_dt"], v["sel_A"], v["sel_B"], v["sel_C"], z,
                            v["sel_grad"])
    assert_close(to_np(out), v[f"sel_{tag}_out"], RTOL, ATOL, "out")
    for got, name in zip(grads, NAMES):
        ref = v[f"sel_{tag}_{name}"]
        atol = _sum_atol(ref) if name in ("dA", "dB", "dC") else ATOL
        assert_close(to_np(got), ref, RTOL, atol, name)


# (B, D, L, N): tiny, ragged (D not a multiple of 64, L not a multiple of 4 or
# 16, N not a multiple of 4), several passes over the states (N > 16), the
# shapes of the reference's own tests (test_scan_parity.py:63-183)
# The forward runs 2 states per lane while 64-channel workgroups would give
# fewer than 4 waves per SIMD, else 4: on a 256-CU MI355X every shape below
# runs 2 except (64, 1024, 64, 16) (1,024 rows of 64 channels), which runs 4.
# The backward likewise runs 2 states per lane below 512 such rows: every shape
# but (64, 1024, 64, 16); test_selective_backward_both_layouts runs both.
SHAPES = [(1, 1, 1, 1), (2, 5, 3, 3), (2, 70, 37, 5), (3, 65, 100, 16), (1, 130, 129, 20),
          (2, 32, 256, 32), (2, 48, 192, 32), (4, 96, 384, 64), (1, 3, 50, 256),
          (64, 1024, 64, 16)]


@pytest.mark.parametrize("gated", [True, False], ids=["gate", "nogate"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_selective_forward_backward_vs_oracle(K, shape, gated):
    Bz, D, L, N = shape
    args = selective_inputs(Bz, D, L, N, seed=Bz + 3 * D + 7 * L + 11 * N, gated=gated)
    announce(f"selective B={Bz} D={D} L={L} N={N} gated={gated}")
    out, chunks, raw, grads = _run(K, *args)
    assert tuple(chunks.shape) == (Bz, D, (L + 31) // 32, 2 * N)
    _check_all(out, grads, *args, what=f"{shape}")
    if not gated:
        assert float(grads[5].abs().max()) == 0.0


# ragged channels and steps (a last tile shorter than half a 32-step tile and
# one longer), several passes over the states, and long rows that the time
# split cuts into segments
LAYOUT_SHAPES = [(2, 70, 37, 5), (3, 65, 100, 16), (1, 130, 129, 20), (4, 96, 384, 64),
                 (1, 3, 50, 256), (1, 64, 1000, 16), (2, 40, 2070, 16)]


@pytest.mark.parametrize("npw", [2, 4])
@pytest.mark.parametrize("shape", LAYOUT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_selective_backward_both_layouts(K, shape, npw, monkeypatch):
    """The backward with 2 and with 4 states per lane (OSSM_SEL_BWD_NPW forces
    the choice the library otherwise makes from the shape), gated."""
    monkeypatch.setenv("OSSM_SEL_BWD_NPW", str(npw))
    Bz, D, L, N = shape
    args = selective_inputs(Bz, D, L, N, seed=5 * Bz + D + 3 * L + N + npw)
    announce(f"selective backward npw={npw} B={Bz} D={D} L={L} N={N}")
    out, _, _, grads = _run(K, *args)
    _check_all(out, grads, *args, what=f"npw{npw} {shape}")


@pytest.mark.parametrize("gated", [True, False], ids=["gate", "nogate"])
@pytest.mark.parametrize("npw", [2, 4])
@pytest.mark.parametrize("shape", LAYOUT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_selective_forward_both_layouts(K, shape, npw, gated, monkeypatch):
    """The [B, D, L] forward with 2 and with 4 states per lane (OSSM_SEL_FWD_NPW
    forces the choice the library otherwise makes from the shape): ragged D
    and L, several passes over the states (N > 16), gated and not; the
    backward consumes that forward's checkpoints and raw outputs."""
    monkeypatch.setenv("OSSM_SEL_FWD_NPW", str(npw))
    Bz, D, L, N = shape
    args = selective_inputs(Bz, D, L, N, seed=7 * Bz + D + 5 * L + N + npw, gated=gated)
    announce(f"selective forward npw={npw} B={Bz} D={D} L={L} N={N} gated={gated}")
    out, _, _, grads = _run(K, *args)
    _check_all(out, grads, *args, what=f"fwd npw{npw} {shape}")


def test_selective_checkpoints_are_states(K):
    """chunk_states rows hold h after steps 32c+15 and 32c+31 (the final state
    past the end): checked against a brute-force recurrence."""
    Bz, D, L, N = 2, 3, 50, 4
    u, dt, A, Bm, Cm, _, _ = selective_inputs(Bz, D, L, N, seed=3, gated=False)
    announce("selective checkpoints")
    _, chunks, _ = K.selective_scan_cuda(to_dev(u), to_dev(dt), to_dev(A), to_dev(Bm), to_dev(Cm))
    h = np.zeros((Bz, D, N))
    hist = []
    for t in range(L):
        h = np.exp(dt[:, :, t, None] * A[None]) * h + dt[:, :, t, None] * Bm[:, None, t] * u[:, :, t, None]
        hist.append(h.copy())
    cs = to_np(chunks)
    for slot in range(2 * cs.shape[2]):
        t = min(16 * slot + 15, L - 1)
        np.testing.assert_allclose(cs[:, :, slot // 2, (slot % 2) * N:(slot % 2 + 1) * N],
                                   hist[t], rtol=1e-5, atol=1e-6, err_msg=f"slot {slot}")


def test_selective_zero_length_and_errors(K):
    import torch

    u, dt, A, Bm, Cm, z, g = selective_inputs(2, 3, 5, 4, seed=4)
    out, chunks, raw = K.selective_scan_cuda(to_dev(u[:, :, :0]), to_dev(dt[:, :, :0]), to_dev(A),
                                             to_dev(Bm[:, :0]), to_dev(Cm[:, :0]))
    assert out.shape == (2, 3, 0) and chunks.shape[2] == 0
    grads = K.selective_scan_cuda_backward(to_dev(g[:, :, :0]), to_dev(u[:, :, :0]),
                                           to_dev(dt[:, :, :0]), to_dev(A), to_dev(Bm[:, :0]),
                                           to_dev(Cm[:, :0]), None, chunks, raw, 16)
    assert float(grads[2].abs().sum()) == 0.0
    with pytest.raises(RuntimeError, match="float32"):
        K.selective_scan_cuda(to_dev(u).double(), to_dev(dt), to_dev(A), to_dev(Bm), to_dev(Cm))
    with pytest.raises(RuntimeError, match="B shape mismatch"):
        K.selective_scan_cuda(to_dev(u), to_dev(dt), to_dev(A), to_dev(Bm[:, :4]), to_dev(Cm))
    big = torch.zeros((3, 257), device="cuda")
    with pytest.raises(RuntimeError, match="supported maximum"):
        K.selective_scan_cuda(to_dev(u), to_dev(dt), big, to_dev(Bm), to_dev(Cm))


def test_selective_config3_full_size(K):
    """BASELINE config 3 (B=256, L=200, D=128, N=16, gated, right-padded
    lengths): every output and gradient vs the oracle.  The padding mask is
    applied by the caller to the upstream gradient, as in the reference's
    sequential-recommendation models."""
    Bz, D, L, N = 256, 128, 200, 16
    u, dt, A, Bm, Cm, z, g = selective_inputs(Bz, D, L, N, seed=33)
    lengths = np.random.default_rng(34).integers(20, 201, size=Bz)
    g = g * (np.arange(L)[None, None, :] < lengths[:, None, None])
    g = g.astype(np.float32)
    announce("selective config3 full")
    out, _, _, grads = _run(K, u, dt, A, Bm, Cm, z, g)
    _check_all(out, grads, u, dt, A, Bm, Cm, z, g, what="config3")


def test_selective_config4_shape_fp32(K):
    """BASELINE config 4 shape (B=16, D=1536, L=2048, N=16) in fp32, every
    batch row: out, du, ddt and dz elementwise at rtol 1e-4 / atol 1e-5
    against the reference CPU kernel's arithmetic (the oracle), dA, dB and dC
    with the magnitude-scaled atol of sums, each with fp64 truth as the
    arbiter where the fp32 reference's own rounding exceeds the bound; and
    linearity of the forward in u (gate-free)."""
    import torch

    Bz, D, L, N = 16, 1536, 2048, 16
    u, dt, A, Bm, Cm, z, g = selective_inputs(Bz, D, L, N, seed=44)
    announce("selective config4-shape fp32")
    out, _, _, grads = _run(K, u, dt, A, Bm, Cm, z, g)
    got = [to_np(out)] + [to_np(x) for x in grads]
    del out, grads
    torch.cuda.empty_cache()
    _check_all_np(got, u, dt, A, Bm, Cm, z, g, what="config4")
    # linearity of y in u (no gate): y(u + 2u') = y(u) + 2 y(u')
    u2 = np.roll(u, 1, axis=1)
    dev = [to_dev(x) for x in (dt, A, Bm, Cm)]
    y1 = K.selective_scan_cuda(to_dev(u), *dev)[0]
    y2 = K.selective_scan_cuda(to_dev(u2), *dev)[0]
    y12 = K.selective_scan_cuda(to_dev(u) + 2 * to_dev(u2), *dev)[0]
    assert rel_fro(to_np(y12), to_np(y1 + 2 * y2)) < 1e-5
    torch.cuda.synchronize()


def _check_all_np(got, u, dt, A, Bm, Cm, z, g, what=""):
    """_check_all on host arrays [out, du, ddt, dA, dB, dC, dz], computing the
    fp32 and fp64 references one after the other to bound host memory."""
    ref = [oracle.selective_forward(u, dt, A, Bm, Cm, z)]
    ref += list(oracle.selective_backward(g, u, dt, A, Bm, Cm, z))
    f64 = [x.astype(np.float64) if x is not None else None for x in (u, dt, A, Bm, Cm, z, g)]
    tru = [oracle.selective_forward(*f64[:6])]
    tru += list(oracle.selective_backward(f64[6], *f64[:6]))
    del f64
    for a, r32, r64, name in zip(got, ref, tru, ("out",) + NAMES):
        atol = _sum_atol(r64) if name in ("dA", "dB", "dC") else ATOL
        assert_parity(a, r32, r64, RTOL, atol, f"{what} {name}")


def test_selective_deterministic(K):
    """Two backward calls on the same inputs give bitwise-identical gradients."""
    args = selective_inputs(3, 200, 300, 16, seed=5)
    announce("selective determinism")
    _, _, _, g1 = _run(K, *args)
    _, _, _, g2 = _run(K, *args)
    for a, b, name in zip(g1, g2, NAMES):
        assert np.array_equal(to_np(a), to_np(b)), name
