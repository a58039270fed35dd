"""GPU parity of the selective D-LinOSS scans (``sdlinoss_<v>_forward/backward``
through the drop-in module, i.e. the C ABI) against the CPU oracle and the
reference's own kernel vectors.

Tolerance (north star): rtol 1e-4 / atol 1e-5 against the fp32 reference
arithmetic; where a long fp32 recurrence misses that bound, the GPU must be
as close to fp64 truth as the fp32 oracle is (``assert_parity``).  Parameter
gradients of broadcast parameters are sums over time and/or batch rows: their
atol scales with the magnitude of the sum.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.gpu_util import announce, assert_close, assert_parity, need_gpu, no_device_errors, to_dev, to_np

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-4, 1e-5
VARIANTS = oracle.VARIANTS
NAMES = ("grad_A", "grad_G", "grad_step", "grad_bu")


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def _shape(tag, L, B, M):
    return {"full": (L, B, M), "bcast_t": (1, B, M), "bcast_b": (L, 1, M), "m": (M,),
            "lm": (L, M), "bm": (B, M)}[tag]


def sdl_inputs(variant, tag, L, B, M, seed, clamp_steps=True):
    """Seeded inputs: a kept in each step's stable band (as DampedLinOSSLayer
    projects it, dlinoss.py:252-267), g ~ U(0, 1), steps mostly sigmoid(N(0,1))
    with some outside (1e-6, 1) so both sides of the dt clamp are exercised."""
    rng = np.random.default_rng(seed)
    shp = _shape(tag, L, B, M)
    g = rng.uniform(0.0, 1.0, shp)
    step = 1.0 / (1.0 + np.exp(-rng.normal(size=shp)))
    if clamp_steps:
        flat = step.reshape(-1)
        flat[::11] = 1.3
        flat[5::13] = -0.2
    dt = np.clip(step, 1e-6, 1.0)
    a = rng.uniform(0.1, 1.0, shp)
    s = dt * g
    lo = (2.0 + s - 2.0 * np.sqrt(1.0 + s)) / (dt * dt)
    hi = (2.0 + s + 2.0 * np.sqrt(1.0 + s)) / (dt * dt)
    if variant in ("imex2", "ex"):
        # explicit damping: keep 1 - dt g >= 0 and dt^2 a small
        g = g * 0.5
        a = np.minimum(a, 0.5 / (dt * dt))
    else:
        a = np.clip(a, lo, hi)
    bu = (rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))).astype(np.complex64)
    go = (rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))).astype(np.complex64)
    return a.astype(np.float32), g.astype(np.float32), step.astype(np.float32), bu, go


def _run(K, variant, A, G, S, bu, go):
    dA, dG, dS, dbu = to_dev(A), to_dev(G), to_dev(S), to_dev(bu)
    states = getattr(K, f"sdlinoss_{variant}_forward")(dA, dG, dS, dbu)
    grads = getattr(K, f"sdlinoss_{variant}_backward")(dA, dG, dS, dbu, states, to_dev(go))
    return states, grads


def _check(variant, A, G, S, bu, go, states, grads, what):
    ref_st = oracle.sdlinoss_forward(variant, A, G, S, bu)
    f64 = [x.astype(np.float64) if x.dtype == np.float32 else x.astype(np.complex128)
           for x in (A, G, S, bu, go)]
    t_st = oracle.sdlinoss_forward(variant, *f64[:4])
    assert_parity(to_np(states), ref_st, t_st, RTOL, ATOL, f"{what} states")
    # the backward from the GPU's own states, as the bridge does
    ref_g = oracle.sdlinoss_backward(variant, A, G, S, bu, to_np(states), go)
    t_g = oracle.sdlinoss_backward(variant, *f64[:4], t_st, f64[4])
    for got, r32, r64, name in zip(grads, ref_g, t_g, NAMES):
        got = to_np(got)
        assert got.shape == r32.shape, f"{what} {name} shape {got.shape} vs {r32.shape}"
        atol = ATOL if name == "grad_bu" else 2e-5 * max(1.0, float(np.abs(r64).max()))
        assert_parity(got, r32, r64, RTOL, atol, f"{what} {name}")


@pytest.mark.parametrize("variant,tag", [(v, t) for v in VARIANTS
                                         for t in ("full", "bcast_t", "bcast_b", "m")
                                         if t == "full" or v in ("imex1", "im")])
def test_sdlinoss_matches_reference_kernel_vectors(K, variant, tag):
    """GPU vs the outputs of the reference's own CPU kernels (fixture), with both
    clamps hit (including S below 1e-6 at the last step)."""
    with np.load(GOLDEN / "sdl_kernel_vectors.npz") as z:
        v = {k: z[k] for k in z.files}
    k = f"{variant}_{tag}"
    announce(f"sdlinoss golden {k}")
    states, grads = _run(K, variant, v[f"{k}_A"], v[f"{k}_G"], v[f"{k}_step"], v["bu"], v["grad"])
    scale = float(np.abs(v[f"{k}_states"]).max())
    assert_close(to_np(states), v[f"{k}_states"], RTOL, ATOL * max(1.0, scale), "states")
    for got, name in zip(grads, NAMES):
        ref = v[f"{k}_{name}"]
        assert tuple(got.shape) == ref.shape, name
        assert_close(to_np(got), ref, RTOL, 2e-5 * max(1.0, float(np.abs(ref).max())), name)


# (L, B, M): tiny, ragged channel counts (B*M not a multiple of 64), several
# forward chunks (128 steps) and backward chunks (64 steps; 128 with parameters
# broadcast over time), long look-back
SHAPES = [(1, 1, 1), (5, 2, 3), (70, 3, 5), (300, 3, 70), (1000, 2, 64), (129, 5, 33)]


@pytest.mark.parametrize("tag", ["full", "bcast_t", "bcast_b", "m", "lm", "bm"])
@pytest.mark.parametrize("variant", VARIANTS)
def test_sdlinoss_vs_oracle_layouts(K, variant, tag):
    L, B, M = 300, 3, 70
    args = sdl_inputs(variant, tag, L, B, M, seed=7 + len(tag))
    announce(f"sdlinoss {variant} {tag} L={L} B={B} M={M}")
    states, grads = _run(K, variant, *args)
    _check(variant, *args, states, grads, f"{variant}/{tag}")


@pytest.mark.parametrize("tag", ["bcast_t", "m", "bm"])
@pytest.mark.parametrize("variant", VARIANTS)
def test_sdlinoss_time_invariant_on_both_kernels(K, variant, tag, monkeypatch):
    """Parameters constant over time run on the oscillatory-scan kernels by
    default (chunk powers, the D-LinOSS tiles), here on a shape with several
    256-step chunks and ragged channels; OSSM_SDL_TB_OSC=0 keeps the selective
    D-LinOSS kernels, checked on the shape they were tuned and validated on
    (L=300; at L=1100 their ex / [B,M] grad_bu has one element in 231,000 at
    2.5x the fp32 oracle's own error against fp64, beyond assert_parity's 2x)."""
    for flag, (L, B, M) in (("1", (1100, 3, 70)), ("0", (300, 3, 70))):
        args = sdl_inputs(variant, tag, L, B, M, seed=31 + len(tag))
        monkeypatch.setenv("OSSM_SDL_TB_OSC", flag)
        announce(f"sdlinoss {variant} {tag} L={L} B={B} M={M} on osc kernels={flag}")
        states, grads = _run(K, variant, *args)
        _check(variant, *args, states, grads, f"{variant}/{tag}/osc={flag}")


@pytest.mark.parametrize("tag", ["bcast_t", "m"])
def test_sdlinoss_long_parameter_reductions(K, tag):
    """Parameters broadcast over time on long rows (the oscillatory-scan
    kernels): each output of [1,B,M] gets one share per chunk, each of [M] one
    per chunk and batch row, added with float atomics in the scan kernel."""
    L, B, M = 4096, 16, 64
    args = sdl_inputs("imex1", tag, L, B, M, seed=21 + len(tag))
    announce(f"sdlinoss imex1 {tag} L={L} B={B} M={M}")
    states, grads = _run(K, "imex1", *args)
    _check("imex1", *args, states, grads, f"imex1/{tag}/long")


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("variant", VARIANTS)
def test_sdlinoss_vs_oracle_shapes(K, variant, shape):
    L, B, M = shape
    args = sdl_inputs(variant, "full", L, B, M, seed=L + 3 * B + 5 * M)
    announce(f"sdlinoss {variant} full L={L} B={B} M={M}")
    states, grads = _run(K, variant, *args)
    _check(variant, *args, states, grads, f"{variant}/{shape}")


def test_sdlinoss_empty_and_errors(K):
    import torch

    a, g, s, bu, go = sdl_inputs("imex1", "full", 4, 2, 3, seed=1)
    dA, dG, dS = to_dev(a), to_dev(g), to_dev(s)
    out = K.sdlinoss_imex1_forward(dA[:0], dG[:0], dS[:0], to_dev(bu)[:0])
    assert tuple(out.shape) == (0, 2, 3, 2)
    grads = K.sdlinoss_imex1_backward(dA[:0], dG[:0], dS[:0], to_dev(bu)[:0], out,
                                      to_dev(go)[:0])
    assert all(float(x.abs().sum()) == 0.0 for x in grads[:3])
    with pytest.raises(RuntimeError, match="bu must have shape"):
        K.sdlinoss_imex1_forward(dA, dG, dS, to_dev(bu)[0])
    with pytest.raises(RuntimeError, match="optional singleton"):
        K.sdlinoss_imex1_forward(dA[:, :1, :].repeat(1, 3, 1), dG, dS, to_dev(bu))
    with pytest.raises(RuntimeError, match="to match bu"):
        K.sdlinoss_imex1_forward(dA, dG, dS, to_dev(bu).to(torch.complex128))
    with pytest.raises(RuntimeError, match="complex64 or complex128"):
        K.sdlinoss_imex1_forward(dA, dG, dS, to_dev(bu).real.contiguous())
    with pytest.raises(RuntimeError, match="grad_output must match"):
        K.sdlinoss_imex1_backward(dA, dG, dS, to_dev(bu), out, to_dev(go)[:2])


def test_sdlinoss_persistent_forward(K, monkeypatch):
    """Per-step parameters on a grid of 512 chunks (more than the device holds
    workgroups at once): the persistent forward (each workgroup several chunks
    in ticket order) and the one-workgroup-per-chunk launch (OSSM_OSC_PERSIST=0)
    against the oracle, with the fp64 arbiter."""
    L, B, M = 4096, 8, 128
    args = sdl_inputs("imex1", "full", L, B, M, seed=21)
    A, G, S, bu, _ = args
    ref = oracle.sdlinoss_forward("imex1", A, G, S, bu)
    t64 = oracle.sdlinoss_forward("imex1", *(x.astype(np.float64) for x in (A, G, S)),
                                  bu.astype(np.complex128))
    announce(f"sdlinoss persistent forward L={L} B={B} M={M}")
    for mode in ("1", "0"):
        monkeypatch.setenv("OSSM_OSC_PERSIST", mode)
        st = to_np(K.sdlinoss_imex1_forward(*(to_dev(x) for x in (A, G, S, bu))))
        assert_parity(st, ref, t64, RTOL, ATOL, f"persist={mode} states")
    no_device_errors()


def test_sdlinoss_repeatable(K):
    """Two runs agree to rounding: the carries between chunks come from the
    decoupled look-back, whose association depends on which records are already
    published, and each chunk's share of the parameter gradients is added with a
    float atomic, so the last bits may differ.  A state is a sum of terms of
    the states' own scale, so its rounding differences are ulps of that scale
    (the largest |state|), not of the state itself: a state near zero may
    differ by ~1e-7 between runs."""
    args = sdl_inputs("im", "bcast_t", 500, 4, 96, seed=9)
    announce("sdlinoss repeatability")
    s1, g1 = _run(K, "im", *args)
    s2, g2 = _run(K, "im", *args)
    s1, s2 = to_np(s1), to_np(s2)
    assert_close(s1, s2, 1e-6, 1e-6 * max(1.0, float(np.abs(s2).max())), "states")
    for a, b, name in zip(g1, g2, NAMES):
        a, b = to_np(a), to_np(b)
        assert_close(a, b, 1e-5, 1e-6 * max(1.0, float(np.abs(b).max())), name)


def _to64(args):
    return [x.astype(np.float64) if x.dtype == np.float32 else x.astype(np.complex128) for x in args]


# fp64 bound: both sides compute the same recurrence in double; the oracle's
# sums over broadcast axes run in another order
RTOL64, ATOL64 = 1e-10, 1e-12


@pytest.mark.parametrize("tag", ["full", "bcast_t", "bcast_b", "m", "lm", "bm"])
@pytest.mark.parametrize("variant", VARIANTS)
def test_sdlinoss_complex128_vs_oracle(K, variant, tag):
    """complex128 inputs (float64 parameters) run on the device, as the
    reference's kernels dispatch them (sdlinoss_imex1_cuda.cu:232, 271)."""
    import torch

    L, B, M = 150, 3, 37
    A, G, S, bu, go = _to64(sdl_inputs(variant, tag, L, B, M, seed=11 + len(tag)))
    announce(f"sdlinoss c128 {variant} {tag} L={L} B={B} M={M}")
    dA, dG, dS, dbu = to_dev(A), to_dev(G), to_dev(S), to_dev(bu)
    states = getattr(K, f"sdlinoss_{variant}_forward")(dA, dG, dS, dbu)
    assert states.dtype == torch.complex128
    grads = getattr(K, f"sdlinoss_{variant}_backward")(dA, dG, dS, dbu, states, to_dev(go))
    ref_st = oracle.sdlinoss_forward(variant, A, G, S, bu)
    scale = max(1.0, float(np.abs(ref_st).max()))
    assert_close(to_np(states), ref_st, RTOL64, ATOL64 * scale, "c128 states")
    ref_g = oracle.sdlinoss_backward(variant, A, G, S, bu, ref_st, go)
    for got, ref, name in zip(grads, ref_g, NAMES):
        got = to_np(got)
        assert got.dtype == ref.dtype and got.shape == ref.shape, name
        assert_close(got, ref, RTOL64, ATOL64 * max(1.0, float(np.abs(ref).max())), f"c128 {name}")


def test_sdlinoss_complex128_golden_and_edges(K):
    """The reference kernel vectors in fp64 (bound set by their fp32
    arithmetic), one-step and single-channel shapes, and empty inputs."""
    import torch

    with np.load(GOLDEN / "sdl_kernel_vectors.npz") as z:
        v = {k: z[k] for k in z.files}
    for variant in VARIANTS:
        k = f"{variant}_full"
        A, G, S, bu, go = _to64([v[f"{k}_A"], v[f"{k}_G"], v[f"{k}_step"], v["bu"], v["grad"]])
        announce(f"sdlinoss c128 golden {k}")
        st = getattr(K, f"sdlinoss_{variant}_forward")(to_dev(A), to_dev(G), to_dev(S), to_dev(bu))
        scale = float(np.abs(v[f"{k}_states"]).max())
        assert_close(to_np(st), v[f"{k}_states"], RTOL, ATOL * max(1.0, scale), "c128 golden states")
    for L, B, M in ((1, 1, 1), (2, 1, 65), (7, 4, 1)):
        A, G, S, bu, go = _to64(sdl_inputs("im", "full", L, B, M, seed=L + B + M))
        announce(f"sdlinoss c128 im L={L} B={B} M={M}")
        st = K.sdlinoss_im_forward(to_dev(A), to_dev(G), to_dev(S), to_dev(bu))
        grads = K.sdlinoss_im_backward(to_dev(A), to_dev(G), to_dev(S), to_dev(bu), st, to_dev(go))
        ref_st = oracle.sdlinoss_forward("im", A, G, S, bu)
        assert_close(to_np(st), ref_st, RTOL64, ATOL64, "c128 edge states")
        for got, ref, name in zip(grads, oracle.sdlinoss_backward("im", A, G, S, bu, ref_st, go), NAMES):
            assert_close(to_np(got), ref, RTOL64, ATOL64 * max(1.0, float(np.abs(ref).max())), name)
    A, G, S, bu, go = _to64(sdl_inputs("imex1", "m", 3, 2, 4, seed=2))
    dA, dG, dS = to_dev(A), to_dev(G), to_dev(S)
    out = K.sdlinoss_imex1_forward(dA, dG, dS, to_dev(bu)[:0])
    assert tuple(out.shape) == (0, 2, 4, 2) and out.dtype == torch.complex128
    grads = K.sdlinoss_imex1_backward(dA, dG, dS, to_dev(bu)[:0], out, to_dev(go)[:0])
    assert all(g.dtype == torch.float64 and float(g.abs().sum()) == 0.0 for g in grads[:3])
