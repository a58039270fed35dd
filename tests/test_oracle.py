"""Pins for the CPU oracle (oracle/): golden fixtures, the reference's own
compiled CPU kernels, independent formulations and fp64 autograd.

CPU only.  Each check is chosen so that a plausible slip in the oracle (a
dropped term, a sign, a transposed operand, a wrong index) fails at least one.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests import _brute

GOLDEN = Path(__file__).resolve().parent / "golden"
VARIANTS = oracle.VARIANTS


@pytest.fixture(scope="module")
def vectors():
    with np.load(GOLDEN / "ref_kernel_vectors.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _close(actual, expected, rtol, atol, what=""):
    np.testing.assert_allclose(actual, expected, rtol=rtol, atol=atol, err_msg=what)


# --------------------------------------------------------------------- D-LinOSS
@pytest.mark.parametrize("variant", VARIANTS)
def test_dlinoss_matches_reference_kernel_vectors(variant, vectors):
    """Oracle vs the reference's own CPU kernels (oracle/_ref), fwd and bwd."""
    v = vectors
    st = oracle.dlinoss_forward(variant, v["dl_a"], v["dl_g"], v["dl_step"], v["dl_bu"])
    _close(st, v[f"dl_{variant}_states"], 1e-5, 1e-5, "states")
    ga, gg, gs, gb = oracle.dlinoss_backward(variant, v["dl_a"], v["dl_g"], v["dl_step"],
                                             v["dl_bu"], v[f"dl_{variant}_states"], v["dl_grad"])
    _close(gb, v[f"dl_{variant}_grad_bu"], 1e-5, 1e-5, "grad_bu")
    for got, key in ((ga, "grad_a"), (gg, "grad_g"), (gs, "grad_step")):
        ref = v[f"dl_{variant}_{key}"]
        _close(got, ref, 1e-5, 1e-5 * np.abs(ref).max(), key)


def _layer_case(variant: str, dtype: str):
    cases = json.loads((GOLDEN / "dlinoss_reference_cases.json").read_text())["cases"]
    return cases[variant][dtype]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("dtype", ["float32", "float64"])
def test_dlinoss_matches_reference_layer_fixture(variant, dtype):
    """Golden layer fixture of the reference (tests/dlinoss_reference_cases.json).

    The layer glue (bu = u B^T, y = Re(x C^T) + D u, loss of the reference test
    test_dlinoss_parity.py:130-137) is written here in numpy; the scan and its
    adjoint come from the oracle.
    """
    c = _layer_case(variant, dtype)
    rt = np.float32 if dtype == "float32" else np.float64
    ct = np.complex64 if dtype == "float32" else np.complex128
    tol = 5e-6 if dtype == "float32" else 1e-9  # the reference test's tolerances
    a, g, step = (np.asarray(c[k], rt) for k in ("A_diag", "G_diag", "step"))
    Bw = np.asarray(c["B"], rt)          # [P, H, 2]
    Cw = np.asarray(c["C"], rt)          # [H, P, 2]
    Dw = np.asarray(c["D"], rt)          # [H]
    u = np.asarray(c["inputs"], rt)      # [B, L, H]
    Bc = (Bw[..., 0] + 1j * Bw[..., 1]).astype(ct)
    bu = np.einsum("blh,ph->lbp", u.astype(ct), Bc).astype(ct)
    states = oracle.dlinoss_forward(variant, a, g, step, bu)   # [L, B, P, 2]
    main = states[..., 1].transpose(1, 0, 2)                   # [B, L, P]
    aux = states[..., 0].transpose(1, 0, 2)
    _close(np.stack([main.real, main.imag], -1), np.asarray(c["states"]["main"]), tol, tol, "main")
    _close(np.stack([aux.real, aux.imag], -1), np.asarray(c["states"]["aux"]), tol, tol, "aux")
    out = main.real @ Cw[..., 0].T - main.imag @ Cw[..., 1].T + u * Dw
    _close(out, np.asarray(c["outputs"]), tol, tol, "outputs")

    # loss = sum(out^2) + |main|^2 + |aux|^2  (complex grads as d/dre + i d/dim)
    g_out = 2 * out
    g_main = np.einsum("blh,hp->blp", g_out, Cw[..., 0] - 1j * Cw[..., 1]) + 2 * main
    g_aux = 2 * aux
    ga, gg, gs, gbu = oracle.dlinoss_backward(
        variant, a, g, step, bu, states,
        g_main.transpose(1, 0, 2).astype(ct), grad_aux=g_aux.transpose(1, 0, 2).astype(ct))
    gB = np.stack([np.einsum("lbp,blh->ph", gbu.real, u), np.einsum("lbp,blh->ph", gbu.imag, u)], -1)
    grads = c["grads"]
    for got, key in ((ga, "A_diag"), (gg, "G_diag"), (gs, "step"), (gB, "B")):
        _close(got, np.asarray(grads[key]), tol, tol, key)


@pytest.mark.parametrize("variant", VARIANTS)
def test_dlinoss_backward_matches_fp64_autograd(variant):
    """Hand-written adjoint vs torch.autograd of a plain fp64 loop."""
    rng = np.random.default_rng(3)
    L, B, P = 19, 2, 5
    a = rng.uniform(0.1, 1.0, P)
    g = rng.uniform(0.0, 1.0, P)
    dt = 1.0 / (1.0 + np.exp(-rng.normal(size=P)))
    bu = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    G = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    ta, tg, tdt = (torch.tensor(x, requires_grad=True) for x in (a, g, dt))
    tbu = torch.tensor(bu, requires_grad=True)
    s = _brute.dlinoss_states(variant, ta, tg, tdt, tbu)
    # real loss whose gradient w.r.t. x = s[...,1] is G (re + i im convention)
    loss = (s[..., 1] * torch.tensor(G).conj()).real.sum()
    loss.backward()
    states = oracle.dlinoss_forward(variant, a, g, dt, bu)
    _close(states, s.detach().numpy(), 1e-12, 1e-12, "states")
    ga, gg, gs, gbu = oracle.dlinoss_backward(variant, a, g, dt, bu, states, G)
    _close(ga, ta.grad.numpy(), 1e-10, 1e-10, "grad_a")
    _close(gg, tg.grad.numpy(), 1e-10, 1e-10, "grad_g")
    _close(gs, tdt.grad.numpy(), 1e-10, 1e-10, "grad_step")
    _close(gbu, tbu.grad.numpy(), 1e-10, 1e-10, "grad_bu")


def test_dlinoss_imex1_matches_official_z_recurrence():
    """imex1 evolves w = dt*z; the official D-LinOSS recurrence keeps z
    (reference test_dlinoss.py:11-35, 174-188)."""
    rng = np.random.default_rng(7)
    L, B, P = 9, 2, 4
    a, g = rng.uniform(size=P), rng.uniform(size=P)
    dt = rng.uniform(size=P) * 0.5 + 0.1
    bu = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    states = oracle.dlinoss_forward("imex1", a, g, dt, bu)
    z = np.zeros((B, P), complex)
    x = np.zeros((B, P), complex)
    for t in range(L):
        z = (z + dt * (-a * x + bu[t])) / (1 + dt * g)
        x = x + dt * z
        _close(states[t, ..., 0] / dt, z, 1e-12, 1e-13, f"z[{t}]")
        _close(states[t, ..., 1], x, 1e-12, 1e-13, f"x[{t}]")


@pytest.mark.parametrize("variant", VARIANTS)
def test_dlinoss_special_cases(variant):
    rng = np.random.default_rng(11)
    P = 6
    a, g = rng.uniform(0.1, 1, P), rng.uniform(0, 1, P)
    dt = 1 / (1 + np.exp(-rng.normal(size=P)))
    zero = np.zeros((5, 3, P), complex)
    assert np.all(oracle.dlinoss_forward(variant, a, g, dt, zero) == 0)
    # linearity: scan(x + 2y) = scan(x) + 2 scan(y)
    x = rng.normal(size=(13, 2, P)) + 1j * rng.normal(size=(13, 2, P))
    y = rng.normal(size=(13, 2, P)) + 1j * rng.normal(size=(13, 2, P))
    sx, sy = (oracle.dlinoss_forward(variant, a, g, dt, v) for v in (x, y))
    _close(oracle.dlinoss_forward(variant, a, g, dt, x + 2 * y), sx + 2 * sy, 1e-12, 1e-12)
    # causality: changing bu at t=7 leaves states before 7 untouched
    x2 = x.copy()
    x2[7] += 1.0
    s2 = oracle.dlinoss_forward(variant, a, g, dt, x2)
    assert np.array_equal(s2[:7], sx[:7]) and not np.array_equal(s2[7:], sx[7:])
    if variant == "ex":  # f2 = 0: x_0 = dt*w_{-1} + x_{-1} = 0
        assert np.all(sx[0, ..., 1] == 0)


# ----------------------------------------------------------------------- LinOSS
def test_linoss_forward_matches_reference_kernel_vectors(vectors):
    v = vectors
    out = oracle.linoss_forward(v["lo_m11"], v["lo_m12"], v["lo_m21"], v["lo_m22"], v["lo_b"])
    _close(out, v["lo_out"], 1e-5, 1e-5)


def test_linoss_matches_reference_layer_snapshot():
    """REFERENCE_LINOSS LinOSS-IM layer snapshot (test_linoss_parity.py:74-204);
    layer glue from linoss.py:199-258, 293-314."""
    ref = json.loads((GOLDEN / "linoss_reference_snapshot.json").read_text())
    A = np.asarray(ref["A_diag"], np.float32)
    Bw = np.asarray(ref["B"], np.float32)                  # [P, H, 2]
    Cw = np.asarray(ref["C"], np.float32).reshape(6, 4, 2)  # [H, P, 2]
    Dw = np.asarray(ref["D"], np.float32)
    steps = np.asarray(ref["steps"], np.float32)
    u = np.asarray(ref["inputs"], np.float32)              # [B, L, H]
    a = np.maximum(A, 0)
    dt = 1 / (1 + np.exp(-steps))
    schur = 1 / (1 + dt * dt * a)
    m11, m12, m21, m22 = 1 - dt * dt * a * schur, -dt * a * schur, dt * schur, schur
    bu = np.einsum("blh,ph->lbp", u, Bw[..., 0] + 1j * Bw[..., 1]).astype(np.complex64)
    b_seq = np.stack([bu * (m11 * dt), bu * (m21 * dt)], -1).astype(np.complex64)
    ms = [m.astype(np.complex64) for m in (m11, m12, m21, m22)]
    st = oracle.linoss_forward(*ms, b_seq)[..., 1].transpose(1, 0, 2)
    out = st.real @ Cw[..., 0].T - st.imag @ Cw[..., 1].T + u * Dw
    _close(out, np.asarray(ref["outputs"]), 5e-6, 5e-6)


def test_linoss_backward_matches_fp64_autograd():
    rng = np.random.default_rng(5)
    L, B, P = 17, 3, 4
    M = (rng.normal(size=(P, 2, 2)) + 1j * rng.normal(size=(P, 2, 2))) * 0.4
    bs = rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))
    G = rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))
    tM = torch.tensor(M, requires_grad=True)
    tb = torch.tensor(bs, requires_grad=True)
    s = _brute.linoss_states(tM, tb)
    (s * torch.tensor(G).conj()).real.sum().backward()
    ms = [M[:, 0, 0], M[:, 0, 1], M[:, 1, 0], M[:, 1, 1]]
    states = oracle.linoss_forward(*ms, bs)
    _close(states, s.detach().numpy(), 1e-12, 1e-12)
    gm, gb = oracle.linoss_backward(*ms, states, G)
    _close(gm, tM.grad.numpy(), 1e-10, 1e-10, "grad_M")
    _close(gb, tb.grad.numpy(), 1e-10, 1e-10, "grad_b")


# -------------------------------------------------------------------- selective
@pytest.mark.parametrize("tag", ["gate", "nogate"])
def test_selective_matches_reference_kernel_vectors(tag, vectors):
    v = vectors
    gate = v["sel_z"] if tag == "gate" else None
    args = (v["sel_u"], v["sel_dt"], v["sel_A"], v["sel_B"], v["sel_C"])
    _close(oracle.selective_forward(*args, gate), v[f"sel_{tag}_out"], 1e-5, 1e-5, "out")
    grads = oracle.selective_backward(v["sel_grad"], *args, gate)
    for got, name in zip(grads, ("du", "ddt", "dA", "dB", "dC", "dz")):
        ref = v[f"sel_{tag}_{name}"]
        _close(got, ref, 1e-5, 1e-5 * max(1.0, np.abs(ref).max()), name)


@pytest.mark.parametrize("gated", [True, False])
def test_selective_backward_matches_fp64_autograd(gated):
    rng = np.random.default_rng(9)
    Bz, D, L, N = 2, 3, 23, 5
    u = rng.normal(size=(Bz, D, L))
    dt = np.log1p(np.exp(rng.normal(size=(Bz, D, L)) - 2))
    A = -np.exp(rng.normal(size=(D, N)))
    Bm, Cm = rng.normal(size=(Bz, L, N)), rng.normal(size=(Bz, L, N))
    z = rng.normal(size=(Bz, D, L)) if gated else None
    G = rng.normal(size=(Bz, D, L))
    ts = [torch.tensor(x, requires_grad=True) for x in (u, dt, A, Bm, Cm)]
    tz = torch.tensor(z, requires_grad=True) if gated else None
    y = _brute.selective(*ts, tz)
    (y * torch.tensor(G)).sum().backward()
    _close(oracle.selective_forward(u, dt, A, Bm, Cm, z), y.detach().numpy(), 1e-12, 1e-12)
    grads = oracle.selective_backward(G, u, dt, A, Bm, Cm, z)
    names = ("du", "ddt", "dA", "dB", "dC")
    for got, t, name in zip(grads, ts, names):
        _close(got, t.grad.numpy(), 1e-10, 1e-10, name)
    if gated:
        _close(grads[5], tz.grad.numpy(), 1e-10, 1e-10, "dz")
    else:
        assert np.all(grads[5] == 0)


def test_reference_module_when_present():
    """oracle/_ref, when built, exports the reference's 21 CPU entry points."""
    if not oracle.have_reference():
        pytest.skip("oracle/_ref not built")
    mod = oracle.reference_module()
    for v in VARIANTS:
        assert hasattr(mod, f"dlinoss_{v}_forward") and hasattr(mod, f"dlinoss_{v}_backward")
    for name in ("linoss_scan", "selective_scan", "selective_scan_backward"):
        assert hasattr(mod, name)


# ----------------------------------------------------------- selective D-LinOSS
@pytest.fixture(scope="module")
def sdl_vectors():
    with np.load(GOLDEN / "sdl_kernel_vectors.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


SDL_CASES = [(v, tag) for v in VARIANTS for tag in ("full", "bcast_t", "bcast_b", "m")
             if tag == "full" or v in ("imex1", "im")]


@pytest.mark.parametrize("variant,tag", SDL_CASES)
def test_sdlinoss_matches_reference_kernel_vectors(variant, tag, sdl_vectors):
    """Oracle vs the reference's own CPU kernels (fixture written from oracle/_ref),
    every accepted parameter layout, both clamps hit."""
    v = sdl_vectors
    k = f"{variant}_{tag}"
    A, G, S = v[f"{k}_A"], v[f"{k}_G"], v[f"{k}_step"]
    st = oracle.sdlinoss_forward(variant, A, G, S, v["bu"])
    scale = np.abs(v[f"{k}_states"]).max()
    _close(st, v[f"{k}_states"], 1e-5, 1e-6 * scale, "states")
    grads = oracle.sdlinoss_backward(variant, A, G, S, v["bu"], v[f"{k}_states"], v["grad"])
    for got, name in zip(grads, ("grad_A", "grad_G", "grad_step", "grad_bu")):
        ref = v[f"{k}_{name}"]
        assert got.shape == ref.shape, name
        _close(got, ref, 1e-4, 1e-5 * max(1.0, np.abs(ref).max()), name)


SDL_SHAPES = {"full": lambda L, B, M: (L, B, M), "bcast_t": lambda L, B, M: (1, B, M),
              "bcast_b": lambda L, B, M: (L, 1, M), "m": lambda L, B, M: (M,)}


@pytest.mark.parametrize("tag", list(SDL_SHAPES))
@pytest.mark.parametrize("variant", VARIANTS)
def test_sdlinoss_backward_matches_fp64_autograd(variant, tag):
    """Hand-written per-step adjoint (and the sum over broadcast axes) vs
    torch.autograd of a plain fp64 loop; steps on both sides of the dt clamp."""
    rng = np.random.default_rng(11)
    L, B, M = 17, 3, 4
    shp = SDL_SHAPES[tag](L, B, M)
    A = rng.uniform(0.1, 1.2, shp)
    G = rng.uniform(0.0, 1.0, shp)
    S = rng.uniform(-0.3, 1.4, shp)
    S[np.abs(S - 1e-6) < 1e-3] = 0.5  # keep away from the clamp's kinks
    S[np.abs(S - 1.0) < 1e-3] = 0.5
    bu = rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))
    Gout = rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))
    tA, tG, tS = (torch.tensor(x, requires_grad=True) for x in (A, G, S))
    tbu = torch.tensor(bu, requires_grad=True)
    s = _brute.sdlinoss_states(variant, tA, tG, tS, tbu)
    loss = (s[..., 1] * torch.tensor(Gout).conj()).real.sum()
    loss.backward()
    states = oracle.sdlinoss_forward(variant, A, G, S, bu)
    _close(states, s.detach().numpy(), 1e-12, 1e-12, "states")
    gA, gG, gS, gbu = oracle.sdlinoss_backward(variant, A, G, S, bu, states, Gout)
    _close(gA, tA.grad.numpy(), 1e-10, 1e-10, "grad_A")
    _close(gG, tG.grad.numpy(), 1e-10, 1e-10, "grad_G")
    _close(gS, tS.grad.numpy(), 1e-10, 1e-10, "grad_step")
    _close(gbu, tbu.grad.numpy(), 1e-10, 1e-10, "grad_bu")


def test_sdlinoss_stiff_clamp_matches_fp64_autograd():
    """S = 1 + dt g below 1e-6 (imex1, im) at the last step: the clamp's zero
    gradient w.r.t. S is honoured."""
    rng = np.random.default_rng(12)
    L, B, M = 9, 2, 3
    for variant in ("imex1", "im"):
        A = rng.uniform(0.1, 1.0, (L, B, M))
        G = rng.uniform(0.0, 1.0, (L, B, M))
        S = rng.uniform(0.1, 0.9, (L, B, M))
        G[-1] = -4.0
        S[-1] = 0.8
        bu = rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))
        Gout = rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))
        tA, tG, tS = (torch.tensor(x, requires_grad=True) for x in (A, G, S))
        tbu = torch.tensor(bu, requires_grad=True)
        s = _brute.sdlinoss_states(variant, tA, tG, tS, tbu)
        (s[..., 1] * torch.tensor(Gout).conj()).real.sum().backward()
        states = oracle.sdlinoss_forward(variant, A, G, S, bu)
        gA, gG, gS, gbu = oracle.sdlinoss_backward(variant, A, G, S, bu, states, Gout)
        for got, ref, name in ((gA, tA.grad, "A"), (gG, tG.grad, "G"), (gS, tS.grad, "step"),
                               (gbu, tbu.grad, "bu")):
            ref = ref.numpy()
            _close(got, ref, 1e-9, 1e-9 * np.abs(ref).max(), f"{variant} grad_{name}")


# ------------------------------------------------------ diagonal scans (LRU, S5)
@pytest.fixture(scope="module")
def diag_vectors():
    with np.load(GOLDEN / "diag_kernel_vectors.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_diag_forward_matches_reference_kernel_vectors(prec, diag_vectors):
    """lru_scan and s5_scan of the reference's CPU build (fixture) agree with the
    restatement; eigenvalues from 0 to 0.999 in modulus, real, negative, imaginary."""
    v = diag_vectors
    got = oracle.diag_forward(v[f"{prec}_lambda"], v[f"{prec}_b"])
    tol = 1e-6 if prec == "f32" else 1e-13
    for name in ("lru", "s5"):
        _close(got, v[f"{prec}_{name}"], tol, tol, name)


def test_diag_forward_matches_reference_complex_literal():
    """The reference test's own literals (test_scan_parity.py:186-349, checked there at
    atol = rtol = 5e-6, :465-474)."""
    d = json.loads((GOLDEN / "complex_scan_reference.json").read_text())
    c = lambda k: np.asarray(d[k])[..., 0] + 1j * np.asarray(d[k])[..., 1]  # noqa: E731
    lam = c("REFERENCE_COMPLEX_LAMBDA").astype(np.complex64)
    b = c("REFERENCE_COMPLEX_B").astype(np.complex64)
    _close(oracle.diag_forward(lam, b), c("REFERENCE_COMPLEX_STATES"), 5e-6, 5e-6)


def test_diag_backward_matches_fp64_autograd():
    """The restated Python backward (lru.py:52-80) against autograd of the plain
    loop, which the reference's own test uses as its oracle (test_scan_parity.py:352-370):
    a dropped conj on lambda or x, or a shifted x_{t-1}, fails here."""
    rng = np.random.default_rng(11)
    L, B, P = 23, 3, 5
    lam = (rng.uniform(0.2, 0.95, P) * np.exp(1j * rng.uniform(-np.pi, np.pi, P)))
    b = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    G = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    tl = torch.tensor(lam, requires_grad=True)
    tb = torch.tensor(b, requires_grad=True)
    x = _brute.diag_states(tl, tb)
    gl, gb = torch.autograd.grad(x, (tl, tb), grad_outputs=torch.tensor(G))
    states = oracle.diag_forward(lam, b)
    _close(states, x.detach().numpy(), 1e-12, 1e-12, "states")
    ol, ob = oracle.diag_backward(lam, states, G)
    _close(ol, gl.numpy(), 1e-10, 1e-10, "grad_lambda")
    _close(ob, gb.numpy(), 1e-10, 1e-10, "grad_b")


def test_diag_special_cases():
    """lambda = 0: x = b and grad_lambda = sum_t g_t conj(b_{t-1}); one step: grad_b =
    grad, grad_lambda = 0; lambda = 1: x is the running sum of b."""
    rng = np.random.default_rng(3)
    L, B, P = 9, 2, 4
    b = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    G = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    zero = np.zeros(P, complex)
    x = oracle.diag_forward(zero, b)
    _close(x, b, 0, 0, "lambda=0 states")
    gl, gb = oracle.diag_backward(zero, x, G)
    _close(gb, G, 0, 0, "lambda=0 grad_b")
    _close(gl, (G[1:] * np.conj(b[:-1])).sum(axis=(0, 1)), 1e-12, 1e-12, "lambda=0 grad_lambda")
    gl1, gb1 = oracle.diag_backward(zero + 0.5, b[:1], G[:1])
    _close(gl1, np.zeros(P), 0, 0, "one step grad_lambda")
    _close(gb1, G[:1], 0, 0, "one step grad_b")
    _close(oracle.diag_forward(np.ones(P, complex), b), np.cumsum(b, axis=0), 1e-12, 1e-12,
           "lambda=1 running sum")
