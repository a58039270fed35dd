"""Seeded random shapes for every scan family, forward and backward, against
the oracle (fp32 reference and fp64 arbiter, the north star's tolerance).

The fixed-shape tests pick their shapes for the tile and layout boundaries;
these draw lengths, batch sizes and channel counts from wide ranges (ragged
everywhere: channel counts that are not multiples of 64, lengths that end
inside a sub-chunk, grids on both sides of the dispatch-order threshold), with
a fixed seed so that every run draws the same cases.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests import test_gpu_diag as diag
from tests import test_gpu_oscillator as osc
from tests import test_gpu_sdlinoss as sdl
from tests import test_gpu_selective as sel
from tests.gpu_util import (announce, assert_parity, dlinoss_inputs, need_gpu, no_device_errors,
                            to_dev, to_np)

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def _draw(seed, n, ranges):
    """n cases of integers, each drawn from its (lo, hi, log) range: uniformly,
    or log-uniformly when log is set."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        case = []
        for lo, hi, log in ranges:
            if log:
                v = int(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))
            else:
                v = int(rng.integers(lo, hi + 1))
            case.append(min(max(v, lo), hi))
        cases.append(tuple(case))
    return cases


# (L, B, P)
OSC_CASES = _draw(101, 24, [(1, 4000, True), (1, 8, False), (1, 300, True)])
# (B, D, L, N)
SEL_CASES = _draw(202, 20, [(1, 4, False), (1, 300, True), (1, 600, True), (1, 40, False)])


@pytest.mark.parametrize("case", range(len(OSC_CASES)))
def test_dlinoss_random_shapes(K, case):
    L, B, P = OSC_CASES[case]
    variant = oracle.VARIANTS[case % 4]
    a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=1000 + case, variant=variant)
    announce(f"random dlinoss {variant} L={L} B={B} P={P}")
    st = osc._fwd(K, variant, a, g, dt, bu)
    grads = osc._bwd(K, variant, a, g, dt, bu, st, go)
    ref = oracle.dlinoss_forward(variant, a, g, dt, bu)
    rgrads = oracle.dlinoss_backward(variant, a, g, dt, bu, ref, go)
    st64, tgrads = osc._oracle64(variant, a, g, dt, bu, go)
    assert_parity(to_np(st), ref, st64, RTOL, ATOL, "states")
    for got, r32, r64, name in zip(grads, rgrads, tgrads, ("grad_a", "grad_g", "grad_step", "grad_bu")):
        atol = ATOL if name == "grad_bu" else osc._param_atol(r64)
        assert_parity(to_np(got), r32, r64, RTOL, atol, name)
    no_device_errors()


@pytest.mark.parametrize("case", range(len(OSC_CASES)))
def test_linoss_random_shapes(K, case):
    L, B, P = OSC_CASES[case]
    ms, b, go = osc._linoss_inputs(L, B, P, seed=2000 + case)
    announce(f"random linoss L={L} B={B} P={P}")
    st = K.linoss_scan(*[to_dev(m) for m in ms], to_dev(b))
    ref = oracle.linoss_forward(*ms, b)
    ms64 = [m.astype(np.complex128) for m in ms]
    st64 = oracle.linoss_forward(*ms64, b.astype(np.complex128))
    assert_parity(to_np(st), ref, st64, RTOL, ATOL, "states")
    gm, gb = K.linoss_scan_backward(*[to_dev(m) for m in ms], st, to_dev(go))
    rgm, rgb = oracle.linoss_backward(*ms, ref, go)
    tgm, tgb = oracle.linoss_backward(*ms64, st64, go.astype(np.complex128))
    assert_parity(to_np(gb), rgb, tgb, RTOL, ATOL, "grad_b")
    assert_parity(to_np(gm), rgm, tgm, RTOL, osc._param_atol(tgm), "grad_m")
    no_device_errors()


@pytest.mark.parametrize("case", range(len(OSC_CASES)))
def test_diag_random_shapes(K, case):
    L, B, P = OSC_CASES[case]
    lam, b, go = diag.diag_inputs(L, B, P, seed=3000 + case)
    announce(f"random lru L={L} B={B} P={P}")
    states, gl, gb = diag._run(K, lam, b, go, "lru" if case % 2 else "s5")
    diag._check(lam, b, go, states, gl, gb, f"random {L}x{B}x{P}")
    no_device_errors()


@pytest.mark.parametrize("case", range(len(OSC_CASES)))
def test_sdlinoss_random_shapes(K, case):
    L, B, M = OSC_CASES[case]
    variant = oracle.VARIANTS[(case + 1) % 4]
    tag = ("full", "bcast_t", "bcast_b", "m", "lm", "bm")[case % 6]
    args = sdl.sdl_inputs(variant, tag, L, B, M, seed=4000 + case)
    announce(f"random sdlinoss {variant} {tag} L={L} B={B} M={M}")
    states, grads = sdl._run(K, variant, *args)
    sdl._check(variant, *args, states, grads, f"random {tag} {L}x{B}x{M}")
    no_device_errors()


@pytest.mark.parametrize("case", range(len(SEL_CASES)))
def test_selective_random_shapes(K, case):
    Bz, D, L, N = SEL_CASES[case]
    gated = case % 2 == 0
    args = sel.selective_inputs(Bz, D, L, N, seed=5000 + case, gated=gated)
    announce(f"random selective B={Bz} D={D} L={L} N={N} gated={gated}")
    out, _, _, grads = sel._run(K, *args)
    sel._check_all(out, grads, *args, what=f"random {Bz}x{D}x{L}x{N}")
    no_device_errors()
