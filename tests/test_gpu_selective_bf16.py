"""GPU parity of the bf16-storage selective scan (``selective_scan_cuda_bf16``,
an extension with no counterpart in the reference, whose extension is fp32
only).

Inputs are drawn in fp32 and rounded to bf16; the oracle runs on exactly those
values.  The kernel widens them exactly, runs the same fp32 recurrence as the
fp32 entry point and rounds each stored value once (round to nearest even), so
two properties pin it:

* against fp64 truth on the bf16 values: every output within one bf16 unit in
  the last place (2**-8 relative) plus the fp32 path's own error;
* against the fp32 entry point on the same (bf16-valued) inputs, rounded by
  torch: at most one bf16 ulp apart everywhere and equal almost everywhere
  (a truncating or biased conversion fails the second part).  ``dz`` is left
  out of this comparison because it reads y back from the bf16 ``raw_outputs``.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.gpu_util import announce, need_gpu, rel_fro, to_dev, to_np
from tests.test_gpu_selective import NAMES, selective_inputs

pytestmark = pytest.mark.gpu

EPS_BF16 = 2.0 ** -8  # one ulp relative, i.e. twice the worst rounding error


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def _bf16_round(x):
    """Round fp32 arrays to bf16 values (torch's conversion is round-to-nearest-even)."""
    import torch

    if x is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).float().numpy()


def _dev_bf16(x):
    import torch

    return None if x is None else to_dev(x).to(torch.bfloat16)


def _np(t):
    return to_np(t.float())


def _ulp_diff(a_bf16, b_bf16):
    """Distance in bf16 units in the last place between two bf16 tensors (same sign or
    zero); computed on their 16-bit patterns as ordered integers."""
    import torch

    def key(t):
        v = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(v < 0, -32768 - v, v)  # sign-magnitude -> ordered

    return (key(a_bf16) - key(b_bf16)).abs()


def _run_bf16(K, u, dt, A, Bm, Cm, z, g):
    dz = _dev_bf16(z)
    out, chunks, raw = K.selective_scan_cuda_bf16(_dev_bf16(u), _dev_bf16(dt), to_dev(A),
                                                  _dev_bf16(Bm), _dev_bf16(Cm), dz)
    grads = K.selective_scan_cuda_bf16_backward(_dev_bf16(g), _dev_bf16(u), _dev_bf16(dt),
                                                to_dev(A), _dev_bf16(Bm), _dev_bf16(Cm), dz, chunks,
                                                raw, 16)
    return out, chunks, raw, grads


def _run_fp32(K, u, dt, A, Bm, Cm, z, g):
    dz = None if z is None else to_dev(z)
    out, chunks, raw = K.selective_scan_cuda(to_dev(u), to_dev(dt), to_dev(A), to_dev(Bm),
                                             to_dev(Cm), dz)
    grads = K.selective_scan_cuda_backward(to_dev(g), to_dev(u), to_dev(dt), to_dev(A),
                                           to_dev(Bm), to_dev(Cm), dz, chunks, raw, 16)
    return out, chunks, raw, grads


def _truth_bound(got, ref64, rel, what):
    scale = max(1.0, float(np.abs(ref64).max()))
    err = np.abs(got.astype(np.float64) - ref64)
    bound = rel * np.abs(ref64) + 2e-5 * scale
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} elements beyond one bf16 ulp of "
                           f"fp64 truth; worst excess {float((err - bound).max()):.3e}")


def _check_vs_fp32(bf, f32, what):
    import torch

    ref = f32.to(torch.bfloat16)
    d = _ulp_diff(bf, ref)
    assert int(d.max()) <= 1, f"{what}: {int(d.max())} bf16 ulps from the rounded fp32 path"
    frac = float((d == 0).float().mean())
    assert frac >= 0.99, f"{what}: only {frac:.4f} of elements equal to the rounded fp32 path"


# (64, 1024, 64, 16) runs the forward with 4 states per lane on a 256-CU
# MI355X, the others with 2 (see test_gpu_selective.SHAPES)
SHAPES = [(1, 1, 1, 1), (2, 70, 37, 5), (3, 65, 100, 16), (1, 130, 129, 20), (2, 48, 192, 32),
          (4, 96, 384, 64), (64, 1024, 64, 16)]


@pytest.mark.parametrize("gated", [True, False], ids=["gate", "nogate"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_selective_bf16_vs_oracle_and_fp32_path(K, shape, gated):
    _bf16_case(K, shape, gated)


@pytest.mark.parametrize("npw", [2, 4])
@pytest.mark.parametrize("shape", [(2, 70, 37, 5), (1, 130, 129, 20), (4, 96, 384, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_selective_bf16_backward_both_layouts(K, shape, npw, monkeypatch):
    """bf16 storage with the backward forced to 2 and to 4 states per lane."""
    monkeypatch.setenv("OSSM_SEL_BWD_NPW", str(npw))
    _bf16_case(K, shape, True)


@pytest.mark.parametrize("npw", [2, 4])
@pytest.mark.parametrize("shape", [(2, 70, 37, 5), (1, 130, 129, 20), (4, 96, 384, 64),
                                   (2, 40, 2070, 16)],
                         ids=lambda s: "x".join(map(str, s)))
def test_selective_bf16_forward_both_layouts(K, shape, npw, monkeypatch):
    """bf16 storage with the forward forced to 2 and to 4 states per lane."""
    monkeypatch.setenv("OSSM_SEL_FWD_NPW", str(npw))
    _bf16_case(K, shape, True)


def _bf16_case(K, shape, gated):
    import torch

    Bz, D, L, N = shape
    args = [_bf16_round(x) if i != 2 else x
            for i, x in enumerate(selective_inputs(Bz, D, L, N, seed=5 + Bz + D + L + N,
                                                   gated=gated))]
    u, dt, A, Bm, Cm, z, g = args
    announce(f"selective bf16 B={Bz} D={D} L={L} N={N} gated={gated}")
    out, chunks, raw, grads = _run_bf16(K, *args)
    assert out.dtype == torch.bfloat16 and chunks.dtype == torch.float32
    assert grads[2].dtype == torch.float32 and grads[3].dtype == torch.bfloat16
    # fp64 truth on the bf16 values
    f64 = [x.astype(np.float64) if x is not None else None for x in args]
    t_out = oracle.selective_forward(*f64[:6])
    t_g = oracle.selective_backward(f64[6], *f64[:6])
    _truth_bound(_np(out), t_out, EPS_BF16, "out")
    for got, ref, name in zip(grads, t_g, NAMES):
        rel = 2 * EPS_BF16 if name == "dz" else EPS_BF16
        if name == "dA":
            rel = 1e-5  # fp32 output: only the fp32 sum's own error
        _truth_bound(_np(got), ref, rel, name)
    # the fp32 entry point on the same values, rounded once
    o32, c32, _, g32 = _run_fp32(K, *args)
    _check_vs_fp32(out, o32, "out")
    assert torch.equal(chunks, c32), "chunk_states differ from the fp32 path"
    for got, ref, name in zip(grads, g32, NAMES):
        if name == "dA":
            assert torch.equal(got, ref), "dA differs from the fp32 path"
        elif name != "dz":
            _check_vs_fp32(got, ref, name)


def test_selective_bf16_config4(K):
    """BASELINE config 4 (B=16, D=1536, L=2048, N=16, bf16 storage): the full
    tensors against the fp32 entry point on the same values (one-ulp rule),
    and one batch row (every per-row output and gradient: out, du, ddt, dB,
    dC, dz) against fp64 truth."""
    Bz, D, L, N = 16, 1536, 2048, 16
    args = [_bf16_round(x) if i != 2 else x
            for i, x in enumerate(selective_inputs(Bz, D, L, N, seed=46))]
    u, dt, A, Bm, Cm, z, g = args
    announce("selective bf16 config4")
    out, chunks, raw, grads = _run_bf16(K, *args)
    o32, c32, _, g32 = _run_fp32(K, *args)
    _check_vs_fp32(out, o32, "out")
    for got, ref, name in zip(grads, g32, NAMES):
        if name == "dA":
            assert rel_fro(_np(got), _np(ref)) == 0.0, "dA"
        elif name != "dz":
            _check_vs_fp32(got, ref, name)
    del o32, c32, g32
    bs = [3]
    sl = lambda x: np.ascontiguousarray(x[bs]).astype(np.float64)  # noqa: E731
    t_out = oracle.selective_forward(sl(u), sl(dt), A.astype(np.float64), sl(Bm), sl(Cm), sl(z))
    _truth_bound(_np(out)[bs], t_out, EPS_BF16, "out slice")
    t_g = oracle.selective_backward(sl(g), sl(u), sl(dt), A.astype(np.float64), sl(Bm), sl(Cm),
                                    sl(z))
    # dB and dC of a batch row are sums over that row's channels only, so the
    # slice's fp64 backward is their exact truth
    for idx, name, rel in ((0, "du", EPS_BF16), (1, "ddt", EPS_BF16), (3, "dB", EPS_BF16),
                           (4, "dC", EPS_BF16), (5, "dz", 2 * EPS_BF16)):
        _truth_bound(_np(grads[idx])[bs], t_g[idx], rel, name + " slice")


def test_selective_bf16_errors(K):
    import torch

    u, dt, A, Bm, Cm, z, g = selective_inputs(2, 3, 8, 4, seed=7)
    with pytest.raises(RuntimeError, match="bfloat16"):
        K.selective_scan_cuda_bf16(to_dev(u), _dev_bf16(dt), to_dev(A), _dev_bf16(Bm),
                                   _dev_bf16(Cm))
    with pytest.raises(RuntimeError, match="A must be float32"):
        K.selective_scan_cuda_bf16(_dev_bf16(u), _dev_bf16(dt), _dev_bf16(A), _dev_bf16(Bm),
                                   _dev_bf16(Cm))
    out, chunks, raw = K.selective_scan_cuda_bf16(_dev_bf16(u[:, :, :0]), _dev_bf16(dt[:, :, :0]),
                                                  to_dev(A), _dev_bf16(Bm[:, :0]),
                                                  _dev_bf16(Cm[:, :0]))
    assert out.dtype == torch.bfloat16 and out.shape == (2, 3, 0)
